// Streaming decode over host-staged layers: the application loop of
// LeanStream examples/end_to_end/main.cu:58-72 on MI355X.
//
// Per layer, through the unchanged Runtime / LayerStep / WeightManager:
//   begin_layer -> update_prediction(rank) -> enqueue_compute (the persistent
//   consumer is pre-enqueued) -> finalize(final) -> completion -> commit({}).
// The transport is HostStagingIO over an SdmaCopyEngine (or a HipCopyEngine): each
// admitted group is one SDMA copy from the pinned host store into the device staging
// arena (slot = logical group), and its completion publishes READY to the queue the
// running kernel consumes. Layers run one after another: a layer's copies start only after
// the previous layer retired, which is after its kernel finished, so the shared
// staging arena never holds bytes a running kernel still reads.
#include <hip/hip_runtime_api.h>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstring>
#include <memory>
#include <new>
#include <thread>
#include <vector>
#include "leanstream/hip_backend.h"
#include "leanstream/hip_copy_engine.h"
#include "leanstream/host_staging_io.h"
#include "leanstream/runtime.h"
#include "leanstream_hip.h"

using namespace leanstream::runtime;

static_assert(sizeof(ls_group_layout) == sizeof(GroupLayout), "group layout record");

namespace {

uint64_t now_ns() {
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

template <class T>
T* pinned(size_t n) {
    void* p = nullptr;
    if (hipHostMalloc(&p, n * sizeof(T), hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) return nullptr;
    std::memset(p, 0, n * sizeof(T));
    return static_cast<T*>(p);
}

struct StreamDecoder {
    ls_stream_setup setup{};
    HipBackend* backend = nullptr;
    // queue and state words shared with the GPU (fine-grained host memory)
    ExecDesc* descriptors = nullptr;
    uint32_t* ready_indices = nullptr;
    QueueControl* control = nullptr;
    uint32_t* io_states = nullptr;
    std::vector<SlotId> cache_slots;
    std::unique_ptr<SdmaCopyEngine> sdma;
    std::unique_ptr<HipCopyEngine> copies;
    std::unique_ptr<HostStagingIO> io;
    std::unique_ptr<Runtime> runtime;
    // the transport's engine, behind a filter that can refuse one group's copies
    CopyEngine engine{};
    std::atomic<uint32_t> fail_group{UINT32_MAX};
    std::atomic<int> fail_error{0};

    static int filtered_submit(void* ctx, uint32_t lane, void* dst, const void* src, uint64_t bytes) {
        auto& d = *static_cast<StreamDecoder*>(ctx);
        const int error = d.fail_error.load(std::memory_order_acquire);
        if (error) {
            const uint64_t g = d.fail_group.load(std::memory_order_relaxed);
            const uint8_t* first = static_cast<const uint8_t*>(d.setup.staging) + g * d.setup.staging_stride;
            if (static_cast<const uint8_t*>(dst) >= first && static_cast<const uint8_t*>(dst) < first + d.setup.staging_stride)
                return error;
        }
        return d.engine.submit(d.engine.context, lane, dst, src, bytes);
    }
    static int filtered_poll(void* ctx, uint32_t lane) {
        auto& d = *static_cast<StreamDecoder*>(ctx);
        return d.engine.poll(d.engine.context, lane);
    }

    // The decoder's commit: this loop installs nothing into a cache (its groups stream every
    // layer), so a layer commits unless its launch raised a status bit. An application
    // install_cache hook on the backend still runs. The backend itself is left untouched:
    // used through its own view after the decoder is gone, it refuses commits without the
    // hook (ENOTSUP) as before.
    static int streamed_commit(void* ctx, uint32_t layer, Span<GroupId> ids) {
        auto& b = *static_cast<HipBackend*>(ctx);
        if (const int rc = b.status_error()) return rc;
        return b.install_cache ? b.install_cache(b.lifecycle_context, layer, ids) : 0;
    }

    ~StreamDecoder() {
        runtime.reset();  // drains every layer
        io.reset();       // drains the copy pump
        copies.reset();
        sdma.reset();
        if (descriptors) (void)hipHostFree(descriptors);
        if (ready_indices) (void)hipHostFree(ready_indices);
        if (control) (void)hipHostFree(control);
        if (io_states) (void)hipHostFree(io_states);
    }

    int init(const ls_stream_setup& s) {
        setup = s;
        backend = static_cast<HipBackend*>(s.backend);
        const uint32_t n = s.group_count;
        descriptors = pinned<ExecDesc>(n);
        ready_indices = pinned<uint32_t>(n);
        control = pinned<QueueControl>(1);
        io_states = pinned<uint32_t>(n + 1);
        if (!descriptors || !ready_indices || !control || !io_states) return ENOMEM;
        cache_slots.assign(n, -1);
        StagingConfig sc;
        if (s.copy_engine == LS_COPY_SDMA) {
            sdma.reset(new SdmaCopyEngine(s.device, s.qd, s.copy_queues, s.copy_chunk));
            engine = sdma->view();
        } else {
            copies.reset(new HipCopyEngine(s.device, s.qd, s.copy_queues));
            engine = copies->view();
        }
        sc.engine.context = this;
        sc.engine.submit = filtered_submit;
        sc.engine.poll = filtered_poll;
        sc.group_count = n;
        sc.qd = s.qd;
        sc.group_bytes = s.group_bytes;
        sc.staging_stride = s.staging_stride;
        io.reset(new HostStagingIO(sc));
        ManagerConfig mc{n, s.qd, s.group_bytes, s.staging_stride, 512, static_cast<ConsumerMode>(s.mode)};
        mc.io_backend = io->backend();
        ComputeBackend view = backend->view();
        view.commit = streamed_commit;
        runtime.reset(new Runtime(mc, view, s.layers));
        return 0;
    }

    DeviceExecQueue queue() const { return {descriptors, ready_indices, control, setup.group_count}; }

    // One layer; times (optional) receives 7 stamps in ns after `origin`.
    int layer(uint32_t id, const ls_stream_layer& L, void* stream, uint64_t origin, uint64_t* times,
              uint64_t* stamps, int timeout_ms) {
        const uint32_t n = setup.group_count;
        auto mark = [&](int k) {
            if (times) times[k] = now_ns() - origin;
        };
        mark(0);
        StagingLayer sl;
        sl.source = static_cast<const uint8_t*>(setup.host_store);
        sl.source_bytes = setup.host_bytes;
        sl.layout = {reinterpret_cast<const GroupLayout*>(L.layout), n};
        sl.staging = static_cast<uint8_t*>(setup.staging);
        sl.staging_bytes = setup.staging_bytes;
        sl.io_states = io_states;
        sl.arrival_ns = L.arrival_ns;
        sl.stamps = stamps;
        int rc = io->bind_layer(sl);
        if (rc) return rc;
        LayerStorage storage;
        storage.layout = sl.layout;
        storage.cache_slots = cache_slots.data();
        storage.staging = setup.staging;
        storage.io_states = io_states;
        storage.queue = queue();
        storage.staging_bytes = setup.staging_bytes;
        LayerStep step;
        rc = runtime->begin_layer(id, storage, &step);
        mark(1);
        if (rc) return rc;
        rc = step.update_prediction({L.rank, L.rank_count});
        mark(2);
        // The selector's io bucket: this loop's own snapshot of the ranked groups not yet
        // READY when the layer is submitted (docs/kernel_selection.md: an application-owned
        // remaining/total snapshot), quantized as the offline table was measured.
        uint32_t remaining = 0;
        for (uint32_t i = 0; i < L.rank_count; ++i) {
            const int32_t g = L.rank[i];
            if (g >= 0 && static_cast<uint32_t>(g) < n &&
                __atomic_load_n(io_states + g, __ATOMIC_ACQUIRE) != kIoReady)
                ++remaining;
        }
        backend->state.io_bucket = quantize_io_load(remaining, L.rank_count);
        if (!rc) rc = step.enqueue_compute(L.input, L.output, stream);
        mark(3);
        if (!rc) rc = step.finalize({L.final_ids, L.final_count});
        mark(4);
        // completion: the launch's own done word (no HIP call on this path)
        const ComputeBackend cb = backend->view();
        const uint64_t deadline = now_ns() + static_cast<uint64_t>(timeout_ms) * 1000000ull;
        bool done = false;
        while (!(done = cb.complete(cb.context, id)) && now_ns() < deadline) {
        }
        if (done) mark(5);
        if (!rc && !done) rc = ETIMEDOUT;
        if (!rc) {
            // a launch that raised a status bit (a bounded wait expired, a descriptor or the
            // queue was rejected, a value was out of range) produced no valid output: the
            // commit refuses it
            rc = step.commit({});
            mark(6);
            if (!rc) return 0;
        }
        // Failure. First cancel: the queue's error word lets workgroups still waiting for
        // READY groups leave at once, and abort is EBUSY until the launch is complete. Then
        // drain the launch stream (its epilogue), so nothing of this layer still reads the
        // staging arena the next layer's copies rewrite. Only then read and clear the status
        // bits: every bit this launch raised belongs to this layer, and the next one starts
        // clean.
        const uint64_t abort_deadline = now_ns() + 5000000000ull;
        int aborted;
        while ((aborted = step.abort()) == EBUSY && now_ns() < abort_deadline) std::this_thread::yield();
        const hipError_t synced = hipStreamSynchronize(static_cast<hipStream_t>(stream));
        if (aborted == EBUSY) (void)step.abort();   // the drained stream holds no workgroup
        if (const int st = backend->status_error()) {
            backend->clear_status();
            if (!rc) rc = st;
        }
        if (synced != hipSuccess) return EIO;
        return rc;
    }
};

}  // namespace

extern "C" {

void* ls_stream_create(const ls_stream_setup* s) {
    if (!s || !s->backend || !s->host_store || !s->staging || !s->group_count || !s->layers || !s->qd ||
        s->qd > 32 || !s->copy_queues || s->copy_queues > 16 || s->copy_engine > LS_COPY_HIP ||
        (s->copy_engine == LS_COPY_HIP && s->copy_queues > kMaxHipCopyStreams) || s->mode > 2 ||
        !static_cast<HipBackend*>(s->backend)->consumes_queue())
        return nullptr;
    auto* d = new (std::nothrow) StreamDecoder;
    if (!d) return nullptr;
    try {
        if (d->init(*s)) {
            delete d;
            return nullptr;
        }
    } catch (...) {
        delete d;
        return nullptr;
    }
    return d;
}

void ls_stream_destroy(void* h) { delete static_cast<StreamDecoder*>(h); }

int ls_stream_queue(void* h, ls_device_queue* out) {
    if (!h || !out) return EINVAL;
    const DeviceExecQueue q = static_cast<StreamDecoder*>(h)->queue();
    out->descriptors = reinterpret_cast<ls_exec_desc*>(q.descriptors);
    out->ready_indices = q.ready_indices;
    out->control = q.control;
    out->capacity = q.capacity;
    return 0;
}

int ls_stream_inject_copy_error(void* h, uint32_t group, int32_t error) {
    if (!h || error < 0) return EINVAL;
    auto& d = *static_cast<StreamDecoder*>(h);
    if (error && group >= d.setup.group_count) return EINVAL;
    d.fail_error.store(0, std::memory_order_release);
    d.fail_group.store(group, std::memory_order_relaxed);
    d.fail_error.store(error, std::memory_order_release);
    return 0;
}

int ls_stream_run(void* h, const ls_stream_layer* layers, uint32_t count, uint32_t first_layer, void* stream,
                  uint64_t* times, uint64_t* stamps, int32_t timeout_ms) {
    if (!h || (count && !layers) || timeout_ms <= 0) return EINVAL;
    auto& d = *static_cast<StreamDecoder*>(h);
    const uint32_t n = d.setup.group_count;
    for (uint32_t i = 0; i < count; ++i)
        if (!layers[i].layout || !layers[i].input || !layers[i].output || (layers[i].rank_count && !layers[i].rank) ||
            (layers[i].final_count && !layers[i].final_ids))
            return EINVAL;
    const uint64_t origin = now_ns();
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t id = (first_layer + i) % d.setup.layers;
        const int rc = d.layer(id, layers[i], stream, origin, times ? times + 7 * static_cast<size_t>(i) : nullptr,
                               stamps ? stamps + 3 * static_cast<size_t>(n) * i : nullptr, timeout_ms);
        if (rc) return rc;
    }
    return 0;
}

}  // extern "C"
