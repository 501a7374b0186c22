// extern "C" surface of libleanstream_hip.so (declared in include/leanstream_hip.h).
#include "leanstream_hip.h"
#include <hip/hip_runtime_api.h>
#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstring>
#include <new>
#include <numeric>
#include <thread>
#include <vector>
#include "leanstream/hip_backend.h"

using namespace leanstream::runtime;

static_assert(sizeof(ls_exec_desc) == sizeof(ExecDesc), "descriptor layout");
static_assert(sizeof(ls_device_queue) == sizeof(DeviceExecQueue), "queue view layout");
static_assert(sizeof(ls_hip_layer_buffers) == sizeof(HipLayerBuffers), "buffer block layout");

namespace {

HipBackend* backend(void* p) { return static_cast<HipBackend*>(p); }

DeviceExecQueue to_queue(const ls_device_queue& v) {
    DeviceExecQueue q;
    q.descriptors = reinterpret_cast<ExecDesc*>(v.descriptors);
    q.ready_indices = v.ready_indices;
    q.control = static_cast<QueueControl*>(v.control);
    q.capacity = v.capacity;
    return q;
}

struct Publisher {
    ExecutionQueue* queue;
    std::vector<uint32_t> order;
    std::vector<uint64_t> offset_ns;
    uint32_t fail_after, fail_code;
    std::thread thread;
    void run() {
        const auto start = std::chrono::steady_clock::now();
        const uint32_t n = static_cast<uint32_t>(order.size());
        for (uint32_t i = 0; i < n; ++i) {
            if (i == fail_after) {
                queue->fail(fail_code);
                return;
            }
            const auto due = start + std::chrono::nanoseconds(offset_ns[i]);
            while (std::chrono::steady_clock::now() < due) {
            }
            queue->publish(order[i]);
        }
        if (fail_after == n) queue->fail(fail_code);
    }
};

}  // namespace

extern "C" {

void* ls_hip_create(void) { return new (std::nothrow) HipBackend(); }
void* ls_hip_create_table(const uint8_t* entries, uint32_t layers, uint32_t buckets) {
    return new (std::nothrow) HipBackend(KernelDecisionTable{entries, layers, buckets});
}
void ls_hip_destroy(void* p) { delete backend(p); }

int ls_hip_bind(void* p, const ls_hip_layer_buffers* b) {
    if (!p || !b) return EINVAL;
    HipLayerBuffers hb;
    std::memcpy(static_cast<void*>(&hb), b, sizeof(hb));
    return backend(p)->bind(hb);
}

int ls_hip_enqueue(void* p, uint32_t layer, uint32_t bucket, uint32_t epoch, const void* input, void* output,
                   void* stream, const ls_exec_desc* core, uint32_t core_count, const ls_device_queue* queue,
                   uint32_t mode) {
    if (!p || !queue || mode > LS_MODE_AUTO) return EINVAL;
    Span<ExecDesc> c{reinterpret_cast<const ExecDesc*>(core), core_count};
    return backend(p)->enqueue({layer, bucket}, input, output, stream, c, to_queue(*queue), epoch,
                               static_cast<ConsumerMode>(mode));
}

int ls_hip_complete(void* p, uint32_t layer) {
    if (!p) return 0;
    ComputeBackend v = backend(p)->view();
    return v.complete(v.context, layer) ? 1 : 0;
}

int ls_hip_compute_backend(void* p, void* out, uint64_t out_bytes) {
    if (!p || !out || out_bytes < sizeof(ComputeBackend)) return EINVAL;
    ComputeBackend v = backend(p)->view();
    std::memcpy(out, &v, sizeof(v));
    return 0;
}

uint32_t ls_hip_status(void* p) { return p ? backend(p)->status() : 0; }
void ls_hip_clear_status(void* p) {
    if (p) backend(p)->clear_status();
}
void ls_hip_set_spin_limit(void* p, uint64_t ticks) {
    if (p) backend(p)->set_spin_limit_ticks(ticks);
}
int ls_hip_set_stage_hook(void* p, int (*arm)(void*), void* context, void* b_done) {
    if (!p) return EINVAL;
    HipBackend& b = *backend(p);
    b.arm_final_prediction = arm;
    b.arm_context = context;
    b.b_done = b_done;
    return 0;
}

int ls_hip_set_epilogue(void* p, const ls_hip_epilogue* e) {
    static_assert(sizeof(ls_hip_epilogue) == sizeof(HipEpilogue), "epilogue block");
    if (!p) return EINVAL;
    return backend(p)->set_epilogue(reinterpret_cast<const HipEpilogue*>(e));
}
int ls_hip_enqueue_chain(void* p, const ls_hip_chain_layer* layers, uint32_t count, void* stream) {
    static_assert(sizeof(ls_hip_chain_layer) == sizeof(HipChainLayer), "chain layer block");
    if (!p) return EINVAL;
    return backend(p)->enqueue_chain(reinterpret_cast<const HipChainLayer*>(layers), count, stream);
}
int ls_hip_set_chain_stamps(void* p, uint64_t* stamps, uint32_t layers) {
    return p ? backend(p)->set_chain_stamps(stamps, layers) : EINVAL;
}
uint32_t ls_hip_chain_workers(void* p) { return p ? backend(p)->chain_workers() : 0; }
uint32_t ls_hip_last_seq(void* p) { return p ? backend(p)->last_seq() : 0; }
uint32_t ls_hip_done_seq(void* p) { return p ? backend(p)->done_seq() : 0; }
uint32_t ls_hip_slices(void* p) { return p ? backend(p)->slices() : 0; }
void ls_hip_set_workers(void* p, uint32_t workers) {
    if (p) backend(p)->set_workers(workers);
}
uint32_t ls_hip_select(void* p, uint32_t layer, uint32_t bucket) {
    return p ? backend(p)->selected({layer, bucket}) : kHipDefault.id;
}
int ls_hip_last_candidate(void* p) { return p ? backend(p)->last_candidate() : -1; }
uint32_t ls_hip_max_workers(void* p) { return p ? backend(p)->max_workers() : 0; }
uint32_t ls_quantize_io_load(uint32_t remaining, uint32_t total, uint32_t buckets) {
    return quantize_io_load(remaining, total, buckets);
}

void* ls_hip_host_alloc(uint64_t bytes) {
    if (!bytes) return nullptr;
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) return nullptr;
    std::memset(p, 0, bytes);
    return p;
}
void ls_hip_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}
void ls_hip_release_u32(void* base, int64_t index, uint32_t value) {
    __atomic_store_n(static_cast<uint32_t*>(base) + index, value, __ATOMIC_RELEASE);
}
int ls_hip_acquire_all(const void* base, int32_t count, uint32_t value, int32_t timeout_ms) {
    if (!base || count < 0) return -1;
    const auto* words = static_cast<const uint32_t*>(base);
    const auto start = std::chrono::steady_clock::now();
    uint32_t spins = 0;
    for (int32_t i = 0; i < count; ++i)
        while (__atomic_load_n(words + i, __ATOMIC_ACQUIRE) != value) {
            if ((++spins & 1023u) == 0 &&
                std::chrono::steady_clock::now() - start > std::chrono::milliseconds(timeout_ms))
                return -2;
        }
    return 0;
}

void* ls_queue_create(const ls_device_queue* v) {
    if (!v) return nullptr;
    return new (std::nothrow) ExecutionQueue(to_queue(*v));
}
void ls_queue_destroy(void* q) { delete static_cast<ExecutionQueue*>(q); }
void ls_queue_reset(void* q, uint32_t epoch) { static_cast<ExecutionQueue*>(q)->reset(epoch); }
void ls_queue_prepare(void* q, uint32_t total) { static_cast<ExecutionQueue*>(q)->prepare(total); }
void ls_queue_append_unpublished(void* q, uint32_t index) { static_cast<ExecutionQueue*>(q)->append_unpublished(index); }
void ls_queue_activate(void* q) { static_cast<ExecutionQueue*>(q)->activate(); }
void ls_queue_seal(void* q, uint32_t total) { static_cast<ExecutionQueue*>(q)->seal(total); }
void ls_queue_publish_all(void* q) { static_cast<ExecutionQueue*>(q)->publish_all(); }
void ls_queue_publish(void* q, uint32_t index) { static_cast<ExecutionQueue*>(q)->publish(index); }
void ls_queue_fail(void* q, uint32_t error) { static_cast<ExecutionQueue*>(q)->fail(error); }

void* ls_publisher_start(void* q, const uint32_t* order, const uint64_t* offset_ns, uint32_t count,
                         uint32_t fail_after, uint32_t fail_code) {
    if (!q || (count && (!order || !offset_ns))) return nullptr;
    auto* pub = new (std::nothrow) Publisher;
    if (!pub) return nullptr;
    pub->queue = static_cast<ExecutionQueue*>(q);
    pub->order.assign(order, order + count);
    pub->offset_ns.assign(offset_ns, offset_ns + count);
    pub->fail_after = fail_after;
    pub->fail_code = fail_code;
    pub->thread = std::thread([pub] { pub->run(); });
    return pub;
}
int ls_publisher_join(void* p) {
    if (!p) return EINVAL;
    auto* pub = static_cast<Publisher*>(p);
    pub->thread.join();
    delete pub;
    return 0;
}

int ls_rank_groups(const float* scores, uint32_t count, uint32_t k, int32_t* out) {
    if ((count && !scores) || (k && !out) || k > count) return -1;
    for (uint32_t i = 0; i < count; ++i)
        if (!std::isfinite(scores[i])) return -3;
    std::vector<int32_t> ids(count);
    std::iota(ids.begin(), ids.end(), 0);
    // strict total order: higher score first, then lower id
    auto before = [scores](int32_t a, int32_t b) { return scores[a] > scores[b] || (scores[a] == scores[b] && a < b); };
    std::partial_sort(ids.begin(), ids.begin() + k, ids.end(), before);
    std::copy_n(ids.begin(), k, out);
    return 0;
}

}  // extern "C"
