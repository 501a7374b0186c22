// Host timing of one layer's control plane on the CPU, for the C1 shape by default (64
// groups of 64 neurons at d = 1024, 16 active): Runtime::begin_layer, the prediction update,
// the compute enqueue (a backend that launches nothing), finalize, the READY publication of
// every active group as its copy completes (the transport's callback into WeightManager and
// ExecutionQueue), completion and commit -- LeanStream's per-layer sequence
// (examples/end_to_end/main.cu:58-72) without the GPU and without the copies' own time.
//
//   control_plane_timing [groups active seconds]   -> one JSON line on stdout
//
// The transport is a stand-in IOBackend: every requested group completes at once (its state
// word READY, then the completion callback), on the calling thread.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "leanstream/runtime.h"

using namespace leanstream::runtime;

namespace {

struct InstantIO {
    IOCompletionCallback callback = nullptr;
    void* arg = nullptr;
    uint32_t epoch = 0;
    uint32_t* states = nullptr;
    uint64_t requests = 0, sequence = 0;
    std::vector<GroupId> pending;

    static InstantIO& of(void* c) { return *static_cast<InstantIO*>(c); }
    static int begin(void* c, IOCompletionCallback cb, void* arg, uint32_t epoch) {
        auto& io = of(c);
        io.callback = cb;
        io.arg = arg;
        io.epoch = epoch;
        return 0;
    }
    static int update(void* c, Span<GroupId> ids) {
        auto& io = of(c);
        io.requests += ids.size;
        for (size_t i = 0; i < ids.size; ++i) io.pending.push_back(ids[i]);
        return 0;
    }
    static int consume(void*, Span<GroupId>) { return 0; }
    static int retire(void*) { return 0; }
    static SlotId ready_slot(void*, GroupId g) { return g; }   // staging slot = logical group
    static uint64_t request_count(void* c) { return of(c).requests; }
    static int wait(void*, int) { return 0; }
    // every requested group's copy completes now, in request order
    void complete_all() {
        for (const GroupId g : pending) {
            __atomic_store_n(states + g, kIoReady, __ATOMIC_RELEASE);
            IOCompletion n{};
            n.epoch = epoch;
            n.logical_group = g;
            n.staging_slot = g;
            n.slot_sequence = ++sequence;
            callback(arg, n);
        }
        pending.clear();
    }
    IOBackend backend() {
        IOBackend b{};
        b.context = this;
        b.begin = begin;
        b.update = update;
        b.consume = consume;
        b.retire = retire;
        b.ready_slot = ready_slot;
        b.requests = request_count;
        b.wait = wait;
        return b;
    }
};

int no_enqueue(void*, uint32_t, const void*, void*, void*, Span<ExecDesc>, DeviceExecQueue, uint32_t, ConsumerMode) {
    return 0;
}
bool always_complete(void*, uint32_t) { return true; }
int commit_nothing(void*, uint32_t, Span<GroupId>) { return 0; }

}  // namespace

int main(int argc, char** argv) {
    const uint32_t groups = argc > 1 ? static_cast<uint32_t>(std::atoi(argv[1])) : 64;
    const uint32_t active = argc > 2 ? static_cast<uint32_t>(std::atoi(argv[2])) : 16;
    const double seconds = argc > 3 ? std::atof(argv[3]) : 1.0;
    const uint64_t group_bytes = 3ull * 1024 * 64 / 2;
    if (!groups || !active || active > groups || seconds <= 0) {
        std::fprintf(stderr, "usage: control_plane_timing [groups active seconds]\n");
        return 2;
    }
    std::vector<GroupLayout> layout(groups);
    std::vector<SlotId> cache(groups, -1);
    std::vector<uint32_t> states(groups + 1, 0);
    std::vector<ExecDesc> desc(groups);
    std::vector<uint32_t> indices(groups);
    QueueControl control{};
    for (uint32_t g = 0; g < groups; ++g) layout[g] = {g, g, g * group_bytes, static_cast<uint32_t>(group_bytes)};
    std::vector<GroupId> rank(active);
    for (uint32_t i = 0; i < active; ++i) rank[i] = static_cast<GroupId>((i * 37 + 11) % groups);

    InstantIO io;
    io.states = states.data();
    ManagerConfig mc{};
    mc.group_count = groups;
    mc.qd = 24;
    mc.group_bytes = group_bytes;
    mc.staging_stride = group_bytes;
    mc.alignment = 512;
    mc.mode = ConsumerMode::Progressive;
    mc.io_backend = io.backend();
    ComputeBackend cb{};
    cb.enqueue = no_enqueue;
    cb.complete = always_complete;
    cb.commit = commit_nothing;
    Runtime runtime(mc, cb);

    LayerStorage storage{};
    storage.layout = {layout.data(), groups};
    storage.cache_slots = cache.data();
    unsigned char staging_word = 0;   // the arena's address only: nothing here reads it
    storage.staging = &staging_word;
    storage.io_states = states.data();
    storage.queue = {desc.data(), indices.data(), &control, groups};

    auto one_layer = [&]() -> int {
        for (auto& w : states) w = kIoEmpty;
        LayerStep step;
        int rc = runtime.begin_layer(0, storage, &step);
        if (!rc) rc = step.update_prediction({rank.data(), rank.size()});
        if (!rc) rc = step.enqueue_compute(nullptr, nullptr, nullptr);
        if (!rc) rc = step.finalize({rank.data(), rank.size()});
        io.complete_all();
        if (!rc) rc = step.commit({});
        if (!rc && control.ready_count != active) rc = -1;
        return rc;
    };
    using clock = std::chrono::steady_clock;
    for (int i = 0; i < 100; ++i)
        if (const int rc = one_layer()) {
            std::fprintf(stderr, "layer failed: %d\n", rc);
            return 1;
        }
    const auto t0 = clock::now();
    const auto end = t0 + std::chrono::duration<double>(seconds);
    uint64_t n = 0;
    do {
        for (int i = 0; i < 256; ++i)
            if (const int rc = one_layer()) {
                std::fprintf(stderr, "layer failed: %d\n", rc);
                return 1;
            }
        n += 256;
    } while (clock::now() < end);
    const double us = std::chrono::duration<double, std::micro>(clock::now() - t0).count() / static_cast<double>(n);
    std::printf("{\"us_per_layer\": %.3f, \"layers\": %llu, \"groups\": %u, \"active\": %u, \"threads\": 1}\n", us,
                static_cast<unsigned long long>(n), groups, active);
    return 0;
}
