// Control-plane trace driver (test infrastructure). The same source is compiled against
// two runtime implementations that share the LeanStream C++ API:
//   - LeanStream's own runtime sources (oracle/_ref, built by `make -C oracle ref-trace`),
//     whose output is committed as tests/golden/runtime_trace.txt;
//   - this repository's runtime (leanstream_amd/csrc/runtime), built by the CPU test,
//     whose output must equal the committed trace line for line.
// Scenarios follow the intent of LeanStream tests/open_source_runtime_test.cpp
// (queue order, descriptor construction, duplicate delivery, error paths, API schedule)
// and tests/kernel_selector_test.cpp, driven through a manual IOBackend
// (weight_manager.h IOBackend) so that every completion is delivered deterministically.
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "leanstream/execution_queue.h"
#include "leanstream/kernel_selector.h"
#include "leanstream/runtime.h"
#include "leanstream/weight_manager.h"

using namespace leanstream::runtime;

namespace {

constexpr int N = 12;       // groups
constexpr uint32_t B = 512; // group bytes

void dump_control(const char* tag, const QueueControl& c) {
    std::printf("%s control ready=%u total=%u epoch=%u batch=%u error=%u path=%u claims=%u\n", tag, c.ready_count,
                c.total_count, c.epoch, c.batch_epoch, c.error, c.consumer_path, c.claim_count);
}

void dump_indices(const char* tag, const uint32_t* idx, uint32_t n) {
    std::printf("%s ready_indices", tag);
    for (uint32_t i = 0; i < n; ++i) std::printf(" %u", idx[i]);
    std::printf("\n");
}

void dump_descs(const char* tag, const ExecDesc* d, size_t n) {
    for (size_t i = 0; i < n; ++i)
        std::printf("%s desc[%zu] logical=%u physical=%u source=%u dest=%u kind=%u\n", tag, i, d[i].logical_group,
                    d[i].physical_group, d[i].source_slot, d[i].dest_slot, static_cast<unsigned>(d[i].source_kind));
}

std::string ids_text(Span<GroupId> ids) {
    std::string s = "[";
    for (size_t i = 0; i < ids.size; ++i) s += (i ? "," : "") + std::to_string(ids[i]);
    return s + "]";
}

// IOBackend whose completions are delivered by the driver, in the driver's order.
struct Manual {
    IOCompletionCallback callback = nullptr;
    void* arg = nullptr;
    uint32_t epoch = 0;
    uint64_t requests = 0, sequence = 0;
    SlotId slot[N];
    Manual() {
        for (int g = 0; g < N; ++g) slot[g] = (g * 5 + 3) % N;
    }
    static Manual& of(void* c) { return *static_cast<Manual*>(c); }
    static int begin(void* c, IOCompletionCallback cb, void* arg, uint32_t epoch) {
        auto& m = of(c);
        m.callback = cb;
        m.arg = arg;
        m.epoch = epoch;
        std::printf("io begin epoch=%u\n", epoch);
        return 0;
    }
    static int update(void* c, Span<GroupId> ids) {
        of(c).requests += ids.size;
        std::printf("io update %s\n", ids_text(ids).c_str());
        return 0;
    }
    static int consume(void* c, Span<GroupId> ids) {
        std::printf("io consume %s\n", ids_text(ids).c_str());
        return 0;
    }
    static int retire(void*) {
        std::printf("io retire\n");
        return 0;
    }
    static SlotId ready_slot(void* c, GroupId g) { return g >= 0 && g < N ? of(c).slot[g] : -1; }
    static uint64_t request_count(void* c) { return of(c).requests; }
    static int wait(void*, int) { return 0; }
    void deliver(GroupId g, SlotId s, int error, uint32_t at_epoch) {
        IOCompletion n{};
        n.epoch = at_epoch;
        n.logical_group = g;
        n.staging_slot = s;
        n.error = error;
        n.slot_sequence = ++sequence;
        callback(arg, n);
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

struct Fixture {
    GroupLayout layout[N];
    SlotId cache[N];
    SlotId dest[N];
    uint32_t states[N + 1] = {};
    std::vector<unsigned char> staging = std::vector<unsigned char>(N * B);
    ExecDesc desc[N] = {};
    uint32_t indices[N] = {};
    QueueControl control{};
    Manual io;
    Fixture() {
        for (int i = 0; i < N; ++i) {
            layout[i] = {static_cast<uint32_t>(i), static_cast<uint32_t>(N - 1 - i), static_cast<uint64_t>(N - 1 - i) * B, B};
            cache[i] = -1;
            dest[i] = (i * 7 + 3) % N;
        }
        cache[0] = 7;
        cache[5] = 2;
    }
    LayerStorage storage(Span<GroupId> core, uint32_t capacity = N, bool with_dest = false) {
        LayerStorage s{};
        s.fd = -1;
        s.layout = {layout, N};
        s.cache_slots = cache;
        s.staging = staging.data();
        s.io_states = states;
        s.core = core;
        s.queue = {desc, indices, &control, capacity};
        s.destination_slots = with_dest ? dest : nullptr;
        return s;
    }
    ManagerConfig config() {
        ManagerConfig c{};
        c.group_count = N;
        c.qd = 1;
        c.group_bytes = B;
        c.staging_stride = B;
        c.alignment = 512;
        c.mode = ConsumerMode::Progressive;
        c.io_backend = io.backend();
        return c;
    }
};

void queue_scenarios() {
    std::printf("== queue\n");
    ExecDesc desc[N] = {};
    uint32_t idx[N] = {};
    QueueControl c{};
    ExecutionQueue q({desc, idx, &c, N});
    q.reset(7);
    q.seal(4);
    for (uint32_t i : {2u, 0u, 3u, 1u}) q.publish(i);
    dump_control("q1", c);
    dump_indices("q1", idx, 4);
    q.reset(8);
    q.seal(0);
    dump_control("q2", c);
    q.reset(9);
    q.prepare(5);
    q.append_unpublished(3);
    q.append_unpublished(0);
    q.activate();
    dump_control("q3a", c);
    q.publish(4);
    q.publish(1);
    dump_control("q3b", c);
    q.fail(5);
    q.fail(7);
    dump_control("q3c", c);
    q.publish(2);
    dump_control("q3d", c);
    dump_indices("q3d", idx, 5);
    q.reset(10);
    q.seal(3);
    q.publish_all();
    dump_control("q4", c);
    dump_indices("q4", idx, 3);
}

void manager_scenarios() {
    std::printf("== manager\n");
    Fixture f;
    WeightManager m(f.config());
    GroupId core[] = {0};
    int rc = m.begin_layer(0, f.storage({core, 1}));
    std::printf("m1 begin rc=%d epoch=%u\n", rc, m.epoch());
    dump_descs("m1 core", m.core_descriptors().data, m.core_descriptors().size);
    GroupId p0[] = {0, 1, 2, 3, 1, 5, 7};
    rc = m.update_prediction({p0, 7});
    std::printf("m1 update rc=%d gen=%llu\n", rc, static_cast<unsigned long long>(m.prediction_generation()));
    f.states[2] = 1;  // in flight
    f.states[3] = 2;  // ready
    GroupId p1[] = {3, 2, 8};
    rc = m.update_prediction({p1, 3});
    std::printf("m1 update rc=%d\n", rc);
    PredictionUpdateOptions budget{};
    budget.io_budget = 1;
    GroupId p2[] = {9, 10, 11};
    rc = m.update_prediction({p2, 3}, budget);
    std::printf("m1 update budget rc=%d\n", rc);
    PredictionUpdateOptions stale{};
    stale.execution_epoch = m.epoch() + 5;
    rc = m.update_prediction({p2, 3}, stale);
    std::printf("m1 update stale rc=%d\n", rc);
    GroupId bad[] = {99};
    rc = m.update_prediction({bad, 1});
    std::printf("m1 update bad rc=%d gen=%llu\n", rc, static_cast<unsigned long long>(m.prediction_generation()));
    for (GroupId g : {0, 2, 3, 4}) {
        GroupState s = m.group_state(g);
        std::printf("m1 state g=%d cache=%d staging=%d io=%u\n", g, s.cache_slot, s.staging_slot,
                    static_cast<unsigned>(s.io_state));
    }
    GroupId final[] = {0, 1, 3, 5, 8};
    rc = m.finalize({final, 5});
    std::printf("m1 finalize rc=%d\n", rc);
    dump_control("m1 after-finalize", f.control);
    dump_indices("m1 after-finalize", f.indices, f.control.ready_count);
    dump_descs("m1 after-finalize", f.desc, f.control.total_count);
    rc = m.finalize({final, 5});
    const int rc2 = m.update_prediction({p1, 3});
    std::printf("m1 finalize again rc=%d update rc=%d\n", rc, rc2);
    f.states[8] = 2;
    f.io.deliver(8, 4, 0, f.io.epoch);
    f.states[1] = 2;
    f.io.deliver(1, 6, 0, f.io.epoch);
    f.io.deliver(8, 4, 0, f.io.epoch);          // duplicate delivery: no republication
    f.io.deliver(3, 9, 0, f.io.epoch - 1);      // stale epoch: ignored
    dump_control("m1 delivered", f.control);
    dump_indices("m1 delivered", f.indices, f.control.ready_count);
    dump_descs("m1 delivered", f.desc, f.control.total_count);
    rc = m.retire();
    std::printf("m1 retire rc=%d requests=%llu\n", rc, static_cast<unsigned long long>(m.read_requests()));
    for (int g = 0; g <= N; ++g) f.states[g] = 0;

    // destination slots, then an I/O error and a later cancel (first error wins)
    rc = m.begin_layer(1, f.storage({core, 1}, N, true));
    std::printf("m2 begin rc=%d epoch=%u\n", rc, m.epoch());
    dump_descs("m2 core", m.core_descriptors().data, m.core_descriptors().size);
    GroupId f2[] = {6, 0, 11, 4};
    rc = m.finalize({f2, 4});
    std::printf("m2 finalize rc=%d\n", rc);
    dump_descs("m2 after-finalize", f.desc, f.control.total_count);
    dump_control("m2 after-finalize", f.control);
    f.io.deliver(11, 1, 0, f.io.epoch);
    f.io.deliver(4, 0, EIO, f.io.epoch);
    m.cancel(ECANCELED);
    dump_control("m2 failed", f.control);
    dump_indices("m2 failed", f.indices, f.control.ready_count);
    rc = m.retire();
    std::printf("m2 retire rc=%d\n", rc);

    // argument errors
    rc = m.begin_layer(2, f.storage({core, 1}));
    std::printf("m3 begin rc=%d\n", rc);
    GroupId dup[] = {0, 1, 1};
    GroupId out[] = {0, 12};
    GroupId no_core[] = {1, 2};
    const int r_dup = m.finalize({dup, 3});
    const int r_out = m.finalize({out, 2});
    const int r_nocore = m.finalize({no_core, 2});
    std::printf("m3 finalize dup=%d out=%d nocore=%d\n", r_dup, r_out, r_nocore);
    rc = m.retire();
    std::printf("m3 retire rc=%d\n", rc);
    GroupId uncached_core[] = {1};
    rc = m.begin_layer(3, f.storage({uncached_core, 1}));
    std::printf("m4 begin uncached core rc=%d\n", rc);
    rc = m.begin_layer(3, f.storage({core, 1}, 2));
    std::printf("m5 begin small queue rc=%d\n", rc);
    GroupId f5[] = {0, 1, 2, 3};
    rc = m.finalize({f5, 4});
    std::printf("m5 finalize rc=%d\n", rc);
    rc = m.retire();
    std::printf("m5 retire rc=%d epoch=%u\n", rc, m.epoch());
    rc = m.retire();
    std::printf("m6 retire idle rc=%d\n", rc);
}

void selector_scenarios() {
    std::printf("== selector\n");
    uint8_t lut[3 * 8];
    for (uint32_t l = 0; l < 3; ++l)
        for (uint32_t b = 0; b < 8; ++b) lut[l * 8 + b] = static_cast<uint8_t>((l * 3 + b) % 5);
    KernelSelector s({lut, 3, 8});
    std::printf("s1");
    for (uint32_t l = 0; l < 4; ++l)
        for (uint32_t b = 0; b < 9; ++b) std::printf(" %u", s.select(l, b));
    std::printf("\n");
    std::printf("s2 default=%u plan_workers=%u\n", KernelSelector{}.select(0, 0), KernelSelector{}.plan({0, 0}).candidate.workers);
    const uint8_t bad[] = {255, 0, 1, 2, 3, 4};
    KernelCandidate candidates[5];
    for (int i = 0; i < 5; ++i) candidates[i] = kKernelCandidates[i];
    candidates[0].available = false;
    candidates[1].workers = 0;
    candidates[3].id = 99;
    KernelSelector invalid({bad, 1, 6}, {candidates, 5});
    std::printf("s3");
    for (uint32_t b = 0; b < 6; ++b) std::printf(" %u", invalid.select(0, b));
    std::printf(" candidate255.workers=%u\n", invalid.candidate(255).workers);
    std::printf("s4 empty-catalog=%u\n", KernelSelector({bad + 5, 1, 1}, {nullptr, 0}).select(0, 0));
    const uint32_t big = 0xffffffffu;
    std::printf("s5 q %u %u %u %u %u %u %u %u\n", quantize_io_load(1, 1), quantize_io_load(10, 8), quantize_io_load(0, 0),
                quantize_io_load(1, 0), quantize_io_load(1, 8, 0), quantize_io_load(0, 8), quantize_io_load(big - 1, big),
                quantize_io_load(big - 1, big, big));
    std::printf("s6");
    for (uint32_t r = 0; r <= 20; ++r) std::printf(" %u", quantize_io_load(r, 17, 5));
    std::printf("\n");
}

struct FakeGpu {
    int launches = 0;
    bool done = false;
    int fail = 0;
};
int fake_enqueue(void* p, uint32_t layer, const void*, void*, void*, Span<ExecDesc> core, DeviceExecQueue q,
                 uint32_t epoch, ConsumerMode mode) {
    auto& g = *static_cast<FakeGpu*>(p);
    ++g.launches;
    std::printf("gpu enqueue layer=%u core=%zu epoch=%u control_epoch=%u mode=%u\n", layer, core.size, epoch,
                q.control->epoch, static_cast<unsigned>(mode));
    return g.fail;
}
bool fake_complete(void* p, uint32_t) { return static_cast<FakeGpu*>(p)->done; }
int fake_commit(void*, uint32_t layer, Span<GroupId> ids) {
    std::printf("gpu commit layer=%u ids=%s\n", layer, ids_text(ids).c_str());
    return 0;
}

void runtime_scenarios() {
    std::printf("== runtime\n");
    Fixture f;
    FakeGpu gpu;
    ComputeBackend cb{};
    cb.context = &gpu;
    cb.enqueue = fake_enqueue;
    cb.complete = fake_complete;
    cb.commit = fake_commit;
    Runtime r(f.config(), cb);
    LayerStep step;
    GroupId core[] = {0}, pred[] = {1, 2}, final[] = {0, 1, 2};
    auto show = [](const char* what, int rc) { std::printf("%s rc=%d\n", what, rc); };
    show("r1 begin", r.begin_layer(0, f.storage({core, 1}), &step));
    show("r1 update", step.update_prediction({pred, 2}));
    show("r1 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
    show("r1 update", step.update_prediction({pred, 2}));
    show("r1 finalize", step.finalize({final, 3}));
    dump_control("r1 finalized", f.control);
    show("r1 update-after-finalize", step.update_prediction({pred, 2}));
    show("r1 commit-while-busy", step.commit({final, 3}));
    f.states[1] = 2;
    f.io.deliver(1, 5, 0, f.io.epoch);
    f.states[2] = 2;
    f.io.deliver(2, 9, 0, f.io.epoch);
    dump_control("r1 delivered", f.control);
    dump_indices("r1 delivered", f.indices, f.control.ready_count);
    show("r1 commit-while-busy", step.commit({final, 3}));
    gpu.done = true;
    show("r1 commit", step.commit({final, 3}));
    show("r1 finalize-after-commit", step.finalize({final, 3}));
    std::printf("r1 launches=%d\n", gpu.launches);
    for (int g = 0; g <= N; ++g) f.states[g] = 0;
    LayerStep old = step;
    gpu.done = false;
    show("r2 begin", r.begin_layer(0, f.storage({core, 1}), &step));
    show("r2 old-step-update", old.update_prediction({pred, 2}));
    show("r2 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
    show("r2 abort-while-busy", step.abort());
    dump_control("r2 aborting", f.control);
    gpu.done = true;
    show("r2 abort", step.abort());
    gpu.fail = EIO;
    gpu.done = false;
    show("r3 begin", r.begin_layer(0, f.storage({core, 1}), &step));
    show("r3 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
    show("r3 abort-while-busy", step.abort());
    dump_control("r3 failed", f.control);
    gpu.done = true;
    show("r3 abort", step.abort());
    std::printf("r3 launches=%d\n", gpu.launches);
}

}  // namespace

// Layout registration and plan reuse, prepare-time validation order, finalize's prefix
// errors and completions that must not publish.
void manager_more_scenarios() {
    std::printf("== manager-more\n");
    Fixture f;
    WeightManager m(f.config());
    GroupId core[] = {0};
    auto show = [](const char* what, int rc) { std::printf("%s rc=%d\n", what, rc); };
    LayerStorage s = f.storage({core, 1});
    s.layout.size = N - 1;
    show("p1 short layout", m.prepare_layer(s));
    s = f.storage({core, 1});
    s.staging_bytes = N * B - 1;
    show("p2 small staging", m.prepare_layer(s));
    s.staging_bytes = N * B;
    show("p3 exact staging", m.prepare_layer(s));
    f.layout[3].logical_group = 2;
    show("p4 duplicate layout", m.prepare_layer(f.storage({core, 1})));
    f.layout[3].logical_group = 3;
    f.layout[4].bytes = B + 1;
    show("p5 group bytes", m.prepare_layer(f.storage({core, 1})));
    f.layout[4].bytes = B;
    GroupId twice[] = {0, 0}, outside[] = {N}, pair[] = {0, 5};
    show("p6 core twice", m.prepare_layer(f.storage({twice, 2})));
    show("p7 core outside", m.prepare_layer(f.storage({outside, 1})));
    const SlotId keep = f.dest[5];
    f.dest[5] = f.dest[0];
    show("p8 core dest clash", m.prepare_layer(f.storage({pair, 2}, N, true)));
    f.dest[5] = keep;
    s = f.storage({core, 1});
    s.io_states = nullptr;
    show("p9 no io states", m.prepare_layer(s));
    show("p10 big queue", m.prepare_layer(f.storage({core, 1}, N + 1)));
    show("p11 core pair", m.prepare_layer(f.storage({pair, 2}, N, true)));
    dump_descs("p11 core", m.core_descriptors().data, m.core_descriptors().size);

    // registered layout (generation 7): a later begin with the same generation and pointer
    // keeps the registration, so edits of the immutable layout are not seen
    s = f.storage({core, 1});
    s.layout_generation = 7;
    show("g1 begin", m.begin_layer(0, s));
    dump_descs("g1 core", m.core_descriptors().data, m.core_descriptors().size);
    show("g1 begin-while-active", m.begin_layer(0, s));
    show("g1 prepare-while-active", m.prepare_layer(s));
    show("g1 retire", m.retire());
    f.layout[0].physical_group = 3;
    show("g2 begin same generation", m.begin_layer(0, s));
    dump_descs("g2 core", m.core_descriptors().data, m.core_descriptors().size);
    show("g2 retire", m.retire());
    s.layout_generation = 8;
    show("g3 begin new generation", m.begin_layer(0, s));
    dump_descs("g3 core", m.core_descriptors().data, m.core_descriptors().size);
    show("g3 retire", m.retire());
    f.layout[0].physical_group = N - 1;

    // prepared plan (generation 3) reused only when every binding matches
    s = f.storage({pair, 2}, N, true);
    s.plan_generation = 3;
    show("q1 prepare", m.prepare_layer(s));
    f.cache[5] = 4;   // not seen when the prepared plan is reused
    show("q1 begin reuse", m.begin_layer(1, s));
    dump_descs("q1 core", m.core_descriptors().data, m.core_descriptors().size);
    show("q1 retire", m.retire());
    s.staging_bytes = N * B;   // a different binding: prepared again
    show("q2 begin changed", m.begin_layer(1, s));
    dump_descs("q2 core", m.core_descriptors().data, m.core_descriptors().size);
    show("q2 retire", m.retire());
    f.cache[5] = 2;

    // argument and state errors of update / finalize
    show("u1 update idle", m.update_prediction({core, 1}));
    show("u1 finalize idle", m.finalize({core, 1}));
    show("u2 begin", m.begin_layer(2, f.storage({pair, 2})));
    show("u2 update null", m.update_prediction({nullptr, 2}));
    show("u2 finalize short", m.finalize({core, 1}));
    show("u2 finalize null", m.finalize({nullptr, 3}));
    GroupId early[] = {0, 5, 6};
    f.states[6] = 2;
    f.io.deliver(6, 8, 0, f.io.epoch);   // before finalize: no plan, nothing published
    dump_control("u2 early delivery", f.control);
    f.io.slot[6] = -1;                   // READY at finalize but the transport has no slot
    show("u2 finalize bad ready slot", m.finalize({early, 3}));
    dump_control("u2 failed", f.control);
    show("u2 retire", m.retire());
    f.io.slot[6] = (6 * 5 + 3) % N;
    f.states[6] = 0;
    show("u3 begin", m.begin_layer(3, f.storage({core, 1}, N, true)));
    GroupId clash[] = {0, 1, 9};
    f.dest[9] = f.dest[1];
    show("u3 finalize dest clash", m.finalize({clash, 3}));
    f.dest[9] = (9 * 7 + 3) % N;
    show("u3 finalize", m.finalize({clash, 3}));
    dump_descs("u3 after-finalize", f.desc, f.control.total_count);
    f.io.deliver(9, N, 0, f.io.epoch);   // slot outside the staging arena: the queue fails
    dump_control("u3 bad slot", f.control);
    show("u3 retire", m.retire());
}

struct DeferringGpu {
    void (*retired)(void*, uint32_t) = nullptr;
    void* context = nullptr;
    uint32_t epoch = 0;
    bool done = false;
};
int deferring_enqueue(void*, uint32_t layer, const void*, void*, void*, Span<ExecDesc> core, DeviceExecQueue,
                      uint32_t epoch, ConsumerMode) {
    std::printf("gpu enqueue layer=%u core=%zu epoch=%u\n", layer, core.size, epoch);
    return 0;
}
bool deferring_complete(void* p, uint32_t) { return static_cast<DeferringGpu*>(p)->done; }
int deferring_commit(void* p, uint32_t layer, Span<GroupId> ids, uint32_t epoch, void (*retired)(void*, uint32_t),
                     void* context) {
    auto& g = *static_cast<DeferringGpu*>(p);
    g.retired = retired;
    g.context = context;
    g.epoch = epoch;
    std::printf("gpu defer_commit layer=%u ids=%s epoch=%u\n", layer, ids_text(ids).c_str(), epoch);
    return 0;
}
void deferring_cancel(void*, uint32_t layer, uint32_t epoch) { std::printf("gpu cancel layer=%u epoch=%u\n", layer, epoch); }

// Deferred commit (retirement from the backend's callback), commit's check order, a
// finalize failure after the launch, and lifecycle argument errors.
void runtime_more_scenarios() {
    std::printf("== runtime-more\n");
    auto show = [](const char* what, int rc) { std::printf("%s rc=%d\n", what, rc); };
    {
        Fixture f;
        DeferringGpu gpu;
        ComputeBackend cb{};
        cb.context = &gpu;
        cb.enqueue = deferring_enqueue;
        cb.complete = deferring_complete;
        cb.defer_commit = deferring_commit;
        cb.cancel = deferring_cancel;
        Runtime r(f.config(), cb, 2);
        LayerStep step, other;
        GroupId core[] = {0}, final[] = {0, 1, 2}, next[] = {1};
        show("d1 begin bad layer", r.begin_layer(2, f.storage({core, 1}), &step));
        show("d1 begin null step", r.begin_layer(0, f.storage({core, 1}), nullptr));
        show("d1 begin", r.begin_layer(0, f.storage({core, 1}), &step));
        show("d1 begin again", r.begin_layer(0, f.storage({core, 1}), &other));
        show("d1 commit-unfinalized", step.commit({next, 1}));
        show("d1 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
        show("d1 enqueue again", step.enqueue_compute(nullptr, nullptr, nullptr));
        show("d1 finalize", step.finalize({final, 3}));
        show("d1 commit", step.commit({next, 1}));
        show("d1 commit-pending", step.commit({next, 1}));
        show("d1 abort-pending", step.abort());
        show("d1 begin-pending", r.begin_layer(0, f.storage({core, 1}), &other));
        gpu.retired(gpu.context, gpu.epoch + 1);   // another epoch: ignored
        show("d1 begin-still-pending", r.begin_layer(0, f.storage({core, 1}), &other));
        gpu.retired(gpu.context, gpu.epoch);
        gpu.retired(gpu.context, gpu.epoch);       // twice: ignored
        show("d1 drain", r.drain());
        show("d1 begin-after-retire", r.begin_layer(0, f.storage({core, 1}), &step));
        show("d1 abort-unlaunched", step.abort());
        show("d1 drain", r.drain());
    }
    {
        Fixture f;
        FakeGpu gpu;
        ComputeBackend cb{};
        cb.context = &gpu;
        cb.enqueue = fake_enqueue;
        cb.complete = fake_complete;
        cb.commit = fake_commit;
        Runtime r(f.config(), cb);
        LayerStep step;
        GroupId core[] = {0}, final[] = {0, 1, 2}, big[N + 1] = {}, outside[] = {N}, twice[] = {1, 1},
                unready[] = {1}, unready_then_outside[] = {1, N}, outside_then_unready[] = {N, 1};
        show("c1 begin", r.begin_layer(0, f.storage({core, 1}), &step));
        show("c1 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
        show("c1 finalize", step.finalize({final, 3}));
        show("c1 commit too many", step.commit({big, N + 1}));
        show("c1 commit null", step.commit({nullptr, 1}));
        show("c1 commit while busy", step.commit({outside, 1}));
        gpu.done = true;
        show("c1 commit outside", step.commit({outside, 1}));
        show("c1 commit twice", step.commit({twice, 2}));
        show("c1 commit unready", step.commit({unready, 1}));
        show("c1 commit unready-then-outside", step.commit({unready_then_outside, 2}));
        show("c1 commit outside-then-unready", step.commit({outside_then_unready, 2}));
        f.states[1] = 2;
        f.io.deliver(1, 5, 0, f.io.epoch);
        f.states[2] = 2;
        f.io.deliver(2, 9, 0, f.io.epoch);
        r.weights(0).cancel(EIO);             // a queue error: commit reports it first
        show("c1 commit after queue error", step.commit({unready, 1}));
        show("c1 abort", step.abort());
        for (int g = 0; g <= N; ++g) f.states[g] = 0;
        gpu.done = false;
        // finalize fails after the launch: the manager and the backend are cancelled
        show("c2 begin", r.begin_layer(0, f.storage({core, 1}), &step));
        show("c2 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
        GroupId bad[] = {0, 1, 1};
        show("c2 finalize dup", step.finalize({bad, 3}));
        dump_control("c2 cancelled", f.control);
        show("c2 finalize again", step.finalize({final, 3}));
        show("c2 commit", step.commit({core, 1}));
        show("c2 abort-while-busy", step.abort());
        gpu.done = true;
        show("c2 abort", step.abort());
        // a backend without commit: ENOTSUP, the step stays open until abort
        cb.commit = nullptr;
        Runtime bare(f.config(), cb);
        show("c3 begin", bare.begin_layer(0, f.storage({core, 1}), &step));
        show("c3 enqueue", step.enqueue_compute(nullptr, nullptr, nullptr));
        GroupId only[] = {0};
        show("c3 finalize", step.finalize({only, 1}));
        show("c3 commit", step.commit({}));
        show("c3 abort", step.abort());
    }
}

int main() {
    queue_scenarios();
    manager_scenarios();
    selector_scenarios();
    runtime_scenarios();
    manager_more_scenarios();
    runtime_more_scenarios();
    std::printf("== end\n");
    return 0;
}
