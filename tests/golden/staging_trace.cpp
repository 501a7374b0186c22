// I/O admission and readiness trace of a WeightManager driven through its transport.
//
// Built two ways, printing the same canonical trace:
//   * default: this repository's WeightManager + HostStagingIO, with a copy engine
//     whose copies are held, released or failed by the script;
//   * -DLS_TRACE_REFERENCE: LeanStream's WeightManager on its built-in O_DIRECT engine
//     (src/io/stream_io.cpp built with -DSTREAM_TESTING), whose reads go through
//     stream_test_pread below, held, released or failed by the same script
//     (the reference's own hook, tests/open_source_runtime_test.cpp:21-29).
// Every step waits until the transport has settled (the expected number of reads or
// copies started, the expected ready count), so the trace is deterministic: group
// states, staging slots, read requests, queue words, publication order, descriptors,
// return codes and a checksum of every staged slot.
#include "leanstream/weight_manager.h"
#ifndef LS_TRACE_REFERENCE
#include "leanstream/host_staging_io.h"
#endif
#include <fcntl.h>
#include <unistd.h>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

using namespace leanstream::runtime;

namespace {

constexpr uint32_t N = 8, QD = 2;
constexpr uint32_t B = 4096;
// io_states words (stream_io.h:8): EMPTY 0, INFLIGHT 1, READY 2, ERROR 3
constexpr uint32_t kReadyWord = 2, kErrorWord = 3;

uint8_t* store = nullptr;  // the packed groups, as on storage: group i at (N-1-i)*B
std::mutex gate_mutex;
std::condition_variable gate_cv;
bool hold[N];
int fail[N];
int started = 0;

void hold_all() {
    std::lock_guard<std::mutex> lock(gate_mutex);
    for (uint32_t g = 0; g < N; ++g) hold[g] = true;
}
void release(uint32_t g, int error = 0) {
    std::lock_guard<std::mutex> lock(gate_mutex);
    hold[g] = false;
    fail[g] = error;
    gate_cv.notify_all();
}
int started_count() {
    std::lock_guard<std::mutex> lock(gate_mutex);
    return started;
}
void await_started(int n) {
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(5);
    while (started_count() < n) {
        if (std::chrono::steady_clock::now() > deadline) {
            std::printf("timeout waiting for %d started (have %d)\n", n, started_count());
            std::exit(1);
        }
        std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
    // nothing else can start: the expected count is the most the queue depth allows
    std::this_thread::sleep_for(std::chrono::milliseconds(20));
    if (started_count() != n) {
        std::printf("unexpected start count %d (expected %d)\n", started_count(), n);
        std::exit(1);
    }
}

}  // namespace

#ifdef LS_TRACE_REFERENCE
extern "C" ssize_t stream_test_pread(int, void* bytes, size_t n, off_t offset) {
    const uint32_t g = N - 1 - static_cast<uint32_t>(offset / B);
    std::unique_lock<std::mutex> lock(gate_mutex);
    ++started;
    gate_cv.notify_all();
    gate_cv.wait(lock, [&] { return !hold[g]; });
    if (fail[g]) {
        errno = fail[g];
        return -1;
    }
    std::memcpy(bytes, store + offset, n);
    return static_cast<ssize_t>(n);
}
#else
struct HeldCopies {
    struct Lane {
        uint8_t* dst;
        const uint8_t* src;
        uint64_t bytes;
        uint32_t group;
    } lanes[32];
    static int submit(void* c, uint32_t lane, void* dst, const void* src, uint64_t bytes) {
        auto& h = *static_cast<HeldCopies*>(c);
        const auto* s = static_cast<const uint8_t*>(src);
        std::lock_guard<std::mutex> lock(gate_mutex);
        h.lanes[lane] = {static_cast<uint8_t*>(dst), s, bytes, N - 1 - static_cast<uint32_t>((s - store) / B)};
        ++started;
        gate_cv.notify_all();
        return 0;
    }
    static int poll(void* c, uint32_t lane) {
        auto& h = *static_cast<HeldCopies*>(c);
        std::lock_guard<std::mutex> lock(gate_mutex);
        const Lane& l = h.lanes[lane];
        if (hold[l.group]) return EAGAIN;
        if (fail[l.group]) return fail[l.group];
        std::memcpy(l.dst, l.src, l.bytes);
        return 0;
    }
};
#endif

namespace {

struct Fixture {
    int fd = -1;
    char path[64] = "/tmp/leanstream-staging-trace-XXXXXX";
    void* arena = nullptr;
    SlotId cache[N];
    uint32_t states[N + 1]{};
    GroupLayout layout[N];
    ExecDesc desc[N]{};
    uint32_t indices[N]{};
    QueueControl control{};
    Fixture() {
        store = static_cast<uint8_t*>(std::aligned_alloc(4096, N * B));
        for (uint32_t i = 0; i < N; ++i) {
            layout[i] = {i, N - 1 - i, uint64_t(N - 1 - i) * B, B};
            cache[i] = -1;
            for (uint32_t j = 0; j < B; ++j) store[(N - 1 - i) * B + j] = static_cast<uint8_t>(i * 37 + j * 11);
        }
        cache[7] = 5;  // one group already resident in the device cache
        fd = mkstemp(path);
        if (fd < 0 || write(fd, store, N * B) != static_cast<ssize_t>(N * B) ||
            fcntl(fd, F_SETFL, fcntl(fd, F_GETFL) | O_DIRECT)) {
            std::printf("fixture file failed\n");
            std::exit(1);
        }
        arena = std::aligned_alloc(4096, N * B);
        std::memset(arena, 0, N * B);
    }
    ~Fixture() {
        close(fd);
        unlink(path);
        std::free(arena);
        std::free(store);
    }
    LayerStorage storage() { return {fd, {layout, N}, cache, arena, states, {}, {desc, indices, &control, N}}; }
};

const char* state_name(IOState s) { return s == IOState::Ready ? "R" : s == IOState::Inflight ? "I" : "E"; }

void print_groups(const char* tag, WeightManager& m, const Fixture& f) {
    std::printf("%s groups", tag);
    for (uint32_t g = 0; g < N; ++g) {
        const GroupState s = m.group_state(static_cast<GroupId>(g));
        std::printf(" %u:%s/%d/%d/w%u", g, state_name(s.io_state), s.cache_slot, s.staging_slot,
                    __atomic_load_n(f.states + g, __ATOMIC_ACQUIRE));
    }
    std::printf(" term=%u requests=%llu\n", __atomic_load_n(f.states + N, __ATOMIC_ACQUIRE),
                static_cast<unsigned long long>(m.read_requests()));
}

void print_queue(const char* tag, const Fixture& f) {
    const QueueControl& c = f.control;
    const uint32_t ready = __atomic_load_n(&c.ready_count, __ATOMIC_ACQUIRE);
    std::printf("%s queue ready=%u total=%u epoch=%u error=%u order=[", tag, ready, c.total_count, c.epoch, c.error);
    for (uint32_t i = 0; i < ready && i < N; ++i) std::printf(i ? ",%u" : "%u", f.indices[i]);
    std::printf("]\n");
    for (uint32_t i = 0; i < c.total_count && i < N; ++i) {
        const ExecDesc& d = f.desc[i];
        std::printf("%s   desc %u = {%u,%u,%u,%u,%u}\n", tag, i, d.logical_group, d.physical_group, d.source_slot,
                    d.dest_slot, static_cast<uint32_t>(d.source_kind));
    }
}

void print_slots(const char* tag, const Fixture& f) {
    std::printf("%s slots", tag);
    for (uint32_t g = 0; g < N; ++g) {
        if (__atomic_load_n(f.states + g, __ATOMIC_ACQUIRE) != kReadyWord) continue;
        uint32_t sum = 0;
        const auto* p = static_cast<const uint8_t*>(f.arena) + g * B;
        for (uint32_t j = 0; j < B; ++j) sum = sum * 31 + p[j];
        std::printf(" %u:%08x", g, sum);
    }
    std::printf("\n");
}

void await_ready(const Fixture& f, uint32_t n) {
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(5);
    while (__atomic_load_n(&f.control.ready_count, __ATOMIC_ACQUIRE) < n) {
        if (std::chrono::steady_clock::now() > deadline) {
            std::printf("timeout waiting for ready_count %u\n", n);
            std::exit(1);
        }
        std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
}

void await_state(const Fixture& f, uint32_t g, uint32_t word) {
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(5);
    while (__atomic_load_n(f.states + g, __ATOMIC_ACQUIRE) != word) {
        if (std::chrono::steady_clock::now() > deadline) {
            std::printf("timeout waiting for group %u state %u\n", g, word);
            std::exit(1);
        }
        std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
}

}  // namespace

int main() {
    Fixture f;
    ManagerConfig config{N, QD, B, B, 512, ConsumerMode::Progressive};
#ifndef LS_TRACE_REFERENCE
    HeldCopies copies;
    StagingConfig sc;
    sc.group_count = N;
    sc.qd = QD;
    sc.group_bytes = B;
    sc.staging_stride = B;
    sc.engine = {&copies, HeldCopies::submit, HeldCopies::poll};
    HostStagingIO io(sc);
    StagingLayer layer;
    layer.source = store;
    layer.source_bytes = N * B;
    layer.layout = {f.layout, N};
    layer.staging = static_cast<uint8_t*>(f.arena);
    layer.staging_bytes = N * B;
    layer.io_states = f.states;
    config.io_backend = io.backend();
    auto bind = [&] { return io.bind_layer(layer); };
#else
    auto bind = [] { return 0; };
#endif
    WeightManager m(config);
    LayerStorage s = f.storage();

    // 1. rank replacement with a full queue depth, non-preemptive in-flight reads
    std::printf("== replacement\n");
    hold_all();
    int rc = bind();
    std::printf("bind rc=%d\n", rc);
    rc = m.begin_layer(0, s);
    std::printf("begin rc=%d epoch=%u\n", rc, m.epoch());
    print_groups("a", m, f);
    GroupId p0[] = {3, 1, 5, 7};
    rc = m.update_prediction({p0, 4});
    await_started(2);
    std::printf("update [3,1,5,7] rc=%d gen=%llu\n", rc, static_cast<unsigned long long>(m.prediction_generation()));
    print_groups("b", m, f);
    GroupId p1[] = {6, 5, 1};
    rc = m.update_prediction({p1, 3});
    std::printf("update [6,5,1] rc=%d\n", rc);
    print_groups("c", m, f);
    release(3);
    await_state(f, 3, kReadyWord);
    await_started(3);
    std::printf("released 3\n");
    print_groups("d", m, f);
    GroupId final0[] = {1, 3, 7, 6, 2};
    rc = m.finalize({final0, 5});
    std::printf("finalize [1,3,7,6,2] rc=%d\n", rc);
    print_queue("e", f);
    print_groups("e", m, f);
    release(1);
    await_ready(f, 3);
    await_started(4);
    std::printf("released 1\n");
    print_queue("f", f);
    print_groups("f", m, f);
    release(2);
    await_ready(f, 4);
    release(6);
    await_ready(f, 5);
    std::printf("released 2, 6\n");
    rc = m.wait_io(2000);
    std::printf("wait rc=%d\n", rc);
    print_queue("g", f);
    print_groups("g", m, f);
    print_slots("g", f);
    rc = m.retire();
    std::printf("retire rc=%d requests=%llu\n", rc, static_cast<unsigned long long>(m.read_requests()));

    // 2. a failed read: terminal error word, no further admissions, queue error
    std::printf("== failure\n");
    hold_all();
    {
        std::lock_guard<std::mutex> lock(gate_mutex);
        started = 0;
    }
    rc = bind();
    rc = m.begin_layer(0, s);
    std::printf("begin rc=%d epoch=%u\n", rc, m.epoch());
    GroupId p2[] = {0, 4, 2};
    rc = m.update_prediction({p2, 3});
    await_started(2);
    std::printf("update [0,4,2] rc=%d\n", rc);
    print_groups("h", m, f);
    release(0);
    await_state(f, 0, kReadyWord);
    await_started(3);
    release(4, EIO);
    await_state(f, 4, kErrorWord);
    std::printf("released 0, failed 4\n");
    print_groups("i", m, f);
    GroupId p3[] = {5};
    rc = m.update_prediction({p3, 1});
    std::printf("update after error rc=%d\n", rc);
    GroupId final1[] = {0, 5};
    rc = m.finalize({final1, 2});
    std::printf("finalize [0,5] rc=%d\n", rc);
    print_queue("j", f);
    release(2);
    await_state(f, 2, kReadyWord);
    rc = m.wait_io(2000);
    std::printf("wait rc=%d\n", rc);
    print_groups("j", m, f);
    rc = m.retire();
    std::printf("retire rc=%d requests=%llu\n", rc, static_cast<unsigned long long>(m.read_requests()));

    // 3. recovery: a new epoch clears the terminal word
    std::printf("== recovery\n");
    hold_all();
    {
        std::lock_guard<std::mutex> lock(gate_mutex);
        started = 0;
        for (uint32_t g = 0; g < N; ++g) fail[g] = 0;
    }
    rc = bind();
    rc = m.begin_layer(0, s);
    std::printf("begin rc=%d epoch=%u\n", rc, m.epoch());
    print_groups("k", m, f);
    GroupId final2[] = {4, 7, 2};
    rc = m.finalize({final2, 3});
    await_started(2);
    std::printf("finalize [4,7,2] rc=%d\n", rc);
    print_queue("l", f);
    print_groups("l", m, f);
    release(2);
    await_ready(f, 2);
    release(4);
    await_ready(f, 3);
    rc = m.wait_io(2000);
    std::printf("wait rc=%d\n", rc);
    print_queue("m", f);
    print_groups("m", m, f);
    print_slots("m", f);
    rc = m.retire();
    std::printf("retire rc=%d requests=%llu\n", rc, static_cast<unsigned long long>(m.read_requests()));
    std::printf("== end\n");
    return 0;
}
