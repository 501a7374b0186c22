// Host-memory staging transport: admission, copy submission and completion.
//
// Behaviour kept from LeanStream src/io/stream_io.cpp (the O_DIRECT engine this
// replaces):
//   * select (:42-59): walk the active rank from its cursor, skipping groups already
//     claimed this session; after consume, fall back to the committed final list;
//   * admission (:73-79): claim + INFLIGHT under the lock, at most qd outstanding, none
//     once the terminal error word is set or the session is closing;
//   * completion (:94-99): terminal errno first (on error), then READY/ERROR with
//     release, then the observer callback, then the credit returns under the lock;
//   * install (:171-190): E2BIG above the rank capacity, EINVAL on an out-of-range id,
//     ESHUTDOWN while closing, EIO after an error; the new rank replaces the old one
//     and admission restarts at its head; consume adds first-seen ids to the
//     committed list;
//   * wait (:258-263): all committed groups READY, or the terminal error;
//   * end (:273-278): stop admissions, drain outstanding copies, return the error word.
// Differences, by design: one pump thread keeps up to qd asynchronous copies in flight
// (instead of qd threads blocking in pread), and an optional per-group arrival time
// delays a copy's submission (the latency of the tier that fills the pinned store).
#include "leanstream/host_staging_io.h"
#include <algorithm>
#include <cerrno>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <stdexcept>
#include <thread>
#include <vector>

namespace leanstream::runtime {

namespace {

uint64_t now_ns() {
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}
void store_word(uint32_t* p, uint32_t v) { __atomic_store_n(p, v, __ATOMIC_RELEASE); }
uint32_t load_word(const uint32_t* p) { return __atomic_load_n(p, __ATOMIC_ACQUIRE); }
void relax() {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#else
    std::this_thread::yield();
#endif
}

StagingConfig checked(const StagingConfig& c) {
    if (!c.group_count || c.group_count > 0x7fffffffu || !c.qd || c.qd > 32 || !c.group_bytes ||
        c.staging_stride < c.group_bytes || c.staging_stride > UINT64_MAX / c.group_count)
        throw std::invalid_argument("staging geometry");
    if (!c.engine.submit || !c.engine.poll) throw std::invalid_argument("a copy engine is required");
    return c;
}

}  // namespace

struct HostStagingIO::Impl {
    struct Copy {
        GroupId id;
        uint64_t due;
        uint32_t lane;
    };

    const StagingConfig config;
    // bound layer (changed only while no session is live)
    StagingLayer layer{};
    std::vector<uint64_t> offset;  // byte offset of logical group g in the source
    std::vector<uint8_t> marks;
    bool bound = false;

    mutable std::mutex mutex;
    std::condition_variable work, changed;
    bool stop = false;
    // session state, under `mutex`
    bool live = false, closing = false, consume = false;
    uint32_t epoch = 0;
    IOCompletionCallback callback = nullptr;
    void* callback_arg = nullptr;
    uint64_t begin_ns = 0;
    std::vector<GroupId> rank, committed;
    std::vector<uint8_t> claimed, in_committed;
    size_t cursor = 0, fallback = 0;
    StagingStatus st{};
    // owned by the pump thread
    std::vector<Copy> waiting, inflight;
    std::vector<uint32_t> free_lanes;
    uint64_t sequence = 0;
    std::thread pump;

    explicit Impl(const StagingConfig& c)
        : config(checked(c)), offset(c.group_count), marks(c.group_count), claimed(c.group_count),
          in_committed(c.group_count) {
        rank.reserve(c.group_count);
        committed.reserve(c.group_count);
        waiting.reserve(c.qd);
        inflight.reserve(c.qd);
        for (uint32_t l = c.qd; l-- > 0;) free_lanes.push_back(l);
        pump = std::thread([this] { run(); });
    }

    ~Impl() {
        retire_session();
        {
            std::lock_guard<std::mutex> lock(mutex);
            stop = true;
        }
        work.notify_all();
        pump.join();
    }

    uint32_t terminal() const { return load_word(layer.io_states + config.group_count); }
    void stamp(GroupId g, int which, uint64_t t) {
        if (layer.stamps) layer.stamps[3 * static_cast<size_t>(g) + which] = t > begin_ns ? t - begin_ns : 1;
    }

    GroupId select() {
        while (cursor < rank.size()) {
            const GroupId g = rank[cursor++];
            if (!claimed[g]) return g;
        }
        if (consume)
            while (fallback < committed.size()) {
                const GroupId g = committed[fallback++];
                if (!claimed[g]) return g;
            }
        return -1;
    }

    // lock held, pump thread
    void admit() {
        if (!live || closing || terminal()) return;
        while (st.outstanding < config.qd) {
            const GroupId g = select();
            if (g < 0) break;
            claimed[g] = 1;
            store_word(layer.io_states + g, kIoInflight);
            ++st.outstanding;
            ++st.admissions;
            const uint64_t t = now_ns();
            stamp(g, 0, t);
            waiting.push_back({g, begin_ns + (layer.arrival_ns ? layer.arrival_ns[g] : 0), 0});
        }
    }

    // pump thread, lock not held
    void finish(GroupId g, int error, uint32_t session_epoch, IOCompletionCallback cb, void* arg) {
        if (error) store_word(layer.io_states + config.group_count, static_cast<uint32_t>(error));
        store_word(layer.io_states + g, error ? kIoError : kIoReady);
        stamp(g, 2, now_ns());
        if (cb) cb(arg, IOCompletion{session_epoch, g, g, error, ++sequence});
        std::lock_guard<std::mutex> lock(mutex);
        --st.outstanding;
        ++st.completions;
        if (error)
            st.error = error;
        else
            st.bytes += config.group_bytes;
        changed.notify_all();
    }

    void run() {
        std::unique_lock<std::mutex> lock(mutex);
        while (!stop) {
            admit();
            if (waiting.empty() && inflight.empty()) {
                work.wait(lock);
                continue;
            }
            const bool drain = closing;
            const uint32_t session_epoch = epoch;
            const IOCompletionCallback cb = callback;
            void* const arg = callback_arg;
            lock.unlock();
            bool progressed = false;
            const uint64_t t = now_ns();
            // submit every admitted copy whose bytes have arrived, in admission order
            for (size_t i = 0; i < waiting.size();) {
                if (!drain && waiting[i].due > t) {
                    ++i;
                    continue;
                }
                Copy c = waiting[i];
                waiting.erase(waiting.begin() + static_cast<std::ptrdiff_t>(i));
                c.lane = free_lanes.back();
                free_lanes.pop_back();
                stamp(c.id, 1, now_ns());
                const int rc = config.engine.submit(config.engine.context, c.lane,
                                                    layer.staging + static_cast<uint64_t>(c.id) * config.staging_stride,
                                                    layer.source + offset[c.id], config.group_bytes);
                progressed = true;
                if (rc) {
                    free_lanes.push_back(c.lane);
                    finish(c.id, rc, session_epoch, cb, arg);
                } else {
                    inflight.push_back(c);
                }
            }
            for (size_t i = 0; i < inflight.size();) {
                const int rc = config.engine.poll(config.engine.context, inflight[i].lane);
                if (rc == EAGAIN) {
                    ++i;
                    continue;
                }
                const Copy c = inflight[i];
                inflight.erase(inflight.begin() + static_cast<std::ptrdiff_t>(i));
                free_lanes.push_back(c.lane);
                finish(c.id, rc, session_epoch, cb, arg);
                progressed = true;
            }
            if (!progressed) relax();
            lock.lock();
        }
    }

    int bind(const StagingLayer& l) {
        std::lock_guard<std::mutex> lock(mutex);
        if (live) return EBUSY;
        bound = false;
        if (!l.source || !l.layout.data || !l.staging || !l.io_states || l.layout.size != config.group_count)
            return EINVAL;
        if (l.staging_bytes < config.group_count * config.staging_stride) return ENOSPC;
        std::fill(marks.begin(), marks.end(), 0);
        for (size_t i = 0; i < l.layout.size; ++i) {
            const GroupLayout& g = l.layout[i];
            if (g.logical_group >= config.group_count || marks[g.logical_group]++ || g.bytes != config.group_bytes)
                return EINVAL;
            if (g.file_offset > l.source_bytes || l.source_bytes - g.file_offset < g.bytes) return ENOSPC;
            offset[g.logical_group] = g.file_offset;
        }
        layer = l;
        bound = true;
        return 0;
    }

    int begin(IOCompletionCallback cb, void* arg, uint32_t e) {
        std::lock_guard<std::mutex> lock(mutex);
        if (live) return EBUSY;
        if (!bound) return EINVAL;
        for (uint32_t g = 0; g <= config.group_count; ++g) store_word(layer.io_states + g, kIoEmpty);
        if (layer.stamps) std::fill_n(layer.stamps, 3 * static_cast<size_t>(config.group_count), 0);
        std::fill(claimed.begin(), claimed.end(), 0);
        std::fill(in_committed.begin(), in_committed.end(), 0);
        rank.clear();
        committed.clear();
        cursor = fallback = 0;
        consume = closing = false;
        st = {};
        st.epoch = e;
        epoch = e;
        callback = cb;
        callback_arg = arg;
        begin_ns = now_ns();
        live = true;
        return 0;
    }

    int install(const GroupId* ids, size_t n, bool final) {
        if (n && !ids) return EINVAL;
        if (n > config.group_count) return E2BIG;
        for (size_t i = 0; i < n; ++i)
            if (ids[i] < 0 || static_cast<uint32_t>(ids[i]) >= config.group_count) return EINVAL;
        std::lock_guard<std::mutex> lock(mutex);
        if (!live) return EINVAL;
        if (closing) return ESHUTDOWN;
        if (terminal()) return EIO;
        rank.assign(ids, ids + n);
        cursor = fallback = 0;
        if (final) {
            consume = true;
            for (size_t i = 0; i < n; ++i)
                if (!in_committed[ids[i]]) {
                    in_committed[ids[i]] = 1;
                    committed.push_back(ids[i]);
                }
        }
        work.notify_one();
        return 0;
    }

    int retire_session() {
        std::unique_lock<std::mutex> lock(mutex);
        if (!live) return 0;
        closing = true;
        work.notify_one();
        changed.wait(lock, [&] { return st.outstanding == 0; });
        st.ended = 1;
        live = false;
        return static_cast<int>(terminal());
    }

    bool committed_ready() const {
        if (!consume) return false;
        for (const GroupId g : committed)
            if (load_word(layer.io_states + g) != kIoReady) return false;
        return true;
    }

    int wait(int timeout_ms) {
        std::unique_lock<std::mutex> lock(mutex);
        if (!live) return EINVAL;
        const bool ok = changed.wait_for(lock, std::chrono::milliseconds(timeout_ms),
                                         [&] { return terminal() != 0 || committed_ready(); });
        return ok ? static_cast<int>(terminal()) : ETIMEDOUT;
    }

    int idle(int timeout_ms) {
        std::unique_lock<std::mutex> lock(mutex);
        if (!live) return 0;
        const bool ok = changed.wait_for(lock, std::chrono::milliseconds(timeout_ms), [&] {
            return terminal() != 0 || (st.outstanding == 0 && cursor >= rank.size() &&
                                       (!consume || fallback >= committed.size()));
        });
        return ok ? static_cast<int>(terminal()) : ETIMEDOUT;
    }

    static Impl& of(void* c) { return *static_cast<Impl*>(c); }
    static int io_begin(void* c, IOCompletionCallback cb, void* arg, uint32_t e) { return of(c).begin(cb, arg, e); }
    static int io_update(void* c, Span<GroupId> ids) { return of(c).install(ids.data, ids.size, false); }
    static int io_consume(void* c, Span<GroupId> ids) { return of(c).install(ids.data, ids.size, true); }
    static int io_retire(void* c) { return of(c).retire_session(); }
    static SlotId io_ready_slot(void* c, GroupId g) {
        return g >= 0 && static_cast<uint32_t>(g) < of(c).config.group_count ? g : -1;
    }
    static uint64_t io_requests(void* c) {
        Impl& m = of(c);
        std::lock_guard<std::mutex> lock(m.mutex);
        return m.st.admissions;
    }
    static int io_wait(void* c, int timeout_ms) { return of(c).wait(timeout_ms); }
};

HostStagingIO::HostStagingIO(StagingConfig c) : impl_(new Impl(c)) {}
HostStagingIO::~HostStagingIO() = default;

int HostStagingIO::bind_layer(const StagingLayer& l) { return impl_->bind(l); }

IOBackend HostStagingIO::backend() {
    IOBackend b;
    b.context = impl_.get();
    b.begin = Impl::io_begin;
    b.update = Impl::io_update;
    b.consume = Impl::io_consume;
    b.retire = Impl::io_retire;
    b.ready_slot = Impl::io_ready_slot;
    b.requests = Impl::io_requests;
    b.wait = Impl::io_wait;
    return b;
}

int HostStagingIO::status(StagingStatus* out) const {
    if (!out) return EINVAL;
    std::lock_guard<std::mutex> lock(impl_->mutex);
    *out = impl_->st;
    out->error = impl_->bound ? static_cast<int32_t>(impl_->terminal()) : 0;
    return 0;
}

int HostStagingIO::wait_idle(int timeout_ms) { return impl_->idle(timeout_ms); }

}  // namespace leanstream::runtime
