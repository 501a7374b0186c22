// WeightManager: one layer's residency plan, prediction admission and ready-queue
// descriptors (the contract of include/leanstream/weight_manager.h; LeanStream
// weight_manager.h:9-72, docs/execution_queue.md, docs/architecture.md).
//
// A manager moves through three phases per layer epoch:
//
//   Closed --begin_layer--> Open --finalize--> Frozen --retire--> Closed
//
//   * prepare_layer validates the bindings, registers the group layout (kept across
//     layers while its (pointer, generation) key is unchanged) and builds the core plan:
//     one Cache descriptor per resident group.
//   * begin_layer reuses a prepared plan whose key equals the new bindings (else prepares
//     again), opens epoch n, resets the queue and starts the transport.
//   * update_prediction hands the transport the new priority list: first occurrences of
//     groups that are neither cached nor already past EMPTY, cut to the I/O budget.
//   * finalize checks the whole final membership before anything is written, then
//     writes the queue descriptors in final order, publishes the prefix that is already
//     readable (cached groups, groups whose bytes arrived) and passes the groups still to
//     read to the transport.
//   * completions (transport threads) publish each READY member exactly once.
//
// The observable behaviour -- descriptors, publication order, queue words, return codes
// and transport calls -- is pinned line by line against LeanStream's own runtime
// (tests/golden/runtime_trace.txt, tests/golden/staging_trace.txt). The transport is
// always a borrowed IOBackend; LeanStream's O_DIRECT engine is not part of this library.
#include "leanstream/weight_manager.h"
#include <algorithm>
#include <atomic>
#include <cerrno>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <vector>

namespace leanstream::runtime {

namespace {

// Per-group marks cleared in O(1): a group is marked when its stamp equals the round.
class GroupMarks {
public:
    explicit GroupMarks(size_t n) : stamp_(n, 0) {}
    void clear() {
        if (++round_ == 0) {   // the round counter wrapped: forget every stamp once
            std::fill(stamp_.begin(), stamp_.end(), 0u);
            round_ = 1;
        }
    }
    // true if i was already marked in this round
    bool mark(size_t i) {
        const bool was = stamp_[i] == round_;
        stamp_[i] = round_;
        return was;
    }
    bool marked(size_t i) const { return stamp_[i] == round_; }

private:
    std::vector<uint32_t> stamp_;
    uint32_t round_ = 1;
};

uint32_t io_word(const uint32_t* states, GroupId g) { return __atomic_load_n(states + g, __ATOMIC_ACQUIRE); }

// The bindings a prepared plan depends on; a plan is reused only for an equal key.
struct PlanKey {
    uint64_t plan_generation = 0, layout_generation = 0, staging_bytes = 0;
    const GroupLayout* layout = nullptr;
    size_t layout_size = 0;
    const SlotId* cache_slots = nullptr;
    const SlotId* destination_slots = nullptr;
    const GroupId* core = nullptr;
    size_t core_size = 0;
    const ExecDesc* mapped_core = nullptr;
    const void* staging = nullptr;
    const uint32_t* io_states = nullptr;
    DeviceExecQueue queue{};

    static PlanKey of(const LayerStorage& s) {
        PlanKey k;
        k.plan_generation = s.plan_generation;
        k.layout_generation = s.layout_generation;
        k.staging_bytes = s.staging_bytes;
        k.layout = s.layout.data;
        k.layout_size = s.layout.size;
        k.cache_slots = s.cache_slots;
        k.destination_slots = s.destination_slots;
        k.core = s.core.data;
        k.core_size = s.core.size;
        k.mapped_core = s.mapped_core_descriptors;
        k.staging = s.staging;
        k.io_states = s.io_states;
        k.queue = s.queue;
        return k;
    }
    // A nonzero plan generation that matches, with every binding equal.
    bool reusable_for(const PlanKey& n) const {
        return n.plan_generation && n.plan_generation == plan_generation && n.layout_generation == layout_generation &&
               n.staging_bytes == staging_bytes && n.layout == layout && n.layout_size == layout_size &&
               n.cache_slots == cache_slots && n.destination_slots == destination_slots && n.core == core &&
               n.core_size == core_size && n.mapped_core == mapped_core && n.staging == staging &&
               n.io_states == io_states && n.queue.descriptors == queue.descriptors &&
               n.queue.ready_indices == queue.ready_indices && n.queue.control == queue.control &&
               n.queue.capacity == queue.capacity;
    }
};

const ManagerConfig& checked(const ManagerConfig& c) {
    const bool geometry_ok = c.group_count && c.group_count <= static_cast<uint32_t>(std::numeric_limits<GroupId>::max()) &&
                             c.group_bytes && c.staging_stride >= c.group_bytes &&
                             c.staging_stride <= std::numeric_limits<size_t>::max() / c.group_count;
    if (!geometry_ok) throw std::invalid_argument("layout geometry/capacity overflow");
    const IOBackend& io = c.io_backend;
    if (!io.begin) throw std::invalid_argument("an IOBackend transport is required");
    if (!(io.update && io.consume && io.retire && io.ready_slot)) throw std::invalid_argument("incomplete IO backend");
    return c;
}

}  // namespace

struct WeightManager::Impl {
    enum class Phase : uint8_t { Closed, Open, Frozen };

    const ManagerConfig config;
    const uint32_t n;
    // layout registry: GroupLayout by logical id, valid for (source, generation)
    std::vector<GroupLayout> layout;
    const GroupLayout* registered_from = nullptr;
    uint64_t registered_generation = 0;
    // core plan
    std::vector<ExecDesc> core_table;   // used when no GPU-visible table is bound
    ExecDesc* core = nullptr;
    uint32_t core_count = 0;
    std::vector<uint8_t> resident;      // member of the core plan
    bool prepared = false;
    PlanKey prepared_key;
    // the open epoch
    LayerStorage bound{};
    std::atomic<Phase> phase{Phase::Closed};
    std::atomic<uint32_t> epoch{0};
    uint64_t generation = 0;
    std::vector<GroupId> admitted;      // the last priority list handed to the transport
    std::vector<int32_t> position;      // queue descriptor index per member (-1: none)
    std::vector<uint8_t> published;     // member already visible to the consumer
    std::vector<GroupId> to_read;       // members the transport still has to deliver
    GroupMarks marks;
    ExecutionQueue queue;
    std::mutex producer;                // serialises every write of the queue

    explicit Impl(const ManagerConfig& c)
        : config(checked(c)), n(c.group_count), layout(n), core_table(n), resident(n), position(n, -1), published(n),
          marks(n) {
        admitted.reserve(n);
        to_read.reserve(n);
    }

    bool valid_group(GroupId g) const { return g >= 0 && static_cast<uint32_t>(g) < n; }
    bool valid_slot(SlotId s) const { return s >= 0 && static_cast<uint32_t>(s) < n; }
    bool is_open() const { return phase.load(std::memory_order_acquire) != Phase::Closed; }
    bool is_frozen() const { return phase.load(std::memory_order_acquire) == Phase::Frozen; }
    const IOBackend& io() const { return config.io_backend; }

    // ---- prepare ----
    int check_bindings(const LayerStorage& s) const {
        const bool complete = s.layout.data && s.cache_slots && s.staging && s.io_states && s.queue.control &&
                              s.queue.descriptors && s.queue.ready_indices;
        if (!complete || s.layout.size != n || s.queue.capacity > n || s.core.size > n || (s.core.size && !s.core.data))
            return EINVAL;
        if (s.staging_bytes && s.staging_bytes < n * config.staging_stride) return ENOSPC;
        return 0;
    }

    int register_layout(const LayerStorage& s) {
        if (s.layout_generation && s.layout_generation == registered_generation && s.layout.data == registered_from)
            return 0;
        registered_from = nullptr;
        registered_generation = 0;
        marks.clear();
        for (size_t i = 0; i < s.layout.size; ++i) {
            const GroupLayout& e = s.layout[i];
            if (e.logical_group >= n || marks.mark(e.logical_group) || e.bytes != config.group_bytes) return EINVAL;
            layout[e.logical_group] = e;
        }
        registered_from = s.layout.data;
        registered_generation = s.layout_generation;
        return 0;
    }

    int plan_core(const LayerStorage& s) {
        std::fill(resident.begin(), resident.end(), 0);
        marks.clear();   // destination rows taken by core groups
        core = s.mapped_core_descriptors ? s.mapped_core_descriptors : core_table.data();
        core_count = static_cast<uint32_t>(s.core.size);
        for (uint32_t i = 0; i < core_count; ++i) {
            const GroupId g = s.core[i];
            if (!valid_group(g) || resident[g] || s.cache_slots[g] < 0) return EINVAL;
            resident[g] = 1;
            uint32_t row = i;
            if (s.destination_slots) {
                const SlotId d = s.destination_slots[g];
                if (!valid_slot(d) || marks.mark(static_cast<size_t>(d))) return EINVAL;
                row = static_cast<uint32_t>(d);
            }
            ExecDesc& e = core[i];
            e.logical_group = static_cast<uint32_t>(g);
            e.physical_group = layout[g].physical_group;
            e.source_slot = static_cast<uint32_t>(s.cache_slots[g]);
            e.dest_slot = row;
            e.source_kind = SourceKind::Cache;
        }
        return 0;
    }

    // ---- finalize ----
    // Members in final order; every core group present, no group twice or outside, the
    // queued ones fit the queue, destination rows (when bound) distinct. Nothing is
    // written before the whole list passed.
    int check_membership(Span<GroupId> ids, uint32_t& queued) {
        marks.clear();
        queued = 0;
        for (size_t i = 0; i < ids.size; ++i) {
            if (!valid_group(ids[i]) || marks.mark(static_cast<size_t>(ids[i]))) return EINVAL;
            queued += resident[ids[i]] ? 0u : 1u;
        }
        for (uint32_t g = 0; g < n; ++g)
            if (resident[g] && !marks.marked(g)) return EINVAL;
        if (queued > bound.queue.capacity) return ENOSPC;
        if (const SlotId* rows = bound.destination_slots) {
            marks.clear();
            for (size_t i = 0; i < ids.size; ++i)
                if (!valid_slot(rows[ids[i]]) || marks.mark(static_cast<size_t>(rows[ids[i]]))) return EINVAL;
        }
        return 0;
    }

    // Queue descriptors of the non-core members, in final order. A cached group is read
    // from its cache slot; the others come from staging (slot filled when READY).
    void write_queue_plan(Span<GroupId> ids) {
        to_read.clear();
        uint32_t next = 0;
        for (size_t i = 0; i < ids.size; ++i) {
            const GroupId g = ids[i];
            if (resident[g]) continue;
            const SlotId cached = bound.cache_slots[g];
            ExecDesc& e = bound.queue.descriptors[next];
            e.logical_group = static_cast<uint32_t>(g);
            e.physical_group = layout[g].physical_group;
            e.source_slot = cached >= 0 ? static_cast<uint32_t>(cached) : 0u;
            e.dest_slot = bound.destination_slots ? static_cast<uint32_t>(bound.destination_slots[g]) : core_count + next;
            e.source_kind = cached >= 0 ? SourceKind::Cache : SourceKind::Staging;
            position[g] = static_cast<int32_t>(next++);
            if (cached < 0) to_read.push_back(g);
        }
    }

    // The prefix visible at activation: cached members and members already READY, in
    // final order. Producer lock held.
    int stage_prefix(Span<GroupId> ids) {
        for (size_t i = 0; i < ids.size; ++i) {
            const GroupId g = ids[i];
            if (resident[g]) continue;
            if (bound.cache_slots[g] < 0) {
                if (io_word(bound.io_states, g) != kIoReady) continue;
                const SlotId slot = io().ready_slot(io().context, g);
                if (!valid_slot(slot)) {
                    queue.fail(EIO);
                    return EIO;
                }
                bound.queue.descriptors[position[g]].source_slot = static_cast<uint32_t>(slot);
            }
            published[g] = 1;
            queue.append_unpublished(static_cast<uint32_t>(position[g]));
        }
        return 0;
    }

    // ---- completions (transport threads) ----
    // Producer lock held: a READY member becomes visible once, reading its staging slot.
    void publish_member(GroupId g, SlotId slot) {
        if (position[g] < 0 || published[g]) return;
        if (slot < 0) slot = io().ready_slot(io().context, g);
        if (!valid_slot(slot)) {
            queue.fail(EIO);
            return;
        }
        ExecDesc& e = bound.queue.descriptors[position[g]];
        e.source_slot = static_cast<uint32_t>(slot);
        e.source_kind = SourceKind::Staging;
        published[g] = 1;
        queue.publish(static_cast<uint32_t>(position[g]));
    }

    bool current(uint32_t at_epoch) const { return is_open() && at_epoch == epoch.load(std::memory_order_relaxed); }

    static void on_delivery(void* arg, const IOCompletion& c) {
        Impl& m = *static_cast<Impl*>(arg);
        if (!m.current(c.epoch)) return;   // a late delivery of another epoch
        if (c.error) {
            std::lock_guard<std::mutex> lock(m.producer);
            if (m.current(c.epoch)) m.queue.fail(static_cast<uint32_t>(c.error));
            return;
        }
        if (!m.valid_group(c.logical_group) || !m.valid_slot(c.staging_slot)) {
            m.queue.fail(EINVAL);
            return;
        }
        // before finalize there is no plan: finalize publishes what is READY by then
        if (!m.is_frozen()) return;
        std::lock_guard<std::mutex> lock(m.producer);
        if (m.current(c.epoch)) m.publish_member(c.logical_group, c.staging_slot);
    }
};

WeightManager::WeightManager(ManagerConfig c) : impl_(new Impl(c)) {}
WeightManager::~WeightManager() = default;

int WeightManager::prepare_layer(const LayerStorage& s) {
    Impl& m = *impl_;
    if (m.is_open()) return EBUSY;
    if (const int rc = m.check_bindings(s)) return rc;
    m.prepared = false;
    if (const int rc = m.register_layout(s)) return rc;
    if (const int rc = m.plan_core(s)) return rc;
    m.prepared = true;
    m.prepared_key = PlanKey::of(s);
    return 0;
}

int WeightManager::begin_layer(uint32_t, const LayerStorage& s) {
    Impl& m = *impl_;
    if (m.is_open()) return EBUSY;
    if (m.epoch.load() == std::numeric_limits<uint32_t>::max()) return EOVERFLOW;
    if (!(m.prepared && m.prepared_key.reusable_for(PlanKey::of(s))))
        if (const int rc = prepare_layer(s)) return rc;
    m.bound = s;
    m.queue.bind(s.queue);
    const uint32_t e = m.epoch.load() + 1;
    m.epoch.store(e);
    m.queue.reset(e);
    std::fill(m.position.begin(), m.position.end(), -1);
    std::fill(m.published.begin(), m.published.end(), 0);
    m.generation = 0;
    m.phase.store(Impl::Phase::Open, std::memory_order_release);
    const int rc = m.io().begin(m.io().context, Impl::on_delivery, &m, e);
    if (rc) m.phase.store(Impl::Phase::Closed, std::memory_order_release);
    return rc;
}

int WeightManager::update_prediction(Span<GroupId> ids) { return update_prediction(ids, {}); }

int WeightManager::update_prediction(Span<GroupId> ids, PredictionUpdateOptions options) {
    Impl& m = *impl_;
    if (m.phase.load(std::memory_order_acquire) != Impl::Phase::Open || (ids.size && !ids.data)) return EINVAL;
    if (options.execution_epoch && options.execution_epoch != m.epoch.load()) return ESTALE;
    m.marks.clear();
    m.admitted.clear();
    for (size_t i = 0; i < ids.size; ++i) {
        const GroupId g = ids[i];
        if (!m.valid_group(g)) return EINVAL;
        if (m.marks.mark(static_cast<size_t>(g))) continue;   // later duplicates keep the first rank
        // cached, in-flight and ready groups never spend the I/O budget
        const bool needs_read = m.bound.cache_slots[g] < 0 && io_word(m.bound.io_states, g) == kIoEmpty;
        if (needs_read && m.admitted.size() < options.io_budget) m.admitted.push_back(g);
    }
    const int rc = m.io().update(m.io().context, {m.admitted.data(), m.admitted.size()});
    if (!rc) ++m.generation;
    return rc;
}

int WeightManager::finalize(Span<GroupId> ids) {
    Impl& m = *impl_;
    if (m.phase.load(std::memory_order_acquire) != Impl::Phase::Open || (ids.size && !ids.data) ||
        ids.size < m.core_count)
        return EINVAL;
    uint32_t queued = 0;
    if (const int rc = m.check_membership(ids, queued)) return rc;
    {
        std::lock_guard<std::mutex> lock(m.producer);
        m.write_queue_plan(ids);
        m.queue.prepare(queued);
        m.phase.store(Impl::Phase::Frozen, std::memory_order_release);
        if (const int rc = m.stage_prefix(ids)) return rc;
        m.queue.activate();
    }
    const int rc = m.io().consume(m.io().context, {m.to_read.data(), m.to_read.size()});
    if (rc) m.queue.fail(static_cast<uint32_t>(rc));
    return rc;
}

int WeightManager::retire() {
    Impl& m = *impl_;
    if (!m.is_open()) return EINVAL;
    // the transport drains its callbacks before the epoch can change
    const int rc = m.io().retire(m.io().context);
    std::lock_guard<std::mutex> lock(m.producer);
    m.phase.store(Impl::Phase::Closed, std::memory_order_release);
    return rc;
}

void WeightManager::cancel(int error) {
    Impl& m = *impl_;
    if (m.is_open()) m.queue.fail(static_cast<uint32_t>(error ? error : ECANCELED));
}

GroupState WeightManager::group_state(GroupId g) const {
    const Impl& m = *impl_;
    GroupState st;
    if (!m.is_open() || !m.valid_group(g)) return st;
    const uint32_t w = io_word(m.bound.io_states, g);
    st.cache_slot = m.bound.cache_slots[g];
    st.io_state = w == kIoReady ? IOState::Ready : w == kIoInflight ? IOState::Inflight : IOState::Empty;
    if (st.io_state != IOState::Empty) st.staging_slot = m.io().ready_slot(m.io().context, g);
    return st;
}

uint64_t WeightManager::prediction_generation() const { return impl_->generation; }
uint32_t WeightManager::epoch() const { return impl_->epoch.load(); }
DeviceExecQueue WeightManager::queue() const { return impl_->bound.queue; }
Span<ExecDesc> WeightManager::core_descriptors() const { return {impl_->core, impl_->core_count}; }

int WeightManager::wait_io(int timeout_ms) {
    const IOBackend& io = impl_->io();
    return io.wait ? io.wait(io.context, timeout_ms) : ENOTSUP;
}

uint64_t WeightManager::read_requests() const {
    const IOBackend& io = impl_->io();
    return io.requests ? io.requests(io.context) : 0;
}

}  // namespace leanstream::runtime
