// Per-layer residency, prediction filtering and descriptor production.
//
// Observable behaviour follows LeanStream src/runtime/weight_manager.cpp:
//   * prepare_layer (:81-108): layout registration keyed by (pointer, generation), core
//     descriptors {g, physical(g), cache_slot(g), dest(g) or i, Cache};
//   * begin_layer (:109-134): optional reuse of a prepared plan, ++epoch, queue reset;
//   * update_prediction (:136-153): first-occurrence dedup, drop cached / non-EMPTY
//     groups, truncate to io_budget, forward to the transport;
//   * finalize (:154-204): validate everything before mutating, then build the queue
//     descriptors in final order {g, physical, slot or 0, dest or core+idx,
//     Cache|Staging}, publish cached and already-READY groups as the initial prefix;
//   * completions (:46-72): publish READY groups with source_slot = ready slot,
//     kind = Staging, exactly once, under the producer lock.
// The transport is always a borrowed IOBackend; the reference's O_DIRECT engine is
// not part of this build.
#include "leanstream/weight_manager.h"
#include <algorithm>
#include <atomic>
#include <cerrno>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <vector>

#ifdef LEANSTREAM_RUNTIME_TESTING
extern "C" void leanstream_test_finalize_hook(int);
#define LS_FINALIZE_POINT(n) leanstream_test_finalize_hook(n)
#else
#define LS_FINALIZE_POINT(n) ((void)0)
#endif

namespace leanstream::runtime {

namespace {

uint32_t load_state(const uint32_t* states, GroupId g) { return __atomic_load_n(states + g, __ATOMIC_ACQUIRE); }

ManagerConfig validated(ManagerConfig c) {
    const bool bad = c.group_count == 0 || c.group_count > static_cast<uint32_t>(std::numeric_limits<int32_t>::max()) ||
                     c.group_bytes == 0 || c.staging_stride < c.group_bytes ||
                     c.staging_stride > std::numeric_limits<size_t>::max() / c.group_count;
    if (bad) throw std::invalid_argument("layout geometry/capacity overflow");
    const IOBackend& io = c.io_backend;
    if (!io.begin) throw std::invalid_argument("an IOBackend transport is required");
    if (!io.update || !io.consume || !io.retire || !io.ready_slot)
        throw std::invalid_argument("incomplete borrowed IO backend");
    return c;
}

}  // namespace

struct WeightManager::Impl {
    ManagerConfig config;
    LayerStorage storage{}, prepared{};
    const GroupLayout* registered = nullptr;
    uint64_t registered_generation = 0;
    std::vector<GroupLayout> layout;
    std::vector<GroupId> priority, final_reads;
    std::vector<int32_t> final_index;
    std::vector<uint8_t> seen, published, in_core;
    std::vector<ExecDesc> own_core;
    ExecDesc* core = nullptr;
    uint32_t core_count = 0;
    ExecutionQueue queue;
    std::mutex producer;
    std::atomic<uint32_t> epoch{0};
    std::atomic<bool> active{false}, finalized{false};
    uint64_t generation = 0;

    explicit Impl(const ManagerConfig& c)
        : config(c), layout(c.group_count), final_index(c.group_count, -1), seen(c.group_count),
          published(c.group_count), in_core(c.group_count), own_core(c.group_count) {
        priority.reserve(c.group_count);
        final_reads.reserve(c.group_count);
    }

    bool in_range(GroupId g) const { return g >= 0 && static_cast<uint32_t>(g) < config.group_count; }
    void clear_seen() { std::fill(seen.begin(), seen.end(), 0); }

    // producer lock held; the completed bytes are already visible to the GPU
    void publish_ready(GroupId g, SlotId slot) {
        const int32_t index = final_index[g];
        if (index < 0 || published[g]) return;
        if (slot < 0) slot = config.io_backend.ready_slot(config.io_backend.context, g);
        if (slot < 0 || static_cast<uint32_t>(slot) >= config.group_count) {
            queue.fail(EIO);
            return;
        }
        ExecDesc& d = storage.queue.descriptors[index];
        d.source_slot = static_cast<uint32_t>(slot);
        d.source_kind = SourceKind::Staging;
        published[g] = 1;
        queue.publish(static_cast<uint32_t>(index));
    }

    static void on_completion(void* arg, const IOCompletion& n) {
        Impl& m = *static_cast<Impl*>(arg);
        if (!m.active.load(std::memory_order_acquire) || n.epoch != m.epoch.load(std::memory_order_relaxed)) return;
        if (n.error) {
            std::lock_guard<std::mutex> lock(m.producer);
            if (m.active && n.epoch == m.epoch) m.queue.fail(static_cast<uint32_t>(n.error));
            return;
        }
        if (!m.in_range(n.logical_group) || n.staging_slot < 0 ||
            static_cast<uint32_t>(n.staging_slot) >= m.config.group_count) {
            m.queue.fail(EINVAL);
            return;
        }
        // Before finalize the plan does not exist; finalize publishes READY groups itself.
        if (!m.finalized.load(std::memory_order_acquire)) return;
        std::lock_guard<std::mutex> lock(m.producer);
        if (m.active && n.epoch == m.epoch) m.publish_ready(n.logical_group, n.staging_slot);
    }
};

WeightManager::WeightManager(ManagerConfig c) : impl_(new Impl(validated(c))) {}
WeightManager::~WeightManager() = default;

int WeightManager::prepare_layer(const LayerStorage& s) {
    Impl& m = *impl_;
    if (m.active) return EBUSY;
    const uint32_t n = m.config.group_count;
    const bool missing = !s.layout.data || !s.cache_slots || !s.staging || !s.io_states || !s.queue.control ||
                         !s.queue.descriptors || !s.queue.ready_indices;
    if (s.layout.size != n || missing || s.queue.capacity > n || (s.core.size && !s.core.data) || s.core.size > n)
        return EINVAL;
    if (s.staging_bytes && s.staging_bytes < n * m.config.staging_stride) return ENOSPC;
    m.prepared = {};
    const bool registered = s.layout_generation && s.layout_generation == m.registered_generation &&
                            s.layout.data == m.registered;
    if (!registered) {
        m.registered = nullptr;
        m.registered_generation = 0;
        m.clear_seen();
        for (size_t i = 0; i < s.layout.size; ++i) {
            const GroupLayout& g = s.layout[i];
            if (g.logical_group >= n || m.seen[g.logical_group]++ || g.bytes != m.config.group_bytes) return EINVAL;
            m.layout[g.logical_group] = g;
        }
        m.registered = s.layout.data;
        m.registered_generation = s.layout_generation;
    }
    std::fill(m.in_core.begin(), m.in_core.end(), 0);
    m.clear_seen();  // destination slots claimed by core groups
    m.core_count = static_cast<uint32_t>(s.core.size);
    m.core = s.mapped_core_descriptors ? s.mapped_core_descriptors : m.own_core.data();
    for (size_t i = 0; i < s.core.size; ++i) {
        const GroupId g = s.core[i];
        if (!m.in_range(g) || m.in_core[g]++ || s.cache_slots[g] < 0) return EINVAL;
        if (s.destination_slots) {
            const SlotId d = s.destination_slots[g];
            if (d < 0 || static_cast<uint32_t>(d) >= n || m.seen[d]++) return EINVAL;
        }
        m.core[i] = {static_cast<uint32_t>(g), m.layout[g].physical_group, static_cast<uint32_t>(s.cache_slots[g]),
                     static_cast<uint32_t>(s.destination_slots ? s.destination_slots[g] : static_cast<SlotId>(i)),
                     SourceKind::Cache};
    }
    m.prepared = s;
    return 0;
}

int WeightManager::begin_layer(uint32_t, const LayerStorage& s) {
    Impl& m = *impl_;
    if (m.active) return EBUSY;
    if (m.epoch == std::numeric_limits<uint32_t>::max()) return EOVERFLOW;
    const LayerStorage& p = m.prepared;
    const bool reuse = s.plan_generation && s.plan_generation == p.plan_generation && s.layout.data == p.layout.data &&
                       s.layout.size == p.layout.size && s.layout_generation == p.layout_generation &&
                       s.cache_slots == p.cache_slots && s.destination_slots == p.destination_slots &&
                       s.core.data == p.core.data && s.core.size == p.core.size &&
                       s.mapped_core_descriptors == p.mapped_core_descriptors && s.queue.control == p.queue.control &&
                       s.queue.descriptors == p.queue.descriptors && s.queue.ready_indices == p.queue.ready_indices &&
                       s.queue.capacity == p.queue.capacity && s.staging == p.staging && s.io_states == p.io_states &&
                       s.staging_bytes == p.staging_bytes;
    if (!reuse) {
        const int rc = prepare_layer(s);
        if (rc) return rc;
    }
    m.storage = s;
    m.queue.bind(s.queue);
    m.queue.reset(++m.epoch);
    std::fill(m.final_index.begin(), m.final_index.end(), -1);
    std::fill(m.published.begin(), m.published.end(), 0);
    m.generation = 0;
    m.finalized = false;
    m.active = true;
    const IOBackend& io = m.config.io_backend;
    const int rc = io.begin(io.context, Impl::on_completion, &m, m.epoch);
    if (rc) m.active = false;
    return rc;
}

int WeightManager::update_prediction(Span<GroupId> ids) { return update_prediction(ids, {}); }

int WeightManager::update_prediction(Span<GroupId> ids, PredictionUpdateOptions options) {
    Impl& m = *impl_;
    if (!m.active || m.finalized || (ids.size && !ids.data)) return EINVAL;
    if (options.execution_epoch && options.execution_epoch != m.epoch) return ESTALE;
    m.clear_seen();
    m.priority.clear();
    for (size_t i = 0; i < ids.size; ++i) {
        const GroupId g = ids[i];
        if (!m.in_range(g)) return EINVAL;
        if (m.seen[g]) continue;
        m.seen[g] = 1;
        // Cached, READY and INFLIGHT groups never spend the I/O budget.
        if (m.storage.cache_slots[g] < 0 && load_state(m.storage.io_states, g) == kIoEmpty) m.priority.push_back(g);
    }
    if (m.priority.size() > options.io_budget) m.priority.resize(options.io_budget);
    const IOBackend& io = m.config.io_backend;
    const int rc = io.update(io.context, {m.priority.data(), m.priority.size()});
    if (!rc) ++m.generation;
    return rc;
}

int WeightManager::finalize(Span<GroupId> ids) {
    Impl& m = *impl_;
    if (!m.active || m.finalized || (ids.size && !ids.data) || ids.size < m.core_count) return EINVAL;
    const uint32_t n = m.config.group_count;
    // 1. validate the whole membership before anything becomes visible
    m.clear_seen();
    m.final_reads.clear();
    uint32_t queued = 0;
    for (size_t i = 0; i < ids.size; ++i) {
        const GroupId g = ids[i];
        if (!m.in_range(g) || m.seen[g]++) return EINVAL;
        if (!m.in_core[g]) ++queued;
    }
    for (uint32_t g = 0; g < n; ++g)
        if (m.in_core[g] && !m.seen[g]) return EINVAL;
    if (queued > m.storage.queue.capacity) return ENOSPC;
    if (m.storage.destination_slots) {
        m.clear_seen();
        for (size_t i = 0; i < ids.size; ++i) {
            const SlotId d = m.storage.destination_slots[ids[i]];
            if (d < 0 || static_cast<uint32_t>(d) >= n || m.seen[d]++) return EINVAL;
        }
    }
    LS_FINALIZE_POINT(0);
    {
        std::lock_guard<std::mutex> lock(m.producer);
        // 2. descriptors in final order, core groups excluded
        uint32_t idx = 0;
        for (size_t i = 0; i < ids.size; ++i) {
            const GroupId g = ids[i];
            if (m.in_core[g]) continue;
            const SlotId slot = m.storage.cache_slots[g];
            const uint32_t dest = m.storage.destination_slots ? static_cast<uint32_t>(m.storage.destination_slots[g])
                                                               : m.core_count + idx;
            m.storage.queue.descriptors[idx] = {static_cast<uint32_t>(g), m.layout[g].physical_group,
                                                slot < 0 ? 0u : static_cast<uint32_t>(slot), dest,
                                                slot < 0 ? SourceKind::Staging : SourceKind::Cache};
            m.final_index[g] = static_cast<int32_t>(idx++);
            if (slot < 0) m.final_reads.push_back(g);
        }
        LS_FINALIZE_POINT(1);
        m.queue.prepare(queued);
        m.finalized.store(true, std::memory_order_release);
        // 3. initial prefix: cached groups and groups whose bytes already arrived
        const IOBackend& io = m.config.io_backend;
        for (size_t i = 0; i < ids.size; ++i) {
            const GroupId g = ids[i];
            if (m.in_core[g]) continue;
            const uint32_t index = static_cast<uint32_t>(m.final_index[g]);
            if (m.storage.cache_slots[g] >= 0) {
                m.published[g] = 1;
                m.queue.append_unpublished(index);
            } else if (load_state(m.storage.io_states, g) == kIoReady) {
                const SlotId source = io.ready_slot(io.context, g);
                if (source < 0 || static_cast<uint32_t>(source) >= n) {
                    m.queue.fail(EIO);
                    return EIO;
                }
                m.storage.queue.descriptors[index].source_slot = static_cast<uint32_t>(source);
                m.published[g] = 1;
                m.queue.append_unpublished(index);
            }
        }
        m.queue.activate();
    }
    LS_FINALIZE_POINT(2);
    const IOBackend& io = m.config.io_backend;
    const int rc = io.consume(io.context, {m.final_reads.data(), m.final_reads.size()});
    if (rc) m.queue.fail(static_cast<uint32_t>(rc));
    return rc;
}

int WeightManager::retire() {
    Impl& m = *impl_;
    if (!m.active) return EINVAL;
    const IOBackend& io = m.config.io_backend;
    const int rc = io.retire(io.context);  // drains callbacks before the epoch can change
    std::lock_guard<std::mutex> lock(m.producer);
    m.active = false;
    return rc;
}

void WeightManager::cancel(int error) {
    if (impl_->active) impl_->queue.fail(static_cast<uint32_t>(error ? error : ECANCELED));
}

GroupState WeightManager::group_state(GroupId g) const {
    const Impl& m = *impl_;
    if (!m.active || !m.in_range(g)) return {};
    const uint32_t s = load_state(m.storage.io_states, g);
    SlotId slot = -1;
    if (s == kIoReady || s == kIoInflight) slot = m.config.io_backend.ready_slot(m.config.io_backend.context, g);
    const IOState state = s == kIoReady ? IOState::Ready : s == kIoInflight ? IOState::Inflight : IOState::Empty;
    return {m.storage.cache_slots[g], slot, state};
}

uint64_t WeightManager::prediction_generation() const { return impl_->generation; }
uint32_t WeightManager::epoch() const { return impl_->epoch; }
DeviceExecQueue WeightManager::queue() const { return impl_->storage.queue; }
Span<ExecDesc> WeightManager::core_descriptors() const { return {impl_->core, impl_->core_count}; }

int WeightManager::wait_io(int timeout_ms) {
    const IOBackend& io = impl_->config.io_backend;
    return io.wait ? io.wait(io.context, timeout_ms) : ENOTSUP;
}

uint64_t WeightManager::read_requests() const {
    const IOBackend& io = impl_->config.io_backend;
    return io.requests ? io.requests(io.context) : 0;
}

}  // namespace leanstream::runtime
