// Per-layer lifecycle around the compute backend (LeanStream src/runtime/runtime.cpp:7-103).
//
// State per layer: active (between begin_layer and commit/abort retirement), enqueued,
// finalized, pending (deferred commit in flight). Rules kept from the reference:
//   * enqueue_compute calls the backend once per epoch; on error the manager and the
//     backend are cancelled, and abort must still prove completion (EBUSY until then);
//   * finalize refuses after a published queue error and cancels on its own failure;
//   * commit requires completion (or a deferred-commit hook), validates the next
//     resident set, and retires the manager; deferred commit retires from the
//     backend's callback, guarded by the epoch so a late callback cannot free a newer bank;
//   * drain waits for every deferred retirement.
#include "leanstream/runtime.h"
#include <algorithm>
#include <atomic>
#include <cassert>
#include <cerrno>

namespace leanstream::runtime {

struct Runtime::LayerContext {
    Runtime* owner;
    WeightManager manager;
    std::vector<GroupId> next_resident;
    std::vector<uint8_t> marks;
    std::atomic<bool> active{false}, pending{false};
    std::atomic<uint32_t> retire_epoch{0};
    bool enqueued = false, finalized = false;
    int error = 0;
    uint32_t layer;
    LayerContext(Runtime* r, uint32_t l, const ManagerConfig& c)
        : owner(r), manager(c), next_resident(c.group_count), marks(c.group_count), layer(l) {}
    bool current(uint32_t epoch) const { return active && epoch == manager.epoch(); }
    void cancel_all(const ComputeBackend& b, int rc, uint32_t epoch) {
        error = rc;
        manager.cancel(rc);
        if (b.cancel) b.cancel(b.context, layer, epoch);
    }
};

Runtime::Runtime(ManagerConfig c, ComputeBackend b, uint32_t n) : backend_(b), mode_(c.mode) {
    layers_.reserve(n);
    for (uint32_t l = 0; l < n; ++l) layers_.emplace_back(new LayerContext(this, l, c));
}

Runtime::~Runtime() {
    const int rc = drain();
    assert(rc != EBUSY);
    (void)rc;
}

WeightManager& Runtime::weights(uint32_t l) { return layers_.at(l)->manager; }

int Runtime::begin_layer(uint32_t l, const LayerStorage& s, LayerStep* step) {
    if (l >= layers_.size() || !step) return EINVAL;
    auto& c = *layers_[l];
    if (c.active.load(std::memory_order_acquire)) return EBUSY;
    const int rc = c.manager.begin_layer(l, s);
    if (rc) return rc;
    c.enqueued = false;
    c.finalized = false;
    c.error = 0;
    c.pending = false;
    c.active = true;
    *step = LayerStep(this, l, c.manager.epoch());
    return 0;
}

int LayerStep::update_prediction(Span<GroupId> ids) { return update_prediction(ids, {}); }

int LayerStep::update_prediction(Span<GroupId> ids, PredictionUpdateOptions options) {
    if (!runtime_) return EINVAL;
    auto& c = *runtime_->layers_[layer_];
    if (!c.current(epoch_) || c.finalized) return EINVAL;
    return c.manager.update_prediction(ids, options);
}

int LayerStep::enqueue_compute(const void* input, void* output, void* stream) {
    if (!runtime_) return EINVAL;
    Runtime& r = *runtime_;
    auto& c = *r.layers_[layer_];
    if (!c.current(epoch_) || c.enqueued || !r.backend_.enqueue || !r.backend_.complete) return EINVAL;
    c.enqueued = true;  // even a failed enqueue may have launched work: abort must wait
    const int rc = r.backend_.enqueue(r.backend_.context, layer_, input, output, stream, c.manager.core_descriptors(),
                                      c.manager.queue(), epoch_, r.mode_);
    if (rc) c.cancel_all(r.backend_, rc, epoch_);
    return rc;
}

int LayerStep::finalize(Span<GroupId> ids) {
    if (!runtime_) return EINVAL;
    auto& c = *runtime_->layers_[layer_];
    if (!c.current(epoch_) || c.finalized) return EINVAL;
    const uint32_t queue_error = __atomic_load_n(&c.manager.queue().control->error, __ATOMIC_ACQUIRE);
    if (queue_error) return static_cast<int>(queue_error);
    const int rc = c.manager.finalize(ids);
    if (!rc)
        c.finalized = true;
    else if (c.enqueued)
        c.cancel_all(runtime_->backend_, rc, epoch_);
    return rc;
}

void Runtime::retire_callback(void* ptr, uint32_t epoch) {
    auto& c = *static_cast<LayerContext*>(ptr);
    Runtime& r = *c.owner;
    uint32_t expected = epoch;
    if (!epoch || !c.retire_epoch.compare_exchange_strong(expected, 0, std::memory_order_acq_rel)) return;
    // The backend has finished GPU use and cache installation for this epoch.
    const int error = c.manager.retire();
    {
        std::lock_guard<std::mutex> lock(r.mutex_);
        c.error = error;
        c.pending = false;
        c.active.store(false, std::memory_order_release);
    }
    r.retired_.notify_all();
}

int LayerStep::commit(Span<GroupId> ids) {
    if (!runtime_) return EINVAL;
    Runtime& r = *runtime_;
    auto& c = *r.layers_[layer_];
    if (!c.current(epoch_) || !c.finalized || !c.enqueued || c.pending) return EINVAL;
    const uint32_t queue_error = __atomic_load_n(&c.manager.queue().control->error, __ATOMIC_ACQUIRE);
    if (queue_error) return static_cast<int>(queue_error);
    if (ids.size > c.next_resident.size() || (ids.size && !ids.data)) return EINVAL;
    const bool deferred = r.backend_.defer_commit != nullptr;
    if (!deferred && !r.backend_.complete(r.backend_.context, layer_)) return EBUSY;
    std::fill(c.marks.begin(), c.marks.end(), 0);
    for (size_t i = 0; i < ids.size; ++i) {
        const GroupId g = ids[i];
        if (g < 0 || static_cast<size_t>(g) >= c.next_resident.size() || c.marks[g]) return EINVAL;
        c.marks[g] = 1;
        if (!deferred) {
            const GroupState st = c.manager.group_state(g);
            if (st.cache_slot < 0 && st.io_state != IOState::Ready) return EAGAIN;
        }
    }
    if (deferred) {
        std::copy_n(ids.data, ids.size, c.next_resident.data());
        c.pending = true;
        c.retire_epoch.store(epoch_, std::memory_order_release);
        const int rc = r.backend_.defer_commit(r.backend_.context, layer_, {c.next_resident.data(), ids.size}, epoch_,
                                               Runtime::retire_callback, &c);
        if (rc) {
            c.pending = false;
            c.retire_epoch = 0;
        }
        return rc;
    }
    if (!r.backend_.commit) return ENOTSUP;
    int rc = r.backend_.commit(r.backend_.context, layer_, ids);
    if (rc) return rc;
    rc = c.manager.retire();
    c.active = false;
    return rc;
}

int LayerStep::abort() {
    if (!runtime_) return EINVAL;
    Runtime& r = *runtime_;
    auto& c = *r.layers_[layer_];
    if (!c.current(epoch_) || c.pending) return EINVAL;
    c.manager.cancel();
    if (c.enqueued && r.backend_.cancel) r.backend_.cancel(r.backend_.context, layer_, epoch_);
    if (c.enqueued && !r.backend_.complete(r.backend_.context, layer_)) return EBUSY;
    const int rc = c.manager.retire();
    c.active = false;
    return rc;
}

int Runtime::drain() {
    std::unique_lock<std::mutex> lock(mutex_);
    for (auto& c : layers_)
        if (c->active && !c->pending) return EBUSY;
    retired_.wait(lock, [&] {
        for (auto& c : layers_)
            if (c->active) return false;
        return true;
    });
    for (auto& c : layers_)
        if (c->error) return c->error;
    return 0;
}

}  // namespace leanstream::runtime
