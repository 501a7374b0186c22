// Runtime / LayerStep: the per-layer lifecycle around a ComputeBackend (the contract of
// include/leanstream/runtime.h; LeanStream runtime.h:10-52, docs/architecture.md).
//
// Every layer has a slot that moves
//
//   Idle --begin_layer--> Open --commit / abort--> Idle
//                          Open --deferred commit--> Retiring --backend callback--> Idle
//
// A LayerStep names (layer, epoch); operations through a step of an older epoch, or on a
// slot that is not Open, are refused with EINVAL.
//   * enqueue_compute submits the layer once. A refused submission may still have
//     launched work, so the manager and the backend are cancelled and abort keeps
//     waiting for the backend's completion.
//   * finalize freezes the membership. A queue error published earlier is returned as
//     is; a finalize failure after the submission cancels both sides.
//   * commit reports a queue error first, then needs the backend's completion (or a
//     deferred-commit hook), the next resident groups readable (cached or READY), and
//     the backend's installation; the manager then retires. With a deferred-commit hook
//     the backend retires the slot later through a callback that names the epoch, so a
//     late or repeated callback is ignored.
//   * abort cancels, waits for completion (EBUSY until then) and retires.
//   * drain waits for every deferred retirement.
// The return codes are pinned against LeanStream's own runtime by
// tests/golden/runtime_trace.txt.
#include "leanstream/runtime.h"
#include <algorithm>
#include <atomic>
#include <cassert>
#include <cerrno>

namespace leanstream::runtime {

struct Runtime::LayerContext {
    enum class Life : uint8_t { Idle, Open, Retiring };

    Runtime& runtime;
    const uint32_t layer;
    WeightManager manager;
    std::atomic<Life> life{Life::Idle};
    std::atomic<uint32_t> retiring_epoch{0};   // the epoch a deferred retirement may end
    bool submitted = false, frozen = false;
    int error = 0;                             // reported by drain
    std::vector<GroupId> next_resident;        // ids handed to a deferred commit
    std::vector<uint8_t> listed;               // duplicate check of commit ids

    LayerContext(Runtime& r, uint32_t l, const ManagerConfig& c)
        : runtime(r), layer(l), manager(c), next_resident(c.group_count), listed(c.group_count) {}

    size_t groups() const { return listed.size(); }
    bool open_at(uint32_t epoch) const {
        return life.load(std::memory_order_acquire) != Life::Idle && epoch == manager.epoch();
    }
    bool retiring() const { return life.load(std::memory_order_acquire) == Life::Retiring; }
    uint32_t queue_error() const { return __atomic_load_n(&manager.queue().control->error, __ATOMIC_ACQUIRE); }

    // Both sides stop consuming: the manager fails the queue, the backend cancels.
    void cancel_both(int rc, uint32_t epoch) {
        error = rc;
        manager.cancel(rc);
        const ComputeBackend& b = runtime.backend_;
        if (b.cancel) b.cancel(b.context, layer, epoch);
    }

    // The commit ids: in range, distinct and, unless the backend defers the commit,
    // readable now. Each id is checked completely before the next one.
    int check_next_resident(Span<GroupId> ids, bool deferred) {
        std::fill(listed.begin(), listed.end(), 0);
        for (size_t i = 0; i < ids.size; ++i) {
            const GroupId g = ids[i];
            if (g < 0 || static_cast<size_t>(g) >= groups() || listed[g]) return EINVAL;
            listed[g] = 1;
            if (deferred) continue;
            const GroupState st = manager.group_state(g);
            if (st.cache_slot < 0 && st.io_state != IOState::Ready) return EAGAIN;
        }
        return 0;
    }

    int finish_direct(Span<GroupId> ids) {
        const ComputeBackend& b = runtime.backend_;
        if (!b.commit) return ENOTSUP;
        if (const int rc = b.commit(b.context, layer, ids)) return rc;
        const int rc = manager.retire();
        life.store(Life::Idle, std::memory_order_release);
        return rc;
    }

    int finish_deferred(Span<GroupId> ids, uint32_t epoch) {
        std::copy_n(ids.data, ids.size, next_resident.data());
        life.store(Life::Retiring, std::memory_order_release);
        retiring_epoch.store(epoch, std::memory_order_release);
        const ComputeBackend& b = runtime.backend_;
        const int rc = b.defer_commit(b.context, layer, {next_resident.data(), ids.size}, epoch,
                                      Runtime::retire_callback, this);
        if (rc) {   // the backend refused: the step stays open
            life.store(Life::Open, std::memory_order_release);
            retiring_epoch.store(0);
        }
        return rc;
    }
};

Runtime::Runtime(ManagerConfig c, ComputeBackend b, uint32_t n) : backend_(b), mode_(c.mode) {
    layers_.reserve(n);
    for (uint32_t l = 0; l < n; ++l) layers_.emplace_back(new LayerContext(*this, l, c));
}

Runtime::~Runtime() {
    const int rc = drain();
    assert(rc != EBUSY);
    (void)rc;
}

WeightManager& Runtime::weights(uint32_t l) { return layers_.at(l)->manager; }

int Runtime::begin_layer(uint32_t l, const LayerStorage& s, LayerStep* step) {
    if (l >= layers_.size() || !step) return EINVAL;
    LayerContext& c = *layers_[l];
    if (c.life.load(std::memory_order_acquire) != LayerContext::Life::Idle) return EBUSY;
    if (const int rc = c.manager.begin_layer(l, s)) return rc;
    c.submitted = c.frozen = false;
    c.error = 0;
    c.life.store(LayerContext::Life::Open, std::memory_order_release);
    *step = LayerStep(this, l, c.manager.epoch());
    return 0;
}

int LayerStep::update_prediction(Span<GroupId> ids) { return update_prediction(ids, {}); }

int LayerStep::update_prediction(Span<GroupId> ids, PredictionUpdateOptions options) {
    if (!runtime_) return EINVAL;
    Runtime::LayerContext& c = *runtime_->layers_[layer_];
    if (!c.open_at(epoch_) || c.frozen) return EINVAL;
    return c.manager.update_prediction(ids, options);
}

int LayerStep::enqueue_compute(const void* input, void* output, void* stream) {
    if (!runtime_) return EINVAL;
    Runtime::LayerContext& c = *runtime_->layers_[layer_];
    const ComputeBackend& b = runtime_->backend_;
    if (!c.open_at(epoch_) || c.submitted || !b.enqueue || !b.complete) return EINVAL;
    c.submitted = true;   // counted as launched even if refused: abort must see completion
    const int rc = b.enqueue(b.context, layer_, input, output, stream, c.manager.core_descriptors(), c.manager.queue(),
                             epoch_, runtime_->mode_);
    if (rc) c.cancel_both(rc, epoch_);
    return rc;
}

int LayerStep::finalize(Span<GroupId> ids) {
    if (!runtime_) return EINVAL;
    Runtime::LayerContext& c = *runtime_->layers_[layer_];
    if (!c.open_at(epoch_) || c.frozen) return EINVAL;
    if (const uint32_t qe = c.queue_error()) return static_cast<int>(qe);
    const int rc = c.manager.finalize(ids);
    if (!rc)
        c.frozen = true;
    else if (c.submitted)
        c.cancel_both(rc, epoch_);
    return rc;
}

void Runtime::retire_callback(void* context, uint32_t epoch) {
    LayerContext& c = *static_cast<LayerContext*>(context);
    uint32_t expected = epoch;
    // only the retirement this commit armed, once
    if (!epoch || !c.retiring_epoch.compare_exchange_strong(expected, 0u, std::memory_order_acq_rel)) return;
    // the backend has finished its GPU use and cache installation for this epoch
    const int rc = c.manager.retire();
    Runtime& r = c.runtime;
    {
        std::lock_guard<std::mutex> lock(r.mutex_);
        c.error = rc;
        c.life.store(LayerContext::Life::Idle, std::memory_order_release);
    }
    r.retired_.notify_all();
}

int LayerStep::commit(Span<GroupId> ids) {
    if (!runtime_) return EINVAL;
    Runtime::LayerContext& c = *runtime_->layers_[layer_];
    const ComputeBackend& b = runtime_->backend_;
    if (!c.open_at(epoch_) || !c.frozen || !c.submitted || c.retiring()) return EINVAL;
    if (const uint32_t qe = c.queue_error()) return static_cast<int>(qe);
    if (ids.size > c.groups() || (ids.size && !ids.data)) return EINVAL;
    const bool deferred = b.defer_commit != nullptr;
    if (!deferred && !b.complete(b.context, layer_)) return EBUSY;
    if (const int rc = c.check_next_resident(ids, deferred)) return rc;
    return deferred ? c.finish_deferred(ids, epoch_) : c.finish_direct(ids);
}

int LayerStep::abort() {
    if (!runtime_) return EINVAL;
    Runtime::LayerContext& c = *runtime_->layers_[layer_];
    const ComputeBackend& b = runtime_->backend_;
    if (!c.open_at(epoch_) || c.retiring()) return EINVAL;
    c.manager.cancel();
    if (c.submitted) {
        if (b.cancel) b.cancel(b.context, layer_, epoch_);
        if (!b.complete(b.context, layer_)) return EBUSY;
    }
    const int rc = c.manager.retire();
    c.life.store(Runtime::LayerContext::Life::Idle, std::memory_order_release);
    return rc;
}

int Runtime::drain() {
    std::unique_lock<std::mutex> lock(mutex_);
    auto life = [](const std::unique_ptr<LayerContext>& c) { return c->life.load(std::memory_order_acquire); };
    // an open step must be committed or aborted by its owner first
    for (auto& c : layers_)
        if (life(c) == LayerContext::Life::Open) return EBUSY;
    retired_.wait(lock, [&] {
        return std::all_of(layers_.begin(), layers_.end(),
                           [&](const std::unique_ptr<LayerContext>& c) { return life(c) == LayerContext::Life::Idle; });
    });
    for (auto& c : layers_)
        if (c->error) return c->error;
    return 0;
}

}  // namespace leanstream::runtime
