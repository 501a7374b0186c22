// CPU producer of the ready queue (LeanStream src/runtime/execution_queue.cpp:4-46).
//
// Publication protocol shared with the GPU consumer:
//   * prepare(total) stores the final descriptor count before anything is published;
//   * activate() release-stores ready_count (the initial prefix) and then epoch, so a
//     consumer that observes the epoch also observes total_count and the prefix;
//   * publish(i) appends i to ready_indices and release-stores ready_count; the
//     batch_epoch word is released when the last descriptor is published;
//   * fail(e) records the first error only.
// Callers serialise producers; descriptor contents and weight bytes must already be
// visible to the GPU before their index is published.
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#include "leanstream/execution_queue.h"
#include <cassert>

namespace leanstream::runtime {

namespace {
inline void release(uint32_t* word, uint32_t value) { __atomic_store_n(word, value, __ATOMIC_RELEASE); }
}  // namespace

void ExecutionQueue::reset(uint32_t epoch) {
    assert(view_.control && view_.descriptors && view_.ready_indices && epoch);
    QueueControl& c = *view_.control;
    epoch_ = epoch;
    tail_ = 0;
    total_ = 0;
    release(&c.epoch, 0);  // stale consumers stop matching before the words below change
    c.ready_count = 0;
    c.reserved = 0;
    c.total_count = 0;
    c.batch_epoch = 0;
    c.error = 0;
    c.consumer_path = 0;
    c.init_arrived = 0;
    c.init_epoch = 0;
    c.claim_count = 0;
}

void ExecutionQueue::prepare(uint32_t total) {
    assert(total <= view_.capacity);
    total_ = total;
    view_.control->total_count = total;
}

void ExecutionQueue::append_unpublished(uint32_t index) {
    assert(tail_ < total_ && index < total_);
#ifdef LEANSTREAM_RUNTIME_TESTING
    for (uint32_t k = 0; k < tail_; ++k) assert(view_.ready_indices[k] != index);
#endif
    view_.ready_indices[tail_] = index;
    ++tail_;
}

void ExecutionQueue::activate() {
    QueueControl& c = *view_.control;
    release(&c.ready_count, tail_);
    release(&c.epoch, epoch_);
    if (tail_ == total_) release(&c.batch_epoch, epoch_);
}

void ExecutionQueue::seal(uint32_t total) {
    prepare(total);
    activate();
}

void ExecutionQueue::publish_all() {
    assert(tail_ == 0);
    for (uint32_t k = 0; k < total_; ++k) view_.ready_indices[k] = k;
    tail_ = total_;
    release(&view_.control->ready_count, tail_);
    release(&view_.control->batch_epoch, epoch_);
}

void ExecutionQueue::publish(uint32_t index) {
    assert(tail_ < total_ && index < total_);
#ifdef LEANSTREAM_RUNTIME_TESTING
    for (uint32_t k = 0; k < tail_; ++k) assert(view_.ready_indices[k] != index);
#endif
    view_.ready_indices[tail_] = index;
    ++tail_;
    release(&view_.control->ready_count, tail_);
    if (tail_ == total_) release(&view_.control->batch_epoch, epoch_);
}

void ExecutionQueue::fail(uint32_t error) {
    uint32_t expected = 0;
    __atomic_compare_exchange_n(&view_.control->error, &expected, error, false, __ATOMIC_RELEASE, __ATOMIC_RELAXED);
}

}  // namespace leanstream::runtime
