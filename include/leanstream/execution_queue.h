// Ready queue shared between the CPU producer and the GPU consumer.
// Word layout follows LeanStream include/leanstream/execution_queue.h:5-34:
//   u32[0] ready_count, u32[2] total_count, u32[3] epoch, u32[4] batch_epoch,
//   u32[5] error, u32[6] consumer_path, byte 64 claim_count, 128 bytes total.
// The MI355X backend keeps this block in fine-grained coherent host memory; the
// CPU publishes with release stores and the GPU polls with system-scope loads.
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#pragma once
#include "types.h"

namespace leanstream::runtime {

struct alignas(64) QueueControl {
    uint32_t ready_count = 0, reserved = 0, total_count = 0, epoch = 0;
    uint32_t batch_epoch = 0, error = 0, consumer_path = 0, init_arrived = 0, init_epoch = 0;
    alignas(64) uint32_t claim_count = 0;  // separate line from the CPU-written words
};
static_assert(offsetof(QueueControl, epoch) == 12, "epoch is word 3");
static_assert(offsetof(QueueControl, claim_count) == 64, "claim_count on its own line");
static_assert(sizeof(QueueControl) == 128, "two cache lines");

struct DeviceExecQueue {
    ExecDesc* descriptors = nullptr;   // final non-core descriptors, in final order
    uint32_t* ready_indices = nullptr; // descriptor indices in publication order
    QueueControl* control = nullptr;
    uint32_t capacity = 0;
};

// Serialized CPU producer. Publication never allocates.
class ExecutionQueue {
public:
    explicit ExecutionQueue(DeviceExecQueue view = {}) : view_(view) {}
    void bind(DeviceExecQueue view) { view_ = view; }
    DeviceExecQueue device_view() const { return view_; }
    void reset(uint32_t epoch);
    void prepare(uint32_t total);
    void append_unpublished(uint32_t index);
    void activate();
    void seal(uint32_t total);
    void publish_all();
    void publish(uint32_t index);
    void fail(uint32_t error);

private:
    DeviceExecQueue view_;
    uint32_t tail_ = 0, epoch_ = 0, total_ = 0;
};

}  // namespace leanstream::runtime
