// Per-layer residency and descriptor producer (LeanStream weight_manager.h:9-72).
// This implementation publishes READY groups through a borrowed IOBackend; the
// reference's O_DIRECT stream engine is not part of this library, so an empty
// io_backend is rejected at construction.
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#pragma once
#include "execution_queue.h"
#include "group_layout.h"
#include <memory>

namespace leanstream::runtime {

// Values of the per-group io_states words (group_count + 1 terminal error word).
enum IoStateWord : uint32_t { kIoEmpty = 0, kIoInflight = 1, kIoReady = 2, kIoError = 3 };

struct IOCompletion {
    uint32_t epoch;
    GroupId logical_group;
    SlotId staging_slot;
    int error;
    uint64_t slot_sequence;
};
using IOCompletionCallback = void (*)(void*, const IOCompletion&);

// Borrowed transport: one call per update/phase, never per-group virtual dispatch.
struct IOBackend {
    void* context = nullptr;
    int (*begin)(void*, IOCompletionCallback, void*, uint32_t epoch) = nullptr;
    int (*update)(void*, Span<GroupId>) = nullptr;
    int (*consume)(void*, Span<GroupId>) = nullptr;
    int (*retire)(void*) = nullptr;
    SlotId (*ready_slot)(void*, GroupId) = nullptr;
    uint64_t (*requests)(void*) = nullptr;
    int (*wait)(void*, int timeout_ms) = nullptr;
};

struct ManagerConfig {
    uint32_t group_count, qd = 24;
    uint64_t group_bytes, staging_stride, alignment = 512;
    ConsumerMode mode = ConsumerMode::BatchCompat;
    IOBackend io_backend{};
};

struct LayerStorage {
    int fd = -1;
    Span<GroupLayout> layout;
    const SlotId* cache_slots = nullptr;          // immutable through the step
    void* staging = nullptr;
    uint32_t* io_states = nullptr;                // group_count + terminal error word
    Span<GroupId> core;
    DeviceExecQueue queue;
    ExecDesc* mapped_core_descriptors = nullptr;  // optional GPU-visible core table
    const SlotId* destination_slots = nullptr;    // optional, indexed by logical id
    uint64_t layout_generation = 0;               // nonzero: immutable registered layout
    uint64_t plan_generation = 0;                 // nonzero: reuse a prepared core plan
    uint64_t staging_bytes = 0;                   // nonzero: validated staging capacity
};

struct PredictionUpdateOptions {
    uint32_t io_budget = UINT32_MAX;  // max new EMPTY candidates admitted
    uint32_t execution_epoch = 0;     // zero: current epoch
    uint32_t diagnostic_point = 0;    // opaque label
};

class WeightManager {
public:
    explicit WeightManager(ManagerConfig);
    ~WeightManager();
    WeightManager(const WeightManager&) = delete;
    WeightManager& operator=(const WeightManager&) = delete;
    int prepare_layer(const LayerStorage&);
    int begin_layer(uint32_t layer, const LayerStorage&);
    int update_prediction(Span<GroupId>);
    int update_prediction(Span<GroupId>, PredictionUpdateOptions);
    int finalize(Span<GroupId> final_groups);
    int retire();
    void cancel(int error = 0);
    GroupState group_state(GroupId) const;
    uint64_t prediction_generation() const;
    uint32_t epoch() const;
    DeviceExecQueue queue() const;
    Span<ExecDesc> core_descriptors() const;
    int wait_io(int timeout_ms);
    uint64_t read_requests() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace leanstream::runtime
