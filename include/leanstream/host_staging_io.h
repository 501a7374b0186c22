// IOBackend that stages packed groups from pinned host memory into a device staging
// arena (LeanStream's IOBackend hook, weight_manager.h:14-23).
//
// It replaces the reference's O_DIRECT pread engine (src/io/stream_io.cpp) on MI355X:
// the "file" is a pinned host store, and each admitted group is one asynchronous
// host-to-device copy through a CopyEngine (hipMemcpyAsync on side streams in this
// build). Admission and state semantics follow stream_io:
//   * io_states[g]: EMPTY -> INFLIGHT at admission -> READY or ERROR at completion;
//     io_states[group_count] is the terminal errno, which stops further admissions
//     (stream_io.cpp:109-125, 129-139);
//   * update() installs a new priority rank (replacement: admission restarts at its
//     head), consume() installs the final rank and commits it; in-flight copies are
//     never cancelled (non-preemptive admission, stream_io.cpp:58-74, 189-237);
//   * at most qd copies are outstanding; a group is admitted at most once per session;
//   * the completion callback runs after the state word is READY and the bytes are
//     visible to device reads; staging slot = logical group (arena offset
//     g * staging_stride, weight_manager.cpp:93-94);
//   * retire() stops admissions and drains every outstanding copy; it does not wait
//     for the GPU (stream_io.cpp:273-278).
// A single pump thread admits, submits and polls; callbacks run on it.
#pragma once
#include "group_layout.h"
#include "weight_manager.h"
#include <memory>

namespace leanstream::runtime {

// Asynchronous host -> device mover, one call per group.
struct CopyEngine {
    void* context = nullptr;
    // Starts copying `bytes` from host `src` to device `dst` on in-flight lane `lane`
    // (lane < qd; a lane is reused only after poll reported it finished). 0 or errno.
    int (*submit)(void*, uint32_t lane, void* dst, const void* src, uint64_t bytes) = nullptr;
    // 0: the lane's bytes are complete and visible to device reads issued afterwards;
    // EAGAIN: still in flight; any other value: the copy failed with that errno.
    int (*poll)(void*, uint32_t lane) = nullptr;
};

struct StagingConfig {
    uint32_t group_count = 0;  // logical groups per layer
    uint32_t qd = 24;          // copies in flight, 1..32
    uint64_t group_bytes = 0, staging_stride = 0;
    CopyEngine engine{};
};

// What one session stages. Bound before WeightManager::begin_layer; the pointed-to
// memory must stay valid and unchanged until retire().
struct StagingLayer {
    const uint8_t* source = nullptr;   // pinned host store (the file)
    uint64_t source_bytes = 0;
    Span<GroupLayout> layout;          // file_offset = byte offset of the group in `source`
    uint8_t* staging = nullptr;        // device arena; logical group g at g * staging_stride
    uint64_t staging_bytes = 0;
    uint32_t* io_states = nullptr;     // [group_count + 1], the manager's LayerStorage::io_states
    // Optional [group_count]: earliest copy start of group g, in ns after begin(). Models
    // the latency of the tier that fills the pinned store; null = bytes already there.
    const uint64_t* arrival_ns = nullptr;
    // Optional [group_count][3]: ns after begin() of admission, copy submission and
    // completion of group g (0 = did not happen).
    uint64_t* stamps = nullptr;
};

struct StagingStatus {
    uint64_t epoch = 0, admissions = 0, completions = 0, bytes = 0, outstanding = 0;
    int32_t error = 0, ended = 0;
};

class HostStagingIO {
public:
    explicit HostStagingIO(StagingConfig);  // throws std::invalid_argument on bad geometry
    ~HostStagingIO();
    HostStagingIO(const HostStagingIO&) = delete;
    HostStagingIO& operator=(const HostStagingIO&) = delete;

    // EBUSY while a session is live (begun and not retired); EINVAL on bad layout,
    // ENOSPC when the arena or the source is too small.
    int bind_layer(const StagingLayer&);
    // The borrowed transport for ManagerConfig::io_backend (context = this object).
    IOBackend backend();
    int status(StagingStatus*) const;
    // Waits until no copy is outstanding and nothing is left to admit (debug/tests).
    int wait_idle(int timeout_ms);

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace leanstream::runtime
