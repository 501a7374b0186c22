// CopyEngines for HostStagingIO on MI355X (host -> device copies of packed groups).
//
// SdmaCopyEngine drives the SDMA copy engines directly through ROCr
// (hsa_amd_memory_async_copy_on_engine, the routine hipMemcpyAsync itself ends in), one
// completion signal per in-flight lane, lanes spread round robin over `engines` SDMA
// engines. No HIP stream or hardware compute queue is involved, so a copy can never be
// ordered behind the persistent consumer kernel that waits for it, and no copy ever needs
// a compute unit.
//
// HipCopyEngine issues hipMemcpyAsync on `streams` side streams (default priority,
// non-blocking with respect to the null stream), one event per lane. Streams share the
// process's hardware queues (GPU_MAX_HW_QUEUES, 4 by default): a copy stream that shares
// one with the stream running the consumer leaves copies queued behind that kernel until
// its bounded waits expire. At most kMaxHipCopyStreams streams are accepted (with the null
// stream and the consumer's stream that fills the default four queues); the SDMA engine
// has no such hazard and is the one to use.
#pragma once
#include "host_staging_io.h"

namespace leanstream::runtime {

inline constexpr uint32_t kMaxHipCopyStreams = 2;

class SdmaCopyEngine {
public:
    // `device` is the HIP device ordinal whose memory receives the copies; `lanes` >= the
    // transport's qd; `engines` SDMA engines used round robin (1..16, clamped to the
    // engines ROCr reports for host -> device); `chunk_bytes` > 0 cuts a group into
    // pieces of that size on successive engines (one engine moves a few GB/s, so pieces
    // shorten a group's latency). Throws std::runtime_error on failure.
    SdmaCopyEngine(int device, uint32_t lanes, uint32_t engines, uint64_t chunk_bytes = 0);
    ~SdmaCopyEngine();
    SdmaCopyEngine(const SdmaCopyEngine&) = delete;
    SdmaCopyEngine& operator=(const SdmaCopyEngine&) = delete;
    CopyEngine view();
    uint32_t engines() const;

private:
    struct Impl;
    Impl* impl_ = nullptr;
};

class HipCopyEngine {
public:
    // `lanes` >= the transport's qd; `streams` copy streams used round robin
    // (1..kMaxHipCopyStreams).
    // Throws std::runtime_error when a stream or event cannot be created.
    HipCopyEngine(int device, uint32_t lanes, uint32_t streams);
    ~HipCopyEngine();
    HipCopyEngine(const HipCopyEngine&) = delete;
    HipCopyEngine& operator=(const HipCopyEngine&) = delete;
    CopyEngine view();

private:
    struct Impl;
    Impl* impl_ = nullptr;
};

}  // namespace leanstream::runtime
