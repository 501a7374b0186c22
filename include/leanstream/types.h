// Core value types shared by the control runtime and the HIP compute backend.
// Layout-compatible with LeanStream's include/leanstream/types.h:5-20 so that
// callers compiled against that header bind to this implementation unchanged.
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#pragma once
#include <cstddef>
#include <cstdint>

namespace leanstream::runtime {

using GroupId = int32_t;  // logical group identifier chosen by the predictor
using SlotId = int32_t;   // cache / staging slot index, negative = none

// Borrowed contiguous view; never owns storage.
template <class T>
struct Span {
    const T* data = nullptr;
    size_t size = 0;
    const T& operator[](size_t i) const { return data[i]; }
};

enum class IOState : uint8_t { Empty, Inflight, Ready };
enum class SourceKind : uint32_t { Cache, Staging };
enum class ConsumerMode : uint8_t { BatchCompat, Progressive, Auto };

struct GroupState {
    SlotId cache_slot = -1;
    SlotId staging_slot = -1;
    IOState io_state = IOState::Empty;
};

// One unit of work for the MLP kernels: five 32-bit words, read by the GPU.
struct ExecDesc {
    uint32_t logical_group;   // predictor-visible identity
    uint32_t physical_group;  // selects the fp16 scale rows
    uint32_t source_slot;     // slot inside the cache or staging arena
    uint32_t dest_slot;       // deterministic partial row / reduction position
    SourceKind source_kind;   // which arena holds the packed bytes
};
static_assert(sizeof(ExecDesc) == 20, "ExecDesc is five 32-bit words");

}  // namespace leanstream::runtime
