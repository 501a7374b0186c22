// O(1) kernel selection (LeanStream src/runtime/kernel_selector.cpp:4-22).
// No allocation, locking, string handling or device calls.
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#include "leanstream/kernel_selector.h"
#include <limits>

namespace leanstream::runtime {

uint32_t quantize_io_load(uint32_t remaining, uint32_t total, uint32_t buckets) noexcept {
    if (total == 0 || buckets == 0) return 0;
    if (remaining >= total) return buckets - 1;
    return static_cast<uint32_t>(static_cast<uint64_t>(remaining) * buckets / total);
}

KernelCandidate KernelSelector::candidate(uint32_t id) const noexcept {
    if (id == fallback_.id) return fallback_;  // the backend's own default geometry
    if (candidates_.data == nullptr || id >= candidates_.size) return fallback_;
    const KernelCandidate& c = candidates_[id];
    const bool usable = c.id == id && c.available && c.workers != 0;
    return usable ? c : fallback_;
}

uint32_t KernelSelector::select(const KernelRuntimeState& s) const noexcept {
    const bool in_table = table_.entries != nullptr && s.layer < table_.layers && s.io_bucket < table_.io_buckets;
    const bool overflow =
        table_.io_buckets != 0 && static_cast<size_t>(table_.layers) > std::numeric_limits<size_t>::max() / table_.io_buckets;
    if (!in_table || overflow) return fallback_.id;
    const uint8_t entry = table_.entries[static_cast<size_t>(s.layer) * table_.io_buckets + s.io_bucket];
    return candidate(entry).id;
}

}  // namespace leanstream::runtime
