// Registration record for one packed group on storage (LeanStream group_layout.h:4).
// Interface kept alike with LeanStream's (MIT, Copyright (c) 2026 LeanStream Authors): see THIRD_PARTY_NOTICES.md.
#pragma once
#include "types.h"

namespace leanstream::runtime {
struct GroupLayout {
    uint32_t logical_group, physical_group;
    uint64_t file_offset;
    uint32_t bytes;
};
}  // namespace leanstream::runtime
