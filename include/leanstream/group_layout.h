// Registration record for one packed group on storage (LeanStream group_layout.h:4).
#pragma once
#include "types.h"

namespace leanstream::runtime {
struct GroupLayout {
    uint32_t logical_group, physical_group;
    uint64_t file_offset;
    uint32_t bytes;
};
}  // namespace leanstream::runtime
