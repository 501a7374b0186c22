// Device building blocks of the gfx950 streaming sparse INT4 MLP kernels, shared by the
// per-layer persistent kernels (streaming_mlp.hip) and the multi-layer chain kernel
// (chain_mlp.hip): memory helpers, exact INT4 dequantisation, gate/up and down-projection
// items (register and LDS-staged walks), the deterministic fixed-point column reduction,
// descriptor access and validation, and the ready-queue mirror and claim protocol.
// Everything here is inline device code; kernels and host code live in the .hip files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "mlp_args.h"

namespace lsamd {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kWgPerCu = 2;          // resident workgroups per CU (register budget 256 per lane)
constexpr int kDnRows = 64;          // rows of one down-item pass: 8 row groups x 8 rows
constexpr int kDescItems = 12;       // item descriptors fetched per round trip (5 words each)
// LDS per wave of the non-staged walks (16-byte vectors): a down item's 256 column sums for
// the re-deal, then (batch rows) the rows' fp16 h for down items shared by the rows.
template <int NB>
constexpr int kNonStagedWaveVecs = (kDnCols * 4 + (NB > 1 ? NB * kDnRows * 2 : 0)) / 16;
constexpr bool kSplitRoles = false;  // all-ready path: gate/up and down items on different workgroups
#ifndef LS_GU_HALVES
#define LS_GU_HALVES 1
#endif
constexpr bool kGuHalves = LS_GU_HALVES;  // one-pass gate/up items are loaded in two halves (GuHalf)
static_assert(kDnCols == 256, "a down item is two scale blocks wide");

// ---------------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------------
// The global-memory view of a pointer (device or host-mapped memory, never LDS). A pointer
// whose address space the compiler cannot infer -- one read from memory, or rebuilt from
// its scalar halves -- is accessed with flat instructions, and flat loads, stores and
// atomics count in lgkmcnt as well as vmcnt: a wave's wait for its own LDS accesses would
// then also wait for them to complete in memory. Through this view they are global
// instructions, counted in vmcnt only.
#if defined(__HIP_DEVICE_COMPILE__)
#define LS_GLOBAL __attribute__((address_space(1)))
#else
#define LS_GLOBAL   // the host pass compiles no device code; address space 1 means something else there
#endif
template <class T>
__device__ __forceinline__ LS_GLOBAL T* glb(T* p) {
    return (LS_GLOBAL T*)p;
}

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(glb(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_agent(const float* p) {
    return __uint_as_float(ld_agent(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void stf_agent(float* p, float v) {
    st_agent(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ uint32_t ld_sys(const uint32_t* p) {
    return __hip_atomic_load(glb(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ld_sys64(const uint32_t* p) {
    return __hip_atomic_load(glb(reinterpret_cast<const uint64_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// All of this thread's earlier memory operations have completed at their point of
// coherence (stores acknowledged, loads returned).
__device__ __forceinline__ void drain_vmem() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint64_t now_ticks() { return wall_clock64(); }

__device__ __forceinline__ u32x4 ld_stream16(const uint8_t* p) {
    return __builtin_nontemporal_load(glb(reinterpret_cast<const u32x4*>(p)));
}
// A plain (L2-retained) 16-byte load, for weight lines that are consumed by several
// instructions (a streaming load may drop the line after its first piece is read).
__device__ __forceinline__ u32x4 ld_cached16(const uint8_t* p) { return *glb(reinterpret_cast<const u32x4*>(p)); }
__device__ __forceinline__ u32x2 ld_stream8(const uint8_t* p) {
    return __builtin_nontemporal_load(glb(reinterpret_cast<const u32x2*>(p)));
}
__device__ __forceinline__ uint32_t ld_stream4(const uint8_t* p) {
    return __builtin_nontemporal_load(glb(reinterpret_cast<const uint32_t*>(p)));
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ _Float16 half_bits(uint16_t v) { return __builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ float round_half(float v) { return (float)(_Float16)v; }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// The wave's index in the workgroup, in a scalar register (the compiler cannot tell that
// threadIdx.x >> 6 is uniform across a wave, and would keep everything derived from it in
// vector registers).
__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
// Lane 0's value for the whole wave (call with lane 0 active).
__device__ __forceinline__ uint32_t wave_bcast(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// One v_bitop3 per pair: magic(w, A, M) = A ? (w ^ M) : M bitwise (truth table 0x6A over
// (w, A, M)). Inside the nibble mask A it flips each nibble's sign bit (two's complement
// -> offset binary q + 8); outside it lays down the fp16 exponent of M. Low nibbles
// become 1024 + (q + 8), high nibbles (mantissa bits 4-7 under exponent 64) 64 + (q + 8);
// the bias subtraction is exact and the scale product is the one rounding.
__device__ __forceinline__ uint32_t magic(uint32_t w, uint32_t mask, uint32_t m) {
    return __builtin_amdgcn_bitop3_b32(w, mask, m, 0x6A);
}

// Exact dequantisation of eight signed nibbles (one 32-bit word) into four fp16
// pairs: out[k] = (w(col k), w(col k+4)) when the word holds one row, or
// (row a, row b) of one column when the halves of the word come from two rows.
__device__ __forceinline__ void dequant8(uint32_t word, h2 s, h2 out[4]) {
    const uint32_t w8 = word >> 8;
    const h2 lo_bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2 hi_bias = {(_Float16)-72.0f, (_Float16)-72.0f};
    out[0] = (as_h2(magic(word, 0x000F000Fu, 0x64086408u)) + lo_bias) * s;
    out[1] = (as_h2(magic(word, 0x00F000F0u, 0x54805480u)) + hi_bias) * s;
    out[2] = (as_h2(magic(w8, 0x000F000Fu, 0x64086408u)) + lo_bias) * s;
    out[3] = (as_h2(magic(w8, 0x00F000F0u, 0x54805480u)) + hi_bias) * s;
}

__device__ __forceinline__ float dot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// Waits until every vector memory load this wave issued has returned (s_waitcnt vmcnt(0);
// expcnt and lgkmcnt at their maxima). The scheduling barriers keep the loads after it
// from being hoisted above the wait.
__device__ __forceinline__ void wait_vector_loads() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------------
// bounded waiting
// ---------------------------------------------------------------------------------
// A bounded wait. The 100 MHz clock is a scalar memory read (s_memrealtime) whose latency
// under a loaded memory system approaches a microsecond, and while one is in flight the
// wave's next LDS access waits too (both count in lgkmcnt). So a wait reads the clock -- and
// looks at its abort flag, where it has one -- only on every kWaitStride-th check (due()):
// a wait that ends sooner reads neither, a long one pays one clock read per kWaitStride
// polls. The bound runs from the first clock read.
constexpr uint32_t kWaitStride = 16;
struct Waiter {
    uint64_t start = 0, limit;
    uint32_t n = 0;
    __device__ explicit Waiter(uint64_t lim) : limit(lim) {}
    __device__ bool due() { return (++n & (kWaitStride - 1u)) == 0u; }
    __device__ bool over() {   // on a due check: has the bound passed?
        const uint64_t t = now_ticks();
        if (!start) {
            start = t;
            return false;
        }
        return t - start > limit;
    }
    __device__ bool expired() { return due() && over(); }
};

__device__ __forceinline__ void stamp(const MlpArgs& a, uint32_t k) {
    if (a.stamps && (threadIdx.x & 63) == 0 && k < kStampSlots)
        a.stamps[(blockIdx.x * kWaves + (threadIdx.x >> 6)) * kStampSlots + k] = now_ticks();
}

// Error path only: the bit is ordered before everything the lane stores afterwards (its
// count-out, a completion word), so a host that sees the launch complete sees the bit.
__device__ __forceinline__ void raise_status(const MlpArgs& a, uint32_t* slot, uint32_t bit) {
    __hip_atomic_fetch_or(glb(a.status), bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
    st_agent(slot + kSyncAbort, 1u);
}

// Lane 0 of the wave checks, on a due check of the wait, whether it must be abandoned (abort
// flag or spin limit exceeded; the latter raises the timeout status). Wave-uniform result:
// every lane counts the same checks.
__device__ __forceinline__ bool wave_should_stop(const MlpArgs& a, uint32_t* slot, Waiter& wt) {
    if (!wt.due()) return false;
    uint32_t st = 0;
    if (lane_id() == 0) {
        if (ld_agent(slot + kSyncAbort)) {
            st = 1;
        } else if (wt.over()) {
            raise_status(a, slot, kStatusTimeout);
            st = 1;
        }
    }
    return __builtin_amdgcn_readfirstlane(st) != 0;
}

// ---------------------------------------------------------------------------------
// Gate/up items. A width-D row of one projection is CPR 16-byte chunks; LPR lanes share a
// row (CPL chunks each), so one wave pass covers NPW neurons; an item is RPL passes
// (about 8 KB of gate/up weights), NPI neurons.
// ---------------------------------------------------------------------------------
template <int D>
struct GuGeom {
    static constexpr int CPR = D / 32;                 // 16-byte chunks per projection row
    static constexpr int LPR = CPR < 64 ? CPR : 64;    // lanes sharing one row
    static constexpr int CPL = CPR / LPR;              // chunks per lane per row
    static constexpr int NPW = 64 / LPR;               // neurons per wave pass
    static constexpr int RPL = CPL >= 4 ? 1 : 4 / CPL;  // passes per item: 32 * CPL * RPL = 128 bytes per lane
    static constexpr int NPI = NPW * RPL;              // neurons per gate/up item
    static constexpr int BLOCKS = D / 128;             // scale blocks per row
    static_assert(D % 256 == 0 && CPR >= 8, "width must be a multiple of 256");
};

// x (every batch row) is shared by the workgroup through LDS, as (k, k+4) fp16 pairs to
// match dequant8, in the order gu_dots reads it: block (k, g) of lane r (words
// 4g .. 4g+3 of its chunk k, x columns 32 (r + LPR k) + 8g .. + 7) of row b at
// xl[b N + (4k + g) LPR + r], so a wave's 64 lanes read 1 KB of consecutive LDS per block.
// Each wave loads a quarter of row 0 as raw 16-byte pieces into registers at its start,
// and every fourth 64-piece block of rows 1 .. batch-1 straight into LDS
// (global_load_lds); once they must have landed (after the wave's first descriptors,
// loaded later and completed in order, or when it leaves) it writes / pairs them in place
// and counts itself in (stage_x); a wave about to compute gate/up waits until all four
// waves are in.
template <int D>
struct XGeom {
    static constexpr int N = D / 8;                               // 16-byte pieces of one row of x
    static constexpr int PER = (N + kThreads - 1) / kThreads;   // row-0 pieces per thread
    static constexpr int INSTR = (N + 63) / 64;                   // 64-piece blocks per row
};

template <int D>
struct XPart {
    u32x4 v[XGeom<D>::PER];
    bool staged;
};

// LDS position of piece `raw` of a row (and back).
template <int D>
__device__ __forceinline__ uint32_t x_position(uint32_t raw) {
    using Gm = GuGeom<D>;
    const uint32_t c = raw >> 2, g = raw & 3, r = c % Gm::LPR, k = c / Gm::LPR;
    return (4 * k + g) * Gm::LPR + r;
}
template <int D>
__device__ __forceinline__ uint32_t x_raw(uint32_t pos) {
    using Gm = GuGeom<D>;
    const uint32_t blk = pos / Gm::LPR, r = pos % Gm::LPR, k = blk >> 2, g = blk & 3;
    return 4 * (r + Gm::LPR * k) + g;
}

__device__ __forceinline__ u32x4 pair_halves(u32x4 w) {   // (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
    return u32x4{__builtin_amdgcn_perm(w.z, w.x, 0x05040100u), __builtin_amdgcn_perm(w.z, w.x, 0x07060302u),
                 __builtin_amdgcn_perm(w.w, w.y, 0x05040100u), __builtin_amdgcn_perm(w.w, w.y, 0x07060302u)};
}

template <int D>
__device__ __forceinline__ void load_x(const uint16_t* x, uint32_t batch, XPart<D>& xp, u32x4* xl) {
    using Xg = XGeom<D>;
    const LS_GLOBAL u32x4* src = glb(reinterpret_cast<const u32x4*>(x));
#pragma unroll
    for (int j = 0; j < Xg::PER; ++j) {
        const int i = threadIdx.x + j * kThreads;
        xp.v[j] = i < Xg::N ? src[i] : u32x4{0, 0, 0, 0};
    }
    xp.staged = false;
    const uint32_t lane = lane_id();
    for (uint32_t j = wave_id(); j < (batch - 1) * Xg::INSTR; j += kWaves) {
        const uint32_t row = 1 + j / Xg::INSTR, pos = (j % Xg::INSTR) * 64 + lane;
        if (pos < (uint32_t)Xg::N) {
            typedef __attribute__((address_space(3))) void* lds_ptr;
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const void*>(reinterpret_cast<const u32x4*>(x) + (size_t)row * Xg::N + x_raw<D>(pos)),
                                             (lds_ptr)(xl + row * Xg::N + (pos - lane)), 16, 0, 0);
        }
    }
}

template <int D>
__device__ __forceinline__ void stage_x(XPart<D>& xp, uint32_t batch, u32x4* xl, uint32_t* count) {
    using Xg = XGeom<D>;
    if (xp.staged) return;
    // The pairing below must not be hoisted above the wave's first descriptor loads (the
    // compiler would, to share it between the call sites): it waits for x, and the
    // descriptors would then be requested only after x arrived. The empty asm pins the
    // registers here; its memory clobber keeps the loads issued before it ahead of it.
#pragma unroll
    for (int j = 0; j < Xg::PER; ++j) asm volatile("" : "+v"(xp.v[j]) : : "memory");
#pragma unroll
    for (int j = 0; j < Xg::PER; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < Xg::N) xl[x_position<D>(i)] = pair_halves(xp.v[j]);
    }
    if (batch > 1) {
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's LDS loads of rows 1.. have landed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const uint32_t lane = lane_id();
        for (uint32_t j = wave_id(); j < (batch - 1) * Xg::INSTR; j += kWaves) {
            const uint32_t row = 1 + j / Xg::INSTR, pos = (j % Xg::INSTR) * 64 + lane;
            if (pos < (uint32_t)Xg::N) xl[row * Xg::N + pos] = pair_halves(xl[row * Xg::N + pos]);
        }
    }
    // A wave's LDS operations execute in order, so the count is raised after its stores
    // land; the fence keeps the compiler from reordering them.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane_id() == 0) __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    xp.staged = true;
}

// Waits until every wave of the workgroup has staged its part of x. Every wave stages its
// part before it can wait for anything else, so this ends; the wall-clock bound only
// guards against a broken invariant.
__device__ __forceinline__ bool wait_x(const MlpArgs& a, uint32_t* slot, const uint32_t* count) {
    if (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= (uint32_t)kWaves) return true;
    Waiter wt(a.spin_limit);
    while (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (uint32_t)kWaves) {
        if (wt.expired()) {
            if (lane_id() == 0) raise_status(a, slot, kStatusTimeout);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}

template <int D>
struct GuItem {
    u32x4 w[GuGeom<D>::RPL][2][GuGeom<D>::CPL];
    uint32_t s[GuGeom<D>::RPL][2][GuGeom<D>::CPL];   // fp16 bits (32-bit registers)
};

// Halves of a gate/up item, loaded one after the other: H = 1 is the first half, H = 2
// the second, H = 0 the whole item. Items of several passes split by pass, one-pass items
// (D >= 8192) by chunk. A wave issues the second half when the first has landed and
// computes the first while the second streams, so only half an item's arithmetic is
// left once the layer's last weight bytes arrive.
template <int D, int H>
struct GuHalf {
    using Gm = GuGeom<D>;
    static constexpr bool BY_PASS = Gm::RPL >= 2;
    static constexpr int P0 = (H == 2 && BY_PASS) ? Gm::RPL / 2 : 0;
    static constexpr int P1 = (H == 1 && BY_PASS) ? Gm::RPL / 2 : Gm::RPL;
    static constexpr int K0 = (H == 2 && !BY_PASS) ? Gm::CPL / 2 : 0;
    static constexpr int K1 = (H == 1 && !BY_PASS) ? Gm::CPL / 2 : Gm::CPL;
    static_assert(BY_PASS || Gm::CPL >= 2, "an item splits by pass or by chunk");
};

// A wave-uniform pointer, in scalar registers: loads then take a scalar base plus a
// 32-bit per-lane offset (the values are uniform; the compiler cannot always prove it).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Issue every load of a gate/up item: neurons n0 .. n0 + nvalid - 1 of the unit whose
// packed bytes start at grp and scale rows at sc; pass p covers neurons n0 + p NPW + sub.
// A full item (every neuron valid) needs no per-lane guard. H selects the half (GuHalf).
template <int D, int H>
__device__ __forceinline__ void gu_issue(const uint8_t* grp, const uint16_t* sc, int n0, int nvalid, GuItem<D>& L) {
    using Gm = GuGeom<D>;
    using Hf = GuHalf<D, H>;
    const int lane = lane_id();
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
    if (nvalid == Gm::NPI) {
#pragma unroll
        for (int p = Hf::P0; p < Hf::P1; ++p) {
            const uint8_t* row = uniform_ptr(grp + (size_t)(n0 + p * Gm::NPW) * (3 * D / 2));
            const LS_GLOBAL uint16_t* srow = glb(uniform_ptr(sc + (size_t)(n0 + p * Gm::NPW) * 3 * Gm::BLOCKS));
            const uint32_t wo = (uint32_t)sub * (3 * D / 2) + 16 * r, so = (uint32_t)sub * 3 * Gm::BLOCKS + (r >> 2);
#pragma unroll
            for (int k = Hf::K0; k < Hf::K1; ++k) {
                L.w[p][0][k] = ld_stream16(row + wo + 16 * Gm::LPR * k);
                L.w[p][1][k] = ld_stream16(row + wo + 16 * Gm::LPR * k + D / 2);
                L.s[p][0][k] = srow[so + (Gm::LPR / 4) * k];
                L.s[p][1][k] = srow[so + (Gm::LPR / 4) * k + Gm::BLOCKS];
            }
        }
        return;
    }
#pragma unroll
    for (int p = Hf::P0; p < Hf::P1; ++p) {
        const int nu = p * Gm::NPW + sub;
        const bool ok = nu < nvalid;
        const int n = n0 + (ok ? nu : 0);
        const uint8_t* row = grp + (size_t)n * (3 * D / 2);
        const LS_GLOBAL uint16_t* srow = glb(sc + (size_t)n * 3 * Gm::BLOCKS);
#pragma unroll
        for (int k = Hf::K0; k < Hf::K1; ++k) {
            const int chunk = r + Gm::LPR * k;
            if (ok) {
                L.w[p][0][k] = ld_stream16(row + 16 * chunk);
                L.w[p][1][k] = ld_stream16(row + D / 2 + 16 * chunk);
                L.s[p][0][k] = srow[chunk >> 2];
                L.s[p][1][k] = srow[Gm::BLOCKS + (chunk >> 2)];
            } else {
                L.w[p][0][k] = u32x4{0, 0, 0, 0};
                L.w[p][1][k] = u32x4{0, 0, 0, 0};
                L.s[p][0][k] = 0;
                L.s[p][1][k] = 0;
            }
        }
    }
}

// x + the value of another lane chosen by a DPP control (row_mask limits the rows
// updated; rows outside it add 0).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

// Sum over each group of LPR consecutive lanes (LPR a power of two <= 64), valid in the
// group's last lane: a butterfly inside 16-lane rows (quad_perm, row_half_mirror,
// row_mirror), then row_bcast15 / row_bcast31 across rows. Fixed order, so the result
// does not depend on timing.
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
    if (LPR >= 2) x = dpp_add<0xB1>(x);          // quad_perm [1,0,3,2]
    if (LPR >= 4) x = dpp_add<0x4E>(x);          // quad_perm [2,3,0,1]
    if (LPR >= 8) x = dpp_add<0x141>(x);         // row_half_mirror
    if (LPR >= 16) x = dpp_add<0x140>(x);        // row_mirror
    if (LPR >= 32) x = dpp_add<0x142, 0xA>(x);   // row_bcast15 into rows 1 and 3
    if (LPR >= 64) x = dpp_add<0x143, 0xC>(x);   // row_bcast31 into rows 2 and 3
    return x;
}

// Finish a gate/up item: dot products, row reductions, activation. Publishes h of
// neurons n0 .. n0 + nvalid - 1 into hrow, each word tagged with the launch sequence
// (the word is its own ready flag).
// With NB > 1 the item's weights are dequantised once and multiplied with x of each of
// the nb batch rows (xl: row 0; row b at xl + b N); h of row b goes to hrow + b G.
// gu_dots adds the dot products of half H of the item (GuHalf) into acc; gu_finish
// reduces and publishes.
template <int D, int NB, int H>
__device__ __forceinline__ void gu_dots(const GuItem<D>& L, const u32x4* xl, uint32_t nb,
                                        float (&acc)[NB][GuGeom<D>::RPL][2]) {
    using Gm = GuGeom<D>;
    using Hf = GuHalf<D, H>;
    const int r = lane_id() % Gm::LPR;
#pragma unroll
    for (int k = Hf::K0; k < Hf::K1; ++k) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t xw[NB][4];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (NB == 1 || (uint32_t)b < nb) {
                    const u32x4 xv = xl[b * XGeom<D>::N + (4 * k + g) * Gm::LPR + r];   // paired (stage_x)
                    xw[b][0] = xv.x;
                    xw[b][1] = xv.y;
                    xw[b][2] = xv.z;
                    xw[b][3] = xv.w;
                }
            }
#pragma unroll
            for (int p = Hf::P0; p < Hf::P1; ++p) {
#pragma unroll
                for (int proj = 0; proj < 2; ++proj) {
                    const _Float16 sv = half_bits((uint16_t)L.s[p][proj][k]);
                    const h2 s2 = {sv, sv};
                    const u32x4 v = L.w[p][proj][k];
                    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
                    h2 w[4];
                    dequant8(words[g], s2, w);
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        if (NB == 1 || (uint32_t)b < nb) {
#pragma unroll
                            for (int q = 0; q < 4; ++q) acc[b][p][proj] = dot2(w[q], as_h2(xw[b][q]), acc[b][p][proj]);
                        }
                    }
                }
            }
        }
    }
}

template <int D, int NB>
__device__ __forceinline__ void gu_finish(float (&acc)[NB][GuGeom<D>::RPL][2], uint64_t* hrow, uint32_t G, int n0,
                                          int nvalid, uint32_t seq, uint32_t nb) {
    using Gm = GuGeom<D>;
    const int lane = lane_id();
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (NB > 1 && (uint32_t)b >= nb) break;
#pragma unroll
        for (int p = 0; p < Gm::RPL; ++p) {
            const float gsum = group_sum<Gm::LPR>(acc[b][p][0]);
            const float usum = group_sum<Gm::LPR>(acc[b][p][1]);
            const int nu = p * Gm::NPW + sub;
            if (r == Gm::LPR - 1 && nu < nvalid) {
                const float g = round_half(gsum);
                const float u = round_half(usum);
                const float sl = round_half(g / (1.0f + __expf(-g)));
                const float h = round_half(sl * u);
                __hip_atomic_store(hrow + b * G + n0 + nu, ((uint64_t)seq << 32) | __float_as_uint(h),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// Down items: one 256-column tile (two scale blocks) of one unit. A pass covers 64 rows:
// lane 8 g + dc holds columns 32 dc .. 32 dc + 31 (one 16-byte load per row, so every
// row is read as whole 128-byte lines) of rows 8 g .. 8 g + 7, plus the h and the two
// down scales of row `lane` (for the LDS exchange).
// ---------------------------------------------------------------------------------
struct DnItem {
    u32x4 w[8];
    uint64_t h;     // tagged h of row r0 + lane (tag == seq and value 0 beyond G)
    uint32_t s;     // down scales of row r0 + lane for the tile's two blocks (0 beyond G)
};

__device__ __forceinline__ uint64_t ld_agent_u64(const uint64_t* p) {
    return __hip_atomic_load(glb(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D>
__device__ __forceinline__ void dn_issue(const uint8_t* grp, const uint16_t* sc, const uint64_t* hrow, int G, int tile,
                                         int r0, uint32_t seq, DnItem& it) {
    constexpr int BLOCKS = D / 128;
    constexpr int RB = 3 * D / 2;
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    // the tile's two scales of a row are adjacent fp16 (block 2 tile is even): one 32-bit load
    if (r0 + kDnRows <= G) {   // every row of the pass exists: no per-lane guard
        const uint8_t* base = uniform_ptr(grp + (size_t)r0 * RB + D + tile * (kDnCols / 2));
        const uint32_t wo = (uint32_t)(8 * g) * RB + dc * 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) it.w[j] = ld_stream16(base + wo + j * RB);
        const uint16_t* srow = uniform_ptr(sc + (size_t)r0 * 3 * BLOCKS + 2 * BLOCKS + 2 * tile);
        it.s = *glb(reinterpret_cast<const uint32_t*>(srow + (uint32_t)lane * 3 * BLOCKS));
        it.h = ld_agent_u64(uniform_ptr(hrow + r0) + lane);
        return;
    }
    const uint8_t* base = grp + D + tile * (kDnCols / 2) + dc * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int n = r0 + 8 * g + j;
        it.w[j] = n < G ? ld_stream16(base + (size_t)n * RB) : u32x4{0, 0, 0, 0};
    }
    const int n = r0 + lane;
    it.s = n < G ? *glb(reinterpret_cast<const uint32_t*>(sc + (size_t)n * 3 * BLOCKS + 2 * BLOCKS + 2 * tile)) : 0u;
    it.h = n < G ? ld_agent_u64(hrow + n) : (uint64_t)seq << 32;
}

// Waits until the h of every row of the pass carries the launch sequence. False when
// the wait was abandoned (abort or timeout).
template <bool BACKOFF = true>
__device__ __forceinline__ bool wait_h_word(const MlpArgs& a, uint32_t* slot, const uint64_t* hrow, int r0,
                                            uint64_t& h) {
    const uint64_t want = a.seq;
    if (__all((h >> 32) == want)) return true;
    const int n = r0 + lane_id();
    Waiter wt(a.spin_limit);
    for (;;) {
        if (wave_should_stop(a, slot, wt)) return false;
        // While more than a quarter of the words are missing the wave waits about 0.2 us
        // between rounds: fewer reads from beyond L2 while the layer's bytes still stream (C2
        // 14.12 -> 13.99 us); with few words missing it polls at once. The batch 2-4 kernels
        // wait without it (C4 batch 4 52.5 -> 52.9 us with it).
        if (BACKOFF && __popcll(__ballot((h >> 32) != want)) > 16)
            __builtin_amdgcn_s_sleep(8);
        else
            __builtin_amdgcn_s_sleep(1);
        if ((h >> 32) != want) h = ld_agent_u64(hrow + n);   // only rows < G can be stale
        if (__all((h >> 32) == want)) return true;
    }
}
template <bool BACKOFF = true>
__device__ __forceinline__ bool dn_wait_h(const MlpArgs& a, uint32_t* slot, const uint64_t* hrow, int G, int r0,
                                          DnItem& it) {
    (void)G;
    return wait_h_word<BACKOFF>(a, slot, hrow, r0, it.h);
}

// Adds one pass into the lane's 32 column partials. The pass's h and scales go through
// this wave's LDS rows (hs: 64 halves; ss: 64 halves per block) so that a lane reads its
// 8 rows as one 16-byte vector each. Rows (8g + 2p, 8g + 2p + 1) share a dot2: v_perm
// pairs their nibbles column by column. Rows beyond G have zero weights, h and scales.
__device__ __forceinline__ void dn_accumulate(const DnItem& it, uint16_t* hs, uint16_t* ss, float acc[32]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    hs[lane] = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)it.h));   // exact: h is fp16
    ss[lane] = (uint16_t)it.s;
    ss[kDnRows + lane] = (uint16_t)(it.s >> 16);
    // The wave's LDS operations execute in order: the stores above land before the
    // loads below. The fence only keeps the compiler from reordering them.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + 8 * g);
    const u32x4 sv = *reinterpret_cast<const u32x4*>(ss + kDnRows * (dc >> 2) + 8 * g);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const u32x4 wa = it.w[2 * p], wb = it.w[2 * p + 1];
        const h2 hab = as_h2(hw[p]), sab = as_h2(sw[p]);
        const uint32_t xa[4] = {wa.x, wa.y, wa.z, wa.w}, xb[4] = {wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h2 w[4];
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x05040100u), sab, w);   // columns 8q + 0..3
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + c] = dot2(w[c], hab, acc[8 * q + c]);
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x07060302u), sab, w);   // columns 8q + 4..7
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + 4 + c] = dot2(w[c], hab, acc[8 * q + 4 + c]);
        }
    }
}

__device__ __forceinline__ float swap_sum32(float x, float y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap_sum16(float x, float y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 8 row groups (lanes 8 g + dc, same dc) in a fixed tree, without LDS.
// v_permlane32_swap exchanges the upper half of one register with the lower half of
// another, so (acc[c], acc[c+16]) summed after a swap leave column c (groups g, g + 4) in
// lanes < 32 and column c + 16 in lanes >= 32; v_permlane16_swap does the same across
// odd / even 16-lane rows with (c, c+8); a row_ror:8 DPP add joins the two group
// parities. Returns this lane's columns 32 dc + 4 g + i (i < 4) of the tile.
__device__ __forceinline__ void dn_reduce(const float acc[32], float out[4]) {
    float s1[16], s2[8];
#pragma unroll
    for (int c = 0; c < 16; ++c) s1[c] = swap_sum32(acc[c], acc[c + 16]);
#pragma unroll
    for (int c = 0; c < 8; ++c) s2[c] = swap_sum16(s1[c], s1[c + 8]);
    // lane (g, dc) now holds 8 of the 32 columns over the groups of g's parity; lane ^ 8
    // holds the same columns over the other parity.
    const bool odd = (lane_id() >> 3) & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x = odd ? s2[4 + i] : s2[i], y = odd ? s2[i] : s2[4 + i];
        out[i] = x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), 0x128, 0xF, 0xF, false));
    }
}

// ---------------------------------------------------------------------------------
// descriptor access and validation
// ---------------------------------------------------------------------------------
struct Unit {
    const uint8_t* grp;     // packed bytes of the group
    const uint16_t* sc;     // scale rows of the group
    uint32_t dest;
    bool ok;
};

__device__ __forceinline__ Unit resolve(const MlpArgs& a, const Bounds& b, ExecDesc d, int D) {
    Unit u;
    const bool staging = d.source_kind == leanstream::runtime::SourceKind::Staging;
    const uint32_t slots = staging ? b.staging_groups : b.cache_groups;
    u.ok = d.source_slot < slots && d.physical_group < b.physical_groups && d.dest_slot < a.slot_capacity &&
           (uint32_t)d.source_kind <= 1u;
    const size_t group_bytes = (size_t)a.group_size * 3 * D / 2;
    u.grp = (staging ? a.staging : a.cache) + (u.ok ? (size_t)d.source_slot * group_bytes : 0);
    u.sc = a.scales + (u.ok ? (size_t)d.physical_group * a.group_size * 3 * (D / 128) : 0);
    u.dest = u.ok ? d.dest_slot : 0;
    return u;
}

// ---------------------------------------------------------------------------------
// Shared workgroup state: per-wave LDS rows for the down items' h / scale exchange, and
// the words the claim path and the path decision share.
// ---------------------------------------------------------------------------------
struct Shared {
    alignas(16) uint16_t hs[kWaves][kDnRows];
    alignas(16) uint16_t ss[kWaves][2 * kDnRows];
    uint32_t word[8];
    uint32_t wpath[kWaves];
    uint32_t wfail[kWaves];
    uint32_t xcount;   // waves that have staged their part of x
};

// The queue state of a launch as one wave learnt it (wave-uniform).
struct Epoch {
    uint32_t known, ok, total, path;
};

// (ok, total, path) of the queue from the word the mirror workgroup publishes. `early`
// is lane 0's look at the word taken at the start of the launch.
__device__ __forceinline__ bool await_epoch(const MlpArgs& a, uint32_t* slot, Epoch& ep, uint32_t early) {
    if (ep.known) return ep.ok != 0;
    uint32_t word = 0;
    if (lane_id() == 0) {
        word = early;
        // kept here: decoded earlier, the word would make the wave wait for every load
        // issued before it (x, the descriptors) at the kernel's start
        asm volatile("" : "+v"(word) : : "memory");
        Waiter wt(a.spin_limit);
        while (!(word & 3u)) {
            if (wt.due()) {
                if (ld_agent(slot + kSyncAbort)) { word = 2; break; }
                if (wt.over()) { raise_status(a, slot, kStatusTimeout); word = 2; break; }
            }
            __builtin_amdgcn_s_sleep(2);
            word = ld_agent(slot + kSyncEpoch);
        }
    }
    word = __builtin_amdgcn_readfirstlane(word);
    ep.known = 1;
    ep.ok = (word & 3u) == 1u;
    ep.path = ep.ok ? (word >> 2) & 3u : 0u;
    ep.total = ep.ok ? word >> 4 : 0u;
    return ep.ok != 0;
}

// ---------------------------------------------------------------------------------
// Compact reduction by deterministic fixed-point accumulation (kAccOne in mlp_args.h).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void st_agent_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A column's value from its accumulator word once all `rows` contributions are in.
__device__ __forceinline__ float acc_value(unsigned long long word, uint32_t rows) {
    const long long sum = (long long)(word & kAccValueMask) - (long long)rows * kAccBias;
    return (float)((double)sum * kAccInv);
}

__device__ __forceinline__ void write_output(const MlpArgs& a, int col, unsigned long long word, uint32_t rows) {
    const float v = acc_value(word, rows);
    if (a.y32) a.y32[col] = v;
    a.y[col] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

// The layer epilogue's arithmetic (LeanStream backends/triton/reduction.py:17-28 with
// PUBLISH; examples/ministral/native/predictor_shared_input.cu:16-41), shared by
// epilogue_kernel and the fused launch's last workgroup. hidden = fp16(fp32 residual + fp32
// y), its square added to the thread's sum (thread t of 256 takes columns t, t + 256, ... in
// order); inverse = 1 / sqrt(sum / width + eps) over a halving tree of the 256 partial sums;
// out = fp16(weight * fp16(hidden * inverse)). Nothing is contracted into a fused
// multiply-add, so the bits are the oracle's.
__device__ __forceinline__ uint16_t epi_hidden(uint16_t res, uint16_t y, float& sum) {
#pragma clang fp contract(off)
    const float a = (float)__builtin_bit_cast(_Float16, res);
    const float b = (float)__builtin_bit_cast(_Float16, y);
    float ab = a + b;
    asm volatile("" : "+v"(ab));   // an fp32 sum rounded to fp16 (no mixed-precision fused form)
    const _Float16 h = (_Float16)ab;
    const float v = (float)h;
    const float sq = v * v;
    sum = sum + sq;
    return __builtin_bit_cast(uint16_t, h);
}
// The workgroup's 256 partial sums (lanes: 256 floats of LDS) -> the row's inverse RMS.
__device__ __forceinline__ float epi_inverse(float sum, float* lanes, uint32_t width, float eps) {
#pragma clang fp contract(off)
    const uint32_t t = threadIdx.x;
    __syncthreads();   // a previous row's reads of lanes are done
    lanes[t] = sum;
    __syncthreads();
    for (uint32_t stride = 128; stride; stride >>= 1) {
        if (t < stride) lanes[t] = lanes[t] + lanes[t + stride];
        __syncthreads();
    }
    return 1.0f / __builtin_sqrtf(lanes[0] / (float)width + eps);
}
__device__ __forceinline__ uint16_t epi_norm(uint16_t hid, float inverse, uint16_t weight) {
#pragma clang fp contract(off)
    float p = (float)__builtin_bit_cast(_Float16, hid) * inverse;
    asm volatile("" : "+v"(p));   // the fp32 product, then fp16 (as the reference rounds)
    const float n = (float)(_Float16)p;
    const float w = (float)__builtin_bit_cast(_Float16, weight);
    return __builtin_bit_cast(uint16_t, (_Float16)(w * n));   // the exact product, rounded once
}

// The accumulator buffer of this launch (two alternate between consecutive launches).
__device__ __forceinline__ unsigned long long* launch_acc(const MlpArgs& a) {
    return a.yacc + (size_t)(a.seq & 1) * a.width * a.batch * kAccStride;
}

// One contribution of a column value: round(v * 2^20) biased by 2^39, count 1 in the
// top field. Out-of-range values are clipped and reported.
__device__ __forceinline__ unsigned long long acc_term(const MlpArgs& a, uint32_t* slot, float value) {
    float v = value * kAccScale;
    if (!(fabsf(v) < (float)(kAccBias - 1))) {  // out of range or NaN: clip and report
        v = v > 0.f ? (float)(kAccBias - 1) : -(float)(kAccBias - 1);
        raise_status(a, slot, kStatusRange);
    }
    return (unsigned long long)(__float2ll_rn(v) + kAccBias) + kAccOne;
}

// Columns of a lane's four sums of a down tile: dn_tile_column(l) + kTileColOff[i]. Each
// atomic instruction then covers 64 consecutive columns (four 128-byte lines).
__device__ __forceinline__ int dn_tile_column(int lane) { return lane; }
__device__ constexpr int kTileColOff[4] = {0, 64, 128, 192};

// The accumulator words returned by a wave's last column additions, checked once the
// next additions are issued (or at the end), so the wave does not wait for the atomics'
// round trip: the contribution that completes a column (count U) writes the output.
// Each atomic instruction covers four runs of 16 consecutive columns (four 128-byte
// lines): a lane's columns are col + kTileColOff[i] (i < n).
struct Pending {
    unsigned long long v[4];
    int col;   // first column of the lane's n; < 0: nothing pending
    int n;     // columns col + kTileColOff[i], i < n (4: 256-column tiles, 1: 64-column quarters)
};

__device__ __forceinline__ void check_pending(const MlpArgs& a, Pending& pd, uint32_t U) {
    if (pd.col >= 0 && U) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < pd.n && (uint32_t)(pd.v[i] >> 52) == U) write_output(a, pd.col + kTileColOff[i], pd.v[i], U);
    }
    pd.col = -1;
}

// One column per lane (the quarters of the staged walk).
__device__ __forceinline__ void add_column(const MlpArgs& a, uint32_t* slot, unsigned long long* yacc, int col,
                                           float c, uint32_t U, Pending& pd) {
    const unsigned long long t = acc_term(a, slot, c);
    const unsigned long long v =
        __hip_atomic_fetch_add(yacc + (size_t)col * kAccStride, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + t;
    check_pending(a, pd, U);
    pd.v[0] = v;
    pd.col = col;
    pd.n = 1;
}

__device__ __forceinline__ void add_columns(const MlpArgs& a, uint32_t* slot, unsigned long long* yacc, int col,
                                            const float c[4], uint32_t U, Pending& pd) {
    unsigned long long n[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned long long t = acc_term(a, slot, c[i]);
        n[i] = __hip_atomic_fetch_add(yacc + (size_t)(col + kTileColOff[i]) * kAccStride, t, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) + t;
    }
    check_pending(a, pd, U);
#pragma unroll
    for (int i = 0; i < 4; ++i) pd.v[i] = n[i];
    pd.col = col;
    pd.n = 4;
}

// Sum over the 8 row groups of 8 column partials, in dn_reduce's tree (row groups g, g ^ 4,
// then g ^ 2, then g ^ 1), so a column gets the bits it gets there. Returns column g of the 8.
__device__ __forceinline__ float dn_reduce8(const float acc[8]) {
    float s1[4], s2[2];
#pragma unroll
    for (int c = 0; c < 4; ++c) s1[c] = swap_sum32(acc[c], acc[c + 4]);
#pragma unroll
    for (int c = 0; c < 2; ++c) s2[c] = swap_sum16(s1[c], s1[c + 2]);
    const bool odd = (lane_id() >> 3) & 1;
    const float x = odd ? s2[1] : s2[0], y = odd ? s2[0] : s2[1];
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), 0x128, 0xF, 0xF, false));
}

// A down item for every batch row at once (batch 2..4, one 64-row pass): the item's pieces
// are dequantised once and multiplied with the h of each row (hb[r]: row r's fp16 h in this
// wave's LDS). The lane's 32 columns go in quarters of 8 (8 partials per row in flight),
// each quarter summed over the row groups at once (dn_reduce8): part[r][q] is column
// 32 dc + 8 q + g of the tile for row r. The dot2 order and the reduction tree are those of
// dn_accumulate and dn_reduce: every row gets the bits a one-row item would give it.
template <int NB>
__device__ __forceinline__ void dn_accumulate_rows(const DnItem& it, const uint16_t (*hb)[kDnRows], uint16_t* ss,
                                                   uint32_t nb, float (&part)[NB][4]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    ss[lane] = (uint16_t)it.s;
    ss[kDnRows + lane] = (uint16_t)(it.s >> 16);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's LDS stores land before its loads
    const u32x4 sv = *reinterpret_cast<const u32x4*>(ss + kDnRows * (dc >> 2) + 8 * g);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {   // columns 8 q + 0..7 of the lane's 32
        float acc[NB][8];
#pragma unroll
        for (int r = 0; r < NB; ++r)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[r][c] = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t xa = it.w[2 * p][q], xb = it.w[2 * p + 1][q];
            const h2 sab = as_h2(sw[p]);
            h2 w0[4], w1[4];
            dequant8(__builtin_amdgcn_perm(xb, xa, 0x05040100u), sab, w0);   // columns 8q + 0..3
            dequant8(__builtin_amdgcn_perm(xb, xa, 0x07060302u), sab, w1);   // columns 8q + 4..7
#pragma unroll
            for (int r = 0; r < NB; ++r) {
                const h2 hab = as_h2(reinterpret_cast<const uint32_t*>(&hb[r][8 * g])[p]);   // rows 8g + 2p, + 1
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    acc[r][c] = dot2(w0[c], hab, acc[r][c]);
                    acc[r][4 + c] = dot2(w1[c], hab, acc[r][4 + c]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NB; ++r)
            if ((uint32_t)r < nb) part[r][q] = dn_reduce8(acc[r]);
    }
}

// Execution counters (diagnostics): a unit counts once all of its down items are done.
__device__ __forceinline__ void count_execution(const MlpArgs& a, uint32_t* slot, uint32_t unit, uint32_t dest,
                                                uint32_t items) {
    if (lane_id() == 0 && add_agent(slot + kSyncUnits + unit * kLine, 1u) == items - 1)
        __hip_atomic_fetch_add(a.executions + dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---------------------------------------------------------------------------------
// Item walk of one wave over units [u0, u1).
// ---------------------------------------------------------------------------------

// Unit (relative to u0) of item i: gate/up items [0, NG), ipu per unit (each serves every
// batch row); then down items, T per batch unit (unit u, row b is batch unit u nb + b;
// nb = 1 when one down item serves every batch row).
// With packs of P units (P > 1, pack_units) a down item stands for its pack's last unit
// (nu units in the range), the one whose publication it waits for.
__device__ __forceinline__ uint32_t item_unit(uint32_t i, uint32_t NG, uint32_t ipu, uint32_t T, uint32_t nb,
                                              uint32_t P = 1, uint32_t nu = 0) {
    if (i < NG) return i / ipu;
    uint32_t v = (i - NG) / T;
    v = nb == 1 ? v : v / nb;
    return P == 1 ? v : min(v * P + P, nu) - 1;
}

// Small groups (G <= 32) at batch 1 (the packed kernels, MlpArgs::pack = 64 / G): a down
// item of the resident (core) range packs the rows of P consecutive core units into one
// 64-row pass (row G j + n is neuron n of the pack's unit j), so a tile column takes one
// contribution per pack instead of one per unit. Core units are in descriptor order, so the
// packs and their sums are the same in every launch. Queue units keep one unit per down item:
// their positions follow the publication order, and one contribution per unit keeps y
// independent of that order.
__device__ __forceinline__ uint32_t pack_units(const MlpArgs& a) { return a.pack > 1 ? a.pack : 1u; }
// Contributions per output column of a fused launch: one per down item of a column tile.
template <bool PACKED>
__device__ __forceinline__ uint32_t column_rows(const MlpArgs& a, uint32_t total) {
    if constexpr (!PACKED) return a.core_count + total;
    const uint32_t P = pack_units(a);
    return (a.core_count + P - 1) / P + total;
}

// How the waves taking part share the items of a unit range: wave w of nw. With
// gu_waves = 0 (mixed) every wave takes the list [gate/up items, down items] at w, w + nw,
// ...: its gate/up items first, then its down items. Otherwise (split) waves
// [0, gu_waves) take only gate/up items and the others only down items, so a wave that
// publishes h never polls for h: its polls and atomics never queue behind its own h
// stores, whose acknowledgement from memory is slow under a full load stream.
struct WaveRole {
    uint32_t w, nw, gu_waves;
};

// The items of one wave: gate/up items g0, g0 + gs, ... (KG of them), then down items
// d0, d0 + ds, ... (K - KG); item(k) is the k-th one's index in the range's list
// (gate/up items [0, NG), then down items).
struct ItemList {
    uint32_t NG, g0, gs, d0, ds, KG, K;
    __device__ __forceinline__ uint32_t item(uint32_t k) const { return k < KG ? g0 + k * gs : NG + d0 + (k - KG) * ds; }
};

__device__ __forceinline__ uint32_t stride_count(uint32_t first, uint32_t n, uint32_t stride) {
    return first < n ? (n - first + stride - 1) / stride : 0u;
}

__device__ __forceinline__ ItemList make_items(const WaveRole& r, uint32_t NG, uint32_t ND) {
    ItemList l;
    l.NG = NG;
    if (r.gu_waves == 0) {
        l.g0 = r.w;
        l.gs = r.nw;
        l.KG = stride_count(r.w, NG, r.nw);
        l.d0 = r.w + l.KG * r.nw - NG;
        l.ds = r.nw;
        l.K = l.KG + stride_count(l.d0, ND, r.nw);
    } else if (r.w < r.gu_waves) {
        l.g0 = r.w;
        l.gs = r.gu_waves;
        l.KG = l.K = stride_count(r.w, NG, r.gu_waves);
        l.d0 = 0;
        l.ds = 1;
    } else {
        l.g0 = 0;
        l.gs = 1;
        l.KG = 0;
        l.d0 = r.w - r.gu_waves;
        l.ds = r.nw - r.gu_waves;
        l.K = stride_count(l.d0, ND, l.ds);
    }
    return l;
}

// The staged walk's lists: one stripe over the gate/up items and then the down quarters,
// as in make_items, with the quarters starting at the next multiple of 4 after the
// gate/up items: with nw a multiple of 4 the four quarters 4t .. 4t + 3 of a tile go to
// the four waves of one workgroup (q = w mod 4). Each wave takes at most one item more
// than an even share, and its items keep the order of the list.
__device__ __forceinline__ ItemList make_staged_items(const WaveRole& r, uint32_t NG, uint32_t NDQ) {
    const uint32_t NGa = (NG + 3u) & ~3u;
    ItemList l;
    l.NG = NG;
    l.g0 = r.w;
    l.gs = r.nw;
    l.KG = stride_count(r.w, NG, r.nw);
    l.d0 = r.w + stride_count(r.w, NGa, r.nw) * r.nw - NGa;   // the stripe's first position >= NGa
    l.ds = r.nw;
    l.K = l.KG + stride_count(l.d0, NDQ, r.nw);
    return l;
}

// Descriptor words of items k0 .. k0 + count - 1 of this wave in one round trip: lane
// 5 j + w holds word w of item k0 + j's unit. A queue position is read from the mirror
// once the mirror has copied it: the wave waits until the mirrored ready count covers
// the last position of the batch (`seen` is the count it last observed).
__device__ __forceinline__ bool fetch_descs(const MlpArgs& a, uint32_t* slot, uint32_t u0, uint32_t& seen,
                                            const ItemList& il, uint32_t k0, uint32_t count, uint32_t ipu,
                                            uint32_t T, uint32_t nb, uint32_t& word, uint32_t P = 1,
                                            uint32_t nu = 0) {
    // units rise along each of the wave's two lists (gate/up, then down items), so the
    // batch's last position is that of its last gate/up or its last down item
    const uint32_t kl = k0 + count - 1;
    uint32_t last = 0;
    if (k0 < il.KG) last = item_unit(il.item(min(kl, il.KG - 1)), il.NG, ipu, T, nb, P, nu);
    if (kl >= il.KG) last = max(last, item_unit(il.item(kl), il.NG, ipu, T, nb, P, nu));
    const uint32_t g = u0 + last;
    const uint32_t need = g >= a.core_count ? g - a.core_count + 1 : 0u;
    if (need > seen) {
        uint32_t ok = 1, ready = 0;
        if (lane_id() == 0) {
            Waiter wt(a.spin_limit);
            while ((ready = ld_agent(slot + kSyncReady)) < need) {
                if (wt.due()) {
                    if (ld_agent(slot + kSyncAbort)) { ok = 0; break; }
                    if (wt.over()) { raise_status(a, slot, kStatusTimeout); ok = 0; break; }
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        if (!__builtin_amdgcn_readfirstlane(ok)) return false;
        seen = __builtin_amdgcn_readfirstlane(ready);
    }
    const uint32_t lane = lane_id();
    word = 0;
    if (lane < 5 * count) {
        const uint32_t j = lane / 5, w = lane - 5 * j;
        const uint32_t g = u0 + item_unit(il.item(k0 + j), il.NG, ipu, T, nb, P, nu);
        word = g < a.core_count ? glb(reinterpret_cast<const uint32_t*>(a.core))[5 * g + w]
                                : ld_agent(a.qmirror + 5 * (g - a.core_count) + w);
    }
    return true;
}

__device__ __forceinline__ bool unit_of(const MlpArgs& a, uint32_t* slot, const Bounds& b, uint32_t word, uint32_t j,
                                        int D, Unit& u) {
    ExecDesc d;
    d.logical_group = __builtin_amdgcn_readlane(word, 5 * j + 0);
    d.physical_group = __builtin_amdgcn_readlane(word, 5 * j + 1);
    d.source_slot = __builtin_amdgcn_readlane(word, 5 * j + 2);
    d.dest_slot = __builtin_amdgcn_readlane(word, 5 * j + 3);
    d.source_kind = (leanstream::runtime::SourceKind)__builtin_amdgcn_readlane(word, 5 * j + 4);
    u = resolve(a, b, d, D);
    if (!u.ok) {
        if (lane_id() == 0) raise_status(a, slot, kStatusBadDescriptor);
        return false;
    }
    return true;
}

// A packed down item's rows (pack_units): lane r holds row r's h pointer, unit and
// destination; `lead` marks the lane of each unit's first row.
struct PackLane {
    const uint64_t* hp;
    uint32_t unit, dest;
    bool lead;
};

// Issues a down item over the rows of `units` consecutive units g0, g0 + 1, ... (G rows each,
// G <= 32): lane r resolves the descriptor of row r's unit (agent-scope loads: queue
// descriptors are mirrored during the launch) and holds that row's scales and h; lane 8 g + dc
// loads columns 32 dc .. 32 dc + 31 of rows 8 g .. 8 g + 7 from their units' groups. Rows past
// the pack have zero weights, scales and h. False (status raised) on an invalid descriptor.
template <int D>
__device__ __forceinline__ bool dn_issue_pack(const MlpArgs& a, uint32_t* slot, const Bounds& b, uint32_t g0,
                                              uint32_t units, int tile, DnItem& it, PackLane& pl) {
    constexpr int BLOCKS = D / 128;
    constexpr int RB = 3 * D / 2;
    const uint32_t G = a.group_size;
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const uint32_t j = (uint32_t)lane / G, n = (uint32_t)lane - j * G;
    const bool valid = j < units;
    Unit u{nullptr, nullptr, 0, true};
    if (valid) {
        const uint32_t gu = g0 + j;
        const uint32_t* w = gu < a.core_count ? reinterpret_cast<const uint32_t*>(a.core) + 5 * gu
                                              : a.qmirror + 5 * (gu - a.core_count);
        ExecDesc d;
        d.logical_group = 0;
        d.physical_group = ld_agent(w + 1);
        d.source_slot = ld_agent(w + 2);
        d.dest_slot = ld_agent(w + 3);
        d.source_kind = (leanstream::runtime::SourceKind)ld_agent(w + 4);
        u = resolve(a, b, d, D);
    }
    if (!__all(u.ok)) {
        if (lane == 0) raise_status(a, slot, kStatusBadDescriptor);
        return false;
    }
    const uint8_t* row = valid ? u.grp + (size_t)n * RB + D + tile * (kDnCols / 2) : nullptr;
    const uint64_t rp = reinterpret_cast<uint64_t>(row);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int r = 8 * g + k;
        const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(r << 2, (int)(uint32_t)rp);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(r << 2, (int)(uint32_t)(rp >> 32));
        const uint8_t* p = reinterpret_cast<const uint8_t*>((uint64_t)hi << 32 | lo);
        it.w[k] = (uint32_t)r / G < units ? ld_stream16(p + dc * 16) : u32x4{0, 0, 0, 0};
    }
    it.s = valid ? *glb(reinterpret_cast<const uint32_t*>(u.sc + (size_t)n * 3 * BLOCKS + 2 * BLOCKS + 2 * tile)) : 0u;
    pl.hp = a.hbuf + (size_t)u.dest * G + n;
    pl.unit = g0 + j;
    pl.dest = u.dest;
    pl.lead = valid && n == 0;
    it.h = valid ? ld_agent_u64(pl.hp) : (uint64_t)a.seq << 32;
    return true;
}

// Waits until every lane's h word carries the launch sequence, reloading from the lane's own
// pointer (lanes already tagged never reload). False when the wait was abandoned.
__device__ __forceinline__ bool wait_h_lanes(const MlpArgs& a, uint32_t* slot, const uint64_t* hp, uint64_t& h) {
    const uint64_t want = a.seq;
    if (__all((h >> 32) == want)) return true;
    Waiter wt(a.spin_limit);
    for (;;) {
        if (wave_should_stop(a, slot, wt)) return false;
        __builtin_amdgcn_s_sleep(1);
        if ((h >> 32) != want) h = ld_agent_u64(hp);
        if (__all((h >> 32) == want)) return true;
    }
}

// The persistent kernels' ninth leading scalar: what a worker's first loads depend on beyond
// the other eight -- the group size, the batch rows and whether the staged walk's down items
// are whole tiles (MlpArgs::group_size <= 256, batch <= kMaxBatch, dn_tile).
__host__ __device__ constexpr uint32_t launch_shape(uint32_t group_size, uint32_t batch, uint32_t dn_tile) {
    return group_size | batch << 16 | (dn_tile == (uint32_t)kDnCols ? 1u << 31 : 0u);
}
__device__ __forceinline__ uint32_t shape_group(uint32_t shape) { return shape & 0xFFFFu; }
__device__ __forceinline__ uint32_t shape_batch(uint32_t shape) { return (shape >> 16) & 0xFFu; }
__device__ __forceinline__ bool shape_tiles(uint32_t shape) { return shape >> 31; }

// The first descriptor batch of the resident range, fetched at the worker's start.
struct Prefetched {
    uint32_t word;
    bool valid;
};

// The first descriptor batch of the resident range on the plain and packed walks, from the
// preloaded arguments alone (process_items' item list for units [0, core_count): G neurons
// per unit, nb batch rows, packs of 64 / G core units on the packed walk).
template <int D, int NB, bool PACKED>
__device__ __forceinline__ void prefetch_core_descs_plain(const ExecDesc* core, uint32_t core_count, uint32_t G,
                                                          uint32_t batch, const WaveRole& role, Prefetched& p) {
    using Gm = GuGeom<D>;
    constexpr uint32_t T = D / kDnCols;
    p.valid = false;
    p.word = 0;
    if (!core_count || !G) return;
    const uint32_t nb = NB == 1 ? 1u : batch;
    const uint32_t ipu = (G + Gm::NPI - 1) / Gm::NPI;
    const uint32_t dnb = NB > 1 && nb > 1 && G <= (uint32_t)kDnRows ? 1u : nb;
    const uint32_t P = PACKED ? (uint32_t)kDnRows / G : 1u;
    const uint32_t NP = (core_count + P - 1) / P;
    const ItemList il = make_items(role, core_count * ipu, NP * dnb * T);
    if (!il.K) return;
    const uint32_t count = min(il.K, (uint32_t)kDescItems);
    const uint32_t lane = lane_id();
    if (lane < 5 * count) {
        const uint32_t j = lane / 5, w = lane - 5 * j;
        const uint32_t g = item_unit(il.item(j), il.NG, ipu, T, dnb, P, core_count);
        p.word = glb(reinterpret_cast<const uint32_t*>(core))[5 * g + w];
    }
    p.valid = true;
}

// Wave-uniform bookkeeping of an item in flight.
struct ItemMeta {
    const uint8_t* grp;
    const uint16_t* sc;
    uint64_t* hrow;
    uint32_t unit, dest, tile, row;   // row: the batch row
    int n0, nvalid;
};

// This wave's items of units [u0, u1) (its share under `role`), one item in flight at a
// time (a one-pass gate/up item in two halves at batch 1). Gate/up items never
// wait for another wave; down items wait for their unit's h (after every gate/up item
// of this wave), so every h is eventually published. With FUSED, the U-th contribution
// of a column writes the output (U = core + queue units, learnt from the epoch word).
template <int D, bool FUSED, int NB, bool PACKED>
__device__ __forceinline__ bool process_items(const MlpArgs& a, Shared& sh, u32x4* stage, uint32_t* slot, const Bounds& b,
                                              unsigned long long* yacc, XPart<D>& xp, u32x4* xl, Epoch& ep,
                                              uint32_t early, Pending& pd, uint32_t u0, uint32_t u1,
                                              const WaveRole& role, const Prefetched& first) {
    using Gm = GuGeom<D>;
    constexpr uint32_t T = D / kDnCols;
    const uint32_t G = a.group_size;
    const uint32_t nb = NB == 1 ? 1u : a.batch;
    const uint32_t nu = u1 - u0;
    const uint32_t ipu = (G + Gm::NPI - 1) / Gm::NPI;   // gate/up items per unit (every batch row)
    const uint32_t NG = nu * ipu;
    // With one 64-row pass (G <= 64) a down item serves every batch row: its pieces are
    // loaded and dequantised once and multiplied with each row's h (dn_accumulate_rows).
    // Larger groups take one down item per batch row and tile.
    const bool dn_rows = NB > 1 && nb > 1 && G <= (uint32_t)kDnRows;
    const uint32_t dnb = dn_rows ? 1u : nb;   // down items per unit and tile
    const uint32_t P = PACKED && u1 <= a.core_count ? pack_units(a) : 1u;   // units per down item (core range)
    const uint32_t NP = (nu + P - 1) / P;              // down items per tile (and batch row)
    const ItemList il = make_items(role, NG, NP * dnb * T);
    const uint32_t K = il.K, KG = il.KG;   // items of this wave; the first KG are gate/up
    // Every exit stages this wave's part of x first (siblings may be waiting for it).
    auto leave = [&](bool r) -> bool {
        stage_x<D>(xp, NB == 1 ? 1u : a.batch, xl, &sh.xcount);
        return r;
    };
    if (!K) return leave(true);
    uint32_t seen = 0;   // mirrored ready count this wave last observed
    // Descriptors first, then x: loads complete in issue order, so the first item's
    // address computation waits for the descriptors only.
    uint32_t word = first.word, k0 = 0;
    if (!first.valid && !fetch_descs(a, slot, u0, seen, il, 0, min(K, (uint32_t)kDescItems), ipu, T, dnb, word, P, nu))
        return leave(false);
    // x was loaded before the descriptors, so (in-order completion) it is in too
    stage_x<D>(xp, NB == 1 ? 1u : a.batch, xl, &sh.xcount);
    const int wave = wave_id();
    uint16_t* hs = sh.hs[wave];
    uint16_t* ss = sh.ss[wave];
    GuItem<D> gi;
    DnItem di;
    ItemMeta m;
    PackLane pl{nullptr, 0, 0, false};
    uint32_t U = 0;
    bool have_u = !FUSED;

    // One item in flight per wave: the memory-level parallelism comes from the number of
    // resident waves, which keeps the registers per wave low and leaves the loads of every
    // other wave to hide this one's compute. Gate/up items
    // come first in every wave's list.
    // Gate/up items in two halves only at batch 1 where an item is one pass (D >= 8192):
    // such layers give every wave several items, and the second half's loads overlap
    // the first half's arithmetic (d=8192, 90 groups: 26.3 -> 26.0 us). With several
    // passes per item (D <= 4096, at most one or two items per wave) the whole item stays
    // in flight: halving the bytes in flight cost more than the overlap gained (d=4096,
    // 58 groups: 14.4 -> 14.9 us); at batch 4 (four dot products per dequantised pair)
    // the halves were 0.2 us slower.
    constexpr bool halves = kGuHalves && NB == 1 && !GuHalf<D, 1>::BY_PASS;
    auto fetch_unit = [&](uint32_t k, Unit& u) -> bool {
        if (k - k0 >= (uint32_t)kDescItems) {
            k0 = k;
            if (!fetch_descs(a, slot, u0, seen, il, k0, min(K - k0, (uint32_t)kDescItems), ipu, T, dnb, word, P, nu))
                return false;
        }
        return unit_of(a, slot, b, word, k - k0, D, u);
    };
    auto issue_gu = [&](uint32_t k, GuItem<D>& gi, ItemMeta& m) -> bool {
        Unit u;
        if (!fetch_unit(k, u)) return false;
        const uint32_t i = il.item(k), rel = i / ipu;
        m.row = 0;
        m.dest = u.dest;
        m.hrow = a.hbuf + (size_t)u.dest * nb * G;   // row 0 of the destination's h rows
        m.n0 = (int)((i - rel * ipu) * Gm::NPI);
        m.nvalid = min(Gm::NPI, (int)G - m.n0);
        m.grp = u.grp;
        m.sc = u.sc;
        if constexpr (halves)
            gu_issue<D, 1>(u.grp, u.sc, m.n0, m.nvalid, gi);
        else
            gu_issue<D, 0>(u.grp, u.sc, m.n0, m.nvalid, gi);
        return true;
    };
    auto issue_dn = [&](uint32_t k, DnItem& di, ItemMeta& m) -> bool {
        Unit u;
        if (!fetch_unit(k, u)) return false;   // a pack's last unit: every unit of it is published
        const uint32_t d = il.item(k) - NG, rel = d / T;
        if constexpr (PACKED) {
            m.row = 0;
            m.unit = u0 + rel * P;
            m.tile = d - rel * T;
            if (!dn_issue_pack<D>(a, slot, b, u0 + rel * P, min(P, nu - rel * P), (int)m.tile, di, pl)) return false;
            if (FUSED && !ep.known && lane_id() == 0) early = ld_agent(slot + kSyncEpoch);
            return true;
        }
        m.row = dnb == 1 ? 0u : rel % dnb;
        m.grp = u.grp;
        m.sc = u.sc;
        m.dest = u.dest;
        m.hrow = a.hbuf + ((size_t)u.dest * nb + m.row) * G;
        m.unit = u0 + (dnb == 1 ? rel : rel / dnb);
        m.tile = d - rel * T;
        dn_issue<D>(u.grp, u.sc, m.hrow, (int)G, (int)m.tile, 0, a.seq, di);
        // a fresh look at the epoch word, in flight with the item (U is needed to finish it)
        if (FUSED && !ep.known && lane_id() == 0) early = ld_agent(slot + kSyncEpoch);
        return true;
    };
    auto compute_gu = [&](uint32_t k, GuItem<D>& gi, const ItemMeta& m) {
        if (a.first_compute && m.n0 == 0 && lane_id() == 0) a.first_compute[m.dest] = now_ticks();
        float acc[NB][Gm::RPL][2];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int p = 0; p < Gm::RPL; ++p) acc[b][p][0] = acc[b][p][1] = 0.f;
        if constexpr (halves) {
            wait_vector_loads();   // the first half has landed: the second goes out now
            gu_issue<D, 2>(m.grp, m.sc, m.n0, m.nvalid, gi);
            gu_dots<D, NB, 1>(gi, xl, nb, acc);
            gu_dots<D, NB, 2>(gi, xl, nb, acc);
        } else {
            gu_dots<D, NB, 0>(gi, xl, nb, acc);
        }
        gu_finish<D, NB>(acc, m.hrow, G, m.n0, m.nvalid, a.seq, nb);
        if (k == 0) stamp(a, kStampFirstData);
    };
    auto compute_dn = [&](uint32_t k, DnItem& di, const ItemMeta& m) -> bool {
        if (!have_u) {
            if (!await_epoch(a, slot, ep, early)) return false;
            U = column_rows<PACKED>(a, ep.total);
            have_u = true;
        }
        const int lane = lane_id();
        float* red = reinterpret_cast<float*>(stage + wave * kNonStagedWaveVecs<NB>);
        if constexpr (NB > 1) {
            if (dn_rows) {
                // every row's h: row 0 came with the item, the others go out now
                uint16_t (*hb)[kDnRows] = reinterpret_cast<uint16_t (*)[kDnRows]>(red + kDnCols);
                uint64_t hr[NB];
                hr[0] = di.h;
#pragma unroll
                for (int r = 1; r < NB; ++r)
                    hr[r] = (uint32_t)r < nb && lane < (int)G ? ld_agent_u64(m.hrow + (size_t)r * G + lane)
                                                              : (uint64_t)a.seq << 32;
#pragma unroll
                for (int r = 0; r < NB; ++r) {
                    if (!wait_h_word<false>(a, slot, m.hrow + (size_t)r * G, 0, hr[r])) return false;
                    hb[r][lane] = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)hr[r]));   // exact
                }
                float part[NB][4];
                dn_accumulate_rows<NB>(di, hb, ss, nb, part);
                const int col0 = dn_tile_column(lane);
#pragma unroll
                for (int r = 0; r < NB; ++r) {
                    if ((uint32_t)r >= nb) break;
                    // re-deal row r's sums as the one-row items do
#pragma unroll
                    for (int q = 0; q < 4; ++q) red[32 * (lane & 7) + 8 * q + (lane >> 3)] = part[r][q];
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    float cs[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) cs[i] = red[col0 + kTileColOff[i]];
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    add_columns(a, slot, yacc, (int)(r * D + m.tile * kDnCols) + col0, cs, U, pd);
                }
                if (a.executions) count_execution(a, slot, m.unit, m.dest, T);
                if (k == KG) stamp(a, kStampDnComputed);
                return true;
            }
        }
        float acc[32];
#pragma unroll
        for (int c = 0; c < 32; ++c) acc[c] = 0.f;
        if constexpr (PACKED) {
            if (!wait_h_lanes(a, slot, pl.hp, di.h)) return false;
            dn_accumulate(di, hs, ss, acc);
        } else {
            for (int r0 = 0; r0 < (int)G; r0 += kDnRows) {
                if (r0) dn_issue<D>(m.grp, m.sc, m.hrow, (int)G, (int)m.tile, r0, a.seq, di);
                if (!dn_wait_h<NB == 1>(a, slot, m.hrow, (int)G, r0, di)) return false;
                dn_accumulate(di, hs, ss, acc);
            }
        }
        float cs[4];
        dn_reduce(acc, cs);
        // re-deal through LDS: lane (g, dc) holds tile columns 32 dc + 4 g + i; lane l adds
        // columns dn_tile_column(l) + kTileColOff[i], as the staged walk does
        *reinterpret_cast<float4*>(red + 32 * (lane & 7) + 4 * (lane >> 3)) = float4{cs[0], cs[1], cs[2], cs[3]};
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const int col0 = dn_tile_column(lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) cs[i] = red[col0 + kTileColOff[i]];
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        add_columns(a, slot, yacc, (int)(m.row * D + m.tile * kDnCols) + col0, cs, U, pd);
        if (a.executions) {
            if constexpr (PACKED) {   // every unit of the pack: its first row's lane counts it
                if (pl.lead && add_agent(slot + kSyncUnits + pl.unit * kLine, 1u) == T - 1)
                    __hip_atomic_fetch_add(a.executions + pl.dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            } else {
                count_execution(a, slot, m.unit, m.dest, T * dnb);
            }
        }
        if (k == KG) stamp(a, kStampDnComputed);
        return true;
    };

    for (uint32_t k = 0; k < KG; ++k) {
        if (!issue_gu(k, gi, m)) return false;
        if (k == 0 && !wait_x(a, slot, &sh.xcount)) return false;
        compute_gu(k, gi, m);
    }
    for (uint32_t k = KG; k < K; ++k) {
        if (!issue_dn(k, di, m)) return false;
        if (!compute_dn(k, di, m)) return false;
    }
    return true;
}

// ---------------------------------------------------------------------------------
// Staged item walk (64-neuron groups, batch 1). Every item is 8 KB of weights -- a gate/up
// item's RPL x 2 x CPL 16-byte pieces per lane, or a down item's 8 row pieces per lane --
// plus one 256-byte block of its scales, and is loaded into one of the wave's two LDS
// slots with global_load_lds, which takes no registers. A wave keeps two items in
// flight: item k + 1 streams in while item k is computed. At the Ministral-8B shape
// (at most one gate/up and one down item per wave) every byte of the layer is requested
// as soon as the wave's descriptors arrive, so the layer's HBM stream is one phase.
//
// Each item is exactly kStageOps load instructions, all into LDS (the compiler tracks no
// register result of them), so `s_waitcnt vmcnt(kStageOps)` before computing item k waits
// for item k and everything issued before it, and leaves item k + 1 in flight.
// ---------------------------------------------------------------------------------
constexpr uint32_t kStagedGroup = 64;              // neurons per group of the staged kernels
// Widths whose staged kernels keep two workgroups per CU (slots + x + Shared <= 80 KB).
constexpr bool staged_width(int width) { return width <= 4096; }
constexpr int kSlotVecs = 512;                     // 16-byte weight pieces of one item
constexpr int kSlotStride = kSlotVecs + 16;        // + 256 bytes of scales
constexpr int kStageOps = 9;                       // load instructions per item
typedef __attribute__((address_space(3))) void* lds_ptr;

// 16 / 4 bytes per lane into LDS: lane l's piece lands at block + 16 l (4 l). Weights are
// read once: non-temporal.
__device__ __forceinline__ void lds_load16(const void* g, u32x4* block) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr)block, 16, 0, 2);
}
__device__ __forceinline__ void lds_load4(const void* g, u32x4* block) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr)block, 4, 0, 0);
}

// vmcnt(N) with the other counters at their maxima; the scheduling barriers keep the LDS
// reads of the awaited item below it.
template <int N>
__device__ __forceinline__ void wait_loads_but() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
    __builtin_amdgcn_sched_barrier(0);
}
// Waits until piece group j (of GROUPS, two loads each, issued after the item's scale
// block) has landed: at most 2 (GROUPS - 1 - j) of the item's loads are outstanding, plus
// AFTER loads issued behind the item (another item already in flight).
template <int GROUPS, int AFTER = 0>
__device__ __forceinline__ void constexpr_wait_group(int j) {
    static_assert(GROUPS == 4, "gate/up items are four piece groups");
    switch (j) {
        case 0: wait_loads_but<6 + AFTER>(); break;
        case 1: wait_loads_but<4 + AFTER>(); break;
        case 2: wait_loads_but<2 + AFTER>(); break;
        default: wait_loads_but<0 + AFTER>(); break;
    }
}

// lgkmcnt(0): this wave's LDS reads of a slot are complete before new pieces land in it.
__device__ __forceinline__ void wait_lds_reads() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_sched_barrier(0);
}

// Gate/up item: neurons n0 .. n0 + NPI - 1 of the unit at grp / sc. Piece (p, proj, k) of
// lane l lands at slot[((p 2 + proj) CPL + k) 64 + l]; the scale block holds, per neuron,
// its B gate then its B up scales (B = D / 128: NPI x 2B fp16 = 256 bytes), lane l loading
// the l-th 32-bit word. Issue order: the scale block, then piece groups j = k RPL + p
// (gate piece, up piece), the order in which gu_dots_staged consumes them, so group j has
// landed once at most 2 (groups - 1 - j) of the item's loads are outstanding.
template <int D>
__device__ __forceinline__ void gu_stage(const uint8_t* grp, const uint16_t* sc, int n0, u32x4* sl) {
    using Gm = GuGeom<D>;
    constexpr int B = D / 128;
    static_assert(Gm::NPI * B == 64, "one 32-bit scale word per lane");
    static_assert(2 * Gm::RPL * Gm::CPL + 1 == kStageOps, "an item is kStageOps loads");
    const int lane = lane_id();
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
    const uint16_t* srow = uniform_ptr(sc + (size_t)n0 * 3 * B);
    lds_load4(srow + (uint32_t)(lane / B) * 3 * B + 2 * (lane % B), sl + kSlotVecs);
    const uint32_t wo = (uint32_t)sub * (3 * D / 2) + 16 * r;
#pragma unroll
    for (int k = 0; k < Gm::CPL; ++k) {
#pragma unroll
        for (int p = 0; p < Gm::RPL; ++p) {
            const uint8_t* row = uniform_ptr(grp + (size_t)(n0 + p * Gm::NPW) * (3 * D / 2));
            lds_load16(row + wo + 16 * Gm::LPR * k, sl + ((p * 2 + 0) * Gm::CPL + k) * 64);
            lds_load16(row + wo + 16 * Gm::LPR * k + D / 2, sl + ((p * 2 + 1) * Gm::CPL + k) * 64);
        }
    }
}

// Down quarter: columns 64 q .. 64 q + 63 of tile `tile` (256 columns) of the unit's 64
// rows: 2 KB of weights and the tile's scales. LDS row r of the slot holds the quarter's
// 32 bytes of unit row r (lane l of load j brings row 32 j + l / 2, half l & 1); word l of
// the scale block holds row l's two scales of the tile (128-column blocks 2 tile, 2 tile +
// 1). The 4 quarters of a tile are taken by the 4 waves of one workgroup, so each 128-byte
// row line is requested by one CU.
template <int D>
__device__ __forceinline__ void dn_stage_quarter(const uint8_t* grp, const uint16_t* sc, int tile, int q, u32x4* sl) {
    constexpr int B = D / 128;
    constexpr int RB = 3 * D / 2;
    const int lane = lane_id();
    const uint16_t* srow = uniform_ptr(sc + 2 * B + 2 * tile);
    lds_load4(srow + (uint32_t)lane * 3 * B, sl + kSlotVecs);
    const uint8_t* base = uniform_ptr(grp + D + tile * (kDnCols / 2) + q * 32);
    const uint32_t wo = (uint32_t)(lane >> 1) * RB + (lane & 1) * 16;
    lds_load16(base + wo, sl);
    lds_load16(base + wo + 32 * RB, sl + 64);
}

// Dequantises lane (g, dc)'s part of staged quarter q -- rows 8 g .. 8 g + 7, columns
// 8 dc .. 8 dc + 7 -- into fp16 (row 2p, row 2p + 1) pairs per column: w[p][c], c < 8. Runs
// while the unit's h is still on its way.
__device__ __forceinline__ void dn_dequant_quarter(const u32x4* sl, int q, h2 (&w)[4][8]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const uint32_t* rows = reinterpret_cast<const uint32_t*>(sl);
    const u32x4* sv = sl + kSlotVecs + 2 * g;   // rows 8 g .. 8 g + 7: both scales each
    const u32x4 s0 = sv[0], s1 = sv[1];
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    // the (row 2p, row 2p + 1) scales of the quarter's block: low or high halves
    const uint32_t pick = (q >> 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t wa = rows[(8 * g + 2 * p) * 8 + dc], wb = rows[(8 * g + 2 * p + 1) * 8 + dc];
        const h2 sab = as_h2(__builtin_amdgcn_perm(sw[2 * p + 1], sw[2 * p], pick));
        dequant8(__builtin_amdgcn_perm(wb, wa, 0x05040100u), sab, &w[p][0]);   // columns 0..3
        dequant8(__builtin_amdgcn_perm(wb, wa, 0x07060302u), sab, &w[p][4]);   // columns 4..7
    }
}

// The quarter's dot products with h of rows 8 g .. 8 g + 7 (hs: the wave's 64 h as fp16):
// acc[c] is column 8 dc + c over the lane's 8 rows.
__device__ __forceinline__ void dn_dot_quarter(const h2 (&w)[4][8], const uint16_t* hs, float (&acc)[8]) {
    const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + 8 * (lane_id() >> 3));
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = dot2(w[p][c], as_h2(hw[p]), acc[c]);
    }
}

// Down tile: columns 256 tile .. 256 tile + 255 of the unit's 64 rows (8 KB). Lane
// 8 g + dc's piece j is row 8 g + j, columns 32 dc .. 32 dc + 31, at slot[j 64 + l]; word l
// of the scale block holds row l's two scales of the tile.
template <int D>
__device__ __forceinline__ void dn_stage_tile(const uint8_t* grp, const uint16_t* sc, int tile, u32x4* sl) {
    constexpr int B = D / 128;
    constexpr int RB = 3 * D / 2;
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const uint16_t* srow = uniform_ptr(sc + 2 * B + 2 * tile);
    lds_load4(srow + (uint32_t)lane * 3 * B, sl + kSlotVecs);
    const uint8_t* base = uniform_ptr(grp + D + tile * (kDnCols / 2));
    const uint32_t wo = (uint32_t)(8 * g) * RB + dc * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) lds_load16(base + wo + j * RB, sl + j * 64);
}

// Dequantisation and dot products of a staged tile in one pass, once h is in (lane (g, dc):
// rows 8 g .. 8 g + 7, columns 32 dc + c; acc[c] over the lane's 8 rows).
__device__ __forceinline__ void dn_accumulate_tile(const u32x4* sl, const uint16_t* hs, float (&acc)[32]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const u32x4* sv = sl + kSlotVecs + 2 * g;
    const u32x4 s0 = sv[0], s1 = sv[1];
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t pick = (dc >> 2) ? 0x07060302u : 0x05040100u;
    const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + 8 * g);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[c] = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const u32x4 va = sl[(2 * p) * 64 + lane], vb = sl[(2 * p + 1) * 64 + lane];
        const uint32_t xa[4] = {va.x, va.y, va.z, va.w}, xb[4] = {vb.x, vb.y, vb.z, vb.w};
        const h2 sab = as_h2(__builtin_amdgcn_perm(sw[2 * p + 1], sw[2 * p], pick));
        const h2 hab = as_h2(hw[p]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h2 w[4];
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x05040100u), sab, w);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + c] = dot2(w[c], hab, acc[8 * q + c]);
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x07060302u), sab, w);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + 4 + c] = dot2(w[c], hab, acc[8 * q + 4 + c]);
        }
    }
}

#ifndef LS_DN_PRE
#define LS_DN_PRE 2
#endif
// Row pairs of a staged down tile dequantised while the unit's h is on its way.
constexpr int kDnPre = LS_DN_PRE;
static_assert(kDnPre >= 0 && kDnPre <= 4, "a tile has four row pairs per lane");

// Dequantises row pairs p < P of lane (g, dc)'s part of a staged tile (rows 8 g + 2 p,
// + 1; columns 32 dc + 8 q + c): w[p][q][c], the operands dn_accumulate_tile forms.
template <int P>
__device__ __forceinline__ void dn_dequant_tile(const u32x4* sl, h2 (&w)[P > 0 ? P : 1][4][8]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const u32x4* sv = sl + kSlotVecs + 2 * g;
    const u32x4 s0 = sv[0], s1 = sv[1];
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t pick = (dc >> 2) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const u32x4 va = sl[(2 * p) * 64 + lane], vb = sl[(2 * p + 1) * 64 + lane];
        const uint32_t xa[4] = {va.x, va.y, va.z, va.w}, xb[4] = {vb.x, vb.y, vb.z, vb.w};
        const h2 sab = as_h2(__builtin_amdgcn_perm(sw[2 * p + 1], sw[2 * p], pick));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x05040100u), sab, &w[p][q][0]);
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x07060302u), sab, &w[p][q][4]);
        }
    }
    // computed here, while h travels (the compiler would otherwise sink them to their uses)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                uint32_t t = __builtin_bit_cast(uint32_t, w[p][q][c]);
                asm volatile("" : "+v"(t));
                w[p][q][c] = as_h2(t);
            }
}

// dn_accumulate_tile with row pairs p < P already dequantised (dn_dequant_tile): the same
// operands in the same order, so the same bits.
template <int P>
__device__ __forceinline__ void dn_accumulate_tile_pre(const u32x4* sl, const uint16_t* hs,
                                                       const h2 (&pre)[P > 0 ? P : 1][4][8], float (&acc)[32]) {
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    const u32x4* sv = sl + kSlotVecs + 2 * g;
    const u32x4 s0 = sv[0], s1 = sv[1];
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t pick = (dc >> 2) ? 0x07060302u : 0x05040100u;
    const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + 8 * g);
    const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
    for (int c = 0; c < 32; ++c) acc[c] = 0.f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const h2 hab = as_h2(hw[p]);
        if (p < P) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[8 * q + c] = dot2(pre[p < P ? p : 0][q][c], hab, acc[8 * q + c]);
            continue;
        }
        const u32x4 va = sl[(2 * p) * 64 + lane], vb = sl[(2 * p + 1) * 64 + lane];
        const uint32_t xa[4] = {va.x, va.y, va.z, va.w}, xb[4] = {vb.x, vb.y, vb.z, vb.w};
        const h2 sab = as_h2(__builtin_amdgcn_perm(sw[2 * p + 1], sw[2 * p], pick));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h2 w[4];
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x05040100u), sab, w);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + c] = dot2(w[c], hab, acc[8 * q + c]);
            dequant8(__builtin_amdgcn_perm(xb[q], xa[q], 0x07060302u), sab, w);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[8 * q + 4 + c] = dot2(w[c], hab, acc[8 * q + 4 + c]);
        }
    }
}

// Sum of a quarter's column partials over the wave's 8 row groups through LDS, in
// dn_reduce's tree ((0 + 4) + (2 + 6)) + ((1 + 5) + (3 + 7)), so that quarters and tiles
// give the same bits. Lane (g, dc) stores its columns 8 dc + c at red[g][12 dc + c] (a
// 12-float stride keeps the 8 lanes of a 16-byte store on distinct banks); lane l returns
// column l. red: 768 floats of the wave's slot.
__device__ __forceinline__ float dn_sum_groups_quarter(const float (&acc)[8], float* red) {
    constexpr int RS = 8 * 12;
    const int lane = lane_id(), g = lane >> 3, dc = lane & 7;
    float4* dst = reinterpret_cast<float4*>(red + g * RS + 12 * dc);
    dst[0] = float4{acc[0], acc[1], acc[2], acc[3]};
    dst[1] = float4{acc[4], acc[5], acc[6], acc[7]};
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's LDS stores land before its loads
    const float* src = red + 12 * (lane >> 3) + (lane & 7);
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = src[j * RS];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return ((r[0] + r[4]) + (r[2] + r[6])) + ((r[1] + r[5]) + (r[3] + r[7]));
}

// gu_dots of a staged item (batch 1): the same arithmetic, pieces and scales from LDS,
// consumed group by group as they land (the item is the newest load of the wave, or loads
// issued after it are stores). `last` runs once the final group has landed, before it is
// computed (the wave issues its next item there).
template <int D, class Last, int AFTER = 0>
__device__ __forceinline__ void gu_dots_staged(const u32x4* sl, const u32x4* xl, float (&acc)[1][GuGeom<D>::RPL][2],
                                               Last&& last) {
    using Gm = GuGeom<D>;
    constexpr int B = D / 128;
    constexpr int GROUPS = Gm::RPL * Gm::CPL;
    const int lane = lane_id();
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
    const uint16_t* scl = reinterpret_cast<const uint16_t*>(sl + kSlotVecs);
#pragma unroll
    for (int k = 0; k < Gm::CPL; ++k) {
        uint32_t xw[4][4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const u32x4 xv = xl[(4 * k + g) * Gm::LPR + r];   // paired (stage_x)
            xw[g][0] = xv.x;
            xw[g][1] = xv.y;
            xw[g][2] = xv.z;
            xw[g][3] = xv.w;
        }
#pragma unroll
        for (int p = 0; p < Gm::RPL; ++p) {
            constexpr_wait_group<GROUPS, AFTER>(k * Gm::RPL + p);
            if (k * Gm::RPL + p == GROUPS - 1) last();
            u32x4 v[2];
            h2 s2[2];
#pragma unroll
            for (int proj = 0; proj < 2; ++proj) {
                v[proj] = sl[((p * 2 + proj) * Gm::CPL + k) * 64 + lane];
                const _Float16 sv = half_bits(scl[(p * Gm::NPW + sub) * 2 * B + proj * B + ((r + Gm::LPR * k) >> 2)]);
                s2[proj] = h2{sv, sv};
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int proj = 0; proj < 2; ++proj) {
                    const uint32_t words[4] = {v[proj].x, v[proj].y, v[proj].z, v[proj].w};
                    h2 w[4];
                    dequant8(words[g], s2[proj], w);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[0][p][proj] = dot2(w[q], as_h2(xw[g][q]), acc[0][p][proj]);
                }
            }
            // the group's products are computed here, before the next group's wait (the
            // compiler would otherwise sink them below the last wait)
            asm volatile("" : "+v"(acc[0][p][0]), "+v"(acc[0][p][1]));
        }
    }
}


// Down items per unit of a staged range of nu units: 64-column quarters when every item
// of the range gets a wave of its own (the 4 quarters of a tile on the 4 waves of a
// workgroup, so the work after h is a quarter of a tile's), whole 256-column tiles
// otherwise (a wave's items follow one another, and fewer of them finish sooner). The
// widest staged kernels take tiles only: the quarter path's registers and code cost them
// more than it saves.
template <int D>
constexpr bool kStagedQuarters = D <= 2048;

template <int D>
__device__ __forceinline__ uint32_t staged_down_items(const WaveRole& r, uint32_t nu, uint32_t dn_tile) {
    constexpr uint32_t T = D / kDnCols, ipu = kStagedGroup / GuGeom<D>::NPI;
    if constexpr (!kStagedQuarters<D>) return T;
    if (dn_tile == kDnCols) return T;   // the candidate asks for whole tiles
    const uint32_t ng = (nu * ipu + 3u) & ~3u;
    return ng + 4 * T * nu <= r.nw ? 4 * T : T;
}

// From the preloaded arguments alone (core, core_count, dn_tile): resident units are never
// waited for and never mirrored, so the batch is the fetch_descs one of the range's first
// items, read from the core table.
template <int D>
__device__ __forceinline__ void prefetch_core_descs(const ExecDesc* core, uint32_t core_count, uint32_t dn_tile,
                                                    const WaveRole& role, Prefetched& p) {
    constexpr uint32_t ipu = kStagedGroup / GuGeom<D>::NPI;
    p.valid = false;
    p.word = 0;
    if (!core_count) return;
    const uint32_t TQ = staged_down_items<D>(role, core_count, dn_tile);
    const ItemList il = make_staged_items(role, core_count * ipu, core_count * TQ);
    if (!il.K) return;
    const uint32_t count = min(il.K, (uint32_t)kDescItems);
    const uint32_t lane = lane_id();
    if (lane < 5 * count) {
        const uint32_t j = lane / 5, w = lane - 5 * j;
        const uint32_t g = item_unit(il.item(j), il.NG, ipu, TQ, 1u);
        p.word = glb(reinterpret_cast<const uint32_t*>(core))[5 * g + w];
    }
    p.valid = true;
}

// This wave's items of units [u0, u1) through its two LDS slots (stage: kWaves x 2 slots).
// Same item lists, waits and reduction as process_items.
template <int D, bool FUSED>
__device__ __forceinline__ bool process_items_staged(const MlpArgs& a, Shared& sh, u32x4* stage, uint32_t* slot,
                                                     const Bounds& b, unsigned long long* yacc, XPart<D>& xp,
                                                     u32x4* xl, Epoch& ep, uint32_t early, Pending& pd, uint32_t u0,
                                                     uint32_t u1, const WaveRole& role, const Prefetched& first) {
    using Gm = GuGeom<D>;
    constexpr uint32_t T = D / kDnCols;
    constexpr uint32_t G = kStagedGroup;
    constexpr uint32_t ipu = G / Gm::NPI;   // gate/up items per unit
    const uint32_t nu = u1 - u0;
    const uint32_t NG = nu * ipu;
    const uint32_t TQ = staged_down_items<D>(role, nu, a.dn_tile);   // down items per unit
    const bool quarters = kStagedQuarters<D> && TQ != T;
    const ItemList il = make_staged_items(role, NG, nu * TQ);
    const uint32_t K = il.K, KG = il.KG;
    auto leave = [&](bool r) -> bool {
        stage_x<D>(xp, 1u, xl, &sh.xcount);
        return r;
    };
    if (!K) return leave(true);
    uint32_t seen = 0, word = first.word, k0 = 0;
    if (!first.valid && !fetch_descs(a, slot, u0, seen, il, 0, min(K, (uint32_t)kDescItems), ipu, TQ, 1u, word))
        return leave(false);
    if (a.stamps) {
        asm volatile("" : : "v"(word));   // the stamp waits for the descriptors
        stamp(a, kStampDescs);
    }
    stage_x<D>(xp, 1u, xl, &sh.xcount);
    const int wave = wave_id();
    const int lane = lane_id();
    uint16_t* hs = sh.hs[wave];
    u32x4* const sl0 = stage + (2 * wave) * kSlotStride;
    u32x4* const sl1 = sl0 + kSlotStride;
    ItemMeta m0, m1;
    uint32_t U = 0;
    bool have_u = !FUSED;

    auto fetch_unit = [&](uint32_t k, Unit& u) -> bool {
        if (k - k0 >= (uint32_t)kDescItems) {
            k0 = k;
            if (!fetch_descs(a, slot, u0, seen, il, k0, min(K - k0, (uint32_t)kDescItems), ipu, TQ, 1u, word))
                return false;
        }
        return unit_of(a, slot, b, word, k - k0, D, u);
    };
    auto issue = [&](uint32_t k, u32x4* sl, ItemMeta& m) -> bool {
        Unit u;
        if (!fetch_unit(k, u)) return false;
        wait_lds_reads();   // the slot's previous item is no longer being read
        m.grp = u.grp;
        m.sc = u.sc;
        m.dest = u.dest;
        m.hrow = a.hbuf + (size_t)u.dest * G;
        if (k < KG) {
            const uint32_t i = il.item(k), rel = i / ipu;
            m.n0 = (int)((i - rel * ipu) * Gm::NPI);
            gu_stage<D>(u.grp, u.sc, m.n0, sl);
        } else if (quarters) {
            // quarter j = 4 (tile of the unit) + q; q is the wave's index in its workgroup
            const uint32_t j = il.item(k) - NG, rel = j / TQ, jt = j - rel * TQ;
            m.unit = u0 + rel;
            m.tile = jt >> 2;
            m.row = jt & 3;   // the quarter
            dn_stage_quarter<D>(u.grp, u.sc, (int)m.tile, (int)m.row, sl);
        } else {
            const uint32_t j = il.item(k) - NG, rel = j / TQ;
            m.unit = u0 + rel;
            m.tile = j - rel * TQ;
            dn_stage_tile<D>(u.grp, u.sc, (int)m.tile, sl);
        }
        return true;
    };
    // next: issues the wave's next item once this one's last piece group has landed
    auto compute_gu = [&](uint32_t k, const u32x4* sl, const ItemMeta& m, auto&& next) -> bool {
        if (k == 0 && !wait_x(a, slot, &sh.xcount)) return false;
        if (a.first_compute && m.n0 == 0 && lane == 0) a.first_compute[m.dest] = now_ticks();
        float acc[1][Gm::RPL][2];
#pragma unroll
        for (int p = 0; p < Gm::RPL; ++p) acc[0][p][0] = acc[0][p][1] = 0.f;
        bool ok = true;
        gu_dots_staged<D>(sl, xl, acc, [&]() {
            if (k < 2) stamp(a, k == 0 ? kStampFirstData : kStampSecondData);
            ok = next();
        });
        if (!ok) return false;
        gu_finish<D, 1>(acc, m.hrow, G, m.n0, Gm::NPI, a.seq, 1u);
        if (k == 0) stamp(a, kStampFirstDone);
        return true;
    };
    auto compute_dn = [&](uint32_t k, u32x4* sl, const ItemMeta& m) -> bool {
        if (!have_u) {
            if (!await_epoch(a, slot, ep, early)) return false;
            U = column_rows<false>(a, ep.total);
            have_u = true;
        }
        // the first look at h goes out first (a quarter is dequantised while it travels)
        DnItem it;
        it.h = ld_agent_u64(uniform_ptr(m.hrow) + lane);
        if (quarters) {
            h2 w[4][8];
            dn_dequant_quarter(sl, (int)m.row, w);
            if (!dn_wait_h(a, slot, m.hrow, (int)G, 0, it)) return false;
            if (k == KG) stamp(a, kStampHReady);
            hs[lane] = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)it.h));   // exact: h is fp16
            __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's LDS store lands before its loads
            float acc[8];
            dn_dot_quarter(w, hs, acc);
            // through the slot: its pieces are in registers
            const float col_sum = dn_sum_groups_quarter(acc, reinterpret_cast<float*>(sl));
            add_column(a, slot, yacc, (int)(m.tile * kDnCols + m.row * 64) + lane, col_sum, U, pd);
        } else {
            h2 pre[kDnPre > 0 ? kDnPre : 1][4][8];
            dn_dequant_tile<kDnPre>(sl, pre);
            if (!dn_wait_h(a, slot, m.hrow, (int)G, 0, it)) return false;
            if (k == KG) stamp(a, kStampHReady);
            hs[lane] = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)it.h));   // exact: h is fp16
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            float acc[32], cs[4];
            dn_accumulate_tile_pre<kDnPre>(sl, hs, pre, acc);
            dn_reduce(acc, cs);
            // re-deal through the slot (its pieces are in registers by now): lane (g, dc)
            // holds tile columns 32 dc + 4 g + i; lane l adds dn_tile_column(l) + kTileColOff[i]
            float* red = reinterpret_cast<float*>(sl);
            *reinterpret_cast<float4*>(red + 32 * (lane & 7) + 4 * (lane >> 3)) = float4{cs[0], cs[1], cs[2], cs[3]};
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
            for (int i = 0; i < 4; ++i) cs[i] = red[dn_tile_column(lane) + kTileColOff[i]];
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            add_columns(a, slot, yacc, (int)(m.tile * kDnCols) + dn_tile_column(lane), cs, U, pd);
        }
        if (a.executions) count_execution(a, slot, m.unit, m.dest, TQ);
        if (k == KG) stamp(a, kStampDnComputed);
        return true;
    };
    // Item k sits in slot sl. A gate/up item is computed group by group as its pieces
    // land; item k + 1 goes out into the other slot once item k has landed, and streams
    // while item k's last group (gate/up) or the whole down item is computed.
    auto step = [&](uint32_t k, u32x4* sl, ItemMeta& m, u32x4* nsl, ItemMeta& nm) -> bool {
        auto next = [&]() -> bool { return k + 1 >= K || issue(k + 1, nsl, nm); };
        // a down item after the wave's last gate/up item waits until that item is computed:
        // its bytes are not needed before h, and issued earlier they compete with the
        // gate/up bytes still streaming, which h waits for (measured: all bytes requested
        // at the start make the layer slower)
        if (k + 1 == KG) return compute_gu(k, sl, m, [] { return true; }) && next();
        if (k < KG) return compute_gu(k, sl, m, next);
        wait_loads_but<0>();
        if (k < 2) stamp(a, k == 0 ? kStampFirstData : kStampSecondData);
        return next() && compute_dn(k, sl, m);
    };
    if (!issue(0, sl0, m0)) return false;
    for (uint32_t k = 0; k < K; k += 2) {
        if (!step(k, sl0, m0, sl1, m1)) return false;
        if (k + 1 < K && !step(k + 1, sl1, m1, sl0, m0)) return false;
    }
    return true;
}

// ---------------------------------------------------------------------------------
// Queue protocol (LeanStream kernels/streaming_mlp.cu:47-79, backends/triton/persistent.py:32-92):
// wait for the layer epoch (or an error), optionally for batch publication, decide once
// per launch between the all-ready fast path and the progressive path (positions
// published while the launch runs), then consume published positions in order: on the
// progressive path every wave waits for the positions of its own stripe of items, or
// (claim_batch > 0) workgroups claim ready positions.
//
// On MI355X the queue lives in host memory behind PCIe, where concurrent reads from
// hundreds of workgroups are served one after another. So exactly one workgroup of
// each launch (the mirror, the last block) reads host memory: it publishes the packed
// (state, path, total) word into the device ring slot, copies every newly published
// position's descriptor into a device-side table in publication order (64 positions
// per round trip, one per lane) and advances a device-side ready count. Workers only
// poll device memory.
// ---------------------------------------------------------------------------------
// One claim log entry (kClaimLogWords), written by one lane of the worker or mirror that takes the range.
__device__ __forceinline__ void log_claim(const MlpArgs& a, uint32_t* slot, uint32_t first, uint32_t count,
                                          uint32_t ready) {
    if (!a.claim_log) return;
    const uint32_t seq = add_agent(slot + kSyncClaims, 1u);
    if (seq >= a.claim_log_cap) return;
    uint32_t* e = a.claim_log + (size_t)seq * kClaimLogWords;
    e[0] = first;
    e[1] = count;
    e[2] = ready;
    e[3] = blockIdx.x;
}

// Runs on wave 0 of the mirror workgroup. `pre` is lane 0's early 64-bit load of
// (total_count, epoch): adjacent words (byte offsets 8 and 12), read as one pair.
__device__ __forceinline__ void mirror_queue(const MlpArgs& a, uint32_t* slot, uint64_t pre) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t state = 0, total = 0, path = 0;
    if (lane == 0) {
        Waiter wt(a.spin_limit);
        uint64_t te = pre;
        for (;;) {
            if ((uint32_t)(te >> 32) == a.epoch) { state = 1; break; }
            if (ld_sys(&a.control->error)) { state = 2; st_agent(slot + kSyncAbort, 1u); break; }
            if (ld_agent(slot + kSyncAbort)) { state = 2; break; }
            if (wt.expired()) { raise_status(a, slot, kStatusTimeout); state = 2; break; }
            __builtin_amdgcn_s_sleep(8);
            te = ld_sys64(&a.control->total_count);
        }
        total = state == 1 ? (uint32_t)te : 0;
        if (state == 1 && (total > a.capacity || a.core_count + total > a.slot_capacity)) {
            raise_status(a, slot, kStatusBadDescriptor);
            state = 2;
        }
        if (state == 1 && total && a.batch_mode) {
            Waiter wb(a.spin_limit);
            for (;;) {
                if (ld_sys(&a.control->batch_epoch) == a.epoch) break;
                if (ld_sys(&a.control->error)) { state = 2; st_agent(slot + kSyncAbort, 1u); break; }
                if (ld_agent(slot + kSyncAbort)) { state = 2; break; }
                if (wb.expired()) { raise_status(a, slot, kStatusTimeout); state = 2; break; }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        if (state == 1 && total) path = ld_sys(&a.control->ready_count) >= total ? 2u : 1u;
        st_agent(slot + kSyncEpoch, pack_epoch(state, path, state == 1 ? total : 0u));
        stamp(a, kStampMirrorEpoch);
    }
    state = wave_bcast(state);
    total = wave_bcast(total);
    const bool by_index = a.claim_batch && wave_bcast(path) == 2u;
    if (state != 1) return;
    if (total == 0 && a.core_count == 0) {
        // no rows at all: the reduction of nothing is zero
        for (uint32_t c = lane; c < a.width * a.batch; c += 64) {
            if (a.y32) a.y32[c] = 0.f;
            a.y[c] = 0;
        }
        return;
    }
    uint32_t mirrored = 0;
    Waiter wt(a.spin_limit);
    while (mirrored < total) {
        uint32_t ready = 0, stop = 0;
        if (lane == 0) {
            ready = min(ld_sys(&a.control->ready_count), total);
            if (ld_sys(&a.control->error)) {
                st_agent(slot + kSyncAbort, 1u);
                stop = 1;
            } else if (ld_agent(slot + kSyncAbort)) {
                stop = 1;
            }
        }
        ready = wave_bcast(ready);
        if (wave_bcast(stop)) return;
        if (ready > mirrored) {
            for (uint32_t base = mirrored; base < ready; base += 64) {
                const uint32_t pos = base + lane;
                if (pos < ready) {
                    // All-ready launches of a pair-claiming candidate consume descriptors by
                    // index (persistent.py:63-69); every other launch by publication position.
                    const uint32_t idx = by_index ? pos : ld_sys(a.ready + pos);
                    const uint32_t* d = reinterpret_cast<const uint32_t*>(a.qdesc + (idx < a.capacity ? idx : 0));
                    uint32_t w[5];
#pragma unroll
                    for (int k = 0; k < 5; ++k) w[k] = ld_sys(d + k);
                    if (idx >= a.capacity) w[3] = 0xffffffffu;  // fails validation on the consumer side
#pragma unroll
                    for (int k = 0; k < 5; ++k) st_agent(a.qmirror + 5 * pos + k, w[k]);
                }
            }
            drain_vmem();  // the whole wave's copies are complete before the count moves
            // Pair-claiming candidates (claim_batch > 0) on the progressive path: the newly
            // ready positions are claimed here, in publication order, as the ranges
            // [head, min(head + claim_batch, ready)) of backends/triton/persistent.py:71-87 --
            // by one claimer, so no two workgroups race for the head -- and logged; every
            // wave then computes the claimed positions' items, as the striped path does.
            if (lane == 0 && a.claim_batch && !by_index)
                for (uint32_t head = mirrored; head < ready;) {
                    const uint32_t end = min(head + a.claim_batch, ready);
                    log_claim(a, slot, head, end - head, ready);
                    head = end;
                }
            if (lane == 0) st_agent(slot + kSyncReady, ready);
            mirrored = ready;
            wt = Waiter(a.spin_limit);  // the bound applies to waiting without progress
        } else {
            if (wt.expired()) {
                if (lane == 0) raise_status(a, slot, kStatusTimeout);
                return;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
}

}  // namespace lsamd
