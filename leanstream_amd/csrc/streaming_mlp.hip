// gfx950 kernels for LeanStream's streaming sparse INT4 MLP.
//
// Arithmetic (LeanStream kernels/streaming_mlp.cu:11-41, backends/triton/core.py:9-17):
//   w      = fp16( q * scale[c/128] ),  q = signed low-nibble-first INT4
//   gate   = sum_c w_gate(c) x(c)   up = sum_c w_up(c) x(c)          (fp32)
//   h      = fp16( fp16(silu(fp16(gate))) * fp16(up) )
//   partial[dest][c] = sum_n h_n w_down(n, c)                         (fp32)
//   y[c]   = fp16( sum over the U destination rows of partial[.][c] )
//
// Work decomposition (MI355X-specific): every descriptor ("unit", one group of G
// neurons) is cut into S items. Item j computes gate/up for neurons
// [j*G/S, (j+1)*G/S) and the down projection for columns [j*d/S, (j+1)*d/S).
// The down half of an item needs h of all G neurons of its unit, so items of
// one unit meet at a per-unit counter. Items are spread over a persistent grid
// sized to the chip, so a 58-group layer occupies every CU.
//
// Exactness: dequantisation is exact. The nibble is biased (x ^ 8) and OR-ed into
// an fp16 magic constant (0x6400 = 1024 for low nibbles, 0x5400 = 64 with a 4-bit
// mantissa offset for high nibbles); subtracting 1032 / 72 yields q exactly, and a
// packed fp16 multiply rounds q*scale once (round-to-nearest-even), which is the
// reference's fp16_rn(float(q)*float(scale)). Products w*x are exact in fp32;
// only the fp32 summation order differs from the reference.
//
// Reduction: each unit's tile is added into int64 fixed-point column accumulators
// (round(v * 2^24)); integer addition is associative, so y does not depend on the order
// in which units finish -- the output is bit-identical across consumer modes,
// publication orders and entry points. The U-th contributor of a column tile converts
// it to fp32 / fp16 and clears it.
//
// Cross-workgroup data (h, accumulators, counters) uses agent-scope relaxed atomics,
// which compile to sc1 loads/stores that are coherent across the eight XCD L2s,
// with an explicit vmcnt(0) wait before each signalling atomic. No acquire or
// release fence is issued inside a spin loop (those expand to whole-L2
// invalidate / write-back). Every wait is bounded by a wall-clock limit; on
// expiry the status word records a timeout and every worker leaves.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "mlp_args.h"
#include "mlp_launch.h"

namespace lsamd {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kMaxRows = kMaxRowsPerThread;   // down-projection rows per thread
constexpr int kMaxDnTiles = 6;       // down-projection tiles prefetched per round by a down worker
constexpr int kGuBuffers = 3;        // gate/up batches in flight per gate/up worker
constexpr int kUnitChunk = 16;       // unit descriptors loaded per parallel descriptor fetch
constexpr int kRedFloats = 4096;     // LDS scratch for the cross-thread column reduction (rpp * tile)
constexpr int kTileScales = 256;     // LDS scale slots per down pair (G * scale blocks of the tile)

// ---------------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_agent(const float* p) {
    return __uint_as_float(ld_agent(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void stf_agent(float* p, float v) {
    st_agent(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ uint32_t ld_sys(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ld_sys64(const uint32_t* p) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_stream8(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ uint32_t ld_stream4(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ _Float16 half_bits(uint16_t v) { return __builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ float round_half(float v) { return (float)(_Float16)v; }

// Exact dequantisation of eight signed nibbles (one 32-bit word) into four fp16
// pairs: out[k] = (w(col k), w(col k+4)) when the word holds one row, or
// (row a, row b) of one column when the halves of the word come from two rows.
__device__ __forceinline__ void dequant8(uint32_t word, h2 s, h2 out[4]) {
    const uint32_t m = word ^ 0x88888888u;      // two's complement -> offset binary
    const uint32_t m8 = m >> 8;
    const h2 lo_bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2 hi_bias = {(_Float16)-72.0f, (_Float16)-72.0f};
    out[0] = (as_h2((m & 0x000F000Fu) | 0x64006400u) + lo_bias) * s;
    out[1] = (as_h2((m & 0x00F000F0u) | 0x54005400u) + hi_bias) * s;
    out[2] = (as_h2((m8 & 0x000F000Fu) | 0x64006400u) + lo_bias) * s;
    out[3] = (as_h2((m8 & 0x00F000F0u) | 0x54005400u) + hi_bias) * s;
}

__device__ __forceinline__ float dot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// ---------------------------------------------------------------------------------
// bounded waiting
// ---------------------------------------------------------------------------------
struct Waiter {
    uint64_t start, limit;
    __device__ Waiter(uint64_t lim) : start(now_ticks()), limit(lim) {}
    __device__ bool expired() const { return now_ticks() - start > limit; }
};

__device__ __forceinline__ void stamp(const MlpArgs& a, uint32_t k) {
    if (a.stamps && threadIdx.x == 0 && k < kStampSlots) a.stamps[blockIdx.x * kStampSlots + k] = now_ticks();
}

__device__ __forceinline__ void raise_status(const MlpArgs& a, uint32_t* slot, uint32_t bit) {
    __hip_atomic_fetch_or(a.status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    st_agent(slot + kSyncAbort, 1u);
}

// ---------------------------------------------------------------------------------
// Geometry of the gate/up half of an item, specialised on width D and neurons per item NS.
// ---------------------------------------------------------------------------------
template <int D, int NS>
struct GuGeom {
    static constexpr int CPR = D / 32;                 // 16-byte chunks per projection row
    static constexpr int LPR = CPR < 64 ? CPR : 64;    // lanes sharing one row
    static constexpr int CPL = CPR / LPR;              // chunks per lane per row
    static constexpr int NPW = 64 / LPR;               // neurons per wave per pass
    static constexpr int NPP = 4 * NPW;                // neurons per workgroup per pass
    static constexpr int PASSES = (NS + NPP - 1) / NPP;
    static constexpr int BLOCKS = D / 128;             // scale blocks per row
    static_assert(D % 256 == 0 && CPR >= 8, "width must be a multiple of 256");
};

// x for this lane's chunks, rearranged into (k, k+4) pairs to match dequant8.
template <int D, int NS>
struct XRegs {
    h2 p[GuGeom<D, NS>::CPL][16];
};

template <int D, int NS>
__device__ __forceinline__ void load_x(const uint16_t* x, XRegs<D, NS>& xr) {
    using Gm = GuGeom<D, NS>;
    const int lane = threadIdx.x & 63;
    const int r = lane % Gm::LPR;
#pragma unroll
    for (int k = 0; k < Gm::CPL; ++k) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(x + 32 * (r + Gm::LPR * k));
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            // halves 8g..8g+7 live in words 4g..4g+3 as (0,1)(2,3)(4,5)(6,7)
            const uint32_t w0 = src[4 * g + 0], w1 = src[4 * g + 1], w2 = src[4 * g + 2], w3 = src[4 * g + 3];
            xr.p[k][4 * g + 0] = as_h2(__builtin_amdgcn_perm(w2, w0, 0x05040100u));  // (x0, x4)
            xr.p[k][4 * g + 1] = as_h2(__builtin_amdgcn_perm(w2, w0, 0x07060302u));  // (x1, x5)
            xr.p[k][4 * g + 2] = as_h2(__builtin_amdgcn_perm(w3, w1, 0x05040100u));  // (x2, x6)
            xr.p[k][4 * g + 3] = as_h2(__builtin_amdgcn_perm(w3, w1, 0x07060302u));  // (x3, x7)
        }
    }
}

template <int D, int NS>
struct GuLoads {
    u32x4 w[GuGeom<D, NS>::PASSES][2][GuGeom<D, NS>::CPL];
    uint32_t s[GuGeom<D, NS>::PASSES][2][GuGeom<D, NS>::CPL];   // fp16 bits (32-bit registers)
};

// Issue every gate/up load of one item. grp points at the unit's packed bytes,
// sc at the unit's scale rows, n0 is the first neuron of the item.
template <int D, int NS>
__device__ __forceinline__ void gu_issue(const uint8_t* grp, const uint16_t* sc, int n0, int nvalid,
                                         GuLoads<D, NS>& L) {
    using Gm = GuGeom<D, NS>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
#pragma unroll
    for (int p = 0; p < Gm::PASSES; ++p) {
        const int nu = p * Gm::NPP + wave * Gm::NPW + sub;   // neuron within the batch
        const bool ok = nu < nvalid;
        const int n = n0 + (ok ? nu : 0);
        const uint8_t* row = grp + (size_t)n * (3 * D / 2);
        const uint16_t* srow = sc + (size_t)n * 3 * Gm::BLOCKS;
#pragma unroll
        for (int k = 0; k < Gm::CPL; ++k) {
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

// Finish gate/up for the item: dot products, row reductions, activation.
// Writes h (fp32, fp16-exact) for neurons n0..n0+NS-1 of unit row `hrow`.
template <int D, int NS>
__device__ __forceinline__ void gu_compute(const GuLoads<D, NS>& L, const XRegs<D, NS>& xr, uint64_t* hrow, int n0,
                                           int nvalid, uint32_t seq) {
    using Gm = GuGeom<D, NS>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
#pragma unroll
    for (int p = 0; p < Gm::PASSES; ++p) {
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int proj = 0; proj < 2; ++proj) {
#pragma unroll
            for (int k = 0; k < Gm::CPL; ++k) {
                const _Float16 sv = half_bits((uint16_t)L.s[p][proj][k]);
                const h2 s2 = {sv, sv};
                const u32x4 v = L.w[p][proj][k];
                const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    h2 w[4];
                    dequant8(words[g], s2, w);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[proj] = dot2(w[q], xr.p[k][4 * g + q], acc[proj]);
                }
            }
        }
        acc[0] = group_sum<Gm::LPR>(acc[0]);
        acc[1] = group_sum<Gm::LPR>(acc[1]);
        const int nu = p * Gm::NPP + wave * Gm::NPW + sub;
        if (r == Gm::LPR - 1 && nu < nvalid) {
            const float g = round_half(acc[0]);
            const float u = round_half(acc[1]);
            const float s = round_half(g / (1.0f + __expf(-g)));
            const float h = round_half(s * u);
            // h tagged with the launch sequence: the word is its own ready flag.
            __hip_atomic_store(hrow + n0 + nu, ((uint64_t)seq << 32) | __float_as_uint(h), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------------
// Down projection of one column tile (tc columns) of one unit, all G neurons.
// Thread t covers 16 columns -- one 8-byte load of 16 nibbles per row -- of rows
// r0, r0 + rpp, ...: lanes = tc / 16 threads share a row, rpp = 256 / lanes rows per
// pass, at most kMaxRows rows per thread (G * tc <= 16384).
// ---------------------------------------------------------------------------------
struct DnLoads {
    u32x2 w[kMaxRows];
};

struct DnGeom {
    int lanes, rpp, rpp_shift, dc, r0, nrows, nbk, nbk_shift;
    __device__ DnGeom(int G, int tc) {
        const int lanes_shift = __builtin_ctz((unsigned)tc) - 4;
        lanes = 1 << lanes_shift;      // threads per row of the tile (tc is a power of two)
        rpp_shift = 8 - lanes_shift;
        rpp = 1 << rpp_shift;          // rows covered per pass of the workgroup
        dc = threadIdx.x & (lanes - 1);
        r0 = threadIdx.x >> lanes_shift;
        nrows = r0 < G ? (G - r0 + rpp - 1) >> rpp_shift : 0;
        nbk_shift = tc > 128 ? 1 : 0;
        nbk = 1 << nbk_shift;          // 128-column scale blocks the tile spans
    }
};

template <int D>
__device__ __forceinline__ void dn_issue(const uint8_t* grp, const DnGeom& gm, int c0, DnLoads& L) {
    const int col = c0 + 16 * gm.dc;
#pragma unroll
    for (int i = 0; i < kMaxRows; ++i) {
        if (i < gm.nrows) {
            const int n = gm.r0 + gm.rpp * i;
            L.w[i] = ld_stream8(grp + (size_t)n * (3 * D / 2) + D + (col >> 1));
        } else {
            L.w[i] = u32x2{0, 0};
        }
    }
}

// This thread's share of the tile's down scales, staged in LDS by stage_round:
// slot t < G * nbk holds row t / nbk, block t % nbk of the tile.
template <int D>
__device__ __forceinline__ uint32_t dn_scale_issue(const uint16_t* sc, const DnGeom& gm, int G, int c0) {
    constexpr int BLOCKS = D / 128;
    const int t = threadIdx.x;
    if (t >= G * gm.nbk) return 0;
    return sc[(size_t)(t >> gm.nbk_shift) * 3 * BLOCKS + 2 * BLOCKS + (c0 >> 7) + (t & (gm.nbk - 1))];
}

__device__ __forceinline__ uint64_t ld_agent_u64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t wave_bcast(uint32_t v) { return __shfl(v, 0, 64); }

// Float offset of the 4-column chunk q of column group dc in a row of the reduction
// scratch (see dn_compute).
__device__ __forceinline__ int red_swizzle(int dc, int q) { return 16 * dc + 4 * ((q + (dc >> 1)) & 3); }

// Down projection of the tile with the pair's h (hs) and scales (ss) staged in LDS.
// Each thread sums its rows in increasing order, two rows per dot2 (v_perm pairs the
// nibbles of rows (j, j+1) column by column), into 16 column partials; the partials
// of the rpp row groups are then summed in LDS in row-group order into
// red[kRedFloats + t], tile column t.
__device__ __forceinline__ void dn_compute(const DnLoads& L, const DnGeom& gm, const uint16_t* hs, const uint16_t* ss,
                                           float* red, int tc) {
    static_assert(kMaxRows == 4, "two row pairs per thread");
    const u32x2 hp = *reinterpret_cast<const u32x2*>(hs + gm.r0 * kMaxRows);  // h of rows (0,1) (2,3)
    const uint32_t hw[2] = {hp.x, hp.y};
    const int blk = gm.dc >> 3;   // 16 dc / 128: scale block within the tile
    float acc[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) acc[c] = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxRows; i += 2) {
        if (i < gm.nrows) {
            const bool pair = i + 1 < gm.nrows;
            const u32x2 wa = L.w[i], wb = pair ? L.w[i + 1] : L.w[i];
            const h2 hab = as_h2(hw[i / 2]);   // second half is zero when !pair
            const int na = gm.r0 + gm.rpp * i, nb = pair ? na + gm.rpp : na;
            const h2 sab = {half_bits(ss[na * gm.nbk + blk]), half_bits(ss[nb * gm.nbk + blk])};
            const uint32_t xa[2] = {wa.x, wa.y}, xb[2] = {wb.x, wb.y};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
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
    // red's first half is free: the previous tile's column sums were read before the
    // barrier that ended it. Row group r0's partial of tile column 16 dc + 4 q + e sits
    // at r0 * tc + swz(dc, q) + e: each thread stores 4 x 16 bytes, and within any 8
    // consecutive lanes the 16-byte chunks fall on distinct banks.
    float* mine = red + gm.r0 * tc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = gm.nrows > 0 ? float4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]}
                                      : float4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<float4*>(mine + red_swizzle(gm.dc, q)) = v;
    }
    __syncthreads();  // also: every thread is done with the previous tile's second half
    for (int t = threadIdx.x; t < tc; t += kThreads) {
        const int at = red_swizzle(t >> 4, (t >> 2) & 3) + (t & 3);
        float v = 0.f;
        for (int r0 = 0; r0 < gm.rpp; r0 += 16) {   // rpp is 16, 32 or 64
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = red[(r0 + r) * tc + at];
#pragma unroll
            for (int r = 0; r < 16; ++r) v += p[r];
        }
        red[kRedFloats + t] = v;   // reduced tile, natural column order
    }
    __syncthreads();
}

// x / G for x < 2^16 (G <= 256) via the launch's reciprocal ceil(2^32 / G): exact, as
// x * (ceil(2^32 / G) - 2^32 / G) < 2^32 / G.
__device__ __forceinline__ uint32_t div_group(const MlpArgs& a, uint32_t x) {
    return (uint32_t)(((uint64_t)x * a.g_recip) >> 32);
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

__device__ __forceinline__ ExecDesc load_core(const MlpArgs& a, uint32_t i) { return a.core[i]; }

// ---------------------------------------------------------------------------------
// Shared workgroup state
// ---------------------------------------------------------------------------------
struct Shared {
    alignas(16) float red[kRedFloats + 256];
    alignas(16) uint16_t hs[kMaxDnTiles * 64 * kMaxRows];   // staged h of a round (stage_round layout)
    uint16_t ss[kMaxDnTiles * kTileScales];                  // staged down scales of a round
    uint32_t pdest[kMaxDnTiles];                             // dest rows of the round's pairs
    uint32_t ulist[kUnitChunk];                              // units of a descriptor fetch
    uint32_t udesc[kUnitChunk][5];                           // their descriptor words
    uint32_t word[8];
    uint32_t desc[5];
    // queue state learnt once per launch: known, ok, total, path
    uint32_t ep_known, ep_ok, ep_total, ep_path;
};

__device__ __forceinline__ void init_shared(Shared& sh) {
    if (threadIdx.x == 0) { sh.ep_known = 0; sh.ep_ok = 0; sh.ep_total = 0; sh.ep_path = 0; }
    for (int i = threadIdx.x; i < kMaxDnTiles * 64 * kMaxRows; i += kThreads) sh.hs[i] = 0;
    __syncthreads();
}

// Thread 0's early, non-blocking look at the mirrored epoch word (0 = not yet known).
__device__ __forceinline__ uint32_t epoch_peek(const Shared& sh, const uint32_t* slot) {
    return threadIdx.x == 0 && !sh.ep_known ? ld_agent(slot + kSyncEpoch) : 0u;
}

// (ok, total, path) of the queue, learnt once per workgroup from the word the mirror
// workgroup publishes. `early` is thread 0's epoch_peek taken before the item's loads.
__device__ __forceinline__ bool await_epoch(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t early) {
    // Every thread reads the flag before thread 0 may write it (barrier in between),
    // so the whole workgroup takes the same branch.
    const uint32_t known = sh.ep_known;
    __syncthreads();
    if (known) return sh.ep_ok != 0;
    if (threadIdx.x == 0) {
        uint32_t word = early;
        Waiter wt(a.spin_limit);
        while (!(word & 3u)) {
            if (ld_agent(slot + kSyncAbort)) { word = 2; break; }
            if (wt.expired()) { raise_status(a, slot, kStatusTimeout); word = 2; break; }
            __builtin_amdgcn_s_sleep(2);
            word = ld_agent(slot + kSyncEpoch);
        }
        const bool ok = (word & 3u) == 1u;
        sh.ep_ok = ok;
        sh.ep_path = ok ? (word >> 2) & 3u : 0u;
        sh.ep_total = ok ? word >> 4 : 0u;
        sh.ep_known = 1;
    }
    __syncthreads();
    return sh.ep_ok != 0;
}

// ---------------------------------------------------------------------------------
// Compact reduction by deterministic fixed-point accumulation (kAccOne in mlp_args.h).
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void st_agent_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void write_output(const MlpArgs& a, int col, unsigned long long word, uint32_t rows) {
    const long long sum = (long long)(word & kAccValueMask) - (long long)rows * kAccBias;
    const float v = (float)((double)sum * kAccInv);
    if (a.y32) a.y32[col] = v;
    a.y[col] = __builtin_bit_cast(uint16_t, (_Float16)v);
}


__device__ __forceinline__ bool load_queue_wg(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t pos, ExecDesc* out);

// h and down scales of a round's pairs staged in LDS. h as the fp16 values each
// down-projection thread multiplies: hs[i * stride + r0 * kMaxRows + j] = h_i[r0 + rpp * j]
// for pair i (stride = rpp * kMaxRows; zero for rows >= G, written once at start).
// Every thread polls its share of the tagged words (dest rows in sh.pdest) until each
// tag carries the launch sequence, then converts (exactly: h is fp16-representable).
// Scales: ss[i * kTileScales + t] = sv[i] (dn_scale_issue). Returns false for the whole
// workgroup when the wait was abandoned.
constexpr int kStageWords = 8;   // h words per thread per staging pass
__device__ __forceinline__ bool stage_round(const MlpArgs& a, uint32_t* slot, Shared& sh, uint32_t npairs,
                                            const DnGeom& gm, int G, const uint32_t (&sv)[kMaxDnTiles]) {
    const uint32_t total = npairs * (uint32_t)G;
    const uint32_t stride = (uint32_t)gm.rpp * kMaxRows;
    const uint64_t want = (uint64_t)a.seq;
    uint32_t* stop_flag = &sh.word[3];
    if (threadIdx.x == 0) *stop_flag = 0;
    __syncthreads();  // pdest written; earlier readers of hs / ss and the flag are done
#pragma unroll
    for (int i = 0; i < kMaxDnTiles; ++i)
        if ((uint32_t)i < npairs && (int)threadIdx.x < G * gm.nbk) sh.ss[i * kTileScales + threadIdx.x] = (uint16_t)sv[i];
    for (uint32_t f0 = 0; f0 < total; f0 += kStageWords * kThreads) {
        uint64_t v[kStageWords];
        const uint64_t* src[kStageWords];
#pragma unroll
        for (int q = 0; q < kStageWords; ++q) {
            const uint32_t f = f0 + threadIdx.x + q * kThreads;
            const uint32_t i = div_group(a, f), n = f - i * G;
            src[q] = f < total ? a.hbuf + (size_t)sh.pdest[i] * G + n : nullptr;
            v[q] = src[q] ? ld_agent_u64(src[q]) : (want << 32);
        }
        uint32_t stop = 0;
        Waiter wt(a.spin_limit);
        for (;;) {
            bool ok = true;
#pragma unroll
            for (int q = 0; q < kStageWords; ++q) ok = ok && (v[q] >> 32) == want;
            if (__all(ok)) break;
            uint32_t st = 0;
            if ((threadIdx.x & 63) == 0) {
                if (ld_agent(slot + kSyncAbort)) {
                    st = 1;
                } else if (wt.expired()) {
                    raise_status(a, slot, kStatusTimeout);
                    st = 1;
                }
            }
            stop = wave_bcast(st);
            if (stop) break;
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int q = 0; q < kStageWords; ++q)
                if ((v[q] >> 32) != want) v[q] = ld_agent_u64(src[q]);
        }
        if (stop) {
            if ((threadIdx.x & 63) == 0) *stop_flag = 1;
            break;
        }
#pragma unroll
        for (int q = 0; q < kStageWords; ++q) {
            const uint32_t f = f0 + threadIdx.x + q * kThreads;
            if (f < total) {
                const uint32_t i = div_group(a, f), n = f - i * G;
                sh.hs[i * stride + (n & (gm.rpp - 1)) * kMaxRows + (n >> gm.rpp_shift)] =
                    __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)v[q]));
            }
        }
    }
    __syncthreads();
    return *stop_flag == 0;
}

// Gate/up batch size of the width-D variant: one pass of the workgroup (4 waves).
template <int D>
struct Batch {
    static constexpr int N = GuGeom<D, 1>::NPP;
};

// Descriptor of global unit `gu` (core units first, then queue positions), validated.
__device__ __forceinline__ bool fetch_unit(const MlpArgs& a, Shared& sh, uint32_t* slot, const Bounds& b, uint32_t gu, int D,
                           Unit* out) {
    ExecDesc d;
    if (gu < a.core_count) {
        d = load_core(a, gu);
    } else if (!load_queue_wg(a, sh, slot, gu - a.core_count, &d)) {
        return false;
    }
    *out = resolve(a, b, d, D);
    if (!out->ok) {
        if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
        return false;
    }
    return true;
}

// Loads the descriptors of units sh.ulist[0..n) (n <= kUnitChunk, written by thread 0)
// in parallel, one word per thread, into sh.udesc: core units from the core array,
// queue positions from the device-side mirror once the mirror has copied them.
// One memory round trip (two when queue positions must first be waited for).
__device__ __forceinline__ bool load_units(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t n) {
    __syncthreads();  // ulist written; earlier readers of udesc are done
    if (threadIdx.x == 0) {
        uint32_t need = 0;  // queue positions that must be mirrored
        for (uint32_t i = 0; i < n; ++i)
            if (sh.ulist[i] >= a.core_count) need = max(need, sh.ulist[i] - a.core_count + 1);
        uint32_t ok = 1;
        if (need) {
            Waiter wt(a.spin_limit);
            while (ld_agent(slot + kSyncReady) < need) {
                if (ld_agent(slot + kSyncAbort)) { ok = 0; break; }
                if (wt.expired()) { raise_status(a, slot, kStatusTimeout); ok = 0; break; }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        sh.word[2] = ok;
    }
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(sh.word[2])) return false;
    if (threadIdx.x < 5 * n) {
        const uint32_t i = threadIdx.x / 5, w = threadIdx.x % 5, g = sh.ulist[i];
        sh.udesc[i][w] = g < a.core_count ? reinterpret_cast<const uint32_t*>(a.core)[5 * g + w]
                                          : ld_agent(a.qmirror + 5 * (g - a.core_count) + w);
    }
    __syncthreads();
    return true;
}

// Unit i of the last load_units, validated (wave-uniform values).
__device__ __forceinline__ bool unit_from(const MlpArgs& a, Shared& sh, uint32_t* slot, const Bounds& b, uint32_t i,
                                          int D, Unit* out) {
    ExecDesc d;
    d.logical_group = __builtin_amdgcn_readfirstlane(sh.udesc[i][0]);
    d.physical_group = __builtin_amdgcn_readfirstlane(sh.udesc[i][1]);
    d.source_slot = __builtin_amdgcn_readfirstlane(sh.udesc[i][2]);
    d.dest_slot = __builtin_amdgcn_readfirstlane(sh.udesc[i][3]);
    d.source_kind = (leanstream::runtime::SourceKind)__builtin_amdgcn_readfirstlane(sh.udesc[i][4]);
    *out = resolve(a, b, d, D);
    if (!out->ok) {
        if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
        return false;
    }
    return true;
}

// ---------------------------------------------------------------------------------
// Gate/up share: batches [g0, g1) of Batch<D>::N neurons (never straddling a unit; unit
// u0 + bi / bpu holds batch bi), kGuBuffers batches in flight, h stored tagged with the
// launch sequence. after_first() runs right after the first batch's loads are issued
// (the caller's own loads go there). Descriptors of units [chunk0, chunk0 + chunk_n) are
// already in sh.udesc from slot chunk_off on; later units are fetched kUnitChunk at a time.
// Never waits for another workgroup's h, so every worker finishes its share.
// ---------------------------------------------------------------------------------
template <int D, class AfterFirst>
__device__ __forceinline__ bool gate_up_share(const MlpArgs& a, Shared& sh, uint32_t* slot, const Bounds& b,
                                              XRegs<D, Batch<D>::N>& xr, bool& have_x, uint32_t u0, uint32_t g0,
                                              uint32_t g1, uint32_t bpu, uint32_t chunk0, uint32_t chunk_n,
                                              uint32_t chunk_off, AfterFirst after_first) {
    constexpr int NB = Batch<D>::N;
    const uint32_t G = a.group_size;
    if (g0 >= g1) return true;
    struct Meta {
        uint64_t* hrow;
        int n0, nvalid;
    };
    const uint32_t ulast = u0 + (g1 - 1) / bpu;      // last unit of the share (inclusive)
    auto issue = [&](uint32_t bi, GuLoads<D, NB>& L, Meta& m) -> bool {
        const uint32_t unit = u0 + bi / bpu;
        if (unit >= chunk0 + chunk_n) {
            chunk0 = unit;
            chunk_n = min((uint32_t)kUnitChunk, ulast + 1 - unit);
            chunk_off = 0;
            if (threadIdx.x == 0)
                for (uint32_t i = 0; i < chunk_n; ++i) sh.ulist[i] = chunk0 + i;
            if (!load_units(a, sh, slot, chunk_n)) return false;
        }
        Unit u;
        if (!unit_from(a, sh, slot, b, chunk_off + unit - chunk0, D, &u)) return false;
        if (threadIdx.x == 0 && a.first_compute && bi % bpu == 0) a.first_compute[u.dest] = now_ticks();
        m.n0 = (int)((bi % bpu) * NB);
        m.nvalid = min(NB, (int)G - m.n0);
        m.hrow = a.hbuf + (size_t)u.dest * G;
        gu_issue<D, NB>(u.grp, u.sc, m.n0, m.nvalid, L);
        return true;
    };
    // Loads return in issue order (vmcnt), so the issue order is the order data can be
    // used in: x, the first batch, then the caller's loads (after_first), then the rest.
    if (!have_x) {
        load_x<D, NB>(a.x, xr);
        have_x = true;
    }
    GuLoads<D, NB> L[kGuBuffers];
    Meta M[kGuBuffers];
#pragma unroll
    for (int q = 0; q < kGuBuffers; ++q) {
        if (g0 + q < g1 && !issue(g0 + q, L[q], M[q])) return false;
        if (q == 0 && !after_first()) return false;
    }
    for (uint32_t bi = g0; bi < g1; bi += kGuBuffers) {
#pragma unroll
        for (int q = 0; q < kGuBuffers; ++q) {
            if (bi + q < g1) {
                gu_compute<D, NB>(L[q], xr, M[q].hrow, M[q].n0, M[q].nvalid, a.seq);
                if (bi + q == g0) stamp(a, kStampFirstData);
                if (bi + q + kGuBuffers < g1 && !issue(bi + q + kGuBuffers, L[q], M[q])) return false;
            }
        }
    }
    return true;
}

// Execution counters (diagnostics): a unit counts once all of its down tiles are done.
__device__ __forceinline__ void count_execution(const MlpArgs& a, uint32_t* slot, uint32_t unit, uint32_t dest,
                                                uint32_t tiles) {
    if (threadIdx.x == 0 && add_agent(slot + kSyncUnits + unit * kLine, 1u) == tiles - 1)
        __hip_atomic_fetch_add(a.executions + dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---------------------------------------------------------------------------------
// Down projection work: the (unit, column tile) pairs of units [u0, u1) in tile-major
// order -- position p is tile p / units, unit p % units -- cut into one contiguous range
// per worker. A worker's consecutive pairs mostly share a column tile, so a run of them
// is summed locally and reaches the column accumulators as one atomic per column. Up to
// kMaxDnTiles pairs per round: their weight loads are issued together, then the h of all
// of them is staged in one polling pass.
// ---------------------------------------------------------------------------------

// Position in the tile-major pair order (relative unit, tile).
struct PairCursor {
    uint32_t unit, tile, units;
    __device__ PairCursor(uint32_t p, uint32_t n) : unit(p % n), tile(p / n), units(n) {}
    __device__ void advance() {
        if (++unit == units) {
            unit = 0;
            ++tile;
        }
    }
};

// Column accumulation of one thread (column c0 + threadIdx.x of the current tile run):
// a local fixed-point sum of m contributions, flushed as one packed atomic; the returned
// word is checked at the next flush (or at the end) so the atomic's latency overlaps work.
struct ColumnRun {
    long long sum = 0;
    uint32_t m = 0;
    int col = -1;
    unsigned long long pend = 0;
    int pend_col = -1;
};

__device__ __forceinline__ void check_pending(const MlpArgs& a, ColumnRun& r, uint32_t U) {
    if (r.pend_col >= 0 && U && (uint32_t)(r.pend >> 52) == U) write_output(a, r.pend_col, r.pend, U);
    r.pend_col = -1;
}

__device__ __forceinline__ void flush_run(const MlpArgs& a, unsigned long long* yacc, ColumnRun& r, uint32_t U) {
    if (r.m == 0) return;
    const unsigned long long add =
        (unsigned long long)(r.sum + (long long)r.m * kAccBias) + (unsigned long long)r.m * kAccOne;
    const unsigned long long now =
        __hip_atomic_fetch_add(yacc + r.col, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
    check_pending(a, r, U);
    r.pend = now;
    r.pend_col = r.col;
    r.sum = 0;
    r.m = 0;
}

// Adds the reduced tile value of this thread's column into its run (new run when the
// column changes). Out-of-range values are clipped and reported.
__device__ __forceinline__ void run_add(const MlpArgs& a, uint32_t* slot, unsigned long long* yacc, ColumnRun& r,
                                        int col, float value, uint32_t U) {
    if (col != r.col) {
        flush_run(a, yacc, r, U);
        r.col = col;
    }
    float v = value * kAccScale;
    if (!(fabsf(v) < (float)(kAccBias - 1))) {  // out of range or NaN: clip and report
        v = v > 0.f ? (float)(kAccBias - 1) : -(float)(kAccBias - 1);
        raise_status(a, slot, kStatusRange);
    }
    r.sum += __float2ll_rn(v);
    r.m += 1;
}

// One round of up to kMaxDnTiles (unit, column tile) pairs of the down projection:
// every weight and scale load of the round is issued first (dn_issue_round), then h and
// the scales are staged in LDS in one polling pass and each pair's tile is computed and
// added into the column runs (dn_finish_round).
struct DnRound {
    DnLoads dl[kMaxDnTiles];
    uint32_t sv[kMaxDnTiles];                        // this thread's staged scale (fp16 bits)
    uint32_t tile[kMaxDnTiles], index[kMaxDnTiles];  // column tile, unit index
    uint32_t npairs;
};

// unit_of(i, &unit) names pair i's validated unit.
template <int D, class UnitOf>
__device__ __forceinline__ bool dn_issue_round(const MlpArgs& a, Shared& sh, const DnGeom& gm, DnRound& rd,
                                               UnitOf unit_of) {
    const int tc = a.dn_tile;
#pragma unroll
    for (int i = 0; i < kMaxDnTiles; ++i) {
        rd.sv[i] = 0;
        if ((uint32_t)i < rd.npairs) {
            Unit u;
            if (!unit_of(i, &u)) return false;
            dn_issue<D>(u.grp, gm, (int)rd.tile[i] * tc, rd.dl[i]);
            rd.sv[i] = dn_scale_issue<D>(u.sc, gm, a.group_size, (int)rd.tile[i] * tc);
            if (threadIdx.x == 0) sh.pdest[i] = u.dest;
        }
    }
    return true;
}

template <int D>
__device__ __forceinline__ bool dn_finish_round(const MlpArgs& a, Shared& sh, uint32_t* slot, unsigned long long* yacc,
                                                const DnGeom& gm, const DnRound& rd, uint32_t U, ColumnRun& run) {
    const int tc = a.dn_tile;
    const uint32_t hstride = (uint32_t)gm.rpp * kMaxRows;
    if (!stage_round(a, slot, sh, rd.npairs, gm, a.group_size, rd.sv)) return false;
#pragma unroll
    for (int i = 0; i < kMaxDnTiles; ++i) {
        if ((uint32_t)i < rd.npairs) {
            dn_compute(rd.dl[i], gm, sh.hs + i * hstride, sh.ss + i * kTileScales, sh.red, tc);
            if (threadIdx.x < (uint32_t)tc)
                run_add(a, slot, yacc, run, (int)rd.tile[i] * tc + threadIdx.x, sh.red[kRedFloats + threadIdx.x], U);
            if (a.executions) count_execution(a, slot, rd.index[i], sh.pdest[i], D / tc);
        }
    }
    return true;
}

// ---------------------------------------------------------------------------------
// Units [u0, u1) on W persistent workers. Every worker takes a share of both halves:
//  - gate/up: a contiguous range of neuron batches (gate_up_share);
//  - down: a contiguous range of the tile-major (unit, column tile) pairs (PairCursor).
// The loads of the first down round are issued right after the first gate/up batch (one
// descriptor fetch covers both), so they stream with the gate/up loads. A worker waits
// for h only after its whole gate/up share is done, hence every h is eventually published.
// ---------------------------------------------------------------------------------
template <int D, bool FUSED>
__device__ __forceinline__ bool process_units(const MlpArgs& a, Shared& sh, uint32_t* slot, const Bounds& b,
                                              unsigned long long* yacc, XRegs<D, Batch<D>::N>& xr, bool& have_x,
                                              uint32_t u0, uint32_t u1, uint32_t k, uint32_t W,
                                              uint32_t early) {
    constexpr int NB = Batch<D>::N;
    const int G = a.group_size;
    const int tc = a.dn_tile;
    const uint32_t T = D / tc;                                    // tiles per unit
    // gate/up share
    const uint32_t bpu = (G + NB - 1) / NB;                       // batches per unit
    const uint32_t nb = (u1 - u0) * bpu;
    const uint32_t per_g = (nb + W - 1) / W;
    const uint32_t g0 = min(k * per_g, nb), g1 = min(g0 + per_g, nb);
    // down share: pairs [s0, s1) of the tile-major order
    const uint32_t nu = u1 - u0;
    const uint32_t P = nu * T;
    const uint32_t per_d = (P + W - 1) / W;
    const uint32_t s0 = min(k * per_d, P), s1 = min(s0 + per_d, P);
    PairCursor cur(s0, nu);   // next down pair
    const DnGeom gm(G, tc);
    // first down round + first gate/up units: one descriptor fetch
    DnRound rd;
    rd.npairs = s0 < s1 ? min((uint32_t)kMaxDnTiles, s1 - s0) : 0u;
#pragma unroll
    for (int i = 0; i < kMaxDnTiles; ++i) {
        rd.tile[i] = 0;
        rd.index[i] = 0;
        if ((uint32_t)i < rd.npairs) {
            rd.tile[i] = cur.tile;
            rd.index[i] = u0 + cur.unit;
            if (threadIdx.x == 0) sh.ulist[i] = u0 + cur.unit;
            cur.advance();
        }
    }
    uint32_t gchunk0 = 0, gchunk_n = 0;
    if (g0 < g1) {
        gchunk0 = u0 + g0 / bpu;
        gchunk_n = min((uint32_t)kUnitChunk - rd.npairs, u0 + (g1 - 1) / bpu + 1 - gchunk0);
        if (threadIdx.x == 0)
            for (uint32_t i = 0; i < gchunk_n; ++i) sh.ulist[rd.npairs + i] = gchunk0 + i;
    }
    if (rd.npairs + gchunk_n && !load_units(a, sh, slot, rd.npairs + gchunk_n)) return false;
    auto issue_down = [&]() {
        return dn_issue_round<D>(a, sh, gm, rd, [&](int i, Unit* u) { return unit_from(a, sh, slot, b, (uint32_t)i, D, u); });
    };
    if (g0 < g1) {
        if (!gate_up_share<D>(a, sh, slot, b, xr, have_x, u0, g0, g1, bpu, gchunk0, gchunk_n, rd.npairs, issue_down))
            return false;
    } else if (!issue_down()) {
        return false;
    }
    if (s0 >= s1) return true;
    uint32_t U = 0;
    if (FUSED) {
        if (!await_epoch(a, sh, slot, early)) return false;
        U = a.core_count + sh.ep_total;
    }
    ColumnRun run;
    for (uint32_t done = s0;;) {
        if (!dn_finish_round<D>(a, sh, slot, yacc, gm, rd, U, run)) return false;
        if (done == s0) stamp(a, kStampDnComputed);
        done += rd.npairs;
        if (done >= s1) break;
        rd.npairs = min((uint32_t)kMaxDnTiles, s1 - done);
#pragma unroll
        for (int i = 0; i < kMaxDnTiles; ++i) {
            if ((uint32_t)i < rd.npairs) {
                rd.tile[i] = cur.tile;
                rd.index[i] = u0 + cur.unit;
                if (threadIdx.x == 0) sh.ulist[i] = u0 + cur.unit;
                cur.advance();
            }
        }
        if (!load_units(a, sh, slot, rd.npairs)) return false;
        if (!dn_issue_round<D>(a, sh, gm, rd,
                               [&](int i, Unit* u) { return unit_from(a, sh, slot, b, (uint32_t)i, D, u); }))
            return false;
    }
    flush_run(a, yacc, run, U);
    check_pending(a, run, U);
    return true;
}

// Process a whole unit inside one workgroup (claim path): gate/up of every neuron, then
// every column tile of the down projection, without cross-workgroup waits.
template <int D, bool FUSED>
__device__ __forceinline__ bool run_unit_solo(const MlpArgs& a, Shared& sh, uint32_t* slot, unsigned long long* yacc,
                                              const XRegs<D, Batch<D>::N>& xr, const Unit& u, uint32_t index) {
    constexpr int NB = Batch<D>::N;
    const int G = a.group_size;
    uint64_t* hrow = a.hbuf + (size_t)u.dest * G;
    if (threadIdx.x == 0 && a.first_compute) a.first_compute[u.dest] = now_ticks();
    for (int n0 = 0; n0 < G; n0 += NB) {
        GuLoads<D, NB> gl;
        gu_issue<D, NB>(u.grp, u.sc, n0, min(NB, G - n0), gl);
        gu_compute<D, NB>(gl, xr, hrow, n0, min(NB, G - n0), a.seq);
    }
    const int tc = a.dn_tile;
    const uint32_t T = D / tc;
    const DnGeom gm(G, tc);
    const uint32_t U = FUSED ? a.core_count + sh.ep_total : 0u;
    ColumnRun run;
    for (uint32_t t0 = 0; t0 < T; t0 += kMaxDnTiles) {
        DnRound rd;
        rd.npairs = min((uint32_t)kMaxDnTiles, T - t0);
#pragma unroll
        for (int i = 0; i < kMaxDnTiles; ++i) {
            rd.tile[i] = t0 + (uint32_t)i;
            rd.index[i] = index;
        }
        if (!dn_issue_round<D>(a, sh, gm, rd, [&](int, Unit* out) {
                *out = u;
                return true;
            }))
            return false;
        if (!dn_finish_round<D>(a, sh, slot, yacc, gm, rd, U, run)) return false;
    }
    flush_run(a, yacc, run, U);
    check_pending(a, run, U);
    return true;
}

// ---------------------------------------------------------------------------------
// Queue protocol (LeanStream kernels/streaming_mlp.cu:47-79, backends/triton/persistent.py:32-92):
// wait for the layer epoch (or an error), optionally for batch publication, decide once
// per launch between the all-ready fast path and the claim path, then consume published
// positions in order.
//
// On MI355X the queue lives in host memory behind PCIe, where concurrent reads from
// hundreds of workgroups are served one after another. So exactly one workgroup of
// each launch (the mirror, the last block) reads host memory: it publishes the packed
// (state, path, total) word into the device ring slot, copies every newly published
// position's descriptor into a device-side table in publication order (64 positions
// per round trip, one per lane) and advances a device-side ready count. Workers only
// poll device memory.
// ---------------------------------------------------------------------------------
// Runs on wave 0 of the mirror workgroup. `pre` is lane 0's early 64-bit load of
// (total_count, epoch): adjacent words (byte offsets 8 and 12), read as one pair.
__device__ __forceinline__ void mirror_queue(const MlpArgs& a, uint32_t* slot, uint64_t pre) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t state = 0, total = 0;
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
        uint32_t path = 0;
        if (state == 1 && total) path = ld_sys(&a.control->ready_count) >= total ? 2u : 1u;
        st_agent(slot + kSyncEpoch, pack_epoch(state, path, state == 1 ? total : 0u));
    }
    state = wave_bcast(state);
    total = wave_bcast(total);
    if (state != 1) return;
    if (total == 0 && a.core_count == 0) {
        // no rows at all: the reduction of nothing is zero
        for (uint32_t c = lane; c < a.width; c += 64) {
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
                    const uint32_t idx = ld_sys(a.ready + pos);
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

// Descriptor of published position `pos` from the device-side table; false when the
// worker must leave (abort or timeout) before the position is mirrored.
__device__ __forceinline__ bool load_queue_wg(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t pos, ExecDesc* out) {
    __syncthreads();  // previous readers of sh.desc / sh.word[2] are done
    if (threadIdx.x == 0) {
        uint32_t ok = 1;
        Waiter wt(a.spin_limit);
        while (ld_agent(slot + kSyncReady) <= pos) {
            if (ld_agent(slot + kSyncAbort)) { ok = 0; break; }
            if (wt.expired()) { raise_status(a, slot, kStatusTimeout); ok = 0; break; }
            __builtin_amdgcn_s_sleep(1);
        }
        if (ok)
            for (int k = 0; k < 5; ++k) sh.desc[k] = ld_agent(a.qmirror + 5 * pos + k);
        sh.word[2] = ok;
    }
    __syncthreads();
    // every lane reads the same words: make them wave-uniform (scalar registers)
    out->logical_group = __builtin_amdgcn_readfirstlane(sh.desc[0]);
    out->physical_group = __builtin_amdgcn_readfirstlane(sh.desc[1]);
    out->source_slot = __builtin_amdgcn_readfirstlane(sh.desc[2]);
    out->dest_slot = __builtin_amdgcn_readfirstlane(sh.desc[3]);
    out->source_kind = (leanstream::runtime::SourceKind)__builtin_amdgcn_readfirstlane(sh.desc[4]);
    return __builtin_amdgcn_readfirstlane(sh.word[2]) != 0;
}

// Claim the next ready pair [head, min(head+2, ready)) (backends/triton/persistent.py:77-86),
// against the mirrored ready count. Returns the number of claimed positions (0 = leave).
__device__ __forceinline__ uint32_t claim_pair(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t total) {
    __syncthreads();  // previous readers of sh.word[5..6] are done
    if (threadIdx.x == 0) {
        uint32_t got = 0, head = 0;
        Waiter wt(a.spin_limit);
        for (;;) {
            if (ld_agent(slot + kSyncAbort)) break;
            const uint32_t ready = ld_agent(slot + kSyncReady);
            head = ld_agent(slot + kSyncClaimHead);
            if (head >= total) break;
            if (head < ready) {
                const uint32_t end = min(head + 2u, min(ready, total));
                uint32_t expected = head;
                if (__hip_atomic_compare_exchange_strong(slot + kSyncClaimHead, &expected, end, __ATOMIC_RELAXED,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    got = end - head;
                    const uint32_t seq = add_agent(slot + kSyncClaims, 1u);
                    if (a.claim_log && seq < a.claim_log_cap) a.claim_log[seq] = head | (got << 24);
                    break;
                }
                continue;
            }
            if (wt.expired()) { raise_status(a, slot, kStatusTimeout); break; }
            __builtin_amdgcn_s_sleep(2);
        }
        sh.word[5] = head;
        sh.word[6] = got;
    }
    __syncthreads();
    return sh.word[6];
}

// Claim path (progressive publication): ready pairs claimed one at a time, each unit of
// a pair processed whole by the claiming workgroup.
template <int D, bool FUSED>
__device__ __forceinline__ void claim_loop(const MlpArgs& a, Shared& sh, uint32_t* slot, const Bounds& b, unsigned long long* yacc,
                           const XRegs<D, Batch<D>::N>& xr, uint32_t total) {
    for (;;) {
        const uint32_t got = claim_pair(a, sh, slot, total);
        if (!got) return;
        const uint32_t head = sh.word[5];
        for (uint32_t k = 0; k < got; ++k) {
            Unit u;
            if (!fetch_unit(a, sh, slot, b, a.core_count + head + k, D, &u)) return;
            if (!run_unit_solo<D, FUSED>(a, sh, slot, yacc, xr, u, a.core_count + head + k)) return;
        }
    }
}

// One persistent worker of a launch: its role share of the resident (core) units, then
// of the queue (all-ready fast path), or the claim loop (progressive path).
// Workers [0, NG) take the gate/up role, the others the down role.
// One persistent worker of a launch: its share of the resident (core) units, then of
// the queue (all-ready fast path), or the claim loop (progressive path).
template <int D, bool FUSED, bool CORE, bool QUEUE>
__device__ __forceinline__ void worker(const MlpArgs& a, const Bounds& b, Shared& sh, uint32_t* slot) {
    const uint32_t W = QUEUE ? gridDim.x - 1 : gridDim.x;
    unsigned long long* yacc = a.yacc + (a.seq & 1) * a.width;
    init_shared(sh);
    XRegs<D, Batch<D>::N> xr;
    bool have_x = false;
    const uint32_t early = epoch_peek(sh, slot);
    if (CORE && a.core_count &&
        !process_units<D, FUSED>(a, sh, slot, b, yacc, xr, have_x, 0, a.core_count, blockIdx.x, W, early))
        return;
    stamp(a, kStampCoreDone);
    if (!QUEUE) return;
    if (!await_epoch(a, sh, slot, early)) return;
    stamp(a, kStampEpoch);
    const uint32_t total = sh.ep_total;
    if (!total) return;
    if (sh.ep_path == 2) {
        process_units<D, FUSED>(a, sh, slot, b, yacc, xr, have_x, a.core_count, a.core_count + total, blockIdx.x, W, 0);
    } else {
        if (!have_x) load_x<D, Batch<D>::N>(a.x, xr);
        claim_loop<D, FUSED>(a, sh, slot, b, yacc, xr, total);
    }
    stamp(a, kStampQueueDone);
}

// The mirror workgroup: wave 0 mirrors the queue while waves 1..3 clear what the next
// launch will use -- the other ring slot and the other accumulator buffer, both last
// used by the previous launch (finished, by stream order).
__device__ __forceinline__ void run_mirror(const MlpArgs& a, uint32_t* slot, uint64_t pre) {
    if (threadIdx.x < 64) {
        mirror_queue(a, slot, pre);
        return;
    }
    const uint32_t t = threadIdx.x - 64, n = kThreads - 64;
    uint32_t* other = a.sync + ((a.seq + 1) & 1) * a.slot_words;
    for (uint32_t i = t; i < a.slot_words; i += n) st_agent(other + i, 0u);
    unsigned long long* other_acc = a.yacc + ((a.seq + 1) & 1) * a.width;
    for (uint32_t i = t; i < a.width; i += n) st_agent_u64(other_acc + i, 0ull);
}

// Completion proof of a launch (replaces a per-launch event): every workgroup counts
// itself out once it has finished, in two levels to keep the count off one contended
// word -- per group of workgroups blk % 8 (kSyncExitGroups), then the last of each
// group in kSyncExit. The very last one stores the launch sequence into the
// host-coherent completion word; all reads of the launch's weights are complete by then.
__device__ __forceinline__ void finish_launch(const MlpArgs& a, uint32_t* slot) {
    __syncthreads();
    if (threadIdx.x != 0) return;
    const uint32_t group = blockIdx.x % 8u;
    const uint32_t members = (gridDim.x + 7u - group) / 8u;
    const uint32_t groups = gridDim.x < 8u ? gridDim.x : 8u;
    if (add_agent(slot + kSyncExitGroups + group * kLine, 1u) == members - 1 &&
        add_agent(slot + kSyncExit, 1u) == groups - 1)
        __hip_atomic_store(a.done, a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ unsigned long long* launch_acc(const MlpArgs& a) { return a.yacc + (a.seq & 1) * a.width; }

// ---------------------------------------------------------------------------------
// Kernels. Persistent launches have gridDim.x = workers + 1; the last block mirrors.
// ---------------------------------------------------------------------------------

// Fused layer: resident (core) units, queue consumption and the compact reduction (the
// contribution completing a column writes it), one persistent launch.
template <int D>
__global__ __launch_bounds__(kThreads, 2) void fused_layer_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    if (blockIdx.x == gridDim.x - 1) {
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
    } else {
        stamp(a, kStampEntry);
        worker<D, true, true, true>(a, b, sh, slot);
        stamp(a, kStampExit);
    }
    finish_launch(a, slot);
}

// Split path, stage A: resident (core) units only; no queue, no conversion.
template <int D>
__global__ __launch_bounds__(kThreads, 2) void stage_a_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    worker<D, false, true, false>(a, b, sh, slot);
}

// Split path, stage B: persistent ready-queue consumer (last block mirrors).
template <int D>
__global__ __launch_bounds__(kThreads, 2) void stage_b_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    if (blockIdx.x == gridDim.x - 1) {
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
        return;
    }
    worker<D, false, false, true>(a, b, sh, slot);
}

// Split path, compact reduction (streaming_mlp.cu:80-84): converts every column's
// accumulator to y32 / y. 256 columns per block.
template <int D>
__global__ __launch_bounds__(kThreads) void reduce_kernel(MlpArgs a) {
    const int col = blockIdx.x * kThreads + threadIdx.x;
    const unsigned long long w = __hip_atomic_load(launch_acc(a) + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    write_output(a, col, w, (uint32_t)(w >> 52));
    finish_launch(a, a.sync + (a.seq & 1) * a.slot_words);   // last kernel of the split launch sequence
}

// Clears both ring slots, the accumulators and the tagged h rows (bind time, after a
// failed enqueue, or when the launch sequence wraps): afterwards no stored tag can match
// a sequence number the next launches use.
__global__ void clear_sync_kernel(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns,
                                  uint64_t* hbuf, uint32_t hwords) {
    // `columns` covers both accumulator buffers
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) st_agent(sync + i, 0u);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < columns; i += stride) st_agent_u64(yacc + i, 0ull);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hwords; i += stride)
        __hip_atomic_store(hbuf + i, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------
// Host-side launch dispatch over the compiled (width, neurons-per-item) variants.
// ---------------------------------------------------------------------------------
namespace {

struct Variant {
    int width;
    const void* fused;
    const void* stage_a;
    const void* stage_b;
    const void* reduce;
};

template <int D>
Variant make_variant() {
    return {D, reinterpret_cast<const void*>(&fused_layer_kernel<D>), reinterpret_cast<const void*>(&stage_a_kernel<D>),
            reinterpret_cast<const void*>(&stage_b_kernel<D>), reinterpret_cast<const void*>(&reduce_kernel<D>)};
}

const Variant* find_variant(int width) {
    static const Variant table[] = {make_variant<256>(),  make_variant<512>(),  make_variant<1024>(),
                                    make_variant<2048>(), make_variant<4096>(), make_variant<8192>()};
    for (const Variant& v : table)
        if (v.width == width) return &v;
    return nullptr;
}

}  // namespace

bool variant_available(int width) { return find_variant(width) != nullptr; }

hipError_t resident_workers(int width, int entry_point, int* per_cu) {
    const Variant* v = find_variant(width);
    if (!v) return hipErrorInvalidValue;
    const void* k = entry_point == kEntryFused ? v->fused : v->stage_b;
    int n = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kThreads, 0);
    if (e == hipSuccess && entry_point != kEntryFused) {
        int na = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&na, v->stage_a, kThreads, 0);
        if (na < n) n = na;
    }
    *per_cu = n;
    return e;
}

hipError_t launch_layer(const LaunchPlan& p, const MlpArgs& args, const Bounds& bounds, hipStream_t stream) {
    const Variant* v = find_variant(p.width);
    if (!v || p.workers < 1) return hipErrorInvalidValue;
    MlpArgs a = args;
    Bounds b = bounds;
    void* kargs[] = {&a, &b};
    if (p.entry_point == kEntryFused)
        return hipLaunchKernel(v->fused, dim3(p.workers + 1), dim3(kThreads), kargs, 0, stream);
    hipError_t e = hipSuccess;
    if (a.core_count) {
        e = hipLaunchKernel(v->stage_a, dim3(p.workers), dim3(kThreads), kargs, 0, stream);
        if (e != hipSuccess) return e;
    }
    e = hipLaunchKernel(v->stage_b, dim3(p.workers + 1), dim3(kThreads), kargs, 0, stream);
    if (e != hipSuccess) return e;
    void* rargs[] = {&a};
    return hipLaunchKernel(v->reduce, dim3(p.width / kThreads), dim3(kThreads), rargs, 0, stream);
}

hipError_t clear_sync(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns, uint64_t* hbuf,
                      uint32_t hwords, hipStream_t stream) {
    const uint32_t most = words > hwords ? words : hwords;
    uint32_t grid = (most + kThreads - 1) / kThreads;
    if (grid > 1024) grid = 1024;
    if (!grid) grid = 1;
    void* kargs[] = {&sync, &words, &yacc, &columns, &hbuf, &hwords};
    return hipLaunchKernel(reinterpret_cast<const void*>(&clear_sync_kernel), dim3(grid), dim3(kThreads), kargs, 0,
                           stream);
}

}  // namespace lsamd
