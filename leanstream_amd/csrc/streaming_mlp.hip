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

constexpr int kThreads = 256;
constexpr int kMaxRows = 16;         // down-projection rows per thread held in registers
constexpr int kRedFloats = 2048;     // LDS scratch for the cross-thread column reduction

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
    uint16_t s[GuGeom<D, NS>::PASSES][2][GuGeom<D, NS>::CPL];
};

// Issue every gate/up load of one item. grp points at the unit's packed bytes,
// sc at the unit's scale rows, n0 is the first neuron of the item.
template <int D, int NS>
__device__ __forceinline__ void gu_issue(const uint8_t* grp, const uint16_t* sc, int n0, GuLoads<D, NS>& L) {
    using Gm = GuGeom<D, NS>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane % Gm::LPR, sub = lane / Gm::LPR;
#pragma unroll
    for (int p = 0; p < Gm::PASSES; ++p) {
        const int nu = p * Gm::NPP + wave * Gm::NPW + sub;   // neuron within the item
        const bool ok = nu < NS;
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

// Finish gate/up for the item: dot products, row reductions, activation.
// Writes h (fp32, fp16-exact) for neurons n0..n0+NS-1 of unit row `hrow`.
template <int D, int NS>
__device__ __forceinline__ void gu_compute(const GuLoads<D, NS>& L, const XRegs<D, NS>& xr, uint64_t* hrow, int n0,
                                           uint32_t seq) {
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
                const _Float16 sv = half_bits(L.s[p][proj][k]);
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
#pragma unroll
        for (int m = 1; m < Gm::LPR; m <<= 1) {
            acc[0] += __shfl_xor(acc[0], m, 64);
            acc[1] += __shfl_xor(acc[1], m, 64);
        }
        const int nu = p * Gm::NPP + wave * Gm::NPW + sub;
        if (r == 0 && nu < NS) {
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
// Down projection of one column tile of one unit (all G neurons), tc columns.
// Thread t owns 8 columns (one packed word per row) and rows r0, r0+rpp, ...
// ---------------------------------------------------------------------------------
struct DnLoads {
    uint32_t w[kMaxRows];
    uint16_t s[kMaxRows];
};

struct DnGeom {
    int dwr, rpp, dc, r0, nrows;
    __device__ DnGeom(int G, int tc) {
        dwr = tc >> 3;                 // packed words per row in the tile
        rpp = kThreads / dwr;          // rows covered per pass of the workgroup
        dc = threadIdx.x % dwr;
        r0 = threadIdx.x / dwr;
        nrows = r0 < G ? (G - r0 + rpp - 1) / rpp : 0;
    }
};

template <int D>
__device__ __forceinline__ void dn_issue(const uint8_t* grp, const uint16_t* sc, const DnGeom& gm, int c0, DnLoads& L) {
    constexpr int BLOCKS = D / 128;
    const int col = c0 + 8 * gm.dc;
#pragma unroll
    for (int i = 0; i < kMaxRows; ++i) {
        if (i < gm.nrows) {
            const int n = gm.r0 + gm.rpp * i;
            L.w[i] = ld_stream4(grp + (size_t)n * (3 * D / 2) + D + (col >> 1));
            L.s[i] = sc[(size_t)n * 3 * BLOCKS + 2 * BLOCKS + (col >> 7)];
        } else {
            L.w[i] = 0;
            L.s[i] = 0;
        }
    }
}

__device__ __forceinline__ uint64_t ld_agent_u64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t wave_bcast(uint32_t v) { return __shfl(v, 0, 64); }

// Down projection of the tile, consuming h as the unit's items publish it. Each lane
// needs h only for its own rows; row pairs are processed in a fixed order, and a wave
// waits (polling the tagged words) only when the next pair's h has not arrived yet,
// so the down-projection arithmetic overlaps the wait for slower sibling items.
// The tile is summed into red[kRedFloats + c] (c < tc): per thread over its rows in
// increasing order (pairs via dot2), then across row groups r0 = 0..rpp-1.
// Returns false (for the whole workgroup) when the wait was abandoned.
__device__ bool dn_compute(const MlpArgs& a, uint32_t* slot, const DnLoads& L, const DnGeom& gm, const uint64_t* hrow,
                           float* red, uint32_t* stop_flag, int tc) {
    const uint64_t want = (uint64_t)a.seq;
    uint64_t hv[kMaxRows];
#pragma unroll
    for (int i = 0; i < kMaxRows; ++i) hv[i] = i < gm.nrows ? ld_agent_u64(hrow + gm.r0 + gm.rpp * i) : (want << 32);
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.f;
    uint32_t stop = 0;
    Waiter wt(a.spin_limit);
#pragma unroll
    for (int i = 0; i < kMaxRows; i += 2) {
        for (;;) {
            const int ok = (hv[i] >> 32) == want && (hv[i + 1] >> 32) == want;
            if (__all(ok) || stop) break;
            uint32_t s = 0;
            if ((threadIdx.x & 63) == 0) {
                if (ld_agent(slot + kSyncAbort)) {
                    s = 1;
                } else if (wt.expired()) {
                    raise_status(a, slot, kStatusTimeout);
                    s = 1;
                }
            }
            stop = wave_bcast(s);
            if (stop) break;
            __builtin_amdgcn_s_sleep(1);
            if ((hv[i] >> 32) != want) hv[i] = ld_agent_u64(hrow + gm.r0 + gm.rpp * i);
            if ((hv[i + 1] >> 32) != want) hv[i + 1] = ld_agent_u64(hrow + gm.r0 + gm.rpp * (i + 1));
        }
        if (stop) break;
        if (i < gm.nrows) {
            const bool pair = i + 1 < gm.nrows;
            const uint32_t wa = L.w[i], wb = pair ? L.w[i + 1] : L.w[i];
            const _Float16 ha = (_Float16)__uint_as_float((uint32_t)hv[i]);
            const _Float16 hb = pair ? (_Float16)__uint_as_float((uint32_t)hv[i + 1]) : (_Float16)0.0f;
            const h2 hab = {ha, hb};
            const h2 sab = {half_bits(L.s[i]), half_bits(pair ? L.s[i + 1] : L.s[i])};
            h2 w[4];
            dequant8(__builtin_amdgcn_perm(wb, wa, 0x05040100u), sab, w);   // columns 0..3
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = dot2(w[c], hab, acc[c]);
            dequant8(__builtin_amdgcn_perm(wb, wa, 0x07060302u), sab, w);   // columns 4..7
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[4 + c] = dot2(w[c], hab, acc[4 + c]);
        }
    }
    if (stop && (threadIdx.x & 63) == 0) *stop_flag = 1;
    __syncthreads();  // red[] may still be read by a previous tile; stop flags are set
    const bool leave = *stop_flag != 0;
    if (!leave) {
        if (gm.nrows > 0) {
#pragma unroll
            for (int c = 0; c < 8; ++c) red[gm.r0 * tc + 8 * gm.dc + c] = acc[c];
        } else if (gm.r0 < gm.rpp) {
#pragma unroll
            for (int c = 0; c < 8; ++c) red[gm.r0 * tc + 8 * gm.dc + c] = 0.f;
        }
    }
    __syncthreads();
    if (leave) return false;
    for (int c = threadIdx.x; c < tc; c += kThreads) {
        float v = 0.f;
        for (int r = 0; r < gm.rpp; ++r) v += red[r * tc + c];
        red[kRedFloats + c] = v;   // reduced tile (second half of the scratch)
    }
    __syncthreads();
    return true;
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
    float red[2 * kRedFloats];
    float hs[256];
    uint32_t word[8];
    uint32_t desc[5];
    // queue state learnt once per launch: known, ok, total, path
    uint32_t ep_known, ep_ok, ep_total, ep_path;
};

__device__ __forceinline__ void init_shared(Shared& sh) {
    if (threadIdx.x == 0) { sh.ep_known = 0; sh.ep_ok = 0; sh.ep_total = 0; sh.ep_path = 0; }
    __syncthreads();
}

// Thread 0's early, non-blocking look at the mirrored epoch word (0 = not yet known).
__device__ __forceinline__ uint32_t epoch_peek(const Shared& sh, const uint32_t* slot) {
    return threadIdx.x == 0 && !sh.ep_known ? ld_agent(slot + kSyncEpoch) : 0u;
}

// (ok, total, path) of the queue, learnt once per workgroup from the word the mirror
// workgroup publishes. `early` is thread 0's epoch_peek taken before the item's loads.
__device__ bool await_epoch(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t early) {
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

// Adds the reduced tile (tile[c], c < tc) into the column words; with U > 0 (fused
// launch) the contribution that completes a column writes its output.
__device__ __forceinline__ void accumulate_tile(const MlpArgs& a, uint32_t* slot, unsigned long long* yacc,
                                                const float* tile, int c0, int tc, uint32_t U) {
    bool clipped = false;
    for (int c = threadIdx.x; c < tc; c += kThreads) {
        float v = tile[c] * kAccScale;
        if (!(fabsf(v) < (float)(kAccBias - 1))) {  // out of range or NaN: clip and report
            clipped = true;
            v = v > 0.f ? (float)(kAccBias - 1) : -(float)(kAccBias - 1);
        }
        const unsigned long long add = (unsigned long long)(__float2ll_rn(v) + kAccBias) + kAccOne;
        if (U) {
            const unsigned long long now =
                __hip_atomic_fetch_add(yacc + c0 + c, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
            if ((uint32_t)(now >> 52) == U) write_output(a, c0 + c, now, U);
        } else {
            __hip_atomic_fetch_add(yacc + c0 + c, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (clipped) raise_status(a, slot, kStatusRange);
}

// ---------------------------------------------------------------------------------
// One cooperative item: gate/up for slice j of unit `unit`, then (once all S slices of
// the unit stored h) the down projection of column tile j into the accumulators.
// FUSED: also count the tile; the U-th contributor converts it.
// ---------------------------------------------------------------------------------
template <int D, int NS, bool FUSED>
__device__ void run_item(const MlpArgs& a, Shared& sh, uint32_t* slot, unsigned long long* yacc, const XRegs<D, NS>& xr,
                         const Unit& u, uint32_t unit, uint32_t j, uint32_t it) {
    const uint32_t sb = kStampItemBase + 7 * (it < 4 ? it : 4);
    stamp(a, sb + 0);
    const uint32_t early = FUSED ? epoch_peek(sh, slot) : 0u;
    const int G = a.group_size;
    const int S = a.slices;
    const int tc = D / S;
    const int c0 = j * tc;
    if (j == 0 && threadIdx.x == 0 && a.first_compute) a.first_compute[u.dest] = now_ticks();
    GuLoads<D, NS> gl;
    gu_issue<D, NS>(u.grp, u.sc, j * NS, gl);
    DnGeom gm(G, tc);
    DnLoads dl;
    dn_issue<D>(u.grp, u.sc, gm, c0, dl);
    gu_compute<D, NS>(gl, xr, a.hbuf + (size_t)u.dest * G, j * NS, a.seq);
    stamp(a, sb + 1);
    if (threadIdx.x == 0) sh.word[3] = 0;
    __syncthreads();
    if (!dn_compute(a, slot, dl, gm, a.hbuf + (size_t)u.dest * G, sh.red, &sh.word[3], tc)) return;
    stamp(a, sb + 3);
    if (FUSED && !await_epoch(a, sh, slot, early)) return;
    accumulate_tile(a, slot, yacc, sh.red + kRedFloats, c0, tc, FUSED ? a.core_count + sh.ep_total : 0u);
    stamp(a, sb + 4);
    if (a.executions) {
        drain_vmem();
        __syncthreads();
        if (threadIdx.x == 0 && add_agent(slot + kSyncUnits + unit * kLine + 1, 1u) == (uint32_t)S - 1)
            __hip_atomic_fetch_add(a.executions + u.dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    stamp(a, sb + 6);
}

// Process a whole unit inside one workgroup (claim path): no cross-workgroup wait.
template <int D, int NS, bool FUSED>
__device__ void run_unit_solo(const MlpArgs& a, Shared& sh, uint32_t* slot, unsigned long long* yacc,
                              const XRegs<D, NS>& xr, const Unit& u) {
    const int S = a.slices;
    const int G = a.group_size;
    // gate/up for every slice first so that the whole h row exists, then the tiles.
    for (int j = 0; j < S; ++j) {
        if (j == 0 && threadIdx.x == 0 && a.first_compute) a.first_compute[u.dest] = now_ticks();
        GuLoads<D, NS> gl;
        gu_issue<D, NS>(u.grp, u.sc, j * NS, gl);
        gu_compute<D, NS>(gl, xr, a.hbuf + (size_t)u.dest * G, j * NS, a.seq);
    }
    const int tc = D / S;
    DnGeom gm(G, tc);
    const uint32_t U = FUSED ? a.core_count + sh.ep_total : 0u;
    for (int j = 0; j < S; ++j) {
        const int c0 = j * tc;
        DnLoads dl;
        dn_issue<D>(u.grp, u.sc, gm, c0, dl);
        if (threadIdx.x == 0) sh.word[3] = 0;
        __syncthreads();
        if (!dn_compute(a, slot, dl, gm, a.hbuf + (size_t)u.dest * G, sh.red, &sh.word[3], tc)) return;
        accumulate_tile(a, slot, yacc, sh.red + kRedFloats, c0, tc, U);
    }
    if (a.executions) {
        drain_vmem();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(a.executions + u.dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
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
__device__ void mirror_queue(const MlpArgs& a, uint32_t* slot, uint64_t pre) {
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
__device__ bool load_queue_wg(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t pos, ExecDesc* out) {
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
    out->logical_group = sh.desc[0];
    out->physical_group = sh.desc[1];
    out->source_slot = sh.desc[2];
    out->dest_slot = sh.desc[3];
    out->source_kind = (leanstream::runtime::SourceKind)sh.desc[4];
    return sh.word[2] != 0;
}

// Claim the next ready pair [head, min(head+2, ready)) (backends/triton/persistent.py:77-86),
// against the mirrored ready count. Returns the number of claimed positions (0 = leave).
__device__ uint32_t claim_pair(const MlpArgs& a, Shared& sh, uint32_t* slot, uint32_t total) {
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

template <int D, int NS, bool FUSED>
__device__ void consume_queue(const MlpArgs& a, Shared& sh, uint32_t* slot, unsigned long long* yacc, const XRegs<D, NS>& xr,
                              const Bounds& b, uint32_t W, uint32_t w, uint32_t first_item, uint32_t it) {
    if (!await_epoch(a, sh, slot, epoch_peek(sh, slot))) return;
    const uint32_t total = sh.ep_total;
    const uint32_t path = sh.ep_path;
    if (!total) return;
    const uint32_t S = a.slices;
    if (path == 2) {
        // all ready: static stripes of (position, slice) items, continuing the
        // round-robin after the core items so every worker gets an equal share.
        const uint32_t n_items = total * S;
        for (uint32_t i = (w + W - (first_item % W)) % W; i < n_items; i += W) {
            const uint32_t pos = i / S, j = i % S;
            ExecDesc d;
            if (!load_queue_wg(a, sh, slot, pos, &d)) return;
            const Unit u = resolve(a, b, d, D);
            if (!u.ok) {
                if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
                return;
            }
            if (threadIdx.x == 0 && j == 0 && a.claim_log && (pos & 1) == 0 && pos / 2 < a.claim_log_cap)
                a.claim_log[pos / 2] = pos | (min(2u, total - pos) << 24);
            run_item<D, NS, FUSED>(a, sh, slot, yacc, xr, u, a.core_count + pos, j, it++);
        }
        return;
    }
    for (;;) {
        const uint32_t got = claim_pair(a, sh, slot, total);
        if (!got) return;
        const uint32_t head = sh.word[5];
        for (uint32_t k = 0; k < got; ++k) {
            ExecDesc d;
            if (!load_queue_wg(a, sh, slot, head + k, &d)) return;
            const Unit u = resolve(a, b, d, D);
            if (!u.ok) {
                if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
                return;
            }
            run_unit_solo<D, NS, FUSED>(a, sh, slot, yacc, xr, u);
        }
    }
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

__device__ __forceinline__ unsigned long long* launch_acc(const MlpArgs& a) { return a.yacc + (a.seq & 1) * a.width; }

// ---------------------------------------------------------------------------------
// Kernels. Persistent launches have gridDim.x = workers + 1; the last block mirrors.
// ---------------------------------------------------------------------------------

// Fused layer: core items (stage A role), queue consumption (stage B role) and the
// compact reduction (U-th contributor of each column tile), one persistent launch.
template <int D, int NS>
__global__ __launch_bounds__(kThreads, 2) void fused_layer_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    const uint32_t W = gridDim.x - 1, w = blockIdx.x;
    if (w == W) {
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
        return;
    }
    stamp(a, kStampEntry);
    unsigned long long* yacc = launch_acc(a);
    const uint32_t S = a.slices;
    const uint32_t n_core = a.core_count * S;
    // the first core descriptor is read before anything else: every later load waits
    // behind it in the in-order return queue
    ExecDesc d0 = w < n_core ? load_core(a, w / S) : ExecDesc{};
    init_shared(sh);
    XRegs<D, NS> xr;
    load_x<D, NS>(a.x, xr);
    stamp(a, kStampXLoaded);
    uint32_t it = 0;
    for (uint32_t i = w; i < n_core; i += W) {
        const uint32_t unit = i / S, j = i % S;
        const Unit u = resolve(a, b, i == w ? d0 : load_core(a, unit), D);
        if (!u.ok) {
            if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
            break;
        }
        run_item<D, NS, true>(a, sh, slot, yacc, xr, u, unit, j, it++);
    }
    consume_queue<D, NS, true>(a, sh, slot, yacc, xr, b, W, w, n_core, it);
    stamp(a, kStampExit);
}

// Split path, stage A: core items only (no queue, no conversion).
template <int D, int NS>
__global__ __launch_bounds__(kThreads, 2) void stage_a_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    unsigned long long* yacc = launch_acc(a);
    init_shared(sh);
    XRegs<D, NS> xr;
    load_x<D, NS>(a.x, xr);
    const uint32_t S = a.slices;
    const uint32_t n_core = a.core_count * S;
    for (uint32_t i = blockIdx.x; i < n_core; i += gridDim.x) {
        const uint32_t unit = i / S, j = i % S;
        const Unit u = resolve(a, b, load_core(a, unit), D);
        if (!u.ok) {
            if (threadIdx.x == 0) raise_status(a, slot, kStatusBadDescriptor);
            return;
        }
        run_item<D, NS, false>(a, sh, slot, yacc, xr, u, unit, j, 0);
    }
}

// Split path, stage B: persistent ready-queue consumer (last block mirrors).
template <int D, int NS>
__global__ __launch_bounds__(kThreads, 2) void stage_b_kernel(MlpArgs a, Bounds b) {
    __shared__ Shared sh;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    const uint32_t W = gridDim.x - 1;
    if (blockIdx.x == W) {
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
        return;
    }
    init_shared(sh);
    XRegs<D, NS> xr;
    load_x<D, NS>(a.x, xr);
    consume_queue<D, NS, false>(a, sh, slot, launch_acc(a), xr, b, W, blockIdx.x, 0, 0);
}

// Split path, compact reduction (streaming_mlp.cu:80-84): converts every column's
// accumulator to y32 / y. 256 columns per block.
template <int D>
__global__ __launch_bounds__(kThreads) void reduce_kernel(MlpArgs a) {
    const int col = blockIdx.x * kThreads + threadIdx.x;
    const unsigned long long w = __hip_atomic_load(launch_acc(a) + col, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    write_output(a, col, w, (uint32_t)(w >> 52));
}

// Clears both ring slots and the accumulators (bind time, or after a failed enqueue).
__global__ void clear_sync_kernel(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns) {
    // `columns` covers both accumulator buffers
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x)
        st_agent(sync + i, 0u);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < columns; i += gridDim.x * blockDim.x)
        st_agent_u64(yacc + i, 0ull);
}

// ---------------------------------------------------------------------------------
// Host-side launch dispatch over the compiled (width, neurons-per-item) variants.
// ---------------------------------------------------------------------------------
namespace {

struct Variant {
    int width, ns;
    const void* fused;
    const void* stage_a;
    const void* stage_b;
    const void* reduce;
};

template <int D, int NS>
Variant make_variant() {
    return {D, NS, reinterpret_cast<const void*>(&fused_layer_kernel<D, NS>),
            reinterpret_cast<const void*>(&stage_a_kernel<D, NS>), reinterpret_cast<const void*>(&stage_b_kernel<D, NS>),
            reinterpret_cast<const void*>(&reduce_kernel<D>)};
}

#define LS_VARIANTS_FOR(D) make_variant<D, 1>(), make_variant<D, 2>(), make_variant<D, 4>(), make_variant<D, 8>()

const Variant* find_variant(int width, int ns) {
    static const Variant table[] = {LS_VARIANTS_FOR(256),  LS_VARIANTS_FOR(512),  LS_VARIANTS_FOR(1024),
                                    LS_VARIANTS_FOR(2048), LS_VARIANTS_FOR(4096), LS_VARIANTS_FOR(8192)};
    for (const Variant& v : table)
        if (v.width == width && v.ns == ns) return &v;
    return nullptr;
}

}  // namespace

bool variant_available(int width, int ns) { return find_variant(width, ns) != nullptr; }

hipError_t resident_workers(int width, int ns, int entry_point, int* per_cu) {
    const Variant* v = find_variant(width, ns);
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
    const Variant* v = find_variant(p.width, p.ns);
    if (!v) return hipErrorInvalidValue;
    MlpArgs a = args;
    Bounds b = bounds;
    void* kargs[] = {&a, &b};
    if (p.entry_point == kEntryFused)
        return hipLaunchKernel(v->fused, dim3(p.workers + 1), dim3(kThreads), kargs, 0, stream);
    hipError_t e = hipSuccess;
    const uint32_t core_items = a.core_count * a.slices;
    if (core_items) {
        const uint32_t grid = core_items < (uint32_t)p.workers ? core_items : (uint32_t)p.workers;
        e = hipLaunchKernel(v->stage_a, dim3(grid), dim3(kThreads), kargs, 0, stream);
        if (e != hipSuccess) return e;
    }
    e = hipLaunchKernel(v->stage_b, dim3(p.workers + 1), dim3(kThreads), kargs, 0, stream);
    if (e != hipSuccess) return e;
    void* rargs[] = {&a};
    return hipLaunchKernel(v->reduce, dim3(p.width / kThreads), dim3(kThreads), rargs, 0, stream);
}

hipError_t clear_sync(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns, hipStream_t stream) {
    uint32_t grid = (words + kThreads - 1) / kThreads;
    if (grid > 1024) grid = 1024;
    if (!grid) grid = 1;
    void* kargs[] = {&sync, &words, &yacc, &columns};
    return hipLaunchKernel(reinterpret_cast<const void*>(&clear_sync_kernel), dim3(grid), dim3(kThreads), kargs, 0,
                           stream);
}

}  // namespace lsamd
