// gfx950 chain kernel: a sequence of sparse INT4 MLP layers in one persistent launch.
//
// Per layer the arithmetic and the work decomposition are those of the staged fused kernel
// (streaming_mlp.hip, batch 1, 64-neuron groups): gate/up items of two neurons and 256-column
// down tiles, staged through two LDS slots per wave, h handed over as tagged words, the down
// contributions accumulated in fixed point so the output does not depend on the order in
// which waves finish. What the chain adds:
//
//   - Layer i + 1's input is layer i's hidden state x_{i+1} = fp16(x_i + fp16(y_i)) (the
//     epilogue's publication, backends/triton/reduction.py:17-22, with the layer's own input
//     as the residual). The lane whose contribution completes column c writes y[c] and the
//     hidden word fp16 | tag << 16 of the next layer's input; a workgroup stages a layer's
//     input into LDS once every word of its quarter carries the tag of the previous layer's
//     sequence. No flag, counter or fence sits between the last column and the next layer.
//   - A wave's items form one stream over the layers: it keeps two items in its LDS slots and
//     issues item j + 2 as soon as item j is computed, whatever layer it belongs to, so the
//     weights of later layers stream while earlier layers finish (the input wait of
//     backends/triton/core.py:20-28, with the loads issued before the wait).
//   - Per-layer completion: every wave counts itself out of each layer once its stores are
//     acknowledged; the supervisor workgroup (the last block) stores each layer's sequence
//     into the host-coherent completion word and releases the layer's optional flag and
//     bell.
//   - The supervisor first mirrors the layer records from pinned host memory into a device
//     ring (one workgroup reads host memory); workers read records from the ring.
//
// Accumulator words reset themselves: the lane that completes a column stores 0, so the two
// accumulator buffers (by sequence parity) are clean for the layer two sequences on once its
// waves have counted out (a wave checks the supervisor's layer count before its first
// column addition of a layer).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "mlp_args.h"
#include "mlp_launch.h"
#include "mlp_device.h"

namespace lsamd {
namespace {

constexpr uint32_t kChainRing = 1024;   // records in the host and device rings (index seq % ring)

// 16-byte load at agent scope (sc1): words stored by other XCDs during this launch.
__device__ __forceinline__ u32x4 ld_agent16(const uint32_t* base, uint32_t byte_offset) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), (short)0, 0x7fffffff, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 16 /* sc1 */);
}

// 16-byte load at system scope (sc0 sc1): pinned host memory the host wrote before the launch.
__device__ __forceinline__ u32x4 ld_sys16(const uint32_t* base, uint32_t byte_offset) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), (short)0, 0x7fffffff, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_offset, 0, 17 /* sc0 sc1 */);
}

__device__ __forceinline__ void chain_stamp(const ChainArgs& c, uint32_t layer, uint32_t k) {
    if (c.stamps && lane_id() == 0)
        c.stamps[((size_t)layer * c.grid * kWaves + blockIdx.x * kWaves + wave_id()) * kStampSlots + k] = now_ticks();
}

// The fields of one layer record a wave works with (wave-uniform).
struct LayerView {
    const ExecDesc* core;
    const uint8_t* cache;
    const uint8_t* staging;
    const uint16_t* scales;
    const uint16_t* x;
    const uint16_t* residual;
    const uint16_t* norm_weight;
    uint16_t* y;
    float* y32;
    uint16_t* hidden;
    uint32_t core_count, cache_groups, staging_groups, physical_groups, seq, chained;
    float eps;
};

// Words j, j + 1 of lane-held record words as a 64-bit value. v_readlane returns a signed
// int: widen it as unsigned, or an address whose low word has bit 31 set is sign-extended
// into a non-canonical pointer.
__device__ __forceinline__ uint64_t lane_u64(uint32_t w, int j) {
    return (uint64_t)(uint32_t)__builtin_amdgcn_readlane(w, j) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(w, j + 1) << 32);
}

__device__ __forceinline__ const uint32_t* record_words(const ChainArgs& c, uint32_t i) {
    return reinterpret_cast<const uint32_t*>(c.recs + i % kChainRing);
}

// Waits until the supervisor has mirrored every record of the launch.
__device__ bool chain_wait_records(const ChainArgs& c, const MlpArgs& a) {
    uint32_t ok = 1;
    if (lane_id() == 0 && ld_agent(c.csync + kChainAvail) < c.count) {
        Waiter wt(c.spin_limit);
        while (ld_agent(c.csync + kChainAvail) < c.count) {
            if (wt.due()) {
                if (ld_agent(c.csync + kSyncAbort)) { ok = 0; break; }
                if (wt.over()) { raise_status(a, c.csync, kStatusTimeout); ok = 0; break; }
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    return wave_bcast(ok) != 0;
}

// Requests record i of the launch: word l in lane l (l < 32). The load is consumed later
// (record_view), so its latency hides behind other work.
__device__ __forceinline__ uint32_t record_load(const ChainArgs& c, uint32_t first, uint32_t i) {
    return lane_id() < (int)kChainRecWords && i < c.count ? ld_agent(record_words(c, first + i) + lane_id()) : 0u;
}

__device__ __forceinline__ LayerView record_view(uint32_t w) {
    auto word = [&](int j) -> uint32_t { return (uint32_t)__builtin_amdgcn_readlane(w, j); };
    LayerView v;
    v.core = reinterpret_cast<const ExecDesc*>(lane_u64(w, 0));
    v.cache = reinterpret_cast<const uint8_t*>(lane_u64(w, 2));
    v.staging = reinterpret_cast<const uint8_t*>(lane_u64(w, 4));
    v.scales = reinterpret_cast<const uint16_t*>(lane_u64(w, 6));
    v.x = reinterpret_cast<const uint16_t*>(lane_u64(w, 8));
    v.residual = reinterpret_cast<const uint16_t*>(lane_u64(w, 10));
    v.norm_weight = reinterpret_cast<const uint16_t*>(lane_u64(w, 12));
    v.y = reinterpret_cast<uint16_t*>(lane_u64(w, 14));
    v.y32 = reinterpret_cast<float*>(lane_u64(w, 16));
    v.hidden = reinterpret_cast<uint16_t*>(lane_u64(w, 18));
    v.core_count = word(24);
    v.cache_groups = word(25);
    v.staging_groups = word(26);
    v.physical_groups = word(27);
    v.seq = word(29);
    v.chained = word(30);
    v.eps = __uint_as_float(word(31));
    return v;
}

// Workgroup state of the chain kernel in LDS.
struct ChainShared {
    alignas(16) uint16_t hs[kWaves][kDnRows];   // a down item's h, per wave
    alignas(16) float partial[kThreads];        // RMSNorm: the sums of squares of the norm's 256 threads
    uint32_t xcount;  // the waves' staged parts of the input, kWaves per staged layer
    uint32_t pcount;  // the waves' sums written to `partial`, kWaves per normalised layer
    uint32_t pread;   // the waves done reading `partial`, kWaves per normalised layer
};

template <int D>
struct ChainGeom {
    static constexpr uint32_t T = D / kDnCols;                          // down tiles per unit
    static constexpr uint32_t IPU = kStagedGroup / GuGeom<D>::NPI;      // gate/up items per unit
};

template <int D>
__device__ __forceinline__ ItemList chain_items(const WaveRole& r, uint32_t units) {
    return make_staged_items(r, units * ChainGeom<D>::IPU, units * ChainGeom<D>::T);
}

// Whether any wave of workgroup `blk` has items in a layer of `units` units (only such
// workgroups stage the layer's input).
template <int D>
__device__ __forceinline__ bool chain_wg_items(uint32_t blk, uint32_t nw, uint32_t units) {
    for (uint32_t q = 0; q < (uint32_t)kWaves; ++q)
        if (chain_items<D>(WaveRole{blk * kWaves + q, nw, 0}, units).K) return true;
    return false;
}

// One staged item of the stream: where its pieces came from and what it computes.
struct ChainItem {
    const uint8_t* grp;
    const uint16_t* sc;
    uint64_t* hrow;
    uint32_t tile, gu;
    int n0;
};

// The issue side of a wave's item stream: the next item to load into a slot.
template <int D>
struct Issuer {
    uint32_t li;        // layer of the next item; == count: no item left
    uint32_t k, k0;     // next item in the wave's list of layer li; first item of the descriptor batch
    uint32_t word;      // descriptor words of items k0 .. k0 + kDescItems - 1 (lane 5 j + w)
    uint32_t rec;       // record words of layer li + 1, requested when the issuer entered layer li
    ItemList il;
    LayerView v;
};

// Descriptor words of items k0 .. k0 + kDescItems - 1 of the issuer's layer (lane 5 j + w).
template <int D>
__device__ __forceinline__ uint32_t issuer_descs(const Issuer<D>& is, uint32_t k0) {
    using Cg = ChainGeom<D>;
    const uint32_t lane = lane_id();
    const uint32_t cnt = min(is.il.K - k0, (uint32_t)kDescItems);
    if (lane >= 5 * cnt) return 0u;
    const uint32_t j = lane / 5, w = lane - 5 * j;
    const uint32_t u = item_unit(is.il.item(k0 + j), is.il.NG, Cg::IPU, Cg::T, 1u);
    return ld_agent(reinterpret_cast<const uint32_t*>(is.v.core) + 5 * u + w);
}

// Moves the issuer from layer li (whose record words are in is.rec for li > start) to the
// first layer >= li in which this wave has items, and requests that layer's first
// descriptors and the next layer's record without waiting for them.
template <int D>
__device__ void issuer_seek(const ChainArgs& c, const WaveRole& role, uint32_t first, Issuer<D>& is) {
    while (is.li < c.count) {
        is.v = record_view(is.rec);
        is.rec = record_load(c, first, is.li + 1);
        is.il = chain_items<D>(role, is.v.core_count);
        if (is.il.K) {
            is.k = 0;
            is.k0 = 0;
            is.word = issuer_descs<D>(is, 0);
            return;
        }
        ++is.li;
    }
}

// Issues the issuer's next item into slot sl (its LDS reads must be complete: they are, the
// wave waits for its LDS operations before the loads), then advances the issuer.
template <int D>
__device__ bool chain_issue(const ChainArgs& c, const MlpArgs& a, const WaveRole& role, uint32_t first,
                            Issuer<D>& is, u32x4* sl, ChainItem& m) {
    using Gm = GuGeom<D>;
    using Cg = ChainGeom<D>;
    const uint32_t lane = lane_id();
    if (is.k - is.k0 >= (uint32_t)kDescItems) {
        is.k0 = is.k;
        is.word = issuer_descs<D>(is, is.k0);
    }
    const uint32_t j = is.k - is.k0;
    ExecDesc d;
    d.physical_group = __builtin_amdgcn_readlane(is.word, 5 * j + 1);
    d.source_slot = __builtin_amdgcn_readlane(is.word, 5 * j + 2);
    d.dest_slot = __builtin_amdgcn_readlane(is.word, 5 * j + 3);
    const uint32_t kind = __builtin_amdgcn_readlane(is.word, 5 * j + 4);
    const bool staging = kind == (uint32_t)leanstream::runtime::SourceKind::Staging;
    const bool ok = kind <= 1u && d.source_slot < (staging ? is.v.staging_groups : is.v.cache_groups) &&
                    d.physical_group < is.v.physical_groups && d.dest_slot < c.slot_capacity;
    if (!ok) {
        if (lane == 0) raise_status(a, c.csync, kStatusBadDescriptor);
        return false;
    }
    constexpr size_t group_bytes = (size_t)kStagedGroup * 3 * D / 2;
    m.grp = (staging ? is.v.staging : is.v.cache) + (size_t)d.source_slot * group_bytes;
    m.sc = is.v.scales + (size_t)d.physical_group * kStagedGroup * 3 * (D / 128);
    m.hrow = c.hbuf + (size_t)d.dest_slot * kStagedGroup;
    wait_lds_reads();   // the slot's previous item is no longer being read
    if (is.k < is.il.KG) {
        const uint32_t i = is.il.item(is.k);
        m.gu = 1;
        m.n0 = (int)((i % Cg::IPU) * Gm::NPI);
        m.tile = 0;
        gu_stage<D>(m.grp, m.sc, m.n0, sl);
    } else {
        const uint32_t i = is.il.item(is.k) - is.il.NG;
        m.gu = 0;
        m.n0 = 0;
        m.tile = i % Cg::T;
        dn_stage_tile<D>(m.grp, m.sc, (int)m.tile, sl);
    }
    if (is.k == 0) chain_stamp(c, is.li, kChainStampIssue);
    if (++is.k == is.il.K) {
        ++is.li;
        issuer_seek<D>(c, role, first, is);
    }
    return true;
}

__device__ __forceinline__ uint32_t lds_count(const uint32_t* count) {
    return __hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits until the workgroup's input count reaches `want` (the layers staged so far). False on
// abort or timeout: a wave that left cannot hold the workgroup forever.
__device__ __forceinline__ bool chain_wait_count(const MlpArgs& a, uint32_t* slot, const uint32_t* count, uint32_t want) {
    if (lds_count(count) >= want) return true;
    Waiter wt(a.spin_limit);
    while (lds_count(count) < want) {
        if (wave_should_stop(a, slot, wt)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}

// Stages this wave's part of layer v's input into the workgroup's LDS (the paired layout of
// stage_x) and raises the input count; the four waves of the workgroup together stage it
// all. The parts follow the RMSNorm of the Ministral epilogue
// (examples/ministral/native/predictor_shared_input.cu:16-41), whose thread t of 256 sums the
// squares of columns t, t + 256, ... in that order: wave w takes threads 64 w .. 64 w + 63,
// lane l thread t = 64 w + l and its columns t + 256 m, so every thread's sum stays one lane's
// sequential sum. The first layer reads its input. A chained layer reads the previous
// sequence's hidden words, each until it carries that sequence's tag, and takes them as they
// are or (with a norm weight) their RMSNorm times the weight: the 256 sums meet in LDS, every
// wave forms the epilogue's halving tree and inverse = 1 / sqrt(sum / d + eps) from them, then
// fp16 of h * inverse, then the fp16 product with the weight. Bit for bit the epilogue's
// result: h is fp16, so h * h is exact in fp32 and fma(h, h, sum) rounds where sum + h * h
// does, and the fp16 product of two fp16 values is the exact product rounded once, as the
// epilogue's fp32 product rounded to fp16 is. `normed` counts the normalised layers staged so
// far, this one included.
//
// Overwriting the input area is safe once any word of the layer carries the new tag: a column
// of layer l completes only after every unit's down item for it, each after its unit's h, so
// every gate/up item of layer l -- the only readers of the area -- is done by then.
template <int D>
__device__ bool chain_stage_part(const ChainArgs& c, const MlpArgs& a, const LayerView& v, uint32_t normed, u32x4* xl,
                                 ChainShared& sh) {
#pragma clang fp contract(off)
    constexpr int Q = D / kThreads;   // columns per lane: t + 256 m
    const uint32_t l = lane_id(), t = 64u * wave_id() + l;
    uint32_t hv[Q];                   // fp16 bits of the lane's columns
    if (!v.chained) {
#pragma unroll
        for (int m = 0; m < Q; ++m) hv[m] = glb(v.x)[t + kThreads * m];
    } else {
        const uint32_t* words = c.xtag + (size_t)((v.seq - 1u) & 1u) * D;
        const uint32_t tag = chain_tag(v.seq - 1u);
        uint32_t wt[Q];   // read-only weights: plain loads, in flight while the words are polled
        if (v.norm_weight) {
#pragma unroll
            for (int m = 0; m < Q; ++m) wt[m] = glb(v.norm_weight)[t + kThreads * m];
        }
        uint32_t q[Q];
        bool have[Q];
#pragma unroll
        for (int m = 0; m < Q; ++m) have[m] = false;
        Waiter wtime(a.spin_limit);
        for (;;) {
#pragma unroll
            for (int m = 0; m < Q; ++m)
                if (!have[m]) q[m] = ld_agent(words + t + kThreads * m);
            bool all = true;
#pragma unroll
            for (int m = 0; m < Q; ++m) {
                have[m] = have[m] || (q[m] >> 16) == tag;
                all = all && have[m];
            }
            if (__all(all)) break;
            if (wave_should_stop(a, c.csync, wtime)) return false;
            // Every workgroup reads the whole row, so while most of it is missing (the previous
            // layer still running) each poll round is D * 4 bytes per workgroup from beyond
            // L2, competing with that layer's own traffic: at d = 4096 the wave sleeps about
            // 1 us between rounds then (C2 chain 14.23 -> 13.62 us per layer), and polls at
            // once when at most a quarter of its words are missing. At d = 1024 (a quarter of
            // the reads, a shorter layer) the longer sleep cost more than it saved.
            if constexpr (D > 1024) {
                uint32_t miss = 0;
#pragma unroll
                for (int m = 0; m < Q; ++m) miss += (uint32_t)__popcll(__ballot(!have[m]));
                if (miss * 4u > 64u * Q)
                    __builtin_amdgcn_s_sleep(40);
                else
                    __builtin_amdgcn_s_sleep(1);
            } else {
                __builtin_amdgcn_s_sleep(1);
            }
        }
        // the input is here: every wave of the workgroup waits for its staging, which now takes
        // the SIMD's issue slots ahead of the co-resident wave (the poll above did not)
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
        for (int m = 0; m < Q; ++m) hv[m] = q[m] & 0xFFFFu;
        if (v.norm_weight) {
            float sum = 0.f;   // thread t's sum of squares
#pragma unroll
            for (int m = 0; m < Q; ++m) {
                const float h = (float)half_bits((uint16_t)hv[m]);
                sum = __builtin_fmaf(h, h, sum);
            }
            // the sums of the previous normalised layer have been read by every wave
            if (!chain_wait_count(a, c.csync, &sh.pread, kWaves * (normed - 1))) return false;
            sh.partial[t] = sum;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's LDS store lands before its count
            if (l == 0) __hip_atomic_fetch_add(&sh.pcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (!chain_wait_count(a, c.csync, &sh.pcount, kWaves * normed)) return false;
            // halving tree: (p[l] + p[l + 128]) + (p[l + 64] + p[l + 192]), then strides 32 .. 1
            float s2 = (sh.partial[l] + sh.partial[l + 128]) + (sh.partial[l + 64] + sh.partial[l + 192]);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the reads above happen before the count below
            if (l == 0) __hip_atomic_fetch_add(&sh.pread, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
            for (int k = 32; k >= 1; k >>= 1) s2 = s2 + __shfl_xor(s2, k);
            const float total = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s2)));
            const float inverse = 1.0f / __builtin_sqrtf(total / (float)D + v.eps);
#pragma unroll
            for (int m = 0; m < Q; ++m) {
                float p = (float)half_bits((uint16_t)hv[m]) * inverse;
                asm volatile("" : "+v"(p));   // the fp32 product, then fp16 (as the epilogue rounds)
                const _Float16 n = (_Float16)p;
                hv[m] = __builtin_bit_cast(uint16_t, (_Float16)(half_bits((uint16_t)wt[m]) * n));
            }
        }
    }
    // Paired layout: piece p = column / 8 holds (8p + j, 8p + j + 4) in its word j, so column
    // 8p + k is half 2 (k & 3) + (k >> 2) of the piece's 16 bytes.
    uint16_t* xh = reinterpret_cast<uint16_t*>(xl);
#pragma unroll
    for (int m = 0; m < Q; ++m) {
        const uint32_t col = t + kThreads * m;
        xh[8 * x_position<D>(col >> 3) + 2 * (col & 3) + ((col >> 2) & 1)] = (uint16_t)hv[m];
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // the wave's LDS stores land before its count
    if (l == 0) __hip_atomic_fetch_add(&sh.xcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return true;
}

// Where a completed column goes, and where its residual came from.
struct ChainOut {
    uint16_t* y;
    float* y32;
    uint16_t* hidden;
    uint32_t* xout;                 // hidden words of the next layer
    unsigned long long* acc;        // the layer's accumulator buffer (reset by the completing lane)
    const uint32_t* prev;           // chained layer: the previous layer's hidden words (null: residual row)
    uint32_t tag;                   // tag of xout's words
    uint32_t prev_tag;              // tag of prev's words
};

// The words returned by a wave's last column additions and the residuals of those columns
// (read while the item's h was on its way), checked at the wave's next additions or the
// end of the layer.
struct ChainPending {
    unsigned long long v[4];
    uint32_t res[4];
    int col;   // < 0: nothing pending
};

// Column `col` is complete (its word holds `rows` contributions): y, y32, the hidden state
// fp16(residual + fp16(y)) (the epilogue's arithmetic) as the next layer's tagged word and in
// the optional hidden row, and the accumulator word back to zero.
__device__ __forceinline__ void chain_output(const ChainOut& o, int col, unsigned long long word, uint32_t rows,
                                             uint32_t res) {
#pragma clang fp contract(off)
    const long long sum = (long long)(word & kAccValueMask) - (long long)rows * kAccBias;
    const float v = (float)((double)sum * kAccInv);
    const _Float16 y16 = (_Float16)v;
    if (o.y32) glb(o.y32)[col] = v;
    glb(o.y)[col] = __builtin_bit_cast(uint16_t, y16);
    float ab = (float)half_bits((uint16_t)res) + (float)y16;
    asm volatile("" : "+v"(ab));   // an fp32 sum rounded to fp16 (no mixed-precision fused form)
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)ab);
    __hip_atomic_store(glb(o.xout) + col, (o.tag << 16) | h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // system scope: the layer's flag publishes the row to other agents
    if (o.hidden) __hip_atomic_store(glb(o.hidden) + col, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    st_agent_u64(o.acc + col, 0ull);
}

__device__ __forceinline__ void chain_check_pending(const ChainOut& o, ChainPending& pd, uint32_t U) {
    if (pd.col >= 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if ((uint32_t)(pd.v[i] >> 52) != U) continue;
            uint32_t r = pd.res[i];
            // a residual word read before its store (not expected: see chain_dn) is read again
            for (int t = 0; o.prev && (r >> 16) != o.prev_tag && t < (1 << 20); ++t) {
                __builtin_amdgcn_s_sleep(1);
                r = ld_agent(o.prev + pd.col + kTileColOff[i]);
            }
            chain_output(o, pd.col + kTileColOff[i], pd.v[i], U, r);
        }
    }
    pd.col = -1;
}

__device__ __forceinline__ void chain_add_columns(const MlpArgs& a, uint32_t* slot, const ChainOut& o, int col,
                                                  const float cs[4], const uint32_t res[4], uint32_t U,
                                                  ChainPending& pd) {
    unsigned long long n[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned long long t = acc_term(a, slot, cs[i]);
        n[i] = __hip_atomic_fetch_add(glb(o.acc) + (col + kTileColOff[i]), t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + t;
    }
    chain_check_pending(o, pd, U);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pd.v[i] = n[i];
        pd.res[i] = res[i];
    }
    pd.col = col;
}

// A gate/up item: once the layer's input is in LDS, its dot products group by group as its
// pieces land (AFTER: the next item's loads are in flight behind it), then h.
template <int D, int AFTER>
__device__ __forceinline__ void chain_gu_dots(const u32x4* sl, const u32x4* xl, const ChainItem& m, uint32_t seq) {
    using Gm = GuGeom<D>;
    float acc[1][Gm::RPL][2];
#pragma unroll
    for (int p = 0; p < Gm::RPL; ++p) acc[0][p][0] = acc[0][p][1] = 0.f;
    auto none = [] {};
    gu_dots_staged<D, decltype(none)&, AFTER>(sl, xl, acc, none);
    gu_finish<D, 1>(acc, m.hrow, kStagedGroup, m.n0, Gm::NPI, seq, 1u);
}

// Row pairs of a chained down tile dequantised before its h is in. A chained layer's tiles
// land long before their h (they are requested while the previous layer finishes), so at
// d = 1024 the whole tile is dequantised ahead (246 registers; 36-layer C1 chain 8.13 ->
// 7.88 us per layer); at d = 4096 two pairs, as in the single-layer kernels (four measured
// equal there: the layer's time is not in its post-h tile work).
template <int D>
constexpr int kChainDnPre = D <= 1024 ? 4 : kDnPre;

// A down tile: the residuals of the lane's four columns and the first look at h requested,
// part of the tile dequantised while they travel, then the dot products, the row-group
// tree, the re-deal through the slot and four column additions.
template <int D>
__device__ __forceinline__ bool chain_dn(const ChainArgs& c, const MlpArgs& a, ChainShared& sh, u32x4* sl,
                                         const ChainItem& m, const ChainOut& o, const LayerView& v, uint32_t U,
                                         ChainPending& pd) {
    const int lane = lane_id();
    const int col = (int)(m.tile * kDnCols) + dn_tile_column(lane);
    uint16_t* hs = sh.hs[wave_id()];
    DnItem it;
    it.h = ld_agent_u64(uniform_ptr(m.hrow) + lane);
    h2 pre[kChainDnPre<D> > 0 ? kChainDnPre<D> : 1][4][8];
    dn_dequant_tile<kChainDnPre<D>>(sl, pre);
    if (!wait_h_word(a, c.csync, m.hrow, 0, it.h)) return false;
    // The residual of a column: the previous layer's hidden word, or the first layer's
    // residual row. Requested once h is in: h of this layer exists only after the previous
    // layer's last column, so every hidden word of that layer has been stored (the tag is
    // checked again when the column completes). Used at completion, after the tile's work.
    uint32_t res[4];
    if (v.chained) {
#pragma unroll
        for (int i = 0; i < 4; ++i) res[i] = ld_agent(o.prev + col + kTileColOff[i]);
    } else {
        const LS_GLOBAL uint16_t* r = glb(v.residual ? v.residual : v.x);
#pragma unroll
        for (int i = 0; i < 4; ++i) res[i] = r[col + kTileColOff[i]];
    }
    hs[lane] = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float((uint32_t)it.h));   // exact: h is fp16
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    float acc[32], cs[4];
    dn_accumulate_tile_pre<kChainDnPre<D>>(sl, hs, pre, acc);
    dn_reduce(acc, cs);
    float* red = reinterpret_cast<float*>(sl);
    *reinterpret_cast<float4*>(red + 32 * (lane & 7) + 4 * (lane >> 3)) = float4{cs[0], cs[1], cs[2], cs[3]};
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int i = 0; i < 4; ++i) cs[i] = red[dn_tile_column(lane) + kTileColOff[i]];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    chain_add_columns(a, c.csync, o, col, cs, res, U, pd);
    return true;
}

// Counts this wave out of layer i (one count per wave and layer, in the layer's own
// counters: a wave may leave a later layer before an earlier one).
__device__ __forceinline__ void chain_count_out(const ChainArgs& c, uint32_t i) {
    if (lane_id() == 0)
        (void)__hip_atomic_fetch_add(glb(c.csync) + kChainExit + (i * 8u + blockIdx.x % 8u) * kLine, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until the supervisor has seen every wave out of `layers` layers of the launch.
__device__ bool chain_wait_layers(const ChainArgs& c, const MlpArgs& a, uint32_t layers) {
    uint32_t ok = 1;
    if (lane_id() == 0 && ld_agent(c.csync + kChainLayersDone) < layers) {
        Waiter wt(c.spin_limit);
        while (ld_agent(c.csync + kChainLayersDone) < layers) {
            if (wt.due()) {
                if (ld_agent(c.csync + kSyncAbort)) { ok = 0; break; }
                if (wt.over()) { raise_status(a, c.csync, kStatusTimeout); ok = 0; break; }
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    return wave_bcast(ok) != 0;
}

template <int D>
__device__ void chain_worker(const ChainArgs& c, uint32_t first, ChainShared& sh, u32x4* xl, u32x4* stage) {
    const uint32_t W = c.grid - 1;
    const uint32_t wave = wave_id();
    const WaveRole role{blockIdx.x * kWaves + wave, W * kWaves, 0};
    MlpArgs a{};
    a.status = c.status;
    a.spin_limit = c.spin_limit;
    // The wave's two slots: `cur` holds the item computed next, `nxt` the one behind it
    // (valid when issued > computed + 1). After an item is computed, the stream's item two
    // ahead goes into its slot and the two trade places (scalar moves; arrays indexed at run
    // time would live in scratch memory, whose accesses count in vmcnt).
    u32x4* sl_cur = stage + (2 * wave) * kSlotStride;
    u32x4* sl_nxt = sl_cur + kSlotStride;
    ChainItem cur{}, nxt{};
    if (threadIdx.x == 0) sh.xcount = sh.pcount = sh.pread = 0;
    __syncthreads();
    uint32_t issued = 0, computed = 0, staged = 0, normed = 0, out = 0;
    // `owed`: the layer this wave has finished but not yet counted out of. Its last stores
    // (the outputs of completed columns) went out before the wave's next item loads, so the
    // wait for the next item's data covers them; the count follows that wait instead of a
    // drain at the end of every layer.
    int owed = -1;
    Issuer<D> is;
    is.li = 0;
    bool ok = chain_wait_records(c, a);
    if (ok) {
        is.rec = record_load(c, first, 0);
        issuer_seek<D>(c, role, first, is);
    }
    if (ok && is.li < c.count) {
        ok = chain_issue<D>(c, a, role, first, is, sl_cur, cur);
        ++issued;
    }
    if (ok && is.li < c.count) {
        ok = chain_issue<D>(c, a, role, first, is, sl_nxt, nxt);
        ++issued;
    }
    uint32_t rec = ok ? record_load(c, first, 0) : 0u;   // the compute side's next record
    auto settle = [&]() {   // count out of the owed layer once its stores are known complete
        if (owed >= 0) {
            chain_count_out(c, (uint32_t)owed);
            ++out;
            owed = -1;
        }
    };
    for (uint32_t i = 0; ok && i < c.count; ++i) {
        const LayerView v = record_view(rec);
        rec = record_load(c, first, i + 1);
        const ItemList il = chain_items<D>(role, v.core_count);
        chain_stamp(c, i, kChainStampXWait);
        if (chain_wg_items<D>(blockIdx.x, role.nw, v.core_count)) {
            ++staged;
            if (v.chained && v.norm_weight) ++normed;
            ok = chain_stage_part<D>(c, a, v, normed, xl, sh);
            __builtin_amdgcn_s_setprio(0);
            if (!ok) break;
            chain_stamp(c, i, kChainStampXIn);
        }
        a.seq = v.seq;
        const ChainOut o{v.y, v.y32, v.hidden, c.xtag + (size_t)(v.seq & 1u) * D, c.yacc + (size_t)(v.seq & 1u) * D,
                         v.chained ? c.xtag + (size_t)((v.seq - 1u) & 1u) * D : nullptr, chain_tag(v.seq),
                         chain_tag(v.seq - 1u)};
        const uint32_t U = v.core_count;
        ChainPending pd;
        pd.col = -1;
        bool first_gu = true, first_dn = true;
        for (uint32_t k = 0; ok && k < il.K; ++k) {
            const bool behind = issued > computed + 1;   // the next item's loads are in flight behind this one
            if (cur.gu) {
                if (!(ok = chain_wait_count(a, c.csync, &sh.xcount, kWaves * staged))) break;
                if (behind) chain_gu_dots<D, kStageOps>(sl_cur, xl, cur, v.seq);
                else chain_gu_dots<D, 0>(sl_cur, xl, cur, v.seq);
                settle();
                if (first_gu) chain_stamp(c, i, kStampFirstDone);
                first_gu = false;
            } else {
                if (behind) wait_loads_but<kStageOps>();
                else wait_loads_but<0>();
                settle();
                if (first_dn) {
                    chain_stamp(c, i, kStampFirstData);
                    // the accumulator buffer was last used two layers earlier: clean once that
                    // layer's waves have all counted out (its completing lanes reset the words)
                    if (!(ok = i < 2 || chain_wait_layers(c, a, i - 1))) break;
                }
                if (!(ok = chain_dn<D>(c, a, sh, sl_cur, cur, o, v, U, pd))) break;
                if (first_dn) chain_stamp(c, i, kStampDnComputed);
                first_dn = false;
            }
            ++computed;
            if (k + 1 == il.K) {
                chain_check_pending(o, pd, U);
                chain_stamp(c, i, kStampDrained);
                owed = (int)i;
                if (issued == computed && is.li >= c.count) {   // no item follows: nothing to wait for later
                    drain_vmem();
                    settle();
                }
            }
            // the freed slot takes the stream's item two ahead, whatever layer it belongs to
            if (ok && issued < computed + 2 && is.li < c.count) {
                ok = chain_issue<D>(c, a, role, first, is, sl_cur, cur);
                ++issued;
            }
            u32x4* const t = sl_cur;
            sl_cur = sl_nxt;
            sl_nxt = t;
            const ChainItem ti = cur;
            cur = nxt;
            nxt = ti;
        }
        if (ok && !il.K) {
            if (owed >= 0) drain_vmem();
            settle();
            chain_count_out(c, i);
            ++out;
        }
    }
    // After a failure: out of every layer not yet counted, so the supervisor finishes. A wave
    // counts its layers in order (a finished layer is owed until the next count), so the
    // counted layers are always 0 .. out - 1.
    drain_vmem();
    settle();
    for (uint32_t i = out; i < c.count; ++i) chain_count_out(c, i);
}

// The supervisor (last workgroup): mirrors the records, then per layer waits until every
// wave has counted out, stores the layer's sequence into the completion word, releases the
// layer's flag and bell, and advances the layer count workers check before reusing an
// accumulator buffer. At the end it zeroes the synchronisation block for the next launch.
__device__ void chain_supervisor(const ChainArgs& c, uint32_t first) {
    if (threadIdx.x >= 64) return;
    const uint32_t lane = lane_id();
    MlpArgs a{};
    a.status = c.status;
    a.spin_limit = c.spin_limit;
    // 16-byte pieces, every load of a batch in flight before the stores (one PCIe round trip
    // per 128 records)
    constexpr uint32_t kPieces = kChainRecWords / 4, kPer = 16;
    for (uint32_t base = 0; base < c.count * kPieces; base += 64 * kPer) {
        u32x4 v[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t p = base + lane + 64 * j;
            if (p < c.count * kPieces)
                v[j] = ld_sys16(reinterpret_cast<const uint32_t*>(c.host_recs + (first + p / kPieces) % kChainRing),
                                16 * (p % kPieces));
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t p = base + lane + 64 * j;
            if (p < c.count * kPieces) {
                uint32_t* d = reinterpret_cast<uint32_t*>(c.recs + (first + p / kPieces) % kChainRing) + 4 * (p % kPieces);
                st_agent(d + 0, v[j].x);
                st_agent(d + 1, v[j].y);
                st_agent(d + 2, v[j].z);
                st_agent(d + 3, v[j].w);
            }
        }
    }
    drain_vmem();
    if (lane == 0) st_agent(c.csync + kChainAvail, c.count);
    const uint32_t W = c.grid - 1;
    const uint32_t want = lane < 8u ? (uint32_t)kWaves * ((W + 7u - lane) / 8u) : 0u;
    bool failed = false;
    for (uint32_t i = 0; i < c.count; ++i) {
        if (!failed) {
            Waiter wt(c.spin_limit);
            for (;;) {
                const uint32_t got = lane < 8u ? ld_agent(c.csync + kChainExit + (i * 8u + lane) * kLine) : 0u;
                if (__all(got >= want)) break;
                if (wt.expired()) {   // a wave cannot leave: report it, then complete anyway
                    if (lane == 0) raise_status(a, c.csync, kStatusTimeout);
                    failed = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        const uint32_t* rw = record_words(c, first + i);
        const uint32_t w = lane < kChainRecWords ? ld_agent(rw + lane) : 0u;
        const uint32_t seq = (uint32_t)__builtin_amdgcn_readlane(w, 29);
        const uint32_t epoch = (uint32_t)__builtin_amdgcn_readlane(w, 28);
        uint32_t* flag = reinterpret_cast<uint32_t*>(lane_u64(w, 20));
        uint32_t* bell = reinterpret_cast<uint32_t*>(lane_u64(w, 22));
        chain_stamp(c, i, kChainStampDone);
        if (lane == 0) {
            // a layer that raised a status bit produced no valid output: its flag and bell stay
            const bool clean = !failed && __hip_atomic_load(glb(c.status), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 0;
            if (clean && flag) __hip_atomic_store(glb(flag), epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            if (clean && bell) (void)__hip_atomic_fetch_add(glb(bell), 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            st_agent(c.csync + kChainLayersDone, i + 1);
            __hip_atomic_store(glb(c.done), seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (failed) return;   // waves may still be running: the host clears the block before the next launch
    for (uint32_t w = lane; w < kChainExit; w += 64) st_agent(c.csync + w, 0u);
    for (uint32_t w = lane; w < c.count * 8u; w += 64) st_agent(c.csync + kChainExit + w * kLine, 0u);
}

template <int D>
__global__ __launch_bounds__(kThreads, kWgPerCu) void chain_kernel(ChainArgs c, uint32_t first) {
    __shared__ ChainShared sh;
    __shared__ u32x4 xl[XGeom<D>::N];
    __shared__ u32x4 stage[2 * kWaves * kSlotStride];
    if (blockIdx.x == c.grid - 1) {
        chain_supervisor(c, first);
        return;
    }
    chain_worker<D>(c, first, sh, xl, stage);
}

template <int D>
const void* chain_kernel_for() {
    return reinterpret_cast<const void*>(&chain_kernel<D>);
}

const void* chain_variant(int width) {
    switch (width) {
        case 1024: return chain_kernel_for<1024>();
        case 4096: return chain_kernel_for<4096>();
        default: return nullptr;
    }
}

}  // namespace

bool chain_available(int width) { return chain_variant(width) != nullptr; }
uint32_t chain_ring() { return kChainRing; }

hipError_t chain_resident(int width, int* per_cu) {
    const void* k = chain_variant(width);
    if (!k) return hipErrorInvalidValue;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k, kThreads, 0);
}

hipError_t launch_chain(const ChainArgs& args, uint32_t first, hipStream_t stream) {
    const void* k = chain_variant((int)args.width);
    if (!k || args.grid < 2 || !args.count || args.count > kChainRing) return hipErrorInvalidValue;
    ChainArgs c = args;
    void* kargs[] = {&c, &first};
    return hipLaunchKernel(k, dim3(c.grid), dim3(kThreads), kargs, 0, stream);
}

}  // namespace lsamd
