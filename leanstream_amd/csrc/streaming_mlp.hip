// gfx950 kernels for LeanStream's streaming sparse INT4 MLP.
//
// Arithmetic (LeanStream kernels/streaming_mlp.cu:11-41, backends/triton/core.py:9-17):
//   w      = fp16( q * scale[c/128] ),  q = signed low-nibble-first INT4
//   gate   = sum_c w_gate(c) x(c)   up = sum_c w_up(c) x(c)          (fp32)
//   h      = fp16( fp16(silu(fp16(gate))) * fp16(up) )
//   y[c]   = fp16( sum over the U destination rows of sum_n h_n w_down(n, c) )  (fp32)
//
// Work decomposition (MI355X-specific). The units of a launch (descriptors, one group of
// G neurons each) are cut into wave-sized items of a few KB of weights:
//   - gate/up items: NPI neurons of one unit (about 8 KB of weights); one 64-lane wave
//     computes their gate and up rows and publishes h;
//   - down items: one 256-column tile (two scale blocks) of one unit over all G rows.
// All gate/up items come first, then the down items (unit-major). Wave w of the
// persistent grid takes items w, w + NW, w + 2 NW, ..., one in flight at a time; with
// two workgroups per CU (8 waves) nearly the whole layer is in flight at once at the
// Ministral-8B shape, and HBM delivers it front to back. A down item needs the h of its
// unit, produced by items about one round earlier, so it is normally ready by the time
// the down weights arrive. Waves of a workgroup never wait for each other on this path;
// a wave waits for h only after all of its own gate/up items.
//
// Exactness: dequantisation is exact (dequant8); products w*x are exact in fp32; only the
// fp32 summation order differs from the reference.
//
// Reduction: a down item's 128 column sums are added into packed fixed-point column
// accumulators (kAccOne in mlp_args.h). Integer addition is associative, so y does not
// depend on the order in which items finish: the output is bit-identical across consumer
// modes, publication orders and entry points. The U-th contribution of a column
// converts it to fp32 / fp16.
//
// Cross-workgroup data (h, accumulators, counters) uses agent-scope relaxed atomics,
// which compile to sc1 loads/stores that are coherent across the eight XCD L2s. An h
// word carries its launch tag in the same 64-bit word, so no fence orders it. No acquire
// or release fence is issued inside a spin loop (those expand to whole-L2 invalidate /
// write-back). Every wait is bounded by a wall-clock limit; on expiry the status word
// records a timeout and every worker leaves.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include "mlp_args.h"
#include "mlp_launch.h"

#include "mlp_device.h"

namespace lsamd {

// One persistent worker workgroup of a launch. Its waves walk their share of the resident
// (core) units' items, then their share of the queue's (waiting for each position to be
// published when the launch started before the queue was complete) or, with claim_batch
// > 0 on the progressive path, the items of the ready positions the workgroup claims,
// which its four waves share. Every range goes through the one call of
// process_items below, so the item loop exists once in the kernel's code (one copy per
// range kind would triple the code and raise the register count).
// Item walks of the persistent kernels: plain (one item in flight per wave, in registers),
// staged (64-neuron groups at batch 1: items staged through LDS slots), packed (groups of at
// most 32 neurons at batch 1: the plain walk with down items over packs of core units).
enum Walk : int { kWalkPlain = 0, kWalkStaged = 1, kWalkPacked = 2 };

// A worker's first loads, from the preloaded arguments only (the kernel then reads its
// argument block): its role, x (one row at batch 1) and, on the staged walk, the first
// descriptor batch of the resident range.
template <int D>
struct WorkerStart {
    WaveRole role;
    XPart<D> xp;
    Prefetched first;
};

template <int D, bool CORE, bool QUEUE, int NB, int WALK>
__device__ __forceinline__ void start_worker(const uint16_t* x, const ExecDesc* core, uint32_t core_count,
                                             uint32_t grid, uint32_t shape, u32x4* xl, WorkerStart<D>& st) {
    const uint32_t W = QUEUE ? grid - 1 : grid;
    // Roles by workgroup: the first gu_wgs workgroups take the gate/up items, the others
    // the down items (one workgroup alone takes both).
    const uint32_t gu_wgs = kSplitRoles && W >= 2 ? (W + 1) / 2 : 0;
    st.role = WaveRole{blockIdx.x * kWaves + wave_id(), W * kWaves, gu_wgs * kWaves};
    const uint32_t G = shape_group(shape), batch = shape_batch(shape);
    load_x<D>(x, NB == 1 ? 1u : batch, st.xp, xl);   // the NB = 1 kernels hold one row of x
    st.first = Prefetched{0, false};
    if constexpr (CORE) {
        if constexpr (WALK == kWalkStaged)
            prefetch_core_descs<D>(core, core_count, shape_tiles(shape) ? kDnCols : 0u, st.role, st.first);
        else
            prefetch_core_descs_plain<D, NB, WALK == kWalkPacked>(core, core_count, G, batch, st.role, st.first);
    }
}

template <int D, bool FUSED, bool CORE, bool QUEUE, int NB, int WALK>
__device__ __forceinline__ void worker(const MlpArgs& a, const Bounds& b, Shared& sh, u32x4* xl, u32x4* stage,
                                       uint32_t* slot, WorkerStart<D>& st) {
    constexpr bool STAGED = WALK == kWalkStaged;
    const WaveRole role = st.role;
    const uint32_t W = QUEUE ? a.grid - 1 : a.grid;
    const uint32_t wave = wave_id();
    unsigned long long* yacc = launch_acc(a);
    XPart<D>& xp = st.xp;
    Prefetched first = st.first;
    Epoch ep = {0, 0, 0, 0};
    Pending pd;
    pd.col = -1;
    pd.n = 0;
    const uint32_t early = (QUEUE || FUSED) && lane_id() == 0 ? ld_agent(slot + kSyncEpoch) : 0u;
    if (threadIdx.x == 0) sh.xcount = 0;   // waves count themselves in once their part of x is staged
    __syncthreads();
    bool ok = true;
    enum : uint32_t { kCore, kDecide, kDone };
    uint32_t phase = CORE ? kCore : kDecide;
    for (;;) {
        uint32_t u0 = 0, u1 = 0, e = early;
        WaveRole r = role;
        if (phase == kCore) {
            u1 = a.core_count;
            phase = kDecide;
        } else if (phase == kDecide) {
            stamp(a, kStampCoreDone);
            if (!QUEUE) break;
            ok = ok && await_epoch(a, slot, ep, early);
            stamp(a, kStampEpoch);
            // One decision for the whole workgroup (claiming synchronises its waves).
            if (lane_id() == 0) sh.wpath[wave] = ok && ep.total ? ep.path : 0u;
            __syncthreads();
            uint32_t path = sh.wpath[0];
            for (int w = 1; w < kWaves; ++w)
                if (sh.wpath[w] != path) path = 0;
            path = __builtin_amdgcn_readfirstlane(path);
            // All positions published before the launch (path 2), or published while it
            // runs (path 1): every wave walks its stripe of the queue's items, waiting for
            // each item's position as needed. Pair-claiming candidates (claim_batch > 0)
            // take the positions in the reference's ranges -- static ranges of descriptor
            // indices when all were ready (persistent.py:63-69), logged here by the worker
            // that owns them; claimed ready ranges otherwise (persistent.py:71-90), taken by
            // the queue mirror -- and deal every range's items to all waves the same way.
            if (path == 2 && a.claim_batch && threadIdx.x == 0)
                for (uint32_t first = blockIdx.x * a.claim_batch; first < ep.total; first += W * a.claim_batch)
                    log_claim(a, slot, first, min(a.claim_batch, ep.total - first), kClaimStatic);
            if (path == 2 || path == 1) {
                u0 = a.core_count;
                u1 = u0 + ep.total;
                phase = kDone;
            } else {
                break;
            }
        } else {
            break;
        }
        if (u1 > u0) {
            if constexpr (STAGED) {
                ok = process_items_staged<D, FUSED>(a, sh, stage, slot, b, yacc, xp, xl, ep, e, pd, u0, u1, r, first);
                first.valid = false;   // only the resident range's first batch is prefetched
            } else {
                ok = process_items<D, FUSED, NB, WALK == kWalkPacked>(a, sh, stage, slot, b, yacc, xp, xl, ep, e, pd,
                                                                      u0, u1, r, first);
                first.valid = false;
            }
        }
    }
    stage_x<D>(xp, NB == 1 ? 1u : a.batch, xl, &sh.xcount);
    if (QUEUE) stamp(a, kStampQueueDone);
    check_pending(a, pd, FUSED && ep.known && ep.ok ? column_rows<WALK == kWalkPacked>(a, ep.total) : 0u);
    if (a.stamps) {
        drain_vmem();
        stamp(a, kStampDrained);
    }
}

// Words of a ring slot a launch uses: the per-unit execution counters (a line per unit from
// kSyncUnits on) only with the optional execution counts. Clearing the rest cost a layer of
// 1434 two-neuron groups 4 us: its slot is 367 KB.
__device__ __forceinline__ uint32_t ring_words_used(const MlpArgs& a) {
    return a.executions ? a.slot_words : (a.slot_words < kSyncUnits ? a.slot_words : kSyncUnits);
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
    for (uint32_t i = t; i < ring_words_used(a); i += n) st_agent(other + i, 0u);
    unsigned long long* other_acc = a.yacc + (size_t)((a.seq + 1) & 1) * a.width * a.batch * kAccStride;
    for (uint32_t i = t; i < a.width * a.batch; i += n) st_agent_u64(other_acc + (size_t)i * kAccStride, 0ull);
}

// Completion proof of a fused launch (replaces a per-launch event). Every worker
// workgroup counts itself out once its memory operations are complete, with a
// non-returning atomic into the counter of its group (blk % 8, so no word takes more
// than an eighth of the increments), and leaves at once. The mirror workgroup, after
// mirroring the queue, polls the eight counters; when every worker is out it stores the
// launch sequence into the host-coherent completion word. All reads of the launch's
// weights and all writes of its outputs are complete by then. (One host store per launch:
// a sign-off per workgroup into host memory made every launch wait for hundreds of PCIe
// writes at its end.)
__device__ __forceinline__ void count_out(uint32_t* slot) {
    drain_vmem();      // this wave's loads have returned, its stores and atomics are acknowledged
    __syncthreads();   // every wave of the workgroup has drained
    if (threadIdx.x == 0)
        (void)__hip_atomic_fetch_add(slot + kSyncExitGroups + (blockIdx.x % 8u) * kLine, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void await_workers(const MlpArgs& a, uint32_t* slot, uint32_t workers,
                                              bool store_done = true) {
    const uint32_t lane = lane_id();
    const uint32_t want = lane < 8u ? (workers + 7u - lane) / 8u : 0u;   // workers b < W with b % 8 == lane
    Waiter wt(a.spin_limit);
    for (;;) {
        const uint32_t got = lane < 8u ? ld_agent(slot + kSyncExitGroups + lane * kLine) : 0u;
        if (__all(got >= want)) break;
        if (wt.expired()) {   // a worker cannot leave: report it, then complete anyway
            if (lane == 0) raise_status(a, slot, kStatusTimeout);
            break;
        }
        // about 0.45 us between rounds while any group is less than half out, then at once
        // (C1 10.28 -> 10.23 us)
        if (__any(lane < 8u && got * 2u < want))
            __builtin_amdgcn_s_sleep(16);
        else
            __builtin_amdgcn_s_sleep(1);
    }
    stamp(a, kStampMirrorDone);
    if (store_done && lane == 0) __hip_atomic_store(a.done, a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The layer's epilogue in the fused launch's last workgroup (256 threads), once every worker
// is out: epilogue_kernel's arithmetic on the same y -- each column's fp16 value formed from
// its accumulator word as the worker that completed it formed it (acc_value), read back at
// agent scope -- one batch row after the other. The inputs known before the launch (row 0's
// residual, the norm weight) are requested while the first wave still waits for the workers
// (epi_prefetch). The flags and the bell are released only when the launch raised no status
// bit and its queue carries no error (a launch whose queue was abandoned writes no rows: its
// columns are incomplete). Then the completion word.
template <int D>
struct EpiInputs {
    uint16_t res[D / kThreads];      // row 0's residual, columns t + 256 j
    uint16_t weight[D / kThreads];   // the norm weight, columns t + 256 j
};

template <int D>
__device__ __forceinline__ void epi_prefetch(const MlpArgs& a, EpiInputs<D>& in) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (uint32_t j = 0; j < D / kThreads; ++j) {
        in.res[j] = a.residual[t + kThreads * j];
        in.weight[j] = a.norm_weight ? a.norm_weight[t + kThreads * j] : (uint16_t)0;
    }
}

// `decision` (LDS, written by thread 0 before the workgroup's barrier): 0 when the launch
// left its queue, else 1 | total << 1 with the queue's total from the mirrored epoch word.
template <int D, bool PACKED>
__device__ __forceinline__ void fused_epilogue(const MlpArgs& a, float* lanes, uint32_t decision,
                                               const EpiInputs<D>& in) {
    constexpr uint32_t PER = D / kThreads;
    static_assert(kThreads == 256 && D % kThreads == 0, "256 threads, whole columns each");
    const uint32_t t = threadIdx.x;
    // the status and queue error words (host memory): their round trip overlaps the rows
    uint32_t status = 0, error = 0;
    if (t == 0) {
        status = ld_sys(a.status);
        error = ld_sys(&a.control->error);
    }
    const bool ok = decision & 1u;
    if (ok) {
        const uint32_t U = column_rows<PACKED>(a, decision >> 1);
        const unsigned long long* acc = launch_acc(a);
        for (uint32_t r = 0; r < a.batch; ++r) {
            const size_t base = (size_t)r * D;
            unsigned long long w[PER];
            uint16_t res[PER];
#pragma unroll
            for (uint32_t j = 0; j < PER; ++j) {
                w[j] = ld_agent_u64(reinterpret_cast<const uint64_t*>(acc) + (base + t + kThreads * j) * kAccStride);
                res[j] = r ? a.residual[base + t + kThreads * j] : in.res[j];
            }
            float sum = 0.f;
            uint16_t hid[PER];
#pragma unroll
            for (uint32_t j = 0; j < PER; ++j) {
                const uint16_t y = __builtin_bit_cast(uint16_t, (_Float16)acc_value(w[j], U));
                hid[j] = epi_hidden(res[j], y, sum);
                a.hidden[base + t + kThreads * j] = hid[j];
            }
            if (a.norm_weight) {
                const float inverse = epi_inverse(sum, lanes, D, a.norm_eps);
#pragma unroll
                for (uint32_t j = 0; j < PER; ++j)
                    a.norm_out[base + t + kThreads * j] = epi_norm(hid[j], inverse, in.weight[j]);
            }
        }
    }
    // this workgroup's stores are visible at system scope before the flags; without flags the
    // completion word orders after them as after a launch's outputs (acknowledged stores)
    if (a.hidden_flag || a.norm_flag || a.bell)
        __atomic_thread_fence(__ATOMIC_RELEASE);
    else
        drain_vmem();
    __syncthreads();
    if (t == 0) {
        if (ok && !status && !error) {
            // both flags follow the rows (the release above, then the barrier); the bell follows
            // the flags: one release between them instead of one per flag
            if (a.hidden_flag) __hip_atomic_store(a.hidden_flag, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (a.norm_flag) __hip_atomic_store(a.norm_flag, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (a.bell) (void)__hip_atomic_fetch_add(a.bell, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        __hip_atomic_store(a.done, a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Completion proof of the split launch sequence, at the end of its last kernel (the
// reduction): every workgroup counts itself out in two levels -- per group blk % 8, then
// the last of each group in kSyncExit -- and the very last one stores the sequence.
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


// ---------------------------------------------------------------------------------
// Kernels. Persistent launches have gridDim.x = workers + 1; the last block mirrors.
// ---------------------------------------------------------------------------------

// LDS of a persistent workgroup beyond Shared and x: the staged kernels' item slots
// (kWaves x 2), or the other kernels' per-wave re-deal rows of the down items.
template <bool STAGED, int NB>
struct StageArea {
    static constexpr int VECS = STAGED ? 2 * kWaves * kSlotStride : kWaves * kNonStagedWaveVecs<NB>;
};

// The arguments a persistent worker needs before its first loads (x, its descriptors,
// the weight arenas, its ring slot, the grid, the launch shape) lead the kernel's argument
// list as scalars, so they can be preloaded into SGPRs at wave start
// (-amdgpu-kernarg-preload-count); the blocks of the remaining arguments are read from
// the kernel-argument segment (late_params) once x and the first descriptors are in flight.
#define LS_HOT_PARAMS                                                                                     \
    const uint16_t *hot_x, const ExecDesc *hot_core, const uint8_t *hot_cache, const uint16_t *hot_scales, \
        uint32_t *slot, uint32_t hot_core_count, uint32_t hot_seq, uint32_t hot_grid, uint32_t hot_shape,     \
        MlpArgs args, Bounds b
__device__ __forceinline__ MlpArgs with_hot(const MlpArgs& args, const uint16_t* x, const ExecDesc* core,
                                            const uint8_t* cache, const uint16_t* scales, uint32_t core_count,
                                            uint32_t seq, uint32_t grid) {
    MlpArgs a = args;
    a.x = x;
    a.core = core;
    a.cache = cache;
    a.scales = scales;
    a.core_count = core_count;
    a.seq = seq;
    a.grid = grid;
    return a;
}

// The persistent kernels' argument segment: LS_HOT_PARAMS in order, each at its natural
// alignment (the code object's argument offsets: args at 56, b right after it).
struct PersistentParams {
    const uint16_t* x;
    const ExecDesc* core;
    const uint8_t* cache;
    const uint16_t* scales;
    uint32_t* slot;
    uint32_t core_count, seq, grid, shape;
    MlpArgs args;
    Bounds b;
};
static_assert(offsetof(PersistentParams, args) == 56 && offsetof(PersistentParams, b) == 56 + sizeof(MlpArgs),
              "argument segment layout of LS_HOT_PARAMS");

// The argument blocks, read where this is called. The compiler loads a kernel's arguments
// at its entry, and the ones it then keeps in vector lanes (more scalars than fit) make the
// wave wait for those loads there, before anything else is issued. Read through an address
// the compiler cannot see through, the blocks' loads follow the ones issued before this call.
template <class P>
__device__ __forceinline__ const P* late_params_as() {
#ifdef __HIP_DEVICE_COMPILE__
    uint64_t p = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
    asm volatile("" : "+s"(p));
    // a constant-address-space pointer: the loads through it stay scalar loads
    return (const P*)reinterpret_cast<const __attribute__((address_space(4))) P*>(p);
#else
    return nullptr;
#endif
}
__device__ __forceinline__ const PersistentParams* late_params() { return late_params_as<PersistentParams>(); }
// `slot` (this launch's ring slot, sync + (seq & 1) slot_words) is a parameter of its own.
#define LS_HOT_ARGS                                                                                   \
    with_hot(late_params()->args, hot_x, hot_core, hot_cache, hot_scales, hot_core_count, hot_seq, hot_grid)
#define LS_LATE_BOUNDS Bounds(late_params()->b)
#define LS_WORKER_START(CORE, QUEUE) \
    start_worker<D, CORE, QUEUE, NB, WALK>(hot_x, hot_core, hot_core_count, hot_grid, hot_shape, xl, st)

// Fused layer: resident (core) units, queue consumption and the compact reduction (the
// contribution completing a column writes it), one persistent launch.
template <int D, int NB, int WALK>
__global__ __launch_bounds__(kThreads, kWgPerCu) void fused_layer_kernel(LS_HOT_PARAMS) {
    static_assert(WALK == kWalkPlain || NB == 1, "the staged and packed walks serve batch 1");
    __shared__ Shared sh;
    __shared__ u32x4 xl[NB * XGeom<D>::N];
    __shared__ u32x4 stage[StageArea<WALK == kWalkStaged, NB>::VECS];
    if (blockIdx.x == hot_grid - 1) {
        const MlpArgs a = LS_HOT_ARGS;
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
        if (a.hidden) {   // the layer's epilogue, here once every worker is out
            EpiInputs<D> in;
            epi_prefetch<D>(a, in);
            uint32_t* decision = reinterpret_cast<uint32_t*>(stage);
            if (threadIdx.x < 64) {
                // the epoch word is final once the queue is mirrored; read while the workers finish
                const uint32_t word = threadIdx.x == 0 ? ld_agent(slot + kSyncEpoch) : 0u;
                await_workers(a, slot, a.grid - 1, false);
                if (threadIdx.x == 0) decision[0] = (word & 3u) == 1u ? 1u | (word >> 4) << 1 : 0u;
            }
            __syncthreads();
            fused_epilogue<D, WALK == kWalkPacked>(a, reinterpret_cast<float*>(stage), decision[0], in);
        } else if (threadIdx.x < 64) {
            await_workers(a, slot, a.grid - 1);
        }
    } else {
        WorkerStart<D> st;
        LS_WORKER_START(true, true);
        const MlpArgs a = LS_HOT_ARGS;
        stamp(a, kStampEntry);
        worker<D, true, true, true, NB, WALK>(a, LS_LATE_BOUNDS, sh, xl, stage, slot, st);
        stamp(a, kStampExit);
        count_out(slot);
    }
}

// Split path, stage A: resident (core) units only; no queue, no conversion.
template <int D, int NB, int WALK>
__global__ __launch_bounds__(kThreads, kWgPerCu) void stage_a_kernel(LS_HOT_PARAMS) {
    __shared__ Shared sh;
    __shared__ u32x4 xl[NB * XGeom<D>::N];
    __shared__ u32x4 stage[StageArea<WALK == kWalkStaged, NB>::VECS];
    WorkerStart<D> st;
    LS_WORKER_START(true, false);
    const MlpArgs a = LS_HOT_ARGS;
    worker<D, false, true, false, NB, WALK>(a, LS_LATE_BOUNDS, sh, xl, stage, slot, st);
}

// Split path, stage B: persistent ready-queue consumer (last block mirrors).
template <int D, int NB, int WALK>
__global__ __launch_bounds__(kThreads, kWgPerCu) void stage_b_kernel(LS_HOT_PARAMS) {
    __shared__ Shared sh;
    __shared__ u32x4 xl[NB * XGeom<D>::N];
    __shared__ u32x4 stage[StageArea<WALK == kWalkStaged, NB>::VECS];
    if (blockIdx.x == hot_grid - 1) {
        const MlpArgs a = LS_HOT_ARGS;
        const uint64_t pre = threadIdx.x == 0 ? ld_sys64(&a.control->total_count) : 0;
        run_mirror(a, slot, pre);
        return;
    }
    WorkerStart<D> st;
    LS_WORKER_START(false, true);
    const MlpArgs a = LS_HOT_ARGS;
    worker<D, false, false, true, NB, WALK>(a, LS_LATE_BOUNDS, sh, xl, stage, slot, st);
}

// Split path, compact reduction (streaming_mlp.cu:80-84): converts every column's
// accumulator to y32 / y. 256 columns per block.
template <int D>
__global__ __launch_bounds__(kThreads) void reduce_kernel(MlpArgs a) {
    const int col = blockIdx.x * kThreads + threadIdx.x;
    const unsigned long long w =
        __hip_atomic_load(launch_acc(a) + (size_t)col * kAccStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    write_output(a, col, w, (uint32_t)(w >> 52));
    finish_launch(a, a.sync + (a.seq & 1) * a.slot_words);   // last kernel of the split launch sequence
}

// Clears both ring slots, the accumulators and the tagged h rows (bind time, after a
// failed enqueue, or when the launch sequence wraps): afterwards no stored tag can match
// a sequence number the next launches use.
__global__ void clear_sync_kernel(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns,
                                  uint64_t* hbuf, uint32_t hwords) {
    // `columns` covers both accumulator buffers, padding included
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) st_agent(sync + i, 0u);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < columns; i += stride) st_agent_u64(yacc + i, 0ull);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hwords; i += stride)
        __hip_atomic_store(hbuf + i, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------
// Dense batched path (batch 5 .. 32, every group a resident core unit): matrix cores.
//
// Per batch row the arithmetic is the batch-1 path's: w = fp16(q * scale) exactly, fp32
// sums of exact products, fp16 roundings of g, u, silu and h, fp32 sum of h * w_down.
// The products run on v_mfma_f32_32x32x16_f16: the dequantised weights and h are fp16
// values by definition, and bf16 x converts to fp16 exactly (8 significant bits; only
// |x| < 2^-17 rounds, by less than 2^-25), so every product is exact in fp32 and only the
// summation order differs. The 32 MFMA rows are the batch rows (rows >= batch are zero).
//
// MFMA fragment layout (v_mfma_f32_32x32x16_f16, checked on gfx950): lane l holds
// A[row l % 32][k 8 (l / 32) + i] and B[k 8 (l / 32) + i][col l % 32], i < 8; result
// element i is C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]. Which k a slot stands for is
// free as long as A and B agree, so each lane feeds the MFMA from its own contiguous loads.
//
// Four launches: x conversion (bf16 -> paired fp16, once per layer), gate/up (h rows in
// fp16), down projection (fp32 partial rows per split of the units), reduction (fixed
// split order, then the completion word).
// ---------------------------------------------------------------------------------
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kDenseCols = 256;    // down-projection columns per workgroup: whole 128-byte weight lines
constexpr int kDenseDnWaves = kDenseCols / 32;   // 32 columns per wave
constexpr int kDensePitch = 72;    // fp16 per LDS row: 64 neurons + 8 (rows stay 16-byte aligned)
constexpr int kDenseGuWaves = 8;   // gate/up waves per workgroup, each reduces D / 8 columns
constexpr int kDensePrefetch = 6;  // units whose down-tile loads are in flight per workgroup (9 loads each)
constexpr int kDenseGuWindow = 3;  // gate/up steps (64 columns) whose weight loads a wave keeps in flight

__device__ __forceinline__ _Float16 bf16_to_f16(uint32_t bits) {
    return (_Float16)__builtin_bit_cast(float, bits << 16);
}

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Workgroup barrier ordering LDS traffic only. __syncthreads() is a release/acquire at
// workgroup scope over all memory, so it waits for every global load of the wave still
// in flight (s_waitcnt vmcnt(0)); the prefetched loads of later units must stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// x (bf16 [batch][D]) -> x16: fp16 MFMA A fragments in dequant8's pairing. Within each
// 8-column group the slots hold columns (0, 4, 1, 5, 2, 6, 3, 7), so one 16-byte piece
// is the A fragment matching a dequantised weight word. The pieces are stored in the
// order the gate/up waves load them: fragment f = 4 (c / 64) + (c % 32) / 8 holds, for
// lane l, row l % 32 and columns 64 (c / 64) + 32 (l / 32) + 8 ((c % 32) / 8) .. + 7 at
// byte 1024 f + 16 l, so every x load of a wave reads one contiguous kilobyte. Rows >=
// batch are zero. Once per layer, shared by every gate/up workgroup.
__device__ __forceinline__ uint32_t x16_piece(uint32_t row, uint32_t c) {   // 16-byte piece index
    const uint32_t f = 4 * (c / 64) + (c % 32) / 8, l = row + 32 * ((c % 64) / 32);
    return 64 * f + l;
}

// Its arguments are scalars preloaded into SGPRs: the load goes out at once.
__global__ __launch_bounds__(kThreads) void dense_x_kernel(const uint16_t* x, uint16_t* x16, uint32_t width,
                                                           uint32_t batch) {
    const uint32_t D = width, groups = D / 8;
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;   // row * groups + group
    const uint32_t row = idx / groups, grp = idx - row * groups;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < batch) v = *glb(reinterpret_cast<const u32x4*>(x + (size_t)row * D + 8 * grp));
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    h8 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = bf16_to_f16((w[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        o[2 * i + 1] = bf16_to_f16((w[(i + 4) >> 1] >> (16 * (i & 1))) & 0xffffu);
    }
    glb(reinterpret_cast<h8*>(x16))[x16_piece(row, 8 * grp)] = o;
}

// Gate/up of one 32-neuron half of one unit for all batch rows. Wave w reduces the
// eighth [w D/8, (w+1) D/8) of the input in NI steps of 64 columns; the eight partial
// tiles meet in LDS. Lane l (neuron 32 half + l % 32, row l % 32 of x) takes 32
// consecutive columns per step: 16 bytes of each weight row and 64 bytes of x16. Up to
// d = 4096 the kernel stays within 128 registers (four waves per SIMD: two workgroups per
// CU, so the whole layer's workgroups are resident at once) with the weights of
// kDenseGuWindow steps in flight per wave.
// The dense kernels' argument segments (each parameter at its natural alignment): the
// leading scalars are preloaded into SGPRs, the blocks are read late (late_params_as).
struct DenseGuParams {
    const ExecDesc* core;
    const uint16_t* x16;
    MlpArgs args;
    Bounds b;
};
static_assert(offsetof(DenseGuParams, args) == 16 && offsetof(DenseGuParams, b) == 16 + sizeof(MlpArgs),
              "argument segment layout of dense_gate_up_kernel");

// The unit's descriptor and the first x16 steps go out from the preloaded arguments; the
// argument blocks are read behind them.
template <int NI>
__global__ __launch_bounds__(64 * kDenseGuWaves, NI <= 8 ? 4 : 2) void dense_gate_up_kernel(
    const ExecDesc* hot_core, const uint16_t* hot_x16, MlpArgs args, Bounds b) {
    __shared__ float red[kDenseGuWaves / 2][2][16][64];   // 32 KB: two workgroups per CU fit
    constexpr uint32_t D = NI * 64 * kDenseGuWaves;
    constexpr uint32_t kq = D / kDenseGuWaves;
    const uint32_t unit = blockIdx.x >> 1, half = blockIdx.x & 1;
    const ExecDesc desc = hot_core[unit];
    const int lane = lane_id();
    const uint32_t w = wave_id();
    const uint32_t n = half * 32 + (lane & 31), hh = lane >> 5, row = lane & 31;
    // x16 of step t (four 16-byte fragments per lane, each wave-contiguous) is loaded two
    // steps ahead, from a ring of three; steps 0 and 1 go out before the weights. Loads
    // complete in issue order, so each step waits only for what it uses.
    const LS_GLOBAL u32x4* xf = glb(reinterpret_cast<const u32x4*>(hot_x16));
    u32x4 xq[3][4];
    auto issue_x = [&](int t, u32x4 (&dst)[4]) {
        const uint32_t k0 = w * kq + 64 * t + 32 * hh;
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[j] = xf[x16_piece(row, k0 + 8 * j)];
    };
    issue_x(0, xq[0]);
    if (NI > 1) issue_x(1, xq[1]);
    const MlpArgs a = late_params_as<DenseGuParams>()->args;
    const Bounds bd = late_params_as<DenseGuParams>()->b;
    const uint32_t G = a.group_size;
    const Unit u = resolve(a, bd, desc, (int)D);
    f32x16 cg = {}, cu = {};
    if (u.ok) {
        const uint8_t* wg = u.grp + (size_t)(n * 3) * (D / 2);
        const uint8_t* wu = wg + D / 2;
        const uint16_t* sg = u.sc + (size_t)(n * 3) * (D / 128);
        const uint16_t* su = sg + D / 128;
        // The weights of WIN steps are in flight: step t's pieces go out into the slot
        // step t - WIN has just been computed from.
        constexpr int WIN = NI < kDenseGuWindow ? NI : kDenseGuWindow;
        u32x4 qg[WIN], qu[WIN];
        auto issue_w = [&](int t) {
            const uint32_t k0 = w * kq + 64 * t + 32 * hh;
            qg[t % WIN] = ld_cached16(wg + k0 / 2);   // a row's 128-byte line serves four steps
            qu[t % WIN] = ld_cached16(wu + k0 / 2);
        };
#pragma unroll
        for (int t = 0; t < WIN; ++t) issue_w(t);
        // The wave's K range covers SB consecutive scale blocks of each row (step t uses
        // block t / 2): one 8-byte load per projection row where SB is a multiple of 4.
        constexpr int SB = NI >= 2 ? NI / 2 : 1;
        uint32_t sgv[SB], suv[SB];
        const uint32_t b0 = NI >= 2 ? w * SB : w / 2;
        if constexpr (SB % 4 == 0) {
#pragma unroll
            for (int i = 0; i < SB; i += 4) {
                const u32x2 gv = *reinterpret_cast<const u32x2*>(sg + b0 + i);
                const u32x2 uv = *reinterpret_cast<const u32x2*>(su + b0 + i);
                sgv[i] = gv.x & 0xffffu; sgv[i + 1] = gv.x >> 16; sgv[i + 2] = gv.y & 0xffffu; sgv[i + 3] = gv.y >> 16;
                suv[i] = uv.x & 0xffffu; suv[i + 1] = uv.x >> 16; suv[i + 2] = uv.y & 0xffffu; suv[i + 3] = uv.y >> 16;
            }
        } else {
#pragma unroll
            for (int i = 0; i < SB; ++i) {
                sgv[i] = sg[b0 + i];
                suv[i] = su[b0 + i];
            }
        }
        // keep every load above ahead of the first MFMA (the scheduler would otherwise
        // sink them next to their uses, leaving two or three in flight per wave)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NI; ++t) {
            if (t + 2 < NI) issue_x(t + 2, xq[(t + 2) % 3]);
            __builtin_amdgcn_sched_barrier(0);
            const int sb = NI >= 2 ? t / 2 : 0;   // constant after unrolling
            const h2 sg2 = {half_bits((uint16_t)sgv[sb]), half_bits((uint16_t)sgv[sb])};
            const h2 su2 = {half_bits((uint16_t)suv[sb]), half_bits((uint16_t)suv[sb])};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const h8 xa = __builtin_bit_cast(h8, xq[t % 3][j]);   // paired (dense_x_kernel)
                h2 wgv[4], wuv[4];
                dequant8(qg[t % WIN][j], sg2, wgv);   // (column 8 j + i, column 8 j + i + 4)
                dequant8(qu[t % WIN][j], su2, wuv);
                h8 bg, bu;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bg[2 * i] = wgv[i].x;
                    bg[2 * i + 1] = wgv[i].y;
                    bu[2 * i] = wuv[i].x;
                    bu[2 * i + 1] = wuv[i].y;
                }
                cg = mfma32(xa, bg, cg);
                cu = mfma32(xa, bu, cu);
            }
            if (t + WIN < NI) issue_w(t + WIN);
        }
    }
    // Fixed-order sum of the eight partial tiles: wave w + 4 into wave w, then waves 0..3.
    constexpr uint32_t HW = kDenseGuWaves / 2;
    if (w >= HW) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            red[w - HW][0][i][lane] = cg[i];
            red[w - HW][1][i][lane] = cu[i];
        }
    }
    __syncthreads();
    if (w < HW) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            red[w][0][i][lane] += cg[i];
            red[w][1][i][lane] += cu[i];
        }
    }
    __syncthreads();
    const uint32_t hstride = a.slot_capacity * G;
#pragma unroll
    for (int r = 0; r < 1024 / (64 * kDenseGuWaves); ++r) {
        const uint32_t e = threadIdx.x + 64 * kDenseGuWaves * r, i = e >> 6, l = e & 63;
        float gsum = 0.f, usum = 0.f;
#pragma unroll
        for (int v = 0; v < (int)HW; ++v) {   // fixed order: deterministic
            gsum += red[v][0][i][l];
            usum += red[v][1][i][l];
        }
        const uint32_t tk = 8 * (i >> 2) + 4 * (l >> 5) + (i & 3);
        if (u.ok && tk < a.batch) {
            const float g = round_half(gsum);
            const float up = round_half(usum);
            const float sl = round_half(g / (1.0f + __expf(-g)));
            a.h16[(size_t)tk * hstride + u.dest * G + half * 32 + (l & 31)] =
                __builtin_bit_cast(uint16_t, (_Float16)(sl * up));
        }
    }
    if (threadIdx.x == 0) {
        if (!u.ok) {
            __hip_atomic_fetch_or(a.status, kStatusBadDescriptor, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        } else if (half == 0 && a.executions) {
            __hip_atomic_fetch_add(a.executions + u.dest, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// One unit's share of a down-projection workgroup's loads. Thread t covers rows
// 4 (t / 32) .. + 3 and columns 8 (t % 32) .. + 7 of the unit's 64 x 256 weight tile: one
// 4-byte load per row (a wave's 32 lanes read a row's whole 128-byte line), that row's
// scale for the columns' block, and 8 bytes of the unit's h rows (batch row t / 16,
// neurons 4 (t % 16) ..).
struct DenseDnLoad {
    uint32_t q[4], sb[4];
    u32x2 hv;
    bool ok;
};

// Branch-free, so that the compiler can count the loads in flight and wait for exactly
// one unit's: a position past the split, and an invalid descriptor, issue the same loads
// at the first word of the h rows for every lane (one line per instruction instead of a
// unit's 8 KB tile again; the h rows are not written by this kernel), with ok = false.
// h rows >= batch are zero (cleared at bind).
__device__ __forceinline__ void dense_dn_issue_desc(const MlpArgs& a, const Bounds& b, ExecDesc d, bool in, uint32_t c0,
                                                    DenseDnLoad& L) {
    const uint32_t D = a.width, G = a.group_size, t = threadIdx.x;
    const uint32_t nq = t >> 5, o = t & 31, hr = t >> 4, hp = t & 15;
    const Unit u = resolve(a, b, d, (int)D);
    L.ok = in && u.ok;   // an invalid descriptor is reported by the gate/up kernel
    const uint8_t* grp = L.ok ? u.grp : reinterpret_cast<const uint8_t*>(a.h16);
    const uint16_t* sc = L.ok ? u.sc : a.h16;
    const uint32_t col = c0 + 8 * o;
    const uint32_t on = L.ok ? 1u : 0u;   // 0: every lane reads the h rows' first word
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t n = 4 * nq + r;
        L.q[r] = *reinterpret_cast<const uint32_t*>(grp + on * ((size_t)(n * 3 + 2) * (D / 2) + col / 2));
        L.sb[r] = sc[on * ((size_t)(n * 3 + 2) * (D / 128) + col / 128)];
    }
    L.hv = *reinterpret_cast<const u32x2*>(a.h16 + on * ((size_t)hr * a.slot_capacity * G + u.dest * G + 4 * hp));
}

__device__ __forceinline__ void dense_dn_issue(const MlpArgs& a, const Bounds& b, uint32_t un, uint32_t u0,
                                               uint32_t u1, uint32_t c0, DenseDnLoad& L) {
    const bool in = un < u1;
    dense_dn_issue_desc(a, b, a.core[in ? un : u0], in, c0, L);
}

// LDS position (in halves) of the 8-neuron granule gr of tile column col: rows of 64
// neurons (128 bytes, so every column starts on the same bank), granules XOR-swizzled by
// (col ^ col >> 3) & 7: eight consecutive columns (the MFMA's 16-byte reads) take eight
// different granule slots, and so do eight columns 8 apart (the 8-byte writes of one
// instruction). Swizzling by bits 3..5 alone left the reads of eight consecutive columns on
// one slot: a third more bank-conflict cycles in the down kernel (SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ uint32_t dn_tile_pos(uint32_t col, uint32_t gr) {
    return col * 64 + 8 * (gr ^ ((col ^ (col >> 3)) & 7));
}

// Down projection of 256 columns over one split of the units. Per unit the workgroup
// dequantises the 64 x 256 weight tile into LDS transposed (column-major, 8-neuron
// granules, so a lane's eight k slots are eight neurons of its column: one 16-byte LDS
// read) and stages the unit's h rows; wave w then runs four MFMAs for columns
// 32 w .. 32 w + 31. The loads of the next kDensePrefetch units are in flight while a
// unit is computed.
__global__ __launch_bounds__(64 * kDenseDnWaves) void dense_down_kernel(MlpArgs a, Bounds b) {
    __shared__ alignas(16) _Float16 wl[kDenseCols * 64];
    __shared__ alignas(16) _Float16 hl[32][kDensePitch];
    const uint32_t D = a.width;
    const uint32_t tiles = D / kDenseCols;
    // XCD-aware order: workgroup blk runs on XCD blk % 8; the tiles of a split go to one
    // XCD (kDenseSplits is a multiple of 8), so the split's h rows and down-scale lines
    // are fetched into that XCD's L2 once instead of once per XCD
    static_assert(kDenseSplits % 8 == 0, "two splits per XCD");
    const uint32_t xcd = blockIdx.x % 8u, j = blockIdx.x / 8u;
    const uint32_t split = xcd + 8u * (j / tiles), ct = j % tiles;
    const uint32_t c0 = ct * kDenseCols;
    const uint32_t per = (a.core_count + a.dsplits - 1) / a.dsplits;
    const uint32_t u0 = min(a.core_count, split * per), u1 = min(a.core_count, u0 + per);
    const uint32_t t = threadIdx.x;
    const int lane = lane_id();
    const uint32_t w = wave_id();
    const uint32_t nq = t >> 5, o = t & 31;    // weight tile: 4-row group, 8-column group
    const uint32_t hr = t >> 4, hp = t & 15;   // h tile: batch row, 4-neuron part
    f32x16 acc = {};
    DenseDnLoad buf[kDensePrefetch];
    if (u0 < u1) {
#pragma unroll
        for (int s = 0; s < kDensePrefetch; ++s) dense_dn_issue(a, b, u0 + s, u0, u1, c0, buf[s]);
        for (uint32_t base = u0; base < u1; base += kDensePrefetch) {
#pragma unroll
            for (int s = 0; s < kDensePrefetch; ++s) {
                if (buf[s].ok) {   // uniform across the workgroup
                    // dequantise the four rows (pairs (column k, column k + 4) per row)
                    h2 v[4][4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const h2 s2 = {half_bits((uint16_t)buf[s].sb[r]), half_bits((uint16_t)buf[s].sb[r])};
                        dequant8(buf[s].q[r], s2, v[r]);
                    }
                    lds_barrier();   // the previous unit's tiles are read
#pragma unroll
                    for (int c = 0; c < 8; ++c) {   // column 8 o + c: rows 4 nq .. 4 nq + 3
                        const int k = c & 3;
                        const bool hi = c >= 4;
                        const h2 r01 = {hi ? v[0][k].y : v[0][k].x, hi ? v[1][k].y : v[1][k].x};
                        const h2 r23 = {hi ? v[2][k].y : v[2][k].x, hi ? v[3][k].y : v[3][k].x};
                        const uint32_t col = 8 * o + c;
                        *reinterpret_cast<u32x2*>(wl + dn_tile_pos(col, nq >> 1) + 4 * (nq & 1)) =
                            u32x2{__builtin_bit_cast(uint32_t, r01), __builtin_bit_cast(uint32_t, r23)};
                    }
                    *reinterpret_cast<u32x2*>(&hl[hr][4 * hp]) = buf[s].hv;
                    lds_barrier();
                    const uint32_t col = 32 * w + (lane & 31);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t gr = 2 * j + (lane >> 5);
                        const h8 ha = *reinterpret_cast<const h8*>(&hl[lane & 31][8 * gr]);
                        const h8 wb = *reinterpret_cast<const h8*>(wl + dn_tile_pos(col, gr));
                        acc = mfma32(ha, wb, acc);
                    }
                }
                dense_dn_issue(a, b, base + kDensePrefetch + s, u0, u1, c0, buf[s]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t tk = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (tk < a.batch) a.dpart[((size_t)split * 32 + tk) * D + c0 + 32 * w + (lane & 31)] = acc[i];
    }
}

// Sum of the splits in a fixed order, fp16 rounding, completion word.
// The queue of a dense launch (batch 5 .. 32) is not consumed: every group of a dense layer
// is a resident core unit. Block 0 of the reduction waits for the layer epoch (bounded) and
// raises kStatusQueueUnconsumed if the layer published queue entries, whose groups the
// output then lacks.
__device__ __forceinline__ void check_dense_queue(const MlpArgs& a, uint32_t* slot) {
    Waiter wt(a.spin_limit);
    for (;;) {
        const uint64_t te = ld_sys64(&a.control->total_count);
        if ((uint32_t)(te >> 32) == a.epoch) {
            if ((uint32_t)te) raise_status(a, slot, kStatusQueueUnconsumed);
            return;
        }
        if (ld_sys(&a.control->error)) {
            raise_status(a, slot, kStatusQueueError);
            return;
        }
        if (wt.expired()) {
            raise_status(a, slot, kStatusTimeout);
            return;
        }
        __builtin_amdgcn_s_sleep(8);
    }
}

struct DenseReduceParams {
    const float* dpart;
    uint32_t width, batch, dsplits;
    MlpArgs args;
};
static_assert(offsetof(DenseReduceParams, args) == 24, "argument segment layout of dense_reduce_kernel");

// The column blocks' split loads go out from the preloaded arguments; the argument block is
// read behind them.
__global__ __launch_bounds__(kThreads) void dense_reduce_kernel(const float* hot_dpart, uint32_t hot_width,
                                                                uint32_t hot_batch, uint32_t hot_dsplits,
                                                                MlpArgs args) {
    // the launch's last block (the column blocks are counted from the preloaded arguments)
    if (blockIdx.x == (hot_batch * hot_width / 4 + kThreads - 1) / kThreads) {
        const MlpArgs a = late_params_as<DenseReduceParams>()->args;
        uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
        // The last block only clears the next launch's ring slot (its last user, the previous
        // launch, has finished: stream order) and checks the layer's queue (a read of host
        // memory), in parallel with the column blocks; this kernel runs in every dense
        // launch, with or without core units.
        uint32_t* other = a.sync + ((a.seq + 1) & 1) * a.slot_words;
        for (uint32_t i = threadIdx.x; i < ring_words_used(a); i += blockDim.x) st_agent(other + i, 0u);
        if (threadIdx.x == 0) check_dense_queue(a, slot);
        finish_launch(a, slot);
        return;
    }
    // four consecutive columns of one row per thread (width is a multiple of 256): every
    // split's 16-byte load in flight
    const uint32_t idx = 4 * (blockIdx.x * kThreads + threadIdx.x);   // row * D + column
    const uint32_t W = hot_width;
    const LS_GLOBAL float4* parts = glb(reinterpret_cast<const float4*>(hot_dpart));
    float4 v = {0.f, 0.f, 0.f, 0.f};
    const bool mine = idx < hot_batch * W;
    if (mine) {
        const uint32_t tk = idx / W, col = idx - tk * W;
        if (hot_dsplits == kDenseSplits) {
            float4 p[kDenseSplits];
#pragma unroll
            for (uint32_t s = 0; s < kDenseSplits; ++s) p[s] = parts[(((size_t)s * 32 + tk) * W + col) / 4];
#pragma unroll
            for (uint32_t s = 0; s < kDenseSplits; ++s) {
                v.x += p[s].x;
                v.y += p[s].y;
                v.z += p[s].z;
                v.w += p[s].w;
            }
        } else {
            for (uint32_t s = 0; s < hot_dsplits; ++s) {
                const float4 q = parts[(((size_t)s * 32 + tk) * W + col) / 4];
                v.x += q.x;
                v.y += q.y;
                v.z += q.z;
                v.w += q.w;
            }
        }
    }
    const MlpArgs a = late_params_as<DenseReduceParams>()->args;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    if (mine) {
        if (a.y32) *reinterpret_cast<float4*>(a.y32 + idx) = v;
        const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.x) |
                            (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.y) << 16;
        const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.z) |
                            (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v.w) << 16;
        *reinterpret_cast<u32x2*>(a.y + idx) = u32x2{lo, hi};
    }
    finish_launch(a, slot);
}

// ---------------------------------------------------------------------------------
// Host-side launch dispatch over the compiled (width, neurons-per-item) variants.
// ---------------------------------------------------------------------------------
namespace {

struct Variant {
    int width;
    // [0] batch 1, [1] batch 2 .. kMaxBatch, [2] batch 1 with 64-neuron groups (staged),
    // [3] batch 1 with groups of at most 32 neurons (packed down items)
    const void* fused[4];
    const void* stage_a[4];
    const void* stage_b[4];
    const void* reduce;
};

// Staged kernels exist only for the widths where they fit two workgroups per CU.
template <int D, template <int, int, int> class K>
const void* staged_kernel() {
    if constexpr (staged_width(D))
        return reinterpret_cast<const void*>(K<D, 1, kWalkStaged>::fn);
    else
        return nullptr;
}

template <int D, int NB, int WALK>
struct FusedK {
    static constexpr auto fn = &fused_layer_kernel<D, NB, WALK>;
};
template <int D, int NB, int WALK>
struct StageAK {
    static constexpr auto fn = &stage_a_kernel<D, NB, WALK>;
};
template <int D, int NB, int WALK>
struct StageBK {
    static constexpr auto fn = &stage_b_kernel<D, NB, WALK>;
};

template <int D, template <int, int, int> class K>
void fill_family(const void* (&out)[4]) {
    out[0] = reinterpret_cast<const void*>(K<D, 1, kWalkPlain>::fn);
    out[1] = reinterpret_cast<const void*>(K<D, kMaxBatch, kWalkPlain>::fn);
    out[2] = staged_kernel<D, K>();
    out[3] = reinterpret_cast<const void*>(K<D, 1, kWalkPacked>::fn);
}

template <int D>
Variant make_variant() {
    Variant v{};
    v.width = D;
    fill_family<D, FusedK>(v.fused);
    fill_family<D, StageAK>(v.stage_a);
    fill_family<D, StageBK>(v.stage_b);
    v.reduce = reinterpret_cast<const void*>(&reduce_kernel<D>);
    return v;
}

// Kernel family of a launch: 0 batch 1, 1 batch 2 .. kMaxBatch, 2 staged (batch 1,
// 64-neuron groups, widths where two workgroups' slots fit a CU's LDS), 3 packed (batch 1,
// groups of at most 32 neurons).
int family(int width, int batch, int group_size, int walk = 0) {
    if (batch > 1) return 1;
    if (walk == 1) return 0;   // the plain walk serves every batch-1 shape
    if (group_size == (int)kStagedGroup && staged_width(width)) return 2;
    return group_size <= (int)kDnRows / 2 ? 3 : 0;
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

hipError_t resident_workers(int width, int entry_point, int batch, int group_size, int* per_cu, int walk) {
    const Variant* v = find_variant(width);
    if (!v || batch < 1 || batch > (int)kMaxBatch) return hipErrorInvalidValue;
    const int nb = family(width, batch, group_size, walk);
    const void* k = entry_point == kEntryFused ? v->fused[nb] : v->stage_b[nb];
    int n = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kThreads, 0);
    if (e == hipSuccess && entry_point != kEntryFused) {
        int na = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&na, v->stage_a[nb], kThreads, 0);
        if (na < n) n = na;
    }
    *per_cu = n;
    return e;
}

hipError_t run_stage_hook(StageHook* hook, hipStream_t stream) {
    if (!hook) return hipSuccess;
    if (hook->arm) hook->rc = hook->arm(hook->context);
    return hook->b_done ? hipEventRecord(hook->b_done, stream) : hipSuccess;
}

hipError_t launch_layer(const LaunchPlan& p, const MlpArgs& args, const Bounds& bounds, hipStream_t stream,
                        StageHook* hook) {
    const Variant* v = find_variant(p.width);
    if (!v || p.workers < 1) return hipErrorInvalidValue;
    MlpArgs a = args;
    Bounds b = bounds;
    if (a.batch < 1 || a.batch > kMaxBatch) return hipErrorInvalidValue;
    const int nb = family(p.width, (int)a.batch, (int)a.group_size, p.walk);
    a.pack = nb == 3 ? kDnRows / a.group_size : 1u;   // units per down item (pack_units)
    // the persistent kernels' leading scalars (LS_HOT_PARAMS), then the argument blocks
    uint32_t grid = (uint32_t)p.workers + 1;
    uint32_t* slot = a.sync + (a.seq & 1) * a.slot_words;
    uint32_t shape = launch_shape(a.group_size, a.batch, a.dn_tile);
    void* kargs[] = {&a.x, &a.core, &a.cache, &a.scales, &slot, &a.core_count, &a.seq, &grid, &shape, &a, &b};
    if (p.entry_point == kEntryFused) {
        a.grid = grid;
        const hipError_t e = hipLaunchKernel(v->fused[nb], dim3(grid), dim3(kThreads), kargs, 0, stream);
        return e == hipSuccess ? run_stage_hook(hook, stream) : e;
    }
    hipError_t e = hipSuccess;
    if (a.core_count) {
        grid = (uint32_t)p.workers;   // stage A has no mirror workgroup
        a.grid = grid;
        e = hipLaunchKernel(v->stage_a[nb], dim3(grid), dim3(kThreads), kargs, 0, stream);
        if (e != hipSuccess) return e;
    }
    grid = (uint32_t)p.workers + 1;
    a.grid = grid;
    e = hipLaunchKernel(v->stage_b[nb], dim3(grid), dim3(kThreads), kargs, 0, stream);
    if (e == hipSuccess) e = run_stage_hook(hook, stream);
    if (e != hipSuccess) return e;
    void* rargs[] = {&a};
    return hipLaunchKernel(v->reduce, dim3(p.width * a.batch / kThreads), dim3(kThreads), rargs, 0, stream);
}

namespace {
const void* dense_gate_up_for(uint32_t width) {
    switch (width) {
        case 512: return reinterpret_cast<const void*>(&dense_gate_up_kernel<1>);
        case 1024: return reinterpret_cast<const void*>(&dense_gate_up_kernel<2>);
        case 2048: return reinterpret_cast<const void*>(&dense_gate_up_kernel<4>);
        case 4096: return reinterpret_cast<const void*>(&dense_gate_up_kernel<8>);
        case 8192: return reinterpret_cast<const void*>(&dense_gate_up_kernel<16>);
        default: return nullptr;
    }
}
}  // namespace

bool dense_available(int width) { return width > 0 && dense_gate_up_for((uint32_t)width) != nullptr; }

hipError_t launch_dense(const MlpArgs& args, const Bounds& bounds, hipStream_t stream) {
    MlpArgs a = args;
    Bounds b = bounds;
    const void* gate_up = dense_gate_up_for(a.width);
    if (a.group_size != 64 || !gate_up || a.batch <= kMaxBatch || a.batch > kMaxDenseBatch || !a.dsplits ||
        !a.h16 || !a.dpart || !a.x16)
        return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    if (a.core_count) {
        uint16_t* x16 = a.x16;
        void* xargs[] = {&a.x, &x16, &a.width, &a.batch};
        e = hipLaunchKernel(reinterpret_cast<const void*>(&dense_x_kernel), dim3(32 * a.width / 8 / kThreads),
                            dim3(kThreads), xargs, 0, stream);
        const uint16_t* cx16 = a.x16;
        void* gargs[] = {&a.core, &cx16, &a, &b};
        if (e == hipSuccess)
            e = hipLaunchKernel(gate_up, dim3(2 * a.core_count), dim3(64 * kDenseGuWaves), gargs, 0, stream);
        void* dargs[] = {&a, &b};
        if (e == hipSuccess)
            e = hipLaunchKernel(reinterpret_cast<const void*>(&dense_down_kernel),
                                dim3(a.width / kDenseCols * a.dsplits), dim3(64 * kDenseDnWaves), dargs, 0, stream);
    } else {
        a.dsplits = 0;   // nothing to sum: y = 0
    }
    if (e != hipSuccess) return e;
    // four columns per thread, plus one block for the ring slot and the queue check
    const float* dpart = a.dpart;
    void* rargs[] = {&dpart, &a.width, &a.batch, &a.dsplits, &a};
    return hipLaunchKernel(reinterpret_cast<const void*>(&dense_reduce_kernel),
                           dim3((a.batch * a.width / 4 + kThreads - 1) / kThreads + 1), dim3(kThreads), rargs, 0,
                           stream);
}

// ---------------------------------------------------------------------------------
// Epilogue: next-hidden publication (LeanStream backends/triton/reduction.py:17-28 with
// PUBLISH) and RMSNorm (examples/ministral/native/predictor_shared_input.cu:16-41), one
// workgroup per row after the layer's launch on the same stream, so every y word of the
// launch is visible to it. hidden = fp16(fp32 residual + fp32 y); RMSNorm: thread t sums
// hidden^2 over columns t, t + 256, ... in order, a halving tree over the 256 partial sums,
// inverse = 1 / sqrt(sum / width + eps) (IEEE square root and division), out =
// fp16(weight * fp16(hidden * inverse)). Products and sums are not contracted into fused
// multiply-adds, so the result is the oracle's bit for bit. The last row's workgroup to
// finish publishes the flags after a system-scope release: hidden_flag and norm_flag, then
// (released after them) bell += 1 -- unless the layer failed: its launch raised a status bit (a
// bounded wait expired, a descriptor or a value was rejected) or its queue carries an error
// (the runtime cancelled the layer; the launch left early). Then y is not the layer's output:
// the rows are written but nothing announces them.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void epilogue_kernel(EpilogueArgs e) {
    __shared__ float lanes[256];
    __shared__ uint32_t last;
    const uint32_t t = threadIdx.x, row = blockIdx.x;
    const uint16_t* y = e.y + (size_t)row * e.width;
    const uint16_t* res = e.residual + (size_t)row * e.width;
    uint16_t* hid = e.hidden + (size_t)row * e.width;
    float sum = 0.f;
    for (uint32_t i = t; i < e.width; i += 256) hid[i] = epi_hidden(res[i], y[i], sum);
    if (e.norm_weight) {
        const float inverse = epi_inverse(sum, lanes, e.width, e.eps);
        uint16_t* out = e.norm_out + (size_t)row * e.width;
        for (uint32_t i = t; i < e.width; i += 256) out[i] = epi_norm(hid[i], inverse, e.norm_weight[i]);
    }
    if (!e.hidden_flag && !e.norm_flag && !e.bell) return;
    // this workgroup's stores are visible at system scope before it counts itself in
    __atomic_thread_fence(__ATOMIC_RELEASE);
    __syncthreads();
    if (t == 0) {
        const uint32_t before = __hip_atomic_fetch_add(e.arrivals, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_SYSTEM);
        last = before == e.rows - 1;
        if (last) {
            __hip_atomic_store(e.arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            // the launch before this one on the stream has finished: its status bits are final
            if (__hip_atomic_load(e.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ||
                (e.queue_error && __hip_atomic_load(e.queue_error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)))
                return;
            // one release for both flags (every row acquired above), one between them and the bell
            __atomic_thread_fence(__ATOMIC_RELEASE);
            if (e.hidden_flag) __hip_atomic_store(e.hidden_flag, e.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (e.norm_flag) __hip_atomic_store(e.norm_flag, e.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (e.bell) (void)__hip_atomic_fetch_add(e.bell, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

hipError_t launch_epilogue(const EpilogueArgs& args, hipStream_t stream) {
    EpilogueArgs e = args;
    if (!e.y || !e.residual || !e.hidden || !e.rows || !e.width || (e.norm_weight && !e.norm_out) || !e.arrivals ||
        !e.status)
        return hipErrorInvalidValue;
    void* kargs[] = {&e};
    return hipLaunchKernel(reinterpret_cast<const void*>(&epilogue_kernel), dim3(e.rows), dim3(256), kargs, 0, stream);
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
