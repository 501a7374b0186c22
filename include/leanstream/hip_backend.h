// MI355X (gfx950) compute backend for the streaming sparse INT4 MLP.
//
// Replaces the CUDA reference enqueue (LeanStream kernels/streaming_mlp.cu:85-93,
// streaming_mlp_candidates.cu:3-11) and the native Triton pre-enqueue
// (backends/triton/enqueue.cpp:26-46, include/leanstream/triton_cuda.h:21-47) behind
// the unchanged ComputeBackend contract (include/leanstream/runtime.h:10-22).
//
// Caller owns every data buffer. bind() is the cold path (validation, occupancy
// query, small device sync state); enqueue() performs no allocation, compilation,
// profiling, device query or synchronisation: it selects a candidate in O(1) and
// launches pre-specialised kernels on the caller's HIP stream.
#pragma once
#include "kernel_selector.h"
#include "runtime.h"

namespace leanstream::runtime {

// CDNA4 candidate catalog. `workers` = persistent workgroups (256 threads each),
// clamped to the co-resident count minus one for the queue-mirror workgroup
// (kAllResident asks for exactly that; the selector rejects 0 workers); every worker
// takes a share of both the gate/up and the down-projection work; entry_point 0 = one
// fused launch (core + ready queue + compact reduction), entry_point 1 = split launches
// (stage A -> stage B -> reduction kernel). group_batch selects how a launch consumes
// positions: 0 = every wave takes its fixed stripe of the queue's items and waits for
// each item's position to be published (a newly ready group is computed by many waves at
// once); n > 0 = the positions are taken in the reference's ranges of n (the ready pairs of
// backends/triton/persistent.py:59-90 for n = 2) -- static descriptor-index ranges when all
// were ready at launch, [head, min(head + n, ready)) claimed in publication order by the
// queue mirror otherwise, every range logged -- and every range's items are dealt to all
// waves as with n = 0. The tile axis of the grid
// (docs/kernel_selection.md:13-19, kernel_selector.h KernelCandidate): unroll = items in
// flight per wave at batch 1 -- 0 the shape's own walk (two, through LDS slots, for
// 64-neuron groups at d <= 4096), 1 the plain walk (one, in registers); tile_size = the
// staged walk's down-item width -- 0 its own choice (64-column quarters when every item
// gets a wave, d <= 2048), 256 whole tiles. A candidate whose axis a shape lacks launches
// as the default does.
inline constexpr uint32_t kAllResident = 1u << 16;
inline constexpr KernelCandidate kHipCandidates[] = {
    {0, 256, "hip_fused_w256", 0, 0, 0, 0, 0},
    {1, kAllResident, "hip_fused_resident", 0, 0, 0, 0, 0},
    {2, 1024, "hip_fused_w1024", 0, 0, 0, 0, 0},
    {3, 256, "hip_split_w256", 0, 0, 0, 0, 1},
    {4, kAllResident, "hip_split_resident", 0, 0, 0, 0, 1},
    {5, kAllResident, "hip_fused_resident_pairs", 0, 0, 0, 2, 0},
    {6, kAllResident, "hip_fused_resident_plain", 0, 0, 1, 0, 0},
    {7, kAllResident, "hip_fused_resident_tiles", 0, 256, 0, 0, 0},
};
inline constexpr uint32_t kHipCandidateCount = 8;
// The default consumes the queue in the reference's ready pairs (persistent.py:59-90): static
// descriptor-index pairs when every position was ready, claimed [head, min(head + 2, ready))
// ranges otherwise, each range's items dealt to every wave.
inline constexpr KernelCandidate kHipDefault = kHipCandidates[5];
inline KernelSelector hip_selector(KernelDecisionTable offline_table = {}) noexcept {
    return KernelSelector(offline_table, {kHipCandidates, kHipCandidateCount}, kHipDefault);
}

// Geometry and caller-owned device buffers of one layer family (same shapes for every
// layer the backend serves). Pointers are device addresses; hidden may be null, in
// which case bind() allocates it (cold path).
struct HipLayerBuffers {
    uint32_t width = 0;            // d, multiple of 256 (256..8192)
    uint32_t group_size = 0;       // G neurons per group
    uint32_t batch = 1;            // tokens per call: 1 .. 4, or 5 .. 32 for the dense matrix-core path
                                   // (group_size 64, core descriptors only, x bf16 [batch][d])
    uint32_t slot_capacity = 0;    // destination rows (>= core + queue capacity)
    uint32_t cache_groups = 0;     // slots in the cache arena
    uint32_t staging_groups = 0;   // slots in the staging arena
    uint32_t physical_groups = 0;  // scale rows / G
    uint32_t queue_capacity = 0;   // largest DeviceExecQueue::capacity used
    const void* cache = nullptr;   // packed groups [cache_groups][G][3][d/2]
    const void* staging = nullptr; // packed groups [staging_groups][G][3][d/2]
    const void* scales = nullptr;  // fp16 [physical_groups*G][3][d/128]
    void* hidden = nullptr;        // u64 [slot_capacity][batch][G]: fp32 bits of h | launch sequence << 32
    void* partial = nullptr;       // reserved, unused: the reduction accumulates in backend-owned fixed point
    void* y32 = nullptr;           // optional fp32 [d] pre-rounding output
    uint32_t* executions = nullptr;     // optional per-destination execution counts
    uint64_t* first_compute = nullptr;  // optional per-destination start stamps
    uint32_t* claim_log = nullptr;      // optional claim log: 4 words per range a workgroup takes
                                        // ({first, count, ready at claim or ~0u, worker}), in the order
                                        // taken; holds queue_capacity ranges
    uint64_t* stamps = nullptr;         // optional per-worker phase stamps [max workers][32]
};

// Optional layer epilogue, run after every enqueue on the same stream (no LeanStream
// C++ counterpart; the Triton reduction's PUBLISH path, backends/triton/reduction.py:17-28,
// and the Ministral RMSNorm, examples/ministral/native/predictor_shared_input.cu:16-41):
// hidden = fp16(fp32 residual + fp32 y) per row, then optionally RMSNorm(hidden) * weight,
// then the flags (system-scope release stores of the enqueue's epoch) and the bell -- withheld
// for a failed layer (a status bit set, or the queue's error word). A fused launch computes it
// in its own last workgroup once every worker is out (its completion word follows); the split
// entry point and the dense path launch it as a kernel after the layer.
// Device pointers, [batch][width] rows; the flags may be host-coherent words.
struct HipEpilogue {
    const void* residual = nullptr;     // fp16 [batch][width]
    void* hidden = nullptr;             // fp16 [batch][width]
    uint32_t* hidden_flag = nullptr;    // optional: epoch once every row of hidden is written
    const void* norm_weight = nullptr;  // optional fp16 [width]
    void* norm_output = nullptr;        // fp16 [batch][width], with norm_weight
    uint32_t* norm_flag = nullptr;      // optional (with norm_weight): epoch once norm_output is written
    uint32_t* bell = nullptr;           // optional: += 1 after the flags
    float norm_eps = 0.f;               // 0 .. 1
};

// One layer of a chain (HipBackend::enqueue_chain): a sequence of layers computed by one
// persistent launch. Layer i's hidden state fp16(residual_i + fp16(y_i)) -- the epilogue's
// publication (backends/triton/reduction.py:17-22) -- is handed over inside the grid: it is
// layer i + 1's residual, and its input either as it is or as RMSNorm(hidden) * norm_weight
// (the Ministral epilogue, examples/ministral/native/predictor_shared_input.cu:16-41). The
// weights of later layers stream while earlier layers finish (no LeanStream C++
// counterpart: the reference submits future layers ahead and gates each on an input-ready
// epoch, docs/architecture.md:9, backends/triton/core.py:20-28). Device pointers; batch 1.
struct HipChainLayer {
    const ExecDesc* core = nullptr;     // device-visible core descriptors (resident groups)
    const void* cache = nullptr;        // packed groups [cache_groups][64][3][d/2]
    const void* staging = nullptr;      // optional packed groups [staging_groups][64][3][d/2]
    const void* scales = nullptr;       // fp16 [physical_groups*64][3][d/128]
    const void* input = nullptr;        // first layer: fp16 [d]; every later layer: nullptr
    const void* residual = nullptr;     // first layer: optional fp16 [d] (nullptr: the input); later: nullptr
    const void* norm_weight = nullptr;  // later layers: optional fp16 [d]: input = RMSNorm(previous hidden) * it
    void* output = nullptr;             // fp16 y [d]
    float* output32 = nullptr;          // optional fp32 y [d] (pre-rounding)
    void* hidden = nullptr;             // optional fp16 [d]: fp16(residual + y)
    uint32_t* hidden_flag = nullptr;    // optional: epoch (system release) once the layer is done
    uint32_t* bell = nullptr;           // optional: += 1 after the flag
    uint32_t core_count = 0;
    uint32_t cache_groups = 0;
    uint32_t staging_groups = 0;
    uint32_t physical_groups = 0;
    uint32_t epoch = 0;
    float norm_eps = 0.f;               // 0 .. 1
};

class HipBackend {
public:
    explicit HipBackend(KernelDecisionTable table = {});
    ~HipBackend();
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    int bind(const HipLayerBuffers&);
    // One layer epoch: A/B/reduction work on `stream` (a hipStream_t).
    int enqueue(KernelRuntimeState, const void* input, void* output, void* stream, Span<ExecDesc> core,
                DeviceExecQueue, uint32_t epoch, ConsumerMode);
    ComputeBackend view();
    // Installs (or, with nullptr, removes) the epilogue of every later enqueue; after bind.
    int set_epilogue(const HipEpilogue*);
    // `count` layers in one persistent launch on `stream` (a hipStream_t); layer i gets
    // sequence last_seq() - count + 1 + i, and the completion word takes each layer's
    // sequence as it finishes (complete() covers the last). ENOTSUP for a geometry without
    // chain kernels (batch 1, 64-neuron groups, d 1024 or 4096), EBUSY while more than the
    // record ring's worth of layers is in flight. No allocation, no synchronisation.
    int enqueue_chain(const HipChainLayer* layers, uint32_t count, void* stream);
    // Diagnostics: per-layer phase stamps of chains of at most `layers` layers
    // ([layers][(chain_workers() + 1) * 4][32] u64, 100 MHz clock); nullptr removes them.
    int set_chain_stamps(uint64_t* stamps, uint32_t layers);
    uint32_t chain_workers() const;   // persistent worker workgroups of a chain launch (0: no chains)
    uint32_t last_seq() const;        // sequence of the last enqueued layer
    uint32_t done_seq() const;        // the completion word: sequence of the last finished layer

    // Optional orchestration at the consumer -> reduction boundary, as TritonBackend's
    // (include/leanstream/triton_cuda.h:30-33, backends/triton/enqueue.cpp:33-36): enqueue
    // calls arm_final_prediction(arm_context) and records b_done (a hipEvent_t, borrowed)
    // between the split sequence's stage B and reduction launches, or right after a fused
    // (or dense) launch, whose consumer and reduction are one kernel. A nonzero arm code is
    // enqueue's return value; unlike the reference the reduction is still launched, so the
    // launch completes and can be aborted like any other.
    void* arm_context = nullptr;
    int (*arm_final_prediction)(void*) = nullptr;
    void* b_done = nullptr;
    // Latest caller-supplied selector state (layer is overwritten per enqueue).
    KernelRuntimeState state{};
    // Optional lifecycle hooks (as in the Triton backend): completion proof and cache
    // installation belong to the application. Without `completed`, completion is the
    // host-coherent word the latest launch's last workgroup stores (no event); without
    // `install_cache`, commit returns ENOTSUP (backends/triton/enqueue.cpp:45).
    void* lifecycle_context = nullptr;
    bool (*completed)(void*, uint32_t) = nullptr;
    int (*install_cache)(void*, uint32_t, Span<GroupId>) = nullptr;

    uint32_t status() const;       // sticky device status bits (lsamd::StatusBit / LS_STATUS_*)
    // The error a commit returns for the current status: 0 (no bit set), ETIMEDOUT (a bounded
    // wait expired) or EIO (a descriptor, the queue or a value was rejected).
    int status_error() const;
    void clear_status();
    void set_spin_limit_ticks(uint64_t ticks) { spin_limit_ = ticks; }
    uint32_t slices() const { return slices_; }
    // Overrides the selected candidate's persistent worker count (0 = the candidate's
    // own value); for tuning sweeps.
    void set_workers(uint32_t workers) { workers_override_ = workers; }
    uint32_t selected(KernelRuntimeState s) const { return selector_.select(s); }
    int last_candidate() const { return last_candidate_; }
    uint32_t max_workers() const { return max_workers_; }
    // False for a backend bound for the dense path (batch 5..32), whose launches compute
    // the resident groups only and do not consume the ready queue.
    bool consumes_queue() const;

private:
    struct Impl;
    Impl* impl_ = nullptr;
    KernelSelector selector_;
    uint64_t spin_limit_ = 200000000ull;  // 2 s of the 100 MHz device clock
    uint32_t slices_ = 0, max_workers_ = 0;
    uint32_t workers_override_ = 0;
    int last_candidate_ = -1;
    static int submit(void*, uint32_t, const void*, void*, void*, Span<ExecDesc>, DeviceExecQueue, uint32_t,
                      ConsumerMode);
    static bool complete(void*, uint32_t);
    static int commit(void*, uint32_t, Span<GroupId>);
};

}  // namespace leanstream::runtime
