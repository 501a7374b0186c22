// Host entry points of the kernel translation unit.
#pragma once
#include <hip/hip_runtime_api.h>
#include "mlp_args.h"

namespace lsamd {

enum EntryPoint : int { kEntryFused = 0, kEntrySplit = 1 };

struct LaunchPlan {
    int width;        // d
    int workers;      // persistent workgroups
    int entry_point;  // kEntryFused or kEntrySplit
    int walk = 0;     // 0: the shape's own walk; 1: the plain walk at batch 1 (one item in flight per wave)
};

bool variant_available(int width);
// Maximum co-resident workgroups per CU for the kernels of an entry point (the kernel
// family depends on the batch and, at batch 1, on the group size).
hipError_t resident_workers(int width, int entry_point, int batch, int group_size, int* per_cu, int walk = 0);
// Fused: one persistent launch. Split: stage A (if core) -> stage B -> reduction.
// Host work at the boundary between the queue consumer and the reduction (LeanStream's
// A -> B -> arm -> event -> reduction order, backends/triton/enqueue.cpp:33-36): the split
// sequence runs it between its stage B and reduction launches; a fused launch, whose
// consumer and reduction are one kernel, right after that launch. The arm's return code
// lands in `rc`; the reduction is launched regardless, so the launch's completion word
// still comes.
struct StageHook {
    int (*arm)(void*);
    void* context;
    hipEvent_t b_done;   // optional: recorded at the boundary
    int rc;
};
hipError_t run_stage_hook(StageHook* hook, hipStream_t stream);
hipError_t launch_layer(const LaunchPlan&, const MlpArgs&, const Bounds&, hipStream_t, StageHook* hook = nullptr);
// Dense batched path (batch > kMaxBatch, core units only): gate/up -> down -> reduction.
hipError_t launch_dense(const MlpArgs&, const Bounds&, hipStream_t);
bool dense_available(int width);   // widths the dense (batch > kMaxBatch) path is compiled for
// Layer epilogue (after the layer's launch, same stream): the next hidden state
// fp16(residual + y) per row, optionally its RMSNorm, then the flags.
struct EpilogueArgs {
    const uint16_t* y;            // fp16 [rows][width]: the layer output
    const uint16_t* residual;     // fp16 [rows][width]
    uint16_t* hidden;             // fp16 [rows][width]
    uint32_t* hidden_flag;        // optional: epoch, system release, once every row is written
    const uint16_t* norm_weight;  // optional fp16 [width]
    uint16_t* norm_out;           // fp16 [rows][width] (with norm_weight)
    uint32_t* norm_flag;          // optional: epoch, after hidden_flag
    uint32_t* bell;               // optional: +1 after the flags
    uint32_t* arrivals;           // device word, zero between launches (the last row block resets it)
    const uint32_t* status;       // the backend's status word: set bits withhold the flags and the bell
    const uint32_t* queue_error;  // optional: the launch's queue error word; nonzero withholds them too
    float eps;
    uint32_t width, rows, epoch;
};
hipError_t launch_epilogue(const EpilogueArgs&, hipStream_t);
// Layer chains (chain_mlp.hip): batch 1, 64-neuron groups, widths chain_available().
bool chain_available(int width);
uint32_t chain_ring();   // records in the host and device rings of a backend (index seq % ring)
hipError_t chain_resident(int width, int* per_cu);
// One persistent launch over args.count layers; `first` = the first layer's sequence % ring.
hipError_t launch_chain(const ChainArgs& args, uint32_t first, hipStream_t stream);
// Zeroes both ring slots, both accumulator buffers and the tagged h rows.
hipError_t clear_sync(uint32_t* sync, uint32_t words, unsigned long long* yacc, uint32_t columns, uint64_t* hbuf,
                      uint32_t hwords, hipStream_t);

}  // namespace lsamd
