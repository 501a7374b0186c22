/* C ABI of the MI355X streaming sparse INT4 MLP library (libleanstream_hip.so).
 *
 * Plain pointers and sizes only. Every entry point names the LeanStream interface it
 * replaces; a binding written against those interfaces maps one-to-one:
 *
 *   ls_hip_create / _create_table / _destroy    <- ls_triton_create / _create_table / _destroy
 *                                                  (include/leanstream/triton_cuda.h:50-52)
 *   ls_hip_bind                                 <- ls_triton_bind (triton_cuda.h:54-55); HIP kernels are
 *                                                  compiled in, so bind takes buffers + geometry
 *   ls_hip_enqueue                              <- ls_triton_enqueue (triton_cuda.h:56) merged with
 *                                                  ComputeBackend::enqueue (include/leanstream/runtime.h:12-13)
 *   ls_hip_complete                             <- ComputeBackend::complete (runtime.h:14)
 *   ls_hip_compute_backend                      <- TritonBackend::view (backends/triton/enqueue.cpp:46)
 *   ls_hip_select / ls_quantize_io_load         <- KernelSelector::select / quantize_io_load
 *                                                  (include/leanstream/kernel_selector.h:26,33)
 *   ls_hip_host_alloc / _free / _release_u32 /
 *   ls_hip_acquire_all                          <- tm_alloc / tm_free / tm_release / tm_acquire_all
 *                                                  (backends/triton/mapped.cpp:9-30)
 *   ls_queue_*                                  <- ExecutionQueue (include/leanstream/execution_queue.h:19-34)
 *   ls_rank_groups                              <- top-k ranking of ls_predict (predictor/predictor_cpu.cpp:192-201)
 *   ls_stream_create / _destroy / _run / _queue <- the end-to-end decode loop over Runtime / LayerStep
 *                                                  (examples/end_to_end/main.cu:58-72) with the I/O
 *                                                  transport replaced: HostStagingIO (pinned host store ->
 *                                                  hipMemcpyAsync) instead of the O_DIRECT engine behind
 *                                                  WeightManager (src/io/stream_io.h:45-65)
 *
 * Return values: 0 on success, a positive errno (EINVAL, ENOTSUP, ...) for rejected
 * arguments, or a positive hipError_t for a failed launch.
 */
#ifndef LEANSTREAM_HIP_H
#define LEANSTREAM_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Five 32-bit words, identical to leanstream::runtime::ExecDesc. */
typedef struct ls_exec_desc {
    uint32_t logical_group, physical_group, source_slot, dest_slot, source_kind;
} ls_exec_desc;

/* Identical to leanstream::runtime::DeviceExecQueue. */
typedef struct ls_device_queue {
    ls_exec_desc* descriptors;
    uint32_t* ready_indices;
    void* control; /* 128-byte QueueControl in host-coherent memory */
    uint32_t capacity;
} ls_device_queue;

/* Identical to leanstream::runtime::HipLayerBuffers. */
typedef struct ls_hip_layer_buffers {
    uint32_t width, group_size, batch, slot_capacity;
    uint32_t cache_groups, staging_groups, physical_groups, queue_capacity;
    const void* cache;
    const void* staging;
    const void* scales;
    void* hidden;
    void* partial;            /* reserved, unused (the reduction accumulates in backend-owned fixed point) */
    void* y32;
    uint32_t* executions;
    uint64_t* first_compute;
    uint32_t* claim_log;      /* optional: 4 words per range taken, queue_capacity ranges */
    uint64_t* stamps;
} ls_hip_layer_buffers;

/* Consumer modes (leanstream::runtime::ConsumerMode). */
enum { LS_MODE_BATCH_COMPAT = 0, LS_MODE_PROGRESSIVE = 1, LS_MODE_AUTO = 2 };
/* Device status bits returned by ls_hip_status. */
enum { LS_STATUS_TIMEOUT = 1, LS_STATUS_QUEUE_ERROR = 2, LS_STATUS_BAD_DESCRIPTOR = 4, LS_STATUS_RANGE = 8,
       LS_STATUS_QUEUE_UNCONSUMED = 16 /* dense (batch 5..32) launch whose layer published queue entries */ };

/* ---- backend ---- */
void* ls_hip_create(void);
void* ls_hip_create_table(const uint8_t* entries, uint32_t layers, uint32_t buckets);
void ls_hip_destroy(void* backend);
int ls_hip_bind(void* backend, const ls_hip_layer_buffers* buffers);
int ls_hip_enqueue(void* backend, uint32_t layer, uint32_t bucket, uint32_t epoch, const void* input, void* output,
                   void* stream, const ls_exec_desc* core, uint32_t core_count, const ls_device_queue* queue,
                   uint32_t mode);
int ls_hip_complete(void* backend, uint32_t layer);
/* Writes a leanstream::runtime::ComputeBackend (context + 5 function pointers). */
int ls_hip_compute_backend(void* backend, void* out_compute_backend, uint64_t out_bytes);
uint32_t ls_hip_status(void* backend);
void ls_hip_clear_status(void* backend);
void ls_hip_set_spin_limit(void* backend, uint64_t ticks_100mhz);
/* TritonBackend::arm_context / arm_final_prediction / b_done (include/leanstream/triton_cuda.h:30-33):
 * every later enqueue calls arm(context) and records b_done (a hipEvent_t, may be NULL) at the
 * consumer -> reduction boundary -- between the split sequence's stage B and reduction launches,
 * after a fused or dense launch. A nonzero arm code is returned by the enqueue, whose launch is
 * nevertheless whole (the reduction runs, the completion word comes). NULL arm and b_done
 * remove the hook. EINVAL for a NULL backend. */
int ls_hip_set_stage_hook(void* backend, int (*arm)(void*), void* context, void* b_done);
/* Identical to leanstream::runtime::HipEpilogue (include/leanstream/hip_backend.h): the layer
 * epilogue run after every later enqueue on the same stream -- hidden = fp16(residual + y)
 * (the Triton reduction's PUBLISH path, backends/triton/reduction.py:17-28), optionally
 * RMSNorm(hidden) * norm_weight (examples/ministral/native/predictor_shared_input.cu:16-41),
 * then hidden_flag / norm_flag receive the enqueue's epoch (system-scope release) and
 * bell += 1. A fused launch (the default entry point, batch 1..4) runs it in its own last
 * workgroup once every worker is out, and its completion word follows the epilogue; the split
 * entry point and the dense path (batch 5..32) launch it after the layer, where the
 * completion word does not cover it. A failed layer -- its launch raised a status bit (sticky
 * until ls_hip_clear_status) or its queue's error word is set -- gets neither flag nor the
 * bell, and its rows are not the layer's output. Readers of hidden wait on the flags. NULL removes
 * it. EINVAL for an unbound backend or an inconsistent block. */
typedef struct ls_hip_epilogue {
    const void* residual;
    void* hidden;
    uint32_t* hidden_flag;
    const void* norm_weight;
    void* norm_output;
    uint32_t* norm_flag;
    uint32_t* bell;
    float norm_eps;
} ls_hip_epilogue;
int ls_hip_set_epilogue(void* backend, const ls_hip_epilogue* epilogue);
/* ---- layer chains ----
 * Identical to leanstream::runtime::HipChainLayer. A sequence of layers computed by one persistent
 * launch (batch 1, 64-neuron groups, width 1024 or 4096). Layer i's hidden state
 * fp16(residual_i + y_i) -- the epilogue's publication (backends/triton/reduction.py:17-22) -- is
 * handed over inside the grid: it is layer i + 1's residual, and its input as it is or, with
 * norm_weight, as RMSNorm(hidden) * norm_weight (examples/ministral/native/predictor_shared_input.cu:
 * 16-41), so later layers' weights stream while earlier layers finish. No LeanStream C++
 * counterpart: LeanStream submits future layers ahead and gates each on an input-ready epoch
 * (docs/architecture.md:9, backends/triton/core.py:20-28). The first layer's input (and optional
 * residual) is read as the stream finds it; every later layer's input and residual must be NULL,
 * and the first layer's norm_weight NULL. Layer i gets sequence ls_hip_last_seq() - count + 1 + i;
 * the completion word (ls_hip_done_seq) takes each layer's sequence once every wave is out of it,
 * and then hidden_flag receives the epoch (system release) and bell += 1, unless a status bit is
 * set. ls_hip_complete covers the whole chain. Returns EINVAL for an invalid block, ENOTSUP for a
 * geometry without chain kernels, EBUSY while more than 1024 layers are in flight. */
typedef struct ls_hip_chain_layer {
    const ls_exec_desc* core;
    const void* cache;
    const void* staging;
    const void* scales;
    const void* input;
    const void* residual;
    const void* norm_weight;
    void* output;
    float* output32;
    void* hidden;
    uint32_t* hidden_flag;
    uint32_t* bell;
    uint32_t core_count, cache_groups, staging_groups, physical_groups, epoch;
    float norm_eps;
} ls_hip_chain_layer;
int ls_hip_enqueue_chain(void* backend, const ls_hip_chain_layer* layers, uint32_t count, void* stream);
/* Diagnostics: per-layer phase stamps of chains of at most `layers` layers,
 * [layers][(ls_hip_chain_workers() + 1) * 4][32] u64 (100 MHz clock); NULL removes them. */
int ls_hip_set_chain_stamps(void* backend, uint64_t* stamps, uint32_t layers);
uint32_t ls_hip_chain_workers(void* backend);
uint32_t ls_hip_last_seq(void* backend);
uint32_t ls_hip_done_seq(void* backend);
/* Down-projection items (256-column tiles) per unit: d / 256. */
uint32_t ls_hip_slices(void* backend);
/* Overrides the selected candidate's persistent worker count (0 = the candidate's own
 * value). No reference counterpart: a tuning knob of the persistent launch. */
void ls_hip_set_workers(void* backend, uint32_t workers);
uint32_t ls_hip_select(void* backend, uint32_t layer, uint32_t bucket);
int ls_hip_last_candidate(void* backend);
uint32_t ls_hip_max_workers(void* backend);
uint32_t ls_quantize_io_load(uint32_t remaining, uint32_t total, uint32_t buckets);

/* ---- allocation-free resident layer ----
 * No counterpart in LeanStream. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): one layer whose
 * groups are all resident (the core descriptors; no ready queue), computed as ls_hip_enqueue
 * computes it (fused persistent kernel, same bits) with its synchronisation words,
 * accumulators and h rows in a per-GPU device array of the library (about 1.9 MB, held until
 * the process ends) instead of the buffers ls_hip_bind allocates. Calls no hipMalloc/hipFree.
 * Stream-ordered: output (fp16 [batch][width]), output32 (optional fp32) and status (optional
 * device-visible word, cleared by the call, LS_STATUS_* bits) are valid once the stream
 * reaches the end of the call. Calls that overlap on one GPU race on the shared array.
 * Limits: width <= 8192 (a multiple of 256 with kernels built for it), batch 1..4 (ENOTSUP
 * above), core_count <= 1024 and core_count * group_size <= 32768 (ENOSPC beyond). */
int ls_hip_core_layer_noalloc(uint32_t width, uint32_t group_size, uint32_t batch, const void* cache,
                              uint32_t cache_groups, const void* scales, uint32_t scale_groups, const ls_exec_desc* core,
                              uint32_t core_count, const void* input, void* output, float* output32, uint32_t* status,
                              void* stream);

/* ---- coherent host memory (fine-grained, GPU-visible at system scope) ---- */
void* ls_hip_host_alloc(uint64_t bytes);
void ls_hip_host_free(void* ptr);
void ls_hip_release_u32(void* base, int64_t index, uint32_t value);
int ls_hip_acquire_all(const void* base, int32_t count, uint32_t value, int32_t timeout_ms);

/* ---- ready-queue producer (serialized; see ExecutionQueue) ---- */
void* ls_queue_create(const ls_device_queue* view);
void ls_queue_destroy(void* queue);
void ls_queue_reset(void* queue, uint32_t epoch);
void ls_queue_prepare(void* queue, uint32_t total);
void ls_queue_append_unpublished(void* queue, uint32_t index);
void ls_queue_activate(void* queue);
void ls_queue_seal(void* queue, uint32_t total);
void ls_queue_publish_all(void* queue);
void ls_queue_publish(void* queue, uint32_t index);
void ls_queue_fail(void* queue, uint32_t error);
/* Background publisher: publishes order[i] at time offset_ns[i] after start (busy
 * wait on the host clock). If fail_after < count, publishes fail_after entries and
 * then fails the queue with fail_code. Returns a handle for ls_publisher_join. */
void* ls_publisher_start(void* queue, const uint32_t* order, const uint64_t* offset_ns, uint32_t count,
                         uint32_t fail_after, uint32_t fail_code);
int ls_publisher_join(void* publisher);

/* ---- group selection ---- */
/* Top-k logical ids by (score descending, id ascending); -1 on non-finite scores. */
int ls_rank_groups(const float* scores, uint32_t count, uint32_t k, int32_t* out);

/* ---- streaming decode over host-staged layers ---- */
/* Copy engines: SDMA engines driven directly (no HIP stream), or hipMemcpyAsync streams. */
enum { LS_COPY_SDMA = 0, LS_COPY_HIP = 1 };
/* Identical to leanstream::runtime::GroupLayout (file_offset = offset in the host store). */
typedef struct ls_group_layout {
    uint32_t logical_group, physical_group;
    uint64_t file_offset;
    uint32_t bytes, reserved;
} ls_group_layout;

typedef struct ls_stream_setup {
    void* backend;            /* ls_hip_create handle, bound with staging = `staging` */
    const void* host_store;   /* pinned host memory holding every layer's packed groups */
    uint64_t host_bytes;
    void* staging;            /* device arena: logical group g at g * staging_stride */
    uint64_t staging_bytes;
    uint64_t group_bytes, staging_stride;
    uint32_t group_count;     /* logical groups per layer */
    uint32_t layers;          /* Runtime layer contexts */
    uint32_t qd;              /* copies in flight, 1..32 */
    uint32_t copy_engine;     /* LS_COPY_SDMA or LS_COPY_HIP */
    uint32_t copy_queues;     /* SDMA engines (1..16) or hipMemcpyAsync streams (1..2), round robin */
    uint32_t copy_chunk;      /* SDMA: bytes per copy piece (0 = one copy per group) */
    uint32_t mode;            /* LS_MODE_* */
    int32_t device;
} ls_stream_setup;

typedef struct ls_stream_layer {
    const ls_group_layout* layout; /* [group_count] */
    const int32_t* rank;           /* update_prediction priority order */
    uint32_t rank_count;
    const int32_t* final_ids;      /* finalize order */
    uint32_t final_count;
    const uint64_t* arrival_ns;    /* optional [group_count]: earliest copy start after begin */
    const void* input;             /* device fp16 x */
    void* output;                  /* device fp16 y */
} ls_stream_layer;

/* NULL on invalid setup or allocation failure. */
void* ls_stream_create(const ls_stream_setup* setup);
void ls_stream_destroy(void* decoder);
/* The decoder's ready queue (descriptors, publication order, control words). */
int ls_stream_queue(void* decoder, ls_device_queue* out);
/* Runs `count` layers in order on `stream` (Runtime layer id = (first_layer + i) % layers).
 * times: optional [count][7] ns after the call's start: begin, after begin_layer, after
 * update_prediction, after enqueue_compute, after finalize, completion observed (left 0
 * when the launch's completion was not observed), after commit. stamps: optional [count][group_count][3] ns after each layer's begin: admission,
 * copy submission, copy completion. Stops at the first failing layer and returns its code
 * (ETIMEDOUT when the kernel does not complete within timeout_ms). */
int ls_stream_run(void* decoder, const ls_stream_layer* layers, uint32_t count, uint32_t first_layer, void* stream,
                  uint64_t* times, uint64_t* stamps, int32_t timeout_ms);
/* Failure injection of the transport (the role of LeanStream's STREAM_TESTING read hook,
 * src/io/stream_io.h): from now on every copy of logical group `group` into the staging
 * arena is refused with `error` (a positive errno) at submission, as a failed read would
 * be; error 0 clears it. The layer then fails with that code through the queue's error
 * word, as a real transport error does. */
int ls_stream_inject_copy_error(void* decoder, uint32_t group, int32_t error);

/* ---- synthetic workload generation on the device (counter-based splitmix64) ---- */
int ls_synth_bytes(void* dst, uint64_t bytes, uint64_t seed, void* stream);
int ls_synth_uniform_f16(void* dst, uint64_t count, uint64_t seed, double lo, double hi, void* stream);
int ls_synth_normal_f16(void* dst, uint64_t count, uint64_t seed, void* stream);
int ls_synth_normal_bf16(void* dst, uint64_t count, uint64_t seed, void* stream);
/* No reference counterpart; a benchmark utility: holds `stream` (one wave) until the host sets
 * the host-coherent word *flag nonzero, or limit_ticks of the 100 MHz device clock pass. Work
 * queued behind it starts back to back once it is released, without the host's submission
 * latency in between. EINVAL for a NULL flag or a zero limit. */
int ls_hold_stream(void* stream, const uint32_t* flag, uint64_t limit_ticks);

#ifdef __cplusplus
}
#endif
#endif
