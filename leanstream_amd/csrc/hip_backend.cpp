// HipBackend: the MI355X ComputeBackend for the streaming sparse INT4 MLP.
// Cold path (bind): validation, geometry choice, occupancy query, device sync state.
// Hot path (enqueue): O(1) candidate selection + one (fused) or three (split) launches
// on the caller's stream; completion is proven by the kernels' own host-coherent words.
#include "leanstream/hip_backend.h"
#include <hip/hip_runtime_api.h>
#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include "mlp_launch.h"

namespace leanstream::runtime {

struct HipBackend::Impl {
    HipLayerBuffers buf{};
    lsamd::MlpArgs base{};
    lsamd::Bounds bounds{};
    uint32_t* sync = nullptr;
    uint32_t* qmirror = nullptr;  // device copy of published queue descriptors
    unsigned long long* yacc = nullptr;  // packed fixed-point column accumulators [2][rows][d][kAccStride]
    uint32_t slot_words = 0;
    uint32_t* status = nullptr;  // host-coherent
    void* owned_hidden = nullptr;
    uint16_t* h16 = nullptr;     // dense path: fp16 h rows
    float* dpart = nullptr;      // dense path: down-projection partial rows
    uint16_t* x16 = nullptr;     // dense path: x converted to paired fp16
    bool dense = false;          // batch > kMaxBatch: every launch takes the matrix-core path
    uint32_t* done = nullptr;    // host-coherent: sequence of the last finished launch
    uint32_t* arrivals = nullptr;  // epilogue row workgroups that finished (zero between launches)
    HipEpilogue epilogue{};
    bool has_epilogue = false;
    uint32_t last_seq = 0;       // sequence of the last enqueued launch (0: none)
    // Layer chains (batch 1, 64-neuron groups, widths lsamd::chain_available): records in a
    // pinned host ring and its device mirror (index seq % ring), the synchronisation block,
    // the self-resetting accumulators [2][d] and the tagged hidden words [2][d].
    lsamd::ChainRec* chain_host = nullptr;
    lsamd::ChainRec* chain_dev = nullptr;
    uint32_t* chain_sync = nullptr;
    unsigned long long* chain_acc = nullptr;
    uint32_t* chain_words = nullptr;
    uint64_t* chain_stamps = nullptr;   // optional diagnostics [layers][grid * 4][32]
    uint32_t chain_stamp_layers = 0;
    int per_cu_chain = 0;
    bool chain_needs_clear = false;
    uint32_t chain_clear_seq = 0;       // sequence at the last clear of the tagged hidden words
    bool needs_clear = true;
    uint32_t seq = 0;
    int cus = 0, per_cu_fused = 0, per_cu_split = 0;
    int per_cu_fused_plain = 0, per_cu_split_plain = 0;   // the plain walk's kernels at batch 1
    bool bound = false;

    void release() {
        if (sync) (void)hipFree(sync);
        if (qmirror) (void)hipFree(qmirror);
        if (yacc) (void)hipFree(yacc);
        if (owned_hidden) (void)hipFree(owned_hidden);
        if (h16) (void)hipFree(h16);
        if (dpart) (void)hipFree(dpart);
        if (x16) (void)hipFree(x16);
        if (status) (void)hipHostFree(status);
        if (done) (void)hipHostFree(done);
        if (arrivals) (void)hipFree(arrivals);
        if (chain_host) (void)hipHostFree(chain_host);
        if (chain_dev) (void)hipFree(chain_dev);
        if (chain_sync) (void)hipFree(chain_sync);
        if (chain_acc) (void)hipFree(chain_acc);
        if (chain_words) (void)hipFree(chain_words);
        chain_host = nullptr;
        chain_dev = nullptr;
        chain_sync = nullptr;
        chain_acc = nullptr;
        chain_words = nullptr;
        chain_stamps = nullptr;
        chain_stamp_layers = 0;
        per_cu_chain = 0;
        arrivals = nullptr;
        has_epilogue = false;
        sync = nullptr;
        qmirror = nullptr;
        yacc = nullptr;
        owned_hidden = nullptr;
        h16 = nullptr;
        dpart = nullptr;
        x16 = nullptr;
        status = nullptr;
        done = nullptr;
        bound = false;
    }
    ~Impl() { release(); }
};

HipBackend::HipBackend(KernelDecisionTable table) : impl_(new Impl), selector_(hip_selector(table)) {}
HipBackend::~HipBackend() { delete impl_; }

int HipBackend::bind(const HipLayerBuffers& b) {
    Impl& p = *impl_;
    if (p.bound) return EBUSY;
    if (!b.width || b.width % 256 || !b.group_size || b.group_size > 256 || !b.slot_capacity || !b.physical_groups ||
        !b.scales || (b.cache_groups && !b.cache) || (b.staging_groups && !b.staging))
        return EINVAL;
    if (!b.batch || b.batch > lsamd::kMaxDenseBatch) return ENOTSUP;
    // batch > kMaxBatch: the dense matrix-core path (64-neuron groups, core units only)
    const bool dense = b.batch > lsamd::kMaxBatch;
    if (dense && (b.group_size != 64 || !lsamd::dense_available(static_cast<int>(b.width)))) return ENOTSUP;
    if (b.slot_capacity > lsamd::kMaxRowsReduced) return EINVAL;  // count field of the accumulators
    if (!lsamd::variant_available(static_cast<int>(b.width))) return ENOTSUP;
    p.buf = b;
    p.dense = dense;
    const uint32_t rows = dense ? 1u : b.batch;   // the batch-1..4 kernels' h rows and accumulators
    const uint32_t units_cap = b.slot_capacity + b.queue_capacity;
    p.slot_words = lsamd::sync_slot_words(units_cap);
    hipError_t e = hipMalloc(&p.sync, sizeof(uint32_t) * 2 * p.slot_words);
    if (e == hipSuccess) e = hipMalloc(&p.qmirror, sizeof(uint32_t) * 5 * std::max<uint32_t>(1, b.queue_capacity));
    if (e == hipSuccess) e = hipMalloc(&p.yacc, sizeof(long long) * 2 * b.width * rows * lsamd::kAccStride);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&p.status), 64, hipHostMallocCoherent | hipHostMallocMapped);
    if (e == hipSuccess && !b.hidden)
        e = hipMalloc(&p.owned_hidden, sizeof(uint64_t) * b.slot_capacity * rows * b.group_size);
    if (e == hipSuccess && dense)
        e = hipMalloc(&p.h16, sizeof(uint16_t) * 32 * b.slot_capacity * b.group_size);
    if (e == hipSuccess && dense)
        e = hipMalloc(&p.dpart, sizeof(float) * lsamd::kDenseSplits * 32 * b.width);
    if (e == hipSuccess && dense) e = hipMalloc(&p.x16, sizeof(uint16_t) * 32 * b.width);
    // h rows >= batch stay zero: the dense down projection reads all 32 rows
    if (e == hipSuccess && dense) e = hipMemset(p.h16, 0, sizeof(uint16_t) * 32 * b.slot_capacity * b.group_size);
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&p.done), 64, hipHostMallocCoherent | hipHostMallocMapped);
    if (e == hipSuccess) e = hipMalloc(&p.arrivals, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(p.arrivals, 0, sizeof(uint32_t));
    int dev = 0;
    if (e == hipSuccess) e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&p.cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int gs = static_cast<int>(b.group_size);
    if (e == hipSuccess)
        e = lsamd::resident_workers(b.width, lsamd::kEntryFused, static_cast<int>(rows), gs, &p.per_cu_fused);
    if (e == hipSuccess)
        e = lsamd::resident_workers(b.width, lsamd::kEntrySplit, static_cast<int>(rows), gs, &p.per_cu_split);
    if (e == hipSuccess && (p.per_cu_fused < 1 || p.per_cu_split < 1 || p.cus * std::min(p.per_cu_fused, p.per_cu_split) < 3))
        e = hipErrorInvalidConfiguration;
    if (e == hipSuccess && !dense && b.batch == 1)
        e = lsamd::resident_workers(b.width, lsamd::kEntryFused, 1, gs, &p.per_cu_fused_plain, 1);
    if (e == hipSuccess && !dense && b.batch == 1)
        e = lsamd::resident_workers(b.width, lsamd::kEntrySplit, 1, gs, &p.per_cu_split_plain, 1);
    if (e == hipSuccess && !dense && b.batch == 1 && std::min(p.per_cu_fused_plain, p.per_cu_split_plain) < 1)
        e = hipErrorInvalidConfiguration;
    // layer chains: the geometry of the staged batch-1 kernels
    const bool chains = !dense && b.batch == 1 && b.group_size == 64 && lsamd::chain_available(static_cast<int>(b.width));
    const uint32_t ring = lsamd::chain_ring();
    if (e == hipSuccess && chains)
        e = hipHostMalloc(reinterpret_cast<void**>(&p.chain_host), sizeof(lsamd::ChainRec) * ring,
                          hipHostMallocCoherent | hipHostMallocMapped);
    if (e == hipSuccess && chains) e = hipMalloc(&p.chain_dev, sizeof(lsamd::ChainRec) * ring);
    if (e == hipSuccess && chains) e = hipMalloc(&p.chain_sync, sizeof(uint32_t) * lsamd::kChainSyncWords);
    if (e == hipSuccess && chains) e = hipMalloc(&p.chain_acc, sizeof(long long) * 2 * b.width);
    if (e == hipSuccess && chains) e = hipMalloc(&p.chain_words, sizeof(uint32_t) * 2 * b.width);
    if (e == hipSuccess && chains) e = lsamd::chain_resident(static_cast<int>(b.width), &p.per_cu_chain);
    if (e == hipSuccess && chains && p.cus * p.per_cu_chain < 2) e = hipErrorInvalidConfiguration;
    if (e == hipSuccess && chains)
        e = lsamd::clear_sync(p.chain_sync, lsamd::kChainSyncWords, p.chain_acc, 2 * b.width,
                              reinterpret_cast<uint64_t*>(p.chain_words), b.width, nullptr);
    uint64_t* hbuf = static_cast<uint64_t*>(b.hidden ? b.hidden : p.owned_hidden);
    if (e == hipSuccess)
        e = lsamd::clear_sync(p.sync, 2 * p.slot_words, p.yacc, 2 * b.width * rows * lsamd::kAccStride, hbuf,
                              b.slot_capacity * rows * b.group_size, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        p.release();
        return static_cast<int>(e);
    }
    *p.status = 0;
    lsamd::MlpArgs& a = p.base;
    a = lsamd::MlpArgs{};
    a.cache = static_cast<const uint8_t*>(b.cache);
    a.staging = static_cast<const uint8_t*>(b.staging);
    a.scales = static_cast<const uint16_t*>(b.scales);
    a.hbuf = static_cast<uint64_t*>(b.hidden ? b.hidden : p.owned_hidden);
    a.y32 = static_cast<float*>(b.y32);
    a.executions = b.executions;
    a.first_compute = b.first_compute;
    a.claim_log = b.claim_log;
    a.claim_log_cap = b.claim_log ? b.queue_capacity : 0;   // ranges (lsamd::kClaimLogWords words each)
    a.stamps = b.stamps;
    a.sync = p.sync;
    a.qmirror = p.qmirror;
    a.yacc = p.yacc;
    a.status = p.status;
    a.width = b.width;
    a.batch = b.batch;
    a.group_size = b.group_size;
    a.slices = b.width / lsamd::kDnCols;
    a.slot_words = p.slot_words;
    a.units_cap = units_cap;
    a.slot_capacity = b.slot_capacity;
    a.h16 = p.h16;
    a.dpart = p.dpart;
    a.x16 = p.x16;
    a.dsplits = dense ? lsamd::kDenseSplits : 0u;
    p.bounds = {b.cache_groups, b.staging_groups, b.physical_groups};
    slices_ = b.width / lsamd::kDnCols;
    max_workers_ = static_cast<uint32_t>(p.cus * p.per_cu_fused) - 1;
    p.needs_clear = false;
    p.chain_needs_clear = false;
    p.chain_clear_seq = 0;
    p.last_seq = 0;
    *p.done = 0;
    p.bound = true;
    return 0;
}

int HipBackend::enqueue_chain(const HipChainLayer* layers, uint32_t count, void* stream) {
    Impl& p = *impl_;
    if (!p.bound || !layers || !count) return EINVAL;
    if (!p.chain_dev) return ENOTSUP;   // geometry without chain kernels
    const uint32_t ring = lsamd::chain_ring();
    if (count > ring / 2) return EINVAL;
    for (uint32_t i = 0; i < count; ++i) {
        const HipChainLayer& l = layers[i];
        // the first layer reads its input; every later one takes the previous hidden state
        if ((i == 0) != (l.input != nullptr) || (i && l.residual) || (!i && l.norm_weight)) return EINVAL;
        if (!(l.norm_eps >= 0.f) || l.norm_eps > 1.f) return EINVAL;
        if (!l.output || !l.cache || !l.scales || (l.core_count && !l.core) || (l.staging_groups && !l.staging))
            return EINVAL;
        if (l.core_count > p.buf.slot_capacity || !l.cache_groups || !l.physical_groups) return EINVAL;
    }
    auto hs = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    // Sequences of a chain are consecutive (tags of the hidden words). Before the launch
    // sequence wraps, or once the tagged words could hold a tag from 32768 sequences back,
    // everything tagged is cleared; after a failed launch the synchronisation block too.
    const bool wrap = p.seq > UINT32_MAX - count - 1;
    if (wrap || p.needs_clear) {
        const uint32_t rows = 1;
        e = lsamd::clear_sync(p.sync, 2 * p.slot_words, p.yacc, 2 * p.buf.width * rows * lsamd::kAccStride, p.base.hbuf,
                              p.buf.slot_capacity * rows * p.buf.group_size, hs);
        if (e != hipSuccess) return static_cast<int>(e);
        p.needs_clear = false;
        if (wrap) p.seq = 0;
    }
    if (status() || p.chain_needs_clear || wrap || p.seq + count - p.chain_clear_seq > lsamd::kChainClearPeriod) {
        e = lsamd::clear_sync(p.chain_sync, lsamd::kChainSyncWords, p.chain_acc, 2 * p.buf.width,
                              reinterpret_cast<uint64_t*>(p.chain_words), p.buf.width, hs);
        if (e != hipSuccess) return static_cast<int>(e);
        p.chain_needs_clear = false;
        p.chain_clear_seq = p.seq;
    }
    const uint32_t seq0 = p.seq + 1;
    // host ring: the records of sequences after the last completed layer are live
    const uint32_t done = __atomic_load_n(p.done, __ATOMIC_ACQUIRE);
    if (p.last_seq && static_cast<int32_t>(seq0 + count - 1 - done) > static_cast<int32_t>(ring)) return EBUSY;
    for (uint32_t i = 0; i < count; ++i) {
        const HipChainLayer& l = layers[i];
        lsamd::ChainRec r{};
        r.core = l.core;
        r.cache = static_cast<const uint8_t*>(l.cache);
        r.staging = static_cast<const uint8_t*>(l.staging);
        r.scales = static_cast<const uint16_t*>(l.scales);
        r.x = static_cast<const uint16_t*>(l.input);
        r.residual = static_cast<const uint16_t*>(l.residual);
        r.norm_weight = static_cast<const uint16_t*>(l.norm_weight);
        r.norm_eps = l.norm_eps;
        r.y = static_cast<uint16_t*>(l.output);
        r.y32 = l.output32;
        r.hidden = static_cast<uint16_t*>(l.hidden);
        r.hidden_flag = l.hidden_flag;
        r.bell = l.bell;
        r.core_count = l.core_count;
        r.cache_groups = l.cache_groups;
        r.staging_groups = l.staging_groups;
        r.physical_groups = l.physical_groups;
        r.epoch = l.epoch;
        r.seq = seq0 + i;
        r.chained = i ? 1u : 0u;
        p.chain_host[(seq0 + i) % ring] = r;
    }
    std::atomic_thread_fence(std::memory_order_release);
    lsamd::ChainArgs c{};
    c.host_recs = p.chain_host;
    c.recs = p.chain_dev;
    c.count = count;
    c.csync = p.chain_sync;
    c.hbuf = p.base.hbuf;
    c.yacc = p.chain_acc;
    c.xtag = p.chain_words;
    c.status = p.status;
    c.done = p.done;
    c.stamps = count <= p.chain_stamp_layers ? p.chain_stamps : nullptr;
    c.width = p.buf.width;
    c.slot_capacity = p.buf.slot_capacity;
    c.grid = static_cast<uint32_t>(p.cus * p.per_cu_chain);
    c.spin_limit = spin_limit_;
    e = lsamd::launch_chain(c, seq0 % ring, hs);
    if (e != hipSuccess) {
        p.chain_needs_clear = true;
        return static_cast<int>(e);
    }
    p.seq = seq0 + count - 1;
    p.last_seq = p.seq;
    last_candidate_ = -1;
    return 0;
}

int HipBackend::set_chain_stamps(uint64_t* stamps, uint32_t layers) {
    Impl& p = *impl_;
    if (!p.bound || !p.chain_dev) return EINVAL;
    p.chain_stamps = layers ? stamps : nullptr;
    p.chain_stamp_layers = stamps ? layers : 0;
    return 0;
}

uint32_t HipBackend::chain_workers() const { return impl_->chain_dev ? static_cast<uint32_t>(impl_->cus * impl_->per_cu_chain) - 1 : 0; }
uint32_t HipBackend::last_seq() const { return impl_->last_seq; }
uint32_t HipBackend::done_seq() const { return impl_->done ? __atomic_load_n(impl_->done, __ATOMIC_ACQUIRE) : 0; }

int HipBackend::enqueue(KernelRuntimeState s, const void* input, void* output, void* stream, Span<ExecDesc> core,
                        DeviceExecQueue q, uint32_t epoch, ConsumerMode mode) {
    Impl& p = *impl_;
    if (!p.bound || !epoch || !input || !output || !q.control || !q.descriptors || !q.ready_indices) return EINVAL;
    if ((core.size && !core.data) || core.size > p.buf.slot_capacity || q.capacity > p.buf.queue_capacity) return EINVAL;
    const KernelCandidate c = selector_.candidate(selector_.select(s));
    const int entry = c.entry_point == lsamd::kEntrySplit ? lsamd::kEntrySplit : lsamd::kEntryFused;
    // unroll = items in flight per wave: 1 asks for the plain walk (batch 1)
    const bool plain = c.unroll == 1 && !p.dense && p.buf.batch == 1;
    const int per_cu = entry == lsamd::kEntryFused ? (plain ? p.per_cu_fused_plain : p.per_cu_fused)
                                                   : (plain ? p.per_cu_split_plain : p.per_cu_split);
    // Persistent workers (plus the mirror workgroup) must be co-resident: a worker's
    // down-projection share waits for h published by other workers.
    const uint32_t resident = static_cast<uint32_t>(p.cus * per_cu) - 1;
    const uint32_t want = workers_override_ ? workers_override_ : c.workers ? c.workers : resident;
    const uint32_t workers = std::max<uint32_t>(1, std::min<uint32_t>(want, resident));
    lsamd::MlpArgs a = p.base;
    a.core = core.data;
    a.core_count = static_cast<uint32_t>(core.size);
    a.qdesc = q.descriptors;
    a.ready = q.ready_indices;
    a.control = q.control;
    a.capacity = q.capacity;
    a.x = static_cast<const uint16_t*>(input);
    a.y = static_cast<uint16_t*>(output);
    a.epoch = epoch;
    a.batch_mode = mode == ConsumerMode::Progressive ? 0u : 1u;
    a.claim_batch = c.group_batch;
    a.dn_tile = c.tile_size == lsamd::kDnCols ? lsamd::kDnCols : 0u;
    a.spin_limit = spin_limit_;
    auto hs = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    // h words are tagged with the launch sequence. A clear (after a failed launch, and
    // before the sequence wraps) zeroes every tag, so no stored tag can match a later one.
    const uint32_t rows = p.dense ? 1u : p.buf.batch;
    if (p.needs_clear || p.seq == UINT32_MAX) {
        e = lsamd::clear_sync(p.sync, 2 * p.slot_words, p.yacc, 2 * p.buf.width * rows * lsamd::kAccStride, a.hbuf,
                              p.buf.slot_capacity * rows * p.buf.group_size, hs);
        if (e != hipSuccess) return static_cast<int>(e);
        p.needs_clear = false;
    }
    // The sequence never takes the value 0 and only moves forward, so neither a tag
    // from before the last clear nor a late completion word can match a newer launch.
    p.seq = p.seq == UINT32_MAX ? 1u : p.seq + 1;
    a.seq = p.seq;
    a.done = p.done;
    const lsamd::LaunchPlan plan{static_cast<int>(p.buf.width), static_cast<int>(workers), entry, plain ? 1 : 0};
    // Batch 5..32: the dense matrix-core path computes the core units (the queue is not
    // consumed: a dense layer's groups are all resident).
    lsamd::StageHook hook{arm_final_prediction, arm_context, static_cast<hipEvent_t>(b_done), 0};
    lsamd::StageHook* hk = arm_final_prediction || b_done ? &hook : nullptr;
    // The fused launch runs the epilogue in its own last workgroup; the split entry point and
    // the dense path launch epilogue_kernel after the layer.
    const bool fused_epilogue = p.has_epilogue && !p.dense && entry == lsamd::kEntryFused;
    if (fused_epilogue) {
        const HipEpilogue& ep = p.epilogue;
        a.residual = static_cast<const uint16_t*>(ep.residual);
        a.hidden = static_cast<uint16_t*>(ep.hidden);
        a.hidden_flag = ep.hidden_flag;
        a.norm_weight = static_cast<const uint16_t*>(ep.norm_weight);
        a.norm_out = static_cast<uint16_t*>(ep.norm_output);
        a.norm_flag = ep.norm_flag;
        a.bell = ep.bell;
        a.norm_eps = ep.norm_eps;
    }
    if (p.dense) {
        e = lsamd::launch_dense(a, p.bounds, hs);
        if (e == hipSuccess) e = lsamd::run_stage_hook(hk, hs);
    } else {
        e = lsamd::launch_layer(plan, a, p.bounds, hs, hk);
    }
    last_candidate_ = static_cast<int>(c.id);
    if (e != hipSuccess) {
        p.needs_clear = true;  // a partial launch may have left a ring slot dirty
        return static_cast<int>(e);
    }
    p.last_seq = a.seq;
    if (p.has_epilogue && !fused_epilogue) {
        const HipEpilogue& ep = p.epilogue;
        lsamd::EpilogueArgs x{};
        x.y = a.y;
        x.residual = static_cast<const uint16_t*>(ep.residual);
        x.hidden = static_cast<uint16_t*>(ep.hidden);
        x.hidden_flag = ep.hidden_flag;
        x.norm_weight = static_cast<const uint16_t*>(ep.norm_weight);
        x.norm_out = static_cast<uint16_t*>(ep.norm_output);
        x.norm_flag = ep.norm_flag;
        x.bell = ep.bell;
        x.arrivals = p.arrivals;
        x.status = p.status;
        x.queue_error = &q.control->error;
        x.eps = ep.norm_eps;
        x.width = p.buf.width;
        x.rows = p.buf.batch;
        x.epoch = epoch;
        e = lsamd::launch_epilogue(x, hs);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    return hook.rc;   // the arm's code: the layer is launched whole either way
}

int HipBackend::set_epilogue(const HipEpilogue* ep) {
    Impl& p = *impl_;
    if (!p.bound) return EINVAL;
    if (!ep) {
        p.has_epilogue = false;
        return 0;
    }
    if (!ep->residual || !ep->hidden || (ep->norm_weight && !ep->norm_output) || (!ep->norm_weight && ep->norm_output) ||
        (ep->norm_flag && !ep->norm_weight) || !(ep->norm_eps >= 0.f) || ep->norm_eps > 1.f)
        return EINVAL;
    p.epilogue = *ep;
    p.has_epilogue = true;
    return 0;
}

bool HipBackend::consumes_queue() const { return !impl_->dense; }

uint32_t HipBackend::status() const { return impl_->status ? __atomic_load_n(impl_->status, __ATOMIC_ACQUIRE) : 0; }
int HipBackend::status_error() const {
    const uint32_t st = status();
    return !st ? 0 : st & lsamd::kStatusTimeout ? ETIMEDOUT : EIO;
}
void HipBackend::clear_status() {
    // a failed chain launch may have left its synchronisation block dirty: the next chain
    // launch clears it first
    if (impl_->status && __atomic_exchange_n(impl_->status, 0u, __ATOMIC_ACQ_REL)) impl_->chain_needs_clear = true;
}

int HipBackend::submit(void* ctx, uint32_t layer, const void* input, void* output, void* stream, Span<ExecDesc> core,
                       DeviceExecQueue q, uint32_t epoch, ConsumerMode mode) {
    auto& b = *static_cast<HipBackend*>(ctx);
    KernelRuntimeState s = b.state;
    s.layer = layer;
    return b.enqueue(s, input, output, stream, core, q, epoch, mode);
}

bool HipBackend::complete(void* ctx, uint32_t layer) {
    auto& b = *static_cast<HipBackend*>(ctx);
    if (b.completed) return b.completed(b.lifecycle_context, layer);
    // Each launch stores its sequence once every one of its workgroups is done (the
    // fused launch's mirror workgroup, or the split sequence's last reduction block):
    // wrap-aware comparison against the last enqueued launch.
    const Impl& p = *b.impl_;
    if (!p.last_seq) return true;
    const uint32_t done = __atomic_load_n(p.done, __ATOMIC_ACQUIRE);
    return static_cast<int32_t>(done - p.last_seq) >= 0;
}

int HipBackend::commit(void* ctx, uint32_t layer, Span<GroupId> ids) {
    auto& b = *static_cast<HipBackend*>(ctx);
    // A launch that raised a status bit (a bounded wait expired -- e.g. CUs held by another
    // process kept the persistent grid from being co-resident --, a descriptor or the queue
    // was rejected, a value was out of range) produced no valid output: the layer is not
    // committed, so LayerStep::commit fails and the caller aborts the step. The bits stay
    // set until clear_status().
    if (const int rc = b.status_error()) return rc;
    // Cache installation is application policy: without the application's hook the
    // backend cannot install anything and says so, as LeanStream's Triton backend does
    // (backends/triton/enqueue.cpp:45).
    return b.install_cache ? b.install_cache(b.lifecycle_context, layer, ids) : ENOTSUP;
}

ComputeBackend HipBackend::view() {
    ComputeBackend v;
    v.context = this;
    v.enqueue = submit;
    v.complete = complete;
    v.commit = commit;
    return v;
}

}  // namespace leanstream::runtime
