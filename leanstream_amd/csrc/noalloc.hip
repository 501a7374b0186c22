// Allocation-free variant of a resident (core-only) layer launch: ls_hip_core_layer_noalloc.
//
// It has no counterpart in LeanStream. It serves callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): the layer's synchronisation words, accumulators and h rows live in a
// file-scope device array, `scratch`, instead of the buffers ls_hip_bind allocates. The
// caller passes the inputs (weights, scales, descriptors, x) and the outputs (y, and
// optionally the fp32 y and a status word), as with ls_hip_enqueue.
//
// Every GPU holds its own copy of `scratch` (kScratchBytes) until the process ends. Its
// device address is taken once per device, on the first call there, with
// hipGetSymbolAddress; host code uses that address, never the array's name. Each call
// clears what it uses with a kernel on the caller's stream, then runs the persistent
// fused layer kernel; calls that overlap on one GPU (different streams) race on the array.
#include <hip/hip_runtime.h>
#include <cerrno>
#include <mutex>
#include "leanstream_hip.h"
#include "mlp_args.h"
#include "mlp_launch.h"

namespace lsamd {
namespace {

// Limits of one call (ENOSPC beyond them).
constexpr uint32_t kNaMaxWidth = 8192;
constexpr uint32_t kNaMaxUnits = 1024;        // core groups
constexpr uint32_t kNaMaxNeurons = 32768;     // core groups x group size
constexpr uint32_t kNaThreads = 256;

// Layout of the array (bytes; every region starts on a 256-byte boundary).
constexpr size_t kOffControl = 0;                    // QueueControl of an empty, sealed queue (128 B)
constexpr size_t kOffStatus = 256;                   // status word (when the caller passes none)
constexpr size_t kOffDone = 512;                     // completion word
constexpr size_t kOffQueue = 768;                    // queue descriptor / ready / mirror words (unread: empty queue)
constexpr size_t kOffSync = 1024;                    // two ring slots
constexpr size_t kSyncBytes = 2 * sizeof(uint32_t) * (kSyncUnits + kNaMaxUnits * kLine);
constexpr size_t kOffAcc = kOffSync + kSyncBytes;    // two accumulator buffers
constexpr size_t kAccBytes = 2 * sizeof(unsigned long long) * kNaMaxWidth * kMaxBatch * kAccStride;
constexpr size_t kOffHidden = kOffAcc + kAccBytes;   // tagged h rows
constexpr size_t kHiddenBytes = sizeof(uint64_t) * kNaMaxNeurons * kMaxBatch;
constexpr size_t kScratchBytes = kOffHidden + kHiddenBytes;
static_assert(kOffSync % 256 == 0 && kOffAcc % 256 == 0 && kOffHidden % 256 == 0, "aligned regions");

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
struct DeviceScratch {
    std::once_flag once;
    uint8_t* ptr = nullptr;   // device address of this device's `scratch`
    int cus = 0;
    hipError_t error = hipSuccess;
};
DeviceScratch g_devices[kMaxDevices];

// Zeroes words [0, words) of the array except the control block, which block 0 writes
// whole: an empty queue sealed for `epoch`. `status` (the caller's word or the array's)
// starts at zero.
__global__ void noalloc_prepare_kernel(uint32_t* base, uint32_t words, uint32_t epoch, uint32_t* status) {
    const uint32_t first = (uint32_t)(kOffControl + sizeof(QueueControl)) / 4;
    for (uint32_t i = first + blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x)
        base[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < sizeof(QueueControl) / 4) {
        // QueueControl words: 0 ready_count, 2 total_count, 3 epoch, the rest zero
        base[kOffControl / 4 + threadIdx.x] = threadIdx.x == 3 ? epoch : 0u;
        if (threadIdx.x == 0) *status = 0u;
    }
}

DeviceScratch* device_scratch(hipError_t* error) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *error = e != hipSuccess ? e : hipErrorInvalidDevice;
        return nullptr;
    }
    DeviceScratch& d = g_devices[dev];
    std::call_once(d.once, [&d, dev] {
        void* p = nullptr;
        d.error = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));   // with device `dev` current
        if (d.error == hipSuccess) d.error = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (d.error == hipSuccess) d.ptr = static_cast<uint8_t*>(p);
    });
    *error = d.error;
    return d.error == hipSuccess ? &d : nullptr;
}

}  // namespace
}  // namespace lsamd

extern "C" int ls_hip_core_layer_noalloc(uint32_t width, uint32_t group_size, uint32_t batch, const void* cache,
                                         uint32_t cache_groups, const void* scales, uint32_t scale_groups,
                                         const ls_exec_desc* core, uint32_t core_count, const void* input,
                                         void* output, float* output32, uint32_t* status, void* stream) {
    using namespace lsamd;
    if (!width || width % 256 || !group_size || group_size > 256 || !batch || !cache || !scales || !cache_groups ||
        !scale_groups || !input || !output || (core_count && !core))
        return EINVAL;
    if (batch > kMaxBatch) return ENOTSUP;   // the dense (batch 5..32) path is not offered here
    if (width > kNaMaxWidth || core_count > kNaMaxUnits || core_count * group_size > kNaMaxNeurons) return ENOSPC;
    if (!variant_available(static_cast<int>(width))) return ENOTSUP;
    hipError_t e = hipSuccess;
    DeviceScratch* d = device_scratch(&e);
    if (!d) return static_cast<int>(e);
    int per_cu = 0;
    e = resident_workers(static_cast<int>(width), kEntryFused, static_cast<int>(batch), static_cast<int>(group_size),
                         &per_cu);
    if (e != hipSuccess) return static_cast<int>(e);
    if (per_cu < 1 || d->cus * per_cu < 2) return static_cast<int>(hipErrorInvalidConfiguration);

    uint8_t* base = d->ptr;
    const uint32_t units = core_count ? core_count : 1u;
    const uint32_t slot_words = sync_slot_words(units);
    // cleared in one pass: the control words, both ring slots and accumulator buffers
    // (their full extents) and the h rows this call uses
    const size_t used = kOffHidden + sizeof(uint64_t) * units * batch * group_size;

    MlpArgs a{};
    a.core = reinterpret_cast<const ExecDesc*>(core);
    a.core_count = core_count;
    a.qdesc = reinterpret_cast<const ExecDesc*>(base + kOffQueue);
    a.ready = reinterpret_cast<const uint32_t*>(base + kOffQueue);
    a.qmirror = reinterpret_cast<uint32_t*>(base + kOffQueue);
    a.control = reinterpret_cast<QueueControl*>(base + kOffControl);
    a.capacity = 0;
    a.x = static_cast<const uint16_t*>(input);
    a.cache = static_cast<const uint8_t*>(cache);
    a.staging = static_cast<const uint8_t*>(cache);
    a.scales = static_cast<const uint16_t*>(scales);
    a.hbuf = reinterpret_cast<uint64_t*>(base + kOffHidden);
    a.yacc = reinterpret_cast<unsigned long long*>(base + kOffAcc);
    a.y = static_cast<uint16_t*>(output);
    a.y32 = output32;
    a.sync = reinterpret_cast<uint32_t*>(base + kOffSync);
    a.status = status ? status : reinterpret_cast<uint32_t*>(base + kOffStatus);
    a.done = reinterpret_cast<uint32_t*>(base + kOffDone);
    a.width = width;
    a.group_size = group_size;
    a.slices = width / kDnCols;
    a.slot_words = slot_words;
    a.units_cap = units;
    a.slot_capacity = units;
    a.epoch = 1;
    a.seq = 1;   // every call clears the tags first, so one sequence value serves all calls
    a.batch_mode = 0;
    a.claim_batch = 0;
    a.batch = batch;
    a.spin_limit = 200000000ull;   // 2 s of the 100 MHz device clock
    const Bounds bounds{cache_groups, 0u, scale_groups};

    auto hs = static_cast<hipStream_t>(stream);
    uint32_t* words = reinterpret_cast<uint32_t*>(base);
    uint32_t nwords = static_cast<uint32_t>(used / 4);
    uint32_t grid = (nwords + kNaThreads - 1) / kNaThreads;
    if (grid > 1024) grid = 1024;
    uint32_t epoch = a.epoch;
    uint32_t* st = a.status;
    void* pargs[] = {&words, &nwords, &epoch, &st};
    e = hipLaunchKernel(reinterpret_cast<const void*>(&noalloc_prepare_kernel), dim3(grid), dim3(kNaThreads), pargs,
                        0, hs);
    if (e != hipSuccess) return static_cast<int>(e);
    const LaunchPlan plan{static_cast<int>(width), d->cus * per_cu - 1, kEntryFused};
    e = launch_layer(plan, a, bounds, hs);
    return e == hipSuccess ? 0 : static_cast<int>(e);
}
