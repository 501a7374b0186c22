// Kernel argument block shared by the host backend and the gfx950 kernels.
// Plain data only; passed by value to every launch.
#pragma once
#include <stdint.h>
#include "leanstream/execution_queue.h"

namespace lsamd {

using leanstream::runtime::ExecDesc;
using leanstream::runtime::QueueControl;

// Per-launch device synchronisation block ("ring slot"). Two slots alternate
// between consecutive launches of one backend; the last worker of launch n
// clears the slot that launch n+1 will use (the one launch n-1 dirtied).
enum SyncWord : uint32_t {
    kSyncExit = 0,       // workers that have finished
    kSyncPath = 1,       // 0 undecided, 1 claim path, 2 all-ready fast path
    kSyncClaimHead = 2,  // next unclaimed ready position (claim path)
    kSyncAbort = 3,      // set on queue error or spin timeout: every worker leaves
    kSyncClaims = 4,     // number of successful claims (claim path)
    kSyncEpochState = 5, // mirror: 0 not yet seen, 1 epoch published, 2 leave (error / abort / timeout)
    kSyncTotal = 6,      // mirror: final queue total_count
    kSyncReady = 7,      // mirror: published positions copied into qmirror
    kSyncTiles = 16,     // [kMaxSlices] completed down-projection tiles per column tile
};
constexpr uint32_t kMaxSlices = 64;
constexpr uint32_t kSyncUnits = kSyncTiles + kMaxSlices;  // [units] gate/up slices done per unit
// then [units] down tiles done per unit, then [units] claim log entries
inline uint32_t sync_slot_words(uint32_t units) { return kSyncUnits + 3 * units; }

// Phase stamps written by thread 0 of each worker when MlpArgs::stamps is set.
constexpr uint32_t kStampSlots = 32;
enum StampPhase : uint32_t {
    kStampEntry = 0, kStampXLoaded = 1, kStampFinish = 30, kStampExit = 31,
    kStampItemBase = 2,  // + 7 * item (items 0..3): start, gu done, siblings, dn done, stored, counted, reduced
};

// Status word bits (host-coherent, sticky until cleared by the host).
enum StatusBit : uint32_t { kStatusTimeout = 1u, kStatusQueueError = 2u, kStatusBadDescriptor = 4u };

// Arena extents used to validate descriptors on the device before any access.
struct Bounds {
    uint32_t cache_groups, staging_groups, physical_groups;
};

struct MlpArgs {
    // work
    const ExecDesc* core;         // device-visible core descriptors
    uint32_t core_count;
    const ExecDesc* qdesc;        // queue descriptors (final order)
    const uint32_t* ready;        // ready_indices (publication order)
    uint32_t* qmirror;            // device copy of published descriptors, in publication order [capacity][5]
    QueueControl* control;        // host-coherent control block
    uint32_t capacity;
    // data
    const uint16_t* x;            // fp16 [d]
    const uint8_t* cache;         // packed groups, slot-major
    const uint8_t* staging;
    const uint16_t* scales;       // fp16 [(physical*G + n)*3 + proj][d/128]
    float* hbuf;                  // fp32 [slot][G] intermediate silu(g)*u
    float* partial;               // fp32 [slot][d]
    uint16_t* y;                  // fp16 [d]
    float* y32;                   // optional fp32 [d] pre-rounding output
    uint32_t* executions;         // optional per-destination execution counters
    uint64_t* first_compute;      // optional per-destination start stamps (100 MHz clock)
    uint32_t* sync;               // base of the two ring slots
    uint32_t* status;             // host-coherent sticky status word
    uint32_t* claim_log;          // optional: per-claim (head | (len << 24)), in claim order
    uint32_t claim_log_cap;       // entries in claim_log
    uint64_t* stamps;             // optional: per-worker phase stamps [workers][kStampSlots] (100 MHz clock)
    // geometry / control
    uint32_t group_size;          // G
    uint32_t slices;              // S: work items per unit (G/S neurons, d/S columns each)
    uint32_t slot_words;          // words per ring slot
    uint32_t units_cap;           // max units (core + queue) the ring slot covers
    uint32_t slot_capacity;       // rows in hbuf/partial
    uint32_t epoch;
    uint32_t seq;                 // launch sequence number (selects the ring slot)
    uint32_t batch_mode;          // 1: wait for batch_epoch before consuming the queue
    uint64_t spin_limit;          // bounded waits, in 100 MHz ticks
};

}  // namespace lsamd
