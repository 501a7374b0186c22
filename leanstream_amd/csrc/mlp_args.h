// Kernel argument block shared by the host backend and the gfx950 kernels.
// Plain data only; passed by value to every launch.
#pragma once
#include <stdint.h>
#include "leanstream/execution_queue.h"

namespace lsamd {

using leanstream::runtime::ExecDesc;
using leanstream::runtime::QueueControl;

// Per-launch device synchronisation block ("ring slot"). Two slots alternate between
// consecutive launches of one backend; launch n clears the slot launch n+1 will use
// (the one launch n-1 dirtied) while it runs. Every polled or contended word sits on
// its own 128-byte line.
constexpr uint32_t kLine = 32;  // 32-bit words per 128-byte line
enum SyncWord : uint32_t {
    kSyncExit = 0 * kLine,        // groups of workgroups (kSyncExitGroups) that have finished
    kSyncEpoch = 1 * kLine,       // mirror: state | path << 2 | total << 4 (state 0 unseen, 1 ok, 2 leave)
    kSyncReady = 2 * kLine,       // mirror: published positions copied into qmirror
    kSyncClaimHead = 3 * kLine,   // next unclaimed ready position (claim path)
    kSyncAbort = 4 * kLine,       // set on queue error or spin timeout: every worker leaves
    kSyncClaims = 5 * kLine,      // number of successful claims (claim path)
};
constexpr uint32_t kSyncExitGroups = 8 * kLine;  // + g * kLine (g < 8): workgroups blk % 8 == g finished
constexpr uint32_t kSyncUnits = 16 * kLine;      // + u * kLine: down tiles of unit u done
// (counted only for the optional execution counters)
inline uint32_t sync_slot_words(uint32_t units) { return kSyncUnits + units * kLine; }

// Deterministic compact reduction. Every (unit, column tile) contribution v is added
// atomically into one 64-bit word per output column:
//     word += (round(v * 2^20) + 2^39) + 2^52
// bits 0..51 hold the biased fixed-point sum, bits 52..63 count the contributions.
// Integer addition is associative, so the final word -- and the fp32 / fp16 output
// decoded from it -- does not depend on the order in which units finish. The atomic
// that brings a column's count to U (the number of destination rows) returns the
// complete sum, so that lane writes the output column directly.
// Bounds: |v| < 2^19 per contribution, U < 4096 rows; resolution 2^-20.
constexpr float kAccScale = 1048576.0f;                 // 2^20
constexpr double kAccInv = 1.0 / 1048576.0;
constexpr long long kAccBias = 1ll << 39;
constexpr unsigned long long kAccOne = 1ull << 52;
constexpr unsigned long long kAccValueMask = kAccOne - 1;
constexpr uint32_t kMaxRowsReduced = 4095;
// 64-bit words between consecutive column accumulators. Dense (1): a wave's 64-column
// atomic instruction is four line requests; one line per column made it 64 requests and
// a Ministral-8B layer twice as slow (the atomics are bound by request count).
constexpr uint32_t kAccStride = 1;
constexpr uint32_t kDnCols = 256;  // columns of one down-projection item (two scale blocks)
constexpr uint32_t kMaxBatch = 4;  // batch rows of one launch (x of every row is kept in LDS)
constexpr uint32_t kMaxDenseBatch = 32;   // batch rows of the dense (matrix-core) path
constexpr uint32_t kDenseSplits = 16;     // unit splits of its down projection

constexpr uint32_t pack_epoch(uint32_t state, uint32_t path, uint32_t total) { return state | (path << 2) | (total << 4); }

// Claim log (candidates that consume the queue in groups of claim_batch positions, the
// ready pairs of backends/triton/persistent.py:63-90): one entry per range a workgroup
// takes, in the order the ranges were taken: {first position, count, ready count the
// claim was made against, worker}. On the all-ready path the ranges are the static pairs
// of descriptor indices (2w + 2kW, +1) and the third word is kClaimStatic.
constexpr uint32_t kClaimLogWords = 4;
constexpr uint32_t kClaimStatic = 0xFFFFFFFFu;

// Phase stamps (100 MHz clock) written by lane 0 of every wave when MlpArgs::stamps is
// set: stamps[(block * 4 + wave) * kStampSlots + phase]; 0 = the wave never got there.
constexpr uint32_t kStampSlots = 32;
enum StampPhase : uint32_t {
    kStampEntry = 0,
    kStampDescs = 1,         // the wave's first descriptors have arrived
    kStampCoreDone = 2, kStampEpoch = 3, kStampQueueDone = 4,
    kStampFirstData = 5,     // first item's weights have landed (staged walk)
    kStampFirstDone = 6,     // first gate/up item computed, h published
    kStampSecondData = 7,    // second item's weights have landed (staged walk)
    kStampHReady = 8,        // first down item: h of its unit complete
    kStampDnComputed = 9,    // first down item computed (atomics issued next)
    kStampDrained = 10,      // last column additions returned
    kStampMirrorEpoch = 12,  // mirror: epoch word published
    kStampMirrorDone = 13,   // mirror: every worker counted out
    kStampExit = 31,
};

// ---------------------------------------------------------------------------------
// Layer chains (chain_mlp.hip): one persistent launch computes a sequence of layers whose
// records the host writes into pinned memory. Layer i publishes its hidden state
// fp16(residual_i + fp16(y_i)) (the epilogue's publication) as tagged words inside the grid;
// layer i + 1 takes it as its residual and, as its input, either the hidden state itself or
// its RMSNorm times the layer's norm weight. A wave streams the items of later layers into
// its LDS slots while earlier layers finish, and waits for a layer's input only before its
// first computation.
// ---------------------------------------------------------------------------------
struct ChainRec {                 // one layer; 128 bytes (whole lines), 32 words
    const ExecDesc* core;         // words 0-1: core descriptors (device-visible)
    const uint8_t* cache;         // 2-3
    const uint8_t* staging;       // 4-5
    const uint16_t* scales;       // 6-7
    const uint16_t* x;            // 8-9: fp16 [d] input of a layer that is not chained
    const uint16_t* residual;     // 10-11: fp16 [d] residual of a layer that is not chained (null: x)
    const uint16_t* norm_weight;  // 12-13: chained layer: input = RMSNorm(previous hidden) * weight
    uint16_t* y;                  // 14-15: fp16 [d]
    float* y32;                   // 16-17: optional fp32 [d]
    uint16_t* hidden;             // 18-19: optional fp16 [d]: fp16(residual + y)
    uint32_t* hidden_flag;        // 20-21: optional: epoch (system release) once the layer is done
    uint32_t* bell;               // 22-23: optional: += 1 after the flag
    uint32_t core_count;          // 24
    uint32_t cache_groups;        // 25
    uint32_t staging_groups;      // 26
    uint32_t physical_groups;     // 27
    uint32_t epoch;               // 28
    uint32_t seq;                 // 29: sequence of the layer (h tags, hidden-word tags, done word)
    uint32_t chained;             // 30: 1 = the input comes from the previous layer's hidden state (seq - 1)
    float norm_eps;               // 31
};
static_assert(sizeof(ChainRec) == 128, "a chain record is one 128-byte line");
constexpr uint32_t kChainRecWords = 32;

// Chain synchronisation block (device memory, kChainSyncWords words; zero between launches).
constexpr uint32_t kChainMaxLayers = 512;   // layers of one launch
enum ChainWord : uint32_t {
    kChainAvail = 1 * kLine,      // records mirrored into the device ring
    kChainLayersDone = 2 * kLine, // layers of the launch whose waves have all counted out
    // kSyncAbort as in a ring slot
    kChainExit = 8 * kLine,       // + (layer * 8 + g) * kLine: waves of workgroups blk % 8 == g out of the layer
};
constexpr uint32_t kChainSyncWords = kChainExit + kChainMaxLayers * 8 * kLine;

struct ChainArgs {
    const ChainRec* host_recs;    // pinned host memory: records of the launch
    ChainRec* recs;               // device copy (the supervisor mirrors the records)
    uint32_t count;               // layers of the launch
    uint32_t* csync;              // chain synchronisation block
    uint64_t* hbuf;               // tagged h [slot_capacity][64] (seq << 32 | fp32 bits)
    unsigned long long* yacc;     // [2][d] fixed-point accumulators, buffer seq & 1; the lane that
                                  // completes a column resets its word
    uint32_t* xtag;               // [2][d] hidden words fp16 | tag << 16, buffer seq & 1
    uint32_t* status;             // host-coherent sticky status word
    uint32_t* done;               // host-coherent: sequence of the last layer whose waves all counted out
    uint64_t* stamps;             // optional [count][grid * 4][kStampSlots]
    uint32_t width;
    uint32_t slot_capacity;
    uint32_t grid;                // workers + the supervisor
    uint64_t spin_limit;
};
// Hidden-word tag of a sequence: never 0, period 65535. The backend clears the tagged words
// at least every 32768 sequences, so no stored tag can match a later sequence.
constexpr uint32_t chain_tag(uint32_t seq) { return seq % 0xFFFFu + 1u; }
constexpr uint32_t kChainClearPeriod = 32768;

// Chain phase stamps (per layer and wave; kStampFirstData, kStampFirstDone, kStampHReady,
// kStampDnComputed, kStampDrained as above).
enum ChainStamp : uint32_t {
    kChainStampIssue = 14,        // the wave's first item of the layer issued
    kChainStampXWait = 15,        // the wave starts waiting for the layer's input
    kChainStampXIn = 16,          // the wave's part of the input staged in LDS
    kChainStampCountOut = 17,     // the wave counted out of the layer
    kChainStampDone = 18,         // supervisor: every wave out of the layer
};

// Status word bits (host-coherent, sticky until cleared by the host).
enum StatusBit : uint32_t {
    kStatusTimeout = 1u, kStatusQueueError = 2u, kStatusBadDescriptor = 4u, kStatusRange = 8u,
    kStatusQueueUnconsumed = 16u,   // a dense (batch > kMaxBatch) launch's layer published queue entries
};

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
    const uint16_t* x;            // fp16 [batch][d]
    const uint8_t* cache;         // packed groups, slot-major
    const uint8_t* staging;
    const uint16_t* scales;       // fp16 [(physical*G + n)*3 + proj][d/128]
    uint64_t* hbuf;               // [slot][batch][G] h = fp16(silu(g)*u) as fp32 bits | launch seq << 32
    unsigned long long* yacc;     // [2][batch][d][kAccStride] packed accumulators (see kAccOne), buffer (seq & 1)
                                  // per launch
    uint16_t* y;                  // fp16 [batch][d]
    float* y32;                   // optional fp32 [batch][d] pre-rounding output
    uint32_t* executions;         // optional per-destination execution counters
    uint64_t* first_compute;      // optional per-destination start stamps (100 MHz clock)
    uint32_t* sync;               // base of the two ring slots
    uint32_t* status;             // host-coherent sticky status word
    uint32_t* done;               // host-coherent: the last workgroup of a launch stores seq
    uint32_t* claim_log;          // optional: kClaimLogWords words per claimed range, in claim order
    uint32_t claim_log_cap;       // entries (ranges) claim_log holds
    uint64_t* stamps;             // optional: per-worker phase stamps [workers][kStampSlots] (100 MHz clock)
    // geometry / control
    uint32_t width;               // d
    uint32_t group_size;          // G
    uint32_t slices;              // down-projection items per unit (d / kDnCols)
    uint32_t slot_words;          // words per ring slot
    uint32_t units_cap;           // max units (core + queue) the ring slot covers
    uint32_t slot_capacity;       // destination rows (rows of hbuf)
    uint32_t epoch;
    uint32_t seq;                 // launch sequence number (selects the ring slot)
    uint32_t batch_mode;          // 1: wait for batch_epoch before consuming the queue
    uint32_t dn_tile;             // staged walk's down items: 0 = its own choice (quarters when every item
                                  // gets a wave, d <= 2048), 256 = whole 256-column tiles
    uint32_t claim_batch;         // progressive path: 0 = every wave takes its stripe of the queue
                                  // positions, waiting for each to be published; n > 0 = workgroups
                                  // claim up to n ready positions at a time
    uint32_t batch;               // rows of x / y (1 .. kMaxBatch; dense path: kMaxBatch + 1 .. kMaxDenseBatch)
    uint32_t grid;                // workgroups of a persistent launch (workers + the mirror)
    uint32_t pack;                // units per down item: 64 / G for the packed kernels, else 1 (set per launch)
    // dense path (batch > kMaxBatch): x is bf16 [batch][d]
    uint16_t* h16;                // fp16 h rows [32][slot_capacity * G]
    float* dpart;                 // fp32 down-projection partial rows [dsplits][32][d]
    uint16_t* x16;                // x as fp16 MFMA A fragments, 32 rows x d (dense_x_kernel; rows >= batch zero)
    uint32_t dsplits;
    uint64_t spin_limit;          // bounded waits, in 100 MHz ticks
    // the layer's epilogue, run by the fused launch's last workgroup once every worker is out
    // (hidden == nullptr: none); the fields of EpilogueArgs (mlp_launch.h) of the same names
    const uint16_t* residual;     // fp16 [batch][d]
    uint16_t* hidden;             // fp16 [batch][d]
    uint32_t* hidden_flag;
    const uint16_t* norm_weight;  // optional fp16 [d]
    uint16_t* norm_out;           // fp16 [batch][d] (with norm_weight)
    uint32_t* norm_flag;
    uint32_t* bell;
    float norm_eps;
};

}  // namespace lsamd
