// Device-side data layout shared by the HIP kernels (leo_kernels.hip) and the
// host runtime (leo_runtime.hip). One "lane" is one independent runtime
// trajectory: a logical story worker (training.rs:1669-1683) or the canonical
// runtime itself. Arrays are structure-of-arrays in HBM, except the per-neuron
// state, which is one 64-byte record per neuron (NeuronField).
#ifndef LEO_DEVICE_H
#define LEO_DEVICE_H

#include <stdint.h>

#include "fast_div.h"
#include "leo_hip_abi.h"

// Device memory pointers in the structures below are global-address-space
// pointers in the kernels' device code (global_* rather than flat memory
// instructions, which would also count against the LDS wait counter); every
// other view, the host runtime included, sees plain pointers of the same size.
#if defined(__HIP_DEVICE_COMPILE__) && defined(LEO_KERNEL_TRANSLATION_UNIT)
#define LEO_GLOBAL __attribute__((address_space(1)))
#else
#define LEO_GLOBAL
#endif

namespace leo {

constexpr uint32_t kSymbols = 258;
constexpr uint32_t kOutputs = 257;
// Neuron-major output row: 257 weights padded to 1,152 B, nine whole 128-byte
// cache lines, so every row starts line-aligned and each learning-signal chunk
// load reads exactly one line (a 1,040 B row would straddle lines).
constexpr uint32_t kOutStride = 288;
constexpr uint32_t kEndIndex = 256;
constexpr uint32_t kRing = 9;             // delay ring: max delay 8 + 1 (runtime.rs:200-208)
constexpr uint32_t kBucketSets = kRing;   // delivery bucket sets of a lane with one-barrier frozen runs
constexpr uint32_t kMaxOrder = 16;        // config.rs:452-456
constexpr uint32_t kThreads = 256;        // threads per workgroup
constexpr uint32_t kMaxBlockNeurons = 1024;
constexpr uint32_t kWaveSize = 64;
constexpr uint32_t kWavesPerGroup = kThreads / kWaveSize;
constexpr uint32_t kMaxWaves = 1024;     // selecting waves per lane (workgroups per lane <= 256)
constexpr uint32_t kMaxLaneWgs = kMaxWaves / kWavesPerGroup;  // workgroups per lane
constexpr uint32_t kFlagWords = 32;       // a barrier arrival flag per 128-byte L2 line
constexpr uint32_t kXcds = 8;            // accelerator complex dies of an MI355X (workgroups dispatched round-robin)

// Touched-neuron bitmap: each block owns ceil(neurons_per_block/32) words,
// so no word is shared by two blocks (and no two selecting waves).
inline __host__ __device__ uint32_t block_words(uint32_t neurons_per_block) { return (neurons_per_block + 31) / 32; }

// Phase-2 window of a selecting wave: touched neurons folded and ranked at
// once (at least one whole block, so a block never spans two windows).
constexpr uint32_t kGroupBlocks = 64;    // blocks per bitmap load round
constexpr uint32_t kWordsPerLane = 8;    // bitmap words per lane per load round
// Delivery entries per target at fixed places (one 64-byte run per target,
// read with the neuron record); further entries go to the target's overflow
// range. Four covers nearly every target of a sparse tick.
constexpr uint32_t kFixedEntries = 4;
inline __host__ __device__ uint32_t window_capacity(uint32_t neurons_per_block) {
    return neurons_per_block > 256 ? neurons_per_block : 256;
}
// Per-wave bytes of the window: u64 keys and u32 entries (capacity each),
// block cutoff keys (G), block starts (G+1), block candidate counts and
// staged winner offsets (G each), and
// the group's bitmap words with their list positions (64*kWordsPerLane each).
inline __host__ __device__ size_t window_bytes(uint32_t neurons_per_block) {
    const size_t c = window_capacity(neurons_per_block);
    const size_t words = 64 * kWordsPerLane;
    return (c * 12 + kGroupBlocks * 8 + (kGroupBlocks + 1) * 4 + kGroupBlocks * 8 + words * 8 + 15) / 16 * 16;
}

// Learning-signal row staging of one wave: 64 output rows, one 128-byte line
// (32 floats) of each at a time, rows padded to 33 floats (conflict-free
// column reads).
constexpr uint32_t kStageRowFloats = 33;
constexpr size_t kStageBytes = 64 * kStageRowFloats * 4;

// Radix counts of a wave's deep-bucket sort, after its window: the current
// pass's 256 scatter offsets and the next pass's 256 counts.
constexpr size_t kDeepHistBytes = 2 * 256 * 4;

// Per-wave share of the dynamic LDS: the phase-2 window (reused by the
// learning-signal staging), then the deep-bucket histogram.
inline __host__ __device__ size_t wave_window_bytes(uint32_t neurons_per_block) {
    const size_t w = window_bytes(neurons_per_block);
    return ((w > kStageBytes ? w : kStageBytes) + 15) / 16 * 16;
}
inline __host__ __device__ size_t wave_lds_bytes(uint32_t neurons_per_block) {
    return wave_window_bytes(neurons_per_block) + kDeepHistBytes;
}

// Dynamic LDS of the step kernel: one share per wave. The binding-cap global
// selection reuses it: the selecting waves' first winner positions
// (kSelectStartsBytes), then keys -- up to kMaxBlockNeurons sorted in place,
// or a tile of select_tile_keys() keys streamed past every key of the lane.
constexpr size_t kSelectStartsBytes = ((kMaxWaves + 1) * 4 + 15) / 16 * 16;
inline size_t step_lds_bytes(uint32_t neurons_per_block) {
    const size_t lists = static_cast<size_t>(kWavesPerGroup) * wave_lds_bytes(neurons_per_block);
    const size_t sort = kSelectStartsBytes + static_cast<size_t>(kMaxBlockNeurons) * 8;
    return ((lists > sort ? lists : sort) + 15) / 16 * 16;
}
inline uint32_t select_tile_keys(uint32_t neurons_per_block) {
    const size_t keys = (step_lds_bytes(neurons_per_block) - kSelectStartsBytes) / 8;
    return static_cast<uint32_t>(keys / kThreads * kThreads);
}

// Step flags (per scheduled step).
enum : uint32_t {
    kStepFrozen = 1u << 0,        // Permission::Frozen
    kStepLearnTrace = 1u << 1,    // learning_trace_enabled (!frozen)
    kStepContext = 1u << 2,       // context enabled (frozen, or survived dropout)
    kStepAllocate = 1u << 3,      // context allocation allowed
    kStepLearn = 1u << 4,         // target present and strength > 0
    kStepOutput = 1u << 5,        // compute logits/probabilities
    kStepNeuralLoss = 1u << 6,    // also record the neural-only loss terms (runtime.rs:1119, 1151-1167)
    // Delays whose events this step's tick may deliver when it emits them (a
    // one-barrier frozen step): bit kStepEarlyShift + log2(delay) is set when
    // the arrival step lies in the same launch and runs no learning trace
    // (the delivery of a trace step activates the delivering slots' traces).
    kStepEarlyShift = 8,
    kStepEarlyMask = 0xfu << 8,
};

// One scheduled step, prepared by the host from the story bytes
// (training.rs:1747-1757) -- the role of LeoPersistentStep (cuda.rs:398-406).
struct StepParams {
    uint32_t symbol;
    int32_t target_index;          // dense output class or -1
    uint32_t flags;
    float supervised_strength;     // strength * target weight
    float strength;                // permission strength (inhibitory homeostasis)
    float plasticity_scale;
};

// Per-step record written by the device (the role of CudaTrainingStepRecord,
// cuda.rs:354-370). The loss itself is -ln(max(p_target,1e-12)) on the host.
struct StepRecord {
    float p_target;
    float population_inhibition;
    uint32_t predicted;
    uint32_t active;
    uint32_t suprathreshold;
    uint32_t block_selected;
    uint32_t clipped;
    uint32_t context_cells;
    uint32_t context_probes;
    uint32_t context_applied;
    uint32_t eligible_rec;
    uint32_t eligible_in;
    uint32_t error_code;
    // work counters of the step (for the algorithmic byte model)
    uint32_t events;            // recurrent events delivered
    uint32_t touched;           // neurons touched
    uint32_t scanned_rec;       // eligible recurrent slots updated
    uint32_t scanned_in;        // eligible input slots updated
    uint32_t destinations;      // learning destinations
    uint32_t active_inhibitory; // active inhibitory sources
    uint32_t learning_slots;    // eligible slots whose update the step applies (nonzero eligibility)
    // neural-only loss terms (kStepNeuralLoss): the maximum of the logits
    // before the context contribution, the serial sum of exp(logit - max),
    // and the target's logit; the loss is max + ln(sum) - logit
    float neural_max;
    float neural_sum;
    float neural_target;
    uint32_t deep_folds;        // buckets of more than 8 deliveries: ranked in registers (low 16 bits),
                                // radix-sorted (high 16 bits)
};

// Device numerical guard codes (the reference's sticky error_flag 1-7,
// cuda_kernels.cu:3276-3588).
enum : uint32_t {
    kErrOutput = 1, kErrBias = 2, kErrContextProjection = 3, kErrContextEmbedding = 4,
    kErrRecurrent = 5, kErrInput = 6, kErrInhibitory = 7, kErrCapacity = 8, kErrBarrier = 9,
};
constexpr uint32_t kNoFail = 0xffffffffu;

// Device-resident scalars of a lane that persist across launches.
struct LaneControl {
    uint32_t tick;                   // current_tick
    float population_inhibition;
    uint32_t parity;                 // which eligible list is current
    uint32_t rec_count[2];
    uint32_t in_count[2];
    uint32_t dest_epoch;             // learning-destination epoch
    uint32_t dest_count;             // entries of this step's destination list
    uint32_t rec_learn_count;        // entries of this step's recurrent learning-slot list
    uint32_t in_learn_count;         // entries of this step's input learning-slot list
    uint32_t history_len;
    uint32_t history[kMaxOrder];
    uint32_t ctx_count;
    uint32_t ctx_probes;
    uint32_t ctx_applied;
    uint32_t ctx_slots[kMaxOrder];
    float ctx_scales[kMaxOrder];
    uint32_t block_selected;
    uint32_t clipped;
    float pop_cutoff;
    uint32_t active_count;
    uint32_t bias_dirty;
    uint32_t ctx_out_dirty;
    // Sticky device guard: the first guard a step trips (kErr* code). A lane
    // whose word is set runs no further steps, in this launch or in later
    // ones, until the host has read the code and clears it.
    uint32_t error_code;
    uint32_t error_step;             // schedule index (within its launch) of the step that tripped it
    uint32_t bias_fail;              // first output whose bias this learning step makes non-finite, or kNoFail
    uint32_t ring_tick[kRing];       // tick whose active set ring slot holds (UINT32_MAX = empty)
    uint32_t ring_count[kRing];      // active count of that tick
    uint32_t ring_early[kRing];      // delays (bit = delay) of that tick's events already delivered at emission
    // The barrier counter has a 128-byte L2 line of its own: its polls and
    // arrivals would otherwise queue behind the per-step counter atomics and
    // the step record's stores to the same line.
    alignas(128) uint32_t barrier;   // lane-group barrier arrival counter
    uint32_t abort;
    uint32_t xcc_mask;               // XCDs the lane's workgroups run on (bit per XCD)
};

// The words a launch's workgroups synchronise through, zero when the launch
// starts: a lane's own (LaneControl::barrier, abort, xcc_mask, cleared before
// each launch), or a planned launch's own zeroed copy.
struct LaunchWords {
    uint32_t barrier;
    uint32_t abort;
    uint32_t xcc_mask;
};
static_assert(offsetof(LaneControl, abort) == offsetof(LaneControl, barrier) + offsetof(LaunchWords, abort) &&
                  offsetof(LaneControl, xcc_mask) == offsetof(LaneControl, barrier) + offsetof(LaunchWords, xcc_mask),
              "a lane's launch words are LaneControl::barrier, abort, xcc_mask");

// Per-tick work counters of the step records, kept per workgroup: workgroup p
// adds to the words of its own 128-byte line (p * kFlagWords + 2 * kind +
// tick parity), and a recording wave sums the P lines. (One shared line
// queues every workgroup's atomics on one L2 channel ahead of each barrier.)
enum CounterKind : uint32_t {
    kCTouched,      // touched neurons
    kCSupra,        // suprathreshold neurons
    kCEvents,       // delivered events
    kCDest,         // learning destinations
    kCInhibitory,   // active inhibitory sources
    kCScanRec,      // eligible recurrent slots scanned
    kCScanIn,       // eligible input slots scanned
    kCLearn,        // learning slots listed
    kCDeep,         // deep bucket folds (StepRecord::deep_folds)
    kCounterKinds
};
static_assert(2 * kCounterKinds <= kFlagWords, "a workgroup's counters fit its line");

// Learned parameters of a lane (private copy for story lanes, the canonical
// image for the canonical runtime).
struct LaneParams {
    float LEO_GLOBAL* threshold;        // N
    float LEO_GLOBAL* rec_weight;       // N*S (slot = src*S + j)
    float LEO_GLOBAL* in_weight;        // 258*F
    float LEO_GLOBAL* out_w;            // N * kOutStride, neuron-major
    float LEO_GLOBAL* bias;             // kOutStride
    uint64_t LEO_GLOBAL* ctx_keys;      // slots
    float LEO_GLOBAL* ctx_emb;          // slots * E
    uint32_t LEO_GLOBAL* ctx_obs;       // slots
    float LEO_GLOBAL* ctx_out;          // 257 * E, output-major
};

// One tensor copied to several lanes (leo_broadcast): the source is read once.
constexpr uint32_t kMaxBroadcast = 64;
struct Broadcast {
    const uint4 LEO_GLOBAL* src;
    uint64_t vectors;                    // 16-byte vectors
    uint32_t count;                      // destinations
    uint4 LEO_GLOBAL* dst[kMaxBroadcast];
};

// Words of a neuron's state record.
enum NeuronField : uint32_t {
    kNMembrane = 0,
    kNActivation = 1,
    kNFatigue = 2,
    kNAdapt0 = 3,       // fast, medium, slow adaptation
    kNBranch0 = 6,      // branch accumulators 0..3 (excitatory, inhibitory, temporal, gate)
    kNLastTick = 10,
    kNRefractory = 11,  // refractory_until
    kNTouched = 12,     // touched epoch: tick+1 when folded (touched) at tick
    kNSelected = 13,    // selected epoch: tick+1 when selected this tick
    kNSpare = 14,       // unused (bucket counts live in LaneDesc::bucket_count)
    kNDestEpoch = 15,   // learning-destination claim epoch
};
constexpr uint32_t kNeuronWords = 16;

// Words of a synapse slot's trace record: the branch, membrane and fatigue
// sensitivities, the three adaptation sensitivities, the eligibility, and the
// tick they were last brought to (u32 bits). One slot's trace is two 16-byte
// quarters of one record.
enum TraceField : uint32_t {
    kTBranch = 0, kTMembrane = 1, kTFatigue = 2, kTAdapt0 = 3, kTEligibility = 6, kTLast = 7,
};
constexpr uint32_t kTraceWords = 8;

// Trace slot marks: a clean slot (0) has not been written since the last
// reset and holds zeros; a listed slot is on the eligible list; a dropped
// slot has left the list and keeps its (sub-epsilon) values.
constexpr uint8_t kMarkClean = 0, kMarkListed = 1, kMarkDropped = 2;

// Everything a kernel needs to run one lane.
struct LaneDesc {
    LaneParams p;
    LaneControl LEO_GLOBAL* ctl;
    // kMaxLaneWgs * kFlagWords: workgroup p's barrier arrival epoch at word
    // p * kFlagWords (cleared by workgroup p before the launch's first barrier)
    uint32_t LEO_GLOBAL* barrier_flags;
    uint32_t LEO_GLOBAL* wg_counts;  // kMaxLaneWgs * kFlagWords: per-workgroup tick counters (CounterKind)
    // neuron state (N)
    // neuron state (N records of kNeuronWords words, fields NeuronField): what
    // one touched neuron needs shares one 64-byte record
    uint32_t LEO_GLOBAL* neuron;
    uint32_t LEO_GLOBAL* touched_list;  // N: per selecting wave, its range's touched neurons (see wave_touched)
    float LEO_GLOBAL* learning_signal;
    uint32_t LEO_GLOBAL* dest_list;     // N: this step's claimed learning destinations (LaneControl dest_count)
    // this step's learning slots: kept eligible slots whose weight update can
    // change the weight (nonzero eligibility), listed by the eligibility phase
    uint32_t LEO_GLOBAL* rec_learn;     // NS (LaneControl rec_learn_count)
    uint32_t LEO_GLOBAL* in_learn;      // NI (LaneControl in_learn_count)
    // Delivery buckets in bucket_sets sets (1, or kBucketSets on a lane that
    // takes frozen runs with one barrier per step): the deliveries of tick t
    // go to set t % bucket_sets, so events emitted up to 8 ticks ahead wait
    // in their own set while the current tick's set is folded.
    uint64_t LEO_GLOBAL* bucket;        // per set: 2 words per entry: delivery-order key, value bits;
                                        // kFixedEntries per target first, then the overflow ranges
    uint32_t LEO_GLOBAL* bucket_count;  // per set: N entry counts (nonzero only with the target's touched bit set)
    uint64_t bucket_stride;             // words of `bucket` per set
    uint64_t LEO_GLOBAL* shadow;        // 2 words per entry: the radix sort's second buffer (shadow_offset)
    // block selection
    uint32_t LEO_GLOBAL* range_winners; // blocks * max_active_per_block: winners of each selecting wave's block
                             // range in block order, compacted from the row of its first block
    float LEO_GLOBAL* range_winner_act; // same layout: activation of each winner
    float LEO_GLOBAL* block_cutoff;     // blocks
    uint32_t LEO_GLOBAL* block_epoch;   // blocks: tick+1 when the block's selection above is current
    uint32_t LEO_GLOBAL* touched_bits;  // per set, blocks * block_words: neurons with deliveries at the set's
                                        // tick, cleared by phase 2
    uint32_t touched_stride;            // words of `touched_bits` per set
    uint32_t bucket_sets;               // 1 or kBucketSets
    uint32_t LEO_GLOBAL* wave_total;    // 2 * kMaxWaves, by tick parity: block winners of each selecting
                                        // wave's block range
    uint32_t LEO_GLOBAL* wave_touched;  // kMaxWaves: touched neurons of each selecting wave's range, listed in
                                        // touched_list from the range's first neuron on
    // ring: per slot, up to max_active_global active neurons, activation, and S snapshot values each
    uint32_t LEO_GLOBAL* ring_active;   // kRing * cap
    float LEO_GLOBAL* ring_act;         // kRing * cap
    float LEO_GLOBAL* ring_value;       // kRing * cap * S
    uint32_t LEO_GLOBAL* ring_edge;     // kRing * cap * S: packed synapse of each snapshot value (target, delay, branch)
    // recurrent traces (N*S): branch, membrane, fatigue, 3 adaptation sensitivities, eligibility
    float LEO_GLOBAL* rec_trace;        // NS records of kTraceWords (TraceField)
    uint8_t LEO_GLOBAL* rec_mark;       // NS: kMark*
    uint32_t LEO_GLOBAL* rec_list;      // 2 * NS
    // input traces (258*F)
    float LEO_GLOBAL* in_trace;         // NI records of kTraceWords (TraceField)
    uint8_t LEO_GLOBAL* in_mark;        // NI: kMark*
    uint32_t LEO_GLOBAL* in_list;       // 2 * NI
    // readout
    float LEO_GLOBAL* logits;           // kOutStride
    float LEO_GLOBAL* probs;            // kOutStride
    float LEO_GLOBAL* errors;           // kOutStride
    float LEO_GLOBAL* ctx_latent;       // E
    // change tracking bitmaps (ParameterChanges)
    uint32_t LEO_GLOBAL* ch_threshold;  // ceil(N/32)
    uint32_t LEO_GLOBAL* ch_rec;        // ceil(NS/32)
    uint32_t LEO_GLOBAL* ch_in;         // ceil(NI/32)
    uint32_t LEO_GLOBAL* ch_out;        // ceil(N/32)
    uint32_t LEO_GLOBAL* ch_ctx;        // ceil(slots/32)
    // schedule for the current launch
    const StepParams LEO_GLOBAL* steps;
    StepRecord LEO_GLOBAL* records;
    uint32_t step_count;
    uint32_t pad;
    // where the launch's first thread stores the lane's outcome of the
    // previous launch (error code, error step, bias fail, tick) before this
    // launch can change it, for a host that reads the outcomes of a queue of
    // launches at once; null: nowhere
    uint32_t LEO_GLOBAL* outcome;
    LaunchWords LEO_GLOBAL* launch;  // this launch's barrier words
    // phase profile (profiling kernel only): per phase, summed wall-clock ticks of
    // workgroup 0's own work [0..kPhases) and of its barrier wait [kPhases..2*kPhases)
    unsigned long long LEO_GLOBAL* phase_profile;
};

constexpr uint32_t kPhases = 8;

// Read-only model data shared by every lane.
struct SharedModel {
    const float LEO_GLOBAL* excitability;
    const uint8_t LEO_GLOBAL* neuron_type;
    const uint32_t LEO_GLOBAL* rec_target;
    const uint8_t LEO_GLOBAL* rec_branch;
    const uint8_t LEO_GLOBAL* rec_delay;
    const uint32_t LEO_GLOBAL* in_target;
    const uint8_t LEO_GLOBAL* in_branch;
    const uint64_t LEO_GLOBAL* bucket_offset;   // N+1
    const uint64_t LEO_GLOBAL* shadow_offset;   // N+1: each deep-capable target's shadow range (entries)
    const uint32_t LEO_GLOBAL* rec_edge;        // N*S: pack_edge(target, delay, branch) of each recurrent slot
    const uint32_t LEO_GLOBAL* in_edge;         // 258*F: pack_edge(target, 1, branch) of each input slot
};

// A recurrent synapse packed into one word: target (28 bits), log2 of the
// delay (1, 2, 4 or 8) and the branch. The model validation guarantees the
// ranges; neuron_count is limited to 2^28.
constexpr uint32_t kEdgeTargetBits = 28;
constexpr uint32_t kMaxPackedNeurons = 1u << kEdgeTargetBits;
inline __host__ __device__ uint32_t pack_edge(uint32_t target, uint32_t delay, uint32_t branch) {
    const uint32_t log2_delay = delay >= 8 ? 3u : delay >= 4 ? 2u : delay >= 2 ? 1u : 0u;
    return target | (log2_delay << kEdgeTargetBits) | (branch << (kEdgeTargetBits + 2));
}
inline __host__ __device__ uint32_t edge_target(uint32_t e) { return e & (kMaxPackedNeurons - 1); }
inline __host__ __device__ uint32_t edge_delay(uint32_t e) { return 1u << ((e >> kEdgeTargetBits) & 3u); }
inline __host__ __device__ uint32_t edge_branch(uint32_t e) { return e >> (kEdgeTargetBits + 2); }

// Deep delivery buckets (more entries in one tick than the in-register
// sort network takes) are folded by the whole wave after a sort of the
// bucket by delivery key (delay class, the emitting neuron's active rank, its
// synapse slot; or class 4 and the input slot), which is unique per entry, so
// each branch's accumulator receives its values in the reference's delivery
// order (runtime.rs:605-639). Up to kDeepRegisterEntries entries are ranked in
// registers; larger buckets, which only targets of that capacity can have, go
// through an LSD radix sort with 8-bit digits between the bucket and the
// target's shadow range, on a compacted key of the significant fields.
constexpr uint32_t kDeepRegisterEntries = 128;
constexpr uint32_t kDeepMaxPasses = 8;
struct DeepSortPlan {
    uint32_t rank_bits;                   // bits of the rank field (active rank or input slot)
    uint32_t slot_bits;                   // bits of the synapse-slot field
    uint32_t passes;                      // radix passes
    uint32_t shift[kDeepMaxPasses];       // digit positions in the sort key, least significant first
    uint32_t bits[kDeepMaxPasses];        // digit widths (<= 8)
};
// Compacted sort key of a bucket entry, ordered as the delivery key: class,
// rank, slot from the most significant bits down (the input items of class 4
// carry their slot in the rank field).
inline __host__ __device__ uint64_t deep_sort_key(uint64_t key, uint32_t rank_bits, uint32_t slot_bits) {
    const uint64_t cls = key >> 61;
    const uint64_t rank = cls < 4 ? (key >> 32) & 0x1fffffffu : (key >> 2) & 0x3fffffffu;
    const uint64_t slot = cls < 4 ? (key >> 2) & 0x3fffffffu : 0u;
    return ((cls << rank_bits | rank) << slot_bits) | slot;
}
// Plan for active ranks below max_active_global, input slots below
// input_fanout and synapse slots below synapses_per_neuron.
inline DeepSortPlan deep_sort_plan(uint32_t cap, uint32_t fanout, uint32_t synapses) {
    auto bits_for = [](uint32_t limit) {
        uint32_t b = 1;
        while (b < 30 && (1ull << b) < limit) ++b;
        return b;
    };
    DeepSortPlan p{};
    p.rank_bits = bits_for(cap > fanout ? cap : fanout);
    p.slot_bits = bits_for(synapses);
    const uint32_t total = p.rank_bits + p.slot_bits + 3;  // + class
    for (uint32_t at = 0; at < total && p.passes < kDeepMaxPasses; at += 8) {
        p.shift[p.passes] = at;
        p.bits[p.passes] = total - at < 8 ? total - at : 8;
        ++p.passes;
    }
    return p;
}

// Words of a lane's parameter-change bitmaps (ParameterChanges): neurons
// (threshold and output rows), recurrent synapses, input synapses, context
// slots.
struct ChangeWords {
    uint64_t neurons, recurrent, input, slots;
};

struct KernelArgs {
    LeoConfig cfg;
    SharedModel m;
    LaneDesc* lanes;
    uint32_t lane_count;
    uint32_t wgs_per_lane;
    uint32_t redundant_global;       // block_count*max_active_per_block <= max_active_global
    uint32_t spin_limit;
    uint32_t lane_stride;            // workgroup b serves lane b % lane_stride (>= lane_count)
    uint32_t local_sync;             // allow XCD-local lane barriers
    // Learning slots are the kept eligible slots with nonzero eligibility:
    // with e == 0 the update -lr*s*(signal*e) is a signed zero, and adding it
    // to a valid weight that is not -0.0 returns the weight unchanged, bit for
    // bit, through the clamp and the sign projection (model.rs:343-380 keeps
    // every weight in bounds and of its source's sign). The host clears this
    // flag when a recurrent or input weight is -0.0 (learning and the merge
    // never produce one from another value); every kept slot is then a
    // learning slot.
    uint32_t skip_zero_eligibility;
    uint32_t select_tile;            // select_tile_keys(neurons_per_block)
    uint32_t profile_part;           // workgroup whose phases the profiling build times (of each lane)
    DeepSortPlan deep;
    FastDiv div_synapses;            // synapses_per_neuron
    FastDiv div_block;               // neurons_per_block
    FastDiv div_block_words;         // block_words(neurons_per_block)
    // A tally launch (the frozen-only build, one lane, host discards the
    // steps' records): no step records and no per-step work counters; the
    // launch's totals go here instead (kTally* words), zeroed by the launch.
    uint32_t LEO_GLOBAL* tally;
};

// Words of a tally launch's totals: per-wave sums added at the end, then the
// recording wave's sums as 64-bit words.
enum : uint32_t {
    kTEvents = 0,  // folded entries, each tick's input injections included
    kTTouched,
    kTInhibitory,
    kTDeepRegister,
    kTDeepRadix,
    kTWaveWords,
    kTActive = 8,   // 64-bit words from here: sum of active counts,
    kTCells = 10,   // context cells,
    kTKeptRec = 12, // eligible recurrent list lengths,
    kTKeptIn = 14,  // eligible input list lengths
    kTallyWords = 16
};

// Batch-end mean of one fixed-parameter tensor (see leo_merge_fixed).
enum : uint32_t { kMergeThreshold = 0, kMergeRecurrent, kMergeInput, kMergeOutput, kMergeBias, kMergeContextOut };

struct MergeArgs {
    float LEO_GLOBAL* canonical;
    const float* const* lanes;   // per-lane pointer to the same tensor
    uint32_t lane_count;
    uint32_t kind;
    uint64_t count;              // logical elements
    uint32_t row;                // logical row length for padded layouts (output: 257)
    uint32_t stride;             // physical row stride (output: kOutStride)
    uint32_t synapses_per_neuron;
    const uint8_t LEO_GLOBAL* neuron_type;
    float weight_min, weight_max;
    unsigned long long LEO_GLOBAL* updates;       // merged elements
    unsigned long long LEO_GLOBAL* lane_changes;  // (element, lane) pairs with a nonzero delta
    uint32_t LEO_GLOBAL* error;
    // Lane groups (batches larger than the resident lanes): kMergeAccumulate
    // continues the lane-ordered f64 sum of each element in acc (and the
    // any-lane-changed flag in any), starting from zero when `first`;
    // kMergeFinalize applies acc / total_lanes to the canonical tensor.
    uint32_t mode;
    uint32_t first;
    uint32_t total_lanes;
    double LEO_GLOBAL* acc;
    uint8_t LEO_GLOBAL* any;
    // Host-stale marks of the canonical image: one bit per merged element
    // (per merged neuron row for the output projection: element / row), or,
    // with stale_flag, one word set when any element of the tensor merges.
    uint32_t LEO_GLOBAL* stale;
    uint32_t stale_flag;
    // Candidate list (leo_merge_candidates): when set, only the listed
    // positions are visited (elements, or rows of `row` elements), `*list_count`
    // of them; the others are unchanged in every lane.
    const uint32_t LEO_GLOBAL* list;
    const unsigned long long LEO_GLOBAL* list_count;
};

// Positions changed in any lane of a group: the OR of the lanes' change
// bitmaps (one bit per element, or per output row), listed in `list`.
struct MergeCandidates {
    const uint32_t* const* bits;  // per-lane bitmap of the tensor
    uint32_t lane_count;
    uint64_t words;
    uint64_t positions;
    uint32_t LEO_GLOBAL* list;
    unsigned long long LEO_GLOBAL* count;
};

// Changed context slots of story lanes for the batch-end keyed merge: each
// slot set in a lane's change bitmap as one packed record (slot, key low and
// high word, observations, E embedding words) in the lane's region of `out`
// (`stride` words), appended at the lane's counter.
struct ContextChanges {
    const uint32_t* const* bits;     // per lane: changed-slot bitmap (ch_ctx)
    const uint64_t* const* keys;     // per lane: ctx_keys
    const uint32_t* const* obs;      // per lane: ctx_obs
    const float* const* emb;         // per lane: ctx_emb
    uint64_t slots;
    uint64_t words;                  // bitmap words per lane
    uint64_t stride;                 // words of `out` per lane
    uint32_t E;
    uint32_t LEO_GLOBAL* out;
    unsigned long long LEO_GLOBAL* counts;  // per lane
};

// Sparse moves between a canonical tensor and a packed buffer: element
// index[k] (row index[k], `row` elements from index*stride, when row > 0)
// of `tensor` to or from packed[k] (packed[k*row .. k*row+row)).
struct SparseMove {
    float LEO_GLOBAL* tensor;
    const uint32_t LEO_GLOBAL* index;
    float LEO_GLOBAL* packed;
    uint64_t count;              // indices
    uint32_t row;                // 0: single elements
    uint32_t stride;
    uint32_t to_tensor;          // 1: scatter packed -> tensor, 0: gather tensor -> packed
};

// Folds a lane's change bitmaps into the host-stale bitmaps and clears them
// (words[i] bitmaps of words each; the last pair holds the dirty flags).
struct FoldArgs {
    uint32_t LEO_GLOBAL* changes[6];
    uint32_t LEO_GLOBAL* stale[6];
    uint64_t words[6];
};
enum : uint32_t { kMergeDirect = 0, kMergeAccumulate = 1, kMergeFinalize = 2 };

}  // namespace leo

#endif
