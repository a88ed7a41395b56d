// Host runtime of the MI355X backend behind the C-ABI in include/leo_hip.h.
//
// It plays the role of the reference's GpuRuntime/CudaRuntime
// (backend.rs:547-794, cuda.rs:1553-9355): it owns the canonical model image on
// the device, a canonical lane (the runtime that trains in place for
// one-worker batches and executes replay), and story lanes for logical
// batches. The training coordinator (training.rs:1539-1954) sits on top:
// document passes, the batch-end lane-ordered mean (device fixed-parameter
// merge + host keyed context merge, parallel.rs:694-1113), and
// bounded-surprise replay.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "launch_plan.h"
#include "leo_device.h"
#include "leo_hip.h"
#include "leo_host.h"

namespace leo {

__global__ void leo_lane_steps(const KernelArgs* args);
__global__ void leo_lane_steps_profiled(const KernelArgs* args);
__global__ void leo_lane_steps_frozen(const KernelArgs* args);
__global__ void leo_lane_outcomes(const KernelArgs* args, uint32_t* out);
__global__ void leo_reset_lanes(KernelArgs args, uint32_t set_tick, uint32_t new_tick);
__global__ void leo_clear_changes(KernelArgs args, ChangeWords w);

__global__ void leo_merge_fixed(MergeArgs m);
__global__ void leo_merge_candidates(MergeCandidates mc);
__global__ void leo_context_changes(ContextChanges g);
__global__ void leo_broadcast(Broadcast b);
__global__ void leo_sparse_move(SparseMove mv);
__global__ void leo_fold_changes(FoldArgs f);

namespace {

thread_local std::string g_error;

#define LEO_HIP_CHECK(expr)                                                                          \
    do {                                                                                             \
        hipError_t status_ = (expr);                                                                 \
        if (status_ != hipSuccess)                                                                   \
            throw Error(status_ == hipErrorOutOfMemory ? LEO_ERR_OUT_OF_MEMORY : LEO_ERR_DEVICE,     \
                        std::string(#expr) + ": " + hipGetErrorString(status_));                     \
    } while (0)

constexpr uint32_t kBegin = 256, kEnd = 257;

// ---------------------------------------------------------------------------
// Device memory: one arena per lane / per image, carved into 256-byte
// aligned arrays.
// ---------------------------------------------------------------------------
struct Arena {
    char* base = nullptr;
    size_t bytes = 0;
    Arena() = default;
    Arena(const Arena&) = delete;
    Arena& operator=(const Arena&) = delete;
    ~Arena() { release(); }
    void release() {
        if (base) (void)hipFree(base);
        base = nullptr;
        bytes = 0;
    }
    void allocate(size_t n) {
        release();
        bytes = n;
        LEO_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&base), std::max<size_t>(n, 256)));
    }
};

// Pinned host staging of the per-launch transfers (step schedules, lane
// descriptors and kernel arguments up; step records and lane control words
// down), on a transfer stream of its own: the step stream waits for the
// uploads through an event, and the transfer stream waits for the step
// stream's kernel through another before the downloads. Space is handed out
// in order and reclaimed only once the transfer stream has drained, so no
// pending copy's source or destination is reused.
struct PinnedStaging {
    char* base = nullptr;
    size_t capacity = 0, used = 0;
    hipStream_t xfer = nullptr;
    // when set, copies go to this stream (the step stream) instead of the
    // transfer stream: its work is ordered already and no event joins the two
    hipStream_t route = nullptr;
    hipEvent_t uploaded = nullptr, computed = nullptr;
    bool pending_uploads = false;
    hipStream_t active() const { return route ? route : xfer; }
    PinnedStaging() = default;
    PinnedStaging(const PinnedStaging&) = delete;
    PinnedStaging& operator=(const PinnedStaging&) = delete;
    ~PinnedStaging() {
        if (xfer) (void)hipStreamSynchronize(xfer);
        if (base) (void)hipHostFree(base);
        if (uploaded) (void)hipEventDestroy(uploaded);
        if (computed) (void)hipEventDestroy(computed);
        if (xfer) (void)hipStreamDestroy(xfer);
    }
    void init() {
        LEO_HIP_CHECK(hipStreamCreateWithFlags(&xfer, hipStreamNonBlocking));
        LEO_HIP_CHECK(hipEventCreateWithFlags(&uploaded, hipEventDisableTiming));
        LEO_HIP_CHECK(hipEventCreateWithFlags(&computed, hipEventDisableTiming));
    }
    static size_t rounded(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }
    // Room for `bytes` more (in rounded pieces) without reclaiming: drains the
    // transfer stream and, if needed, grows the buffer first.
    void reserve(size_t bytes) {
        if (used + bytes <= capacity) return;
        drain();
        if (bytes <= capacity) return;
        if (base) LEO_HIP_CHECK(hipHostFree(base));
        base = nullptr;
        capacity = std::max<size_t>({rounded(bytes), 2 * capacity, size_t(1) << 20});
        LEO_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&base), capacity, hipHostMallocDefault));
    }
    char* take(size_t bytes) {
        const size_t need = rounded(bytes);
        reserve(need);
        char* p = base + used;
        used += need;
        return p;
    }
    void h2d(void* dst, const void* src, size_t bytes) {
        if (!bytes) return;
        char* p = take(bytes);
        std::memcpy(p, src, bytes);
        LEO_HIP_CHECK(hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, active()));
        if (!route) pending_uploads = true;
    }
    // one upload of pieces placed at byte offsets of `dst` (the bytes between
    // pieces are left undefined)
    struct Piece {
        const void* src;
        size_t bytes, at;
    };
    void h2d_gather(void* dst, std::initializer_list<Piece> pieces) {
        size_t bytes = 0;
        for (const Piece& piece : pieces) bytes = std::max(bytes, piece.at + piece.bytes);
        char* p = take(bytes);
        for (const Piece& piece : pieces)
            if (piece.bytes) std::memcpy(p + piece.at, piece.src, piece.bytes);
        LEO_HIP_CHECK(hipMemcpyAsync(dst, p, bytes, hipMemcpyHostToDevice, active()));
        if (!route) pending_uploads = true;
    }
    // the stream `s` waits for every upload issued so far
    void publish(hipStream_t s) {
        if (!pending_uploads || route == s) return;
        LEO_HIP_CHECK(hipEventRecord(uploaded, xfer));
        LEO_HIP_CHECK(hipStreamWaitEvent(s, uploaded, 0));
        pending_uploads = false;
    }
    // later transfers start after the work queued on `s` so far
    void follow(hipStream_t s) {
        if (route == s) return;
        LEO_HIP_CHECK(hipEventRecord(computed, s));
        LEO_HIP_CHECK(hipStreamWaitEvent(xfer, computed, 0));
    }
    // a download into staging space; valid after drain()
    const char* d2h(const void* src, size_t bytes) {
        char* p = take(bytes);
        if (bytes) LEO_HIP_CHECK(hipMemcpyAsync(p, src, bytes, hipMemcpyDeviceToHost, active()));
        return p;
    }
    // every copy issued so far is complete
    void wait() {
        if (xfer) LEO_HIP_CHECK(hipStreamSynchronize(xfer));
        if (route) LEO_HIP_CHECK(hipStreamSynchronize(route));
    }
    void drain() {
        wait();
        used = 0;
    }
};

// Routes the staging's copies onto `s` while in scope, after everything
// already queued on the transfer stream (uploads and downloads alike). The
// copies issued outside the scope keep their own event handoffs.
struct StagingRoute {
    PinnedStaging& staging;
    StagingRoute(PinnedStaging& st, hipStream_t s) : staging(st) {
        staging.pending_uploads = true;
        staging.publish(s);
        staging.route = s;
    }
    ~StagingRoute() { staging.route = nullptr; }
    StagingRoute(const StagingRoute&) = delete;
    StagingRoute& operator=(const StagingRoute&) = delete;
};

struct Layout {
    size_t cursor = 0;
    template <class T>
    size_t add(size_t count) {
        size_t at = cursor;
        cursor += (count * sizeof(T) + 255) & ~static_cast<size_t>(255);
        return at;
    }
};

struct Sizes {
    uint64_t n, s, f, ns, ni, slots, e, blocks, block_words, limit, cap, bucket_total, shadow_total;
    uint64_t words(uint64_t count) const { return (count + 31) / 32; }
};

float plasticity_step(uint32_t window, uint32_t& phase, bool end_document) {  // config.rs:137-145
    uint32_t w = std::max<uint32_t>(window, 1);
    uint32_t step = std::min(phase, w - 1) + 1;
    if (step == w || end_document) {
        phase = 0;
        return static_cast<float>(step);
    }
    phase = step;
    return 0.0f;
}

bool context_survives_dropout(uint64_t seed, uint64_t tick, uint32_t symbol, float rate) {  // runtime.rs:103-116
    if (rate <= 0.0f) return true;
    uint64_t v = seed ^ (tick * 0x9e3779b97f4a7c15ULL) ^ (static_cast<uint64_t>(symbol) * 0xbf58476d1ce4e5b9ULL);
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
    v ^= v >> 31;
    float draw = static_cast<float>(static_cast<uint32_t>(v >> 40)) / static_cast<float>(1u << 24);
    return draw >= rate;
}

float permission_strength(const LeoHostConfig& c, int32_t permission) {  // permission.rs:24-31
    switch (permission) {
        case LEO_FROZEN: return 0.0f;
        case LEO_PROVISIONAL: return c.provisional_strength;
        case LEO_TRAINING: return c.training_strength;
        case LEO_VERIFIED: return c.verified_strength;
        default: throw Error(LEO_ERR_INVALID_ARGUMENT, "unknown permission");
    }
}

struct HostStep {
    uint32_t symbol;
    int32_t target;  // external symbol or -1
};

// Lane: transient state (+ optionally its own learned-parameter copy).
struct Lane {
    Arena state;
    Arena params;
    LaneDesc desc{};
    Arena schedule;  // header (single-lane launches), steps, records
    uint32_t schedule_capacity = 0;
    // host mirrors of per-runtime scalars (deterministic from the schedule)
    uint32_t tick = 0;
    uint32_t plasticity_phase = 0;
    bool persistent_activity = false;
    // the host has reported this lane's device guard: its sticky error word
    // is cleared before the next work queued on the lane
    bool error_seen = false;
};

}  // namespace

}  // namespace leo

struct LeoHipRuntime {
    LeoHostConfig cfg{};
    leo::Sizes z{};
    int device = 0;
    hipStream_t stream = nullptr;
    int cus = 0;
    int coop_blocks_per_cu = 0;
    leo::Arena shared;
    leo::SharedModel sm{};
    leo::Arena canon_params;
    leo::LaneParams canon{};
    std::unique_ptr<leo::Lane> canonical;
    std::vector<std::unique_ptr<leo::Lane>> lanes;
    uint32_t max_lanes = 0;
    leo::Arena lane_descs;     // LaneDesc[max(1,max_lanes)]
    leo::Arena replay_results;   // a canonical run's launch outcomes and step records
    leo::Arena replay_plan;      // a canonical run's launch headers and step parameters
    leo::Arena launch_block;     // a launch of several lanes: arguments, descriptors, schedules, results
    std::vector<hipEvent_t> chunk_events;  // a canonical run's result chunks downloaded
    leo::Arena merge_acc;        // f64 sums + changed flags of the lane-group merge
    leo::Arena merge_list;       // candidate positions of one tensor's merge
    uint32_t resident_lanes = 0; // story lanes that fit on the device at once
    uint32_t max_steps_override = 0;
    float last_launch_ms = 0.0f;  // duration of the latest lane-steps launch (HIP events)
    double canonical_step_ms = 0.0;  // slowest per-step average of a timed canonical replay launch
    leo::Arena merge_scratch;  // lane pointer table + counters
    leo::Arena ctx_scratch;    // the story lanes' changed context slots (download_lane_contexts)
    // Host-stale marks of the canonical image: elements changed since the
    // caller's host mirror was last synchronised that the change bitmaps no
    // longer hold (tracking restarts fold them in here; the batch-end mean and
    // the keyed context merge mark them directly). Sets: threshold, recurrent,
    // input, output rows, context slots; then the bias / context output flags.
    leo::Arena stale;
    uint32_t* stale_bits[5] = {};
    uint32_t* stale_flags = nullptr;  // [0] bias, [1] context output projection
    leo::Arena move_scratch;          // packed indices and values of sparse moves
    // host copies of the read-only topology (device copies are immutable)
    std::vector<float> excitability;
    std::vector<uint8_t> neuron_type, rec_branch, rec_delay, in_branch;
    std::vector<uint32_t> rec_target, in_target;
    // host mirrors of model scalars
    uint64_t generation = 0, revision = 0;
    LeoStatistics stats{};
    bool tracking = false;
    // a recurrent or input weight of the canonical model is -0.0 (see
    // KernelArgs::skip_zero_eligibility)
    bool negative_zero_weights = false;
    std::atomic<bool> busy{false};
    uint32_t wgs_override = 0;
    uint32_t canonical_wgs_override = 0;
    bool local_sync = true;
    LeoKernelStats telemetry{};
    bool phase_profile = false;
    // delivery bucket sets of the canonical lane: kBucketSets lets its frozen
    // runs take one barrier per step; 1 (LEO_HIP_BUCKET_SETS=1, or too little
    // device memory) keeps two
    uint32_t canonical_sets = leo::kBucketSets;
    uint32_t profile_part = 0;  // LEO_HIP_PROFILE_PART: the workgroup of each lane the phase profile times
    // launches whose steps are all frozen without output run the step kernel
    // built for them (LEO_HIP_FROZEN_KERNEL=0: never)
    bool frozen_kernel = true;
    // the replay's frozen-only launches keep only their totals, not a record
    // per step (LEO_HIP_TALLY=0: records)
    bool tally_launches = true;
    double wall_clock_khz = 0.0;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    std::vector<hipEvent_t> launch_events;  // timing events of queued launches (pairs)
    leo::PinnedStaging staging;  // per-launch transfers (transfer stream + pinned buffer)
    ~LeoHipRuntime() {
        if (staging.xfer) (void)hipStreamSynchronize(staging.xfer);
        for (hipEvent_t e : launch_events) (void)hipEventDestroy(e);
        for (hipEvent_t e : chunk_events) (void)hipEventDestroy(e);
    }
};

namespace leo {

int32_t set_error(int32_t code, const std::string& message) {
    g_error = message;
    return code;
}

namespace {

struct BusyGuard {
    LeoHipRuntime* h;
    explicit BusyGuard(LeoHipRuntime* rt) : h(rt) {
        if (!h) throw Error(LEO_ERR_INVALID_ARGUMENT, "null runtime handle");
        bool expected = false;
        if (!h->busy.compare_exchange_strong(expected, true))
            throw Error(LEO_ERR_BUSY, "concurrent call on one runtime handle");
        LEO_HIP_CHECK(hipSetDevice(h->device));
    }
    ~BusyGuard() { h->busy.store(false); }
};

Sizes sizes_of(const LeoHostConfig& c) {
    Sizes z{};
    z.n = c.device.neuron_count;
    z.s = c.device.synapses_per_neuron;
    z.f = c.device.input_fanout;
    z.ns = z.n * z.s;
    z.ni = static_cast<uint64_t>(kSymbols) * z.f;
    z.slots = static_cast<uint64_t>(c.device.context_max_order) * c.device.context_slots_per_order;
    z.e = c.device.context_embedding_dim;
    z.blocks = c.device.block_count;
    z.block_words = block_words(c.device.neurons_per_block);
    z.limit = c.device.max_active_per_block;
    z.cap = c.device.max_active_global;
    return z;
}

void upload(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes) LEO_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
}
void download(void* dst, const void* src, size_t bytes, hipStream_t s) {
    if (bytes) LEO_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
}
void sync(hipStream_t s) { LEO_HIP_CHECK(hipStreamSynchronize(s)); }

// Allocate a learned-parameter image.
LaneParams allocate_params(Arena& arena, const Sizes& z, hipStream_t stream) {
    Layout l;
    size_t o_th = l.add<float>(z.n), o_rw = l.add<float>(z.ns), o_iw = l.add<float>(z.ni);
    size_t o_ow = l.add<float>(z.n * kOutStride), o_b = l.add<float>(kOutStride);
    size_t o_ck = l.add<uint64_t>(z.slots), o_ce = l.add<float>(z.slots * z.e), o_co = l.add<uint32_t>(z.slots);
    size_t o_cw = l.add<float>(static_cast<uint64_t>(kOutputs) * z.e);
    arena.allocate(l.cursor);
    LaneParams p{};
    p.threshold = reinterpret_cast<float*>(arena.base + o_th);
    p.rec_weight = reinterpret_cast<float*>(arena.base + o_rw);
    p.in_weight = reinterpret_cast<float*>(arena.base + o_iw);
    p.out_w = reinterpret_cast<float*>(arena.base + o_ow);
    p.bias = reinterpret_cast<float*>(arena.base + o_b);
    p.ctx_keys = reinterpret_cast<uint64_t*>(arena.base + o_ck);
    p.ctx_emb = reinterpret_cast<float*>(arena.base + o_ce);
    p.ctx_obs = reinterpret_cast<uint32_t*>(arena.base + o_co);
    p.ctx_out = reinterpret_cast<float*>(arena.base + o_cw);
    // zero on the runtime's stream: a non-blocking stream is not ordered after the null stream
    LEO_HIP_CHECK(hipMemsetAsync(arena.base, 0, arena.bytes, stream));
    LEO_HIP_CHECK(hipStreamSynchronize(stream));
    return p;
}

// The canonical parameters into every lane of `lanes` (fork(base.clone())
// for a story group): one leo_broadcast per tensor reads the canonical copy
// once for up to kMaxBroadcast lanes; a tensor whose size or addresses are
// not in 16-byte units is copied lane by lane.
void broadcast_params(LeoHipRuntime* h, const std::vector<Lane*>& lanes) {
    const Sizes& z = h->z;
    struct Tensor {
        void* (*field)(const LaneParams&);
        size_t bytes;
    };
    const Tensor tensors[] = {
        {[](const LaneParams& p) -> void* { return p.threshold; }, z.n * 4},
        {[](const LaneParams& p) -> void* { return p.rec_weight; }, z.ns * 4},
        {[](const LaneParams& p) -> void* { return p.in_weight; }, z.ni * 4},
        {[](const LaneParams& p) -> void* { return p.out_w; }, z.n * kOutStride * 4},
        {[](const LaneParams& p) -> void* { return p.bias; }, kOutStride * 4},
        {[](const LaneParams& p) -> void* { return p.ctx_keys; }, z.slots * 8},
        {[](const LaneParams& p) -> void* { return p.ctx_emb; }, z.slots * z.e * 4},
        {[](const LaneParams& p) -> void* { return p.ctx_obs; }, z.slots * 4},
        {[](const LaneParams& p) -> void* { return p.ctx_out; }, kOutputs * z.e * 4},
    };
    auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    for (const Tensor& t : tensors) {
        if (t.bytes == 0) continue;
        const void* src = t.field(h->canon);
        bool vectors = t.bytes % 16 == 0 && aligned(src);
        for (Lane* l : lanes) vectors = vectors && aligned(t.field(l->desc.p));
        if (!vectors) {
            for (Lane* l : lanes)
                LEO_HIP_CHECK(hipMemcpyAsync(t.field(l->desc.p), src, t.bytes, hipMemcpyDeviceToDevice, h->stream));
            continue;
        }
        for (size_t at = 0; at < lanes.size(); at += kMaxBroadcast) {
            Broadcast b{};
            b.src = static_cast<const uint4*>(src);
            b.vectors = t.bytes / 16;
            b.count = static_cast<uint32_t>(std::min<size_t>(kMaxBroadcast, lanes.size() - at));
            for (uint32_t i = 0; i < b.count; ++i) b.dst[i] = static_cast<uint4*>(t.field(lanes[at + i]->desc.p));
            const uint64_t grid = std::min<uint64_t>((b.vectors + kThreads - 1) / kThreads, 8 * static_cast<uint64_t>(h->cus));
            hipLaunchKernelGGL(leo_broadcast, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, h->stream, b);
            LEO_HIP_CHECK(hipGetLastError());
        }
    }
}

// Bytes of one delivery bucket set (entries, counts, touched bitmap).
size_t bucket_set_bytes(const Sizes& z) {
    return static_cast<size_t>(2 * z.bucket_total) * 8 + static_cast<size_t>(z.n) * 4 +
           static_cast<size_t>(z.blocks * z.block_words) * 4;
}

// Bucket sets of the canonical lane: the extra sets take at most a quarter
// of the free device memory.
uint32_t canonical_bucket_sets(const LeoHipRuntime* h) {
    if (h->canonical_sets == 1) return 1;
    size_t free_bytes = 0, total_bytes = 0;
    LEO_HIP_CHECK(hipMemGetInfo(&free_bytes, &total_bytes));
    return (kBucketSets - 1) * bucket_set_bytes(h->z) <= free_bytes / 4 ? kBucketSets : 1u;
}

// Lane state with `sets` delivery bucket sets (1, or kBucketSets for a lane
// that takes frozen runs with one barrier per step).
void allocate_lane_state(Lane& lane, const Sizes& z, hipStream_t stream, uint32_t sets = 1) {
    Layout l;
    size_t o_ctl = l.add<LaneControl>(1), o_flag = l.add<uint32_t>(kMaxLaneWgs * kFlagWords);
    size_t o_cnt = l.add<uint32_t>(kMaxLaneWgs * kFlagWords);
    size_t o_neu = l.add<uint32_t>(kNeuronWords * z.n), o_tl = l.add<uint32_t>(z.n);
    size_t o_ls = l.add<float>(z.n), o_dl = l.add<uint32_t>(z.n), o_bk = l.add<uint64_t>(2 * z.bucket_total * sets);
    size_t o_bc = l.add<uint32_t>(z.n * sets);
    size_t o_rl = l.add<uint32_t>(z.ns), o_il = l.add<uint32_t>(z.ni);
    size_t o_sh = l.add<uint64_t>(2 * std::max<uint64_t>(z.shadow_total, 1));
    size_t o_bw = l.add<uint32_t>(z.blocks * z.limit), o_bcut = l.add<float>(z.blocks);
    size_t o_bwa = l.add<float>(z.blocks * z.limit);
    size_t o_wt = l.add<uint32_t>(2 * kMaxWaves), o_wtt = l.add<uint32_t>(kMaxWaves);
    size_t o_bep = l.add<uint32_t>(z.blocks), o_tb = l.add<uint32_t>(z.blocks * z.block_words * sets);
    size_t o_ra = l.add<uint32_t>(kRing * z.cap), o_rv = l.add<float>(kRing * z.cap), o_rval = l.add<float>(kRing * z.cap * z.s);
    size_t o_redge = l.add<uint32_t>(kRing * z.cap * z.s);
    size_t o_rt = l.add<float>(kTraceWords * z.ns), o_rm = l.add<uint8_t>(z.ns), o_rlist = l.add<uint32_t>(2 * z.ns);
    size_t o_it = l.add<float>(kTraceWords * z.ni), o_im = l.add<uint8_t>(z.ni), o_ilist = l.add<uint32_t>(2 * z.ni);
    size_t o_lg = l.add<float>(kOutStride), o_pr = l.add<float>(kOutStride), o_er = l.add<float>(kOutStride);
    size_t o_lat = l.add<float>(std::max<uint64_t>(z.e, 1));
    size_t o_cth = l.add<uint32_t>(z.words(z.n)), o_crec = l.add<uint32_t>(z.words(z.ns)), o_cin = l.add<uint32_t>(z.words(z.ni));
    size_t o_cout = l.add<uint32_t>(z.words(z.n)), o_cctx = l.add<uint32_t>(z.words(z.slots));
    size_t o_prof = l.add<unsigned long long>(2 * kPhases);
    lane.state.allocate(l.cursor);
    char* b = lane.state.base;
    LaneDesc& d = lane.desc;
    d.ctl = reinterpret_cast<LaneControl*>(b + o_ctl);
    d.launch = reinterpret_cast<LaunchWords*>(&d.ctl->barrier);
    d.barrier_flags = reinterpret_cast<uint32_t*>(b + o_flag);
    d.wg_counts = reinterpret_cast<uint32_t*>(b + o_cnt);
    d.neuron = reinterpret_cast<uint32_t*>(b + o_neu);
    d.touched_list = reinterpret_cast<uint32_t*>(b + o_tl);

    d.learning_signal = reinterpret_cast<float*>(b + o_ls);
    d.dest_list = reinterpret_cast<uint32_t*>(b + o_dl);
    d.shadow = reinterpret_cast<uint64_t*>(b + o_sh);
    d.rec_learn = reinterpret_cast<uint32_t*>(b + o_rl);
    d.in_learn = reinterpret_cast<uint32_t*>(b + o_il);
    d.bucket = reinterpret_cast<uint64_t*>(b + o_bk);
    d.bucket_count = reinterpret_cast<uint32_t*>(b + o_bc);
    d.bucket_stride = 2 * z.bucket_total;
    d.bucket_sets = sets;
    d.touched_stride = static_cast<uint32_t>(z.blocks * z.block_words);
    d.range_winners = reinterpret_cast<uint32_t*>(b + o_bw);
    d.range_winner_act = reinterpret_cast<float*>(b + o_bwa);
    d.block_cutoff = reinterpret_cast<float*>(b + o_bcut);
    d.wave_total = reinterpret_cast<uint32_t*>(b + o_wt);
    d.wave_touched = reinterpret_cast<uint32_t*>(b + o_wtt);
    d.block_epoch = reinterpret_cast<uint32_t*>(b + o_bep);
    d.touched_bits = reinterpret_cast<uint32_t*>(b + o_tb);
    d.ring_active = reinterpret_cast<uint32_t*>(b + o_ra);
    d.ring_act = reinterpret_cast<float*>(b + o_rv);
    d.ring_value = reinterpret_cast<float*>(b + o_rval);
    d.ring_edge = reinterpret_cast<uint32_t*>(b + o_redge);
    d.rec_trace = reinterpret_cast<float*>(b + o_rt);
    d.rec_mark = reinterpret_cast<uint8_t*>(b + o_rm);
    d.rec_list = reinterpret_cast<uint32_t*>(b + o_rlist);
    d.in_trace = reinterpret_cast<float*>(b + o_it);
    d.in_mark = reinterpret_cast<uint8_t*>(b + o_im);
    d.in_list = reinterpret_cast<uint32_t*>(b + o_ilist);
    d.logits = reinterpret_cast<float*>(b + o_lg);
    d.probs = reinterpret_cast<float*>(b + o_pr);
    d.errors = reinterpret_cast<float*>(b + o_er);
    d.ctx_latent = reinterpret_cast<float*>(b + o_lat);
    d.ch_threshold = reinterpret_cast<uint32_t*>(b + o_cth);
    d.ch_rec = reinterpret_cast<uint32_t*>(b + o_crec);
    d.ch_in = reinterpret_cast<uint32_t*>(b + o_cin);
    d.ch_out = reinterpret_cast<uint32_t*>(b + o_cout);
    d.ch_ctx = reinterpret_cast<uint32_t*>(b + o_cctx);
    d.phase_profile = reinterpret_cast<unsigned long long*>(b + o_prof);
    LEO_HIP_CHECK(hipMemsetAsync(b, 0, lane.state.bytes, stream));
    LEO_HIP_CHECK(hipStreamSynchronize(stream));
}

void clear_changes(const Lane& lane, const Sizes& z, hipStream_t s) {
    const LaneDesc& d = lane.desc;
    LEO_HIP_CHECK(hipMemsetAsync(d.ch_threshold, 0, z.words(z.n) * 4, s));
    LEO_HIP_CHECK(hipMemsetAsync(d.ch_rec, 0, z.words(z.ns) * 4, s));
    LEO_HIP_CHECK(hipMemsetAsync(d.ch_in, 0, z.words(z.ni) * 4, s));
    LEO_HIP_CHECK(hipMemsetAsync(d.ch_out, 0, z.words(z.n) * 4, s));
    LEO_HIP_CHECK(hipMemsetAsync(d.ch_ctx, 0, z.words(z.slots) * 4, s));
    static_assert(offsetof(LaneControl, ctx_out_dirty) == offsetof(LaneControl, bias_dirty) + 4, "cleared together");
    LEO_HIP_CHECK(hipMemsetAsync(&d.ctl->bias_dirty, 0, 8, s));  // bias_dirty, ctx_out_dirty
}

// ---------------------------------------------------------------------------
// Host-stale marks of the canonical image and sparse moves (the reference GPU
// adapter's change lists and gather/scatter kernels, cuda.rs:5657-5760,
// 2869-3080).
// ---------------------------------------------------------------------------
uint64_t set_size(const Sizes& z, int set) {
    const uint64_t counts[5] = {z.n, z.ns, z.ni, z.n, z.slots};
    return counts[set];
}

void allocate_stale(LeoHipRuntime* h) {
    const Sizes& z = h->z;
    Layout l;
    size_t at[5];
    for (int i = 0; i < 5; ++i) at[i] = l.add<uint32_t>(z.words(set_size(z, i)));
    const size_t flags = l.add<uint32_t>(2);
    h->stale.allocate(l.cursor);
    for (int i = 0; i < 5; ++i) h->stale_bits[i] = reinterpret_cast<uint32_t*>(h->stale.base + at[i]);
    h->stale_flags = reinterpret_cast<uint32_t*>(h->stale.base + flags);
    LEO_HIP_CHECK(hipMemsetAsync(h->stale.base, 0, h->stale.bytes, h->stream));
}

void clear_stale(LeoHipRuntime* h) { LEO_HIP_CHECK(hipMemsetAsync(h->stale.base, 0, h->stale.bytes, h->stream)); }

uint32_t* change_bits(const LaneDesc& d, int set) {
    uint32_t* bits[5] = {d.ch_threshold, d.ch_rec, d.ch_in, d.ch_out, d.ch_ctx};
    return bits[set];
}

// Tracking restart of the canonical runtime: its change sets and dirty flags
// move into the host-stale marks and start empty.
void fold_changes(LeoHipRuntime* h) {
    const LaneDesc& d = h->canonical->desc;
    FoldArgs f{};
    uint64_t widest = 2;
    for (int i = 0; i < 5; ++i) {
        f.changes[i] = change_bits(d, i);
        f.stale[i] = h->stale_bits[i];
        f.words[i] = h->z.words(set_size(h->z, i));
        widest = std::max(widest, f.words[i]);
    }
    static_assert(offsetof(LaneControl, ctx_out_dirty) == offsetof(LaneControl, bias_dirty) + 4, "flag pair");
    f.changes[5] = &d.ctl->bias_dirty;
    f.stale[5] = h->stale_flags;
    f.words[5] = 2;
    const uint64_t blocks = std::min<uint64_t>((widest + kThreads - 1) / kThreads, 2048);
    hipLaunchKernelGGL(leo_fold_changes, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, h->stream, f);
    LEO_HIP_CHECK(hipGetLastError());
}

// Scratch of the allocation-free packed commit
// (leo_hip_commit_packed_host_model_no_alloc): a file-scope device array, one
// copy per GPU, held until the process ends. Host code uses its per-device
// address from hipGetSymbolAddress, never the array's name. Every call on a
// GPU shares that GPU's copy, so calls on one GPU (from any runtime) take
// that GPU's lock for the whole commit, through its final synchronisation,
// and run one after another.
constexpr size_t kStaticScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
char* g_scratch_ptr[kMaxScratchDevices] = {};
std::mutex g_scratch_user[kMaxScratchDevices];  // held by the commit that stages through the device's copy

// The device address of `scratch` on `device` (which must be current),
// looked up once per device.
char* static_scratch(int device) {
    if (device < 0 || device >= kMaxScratchDevices)
        throw Error(LEO_ERR_DEVICE, "device index beyond the static scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        LEO_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) throw Error(LEO_ERR_DEVICE, "static scratch has no device address");
        g_scratch_ptr[device] = static_cast<char*>(ptr);
    }
    return g_scratch_ptr[device];
}

// Bytes a sparse move of `count` elements (rows of `per`) stages: the u32
// indices (256-byte aligned) and the values.
size_t move_bytes(uint64_t count, uint64_t per) {
    return count ? ((count * 4 + 255) & ~size_t(255)) + count * per * 4 : 0;
}

// Device staging of sparse moves: the runtime's growable scratch, or a
// fixed buffer that must not grow (the allocation-free entry point).
struct Staging {
    char* fixed = nullptr;   // non-null: use this buffer of `capacity` bytes, never allocate
    size_t capacity = 0;
};

// Moves `count` elements (rows of `row` elements at `stride` when row > 0)
// between a canonical tensor and the host: gathers into `values` when
// to_tensor is false, scatters `values` when true.
void sparse_move(LeoHipRuntime* h, float* tensor, const uint32_t* index, uint64_t count, uint32_t row, uint32_t stride,
                 const float* values_in, float* values_out, bool to_tensor, const Staging& staging = Staging{}) {
    if (count == 0) return;
    const uint64_t per = row ? row : 1;
    const size_t index_bytes = (count * 4 + 255) & ~size_t(255);
    const size_t need = index_bytes + count * per * 4;
    char* base = staging.fixed;
    if (base) {
        if (need > staging.capacity)
            throw Error(LEO_ERR_INVALID_ARGUMENT, "sparse move of " + std::to_string(need) +
                                                      " bytes exceeds the fixed scratch of " +
                                                      std::to_string(staging.capacity) + " bytes");
    } else {
        if (h->move_scratch.bytes < need) h->move_scratch.allocate(need);
        base = h->move_scratch.base;
    }
    upload(base, index, count * 4, h->stream);
    if (to_tensor) upload(base + index_bytes, values_in, count * per * 4, h->stream);
    SparseMove mv{};
    mv.tensor = tensor;
    mv.index = reinterpret_cast<const uint32_t*>(base);
    mv.packed = reinterpret_cast<float*>(base + index_bytes);
    mv.count = count;
    mv.row = row;
    mv.stride = stride;
    mv.to_tensor = to_tensor ? 1u : 0u;
    const uint64_t blocks = std::min<uint64_t>((count * per + kThreads - 1) / kThreads, 4096);
    hipLaunchKernelGGL(leo_sparse_move, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, h->stream, mv);
    LEO_HIP_CHECK(hipGetLastError());
    if (!to_tensor) download(values_out, base + index_bytes, count * per * 4, h->stream);
    sync(h->stream);
}

KernelArgs kernel_args(LeoHipRuntime* h, LaneDesc* lanes, uint32_t count, uint32_t P) {
    KernelArgs a{};
    a.cfg = h->cfg.device;
    a.m = h->sm;
    a.lanes = lanes;
    a.lane_count = count;
    a.wgs_per_lane = P;
    a.redundant_global = (static_cast<uint64_t>(h->z.blocks) * h->z.limit <= h->z.cap) ? 1 : 0;
    a.spin_limit = 1u << 26;
    a.lane_stride = count;
    a.local_sync = h->local_sync ? 1 : 0;
    a.div_synapses = make_fast_div(h->cfg.device.synapses_per_neuron);
    a.div_block = make_fast_div(h->cfg.device.neurons_per_block);
    a.div_block_words = make_fast_div(block_words(h->cfg.device.neurons_per_block));
    a.skip_zero_eligibility = h->negative_zero_weights ? 0u : 1u;
    a.select_tile = select_tile_keys(h->cfg.device.neurons_per_block);
    a.profile_part = std::min(h->profile_part, P > 0 ? P - 1 : 0u);
    a.deep = deep_sort_plan(h->cfg.device.max_active_global, h->cfg.device.input_fanout,
                            h->cfg.device.synapses_per_neuron);
    return a;
}

// Reset transient state of the given lanes (runtime.rs:365-425). Descriptors
// of these lanes must already be resident at `descs` (default:
// lane_descs[0..count)).
void reset_lanes(LeoHipRuntime* h, uint32_t count, bool set_tick, uint32_t new_tick, LaneDesc* descs = nullptr) {
    if (!descs) descs = reinterpret_cast<LaneDesc*>(h->lane_descs.base);
    KernelArgs a = kernel_args(h, descs, count, 1);
    // about eight workgroups per CU in all, at least 64 per lane
    const uint32_t parts = std::max<uint32_t>(64, static_cast<uint32_t>(8 * h->cus) / std::max<uint32_t>(count, 1));
    uint32_t grid = count * parts;
    hipLaunchKernelGGL(leo_reset_lanes, dim3(grid), dim3(kThreads), 0, h->stream, a, set_tick ? 1u : 0u, new_tick);
    LEO_HIP_CHECK(hipGetLastError());
}

// The change bitmaps of the lanes whose descriptors are resident at
// lane_descs[0..count), in one kernel for all of them.
void clear_lane_changes(LeoHipRuntime* h, uint32_t count) {
    const Sizes& z = h->z;
    const ChangeWords w{z.words(z.n), z.words(z.ns), z.words(z.ni), z.words(z.slots)};
    KernelArgs a = kernel_args(h, reinterpret_cast<LaneDesc*>(h->lane_descs.base), count, 1);
    const uint32_t parts = std::max<uint32_t>(16, static_cast<uint32_t>(8 * h->cus) / std::max<uint32_t>(count, 1));
    hipLaunchKernelGGL(leo_clear_changes, dim3(count * parts), dim3(kThreads), 0, h->stream, a, w);
    LEO_HIP_CHECK(hipGetLastError());
}

// Lane descriptors go up through the pinned staging; the step stream waits for
// them, and they wait for the step stream's queued work (which may still read
// the descriptors they replace).
void stage_descs(LeoHipRuntime* h, const std::vector<Lane*>& lanes) {
    std::vector<LaneDesc> host(lanes.size());
    for (size_t i = 0; i < lanes.size(); ++i) host[i] = lanes[i]->desc;
    h->staging.follow(h->stream);
    h->staging.h2d(h->lane_descs.base, host.data(), host.size() * sizeof(LaneDesc));
    h->staging.publish(h->stream);
}

// Clears the sticky error word of a lane whose guard the host has already
// reported, on `stream`, ahead of the next work queued there.
void clear_reported_error(Lane& lane, hipStream_t stream) {
    if (!lane.error_seen) return;
    LEO_HIP_CHECK(hipMemsetAsync(&lane.desc.ctl->error_code, 0, 4, stream));
    lane.error_seen = false;
}

// A reset's device part (the lanes' descriptors up, then leo_reset_lanes) and
// its host mirrors.
void reset_lane_device(LeoHipRuntime* h, const std::vector<Lane*>& lanes, bool set_tick, uint32_t new_tick) {
    for (Lane* l : lanes) clear_reported_error(*l, h->stream);
    stage_descs(h, lanes);
    reset_lanes(h, static_cast<uint32_t>(lanes.size()), set_tick, new_tick);
}
void reset_lane_mirrors(const std::vector<Lane*>& lanes, bool set_tick, uint32_t new_tick) {
    for (Lane* l : lanes) {
        if (set_tick) l->tick = new_tick;
        l->plasticity_phase = 0;
        l->persistent_activity = false;
    }
}
void reset_lane_objects(LeoHipRuntime* h, const std::vector<Lane*>& lanes, bool set_tick, uint32_t new_tick) {
    reset_lane_device(h, lanes, set_tick, new_tick);
    reset_lane_mirrors(lanes, set_tick, new_tick);
}

// Launch shape of `lanes` lanes: the wanted workgroups per lane, capped by the
// cooperative capacity (launch_plan.h).
LanePlan choose_wgs_per_lane(LeoHipRuntime* h, uint32_t lanes, bool canonical) {
    uint32_t want;
    if (canonical && h->canonical_wgs_override) {
        want = h->canonical_wgs_override;
    } else if (h->wgs_override) {
        want = h->wgs_override;
    } else {
        // one selecting wave per block (the last workgroup selects nothing),
        // and about one workgroup per 32K edges
        uint64_t by_blocks = (h->z.blocks + kWavesPerGroup - 1) / kWavesPerGroup + 1;
        uint64_t by_edges = h->z.ns / 32768;
        want = static_cast<uint32_t>(std::max<uint64_t>(1, std::max(by_blocks, by_edges)));
        want = std::min<uint32_t>(want, 64);
        if (canonical) {
            // the canonical lane is latency-bound (replay): its workgroups
            // share one XCD, one per CU (measured: a second workgroup per CU
            // slows its steps), at least 8 of them (measured at 1,024 units:
            // 41 us per step with 8, 53 us with the 2 the blocks ask for)
            const uint32_t per_xcd = std::max<uint32_t>(1, static_cast<uint32_t>(h->cus) / kXcds);
            want = std::min<uint32_t>(std::max<uint32_t>(want, 8), per_xcd);
        }
    }
    return plan_lanes(lanes, want, static_cast<uint32_t>(h->cus), static_cast<uint32_t>(h->coop_blocks_per_cu),
                      kMaxWaves / kWavesPerGroup, kXcds);
}

StepParams make_step(const LeoHostConfig& c, Lane& lane, uint32_t symbol, int32_t target, int32_t permission,
                     uint32_t tick, bool output) {
    if (symbol >= kSymbols) throw Error(LEO_ERR_INVALID_ARGUMENT, "invalid input symbol: " + std::to_string(symbol));
    int32_t target_index = -1;
    if (target >= 0) {
        uint32_t t = static_cast<uint32_t>(target);
        if (t < 256) target_index = static_cast<int32_t>(t);
        else if (t == kEnd) target_index = static_cast<int32_t>(kEndIndex);
        else throw Error(LEO_ERR_INVALID_ARGUMENT, "invalid output target: " + std::to_string(t));
    }
    const bool frozen = permission == LEO_FROZEN;
    const float strength = permission_strength(c, permission);
    StepParams sp{};
    sp.symbol = symbol;
    sp.target_index = target_index;
    bool ctx = frozen || context_survives_dropout(c.seed, tick, symbol, c.context_dropout_rate);
    sp.flags = (frozen ? kStepFrozen : kStepLearnTrace) | (ctx ? kStepContext : 0u) | ((!frozen && ctx) ? kStepAllocate : 0u);
    const bool learn = target_index >= 0 && strength > 0.0f;
    if (output || learn) sp.flags |= kStepOutput;
    sp.strength = strength;
    if (learn) {
        sp.flags |= kStepLearn;
        float weight = static_cast<uint32_t>(target_index) == kEndIndex ? c.end_document_weight : 1.0f;
        sp.supervised_strength = strength * weight;
        sp.plasticity_scale = plasticity_step(c.plasticity_window, lane.plasticity_phase,
                                              static_cast<uint32_t>(target_index) == kEndIndex);
    }
    return sp;
}

constexpr size_t kAllSteps = ~size_t(0);

// A step the frozen-only step kernel runs: frozen, with neither learning nor
// output (the replay's prefix steps, advance_frozen_batch).
inline bool frozen_only_step(const StepParams& sp) {
    return (sp.flags & kStepFrozen) && !(sp.flags & (kStepLearnTrace | kStepAllocate | kStepLearn | kStepOutput));
}

struct LaneRun {
    Lane* lane;
    std::vector<StepParams> steps;
    std::vector<StepRecord> records;
    // steps that ran to the end: all of them, or those before the step whose
    // numerical guard stopped the lane
    size_t completed = kAllSteps;
    // the lane's plasticity phase before each step (canonical schedules), to
    // put the host mirror back where a stopped step left it
    std::vector<uint32_t> phase;
};

// Algorithmic HBM bytes of one lane-step: each DRAM-resident element a phase
// touches counts once (read 1x, read-modify-write 2x); lane-private vectors of
// at most 64 KB (logits, errors, bias, context projection) are on-chip and not
// counted. FP32/u32 = 4 B, u8 = 1 B.
//   29 per delivered event      emission snapshot 8 + slot meta/value 13 + branch RMW 8
//   17 per injected input slot  target/branch/weight 9 + branch RMW 8
//   72 per activated trace      last-tick RMW 16 + 6 sensitivities RMW 48 + mark/list 8
//  172 per touched neuron       branches, ticks, membrane, fatigue, adaptation, refractory,
//                               threshold, excitability, candidate, surrogate, homeostasis
//  140 per eligible slot scan   meta 5 + 7 FP32 + tick RMW 72 + list/mark 12 + destination 40 + list 4 + epoch 8
//   60 per active neuron        post-activation state RMW + ring entry
//    8 per active edge          emission snapshot weight read + value write
// 1028 per active neuron        readout row gather (output computed)
// 1032 per destination          learning-signal row read + signal write (destinations: the
//                               targets of learning slots, the kept eligible slots whose
//                               eligibility is nonzero; no update reads another signal)
// 2056 per active neuron        output row RMW (learning step)
//   37 per learning slot        weight RMW 8 + eligibility 4 + target 4 + signal 4 + list 4 + marks/type 13
//   28 per inhibitory edge      target activation 4 + weight RMW 8 + target 4 + mark 8 + eligibility 4
//    4 per context cell * E     embedding row read
double step_bytes(const LeoHostConfig& c, const StepParams& sp, const StepRecord& r) {
    const double S = c.device.synapses_per_neuron, F = c.device.input_fanout, E = c.device.context_embedding_dim;
    const bool lam = (sp.flags & kStepLearnTrace) != 0;
    const bool sig = (sp.flags & kStepLearn) != 0;
    const bool pi = sig && sp.plasticity_scale > 0.0f;
    const bool out = (sp.flags & kStepOutput) != 0;
    double b = 29.0 * r.events + 17.0 * F + 172.0 * r.touched + 60.0 * r.active + 8.0 * r.active * S +
               4.0 * r.context_cells * E;
    if (lam) b += 72.0 * (static_cast<double>(r.events) + F) + 140.0 * (static_cast<double>(r.scanned_rec) + r.scanned_in);
    if (out) b += 1028.0 * r.active;
    if (pi) b += 1032.0 * r.destinations + 37.0 * r.learning_slots;
    if (sig) b += 2056.0 * r.active + 28.0 * r.active_inhibitory * S;
    return b;
}

// `tally`: the totals of a tally launch (one lane of frozen steps without
// output), which stand for its steps' work counters; step_bytes is linear in
// them for such steps.
void account_launch(LeoHipRuntime* h, const std::vector<LaneRun>& runs, float ms, bool canonical,
                    const char* tally = nullptr) {
    LeoKernelStats& t = h->telemetry;
    const int section = canonical ? 1 : 0;
    t.launches += 1;
    t.kernel_ms += ms;
    t.section_launches[section] += 1;
    t.section_kernel_ms[section] += ms;
    if (tally) {
        uint32_t w[kTallyWords];
        std::memcpy(w, tally, sizeof(w));
        auto wide = [&](uint32_t at) {
            uint64_t v;
            std::memcpy(&v, w + at, sizeof(v));
            return v;
        };
        const double S = h->cfg.device.synapses_per_neuron, F = h->cfg.device.input_fanout;
        const double E = h->cfg.device.context_embedding_dim;
        const uint64_t n = runs[0].steps.size(), active = wide(kTActive), cells = wide(kTCells);
        // the folds counted each tick's F injections with the recurrent events
        // (a step record counts folded - F)
        const uint64_t injected = static_cast<uint64_t>(h->cfg.device.input_fanout) * n;
        const uint64_t events = w[kTEvents] > injected ? w[kTEvents] - injected : 0;
        const double bytes = 29.0 * static_cast<double>(events) + 17.0 * F * static_cast<double>(n) + 172.0 * w[kTTouched] +
                             60.0 * static_cast<double>(active) + 8.0 * static_cast<double>(active) * S +
                             4.0 * static_cast<double>(cells) * E;
        t.lane_steps += n;
        t.algorithmic_bytes += bytes;
        t.section_lane_steps[section] += n;
        t.section_bytes[section] += bytes;
        t.events += events;
        t.touched += w[kTTouched];
        t.active += active;
        t.kept_rec += wide(kTKeptRec);
        t.kept_in += wide(kTKeptIn);
        t.deep_register_folds += w[kTDeepRegister];
        t.deep_radix_folds += w[kTDeepRadix];
        t.active_inhibitory += w[kTInhibitory];
        return;
    }
    for (const LaneRun& run : runs) {
        for (size_t i = 0; i < run.steps.size(); ++i) {
            const StepRecord& r = run.records[i];
            const double bytes = step_bytes(h->cfg, run.steps[i], r);
            t.lane_steps += 1;
            t.algorithmic_bytes += bytes;
            t.section_lane_steps[section] += 1;
            t.section_bytes[section] += bytes;
            t.events += r.events;
            t.touched += r.touched;
            t.active += r.active;
            t.scanned_rec += r.scanned_rec;
            t.scanned_in += r.scanned_in;
            t.kept_rec += r.eligible_rec;
            t.kept_in += r.eligible_in;
            t.learning_slots += r.learning_slots;
            t.deep_register_folds += r.deep_folds & 0xffffu;
            t.deep_radix_folds += r.deep_folds >> 16;
            t.destinations += r.destinations;
            t.active_inhibitory += r.active_inhibitory;
        }
    }
}

// One cooperative launch over all given lanes (each with its own schedule).
// One launch of the step kernel queued on the runtime's streams: its lanes'
// schedules, where its step records and control words arrive in pinned
// memory, its timing events and the ticks its lanes must reach.
struct QueuedLaunch {
    std::vector<LaneRun> runs;
    std::vector<const char*> records, ctl;
    const char* outcomes = nullptr;  // instead of ctl: four outcome words per lane
    const char* tally = nullptr;     // a tally launch's totals (kTally* words) instead of step records
    std::vector<uint32_t> end_tick;
    hipEvent_t start = nullptr, stop = nullptr;
    bool canonical = false;
};

// Pinned staging bytes one launch of these schedules moves (its uploads and
// downloads; a reset's descriptors take one more rounded LaneDesc group).
size_t launch_staging_bytes(size_t lanes, const std::vector<size_t>& steps) {
    size_t staged = PinnedStaging::rounded(lanes * sizeof(LaneDesc)) + PinnedStaging::rounded(sizeof(KernelArgs));
    for (size_t n : steps)
        staged += PinnedStaging::rounded(n * sizeof(StepParams)) + PinnedStaging::rounded(n * sizeof(StepRecord)) +
                  PinnedStaging::rounded(sizeof(LaneControl));
    return staged;
}

// A lane's schedule buffer: a header, then the step parameters, then the
// step records. A launch of one lane keeps its kernel arguments and lane
// descriptor in the header, so that they go up with the schedule in one copy.
constexpr size_t kHeaderArgs = 0, kHeaderDesc = 512, kScheduleHeader = 1024;
static_assert(sizeof(KernelArgs) <= kHeaderDesc && sizeof(LaneDesc) <= kScheduleHeader - kHeaderDesc,
              "schedule header");

// Every lane's schedule buffer holds `steps` steps (allocated while nothing
// queued can be reading the old one).
void ensure_schedule(Lane& lane, size_t steps) {
    const uint32_t need = static_cast<uint32_t>(std::max<size_t>(steps, 1));
    if (need <= lane.schedule_capacity) return;
    const uint32_t cap = std::max<uint32_t>(need, 256);
    lane.schedule.allocate(kScheduleHeader + static_cast<size_t>(cap) * (sizeof(StepParams) + sizeof(StepRecord)) +
                           512);
    lane.schedule_capacity = cap;
}

// The delays whose events a step's tick may deliver at emission: the arrival
// step is in the same launch and runs no learning trace.
void mark_early_delivery(std::vector<StepParams>& steps) {
    for (size_t i = 0; i < steps.size(); ++i) {
        uint32_t early = 0;
        for (uint32_t dl = 0; dl < 4; ++dl) {
            const size_t at = i + (size_t(1) << dl);
            if (at < steps.size() && !(steps[at].flags & kStepLearnTrace)) early |= 1u << dl;
        }
        steps[i].flags = (steps[i].flags & ~static_cast<uint32_t>(kStepEarlyMask)) | (early << kStepEarlyShift);
    }
}

void check_tick_range(const LeoHipRuntime* h, uint32_t tick, size_t steps) {
    const uint64_t end = static_cast<uint64_t>(tick) + steps;
    if (end + static_cast<uint64_t>(h->cfg.device.refractory_ticks) + 2 >= 0xffffffffULL)
        throw Error(LEO_ERR_UNSUPPORTED, "lane tick would exceed the 32-bit device tick range");
}

bool frozen_only_steps(const std::vector<StepParams>& steps) {
    for (const StepParams& sp : steps)
        if (!frozen_only_step(sp)) return false;
    return true;
}

// The step kernel build: the profiling build, the frozen-only build when
// every step of the launch is frozen without output (and the lanes select
// redundantly), else the general one.
const void* step_kernel(const LeoHipRuntime* h, bool frozen_only, bool redundant_global) {
    if (h->phase_profile) return reinterpret_cast<const void*>(&leo_lane_steps_profiled);
    return h->frozen_kernel && redundant_global && frozen_only ? reinterpret_cast<const void*>(&leo_lane_steps_frozen)
                                                               : reinterpret_cast<const void*>(&leo_lane_steps);
}

// Queues one launch without waiting for it: uploads through the pinned
// staging (after the step stream's queued work, which may still read the
// buffers they replace), the control words' clears and the kernel, then the
// downloads on the transfer stream. The caller has reserved the staging
// space of everything it queues before the next drain, and sized the
// schedule buffers. The lanes' host tick mirrors advance at once.
QueuedLaunch enqueue_lanes(LeoHipRuntime* h, std::vector<LaneRun> runs, hipEvent_t start, hipEvent_t stop) {
    QueuedLaunch q;
    const uint32_t count = static_cast<uint32_t>(runs.size());
    for (auto& r : runs) check_tick_range(h, r.lane->tick, r.steps.size());
    // lanes are padded to a multiple of the XCD count so that each lane's
    // workgroups land on one XCD (see lane_steps)
    q.canonical = count == 1 && runs[0].lane == h->canonical.get();
    const LanePlan plan = choose_wgs_per_lane(h, count, q.canonical);
    const uint32_t P = plan.P, stride = plan.stride;
    if (P > kMaxLaneWgs) throw Error(LEO_ERR_INTERNAL, "more workgroups per lane than barrier flags");
    h->staging.follow(h->stream);  // the uploads replace what queued work may still read
    if (static_cast<uint64_t>(plan.grid) > cooperative_capacity(h->cus, h->coop_blocks_per_cu))
        throw Error(LEO_ERR_INTERNAL, "cooperative launch exceeds the resident workgroup capacity");
    const bool single = count == 1;
    for (auto& r : runs) {
        mark_early_delivery(r.steps);
        clear_reported_error(*r.lane, h->staging.active());
    }
    KernelArgs a;
    const KernelArgs* device_args = nullptr;
    // Several lanes share one launch block: kernel arguments, descriptors,
    // each lane's zeroed barrier words (a 128-byte line each), then the
    // schedules (one upload), then the step records and the lanes' outcome
    // words, which leo_lane_outcomes gathers there (one download).
    size_t block_records = 0, block_outcomes = 0;
    std::vector<size_t> record_at(count);
    if (single) {
        // a single lane's kernel arguments and descriptor go up with its
        // schedule, in the header of the lane's schedule buffer
        LaneRun& r = runs[0];
        Lane& lane = *r.lane;
        if (r.steps.size() > lane.schedule_capacity) throw Error(LEO_ERR_INTERNAL, "schedule buffer not sized");
        lane.desc.steps = reinterpret_cast<const StepParams*>(lane.schedule.base + kScheduleHeader);
        lane.desc.records = reinterpret_cast<StepRecord*>(
            lane.schedule.base + kScheduleHeader +
            ((static_cast<size_t>(lane.schedule_capacity) * sizeof(StepParams) + 255) & ~size_t(255)));
        lane.desc.step_count = static_cast<uint32_t>(r.steps.size());
        // cleared after the previous launch's control words have been
        // downloaded (a launch queued behind a failed one finds the error
        // word set and runs nothing)
        LEO_HIP_CHECK(hipMemsetAsync(lane.desc.launch, 0, sizeof(LaunchWords), h->staging.active()));
        char* header = lane.schedule.base;
        a = kernel_args(h, reinterpret_cast<LaneDesc*>(header + kHeaderDesc), 1, P);
        a.lane_stride = stride;
        h->staging.h2d_gather(header, {{&a, sizeof(KernelArgs), kHeaderArgs},
                                       {&lane.desc, sizeof(LaneDesc), kHeaderDesc},
                                       {r.steps.data(), r.steps.size() * sizeof(StepParams), kScheduleHeader}});
        device_args = reinterpret_cast<const KernelArgs*>(header + kHeaderArgs);
    } else {
        constexpr size_t kWordsStride = 128;
        const size_t descs_at = kHeaderDesc;
        const size_t words_at = PinnedStaging::rounded(descs_at + count * sizeof(LaneDesc));
        size_t cursor = PinnedStaging::rounded(words_at + count * kWordsStride);
        std::vector<size_t> steps_at(count);
        for (uint32_t i = 0; i < count; ++i) {
            steps_at[i] = cursor;
            cursor += PinnedStaging::rounded(runs[i].steps.size() * sizeof(StepParams));
        }
        const size_t upload = cursor;
        block_records = cursor;
        for (uint32_t i = 0; i < count; ++i) {
            record_at[i] = cursor;
            cursor += PinnedStaging::rounded(runs[i].steps.size() * sizeof(StepRecord));
        }
        block_outcomes = cursor;
        cursor += PinnedStaging::rounded(count * 4 * sizeof(uint32_t));
        if (h->launch_block.bytes < cursor) h->launch_block.allocate(cursor);
        char* block = h->launch_block.base;
        char* image = h->staging.take(upload);
        for (uint32_t i = 0; i < count; ++i) {
            LaneDesc d = runs[i].lane->desc;
            d.steps = reinterpret_cast<const StepParams*>(block + steps_at[i]);
            d.records = reinterpret_cast<StepRecord*>(block + record_at[i]);
            d.step_count = static_cast<uint32_t>(runs[i].steps.size());
            d.launch = reinterpret_cast<LaunchWords*>(block + words_at + i * kWordsStride);
            std::memcpy(image + descs_at + i * sizeof(LaneDesc), &d, sizeof(LaneDesc));
            std::memset(image + words_at + i * kWordsStride, 0, sizeof(LaunchWords));
            if (!runs[i].steps.empty())
                std::memcpy(image + steps_at[i], runs[i].steps.data(), runs[i].steps.size() * sizeof(StepParams));
        }
        a = kernel_args(h, reinterpret_cast<LaneDesc*>(block + descs_at), count, P);
        a.lane_stride = stride;
        std::memcpy(image, &a, sizeof(KernelArgs));
        LEO_HIP_CHECK(hipMemcpyAsync(block, image, upload, hipMemcpyHostToDevice, h->staging.active()));
        device_args = reinterpret_cast<const KernelArgs*>(block);
    }
    if (!h->staging.route) h->staging.pending_uploads = true;
    h->staging.publish(h->stream);
    void* params[] = {&device_args};
    bool frozen_only = true;
    for (const LaneRun& r : runs) frozen_only = frozen_only && frozen_only_steps(r.steps);
    const void* kernel = step_kernel(h, frozen_only, a.redundant_global != 0);
    if (h->phase_profile)
        for (auto& r : runs) LEO_HIP_CHECK(hipMemsetAsync(r.lane->desc.phase_profile, 0, 2 * kPhases * 8, h->stream));
    q.start = start;
    q.stop = stop;
    LEO_HIP_CHECK(hipEventRecord(start, h->stream));
    LEO_HIP_CHECK(hipLaunchCooperativeKernel(kernel, dim3(stride * P), dim3(kThreads), params,
                                             step_lds_bytes(h->cfg.device.neurons_per_block), h->stream));
    LEO_HIP_CHECK(hipEventRecord(stop, h->stream));
    if (!single) {
        char* block = h->launch_block.base;
        hipLaunchKernelGGL(leo_lane_outcomes, dim3((count + kThreads - 1) / kThreads), dim3(kThreads), 0, h->stream,
                           device_args, reinterpret_cast<uint32_t*>(block + block_outcomes));
        LEO_HIP_CHECK(hipGetLastError());
    }
    h->staging.follow(h->stream);
    q.records.resize(count);
    q.ctl.resize(count);
    if (!single) {
        char* block = h->launch_block.base;
        const size_t end = block_outcomes + PinnedStaging::rounded(count * 4 * sizeof(uint32_t));
        const char* down = h->staging.d2h(block + block_records, end - block_records);
        for (uint32_t i = 0; i < count; ++i) q.records[i] = down + (record_at[i] - block_records);
        q.outcomes = down + (block_outcomes - block_records);
    }
    for (uint32_t i = 0; i < count; ++i) {
        if (single) {
            q.records[i] = h->staging.d2h(runs[i].lane->desc.records, runs[i].steps.size() * sizeof(StepRecord));
            q.ctl[i] = h->staging.d2h(runs[i].lane->desc.ctl, sizeof(LaneControl));
        }
        runs[i].lane->tick += static_cast<uint32_t>(runs[i].steps.size());
        q.end_tick.push_back(runs[i].lane->tick);
    }
    q.runs = std::move(runs);
    return q;
}

// The reference's error text for a device guard code (runtime.rs:1297, :1352,
// :1373, :1483, :1515, :1556).
std::string guard_message(uint32_t code, uint32_t bias_index) {
    switch (code) {
        case kErrBias: return "output bias " + std::to_string(bias_index) + " became non-finite";
        case kErrContextProjection: return "non-finite context output update rejected";
        case kErrContextEmbedding: return "non-finite context embedding update rejected";
        case kErrRecurrent: return "non-finite recurrent update rejected";
        case kErrInput: return "non-finite input update rejected";
        case kErrInhibitory: return "non-finite inhibitory update rejected";
        default: return "non-finite output update rejected";
    }
}

// Completes a queued launch once the transfer stream has drained past it:
// records, timing, telemetry, and the device's error and tick checks.
void complete_launch(LeoHipRuntime* h, QueuedLaunch& q) {
    const uint32_t count = static_cast<uint32_t>(q.runs.size());
    std::vector<LaneControl> ctl(count);
    for (uint32_t i = 0; i < count; ++i) {
        if (q.tally) {
            // no step records: the steps' metrics are not used, the work counters come from the totals
            q.runs[i].records.assign(q.runs[i].steps.size(), StepRecord{});
        } else {
            q.runs[i].records.resize(q.runs[i].steps.size());
            std::memcpy(q.runs[i].records.data(), q.records[i], q.runs[i].steps.size() * sizeof(StepRecord));
        }
        if (q.outcomes) {
            uint32_t w[4];
            std::memcpy(w, q.outcomes + 4 * sizeof(uint32_t) * i, sizeof(w));
            ctl[i].error_code = w[0];
            ctl[i].error_step = w[1];
            ctl[i].bias_fail = w[2];
            ctl[i].tick = w[3];
        } else {
            std::memcpy(&ctl[i], q.ctl[i], sizeof(LaneControl));
        }
    }
    float ms = 0.0f;
    LEO_HIP_CHECK(hipEventElapsedTime(&ms, q.start, q.stop));
    h->last_launch_ms = ms;
    account_launch(h, q.runs, ms, q.canonical, q.tally);
    if (h->phase_profile) {
        // lane 0 of the launch is representative (lanes run the same phase sequence)
        unsigned long long prof[2 * kPhases];
        download(prof, q.runs[0].lane->desc.phase_profile, sizeof(prof), h->stream);
        sync(h->stream);
        for (uint32_t p = 0; p < kPhases; ++p) {
            h->telemetry.phase_work_us[p] += static_cast<double>(prof[p]) / h->wall_clock_khz * 1e3;
            h->telemetry.phase_wait_us[p] += static_cast<double>(prof[kPhases + p]) / h->wall_clock_khz * 1e3;
        }
    }
    for (uint32_t i = 0; i < count; ++i) {
        if (ctl[i].error_code != 0) {
            const uint32_t code = ctl[i].error_code;
            LaneRun& run = q.runs[i];
            run.lane->error_seen = true;
            if (code == kErrBarrier) throw Error(LEO_ERR_DEVICE, "device lane barrier timed out");
            if (code == kErrCapacity)
                throw Error(LEO_ERR_UNSUPPORTED, "global selection exceeds the device sort capacity");
            // a numerical guard stopped the lane after the learning phase of
            // step error_step (runtime.rs: the step returns its error there):
            // the steps before it ran to the end, and the kernel left the tick
            // after the stopped step
            run.completed = std::min<size_t>(ctl[i].error_step, run.steps.size());
            run.lane->tick = ctl[i].tick;
            throw Error(LEO_ERR_NUMERICAL, guard_message(code, ctl[i].bias_fail) + " (device guard " +
                                               std::to_string(code) + ")");
        }
        if (ctl[i].tick != q.end_tick[i]) throw Error(LEO_ERR_INTERNAL, "device lane tick diverged from the host mirror");
    }
}

void run_lanes_once(LeoHipRuntime* h, std::vector<LaneRun>& runs) {
    const uint32_t count = static_cast<uint32_t>(runs.size());
    if (count == 0) return;
    std::vector<size_t> steps;
    for (auto& r : runs) {
        steps.push_back(r.steps.size());
        ensure_schedule(*r.lane, r.steps.size());
    }
    h->staging.reserve(launch_staging_bytes(count, steps));
    QueuedLaunch q = enqueue_lanes(h, std::move(runs), h->ev_start, h->ev_stop);
    LEO_HIP_CHECK(hipStreamSynchronize(h->staging.xfer));  // the kernel and its downloads are complete
    try {
        complete_launch(h, q);
    } catch (...) {
        runs = std::move(q.runs);
        h->staging.drain();
        throw;
    }
    runs = std::move(q.runs);
    h->staging.drain();
}

// Steps of the first launch of a long schedule: a launch stays around a
// second even when every synapse slot of every lane is eligible (about 140
// bytes per slot and step at ~4 TB/s), so a long schedule never becomes one
// multi-minute dispatch.
size_t max_steps_per_launch(const LeoHipRuntime* h, size_t lanes) {
    if (h->max_steps_override) return h->max_steps_override;
    const double bytes_per_step = static_cast<double>(h->z.ns) * 140.0 * static_cast<double>(std::max<size_t>(lanes, 1));
    const double steps = 4e12 / std::max(bytes_per_step, 1.0);
    return static_cast<size_t>(std::min(4096.0, std::max(8.0, steps)));
}

// The first launch of a canonical replay segment: the worst-case bound until
// a replay launch has been timed, then as many steps as the slowest timed
// replay launch's per-step average fits in a quarter of a second.
size_t first_canonical_chunk(const LeoHipRuntime* h) {
    const size_t bound = max_steps_per_launch(h, 1);
    if (h->max_steps_override || h->canonical_step_ms <= 0.0) return bound;
    const double fit = 250.0 / h->canonical_step_ms;
    return static_cast<size_t>(std::min(4096.0, std::max(static_cast<double>(bound), fit)));
}

// Later launches of a long schedule are sized from the last one's measured
// duration toward a quarter of a second (at most 4x growth per launch), so
// the step cost actually seen, not the worst case, sets the launch count.
size_t next_chunk(const LeoHipRuntime* h, size_t chunk) {
    if (h->max_steps_override) return h->max_steps_override;
    constexpr double kTargetMs = 250.0;
    const double factor = std::min(4.0, kTargetMs / std::max<double>(h->last_launch_ms, 0.01));
    const double next = static_cast<double>(chunk) * factor;
    return static_cast<size_t>(std::min(4096.0, std::max(8.0, next)));
}

// Runs the lanes' schedules, in several launches when they are long.
void run_lanes(LeoHipRuntime* h, std::vector<LaneRun>& runs) {
    size_t longest = 0;
    for (const LaneRun& r : runs) longest = std::max(longest, r.steps.size());
    size_t chunk = max_steps_per_launch(h, runs.size());
    if (longest <= chunk) {
        run_lanes_once(h, runs);
        return;
    }
    for (LaneRun& r : runs) r.records.resize(r.steps.size());
    for (size_t at = 0; at < longest;) {
        const size_t step = chunk;
        std::vector<LaneRun> part;
        std::vector<size_t> index;
        for (size_t i = 0; i < runs.size(); ++i) {
            const size_t n = runs[i].steps.size();
            if (at >= n) continue;
            const size_t end = std::min(n, at + step);
            part.push_back(LaneRun{runs[i].lane, std::vector<StepParams>(runs[i].steps.begin() + at,
                                                                         runs[i].steps.begin() + end), {}});
            index.push_back(i);
        }
        auto keep = [&] {
            for (size_t k = 0; k < part.size(); ++k) {
                std::copy(part[k].records.begin(), part[k].records.end(), runs[index[k]].records.begin() + at);
                if (part[k].completed != kAllSteps) runs[index[k]].completed = at + part[k].completed;
            }
        };
        try {
            run_lanes_once(h, part);
        } catch (...) {
            keep();
            throw;
        }
        keep();
        at += step;
        chunk = next_chunk(h, step);
    }
}

// Statistics of one step (runtime.rs:1595-1622) from its device record.
void account_step(LeoStatistics& st, const StepParams& sp, const StepRecord& rec, float loss, uint32_t synapses) {
    if (sp.flags & kStepFrozen) return;
    if (sp.symbol < 256) st.processed_bytes += 1;
    if (sp.target_index >= 0) {
        st.training_loss_sum += static_cast<double>(loss);
        st.training_targets += 1;
    }
    st.active_neurons_sum += rec.active;
    st.active_neurons_peak = std::max<uint64_t>(st.active_neurons_peak, rec.active);
    st.synaptic_events += static_cast<uint64_t>(rec.active) * synapses;
    st.persistent_ticks += 1;
}

float step_loss(const StepParams& sp, const StepRecord& rec) {
    if (sp.target_index < 0) return NAN;
    return -std::log(std::max(rec.p_target, 1.0e-12f));  // runtime.rs:471 (glibc logf)
}

LeoStepMetrics to_metrics(const StepParams& sp, const StepRecord& rec, float loss) {
    LeoStepMetrics m{};
    m.loss = loss;
    m.has_loss = sp.target_index >= 0 ? 1 : 0;
    m.predicted_symbol = rec.predicted < 256 ? rec.predicted : kEnd;
    m.active_neurons = rec.active;
    m.suprathreshold_neurons = rec.suprathreshold;
    m.block_selected_neurons = rec.block_selected;
    m.global_cap_clipped_neurons = rec.clipped;
    m.population_inhibition = rec.population_inhibition;
    m.context_cells = rec.context_cells;
    m.context_probes = rec.context_probes;
    m.context_applied = rec.context_applied;
    m.eligible_recurrent_synapses = rec.eligible_rec;
    m.eligible_input_synapses = rec.eligible_in;
    m.target_probability = sp.target_index >= 0 ? rec.p_target : NAN;
    m.error_code = rec.error_code;
    return m;
}

// The canonical runtime's host mirrors after its steps ran (statistics,
// revision, persistent activity, as Runtime::step keeps them), and the steps'
// metrics appended to `out`.
void absorb_canonical(LeoHipRuntime* h, const LaneRun& r, std::vector<LeoStepMetrics>& out) {
    for (size_t i = 0; i < r.steps.size(); ++i) {
        float loss = step_loss(r.steps[i], r.records[i]);
        account_step(h->stats, r.steps[i], r.records[i], loss, h->cfg.device.synapses_per_neuron);
        if (r.steps[i].flags & kStepLearn) h->revision += 1;
        if (!(r.steps[i].flags & kStepFrozen)) r.lane->persistent_activity = true;
        LeoStepMetrics m = to_metrics(r.steps[i], r.records[i], loss);
        m.emitted_events = r.records[i].active * h->cfg.device.synapses_per_neuron;
        out.push_back(m);
    }
}

// After a numerical guard stopped the canonical lane: the steps before the
// stopped one count as the reference counts them (the stopped step's error
// returns before its revision, homeostasis and statistics), and the
// plasticity phase is the one the stopped step started from.
void absorb_stopped(LeoHipRuntime* h, LaneRun& r, std::vector<LeoStepMetrics>& out) {
    if (r.completed == kAllSteps) return;
    const size_t n = std::min(r.completed, r.records.size());
    if (r.completed < r.phase.size()) r.lane->plasticity_phase = r.phase[r.completed];
    r.steps.resize(n);
    r.records.resize(n);
    absorb_canonical(h, r, out);
}

// Execute steps on the canonical runtime; stats and revision update the
// canonical mirrors exactly as Runtime::step does.
// `outputs[i]` asks for the readout of step i even when it does not learn.
std::vector<LeoStepMetrics> canonical_steps(LeoHipRuntime* h, const std::vector<HostStep>& steps,
                                            const std::vector<int32_t>& permissions, const std::vector<bool>& outputs) {
    Lane& lane = *h->canonical;
    LaneRun run{&lane, {}, {}};
    run.steps.reserve(steps.size());
    uint32_t tick = lane.tick;
    for (size_t i = 0; i < steps.size(); ++i) {
        run.phase.push_back(lane.plasticity_phase);
        run.steps.push_back(
            make_step(h->cfg, lane, steps[i].symbol, steps[i].target, permissions[i], tick++, outputs[i]));
    }
    std::vector<LaneRun> runs;
    runs.push_back(std::move(run));
    std::vector<LeoStepMetrics> out;
    try {
        run_lanes(h, runs);
    } catch (...) {
        absorb_stopped(h, runs[0], out);
        throw;
    }
    out.reserve(steps.size());
    absorb_canonical(h, runs[0], out);
    return out;
}

std::vector<LeoStepMetrics> canonical_steps(LeoHipRuntime* h, const std::vector<HostStep>& steps,
                                            const std::vector<int32_t>& permissions, bool output) {
    return canonical_steps(h, steps, permissions, std::vector<bool>(steps.size(), output));
}

void canonical_reset(LeoHipRuntime* h) {
    std::vector<Lane*> lanes{h->canonical.get()};
    reset_lane_objects(h, lanes, false, 0);
    sync(h->stream);
}

// A run of canonical steps after an optional reset (one replay segment).
struct CanonicalSegment {
    bool reset_before = false;
    std::vector<HostStep> steps;
    std::vector<int32_t> permissions;
};

// Frozen prefix steps at the start of a replay segment (the permission alone
// makes a canonical step frozen without output: make_step).
size_t leading_frozen_steps(const CanonicalSegment& seg) {
    size_t n = 0;
    while (n < seg.permissions.size() && seg.permissions[n] == LEO_FROZEN) ++n;
    return n;
}
// The shortest leading frozen run that is launched on its own.
constexpr size_t kFrozenLaunchMin = 64;
// Launches whose results come down in one copy.
constexpr size_t kResultChunk = 32;

// Runs the segments on the canonical runtime as the sequential executor
// would (reset, then the steps, segment by segment), with every reset,
// upload, launch and results download queued back to back before the host
// waits for the first results. Launches take the first launch's step count,
// then four times the previous one (at most 4096); the results do not depend
// on how the steps are cut into launches. Metrics of the steps are appended
// to `out` in order.
void run_canonical_segments(LeoHipRuntime* h, const std::vector<CanonicalSegment>& segments,
                            std::vector<LeoStepMetrics>& out) {
    Lane& lane = *h->canonical;
    if (h->phase_profile) {  // the profiling build reads its clocks launch by launch
        for (const CanonicalSegment& seg : segments) {
            if (seg.reset_before) canonical_reset(h);
            auto m = canonical_steps(h, seg.steps, seg.permissions, false);
            out.insert(out.end(), m.begin(), m.end());
        }
        return;
    }
    // launch cuts and the staging they need, known before anything is queued
    std::vector<std::vector<size_t>> cuts(segments.size());
    size_t staged = 0, launches = 0;
    for (size_t k = 0; k < segments.size(); ++k) {
        if (segments[k].reset_before) staged += PinnedStaging::rounded(sizeof(LaneDesc));
        size_t chunk = first_canonical_chunk(h);
        // a long leading run of frozen prefix steps gets launches of its own
        // (the frozen-only kernel's), the rest of the segment the others
        const size_t frozen_run = h->frozen_kernel ? leading_frozen_steps(segments[k]) : 0;
        const size_t split = frozen_run >= kFrozenLaunchMin ? frozen_run : 0;
        for (size_t at = 0; at < segments[k].steps.size();) {
            const size_t end = at < split ? split : segments[k].steps.size();
            const size_t n = std::min(chunk, end - at);
            cuts[k].push_back(n);
            staged += launch_staging_bytes(1, {n});
            at += n;
            chunk = std::min<size_t>(4096, chunk * 4);
        }
        launches += cuts[k].size();
    }
    if (launches == 0) {
        for (const CanonicalSegment& seg : segments)
            if (seg.reset_before) canonical_reset(h);
        return;
    }
    // The launches' step records and outcomes stay on the device: each launch
    // stores its predecessor's outcome as it starts, in the slot in front of
    // its own records. They come down in chunks of launches, one copy behind
    // a chunk's last launch, and the host takes a chunk in while the later
    // launches run (a launch's outcome arrives with its successor's chunk;
    // the last launch's, with the lane's control words).
    constexpr size_t kSlot = 256, kTallyAt = 64;
    static_assert(kTallyAt >= 4 * sizeof(uint32_t) && kTallyAt + kTallyWords * sizeof(uint32_t) <= kSlot,
                  "outcome and totals share a launch's slot");
    std::vector<size_t> record_at;
    size_t results_bytes = 0;
    for (const auto& c : cuts)
        for (size_t n : c) {
            results_bytes += kSlot;
            record_at.push_back(results_bytes);
            results_bytes += PinnedStaging::rounded(n * sizeof(StepRecord));
        }
    auto records_end = [&](size_t i) { return i + 1 < launches ? record_at[i + 1] - kSlot : results_bytes; };
    // Every launch's kernel arguments, lane descriptor, zeroed barrier words
    // and step parameters go up in one copy before the first launch, so that
    // the stream holds nothing between two launches of a segment but their
    // timing events.
    constexpr size_t kPlanDesc = 512, kPlanWords = 960, kPlanHeader = 1024;
    static_assert(sizeof(KernelArgs) <= kPlanDesc && kPlanDesc + sizeof(LaneDesc) <= kPlanWords &&
                      kPlanWords + sizeof(LaunchWords) <= kPlanHeader,
                  "launch plan header");
    std::vector<size_t> plan_at;
    size_t plan_bytes = 0;
    for (const auto& c : cuts)
        for (size_t n : c) {
            plan_at.push_back(plan_bytes);
            plan_bytes += kPlanHeader + PinnedStaging::rounded(n * sizeof(StepParams));
        }
    staged += results_bytes + PinnedStaging::rounded(sizeof(LaneControl));
    sync(h->stream);
    if (h->replay_results.bytes < results_bytes) h->replay_results.allocate(results_bytes);
    if (h->replay_plan.bytes < plan_bytes) h->replay_plan.allocate(plan_bytes);
    const size_t chunks = (launches + kResultChunk - 1) / kResultChunk;
    while (h->chunk_events.size() < chunks) {
        hipEvent_t e;
        LEO_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        h->chunk_events.push_back(e);
    }
    h->staging.reserve(staged);
    while (h->launch_events.size() < 2 * launches) {
        hipEvent_t e;
        LEO_HIP_CHECK(hipEventCreate(&e));
        h->launch_events.push_back(e);
    }
    const LanePlan shape = choose_wgs_per_lane(h, 1, true);
    const uint32_t P = shape.P, stride = shape.stride;
    if (P > kMaxLaneWgs) throw Error(LEO_ERR_INTERNAL, "more workgroups per lane than barrier flags");
    if (static_cast<uint64_t>(shape.grid) > cooperative_capacity(h->cus, h->coop_blocks_per_cu))
        throw Error(LEO_ERR_INTERNAL, "cooperative launch exceeds the resident workgroup capacity");
    // the host part, in the executor's order: the lane's mirrors through the
    // resets and steps, every launch's schedule and header
    char* results = h->replay_results.base;
    char* plan = h->replay_plan.base;
    char* image = h->staging.take(plan_bytes);
    std::vector<QueuedLaunch> queued;
    std::vector<const void*> kernels;
    std::vector<const KernelArgs*> device_args;
    std::vector<bool> tallied;
    queued.reserve(launches);
    for (size_t k = 0; k < segments.size(); ++k) {
        const CanonicalSegment& seg = segments[k];
        if (seg.reset_before) reset_lane_mirrors({&lane}, false, 0);
        size_t at = 0;
        for (size_t n : cuts[k]) {
            const size_t i = queued.size();
            LaneRun run{&lane, {}, {}};
            run.steps.reserve(n);
            check_tick_range(h, lane.tick, n);
            uint32_t tick = lane.tick;
            for (size_t j = at; j < at + n; ++j) {
                run.phase.push_back(lane.plasticity_phase);
                run.steps.push_back(make_step(h->cfg, lane, seg.steps[j].symbol, seg.steps[j].target,
                                              seg.permissions[j], tick++, false));
            }
            mark_early_delivery(run.steps);
            char* dev = plan + plan_at[i];
            LaneDesc desc = lane.desc;
            desc.steps = reinterpret_cast<const StepParams*>(dev + kPlanHeader);
            desc.records = reinterpret_cast<StepRecord*>(results + record_at[i]);
            desc.step_count = static_cast<uint32_t>(n);
            desc.outcome = i > 0 ? reinterpret_cast<uint32_t*>(results + record_at[i] - kSlot) : nullptr;
            desc.launch = reinterpret_cast<LaunchWords*>(dev + kPlanWords);
            KernelArgs a = kernel_args(h, reinterpret_cast<LaneDesc*>(dev + kPlanDesc), 1, P);
            a.lane_stride = stride;
            // the replay discards frozen steps' metrics: a frozen-only launch
            // keeps only its totals, in its slot after the predecessor's outcome
            const void* kernel = step_kernel(h, frozen_only_steps(run.steps), a.redundant_global != 0);
            const bool tally = h->tally_launches && kernel == reinterpret_cast<const void*>(&leo_lane_steps_frozen);
            if (tally) a.tally = reinterpret_cast<uint32_t*>(results + record_at[i] - kSlot + kTallyAt);
            char* img = image + plan_at[i];
            std::memcpy(img, &a, sizeof(KernelArgs));
            std::memcpy(img + kPlanDesc, &desc, sizeof(LaneDesc));
            std::memset(img + kPlanWords, 0, sizeof(LaunchWords));
            std::memcpy(img + kPlanHeader, run.steps.data(), n * sizeof(StepParams));
            kernels.push_back(kernel);
            device_args.push_back(reinterpret_cast<const KernelArgs*>(dev));
            lane.tick += static_cast<uint32_t>(n);
            QueuedLaunch q;
            q.runs.push_back(std::move(run));
            q.records.resize(1);
            q.ctl.resize(1);
            q.end_tick.push_back(lane.tick);
            q.start = h->launch_events[2 * i];
            q.stop = h->launch_events[2 * i + 1];
            q.canonical = true;
            tallied.push_back(tally);
            queued.push_back(std::move(q));
            at += n;
        }
    }
    // the device part: one stream, in queue order (no event handoff between
    // streams): the upload, then resets, launches and result downloads
    std::vector<size_t> chunk_from;
    std::vector<const char*> chunk_host;
    const char* last_ctl = nullptr;
    StagingRoute on_step_stream(h->staging, h->stream);
    LEO_HIP_CHECK(hipMemcpyAsync(plan, image, plan_bytes, hipMemcpyHostToDevice, h->stream));
    const uint32_t lds = step_lds_bytes(h->cfg.device.neurons_per_block);
    size_t i = 0;
    for (size_t k = 0; k < segments.size(); ++k) {
        if (segments[k].reset_before) {
            if (cuts[k].empty()) {
                reset_lane_device(h, {&lane}, false, 0);
            } else {
                // the descriptor in the next launch's header holds the lane's
                // state as the reset reads it
                clear_reported_error(lane, h->stream);
                reset_lanes(h, 1, false, 0, reinterpret_cast<LaneDesc*>(plan + plan_at[i] + kPlanDesc));
            }
        }
        for (size_t c = 0; c < cuts[k].size(); ++c, ++i) {
            clear_reported_error(lane, h->stream);
            void* params[] = {&device_args[i]};
            LEO_HIP_CHECK(hipEventRecord(queued[i].start, h->stream));
            LEO_HIP_CHECK(hipLaunchCooperativeKernel(kernels[i], dim3(stride * P), dim3(kThreads), params, lds, h->stream));
            LEO_HIP_CHECK(hipEventRecord(queued[i].stop, h->stream));
            if ((i + 1) % kResultChunk == 0 || i + 1 == launches) {
                if (i + 1 == launches) last_ctl = h->staging.d2h(lane.desc.ctl, sizeof(LaneControl));
                const size_t from = record_at[(i / kResultChunk) * kResultChunk] - kSlot;
                chunk_from.push_back(from);
                chunk_host.push_back(h->staging.d2h(results + from, records_end(i) - from));
                LEO_HIP_CHECK(hipEventRecord(h->chunk_events[i / kResultChunk], h->stream));
            }
        }
    }
    // where a device offset of the results arrived, once its chunk is in
    size_t chunks_in = 0;
    auto arrived = [&](size_t i, size_t offset) {
        const size_t c = i / kResultChunk;
        for (; chunks_in <= c; ++chunks_in) LEO_HIP_CHECK(hipEventSynchronize(h->chunk_events[chunks_in]));
        return chunk_host[c] + (offset - chunk_from[c]);
    };
    try {
        for (size_t i = 0; i < queued.size(); ++i) {
            QueuedLaunch& q = queued[i];
            // the outcome as the successor found it, or the control words
            LaneControl outcome{};
            if (i + 1 < queued.size()) {
                uint32_t w[4];
                std::memcpy(w, arrived(i + 1, record_at[i + 1] - kSlot), sizeof(w));
                outcome.error_code = w[0];
                outcome.error_step = w[1];
                outcome.bias_fail = w[2];
                outcome.tick = w[3];
            } else {
                arrived(i, record_at[i]);
                std::memcpy(&outcome, last_ctl, sizeof(LaneControl));
            }
            q.records[0] = arrived(i, record_at[i]);
            q.ctl[0] = reinterpret_cast<const char*>(&outcome);
            if (tallied[i]) q.tally = arrived(i, record_at[i] - kSlot + kTallyAt);
            try {
                complete_launch(h, q);
            } catch (...) {
                // the launches queued behind a stopped one found the sticky
                // error word set and ran nothing
                absorb_stopped(h, q.runs[0], out);
                throw;
            }
            if (const size_t n = q.runs[0].steps.size())
                h->canonical_step_ms = std::max(h->canonical_step_ms, static_cast<double>(h->last_launch_ms) / n);
            absorb_canonical(h, q.runs[0], out);
        }
    } catch (...) {
        h->staging.drain();
        throw;
    }
    h->staging.drain();
}

void canonical_finish_document(LeoHipRuntime* h) {  // runtime.rs:357-363
    if (h->canonical->persistent_activity) h->stats.processed_stories += 1;
    canonical_reset(h);
}

std::vector<HostStep> document_steps(const uint8_t* story, size_t len) {  // training.rs:1747-1757
    std::vector<HostStep> steps;
    steps.reserve(len + 1);
    steps.push_back({kBegin, story[0]});
    for (size_t i = 0; i + 1 < len; ++i) steps.push_back({story[i], story[i + 1]});
    steps.push_back({story[len - 1], static_cast<int32_t>(kEnd)});
    return steps;
}

bool has_negative_zero(const float* v, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t bits;
        std::memcpy(&bits, v + i, 4);
        if (bits == 0x80000000u) return true;
    }
    return false;
}

// Host layouts <-> device layouts.
void upload_model(LeoHipRuntime* h, const LeoModelView& m) {
    const Sizes& z = h->z;
    hipStream_t s = h->stream;
    h->negative_zero_weights = has_negative_zero(m.rec_weight, z.ns) || has_negative_zero(m.in_weight, z.ni);
    upload(h->canon.threshold, m.threshold, z.n * 4, s);
    upload(h->canon.rec_weight, m.rec_weight, z.ns * 4, s);
    upload(h->canon.in_weight, m.in_weight, z.ni * 4, s);
    std::vector<float> rows(z.n * kOutStride, 0.0f);
    for (uint64_t o = 0; o < kOutputs; ++o)
        for (uint64_t n = 0; n < z.n; ++n) rows[n * kOutStride + o] = m.out_weight[o * z.n + n];
    upload(h->canon.out_w, rows.data(), rows.size() * 4, s);
    std::vector<float> bias(kOutStride, 0.0f);
    std::copy(m.bias, m.bias + kOutputs, bias.begin());
    upload(h->canon.bias, bias.data(), kOutStride * 4, s);
    upload(h->canon.ctx_keys, m.ctx_keys, z.slots * 8, s);
    upload(h->canon.ctx_emb, m.ctx_emb, z.slots * z.e * 4, s);
    upload(h->canon.ctx_obs, m.ctx_obs, z.slots * 4, s);
    upload(h->canon.ctx_out, m.ctx_out, kOutputs * z.e * 4, s);
    sync(s);
    h->generation = m.generation;
    h->revision = m.parameter_revision;
    h->stats = m.statistics;
}

void upload_topology(LeoHipRuntime* h, const LeoModelView& m) {
    const Sizes& z = h->z;
    h->excitability.assign(m.excitability, m.excitability + z.n);
    h->neuron_type.assign(m.neuron_type, m.neuron_type + z.n);
    h->rec_target.assign(m.rec_target, m.rec_target + z.ns);
    h->rec_branch.assign(m.rec_branch, m.rec_branch + z.ns);
    h->rec_delay.assign(m.rec_delay, m.rec_delay + z.ns);
    h->in_target.assign(m.in_target, m.in_target + z.ni);
    h->in_branch.assign(m.in_branch, m.in_branch + z.ni);
    // per-target delivery bucket capacity: recurrent in-degree + the largest
    // number of times one input row names the target
    std::vector<uint64_t> cap(z.n, 0);
    for (uint64_t i = 0; i < z.ns; ++i) cap[m.rec_target[i]] += 1;
    std::vector<uint32_t> row_count(z.n, 0), row_max(z.n, 0);
    for (uint64_t sym = 0; sym < kSymbols; ++sym) {
        for (uint64_t i = 0; i < z.f; ++i) {
            uint32_t t = m.in_target[sym * z.f + i];
            row_count[t] += 1;
            row_max[t] = std::max(row_max[t], row_count[t]);
        }
        for (uint64_t i = 0; i < z.f; ++i) row_count[m.in_target[sym * z.f + i]] = 0;
    }
    // entries p < kFixedEntries of target n live at kFixedEntries*n + p; the
    // rest at offsets[n] + (p - kFixedEntries), after the fixed entries
    std::vector<uint64_t> offsets(z.n + 1, 0);
    offsets[0] = kFixedEntries * z.n;
    for (uint64_t n = 0; n < z.n; ++n) {
        const uint64_t need = cap[n] + row_max[n];
        offsets[n + 1] = offsets[n] + (need > kFixedEntries ? need - kFixedEntries : 0);
    }
    h->z.bucket_total = offsets[z.n];
    // sort space of the deep buckets: every target whose bucket can hold
    // more entries than the in-register sort takes gets a range of its
    // capacity (the radix sort's second buffer)
    std::vector<uint64_t> shadow(z.n + 1, 0);
    for (uint64_t n = 0; n < z.n; ++n) {
        const uint64_t need = cap[n] + row_max[n];
        shadow[n + 1] = shadow[n] + (need > kDeepRegisterEntries ? need : 0);
    }
    h->z.shadow_total = shadow[z.n];
    Layout l;
    size_t o_ex = l.add<float>(z.n), o_ty = l.add<uint8_t>(z.n), o_rt = l.add<uint32_t>(z.ns);
    size_t o_rb = l.add<uint8_t>(z.ns), o_rd = l.add<uint8_t>(z.ns), o_it = l.add<uint32_t>(z.ni);
    size_t o_ib = l.add<uint8_t>(z.ni), o_off = l.add<uint64_t>(z.n + 1), o_edge = l.add<uint32_t>(z.ns);
    size_t o_sho = l.add<uint64_t>(z.n + 1), o_iedge = l.add<uint32_t>(z.ni);
    h->shared.allocate(l.cursor);
    char* b = h->shared.base;
    h->sm.excitability = reinterpret_cast<const float*>(b + o_ex);
    h->sm.neuron_type = reinterpret_cast<const uint8_t*>(b + o_ty);
    h->sm.rec_target = reinterpret_cast<const uint32_t*>(b + o_rt);
    h->sm.rec_branch = reinterpret_cast<const uint8_t*>(b + o_rb);
    h->sm.rec_delay = reinterpret_cast<const uint8_t*>(b + o_rd);
    h->sm.in_target = reinterpret_cast<const uint32_t*>(b + o_it);
    h->sm.in_branch = reinterpret_cast<const uint8_t*>(b + o_ib);
    h->sm.bucket_offset = reinterpret_cast<const uint64_t*>(b + o_off);
    h->sm.rec_edge = reinterpret_cast<const uint32_t*>(b + o_edge);
    h->sm.shadow_offset = reinterpret_cast<const uint64_t*>(b + o_sho);
    h->sm.in_edge = reinterpret_cast<const uint32_t*>(b + o_iedge);
    std::vector<uint32_t> edges(z.ns);
    for (uint64_t i = 0; i < z.ns; ++i) edges[i] = pack_edge(m.rec_target[i], m.rec_delay[i], m.rec_branch[i]);
    std::vector<uint32_t> in_edges(z.ni);  // the delay field is unused (log2 delay 0)
    for (uint64_t i = 0; i < z.ni; ++i) in_edges[i] = pack_edge(m.in_target[i], 1, m.in_branch[i]);
    hipStream_t s = h->stream;
    upload(b + o_ex, m.excitability, z.n * 4, s);
    upload(b + o_ty, m.neuron_type, z.n, s);
    upload(b + o_rt, m.rec_target, z.ns * 4, s);
    upload(b + o_rb, m.rec_branch, z.ns, s);
    upload(b + o_rd, m.rec_delay, z.ns, s);
    upload(b + o_it, m.in_target, z.ni * 4, s);
    upload(b + o_ib, m.in_branch, z.ni, s);
    upload(b + o_off, offsets.data(), offsets.size() * 8, s);
    upload(b + o_sho, shadow.data(), shadow.size() * 8, s);
    upload(b + o_edge, edges.data(), z.ns * 4, s);
    upload(b + o_iedge, in_edges.data(), z.ni * 4, s);
    sync(s);
}

void download_model(LeoHipRuntime* h, LeoModelView& m) {
    const Sizes& z = h->z;
    hipStream_t s = h->stream;
    std::copy(h->excitability.begin(), h->excitability.end(), m.excitability);
    std::copy(h->neuron_type.begin(), h->neuron_type.end(), m.neuron_type);
    std::copy(h->rec_target.begin(), h->rec_target.end(), m.rec_target);
    std::copy(h->rec_branch.begin(), h->rec_branch.end(), m.rec_branch);
    std::copy(h->rec_delay.begin(), h->rec_delay.end(), m.rec_delay);
    std::copy(h->in_target.begin(), h->in_target.end(), m.in_target);
    std::copy(h->in_branch.begin(), h->in_branch.end(), m.in_branch);
    download(m.threshold, h->canon.threshold, z.n * 4, s);
    download(m.rec_weight, h->canon.rec_weight, z.ns * 4, s);
    download(m.in_weight, h->canon.in_weight, z.ni * 4, s);
    std::vector<float> rows(z.n * kOutStride);
    download(rows.data(), h->canon.out_w, rows.size() * 4, s);
    std::vector<float> bias(kOutStride);
    download(bias.data(), h->canon.bias, kOutStride * 4, s);
    download(m.ctx_keys, h->canon.ctx_keys, z.slots * 8, s);
    download(m.ctx_emb, h->canon.ctx_emb, z.slots * z.e * 4, s);
    download(m.ctx_obs, h->canon.ctx_obs, z.slots * 4, s);
    download(m.ctx_out, h->canon.ctx_out, kOutputs * z.e * 4, s);
    sync(s);
    for (uint64_t o = 0; o < kOutputs; ++o)
        for (uint64_t n = 0; n < z.n; ++n) m.out_weight[o * z.n + n] = rows[n * kOutStride + o];
    std::copy(bias.begin(), bias.begin() + kOutputs, m.bias);
    m.generation = h->generation;
    m.parameter_revision = h->revision;
    m.statistics = h->stats;
}

// ---------------------------------------------------------------------------
// Keyed context merge on the host (parallel.rs:916-973, 1024-1113, 1226-1233).
// ---------------------------------------------------------------------------
struct HostContext {
    std::vector<uint64_t> keys;
    std::vector<uint32_t> obs;
    std::vector<float> emb;
};

int64_t find_context_slot(const HostContext& c, const LeoHostConfig& cfg, size_t order, uint64_t key) {
    const uint64_t spo = cfg.device.context_slots_per_order;
    const uint64_t base = (order - 1) * spo, start = key % spo;
    for (uint64_t off = 0; off < cfg.device.context_probe_limit; ++off) {
        uint64_t slot = base + (start + off) % spo;
        if (c.keys[slot] == key) return static_cast<int64_t>(slot);
    }
    return -1;
}

int64_t resolve_context_slot(HostContext& c, const LeoHostConfig& cfg, size_t order, uint64_t key, bool allocate,
                             size_t E) {  // model.rs:173-221
    const uint64_t spo = cfg.device.context_slots_per_order;
    const uint64_t base = (order - 1) * spo, start = key % spo;
    int64_t empty = -1;
    uint64_t weakest = base + start;
    uint32_t weakest_obs = UINT32_MAX;
    for (uint64_t off = 0; off < cfg.device.context_probe_limit; ++off) {
        uint64_t slot = base + (start + off) % spo;
        if (c.keys[slot] == key) return static_cast<int64_t>(slot);
        if (c.keys[slot] == 0 && empty < 0) empty = static_cast<int64_t>(slot);
        if (c.obs[slot] < weakest_obs) {
            weakest_obs = c.obs[slot];
            weakest = slot;
        }
    }
    if (!allocate) return -1;
    uint64_t slot = empty >= 0 ? static_cast<uint64_t>(empty) : weakest;
    if (c.keys[slot] != key) {
        c.keys[slot] = key;
        c.obs[slot] = 0;
        std::fill(c.emb.begin() + slot * E, c.emb.begin() + (slot + 1) * E, 0.0f);
    }
    return static_cast<int64_t>(slot);
}

HostContext download_context(LeoHipRuntime* h, const LaneParams& p) {
    const Sizes& z = h->z;
    HostContext c;
    c.keys.resize(z.slots);
    c.obs.resize(z.slots);
    c.emb.resize(z.slots * z.e);
    download(c.keys.data(), p.ctx_keys, z.slots * 8, h->stream);
    download(c.obs.data(), p.ctx_obs, z.slots * 4, h->stream);
    download(c.emb.data(), p.ctx_emb, z.slots * z.e * 4, h->stream);
    return c;
}

std::vector<uint32_t> download_bits(LeoHipRuntime* h, const uint32_t* bits, uint64_t count) {
    std::vector<uint32_t> v((count + 31) / 32);
    download(v.data(), bits, v.size() * 4, h->stream);
    return v;
}

std::vector<uint64_t> bits_to_indices(const std::vector<uint32_t>& bits, uint64_t count) {
    std::vector<uint64_t> out;
    for (uint64_t w = 0; w < bits.size(); ++w) {
        uint32_t v = bits[w];
        while (v) {
            int b = __builtin_ctz(v);
            uint64_t idx = w * 32 + static_cast<uint64_t>(b);
            if (idx < count) out.push_back(idx);
            v &= v - 1;
        }
    }
    return out;
}

// A story lane's changed context slots (the slots of its change bitmap):
// slot, key, observations and embedding row of each, in no particular order.
struct LaneContext {
    std::vector<uint32_t> slot;
    std::vector<uint64_t> key;
    std::vector<uint32_t> obs;
    std::vector<float> emb;
};

// The changed context slots of story lanes, gathered on the device
// (leo_context_changes) and downloaded: one record per changed slot instead
// of every lane's whole tables.
void download_lane_contexts(LeoHipRuntime* h, const std::vector<Lane*>& lanes, std::vector<LaneContext>& lane_ctx) {
    const Sizes& z = h->z;
    const uint32_t L = static_cast<uint32_t>(lanes.size());
    if (L == 0) return;
    const uint64_t rec_words = 4 + z.e, stride = z.slots * rec_words;
    const size_t tables = 4 * static_cast<size_t>(L) * sizeof(void*);
    const size_t counts_at = (tables + 255) & ~size_t(255);
    const size_t out_at = (counts_at + L * 8 + 255) & ~size_t(255);
    const size_t need = out_at + static_cast<size_t>(L) * stride * 4;
    if (h->ctx_scratch.bytes < need) h->ctx_scratch.allocate(need);
    std::vector<const void*> ptrs(4 * L);
    for (uint32_t l = 0; l < L; ++l) {
        const LaneDesc& d = lanes[l]->desc;
        ptrs[0 * L + l] = d.ch_ctx;
        ptrs[1 * L + l] = d.p.ctx_keys;
        ptrs[2 * L + l] = d.p.ctx_obs;
        ptrs[3 * L + l] = d.p.ctx_emb;
    }
    char* base = h->ctx_scratch.base;
    upload(base, ptrs.data(), tables, h->stream);
    auto* counts = reinterpret_cast<unsigned long long*>(base + counts_at);
    LEO_HIP_CHECK(hipMemsetAsync(counts, 0, L * 8, h->stream));
    ContextChanges g{};
    g.bits = reinterpret_cast<const uint32_t* const*>(base);
    g.keys = reinterpret_cast<const uint64_t* const*>(base + 1 * L * sizeof(void*));
    g.obs = reinterpret_cast<const uint32_t* const*>(base + 2 * L * sizeof(void*));
    g.emb = reinterpret_cast<const float* const*>(base + 3 * L * sizeof(void*));
    g.slots = z.slots;
    g.words = z.words(z.slots);
    g.stride = stride;
    g.E = static_cast<uint32_t>(z.e);
    g.out = reinterpret_cast<uint32_t*>(base + out_at);
    g.counts = counts;
    const uint64_t blocks = std::min<uint64_t>((g.words + kThreads - 1) / kThreads, 64);
    hipLaunchKernelGGL(leo_context_changes, dim3(static_cast<uint32_t>(std::max<uint64_t>(blocks, 1)), L),
                       dim3(kThreads), 0, h->stream, g);
    LEO_HIP_CHECK(hipGetLastError());
    std::vector<unsigned long long> n(L);
    download(n.data(), counts, L * 8, h->stream);
    sync(h->stream);
    std::vector<uint32_t> packed;
    for (uint32_t l = 0; l < L; ++l) {
        if (n[l] > z.slots) throw Error(LEO_ERR_INTERNAL, "more changed context slots than slots");
        packed.resize(n[l] * rec_words);
        if (n[l]) download(packed.data(), g.out + l * stride, packed.size() * 4, h->stream);
        sync(h->stream);
        LaneContext c;
        c.slot.resize(n[l]);
        c.key.resize(n[l]);
        c.obs.resize(n[l]);
        c.emb.resize(n[l] * z.e);
        for (uint64_t k = 0; k < n[l]; ++k) {
            const uint32_t* r = packed.data() + k * rec_words;
            c.slot[k] = r[0];
            c.key[k] = static_cast<uint64_t>(r[1]) | (static_cast<uint64_t>(r[2]) << 32);
            c.obs[k] = r[3];
            std::memcpy(c.emb.data() + k * z.e, r + 4, z.e * 4);
        }
        lane_ctx.push_back(std::move(c));
    }
}

size_t merge_context_downloaded(LeoHipRuntime* h, const std::vector<LaneContext>& lane_ctx);

size_t merge_context(LeoHipRuntime* h, const std::vector<Lane*>& lanes) {
    std::vector<LaneContext> lane_ctx;
    download_lane_contexts(h, lanes, lane_ctx);
    return merge_context_downloaded(h, lane_ctx);
}

// Keyed context merge (parallel.rs:1024-1113, projection and validation
// :1169-1345) over every lane's changed context slots. Each (order, key)
// gets one f64 sum per embedding column, accumulated lane by lane in lane
// order (a key appears at most once in a lane's table), so the sums are those
// of the reference's per-key walk over the workers; an open-addressing table
// finds a key's sum in one probe run instead of a scan over every lane.
size_t merge_context_downloaded(LeoHipRuntime* h, const std::vector<LaneContext>& lane_ctx) {
    const Sizes& z = h->z;
    const size_t E = z.e;
    const uint64_t spo = h->cfg.device.context_slots_per_order;
    HostContext master = download_context(h, h->canon);
    sync(h->stream);
    const HostContext before = master;
    const size_t lanes = lane_ctx.size();
    struct Merged {
        size_t order;
        uint64_t key;
        uint64_t obs;
        size_t sum_at;  // first of E f64 sums in `sums`
    };
    std::vector<Merged> merged;
    std::vector<double> sums;
    size_t changed_slots = 0;
    for (const LaneContext& t : lane_ctx) changed_slots += t.slot.size();
    size_t cap = 64;
    while (cap < 2 * changed_slots) cap <<= 1;
    std::vector<int64_t> table(cap, -1);
    auto bucket_of = [&](size_t order, uint64_t key) {
        uint64_t x = key ^ (static_cast<uint64_t>(order) * 0x9E3779B97F4A7C15ULL);
        x ^= x >> 29;
        x *= 0xBF58476D1CE4E5B9ULL;
        x ^= x >> 32;
        return static_cast<size_t>(x) & (cap - 1);
    };
    std::vector<float> delta(E);
    // per-lane deltas against the pre-merge canonical (context_deltas_for_slots)
    for (size_t li = 0; li < lanes; ++li) {
        const LaneContext& t = lane_ctx[li];
        for (size_t k = 0; k < t.slot.size(); ++k) {
            const uint64_t slot = t.slot[k], key = t.key[k];
            if (key == 0) continue;
            const size_t order = static_cast<size_t>(slot / spo + 1);
            const int64_t bslot = find_context_slot(master, h->cfg, order, key);
            const uint32_t bobs = bslot >= 0 ? master.obs[static_cast<size_t>(bslot)] : 0;
            bool changed = false;
            for (size_t e = 0; e < E; ++e) {
                const float b = bslot >= 0 ? master.emb[static_cast<size_t>(bslot) * E + e] : 0.0f;
                delta[e] = t.emb[k * E + e] - b;
                changed |= delta[e] != 0.0f;
            }
            const uint32_t obs_inc = t.obs[k] > bobs ? t.obs[k] - bobs : 0;
            if (!changed && obs_inc == 0) continue;
            size_t at = bucket_of(order, key);
            while (table[at] >= 0 && (merged[static_cast<size_t>(table[at])].order != order ||
                                      merged[static_cast<size_t>(table[at])].key != key))
                at = (at + 1) & (cap - 1);
            if (table[at] < 0) {
                table[at] = static_cast<int64_t>(merged.size());
                merged.push_back(Merged{order, key, 0, sums.size()});
                sums.resize(sums.size() + E, 0.0);
            }
            Merged& m = merged[static_cast<size_t>(table[at])];
            for (size_t e = 0; e < E; ++e) {
                if (!std::isfinite(delta[e])) throw Error(LEO_ERR_INTERNAL, "invalid keyed context worker delta");
                sums[m.sum_at + e] += static_cast<double>(delta[e]);
            }
            m.obs += obs_inc;
        }
    }
    std::sort(merged.begin(), merged.end(), [](const Merged& a, const Merged& b) {
        if (a.obs != b.obs) return a.obs > b.obs;
        return std::make_pair(a.order, a.key) < std::make_pair(b.order, b.key);
    });
    const double divisor = static_cast<double>(lanes);
    for (const Merged& m : merged) {
        int64_t slot = resolve_context_slot(master, h->cfg, m.order, m.key, true, E);
        for (size_t e = 0; e < E; ++e)
            master.emb[static_cast<size_t>(slot) * E + e] += static_cast<float>(sums[m.sum_at + e] / divisor);
        uint32_t inc = static_cast<uint32_t>(std::min<uint64_t>(m.obs, UINT32_MAX));
        uint32_t& o = master.obs[static_cast<size_t>(slot)];
        o = (o > UINT32_MAX - inc) ? UINT32_MAX : o + inc;
    }
    // projection + validation of the merged embeddings (parallel.rs:1226-1233,
    // 1317-1333): the slot of every key a worker changed, each once (the
    // clamp is idempotent, so a key changed by several workers is projected
    // the same)
    const float wmin = h->cfg.device.weight_min, wmax = h->cfg.device.weight_max;
    for (const Merged& m : merged) {
        int64_t slot = resolve_context_slot(master, h->cfg, m.order, m.key, false, E);
        if (slot < 0) continue;
        for (size_t e = 0; e < E; ++e) {
            float& w = master.emb[static_cast<size_t>(slot) * E + e];
            if (w < wmin) w = wmin;
            if (w > wmax) w = wmax;
            if (!std::isfinite(w)) throw Error(LEO_ERR_INTERNAL, "merged context embedding violates canonical parameter bounds");
        }
    }
    upload(h->canon.ctx_keys, master.keys.data(), z.slots * 8, h->stream);
    upload(h->canon.ctx_obs, master.obs.data(), z.slots * 4, h->stream);
    upload(h->canon.ctx_emb, master.emb.data(), z.slots * z.e * 4, h->stream);
    // the slots the merge rewrote are host-stale
    std::vector<uint32_t> stale = download_bits(h, h->stale_bits[4], z.slots);
    sync(h->stream);
    for (uint64_t slot = 0; slot < z.slots; ++slot) {
        const bool changed = master.keys[slot] != before.keys[slot] || master.obs[slot] != before.obs[slot] ||
                             !std::equal(master.emb.begin() + slot * E, master.emb.begin() + (slot + 1) * E,
                                         before.emb.begin() + slot * E);
        if (changed) stale[slot >> 5] |= 1u << (slot & 31);
    }
    upload(h->stale_bits[4], stale.data(), stale.size() * 4, h->stream);
    sync(h->stream);
    return merged.size();
}

// f64 sums + changed flags for every fixed-parameter element (lane groups).
size_t merge_accumulator_bytes(const Sizes& z) {
    const uint64_t elements = z.n + z.ns + z.ni + z.n * kOutputs + kOutputs + kOutputs * z.e;
    // f64 sums and flags of the lane groups, and the candidate list (at most
    // one position per element of the largest bitmap-tracked tensor)
    return static_cast<size_t>(elements) * 9 + static_cast<size_t>(std::max({z.n, z.ns, z.ni})) * 4 + 256;
}

// Device mean of every fixed-parameter tensor (parallel.rs:746-782). kMergeDirect
// merges `lanes` into the canonical tensors; with lane groups, kMergeAccumulate
// adds one group's lanes (in lane order) to the f64 accumulators and
// kMergeFinalize applies them over `total_lanes`.
uint64_t merge_fixed(LeoHipRuntime* h, const std::vector<Lane*>& lanes, uint32_t mode = kMergeDirect,
                     bool first = true, uint32_t total_lanes = 0) {
    const Sizes& z = h->z;
    const uint32_t L = static_cast<uint32_t>(lanes.size());
    // scratch: 6 pointer tables of L entries, 4 bitmap tables, counters, error word
    size_t need = 10 * L * sizeof(float*) + 256;  // + counters
    if (h->merge_scratch.bytes < need) {
        h->merge_scratch.allocate(need);
    }
    std::vector<const float*> tables(6 * L);
    for (uint32_t l = 0; l < L; ++l) {
        const LaneParams& p = lanes[l]->desc.p;
        tables[0 * L + l] = p.threshold;
        tables[1 * L + l] = p.rec_weight;
        tables[2 * L + l] = p.in_weight;
        tables[3 * L + l] = p.out_w;
        tables[4 * L + l] = p.bias;
        tables[5 * L + l] = p.ctx_out;
    }
    // the lanes' change bitmaps of the four tensors they track per element
    // (output weights per neuron row)
    std::vector<const uint32_t*> bit_tables(4 * L);
    for (uint32_t l = 0; l < L; ++l) {
        const LaneDesc& d = lanes[l]->desc;
        bit_tables[0 * L + l] = d.ch_threshold;
        bit_tables[1 * L + l] = d.ch_rec;
        bit_tables[2 * L + l] = d.ch_in;
        bit_tables[3 * L + l] = d.ch_out;
    }
    char* base = h->merge_scratch.base;
    upload(base, tables.data(), tables.size() * sizeof(float*), h->stream);
    upload(base + 6 * L * sizeof(float*), bit_tables.data(), bit_tables.size() * sizeof(uint32_t*), h->stream);
    // counters: merged elements, changed lane values, the candidate count, then the error word
    auto* counter = reinterpret_cast<unsigned long long*>(base + 10 * L * sizeof(float*));
    auto* error = reinterpret_cast<uint32_t*>(counter + 3);
    LEO_HIP_CHECK(hipMemsetAsync(counter, 0, 32, h->stream));
    LEO_HIP_CHECK(hipEventRecord(h->ev_start, h->stream));
    struct Job {
        float* canonical;
        uint32_t kind;
        uint64_t count;
        uint32_t row, stride;
    };
    const Job jobs[6] = {
        {h->canon.threshold, 0, z.n, 0, 0},
        {h->canon.rec_weight, 1, z.ns, 0, 0},
        {h->canon.in_weight, 2, z.ni, 0, 0},
        {h->canon.out_w, 3, z.n * kOutputs, kOutputs, kOutStride},
        {h->canon.bias, 4, kOutputs, 0, 0},
        {h->canon.ctx_out, 5, kOutputs * z.e, 0, 0},
    };
    uint64_t elements = 0;
    for (int j = 0; j < 6; ++j) elements += jobs[j].count;
    if (mode != kMergeDirect && h->merge_acc.bytes < elements * 9) h->merge_acc.allocate(elements * 9);
    // lane groups: every element's group flag starts clear (an element listed
    // first in a later group starts its sum from zero)
    if (mode == kMergeAccumulate && first)
        LEO_HIP_CHECK(hipMemsetAsync(h->merge_acc.base + elements * 8, 0, elements, h->stream));
    const uint64_t max_positions = std::max({z.n, z.ns, z.ni});
    if (mode != kMergeFinalize && h->merge_list.bytes < max_positions * 4) h->merge_list.allocate(max_positions * 4);
    uint64_t acc_at = 0;
    uint32_t candidate_launches = 0;
    double bitmap_bytes = 0.0;
    for (int j = 0; j < 6; ++j) {
        MergeArgs m{};
        m.mode = mode;
        m.first = first ? 1u : 0u;
        m.total_lanes = total_lanes;
        if (mode != kMergeDirect) {
            m.acc = reinterpret_cast<double*>(h->merge_acc.base) + acc_at;
            m.any = reinterpret_cast<uint8_t*>(h->merge_acc.base + elements * 8) + acc_at;
        }
        acc_at += jobs[j].count;
        m.canonical = jobs[j].canonical;
        m.lanes = reinterpret_cast<const float* const*>(base + static_cast<size_t>(j) * L * sizeof(float*));
        m.lane_count = L;
        m.kind = jobs[j].kind;
        m.count = jobs[j].count;
        m.row = jobs[j].row;
        m.stride = jobs[j].stride;
        m.synapses_per_neuron = static_cast<uint32_t>(z.s);
        m.neuron_type = h->sm.neuron_type;
        m.weight_min = h->cfg.device.weight_min;
        m.weight_max = h->cfg.device.weight_max;
        m.updates = counter;
        m.lane_changes = counter + 1;
        m.error = error;
        // merged canonical elements are host-stale (bias and context output: whole)
        m.stale = jobs[j].kind == kMergeBias ? h->stale_flags
                  : jobs[j].kind == kMergeContextOut ? h->stale_flags + 1
                  : h->stale_bits[jobs[j].kind];
        m.stale_flag = (jobs[j].kind == kMergeBias || jobs[j].kind == kMergeContextOut) ? 1u : 0u;
        if (mode != kMergeFinalize && j < 4) {
            // positions changed in any lane (every merged element is among them)
            const uint64_t positions = j == 3 ? z.n : jobs[j].count;
            MergeCandidates mc{};
            mc.bits = reinterpret_cast<const uint32_t* const*>(base + 6 * L * sizeof(float*) +
                                                               static_cast<size_t>(j) * L * sizeof(uint32_t*));
            mc.lane_count = L;
            mc.words = z.words(positions);
            mc.positions = positions;
            mc.list = reinterpret_cast<uint32_t*>(h->merge_list.base);
            mc.count = counter + 2;
            LEO_HIP_CHECK(hipMemsetAsync(counter + 2, 0, 8, h->stream));
            const uint64_t cblocks = std::min<uint64_t>((mc.words + kThreads - 1) / kThreads, 4096);
            hipLaunchKernelGGL(leo_merge_candidates, dim3(static_cast<uint32_t>(std::max<uint64_t>(cblocks, 1))),
                               dim3(kThreads), 0, h->stream, mc);
            LEO_HIP_CHECK(hipGetLastError());
            m.list = mc.list;
            m.list_count = mc.count;
            candidate_launches += 1;
            bitmap_bytes += 4.0 * static_cast<double>(mc.words) * L;
        }
        uint64_t blocks = std::min<uint64_t>((m.count + kThreads - 1) / kThreads, 4096);
        hipLaunchKernelGGL(leo_merge_fixed, dim3(static_cast<uint32_t>(std::max<uint64_t>(blocks, 1))), dim3(kThreads), 0,
                           h->stream, m);
        LEO_HIP_CHECK(hipGetLastError());
    }
    LEO_HIP_CHECK(hipEventRecord(h->ev_stop, h->stream));
    unsigned long long counts[2] = {0, 0};
    uint32_t err = 0;
    download(counts, counter, 16, h->stream);
    download(&err, error, 4, h->stream);
    sync(h->stream);
    const unsigned long long updates = counts[0];
    float ms = 0.0f;
    LEO_HIP_CHECK(hipEventElapsedTime(&ms, h->ev_start, h->ev_stop));
    LeoKernelStats& t = h->telemetry;
    t.merge_launches += 6 + candidate_launches;
    t.merge_ms += ms;
    // algorithmic bytes of the mean: the lanes' change bitmaps the candidate
    // pass ORs, 24 per changed lane value, 4 (L+1) per merged element
    t.merge_lane_changes += counts[1];
    t.merge_bytes += bitmap_bytes + 24.0 * static_cast<double>(counts[1]);
    if (mode != kMergeAccumulate) {
        const double lanes_total = mode == kMergeFinalize ? total_lanes : L;
        t.merge_elements += updates;
        t.merge_bytes += 4.0 * (lanes_total + 1.0) * static_cast<double>(updates);
    }
    if (err) throw Error(LEO_ERR_INTERNAL, "merged parameter became non-finite");
    return updates;
}

Lane& story_lane(LeoHipRuntime* h, uint32_t index) {
    while (h->lanes.size() <= index) {
        auto lane = std::make_unique<Lane>();
        allocate_lane_state(*lane, h->z, h->stream);
        lane->desc.p = allocate_params(lane->params, h->z, h->stream);
        h->lanes.push_back(std::move(lane));
    }
    return *h->lanes[index];
}

void story_batch(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count, int32_t permission,
                 float* losses_out, LeoBatchReport& rep) {
    if (count == 0) throw Error(LEO_ERR_INVALID_ARGUMENT, "training batch cannot be empty");
    for (uint32_t i = 0; i < count; ++i)
        if (offsets[i + 1] <= offsets[i]) throw Error(LEO_ERR_UNSUPPORTED, "empty stories are not supported in a device batch");
    // stories run in groups of the lanes that fit on the device, as few
    // groups as that allows, with the stories split evenly over them (a
    // group's launch then gives each lane the same share of the workgroups:
    // at D, 32 + 32 lanes of 16 workgroups ran the story pass 14% faster than
    // 54 + 10 lanes of 9 and 32); the groups' lanes join the batch-end mean
    // in story order
    const uint32_t resident = std::max<uint32_t>(1, std::min(h->resident_lanes, h->max_lanes));
    const uint32_t groups = (count + resident - 1) / resident;
    const uint32_t per_group = (count + groups - 1) / groups;
    const uint32_t S = h->cfg.device.synapses_per_neuron;
    LeoStatistics merged = h->stats;
    uint64_t revision_increment = 0;
    double weighted = 0.0;
    uint64_t targets = 0;
    size_t cursor = 0;
    double run_seconds = 0.0, merge_seconds = 0.0;
    std::vector<LaneContext> group_ctx;
    std::vector<Lane*> lanes;
    for (uint32_t g = 0; g < groups; ++g) {
        auto t0 = std::chrono::steady_clock::now();
        const uint32_t lo = g * per_group, hi = std::min(count, lo + per_group);
        lanes.clear();
        for (uint32_t i = lo; i < hi; ++i) lanes.push_back(&story_lane(h, i - lo));
        broadcast_params(h, lanes);  // fork(base.clone())
        reset_lane_objects(h, lanes, true, 0);  // Runtime::new (tick 0) + begin_document
        clear_lane_changes(h, static_cast<uint32_t>(lanes.size()));  // enable_parameter_tracking
        std::vector<LaneRun> runs;
        for (uint32_t i = lo; i < hi; ++i) {
            LaneRun r{lanes[i - lo], {}, {}};
            auto steps = document_steps(bytes + offsets[i], static_cast<size_t>(offsets[i + 1] - offsets[i]));
            uint32_t tick = 0;
            for (auto& st : steps)
                r.steps.push_back(make_step(h->cfg, *lanes[i - lo], st.symbol, st.target, permission, tick++, true));
            runs.push_back(std::move(r));
        }
        run_lanes(h, runs);
        auto t1 = std::chrono::steady_clock::now();
        run_seconds += std::chrono::duration<double>(t1 - t0).count();
        // per-lane statistics deltas (parallel.rs:1115-1137) and revision increments
        for (uint32_t i = lo; i < hi; ++i) {
            const LaneRun& run = runs[i - lo];
            LeoStatistics st = h->stats;  // the forked worker starts from the canonical statistics
            double loss_sum = 0.0;
            uint64_t steps_with_loss = 0;
            bool activity = false;
            for (size_t k = 0; k < run.steps.size(); ++k) {
                const StepParams& sp = run.steps[k];
                const StepRecord& rec = run.records[k];
                float loss = step_loss(sp, rec);
                account_step(st, sp, rec, loss, S);
                if (!(sp.flags & kStepFrozen)) activity = true;
                if (sp.flags & kStepLearn) revision_increment += 1;
                float recorded = sp.target_index >= 0 ? loss : 0.0f;  // record_training_step
                loss_sum += static_cast<double>(recorded);
                steps_with_loss += 1;
                if (losses_out) losses_out[cursor++] = recorded;
                rep.activity_steps += 1;
                rep.active_neurons_sum += rec.active;
                rep.emitted_events += static_cast<uint64_t>(rec.active) * S;
            }
            if (activity) st.processed_stories += 1;  // finish_document
            double mean = loss_sum / static_cast<double>(std::max<uint64_t>(steps_with_loss, 1));
            weighted += mean * static_cast<double>(steps_with_loss);
            targets += steps_with_loss;
            merged.processed_bytes += st.processed_bytes - h->stats.processed_bytes;
            merged.processed_stories += st.processed_stories - h->stats.processed_stories;
            merged.training_loss_sum += st.training_loss_sum - h->stats.training_loss_sum;
            merged.training_targets += st.training_targets - h->stats.training_targets;
            merged.active_neurons_sum += st.active_neurons_sum - h->stats.active_neurons_sum;
            merged.active_neurons_peak = std::max(merged.active_neurons_peak, st.active_neurons_peak);
            merged.synaptic_events += st.synaptic_events - h->stats.synaptic_events;
            merged.persistent_ticks += st.persistent_ticks - h->stats.persistent_ticks;
        }
        if (groups > 1) {
            merge_fixed(h, lanes, kMergeAccumulate, g == 0, count);
            download_lane_contexts(h, lanes, group_ctx);
            sync(h->stream);
            merge_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
        }
    }
    // batch-end mean (parallel.rs:715-798): fixed tensors on the device, keyed context on the host
    auto t2 = std::chrono::steady_clock::now();
    uint64_t fixed, ctx;
    if (groups == 1) {
        fixed = merge_fixed(h, lanes);
        ctx = merge_context(h, lanes);
    } else {
        fixed = merge_fixed(h, {}, kMergeFinalize, false, count);
        ctx = merge_context_downloaded(h, group_ctx);
    }
    h->stats = merged;
    h->revision += revision_increment;
    canonical_reset(h);  // runtime.reset_transient_state() after the merge
    auto t3 = std::chrono::steady_clock::now();
    merge_seconds += std::chrono::duration<double>(t3 - t2).count();
    rep.mean_loss = weighted / static_cast<double>(std::max<uint64_t>(targets, 1));
    rep.targets = targets;
    rep.stories = count;
    rep.merge_workers = count;
    rep.merge_fixed_parameter_updates = fixed;
    rep.merge_context_keys = ctx;
    rep.story_seconds += run_seconds;
    rep.merge_seconds += merge_seconds;
}

// Frozen evaluation (validation.rs:65-154). Story lanes borrow the canonical
// parameters for the launch: frozen steps allocate no context slot and run no
// learning or homeostasis, so nothing writes them.
struct BorrowedParams {
    std::vector<std::pair<Lane*, LaneParams>> saved;
    ~BorrowedParams() {
        for (auto& [lane, p] : saved) lane->desc.p = p;
    }
};

void evaluate_stories(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                      float* losses_out, LeoEvaluationReport& rep) {
    std::vector<uint32_t> stories;
    for (uint32_t i = 0; i < count; ++i) {
        if (offsets[i + 1] < offsets[i]) throw Error(LEO_ERR_INVALID_ARGUMENT, "story offsets must not decrease");
        if (offsets[i + 1] > offsets[i]) stories.push_back(i);  // validation.rs:86-88 skips empty stories
    }
    const uint32_t S = h->cfg.device.synapses_per_neuron, E = h->cfg.device.context_embedding_dim;
    const uint32_t resident = std::max<uint32_t>(1, std::min(h->resident_lanes, h->max_lanes));
    const size_t groups = (stories.size() + resident - 1) / resident;
    const size_t per_group = groups > 0 ? (stories.size() + groups - 1) / groups : 1;  // even groups, as above
    const float uniform_loss = std::log(static_cast<float>(kOutputs));  // loss_from_logits fallback
    uint32_t tick = h->canonical->tick;
    double loss_sum = 0.0;
    uint64_t correct = 0;
    size_t cursor = 0;
    rep.neuron_count = h->z.n;
    for (size_t lo = 0; lo < stories.size(); lo += per_group) {
        const size_t hi = std::min(stories.size(), lo + per_group);
        BorrowedParams borrowed;
        std::vector<LaneRun> runs;
        std::vector<std::vector<HostStep>> host_steps;
        for (size_t k = lo; k < hi; ++k) {
            Lane& lane = story_lane(h, static_cast<uint32_t>(k - lo));
            borrowed.saved.push_back({&lane, lane.desc.p});
            lane.desc.p = h->canon;
            // begin_document at the tick one runtime scoring the stories in
            // order would have reached
            std::vector<Lane*> one{&lane};
            reset_lane_objects(h, one, true, tick);
            const uint32_t s = stories[k];
            host_steps.push_back(document_steps(bytes + offsets[s], static_cast<size_t>(offsets[s + 1] - offsets[s])));
            LaneRun run{&lane, {}, {}};
            for (const HostStep& st : host_steps.back()) {
                StepParams sp = make_step(h->cfg, lane, st.symbol, st.target, LEO_FROZEN, tick++, true);
                sp.flags |= kStepNeuralLoss;
                run.steps.push_back(sp);
            }
            runs.push_back(std::move(run));
        }
        run_lanes(h, runs);
        // record_evaluation_step + ActivityDiagnostics::record, story by story
        for (size_t k = 0; k < runs.size(); ++k) {
            const LaneRun& run = runs[k];
            for (size_t i = 0; i < run.steps.size(); ++i) {
                const StepParams& sp = run.steps[i];
                const StepRecord& r = run.records[i];
                const float loss = step_loss(sp, r);
                if (losses_out) losses_out[cursor++] = loss;
                loss_sum += static_cast<double>(loss);
                rep.targets += 1;
                const uint32_t predicted = r.predicted < 256 ? r.predicted : kEnd;
                if (predicted == static_cast<uint32_t>(host_steps[k][i].target)) correct += 1;
                rep.steps += 1;
                rep.active_neurons_sum += r.active;
                rep.active_neurons_peak = std::max<uint64_t>(rep.active_neurons_peak, r.active);
                rep.emitted_events += static_cast<uint64_t>(r.active) * S;
                rep.suprathreshold_sum += r.suprathreshold;
                rep.block_selected_sum += r.block_selected;
                rep.cap_clipped_sum += r.clipped;
                if (r.clipped > 0) rep.cap_hit_steps += 1;
                rep.population_inhibition_sum += static_cast<double>(r.population_inhibition);
                rep.population_inhibition_peak = std::max(rep.population_inhibition_peak, r.population_inhibition);
                // frozen steps apply no learning: mean |eligibility| is 0
                rep.eligibility_count += static_cast<uint64_t>(r.eligible_rec) + r.eligible_in;
                rep.context_cells_sum += r.context_cells;
                rep.context_probes_sum += r.context_probes;
                if (r.context_applied) rep.context_applied_steps += 1;
                const bool finite_sum = std::isfinite(r.neural_sum) && r.neural_sum > 0.0f;
                const float neural = finite_sum ? (r.neural_max + std::log(r.neural_sum)) - r.neural_target : uniform_loss;
                rep.context_loss_gain_sum += static_cast<double>(neural - loss);
                rep.output_madds_sum += static_cast<uint64_t>(r.active) * kOutputs +
                                        static_cast<uint64_t>(r.context_cells) * E +
                                        (r.context_cells > 0 ? static_cast<uint64_t>(E) * kOutputs : 0);
            }
            const uint32_t s = stories[lo + k];
            rep.processed_bytes += offsets[s + 1] - offsets[s];
            rep.processed_stories += 1;
        }
    }
    // finish_document of the last story: the canonical runtime ends reset,
    // its tick past every evaluated step
    std::vector<Lane*> canonical{h->canonical.get()};
    reset_lane_objects(h, canonical, true, tick);
    sync(h->stream);
    rep.loss = loss_sum / static_cast<double>(std::max<uint64_t>(rep.targets, 1));
    rep.bits_per_byte = rep.loss / std::log(2.0);
    rep.accuracy = static_cast<double>(correct) / static_cast<double>(std::max<uint64_t>(rep.targets, 1));
}

// synchronize_model on a host mirror (cuda.rs:2817-2825, 5657-5760): every
// element marked changed (tracked) or host-stale is gathered from the
// canonical image into the mirror; then nothing is stale.
void synchronize_host(LeoHipRuntime* h, LeoModelView& m) {
    const Sizes& z = h->z;
    const LaneDesc& d = h->canonical->desc;
    std::vector<std::vector<uint32_t>> bits(5), stale(5);
    for (int i = 0; i < 5; ++i) {
        bits[i] = download_bits(h, change_bits(d, i), set_size(z, i));
        stale[i] = download_bits(h, h->stale_bits[i], set_size(z, i));
    }
    uint32_t flags[2] = {0, 0}, stale_flags[2] = {0, 0};
    download(flags, &d.ctl->bias_dirty, 8, h->stream);
    download(stale_flags, h->stale_flags, 8, h->stream);
    sync(h->stream);
    std::vector<uint32_t> index[5];
    for (int i = 0; i < 5; ++i) {
        for (size_t w = 0; w < bits[i].size(); ++w) bits[i][w] |= stale[i][w];
        for (uint64_t v : bits_to_indices(bits[i], set_size(z, i))) index[i].push_back(static_cast<uint32_t>(v));
    }
    float* single_targets[3] = {m.threshold, m.rec_weight, m.in_weight};
    float* single_sources[3] = {h->canon.threshold, h->canon.rec_weight, h->canon.in_weight};
    for (int i = 0; i < 3; ++i) {
        std::vector<float> values(index[i].size());
        sparse_move(h, single_sources[i], index[i].data(), index[i].size(), 0, 0, nullptr, values.data(), false);
        for (size_t k = 0; k < index[i].size(); ++k) single_targets[i][index[i][k]] = values[k];
    }
    {
        // output rows: neuron-major on the device, output-major on the host
        const std::vector<uint32_t>& rows = index[3];
        std::vector<float> values(rows.size() * kOutputs);
        sparse_move(h, h->canon.out_w, rows.data(), rows.size(), kOutputs, kOutStride, nullptr, values.data(), false);
        for (size_t k = 0; k < rows.size(); ++k)
            for (uint64_t o = 0; o < kOutputs; ++o) m.out_weight[o * z.n + rows[k]] = values[k * kOutputs + o];
    }
    if (!index[4].empty()) {
        // the context tables are small: read whole, copy the marked slots
        HostContext c = download_context(h, h->canon);
        sync(h->stream);
        for (uint32_t slot : index[4]) {
            m.ctx_keys[slot] = c.keys[slot];
            m.ctx_obs[slot] = c.obs[slot];
            std::copy(c.emb.begin() + slot * z.e, c.emb.begin() + (slot + 1) * z.e, m.ctx_emb + slot * z.e);
        }
    }
    if (flags[0] | stale_flags[0]) download(m.bias, h->canon.bias, kOutputs * 4, h->stream);
    if (flags[1] | stale_flags[1]) download(m.ctx_out, h->canon.ctx_out, kOutputs * z.e * 4, h->stream);
    clear_stale(h);
    sync(h->stream);
    m.generation = h->generation;
    m.parameter_revision = h->revision;
    m.statistics = h->stats;
}

// PackedSparseModelUpdate::apply_to_model (parallel.rs:186-302) on the
// canonical device image, with the reference's index and size checks.
void apply_packed(LeoHipRuntime* h, const LeoPackedUpdate& u, bool end_tracking, const Staging& staging = Staging{}) {
    const Sizes& z = h->z;
    auto need = [](bool ok, const char* what) {
        if (!ok) throw Error(LEO_ERR_INVALID_ARGUMENT, what);
    };
    auto check_indices = [&](const uint32_t* idx, const void* values, uint64_t count, uint64_t limit, const char* label) {
        need(count == 0 || (idx && values), label);
        for (uint64_t k = 0; k < count; ++k)
            if (idx[k] >= limit) throw Error(LEO_ERR_INVALID_ARGUMENT, std::string(label) + " packed sparse index is outside model");
    };
    check_indices(u.threshold_indices, u.threshold_values, u.threshold_count, z.n, "threshold");
    check_indices(u.recurrent_indices, u.recurrent_values, u.recurrent_count, z.ns, "recurrent");
    check_indices(u.input_indices, u.input_values, u.input_count, z.ni, "input");
    check_indices(u.output_neurons, u.output_values_by_neuron, u.output_count, z.n, "packed output neuron");
    check_indices(u.context_slots, u.context_embeddings, u.context_count, z.slots, "packed context slot");
    need(u.context_count == 0 || (u.context_keys && u.context_observations), "packed context rows have invalid dimensions");
    if (staging.fixed) {
        // every move must fit before the first one writes
        const size_t largest = std::max({move_bytes(u.threshold_count, 1), move_bytes(u.recurrent_count, 1),
                                         move_bytes(u.input_count, 1), move_bytes(u.output_count, kOutputs),
                                         move_bytes(u.context_count, std::max<uint64_t>(z.e, 2))});
        if (largest > staging.capacity)
            throw Error(LEO_ERR_INVALID_ARGUMENT, "packed update needs " + std::to_string(largest) +
                                                      " bytes of scratch for one tensor; the allocation-free entry "
                                                      "point holds " + std::to_string(staging.capacity));
    }
    sparse_move(h, h->canon.threshold, u.threshold_indices, u.threshold_count, 0, 0, u.threshold_values, nullptr, true,
                staging);
    sparse_move(h, h->canon.rec_weight, u.recurrent_indices, u.recurrent_count, 0, 0, u.recurrent_values, nullptr, true,
                staging);
    sparse_move(h, h->canon.in_weight, u.input_indices, u.input_count, 0, 0, u.input_values, nullptr, true, staging);
    sparse_move(h, h->canon.out_w, u.output_neurons, u.output_count, kOutputs, kOutStride, u.output_values_by_neuron,
                nullptr, true, staging);
    if (u.context_count) {
        // keys as rows of two 32-bit words, observations as words, embeddings
        // as rows of E (moves copy the bits)
        sparse_move(h, reinterpret_cast<float*>(h->canon.ctx_keys), u.context_slots, u.context_count, 2, 2,
                    reinterpret_cast<const float*>(u.context_keys), nullptr, true, staging);
        sparse_move(h, reinterpret_cast<float*>(h->canon.ctx_obs), u.context_slots, u.context_count, 0, 0,
                    reinterpret_cast<const float*>(u.context_observations), nullptr, true, staging);
        sparse_move(h, h->canon.ctx_emb, u.context_slots, u.context_count, static_cast<uint32_t>(z.e),
                    static_cast<uint32_t>(z.e), u.context_embeddings, nullptr, true, staging);
    }
    if (u.output_bias) upload(h->canon.bias, u.output_bias, kOutputs * 4, h->stream);
    if (u.context_output_weights) upload(h->canon.ctx_out, u.context_output_weights, kOutputs * z.e * 4, h->stream);
    // the mirror that packed this update holds the bias / projection it carries
    uint32_t carried[2] = {u.output_bias ? 1u : 0u, u.context_output_weights ? 1u : 0u};
    for (int k = 0; k < 2; ++k)
        if (carried[k]) LEO_HIP_CHECK(hipMemsetAsync(h->stale_flags + k, 0, 4, h->stream));
    sync(h->stream);
    if (has_negative_zero(u.recurrent_values, u.recurrent_count) || has_negative_zero(u.input_values, u.input_count))
        h->negative_zero_weights = true;
    h->generation = u.generation;
    h->revision = u.parameter_revision;
    h->stats = u.statistics;
    if (end_tracking) h->tracking = false;
}

// training.rs:1782-1830
std::vector<std::pair<size_t, size_t>> select_replay_ranges(const std::vector<float>& losses, float fraction,
                                                            size_t segment) {
    std::vector<std::pair<size_t, size_t>> selected;
    const size_t n = losses.size();
    if (n == 0 || !std::isfinite(fraction) || fraction <= 0.0f || segment == 0) return selected;
    size_t budget = static_cast<size_t>(
        std::max(1.0, std::ceil(static_cast<double>(n) * static_cast<double>(std::min(fraction, 1.0f)))));
    std::vector<size_t> order(n);
    for (size_t i = 0; i < n; ++i) order[i] = i;
    auto key = [](float v) {
        int32_t b;
        std::memcpy(&b, &v, 4);
        return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
    };
    std::sort(order.begin(), order.end(), [&](size_t l, size_t r) {
        int32_t kl = key(losses[l]), kr = key(losses[r]);
        if (kl != kr) return kl > kr;
        return l < r;
    });
    size_t chosen = 0;
    for (size_t p : order) {
        if (chosen >= budget) break;
        float loss = losses[p];
        if (!std::isfinite(loss) || loss <= 0.0f) continue;
        size_t width = std::min(std::min(segment, budget - chosen), n);
        size_t start = p >= width / 2 ? p - width / 2 : 0;
        size_t end = std::min(start + width, n);
        start = end >= width ? end - width : 0;
        bool overlap = false;
        for (auto& r : selected)
            if (r.first < end && start < r.second) overlap = true;
        if (overlap) continue;
        chosen += end - start;
        selected.push_back({start, end});
    }
    std::sort(selected.begin(), selected.end());
    return selected;
}

// One story's replay on the canonical runtime: its segments, and whether the
// replay ends with a reset of the runtime.
struct StoryReplay {
    std::vector<CanonicalSegment> segments;
    bool cleanup = false;
};

// Plans one story's replay (training.rs:162-255, 394-470, 1848-1954): the
// selected ranges as canonical segments; the prefix and target step counts go
// into the report.
StoryReplay plan_replay(LeoHipRuntime* h, const uint8_t* story, size_t len, const std::vector<float>& losses,
                        int32_t permission, LeoBatchReport& rep) {
    StoryReplay plan;
    auto ranges = select_replay_ranges(losses, h->cfg.replay_fraction, h->cfg.replay_segment_bytes);
    rep.replay_segments += ranges.size();
    if (ranges.empty() || len == 0) return plan;
    auto position_step = [&](size_t p, bool supervised) {
        HostStep s{p == 0 ? kBegin : story[p - 1], -1};
        if (supervised) s.target = p < len ? static_cast<int32_t>(story[p]) : static_cast<int32_t>(kEnd);
        return s;
    };
    std::vector<CanonicalSegment> segments;
    // the cleanup after the replay belongs to its last range: a skipped last
    // range leaves the runtime as the previous range left it
    // (replay_target_range_impl, training.rs:1848-1870, 1938)
    bool cleanup = true;
    if (h->cfg.replay_stateful_batch) {
        CanonicalSegment seg;
        seg.reset_before = true;
        const size_t terminal = len + 1;
        size_t cursor = 0;
        for (auto [rs, re] : ranges) {
            size_t start = std::max(std::min(rs, terminal), cursor);
            size_t end = std::max(std::min(re, terminal), start);
            for (size_t p = cursor; p < start; ++p) {
                seg.steps.push_back(position_step(p, false));
                seg.permissions.push_back(LEO_FROZEN);
                rep.replay_prefix_steps += 1;
            }
            for (size_t p = start; p < end; ++p) {
                seg.steps.push_back(position_step(p, true));
                seg.permissions.push_back(permission);
                rep.replay_steps += 1;
            }
            cursor = end;
        }
        segments.push_back(std::move(seg));
    } else {
        for (auto [rs, re] : ranges) {
            cleanup = !(rs >= re || rs > len);
            if (!cleanup) continue;
            size_t end = std::min(re, len + 1);
            CanonicalSegment seg;
            seg.reset_before = true;  // begin_document_deferred_for_replay
            size_t next = rs;
            if (next > 0) {
                seg.steps.push_back({kBegin, -1});
                seg.permissions.push_back(LEO_FROZEN);
                for (size_t i = 0; i + 1 < next; ++i) {
                    seg.steps.push_back({story[i], -1});
                    seg.permissions.push_back(LEO_FROZEN);
                }
                rep.replay_prefix_steps += next;
            }
            if (next == 0) {
                seg.steps.push_back({kBegin, story[0]});
                seg.permissions.push_back(permission);
                rep.replay_steps += 1;
                next = 1;
            }
            for (size_t p = next; p < end; ++p) {
                seg.steps.push_back(position_step(p, true));
                seg.permissions.push_back(permission);
                rep.replay_steps += 1;
            }
            segments.push_back(std::move(seg));
        }
        if (segments.empty()) return plan;
    }
    plan.segments = std::move(segments);
    plan.cleanup = cleanup;
    return plan;
}

// Replays the stories of a batch one after another on the canonical runtime,
// queued as one run of segments with one wait at the end. Every story's first
// segment starts with a reset, so the reset that ends a story's replay is
// queued only when no later story's segment follows it (a second reset with
// no step between changes nothing).
void replay_stories(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                    const std::vector<std::vector<float>>& losses, int32_t permission, LeoBatchReport& rep) {
    std::vector<CanonicalSegment> segments;
    bool cleanup = false;
    for (uint32_t i = 0; i < count; ++i) {
        StoryReplay plan = plan_replay(h, bytes + offsets[i], static_cast<size_t>(offsets[i + 1] - offsets[i]),
                                       losses[i], permission, rep);
        if (plan.segments.empty()) continue;
        for (CanonicalSegment& seg : plan.segments) segments.push_back(std::move(seg));
        cleanup = plan.cleanup;
    }
    if (segments.empty()) return;
    std::vector<LeoStepMetrics> metrics;
    run_canonical_segments(h, segments, metrics);
    size_t at = 0;
    for (const CanonicalSegment& seg : segments)
        for (int32_t perm : seg.permissions) {
            const LeoStepMetrics& m = metrics[at++];
            if (perm == LEO_FROZEN) continue;
            rep.activity_steps += 1;
            rep.active_neurons_sum += m.active_neurons;
            rep.emitted_events += m.emitted_events;
        }
    if (cleanup) canonical_reset(h);
}

}  // namespace
}  // namespace leo

using leo::Error;
using leo::guarded;

extern "C" {

int32_t leo_hip_last_error(char* buffer, size_t capacity) {
    if (!buffer || capacity == 0) return LEO_ERR_INVALID_ARGUMENT;
    std::snprintf(buffer, capacity, "%s", leo::g_error.c_str());
    return LEO_OK;
}

int32_t leo_hip_abi_version(void) { return LEO_HIP_ABI_VERSION; }

int32_t leo_splitmix64(uint64_t seed, uint64_t* out, uint64_t count) {
    return guarded([&] {
        if (!out && count) throw Error(LEO_ERR_INVALID_ARGUMENT, "null output");
        leo::splitmix64_stream(seed, out, count);
    });
}

int32_t leo_model_initialize(const LeoHostConfig* config, LeoModelView* out) {
    return guarded([&] {
        if (!config || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::model_initialize(*config, *out);
    });
}

int32_t leo_model_initialize_synthetic(const LeoHostConfig* config, uint32_t topology, float exponent,
                                       uint32_t in_degree_cap, float weight_sigma, LeoModelView* out) {
    return guarded([&] {
        if (!config || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::model_initialize_synthetic(*config, topology, exponent, in_degree_cap, weight_sigma, *out);
    });
}

int32_t leo_model_validate(const LeoHostConfig* config, const LeoModelView* model) {
    return guarded([&] {
        if (!config || !model) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::model_validate(*config, *model);
    });
}

int32_t leo_synthetic_stories(uint64_t seed, uint32_t count, double mean, double stddev, uint32_t min_len,
                              uint32_t max_len, uint8_t* bytes, uint64_t capacity, uint64_t* offsets) {
    return guarded([&] {
        if (!bytes || !offsets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::synthetic_stories(seed, count, mean, stddev, min_len, max_len, bytes, capacity, offsets);
    });
}

int32_t leo_hip_create(const LeoHostConfig* config, const LeoModelView* model, int32_t device, uint32_t max_lanes,
                       LeoHipRuntime** out) {
    return guarded([&] {
        if (!config || !model || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::model_validate(*config, *model);
        if (static_cast<uint64_t>(config->device.neuron_count) * config->device.synapses_per_neuron >= (1ull << 31))
            throw Error(LEO_ERR_UNSUPPORTED, "neuron_count * synapses_per_neuron at or above 2^31 is not supported");
        if (config->device.neuron_count > leo::kMaxPackedNeurons)
            throw Error(LEO_ERR_UNSUPPORTED, "neuron_count above 2^28 is not supported by the packed synapse layout");
        if (config->device.neurons_per_block > leo::kMaxBlockNeurons)
            throw Error(LEO_ERR_UNSUPPORTED, "neurons_per_block above 1024 is not supported by the device selection");
        // neuron records and the fixed delivery entries are read with 32-bit
        // buffer offsets (64 bytes per neuron)
        if (static_cast<uint64_t>(config->device.neuron_count) * leo::kNeuronWords * 4 >= (1ull << 32))
            throw Error(LEO_ERR_UNSUPPORTED, "neuron_count above 2^26 is not supported by the neuron records");
        int devices = 0;
        if (hipGetDeviceCount(&devices) != hipSuccess || devices <= 0)
            throw Error(LEO_ERR_DEVICE, "GPU backend requested, but no HIP device is available");
        if (device < 0 || device >= devices) throw Error(LEO_ERR_DEVICE, "HIP device index out of range");
        hipDeviceProp_t prop{};
        LEO_HIP_CHECK(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            throw Error(LEO_ERR_DEVICE, std::string("this build targets gfx950; device reports ") + prop.gcnArchName);
        int coop = 0;
        LEO_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device));
        if (!coop) throw Error(LEO_ERR_DEVICE, "device does not support cooperative launches");
        auto h = std::make_unique<LeoHipRuntime>();
        h->cfg = *config;
        h->z = leo::sizes_of(*config);
        h->device = device;
        h->max_lanes = std::max<uint32_t>(max_lanes, 1);
        LEO_HIP_CHECK(hipSetDevice(device));
        LEO_HIP_CHECK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
        LEO_HIP_CHECK(hipEventCreate(&h->ev_start));
        LEO_HIP_CHECK(hipEventCreate(&h->ev_stop));
        h->staging.init();
        h->cus = prop.multiProcessorCount;
        // cooperative capacity: the smaller occupancy of the step kernel and
        // its phase-profiling build (either may be launched on the same grid)
        int occupancy[3] = {0, 0, 0};
        const void* step_kernels[3] = {reinterpret_cast<const void*>(&leo::leo_lane_steps),
                                       reinterpret_cast<const void*>(&leo::leo_lane_steps_profiled),
                                       reinterpret_cast<const void*>(&leo::leo_lane_steps_frozen)};
        for (int k = 0; k < 3; ++k)
            LEO_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &occupancy[k], step_kernels[k], leo::kThreads, leo::step_lds_bytes(config->device.neurons_per_block)));
        h->coop_blocks_per_cu = std::min({occupancy[0], occupancy[1], occupancy[2]});
        if (h->coop_blocks_per_cu <= 0) throw Error(LEO_ERR_DEVICE, "step kernel cannot be resident");
        if (const char* env = std::getenv("LEO_HIP_WGS_PER_LANE")) h->wgs_override = static_cast<uint32_t>(std::atoi(env));
        if (const char* env = std::getenv("LEO_HIP_CANONICAL_WGS"))
            h->canonical_wgs_override = static_cast<uint32_t>(std::atoi(env));
        if (const char* env = std::getenv("LEO_HIP_AGENT_SYNC")) h->local_sync = std::atoi(env) == 0;
        if (const char* env = std::getenv("LEO_HIP_MAX_STEPS_PER_LAUNCH"))
            h->max_steps_override = static_cast<uint32_t>(std::max(1, std::atoi(env)));
        if (const char* env = std::getenv("LEO_HIP_PHASE_PROFILE")) h->phase_profile = std::atoi(env) != 0;
        if (const char* env = std::getenv("LEO_HIP_BUCKET_SETS"))
            h->canonical_sets = std::atoi(env) == 1 ? 1u : leo::kBucketSets;
        if (const char* env = std::getenv("LEO_HIP_PROFILE_PART"))
            h->profile_part = static_cast<uint32_t>(std::max(0, std::atoi(env)));
        if (const char* env = std::getenv("LEO_HIP_FROZEN_KERNEL")) h->frozen_kernel = std::atoi(env) != 0;
        if (const char* env = std::getenv("LEO_HIP_TALLY")) h->tally_launches = std::atoi(env) != 0;
        int clock_khz = 0;
        LEO_HIP_CHECK(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, device));
        h->wall_clock_khz = clock_khz > 0 ? clock_khz : 100000.0;
        leo::upload_topology(h.get(), *model);
        h->canon = leo::allocate_params(h->canon_params, h->z, h->stream);
        leo::upload_model(h.get(), *model);
        h->canonical = std::make_unique<leo::Lane>();
        leo::allocate_lane_state(*h->canonical, h->z, h->stream, leo::canonical_bucket_sets(h.get()));
        h->canonical->desc.p = h->canon;
        leo::allocate_stale(h.get());
        (void)leo::static_scratch(device);  // set-up of the allocation-free entry point on this device
        h->lane_descs.allocate(sizeof(leo::LaneDesc) * std::max<uint32_t>(h->max_lanes, 1));
        std::vector<leo::Lane*> lanes{h->canonical.get()};
        leo::reset_lane_objects(h.get(), lanes, true, 0);  // Runtime::new: tick 0, empty state
        leo::sync(h->stream);
        // story lanes resident at once: the first lane is allocated now to
        // measure it; larger batches run in groups of this many lanes
        leo::Lane& first = leo::story_lane(h.get(), 0);
        const size_t per_lane = first.state.bytes + first.params.bytes;
        size_t free_bytes = 0, total_bytes = 0;
        LEO_HIP_CHECK(hipMemGetInfo(&free_bytes, &total_bytes));
        const size_t reserve = leo::merge_accumulator_bytes(h->z) + (size_t(1) << 30);
        const size_t fit = free_bytes > reserve ? (free_bytes - reserve) / std::max<size_t>(per_lane, 1) : 0;
        h->resident_lanes = static_cast<uint32_t>(std::min<size_t>(h->max_lanes, 1 + fit));
        // one cooperative launch holds at most cus * coop_blocks_per_cu
        // workgroups, one per lane at the least (lanes padded to the XCDs)
        h->resident_lanes = std::min(h->resident_lanes, leo::cooperative_lane_limit(static_cast<uint32_t>(h->cus),
                                                                                static_cast<uint32_t>(h->coop_blocks_per_cu),
                                                                                leo::kXcds));
        if (const char* env = std::getenv("LEO_HIP_RESIDENT_LANES"))
            h->resident_lanes = std::max<uint32_t>(1, std::min<uint32_t>(h->resident_lanes, std::atoi(env)));
        *out = h.release();
    });
}

void leo_hip_destroy(LeoHipRuntime* runtime) {
    if (!runtime) return;
    (void)hipSetDevice(runtime->device);
    (void)hipStreamSynchronize(runtime->stream);
    hipStream_t s = runtime->stream;
    hipEvent_t e0 = runtime->ev_start, e1 = runtime->ev_stop;
    delete runtime;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
}

int32_t leo_hip_begin_document(LeoHipRuntime* h) {
    return guarded([&] {
        leo::BusyGuard g(h);
        leo::canonical_reset(h);
    });
}

int32_t leo_hip_finish_document(LeoHipRuntime* h) {
    return guarded([&] {
        leo::BusyGuard g(h);
        leo::canonical_finish_document(h);
    });
}

int32_t leo_hip_reset_transient_state(LeoHipRuntime* h) {
    return guarded([&] {
        leo::BusyGuard g(h);
        leo::canonical_reset(h);
    });
}

int32_t leo_hip_enable_parameter_tracking(LeoHipRuntime* h) {
    return guarded([&] {
        leo::BusyGuard g(h);
        // the GPU adapter starts a fresh change set on every call
        // (cuda.rs:2827-2837; the coordinator calls it before each batch's
        // replay, training.rs:1628), unlike the CPU Runtime's no-op when
        // tracking is already on (runtime.rs:310-320)
        h->tracking = true;
        leo::fold_changes(h);  // the changes so far stay marked for the host mirror
        leo::sync(h->stream);
    });
}

int32_t leo_hip_step(LeoHipRuntime* h, uint32_t symbol, int32_t target, int32_t permission, LeoStepMetrics* out) {
    return guarded([&] {
        leo::BusyGuard g(h);
        auto m = leo::canonical_steps(h, {{symbol, target}}, {permission}, true);
        if (out) *out = m[0];
    });
}

int32_t leo_hip_training_step_batch(LeoHipRuntime* h, const uint32_t* symbols, const int32_t* targets, uint32_t count,
                                    int32_t permission, LeoStepMetrics* out) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (count == 0) return;
        if (!symbols || !targets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null step arrays");
        std::vector<leo::HostStep> steps(count);
        for (uint32_t i = 0; i < count; ++i) steps[i] = {symbols[i], targets[i]};
        auto m = leo::canonical_steps(h, steps, std::vector<int32_t>(count, permission), true);
        if (out) std::copy(m.begin(), m.end(), out);
    });
}

int32_t leo_hip_advance_frozen_batch(LeoHipRuntime* h, const uint32_t* symbols, uint32_t count) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (count == 0) return;
        std::vector<leo::HostStep> steps(count);
        for (uint32_t i = 0; i < count; ++i) steps[i] = {symbols[i], -1};
        leo::canonical_steps(h, steps, std::vector<int32_t>(count, LEO_FROZEN), false);
    });
}

int32_t leo_hip_replay_streaming_batch(LeoHipRuntime* h, const uint32_t* symbols, const int32_t* targets,
                                       uint32_t count, int32_t permission, LeoStepMetrics* out, uint32_t* supervised) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (supervised) *supervised = 0;
        if (count == 0) return;
        if (!symbols || !targets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null step arrays");
        std::vector<leo::HostStep> steps(count);
        std::vector<int32_t> perms(count);
        std::vector<bool> outputs(count);
        for (uint32_t i = 0; i < count; ++i) {
            steps[i] = {symbols[i], targets[i]};
            perms[i] = targets[i] >= 0 ? permission : LEO_FROZEN;
            outputs[i] = targets[i] >= 0;
        }
        auto m = leo::canonical_steps(h, steps, perms, outputs);
        uint32_t k = 0;
        for (uint32_t i = 0; i < count; ++i)
            if (targets[i] >= 0) {
                if (out) out[k] = m[i];
                ++k;
            }
        if (supervised) *supervised = k;
    });
}

int32_t leo_hip_training_story_batch(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                                     int32_t permission, float* losses_out, LeoBatchReport* report) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!bytes || !offsets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null story arrays");
        LeoBatchReport rep{};
        leo::story_batch(h, bytes, offsets, count, permission, losses_out, rep);
        if (report) *report = rep;
    });
}

int32_t leo_hip_train_batch(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                            int32_t permission, uint32_t replay_enabled, float* losses_out, LeoBatchReport* report) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!bytes || !offsets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null story arrays");
        if (count == 0) throw Error(LEO_ERR_INVALID_ARGUMENT, "training batch cannot be empty");
        LeoBatchReport rep{};
        std::vector<std::vector<float>> losses(count);
        auto t0 = std::chrono::steady_clock::now();
        if (count == 1) {
            // training.rs:1548-1582: the canonical runtime trains in place
            size_t len = static_cast<size_t>(offsets[1] - offsets[0]);
            if (len > 0) {
                leo::canonical_reset(h);  // begin_document
                auto steps = leo::document_steps(bytes + offsets[0], len);
                auto m = leo::canonical_steps(h, steps, std::vector<int32_t>(steps.size(), permission), true);
                double sum = 0.0;
                for (auto& s : m) {
                    float loss = s.has_loss ? s.loss : 0.0f;
                    losses[0].push_back(loss);
                    sum += static_cast<double>(loss);
                    rep.activity_steps += 1;
                    rep.active_neurons_sum += s.active_neurons;
                    rep.emitted_events += s.emitted_events;
                }
                leo::canonical_finish_document(h);
                rep.mean_loss = sum / static_cast<double>(std::max<size_t>(losses[0].size(), 1));
            }
            rep.targets = losses[0].size();
            rep.stories = 1;
            rep.merge_workers = 1;
            rep.story_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        } else {
            std::vector<float> flat(static_cast<size_t>(offsets[count] - offsets[0]) + count);
            leo::story_batch(h, bytes, offsets, count, permission, flat.data(), rep);
            size_t cursor = 0;
            for (uint32_t i = 0; i < count; ++i) {
                size_t n = static_cast<size_t>(offsets[i + 1] - offsets[i]) + 1;
                losses[i].assign(flat.begin() + cursor, flat.begin() + cursor + n);
                cursor += n;
            }
        }
        if (losses_out) {
            size_t cursor = 0;
            for (auto& l : losses) {
                std::copy(l.begin(), l.end(), losses_out + cursor);
                cursor += l.size();
            }
        }
        auto t1 = std::chrono::steady_clock::now();
        if (replay_enabled) leo::replay_stories(h, bytes, offsets, count, losses, permission, rep);
        rep.replay_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
        if (report) *report = rep;
    });
}

int32_t leo_hip_evaluate(LeoHipRuntime* h, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                         float* losses_out, LeoEvaluationReport* report) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (count > 0 && (!bytes || !offsets)) throw Error(LEO_ERR_INVALID_ARGUMENT, "null story arrays");
        LeoEvaluationReport rep{};
        leo::evaluate_stories(h, bytes, offsets, count, losses_out, rep);
        if (report) *report = rep;
    });
}

int32_t leo_hip_download_model(LeoHipRuntime* h, LeoModelView* out) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null model view");
        leo::download_model(h, *out);
        leo::clear_stale(h);
        leo::sync(h->stream);
    });
}

int32_t leo_hip_upload_model(LeoHipRuntime* h, const LeoModelView* model) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!model) throw Error(LEO_ERR_INVALID_ARGUMENT, "null model view");
        leo::model_validate(h->cfg, *model);
        leo::upload_topology(h, *model);
        leo::upload_model(h, *model);
        // bucket capacities may have changed: story lanes are rebuilt on demand
        h->lanes.clear();
        leo::LaneParams p = h->canon;
        uint32_t tick = h->canonical->tick;
        leo::allocate_lane_state(*h->canonical, h->z, h->stream, leo::canonical_bucket_sets(h));
        h->canonical->desc.p = p;
        std::vector<leo::Lane*> lanes{h->canonical.get()};
        leo::reset_lane_objects(h, lanes, true, tick);
        // the caller's mirror is the model just uploaded
        leo::clear_changes(*h->canonical, h->z, h->stream);
        leo::clear_stale(h);
        leo::sync(h->stream);
    });
}

int32_t leo_hip_synchronize_model(LeoHipRuntime* h, LeoModelView* mirror) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!mirror) throw Error(LEO_ERR_INVALID_ARGUMENT, "null model view");
        leo::synchronize_host(h, *mirror);
    });
}

int32_t leo_hip_synchronize_packed_model(LeoHipRuntime* h, const LeoPackedUpdate* update) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!update) throw Error(LEO_ERR_INVALID_ARGUMENT, "null packed update");
        leo::apply_packed(h, *update, true);
    });
}

int32_t leo_hip_commit_packed_host_model(LeoHipRuntime* h, const LeoPackedUpdate* update) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!update) throw Error(LEO_ERR_INVALID_ARGUMENT, "null packed update");
        leo::apply_packed(h, *update, false);
    });
}

int32_t leo_hip_commit_packed_host_model_no_alloc(LeoHipRuntime* h, const LeoPackedUpdate* update) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (!update) throw Error(LEO_ERR_INVALID_ARGUMENT, "null packed update");
        leo::Staging staging;
        staging.fixed = leo::static_scratch(h->device);
        staging.capacity = leo::kStaticScratchBytes;
        // apply_packed synchronises its stream before returning, so the
        // device's copy is free again when the lock is released
        std::lock_guard<std::mutex> lock(leo::g_scratch_user[h->device]);
        leo::apply_packed(h, *update, false, staging);
    });
}

int32_t leo_hip_parameter_changes(LeoHipRuntime* h, int32_t which, uint64_t* out, uint64_t capacity, uint64_t* count,
                                  uint32_t* bias_dirty, uint32_t* context_output_dirty) {
    return guarded([&] {
        leo::BusyGuard g(h);
        const leo::LaneDesc& d = h->canonical->desc;
        const leo::Sizes& z = h->z;
        const uint32_t* bits = nullptr;
        uint64_t n = 0;
        switch (which) {
            case LEO_CHANGED_THRESHOLD: bits = d.ch_threshold; n = z.n; break;
            case LEO_CHANGED_RECURRENT: bits = d.ch_rec; n = z.ns; break;
            case LEO_CHANGED_INPUT: bits = d.ch_in; n = z.ni; break;
            case LEO_CHANGED_OUTPUT_NEURONS: bits = d.ch_out; n = z.n; break;
            case LEO_CHANGED_CONTEXT_SLOTS: bits = d.ch_ctx; n = z.slots; break;
            default: throw Error(LEO_ERR_INVALID_ARGUMENT, "unknown change set");
        }
        std::vector<uint64_t> idx;
        uint32_t flags[2] = {0, 0};
        if (h->tracking) {
            auto v = leo::download_bits(h, bits, n);
            leo::download(flags, &d.ctl->bias_dirty, 8, h->stream);
            leo::sync(h->stream);
            idx = leo::bits_to_indices(v, n);
        }
        if (count) *count = idx.size();
        if (out)
            for (uint64_t i = 0; i < std::min<uint64_t>(capacity, idx.size()); ++i) out[i] = idx[i];
        if (bias_dirty) *bias_dirty = flags[0];
        if (context_output_dirty) *context_output_dirty = flags[1];
    });
}

int32_t leo_hip_probabilities(LeoHipRuntime* h, float* out257) {
    return guarded([&] {
        leo::BusyGuard g(h);
        leo::download(out257, h->canonical->desc.probs, leo::kOutputs * 4, h->stream);
        leo::sync(h->stream);
    });
}

int32_t leo_hip_read_list(LeoHipRuntime* h, int32_t which, uint64_t* out, uint64_t capacity, uint64_t* count) {
    return guarded([&] {
        leo::BusyGuard g(h);
        const leo::LaneDesc& d = h->canonical->desc;
        leo::LaneControl ctl{};
        leo::download(&ctl, d.ctl, sizeof(ctl), h->stream);
        leo::sync(h->stream);
        std::vector<uint32_t> v;
        bool sorted = true;
        const uint32_t last = ctl.tick - 1;
        switch (which) {
            case LEO_LIST_ACTIVE: {
                uint32_t rs = last % leo::kRing;
                uint32_t n = (ctl.tick > 0 && ctl.ring_tick[rs] == last) ? ctl.ring_count[rs] : 0;
                v.resize(n);
                leo::download(v.data(), d.ring_active + static_cast<uint64_t>(rs) * h->z.cap, n * 4, h->stream);
                sorted = false;
                break;
            }
            case LEO_LIST_TOUCHED: {
                // neurons whose touched epoch is the last tick's (tick + 1)
                if (ctl.tick == 0) break;
                std::vector<uint32_t> rec(h->z.n * leo::kNeuronWords);
                leo::download(rec.data(), d.neuron, rec.size() * 4, h->stream);
                leo::sync(h->stream);
                for (uint32_t n = 0; n < h->z.n; ++n)
                    if (rec[static_cast<size_t>(n) * leo::kNeuronWords + leo::kNTouched] == ctl.tick) v.push_back(n);
                break;
            }
            case LEO_LIST_ELIGIBLE_REC: {
                uint32_t n = ctl.rec_count[ctl.parity];
                v.resize(n);
                leo::download(v.data(), d.rec_list + static_cast<uint64_t>(ctl.parity) * h->z.ns, n * 4, h->stream);
                break;
            }
            case LEO_LIST_ELIGIBLE_IN: {
                uint32_t n = ctl.in_count[ctl.parity];
                v.resize(n);
                leo::download(v.data(), d.in_list + static_cast<uint64_t>(ctl.parity) * h->z.ni, n * 4, h->stream);
                break;
            }
            default: throw Error(LEO_ERR_INVALID_ARGUMENT, "unknown list");
        }
        leo::sync(h->stream);
        if (sorted) std::sort(v.begin(), v.end());
        if (count) *count = v.size();
        if (out)
            for (uint64_t i = 0; i < std::min<uint64_t>(capacity, v.size()); ++i) out[i] = v[i];
    });
}

int32_t leo_hip_read_active(LeoHipRuntime* h, uint64_t* neurons, float* activations, uint64_t capacity,
                            uint64_t* count) {
    return guarded([&] {
        leo::BusyGuard g(h);
        const leo::LaneDesc& d = h->canonical->desc;
        leo::LaneControl ctl{};
        leo::download(&ctl, d.ctl, sizeof(ctl), h->stream);
        leo::sync(h->stream);
        // the ring entry of the last tick (a reset empties the ring)
        const uint32_t last = ctl.tick - 1, rs = last % leo::kRing;
        const uint32_t n = (ctl.tick > 0 && ctl.ring_tick[rs] == last) ? ctl.ring_count[rs] : 0;
        std::vector<uint32_t> ids(n);
        std::vector<float> values(n);
        const uint64_t at = static_cast<uint64_t>(rs) * h->z.cap;
        leo::download(ids.data(), d.ring_active + at, n * 4, h->stream);
        leo::download(values.data(), d.ring_act + at, n * 4, h->stream);
        leo::sync(h->stream);
        if (count) *count = n;
        const uint64_t k = std::min<uint64_t>(capacity, n);
        for (uint64_t i = 0; i < k; ++i) {
            if (neurons) neurons[i] = ids[i];
            if (activations) activations[i] = values[i];
        }
    });
}

int32_t leo_hip_read_state(LeoHipRuntime* h, int32_t which, float* out, uint64_t count) {
    return guarded([&] {
        leo::BusyGuard g(h);
        const leo::LaneDesc& d = h->canonical->desc;
        const leo::Sizes& z = h->z;
        const float* src = nullptr;
        uint64_t n = 0;
        // per-neuron state: `words` consecutive words of each neuron's record
        uint32_t field = 0, words = 0;
        if ((which >= LEO_STATE_REC_BS && which <= LEO_STATE_REC_E) || (which >= LEO_STATE_IN_BS && which <= LEO_STATE_IN_E)) {
            // one word of each slot's trace record
            const bool rec = which <= LEO_STATE_REC_E;
            const uint64_t slots = rec ? z.ns : z.ni;
            const uint32_t word = static_cast<uint32_t>(which - (rec ? LEO_STATE_REC_BS : LEO_STATE_IN_BS));
            if (count != slots) throw Error(LEO_ERR_INVALID_ARGUMENT, "state size mismatch: expected " + std::to_string(slots));
            std::vector<float> all(slots * leo::kTraceWords);
            leo::download(all.data(), rec ? d.rec_trace : d.in_trace, all.size() * 4, h->stream);
            leo::sync(h->stream);
            for (uint64_t i = 0; i < slots; ++i) out[i] = all[i * leo::kTraceWords + word];
            return;
        } else {
            switch (which) {
                case LEO_STATE_MEMBRANE: field = leo::kNMembrane; words = 1; break;
                case LEO_STATE_ACTIVATION: field = leo::kNActivation; words = 1; break;
                case LEO_STATE_FATIGUE: field = leo::kNFatigue; words = 1; break;
                case LEO_STATE_BRANCHES: field = leo::kNBranch0; words = 4; break;
                case LEO_STATE_ADAPT0: field = leo::kNAdapt0; words = 1; break;
                case LEO_STATE_ADAPT1: field = leo::kNAdapt0 + 1; words = 1; break;
                case LEO_STATE_ADAPT2: field = leo::kNAdapt0 + 2; words = 1; break;
                case LEO_STATE_SURROGATE:
                    throw Error(LEO_ERR_UNSUPPORTED, "surrogates are evaluated where the eligibility update uses them, not stored");
                case LEO_STATE_LOGITS: src = d.logits; n = leo::kOutputs; break;
                case LEO_STATE_PROBABILITIES: src = d.probs; n = leo::kOutputs; break;
                case LEO_STATE_ERRORS: src = d.errors; n = leo::kOutputs; break;
                case LEO_STATE_LEARNING_SIGNAL: src = d.learning_signal; n = z.n; break;
                default: throw Error(LEO_ERR_INVALID_ARGUMENT, "unknown state selector");
            }
        }
        if (words) n = static_cast<uint64_t>(words) * z.n;
        if (count != n) throw Error(LEO_ERR_INVALID_ARGUMENT, "state size mismatch: expected " + std::to_string(n));
        if (words) {
            std::vector<float> rec(z.n * leo::kNeuronWords);
            leo::download(rec.data(), d.neuron, rec.size() * 4, h->stream);
            leo::sync(h->stream);
            for (uint64_t i = 0; i < z.n; ++i)
                for (uint32_t w = 0; w < words; ++w) out[i * words + w] = rec[i * leo::kNeuronWords + field + w];
            return;
        }
        leo::download(out, src, n * 4, h->stream);
        leo::sync(h->stream);
    });
}

uint64_t leo_hip_current_tick(const LeoHipRuntime* h) { return h ? h->canonical->tick : 0; }

int32_t leo_hip_kernel_stats(LeoHipRuntime* h, LeoKernelStats* out, int32_t reset) {
    return guarded([&] {
        leo::BusyGuard g(h);
        if (out) {
            *out = h->telemetry;
            out->resident_lanes = h->resident_lanes;
        }
        if (reset) h->telemetry = LeoKernelStats{};
    });
}

}  // extern "C"
