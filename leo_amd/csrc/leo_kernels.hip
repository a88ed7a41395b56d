// HIP kernels for gfx950: Leo's per-byte training step (runtime.rs:427-535)
// over independent lanes, the transient-state reset (runtime.rs:365-425) and
// the batch-end lane-ordered mean of the fixed parameters (parallel.rs:694-1022,
// 1169-1345).
//
// Execution model. One cooperative launch runs a chunk of steps for every
// lane. Lane l owns workgroups {l, l+L, l+2L, ...} (blockIdx % L), so with L a
// multiple of the 8 XCDs every workgroup of a lane sits on one XCD and its L2.
// Phases of a step are separated by a lane-group barrier (an arrival counter
// per lane), not a grid barrier: lanes never wait on each other.
//
// Exactness. Every FP32 operation is the reference's operation in the
// reference's order: the file is compiled with -ffp-contract=off, per-target
// branch accumulation is a sequential fold in CPU delivery order (sorted by
// (emission delay class, active rank, slot)), the logit/signal/softmax sums
// are serial, exp is glibc_expf_nonpositive and powi is compiler-rt's
// square-and-multiply.

#include <hip/hip_runtime.h>

#include "glibc_expf.h"
#include "leo_device.h"

namespace leo {

constexpr uint8_t BR_EXC = 0, BR_INH = 1, BR_TEMP = 2, BR_GATE = 3;

__device__ __forceinline__ float clampf(float v, float lo, float hi) {  // Rust f32::clamp
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}
__device__ __forceinline__ float maxnum(float a, float b) {  // Rust f32::max
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}
__device__ __forceinline__ bool finitef(float v) { return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u; }

// compiler-rt powisf2 (Rust f32::powi with a runtime exponent).
__device__ __forceinline__ float powisf2(float a, int b) {
    float r = 1.0f;
    while (true) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return r;
}
// runtime.rs:78-85
__device__ __forceinline__ float decay_for_elapsed(float base, uint32_t elapsed) {
    if (elapsed == 0) return 1.0f;
    if (elapsed == 1) return base;
    return powisf2(base, static_cast<int>(elapsed > 0x7fffffffu ? 0x7fffffffu : elapsed));
}
// learning.rs:7-24
__device__ __forceinline__ float analog_rank_surrogate(float margin, float cutoff, bool selected, float width,
                                                       float gain) {
    float direct = (selected && margin > 0.0f && margin < 1.0f) ? 1.0f : 0.0f;
    if (width <= 0.0f || gain <= 0.0f) return direct;
    float boundary = clampf(1.0f - fabsf(margin - cutoff) / width, 0.0f, 1.0f);
    return direct + gain * boundary;
}
// learning.rs:29-51
__device__ __forceinline__ float branch_jacobian(uint8_t br, float exc, float temporal, float gate_acc) {
    float gate = clampf(gate_acc, 0.0f, 1.0f);
    if (br == BR_EXC || br == BR_INH) return exc;
    if (br == BR_TEMP) return exc * gate;
    if (br == BR_GATE) {
        float d = (gate_acc > 0.0f && gate_acc < 1.0f) ? 1.0f : 0.0f;
        return exc * temporal * d;
    }
    return 0.0f;
}
__device__ __forceinline__ float bounded(float v, float m) { return clampf(v, -m, m); }

// runtime.rs:679-690
__device__ uint64_t context_key(const uint32_t* history, uint32_t len, uint32_t order) {
    uint64_t h = 0xcbf29ce484222325ULL ^ static_cast<uint64_t>(order);
    for (uint32_t i = len - order; i < len; ++i) {
        uint32_t s = history[i];
        for (int b = 0; b < 4; ++b) {
            h ^= static_cast<uint64_t>((s >> (8 * b)) & 0xffu);
            h *= 0x100000001b3ULL;
        }
    }
    return h < 1 ? 1 : h;
}

__device__ __forceinline__ void set_error(LaneControl* ctl, uint32_t code) { atomicCAS(&ctl->error_code, 0u, code); }
__device__ __forceinline__ void mark_bit(uint32_t* bits, uint32_t index) { atomicOr(&bits[index >> 5], 1u << (index & 31)); }

// Workgroup-wide sum of a per-thread count, added to *global once.
__device__ void add_count(uint32_t* global, uint32_t local) {
    __shared__ uint32_t s_count;
    if (threadIdx.x == 0) s_count = 0;
    __syncthreads();
    if (local) atomicAdd(&s_count, local);
    __syncthreads();
    if (threadIdx.x == 0 && s_count) atomicAdd(global, s_count);
}

// Lane-group barrier. Every thread publishes its writes with an agent-scope
// fence, thread 0 arrives on the lane's counter and waits for all P
// workgroups, and the acquire fence afterwards makes the other workgroups'
// writes visible. The wait is bounded: on timeout the lane is aborted and
// every workgroup leaves the step loop, so the grid always drains.
__device__ bool lane_barrier(LaneControl* ctl, uint32_t P, uint32_t& target, uint32_t spin_limit) {
    __shared__ uint32_t s_abort;
    if (P == 1) {
        __syncthreads();
        return true;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        target += P;
        __hip_atomic_fetch_add(&ctl->barrier, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        uint32_t aborted = 0;
        while (__hip_atomic_load(&ctl->barrier, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (__hip_atomic_load(&ctl->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                aborted = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            if (++spins > spin_limit) {
                __hip_atomic_store(&ctl->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                set_error(ctl, kErrBarrier);
                aborted = 1;
                break;
            }
        }
        s_abort = aborted;
    }
    __syncthreads();
    __threadfence();
    return s_abort == 0;
}

// Bitonic sort (ascending) of n = power of two keys in LDS by the workgroup.
__device__ void bitonic_sort_lds(uint64_t* keys, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
                uint32_t ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = keys[i], b = keys[ixj];
                    bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        keys[i] = b;
                        keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ uint32_t next_pow2(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Selection key: ascending order == (activation desc, rotated tie key asc)
// (runtime.rs:987-1009); activation > 0 so its bit pattern is monotone.
__device__ __forceinline__ uint64_t selection_key(float act, uint32_t tie) {
    return (static_cast<uint64_t>(~__float_as_uint(act)) << 32) | tie;
}
__device__ __forceinline__ float key_activation(uint64_t key) { return __uint_as_float(~static_cast<uint32_t>(key >> 32)); }

struct StepCtx {
    const KernelArgs* a;
    const LaneDesc* d;
    LaneControl* ctl;
    uint32_t tick;
    uint32_t part;     // workgroup index within the lane group
    uint32_t P;
    uint32_t gtid;
    uint32_t gstride;
    uint32_t parity;   // current eligible list
    uint32_t dest_epoch;
};

// ---------------------------------------------------------------------------
// Phase 1: start_tick (runtime.rs:537-561), event delivery scatter
// (runtime.rs:605-625) and injection (runtime.rs:627-639). Trace activation
// (runtime.rs:710-766) is slot-local; branch adds go to per-target buckets
// keyed by CPU delivery order and are folded in phase 2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void touch(const StepCtx& c, uint32_t n) {
    const LaneDesc& d = *c.d;
    uint32_t old = atomicExch(&d.touched_epoch[n], c.tick + 1);
    if (old != c.tick + 1) {
        uint32_t pos = atomicAdd(&c.ctl->tick_touched[c.tick & 1], 1u);
        d.touched_list[pos] = n;
    }
}

__device__ __forceinline__ void advance_trace(float* planes, uint64_t plane, uint32_t* last, uint32_t slot,
                                              uint32_t tick, const LeoConfig& cfg) {
    uint32_t e = tick - last[slot];
    if (e == 0) return;
    planes[slot] *= decay_for_elapsed(cfg.branch_decay, e);
    planes[plane + slot] *= decay_for_elapsed(cfg.membrane_decay, e);
    planes[2 * plane + slot] *= decay_for_elapsed(cfg.fatigue_decay, e);
    planes[3 * plane + slot] *= decay_for_elapsed(cfg.adaptation_fast_decay, e);
    planes[4 * plane + slot] *= decay_for_elapsed(cfg.adaptation_medium_decay, e);
    planes[5 * plane + slot] *= decay_for_elapsed(cfg.adaptation_slow_decay, e);
    last[slot] = tick;
}

// Late fields of a step record: work counters complete only after the step's
// last barrier, so the record is finished by the next step (or kernel end).
__device__ void finalize_record(const LaneDesc& d, LaneControl* ctl, uint32_t step_index, uint32_t tick) {
    StepRecord& rec = d.records[step_index];
    const uint32_t k = tick & 1;
    rec.events = ctl->tick_events[k];
    rec.touched = ctl->tick_touched[k];
    rec.scanned_rec = ctl->tick_scan_rec[k];
    rec.scanned_in = ctl->tick_scan_in[k];
    rec.destinations = ctl->tick_dest[k];
    rec.active_inhibitory = ctl->tick_ainh[k];
}

__device__ void phase_deliver(const StepCtx& c, const StepParams& sp, uint32_t step_index) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t S = cfg.synapses_per_neuron, F = cfg.input_fanout, cap = cfg.max_active_global;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * S;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * F;
    const bool trace = (sp.flags & kStepLearnTrace) != 0;
    const uint32_t tick = c.tick;
    if (c.part == 0 && threadIdx.x == 0) {
        LaneControl* ctl = c.ctl;
        if (step_index > 0) finalize_record(d, ctl, step_index - 1, tick - 1);
        const uint32_t n = (tick + 1) & 1;
        ctl->tick_touched[n] = 0;
        ctl->tick_supra[n] = 0;
        ctl->tick_events[n] = 0;
        ctl->tick_dest[n] = 0;
        ctl->tick_ainh[n] = 0;
        ctl->tick_scan_rec[n] = 0;
        ctl->tick_scan_in[n] = 0;
        ctl->rec_count[c.parity ^ 1] = 0;
        ctl->in_count[c.parity ^ 1] = 0;
    }
    // previous active set (runtime.rs:544-555)
    uint32_t prev_slot = (tick + kRing - 1) % kRing;
    uint32_t prev_count = (tick > 0 && c.ctl->ring_tick[prev_slot] == tick - 1) ? c.ctl->ring_count[prev_slot] : 0;
    // delivery classes: delay 8, 4, 2, 1 in that order (chronological by emission tick)
    uint32_t cls_slot[4], cls_count[4], cls_off[5];
    cls_off[0] = prev_count;
    for (int k = 0; k < 4; ++k) {
        uint32_t delay = 8u >> k;
        uint32_t rs = (tick + kRing - delay) % kRing;
        bool valid = tick >= delay && c.ctl->ring_tick[rs] == tick - delay;
        cls_slot[k] = rs;
        cls_count[k] = valid ? c.ctl->ring_count[rs] : 0;
        cls_off[k + 1] = cls_off[k] + cls_count[k] * S;
    }
    const uint32_t total = cls_off[4] + F;
    uint32_t delivered = 0;
    for (uint32_t item = c.gtid; item < total; item += c.gstride) {
        if (item < prev_count) {
            uint32_t n = d.ring_active[static_cast<uint64_t>(prev_slot) * cap + item];
            d.activation[n] = 0.0f;
            touch(c, n);
        } else if (item < cls_off[4]) {
            int k = 0;
            while (item >= cls_off[k + 1]) ++k;
            uint32_t local = item - cls_off[k];
            uint32_t r = local / S, j = local % S;
            uint64_t rbase = static_cast<uint64_t>(cls_slot[k]) * cap + r;
            uint32_t src = d.ring_active[rbase];
            uint64_t slot = static_cast<uint64_t>(src) * S + j;
            if (a.m.rec_delay[slot] != (8u >> k)) continue;
            delivered += 1;
            float act = d.ring_act[rbase];
            float value = d.ring_value[rbase * S + j];
            uint32_t target = a.m.rec_target[slot];
            uint8_t br = a.m.rec_branch[slot];
            if (trace) {
                advance_trace(d.rec_trace, NS, d.rec_last, static_cast<uint32_t>(slot), tick, cfg);
                d.rec_trace[slot] += act;
                if (!d.rec_mark[slot]) {
                    d.rec_mark[slot] = 1;
                    uint32_t pos = atomicAdd(&c.ctl->rec_count[c.parity], 1u);
                    d.rec_list[static_cast<uint64_t>(c.parity) * NS + pos] = static_cast<uint32_t>(slot);
                }
            }
            if (target < cfg.neuron_count && br <= BR_GATE) {
                touch(c, target);
                uint32_t pos = atomicAdd(&d.bucket_count[target], 1u);
                uint64_t key = (static_cast<uint64_t>(k) << 61) | (static_cast<uint64_t>(r) << 32) |
                               (static_cast<uint64_t>(j) << 2) | br;
                uint64_t at = a.m.bucket_offset[target] + pos;
                d.bucket[2 * at] = key;
                d.bucket[2 * at + 1] = __float_as_uint(value);
            }
        } else {
            uint32_t i = item - cls_off[4];
            uint64_t slot = static_cast<uint64_t>(sp.symbol) * F + i;
            uint32_t target = a.m.in_target[slot];
            uint8_t br = a.m.in_branch[slot];
            float value = d.p.in_weight[slot];
            if (trace) {
                advance_trace(d.in_trace, NI, d.in_last, static_cast<uint32_t>(slot), tick, cfg);
                d.in_trace[slot] += 1.0f;
                if (!d.in_mark[slot]) {
                    d.in_mark[slot] = 1;
                    uint32_t pos = atomicAdd(&c.ctl->in_count[c.parity], 1u);
                    d.in_list[static_cast<uint64_t>(c.parity) * NI + pos] = static_cast<uint32_t>(slot);
                }
            }
            if (target < cfg.neuron_count && br <= BR_GATE) {
                touch(c, target);
                uint32_t pos = atomicAdd(&d.bucket_count[target], 1u);
                uint64_t key = (4ULL << 61) | (static_cast<uint64_t>(i) << 2) | br;
                uint64_t at = a.m.bucket_offset[target] + pos;
                d.bucket[2 * at] = key;
                d.bucket[2 * at + 1] = __float_as_uint(value);
            }
        }
    }
    add_count(&c.ctl->tick_events[tick & 1], delivered);
}

// ---------------------------------------------------------------------------
// Phase 2: bring each touched neuron to the current tick (runtime.rs:576-603)
// and fold its delivered values in CPU order; resolve the context
// (runtime.rs:641-677, model.rs:173-221) on one thread.
// ---------------------------------------------------------------------------
__device__ void context_resolve(const StepCtx& c, const StepParams& sp) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = *c.d;
    LaneControl* ctl = c.ctl;
    const uint32_t max_order = cfg.context_max_order, E = cfg.context_embedding_dim;
    uint32_t len = ctl->history_len;
    if (len == max_order) {
        for (uint32_t i = 1; i < len; ++i) ctl->history[i - 1] = ctl->history[i];
        len -= 1;
    }
    ctl->history[len++] = sp.symbol;
    ctl->history_len = len;
    const bool enabled = (sp.flags & kStepContext) != 0;
    const bool allocate = (sp.flags & kStepAllocate) != 0;
    ctl->ctx_applied = enabled ? 1u : 0u;
    uint32_t count = 0, probes = 0;
    if (enabled) {
        const float confidence_target = static_cast<float>(cfg.context_confidence_observations);
        const uint32_t spo = cfg.context_slots_per_order;
        float scale_sum = 0.0f;
        for (uint32_t order = 1; order <= len; ++order) {
            uint64_t key = context_key(ctl->history, len, order);
            uint64_t base = static_cast<uint64_t>(order - 1) * spo;
            uint64_t start = key % spo;
            int64_t found = -1, empty = -1;
            uint64_t weakest = base + start;
            uint32_t weakest_obs = 0xffffffffu;
            for (uint32_t off = 0; off < cfg.context_probe_limit; ++off) {
                uint64_t slot = base + (start + off) % spo;
                probes += 1;
                uint64_t existing = d.p.ctx_keys[slot];
                if (existing == key) {
                    found = static_cast<int64_t>(slot);
                    break;
                }
                if (existing == 0 && empty < 0) empty = static_cast<int64_t>(slot);
                uint32_t obs = d.p.ctx_obs[slot];
                if (obs < weakest_obs) {
                    weakest_obs = obs;
                    weakest = slot;
                }
            }
            if (found < 0) {
                if (!allocate) continue;
                uint64_t slot = empty >= 0 ? static_cast<uint64_t>(empty) : weakest;
                if (d.p.ctx_keys[slot] != key) {
                    d.p.ctx_keys[slot] = key;
                    d.p.ctx_obs[slot] = 0;
                    for (uint32_t e = 0; e < E; ++e) d.p.ctx_emb[slot * E + e] = 0.0f;
                }
                found = static_cast<int64_t>(slot);
            }
            float obs = static_cast<float>(d.p.ctx_obs[found]);
            float confidence = obs / (obs + confidence_target);
            float scale = confidence * static_cast<float>(order);
            ctl->ctx_slots[count] = static_cast<uint32_t>(found);
            ctl->ctx_scales[count] = scale;
            count += 1;
            scale_sum += scale;
        }
        if (scale_sum > 0.0f)
            for (uint32_t i = 0; i < count; ++i) ctl->ctx_scales[i] = ctl->ctx_scales[i] / scale_sum;
    }
    ctl->ctx_count = count;
    ctl->ctx_probes = probes;
}

__device__ void phase_fold(const StepCtx& c, const StepParams& sp) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count;
    const uint32_t tick = c.tick;
    if (c.part == 0 && threadIdx.x == 0) context_resolve(c, sp);
    const uint32_t touched = c.ctl->tick_touched[tick & 1];
    for (uint32_t i = c.gtid; i < touched; i += c.gstride) {
        uint32_t n = d.touched_list[i];
        float b0 = d.branches[4 * n], b1 = d.branches[4 * n + 1], b2 = d.branches[4 * n + 2], b3 = d.branches[4 * n + 3];
        uint32_t e = tick - d.last_tick[n];
        if (e > 0) {
            float bd = decay_for_elapsed(cfg.branch_decay, e);
            b0 *= bd;
            b1 *= bd;
            b2 *= bd;
            b3 *= bd;
            d.membrane[n] *= decay_for_elapsed(cfg.membrane_decay, e);
            d.fatigue[n] *= decay_for_elapsed(cfg.fatigue_decay, e);
            d.adapt[n] *= decay_for_elapsed(cfg.adaptation_fast_decay, e);
            d.adapt[N + n] *= decay_for_elapsed(cfg.adaptation_medium_decay, e);
            d.adapt[2 * N + n] *= decay_for_elapsed(cfg.adaptation_slow_decay, e);
            d.last_tick[n] = tick;
        }
        uint32_t cnt = d.bucket_count[n];
        if (cnt > 0) {
            uint64_t* ent = d.bucket + 2 * a.m.bucket_offset[n];
            // insertion sort by order key (entries are (key, value) pairs)
            for (uint32_t x = 1; x < cnt; ++x) {
                uint64_t k = ent[2 * x], v = ent[2 * x + 1];
                uint32_t y = x;
                while (y > 0 && ent[2 * (y - 1)] > k) {
                    ent[2 * y] = ent[2 * (y - 1)];
                    ent[2 * y + 1] = ent[2 * (y - 1) + 1];
                    --y;
                }
                ent[2 * y] = k;
                ent[2 * y + 1] = v;
            }
            for (uint32_t x = 0; x < cnt; ++x) {
                float v = __uint_as_float(static_cast<uint32_t>(ent[2 * x + 1]));
                switch (static_cast<uint32_t>(ent[2 * x]) & 3u) {
                    case 0: b0 += v; break;
                    case 1: b1 += v; break;
                    case 2: b2 += v; break;
                    default: b3 += v; break;
                }
            }
            d.bucket_count[n] = 0;
        }
        d.branches[4 * n] = b0;
        d.branches[4 * n + 1] = b1;
        d.branches[4 * n + 2] = b2;
        d.branches[4 * n + 3] = b3;
    }
}

// ---------------------------------------------------------------------------
// Phase 3: drive, membrane and per-block top-k (runtime.rs:940-1011); with a
// non-binding global cap also activation, selection marks and surrogates
// (runtime.rs:1060-1067, 787-803).
// ---------------------------------------------------------------------------
__device__ void surrogate_for(const StepCtx& c, uint32_t n, float block_cutoff, float pop_cutoff) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = *c.d;
    if (d.refractory_until[n] > c.tick) {
        d.surrogate[n] = 0.0f;
        return;
    }
    float margin = d.membrane[n] - d.p.threshold[n];
    float cutoff = maxnum(block_cutoff, pop_cutoff);
    bool selected = d.selected_epoch[n] == c.tick + 1;
    d.surrogate[n] = analog_rank_surrogate(margin, cutoff, selected, cfg.surrogate_width, cfg.surrogate_gain);
}

__device__ void phase_select(const StepCtx& c, uint64_t* s_keys, uint32_t* s_u32) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, nb = cfg.neurons_per_block, limit = cfg.max_active_per_block;
    const uint32_t tick = c.tick;
    const uint32_t rot = tick % N;
    const float pi = c.ctl->population_inhibition;
    const uint32_t M = next_pow2(nb);
    for (uint32_t b = c.part; b < cfg.block_count; b += c.P) {
        if (threadIdx.x == 0) s_u32[0] = 0;
        __syncthreads();
        uint32_t local_candidates = 0;
        for (uint32_t idx = threadIdx.x; idx < M; idx += kThreads) {
            uint64_t key = ~0ULL;
            if (idx < nb) {
                uint32_t n = b * nb + idx;
                if (d.touched_epoch[n] == tick + 1 && !(d.refractory_until[n] > tick)) {
                    float gate = clampf(d.branches[4 * n + BR_GATE], 0.0f, 1.0f);
                    float inhibitory = d.branches[4 * n + BR_INH];
                    float net = d.branches[4 * n + BR_EXC] + d.branches[4 * n + BR_TEMP] * gate + inhibitory;
                    float adaptation = d.adapt[n] + d.adapt[N + n] + d.adapt[2 * N + n];
                    float drive = a.m.excitability[n] * net - d.fatigue[n] - adaptation - pi;
                    float m = d.membrane[n] + drive;
                    d.membrane[n] = m;
                    float act = clampf(m - d.p.threshold[n], 0.0f, 1.0f);
                    if (act > 0.0f) {
                        key = selection_key(act, (n + N - rot) % N);
                        local_candidates += 1;
                    }
                }
            }
            s_keys[idx] = key;
        }
        if (local_candidates) atomicAdd(&s_u32[0], local_candidates);
        __syncthreads();
        const uint32_t count = s_u32[0];
        if (count > 0) bitonic_sort_lds(s_keys, M);
        const uint32_t winners = count < limit ? count : limit;
        const float cutoff = count > limit ? key_activation(s_keys[limit]) : 0.0f;
        for (uint32_t i = threadIdx.x; i < winners; i += kThreads) {
            uint64_t key = s_keys[i];
            uint32_t n = (static_cast<uint32_t>(key) + rot) % N;
            d.block_winners[static_cast<uint64_t>(b) * limit + i] = n;
            if (a.redundant_global) {
                d.activation[n] = key_activation(key);
                d.selected_epoch[n] = tick + 1;
            }
        }
        if (threadIdx.x == 0) {
            d.block_count[b] = winners;
            d.block_cutoff[b] = cutoff;
            if (count) atomicAdd(&c.ctl->tick_supra[tick & 1], count);
        }
        __syncthreads();
        if (a.redundant_global) {
            for (uint32_t idx = threadIdx.x; idx < nb; idx += kThreads) {
                uint32_t n = b * nb + idx;
                if (d.touched_epoch[n] == tick + 1) surrogate_for(c, n, cutoff, 0.0f);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Phase 4a (workgroup 0): concatenate block winners into the active list of
// this tick's ring slot; with a binding global cap, sort and truncate
// (runtime.rs:1013-1057); update population inhibition (runtime.rs:1076-1082).
// ---------------------------------------------------------------------------
__device__ void build_active(const StepCtx& c, uint64_t* s_keys, uint32_t* s_u32) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, limit = cfg.max_active_per_block, cap = cfg.max_active_global;
    const uint32_t tick = c.tick;
    const uint32_t rs = tick % kRing;
    uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    // exclusive scan of block winner counts, in block order
    uint32_t running = 0;
    const bool redundant = a.redundant_global != 0;
    for (uint32_t base = 0; base < cfg.block_count; base += kThreads) {
        uint32_t b = base + threadIdx.x;
        uint32_t v = b < cfg.block_count ? d.block_count[b] : 0;
        s_u32[threadIdx.x] = v;
        __syncthreads();
        for (uint32_t off = 1; off < kThreads; off <<= 1) {
            uint32_t add = threadIdx.x >= off ? s_u32[threadIdx.x - off] : 0;
            __syncthreads();
            s_u32[threadIdx.x] += add;
            __syncthreads();
        }
        uint32_t incl = s_u32[threadIdx.x];
        uint32_t start = running + incl - v;
        if (redundant) {
            for (uint32_t i = 0; i < v; ++i) {
                uint32_t n = d.block_winners[static_cast<uint64_t>(b) * limit + i];
                act_list[start + i] = n;
                act_val[start + i] = d.activation[n];
            }
        } else {
            for (uint32_t i = 0; i < v; ++i) {
                uint32_t n = d.block_winners[static_cast<uint64_t>(b) * limit + i];
                if (start + i < kMaxBlockNeurons) {
                    float act = clampf(d.membrane[n] - d.p.threshold[n], 0.0f, 1.0f);
                    s_keys[start + i] = selection_key(act, (n + N - tick % N) % N);
                }
            }
        }
        uint32_t chunk_total = s_u32[kThreads - 1];
        __syncthreads();
        running += chunk_total;
    }
    uint32_t active = running, clipped = 0;
    float pop_cutoff = 0.0f;
    if (!redundant) {
        if (running > kMaxBlockNeurons) {
            if (threadIdx.x == 0) set_error(c.ctl, kErrCapacity);
            active = 0;
        } else {
            uint32_t M = next_pow2(running < 2 ? 2 : running);
            for (uint32_t i = running + threadIdx.x; i < M; i += kThreads) s_keys[i] = ~0ULL;
            __syncthreads();
            bitonic_sort_lds(s_keys, M);
            active = running < cap ? running : cap;
            clipped = running - active;
            if (running > cap) pop_cutoff = clampf(key_activation(s_keys[cap]), 0.0f, cfg.population_inhibition_max);
            for (uint32_t i = threadIdx.x; i < active; i += kThreads) {
                uint64_t key = s_keys[i];
                uint32_t n = (static_cast<uint32_t>(key) + tick % N) % N;
                float act = key_activation(key);
                act_list[i] = n;
                act_val[i] = act;
                d.activation[n] = act;
                d.selected_epoch[n] = tick + 1;
            }
        }
    }
    if (threadIdx.x == 0) {
        LaneControl* ctl = c.ctl;
        ctl->active_count = active;
        ctl->block_selected = running;
        ctl->clipped = clipped;
        ctl->pop_cutoff = pop_cutoff;
        ctl->ring_tick[rs] = tick;
        ctl->ring_count[rs] = active;
        float activity = static_cast<float>(active) / static_cast<float>(N);
        float err = activity - cfg.target_activity;
        ctl->population_inhibition =
            clampf(ctl->population_inhibition + cfg.population_inhibition_rate * err, 0.0f, cfg.population_inhibition_max);
    }
}

// ---------------------------------------------------------------------------
// Phase 4 (rest of the lane): forward eligibilities (runtime.rs:805-918).
// Kept slots are compacted into the other list; dropped slots are unmarked.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool update_slot(const StepCtx& c, float* planes, uint64_t plane, uint32_t* last,
                                            uint32_t slot, uint32_t dst, uint8_t br) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = *c.d;
    const uint32_t tick = c.tick;
    float bs = planes[slot], ms = planes[plane + slot], fs = planes[2 * plane + slot];
    float as0 = planes[3 * plane + slot], as1 = planes[4 * plane + slot], as2 = planes[5 * plane + slot];
    float e = planes[6 * plane + slot];
    uint32_t el = tick - last[slot];
    if (el > 0) {
        bs *= decay_for_elapsed(cfg.branch_decay, el);
        ms *= decay_for_elapsed(cfg.membrane_decay, el);
        fs *= decay_for_elapsed(cfg.fatigue_decay, el);
        as0 *= decay_for_elapsed(cfg.adaptation_fast_decay, el);
        as1 *= decay_for_elapsed(cfg.adaptation_medium_decay, el);
        as2 *= decay_for_elapsed(cfg.adaptation_slow_decay, el);
        last[slot] = tick;
    }
    const bool touched = d.touched_epoch[dst] == tick + 1;
    float elig;
    if (!touched || d.refractory_until[dst] > tick) {
        elig = e * cfg.eligibility_decay;
    } else {
        float jac = branch_jacobian(br, c.a->m.excitability[dst], d.branches[4 * dst + BR_TEMP], d.branches[4 * dst + BR_GATE]);
        float sur = d.surrogate[dst];
        float asum = as0 + as1 + as2;
        ms = ms + jac * bs - fs - asum;
        elig = sur * ms;
    }
    if (touched && d.selected_epoch[dst] == tick + 1) {
        fs += cfg.fatigue_gain * elig;
        as0 += cfg.adaptation_fast_gain * elig;
        as1 += cfg.adaptation_medium_gain * elig;
        as2 += cfg.adaptation_slow_gain * elig;
    }
    planes[slot] = bs;
    planes[plane + slot] = ms;
    planes[2 * plane + slot] = fs;
    planes[3 * plane + slot] = as0;
    planes[4 * plane + slot] = as1;
    planes[5 * plane + slot] = as2;
    planes[6 * plane + slot] = elig;
    float mag = maxnum(maxnum(maxnum(fabsf(bs), fabsf(ms)), fabsf(fs)), fabsf(elig));
    mag = maxnum(mag, fabsf(as0));
    mag = maxnum(mag, fabsf(as1));
    mag = maxnum(mag, fabsf(as2));
    return mag > cfg.eligibility_epsilon;
}

__device__ void phase_eligibility(const StepCtx& c) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * cfg.synapses_per_neuron;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint32_t p = c.parity, q = c.parity ^ 1;
    const uint32_t rec_n = c.ctl->rec_count[p];
    if (c.part == 0 && threadIdx.x == 0) {
        c.ctl->tick_scan_rec[c.tick & 1] = rec_n;
        c.ctl->tick_scan_in[c.tick & 1] = c.ctl->in_count[p];
    }
    const uint32_t* rec_cur = d.rec_list + p * NS;
    uint32_t* rec_next = d.rec_list + q * NS;
    for (uint32_t i = c.gtid; i < rec_n; i += c.gstride) {
        uint32_t slot = rec_cur[i];
        if (update_slot(c, d.rec_trace, NS, d.rec_last, slot, a.m.rec_target[slot], a.m.rec_branch[slot])) {
            uint32_t pos = atomicAdd(&c.ctl->rec_count[q], 1u);
            rec_next[pos] = slot;
        } else {
            d.rec_mark[slot] = 0;
        }
    }
    const uint32_t in_n = c.ctl->in_count[p];
    const uint32_t* in_cur = d.in_list + p * NI;
    uint32_t* in_next = d.in_list + q * NI;
    for (uint32_t i = c.gtid; i < in_n; i += c.gstride) {
        uint32_t slot = in_cur[i];
        if (update_slot(c, d.in_trace, NI, d.in_last, slot, a.m.in_target[slot], a.m.in_branch[slot])) {
            uint32_t pos = atomicAdd(&c.ctl->in_count[q], 1u);
            in_next[pos] = slot;
        } else {
            d.in_mark[slot] = 0;
        }
    }
}

// ---------------------------------------------------------------------------
// Phase 5: post-activation dynamics (runtime.rs:920-938), emission snapshot
// (runtime.rs:1084-1106), and on one workgroup the readout, softmax and
// errors (runtime.rs:1108-1197, 1205-1206).
// ---------------------------------------------------------------------------
__device__ void readout(const StepCtx& c, const StepParams& sp, float* s_f, float* s_f2, uint32_t* s_u32, uint32_t step_index) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    LaneControl* ctl = c.ctl;
    const uint32_t cap = cfg.max_active_global, E = cfg.context_embedding_dim;
    const uint32_t rs = c.tick % kRing;
    const uint32_t A = ctl->active_count;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const uint32_t ctx_count = ctl->ctx_count;
    // context latent (runtime.rs:1120-1136)
    float* s_lat = s_f2;
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        float lat = 0.0f;
        for (uint32_t i = 0; i < ctx_count; ++i) {
            float scale = ctl->ctx_scales[i];
            if (scale <= 0.0f) continue;
            lat += d.p.ctx_emb[static_cast<uint64_t>(ctl->ctx_slots[i]) * E + e] * scale;
        }
        s_lat[e] = lat;
        d.ctx_latent[e] = lat;
    }
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) {
        float l = d.p.bias[o];
        for (uint32_t r = 0; r < A; ++r) l += d.p.out_w[static_cast<uint64_t>(act_list[r]) * kOutStride + o] * act_val[r];
        if (ctx_count > 0) {
            float contribution = 0.0f;
            for (uint32_t e = 0; e < E; ++e) contribution += d.p.ctx_out[o * E + e] * s_lat[e];
            l += contribution;
        }
        s_f[o] = l;
        d.logits[o] = l;
    }
    __syncthreads();
    // maximum (order-independent), exp, serial sum (runtime.rs:1169-1188)
    if (threadIdx.x == 0) {
        float mx = -INFINITY;
        for (uint32_t o = 0; o < kOutputs; ++o) mx = maxnum(mx, s_f[o]);
        s_f2[kThreads] = mx;
    }
    __syncthreads();
    const float mx = s_f2[kThreads];
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) s_f2[o] = glibc_expf_nonpositive(s_f[o] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (uint32_t o = 0; o < kOutputs; ++o) sum += s_f2[o];
        s_f[kOutStride] = sum;
    }
    __syncthreads();
    const float sum = s_f[kOutStride];
    const bool uniform = !finitef(sum) || sum <= 0.0f;
    for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) {
        float p = uniform ? 1.0f / static_cast<float>(kOutputs) : s_f2[o] / sum;
        s_f[o] = p;
        d.probs[o] = p;
        float err = p;
        if (static_cast<int32_t>(o) == sp.target_index) err = p - 1.0f;
        d.errors[o] = err;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t best = 0;
        for (uint32_t o = 1; o < kOutputs; ++o) {
            // total order on non-negative probabilities == bit order
            if (__float_as_uint(s_f[o]) > __float_as_uint(s_f[best])) best = o;
        }
        StepRecord& rec = d.records[step_index];
        rec.p_target = sp.target_index >= 0 ? s_f[sp.target_index] : 0.0f;
        rec.predicted = best;
    }
    __syncthreads();
}

__device__ void phase_post(const StepCtx& c, const StepParams& sp, uint32_t step_index, float* s_f, float* s_f2,
                           uint32_t* s_u32) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t S = cfg.synapses_per_neuron, cap = cfg.max_active_global;
    const uint32_t rs = c.tick % kRing;
    const uint32_t A = c.ctl->active_count;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const uint32_t total = A + A * S;
    const uint32_t N = cfg.neuron_count;
    const uint32_t refractory = c.tick + cfg.refractory_ticks + 1;
    uint32_t inhibitory = 0;
    for (uint32_t item = c.gtid; item < total; item += c.gstride) {
        if (item < A) {
            uint32_t n = act_list[item];
            inhibitory += a.m.neuron_type[n] != 0 ? 1u : 0u;
            float act = d.activation[n];
            d.fatigue[n] += cfg.fatigue_gain * act;
            d.adapt[n] += cfg.adaptation_fast_gain * act;
            d.adapt[N + n] += cfg.adaptation_medium_gain * act;
            d.adapt[2 * N + n] += cfg.adaptation_slow_gain * act;
            d.membrane[n] -= d.p.threshold[n] * cfg.membrane_reset_fraction;
            d.refractory_until[n] = refractory;
        } else {
            uint32_t local = item - A;
            uint32_t r = local / S, j = local % S;
            uint64_t rb = static_cast<uint64_t>(rs) * cap + r;
            d.ring_value[rb * S + j] = act_val[r] * d.p.rec_weight[static_cast<uint64_t>(act_list[r]) * S + j];
        }
    }
    add_count(&c.ctl->tick_ainh[c.tick & 1], inhibitory);
    const uint32_t readout_wg = c.P - 1;
    if ((sp.flags & kStepOutput) && c.part == readout_wg) readout(c, sp, s_f, s_f2, s_u32, step_index);
    if (c.part == readout_wg && threadIdx.x == 0) {
        StepRecord& rec = d.records[step_index];
        if (!(sp.flags & kStepOutput)) {
            rec.p_target = 0.0f;
            rec.predicted = 0;
        }
        LaneControl* ctl = c.ctl;
        rec.population_inhibition = ctl->population_inhibition;
        rec.active = A;
        rec.suprathreshold = ctl->tick_supra[c.tick & 1];
        rec.block_selected = ctl->block_selected;
        rec.clipped = ctl->clipped;
        rec.context_cells = ctl->ctx_count;
        rec.context_probes = ctl->ctx_probes;
        rec.context_applied = ctl->ctx_applied;
        rec.eligible_rec = ctl->rec_count[c.parity];
        rec.eligible_in = ctl->in_count[c.parity];
        rec.error_code = 0;
    }
}

// ---------------------------------------------------------------------------
// Phase 6: learning destinations and signals (runtime.rs:1214-1263).
// ---------------------------------------------------------------------------
__device__ void phase_signals(const StepCtx& c, float* s_err) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * cfg.synapses_per_neuron;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) s_err[o] = d.errors[o];
    __syncthreads();
    const uint32_t rec_n = c.ctl->rec_count[c.parity], in_n = c.ctl->in_count[c.parity];
    const uint32_t A = c.ctl->active_count;
    const uint32_t rs = c.tick % kRing;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cfg.max_active_global;
    const uint32_t* rec_cur = d.rec_list + c.parity * NS;
    const uint32_t* in_cur = d.in_list + c.parity * NI;
    const uint32_t total = rec_n + in_n + A;
    uint32_t claimed = 0;
    for (uint32_t item = c.gtid; item < total; item += c.gstride) {
        uint32_t dst;
        if (item < rec_n) dst = a.m.rec_target[rec_cur[item]];
        else if (item < rec_n + in_n) dst = a.m.in_target[in_cur[item - rec_n]];
        else dst = act_list[item - rec_n - in_n];
        if (atomicExch(&d.dest_epoch[dst], c.dest_epoch) == c.dest_epoch) continue;
        claimed += 1;
        const float* row = d.p.out_w + static_cast<uint64_t>(dst) * kOutStride;
        float signal = 0.0f;
        for (uint32_t o = 0; o < kOutputs; ++o) signal += row[o] * s_err[o];
        d.learning_signal[dst] = signal;
    }
    add_count(&c.ctl->tick_dest[c.tick & 1], claimed);
}

// ---------------------------------------------------------------------------
// Phase 7: output/bias/context updates (runtime.rs:1265-1303, 1318-1384),
// recurrent and input synapses (runtime.rs:1451-1523), inhibitory
// homeostasis (runtime.rs:1525-1565) and threshold homeostasis
// (runtime.rs:1567-1593).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float inhibitory_step(const LeoConfig& cfg, float w, float src_act, float tgt_act, float strength) {
    float err = tgt_act - cfg.target_activity;
    float delta = bounded(-cfg.inhibitory_learning_rate * strength * src_act * err, cfg.max_update);
    return clampf(w + delta, cfg.weight_min, 0.0f);
}

__device__ void context_update(const StepCtx& c, const StepParams& sp, float* s_err, float* s_grad) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = *c.d;
    LaneControl* ctl = c.ctl;
    const uint32_t E = cfg.context_embedding_dim, count = ctl->ctx_count;
    const float lr = cfg.context_learning_rate, mu = cfg.max_update, wmin = cfg.weight_min, wmax = cfg.weight_max;
    const float strength = sp.supervised_strength;
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        float g = 0.0f;
        for (uint32_t o = 0; o < kOutputs; ++o) g += d.p.ctx_out[o * E + e] * s_err[o];
        s_grad[e] = g;
    }
    __syncthreads();
    if (threadIdx.x == 0) ctl->ctx_out_dirty = 1;
    for (uint32_t i = threadIdx.x; i < kOutputs * E; i += kThreads) {
        uint32_t o = i / E, e = i % E;
        float gradient = s_err[o] * d.ctx_latent[e];
        float delta = bounded(-lr * strength * gradient, mu);
        float updated = clampf(d.p.ctx_out[i] + delta, wmin, wmax);
        if (!finitef(updated)) set_error(ctl, kErrContextProjection);
        d.p.ctx_out[i] = updated;
    }
    for (uint32_t i = threadIdx.x; i < count * E; i += kThreads) {
        uint32_t k = i / E, e = i % E;
        uint64_t slot = ctl->ctx_slots[k];
        float gradient = ctl->ctx_scales[k] * s_grad[e];
        float delta = bounded(-lr * strength * gradient, mu);
        float updated = clampf(d.p.ctx_emb[slot * E + e] + delta, wmin, wmax);
        if (!finitef(updated)) set_error(ctl, kErrContextEmbedding);
        d.p.ctx_emb[slot * E + e] = updated;
    }
    for (uint32_t k = threadIdx.x; k < count; k += kThreads) {
        uint32_t slot = ctl->ctx_slots[k];
        mark_bit(d.ch_ctx, slot);
        uint32_t obs = d.p.ctx_obs[slot];
        d.p.ctx_obs[slot] = obs == 0xffffffffu ? obs : obs + 1;
    }
    __syncthreads();
}

__device__ void phase_learn(const StepCtx& c, const StepParams& sp, float* s_err, float* s_grad) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = *c.d;
    const LeoConfig& cfg = a.cfg;
    LaneControl* ctl = c.ctl;
    const uint32_t S = cfg.synapses_per_neuron, cap = cfg.max_active_global;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * S;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint32_t tick = c.tick;
    const bool learn = (sp.flags & kStepLearn) != 0;
    const bool plastic = learn && sp.plasticity_scale > 0.0f;
    const uint32_t A = ctl->active_count;
    const uint32_t rs = tick % kRing;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const float mu = cfg.max_update, wmin = cfg.weight_min, wmax = cfg.weight_max;
    if (learn) {
        for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) s_err[o] = d.errors[o];
        __syncthreads();
        const float ss = sp.supervised_strength;
        const float olr = cfg.output_learning_rate;
        // output rows of active neurons
        const uint32_t out_items = A * kOutputs;
        for (uint32_t item = c.gtid; item < out_items; item += c.gstride) {
            uint32_t r = item / kOutputs, o = item % kOutputs;
            uint32_t n = act_list[r];
            float act = act_val[r];
            if (o == 0) mark_bit(d.ch_out, n);
            float raw = -olr * ss * s_err[o] * act;
            float* w = d.p.out_w + static_cast<uint64_t>(n) * kOutStride + o;
            *w = clampf(*w + bounded(raw, mu), wmin, wmax);
        }
        // bias and context projection on the readout workgroup
        if (c.part == c.P - 1) {
            for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) {
                float raw = -olr * ss * s_err[o];
                float b = d.p.bias[o] + bounded(raw, mu);
                if (!finitef(b)) set_error(ctl, kErrBias);
                d.p.bias[o] = b;
            }
            if (threadIdx.x == 0) ctl->bias_dirty = 1;
            if (ctl->ctx_applied && ctl->ctx_count > 0) context_update(c, sp, s_err, s_grad);
        }
        if (plastic) {
            const float cs = ss * sp.plasticity_scale;
            const float lr = cfg.recurrent_learning_rate;
            const uint32_t rec_n = ctl->rec_count[c.parity];
            const uint32_t* rec_cur = d.rec_list + c.parity * NS;
            for (uint32_t i = c.gtid; i < rec_n; i += c.gstride) {
                uint32_t slot = rec_cur[i];
                uint32_t dst = a.m.rec_target[slot];
                uint32_t src = slot / S;
                float e = d.rec_trace[6 * NS + slot];
                float gradient = d.learning_signal[dst] * e;
                float delta = bounded(-lr * cs * gradient, mu);
                float old_w = d.p.rec_weight[slot];
                float nw = clampf(old_w + delta, wmin, wmax);
                const bool excitatory = a.m.neuron_type[src] == 0;
                nw = excitatory ? maxnum(nw, 0.0f) : fminf(nw, 0.0f);
                if (!finitef(nw)) set_error(ctl, kErrRecurrent);
                bool changed = nw != old_w;
                if (!excitatory && d.selected_epoch[src] == tick + 1) {
                    float tgt_act = d.activation[dst] > 0.0f ? 1.0f : 0.0f;
                    float nw2 = inhibitory_step(cfg, nw, d.activation[src], tgt_act, sp.strength);
                    if (!finitef(nw2)) set_error(ctl, kErrInhibitory);
                    changed = changed || nw2 != nw;
                    nw = nw2;
                }
                if (changed) mark_bit(d.ch_rec, slot);
                d.p.rec_weight[slot] = nw;
            }
            const uint32_t in_n = ctl->in_count[c.parity];
            const uint32_t* in_cur = d.in_list + c.parity * NI;
            for (uint32_t i = c.gtid; i < in_n; i += c.gstride) {
                uint32_t slot = in_cur[i];
                uint32_t dst = a.m.in_target[slot];
                float e = d.in_trace[6 * NI + slot];
                float gradient = d.learning_signal[dst] * e;
                float delta = bounded(-lr * cs * gradient, mu);
                float old_w = d.p.in_weight[slot];
                float nw = clampf(old_w + delta, 0.0f, wmax);
                if (!finitef(nw)) set_error(ctl, kErrInput);
                if (nw != old_w) mark_bit(d.ch_in, slot);
                d.p.in_weight[slot] = nw;
            }
        }
        // inhibitory homeostasis on the rows of active inhibitory sources not
        // already handled with their eligible slot above
        const uint32_t inh_items = A * S;
        for (uint32_t item = c.gtid; item < inh_items; item += c.gstride) {
            uint32_t r = item / S, j = item % S;
            uint32_t src = act_list[r];
            if (a.m.neuron_type[src] == 0) continue;
            uint64_t slot = static_cast<uint64_t>(src) * S + j;
            if (plastic && d.rec_mark[slot]) continue;
            uint32_t dst = a.m.rec_target[slot];
            float tgt_act = d.activation[dst] > 0.0f ? 1.0f : 0.0f;
            float old_w = d.p.rec_weight[slot];
            float nw = inhibitory_step(cfg, old_w, d.activation[src], tgt_act, sp.strength);
            if (!finitef(nw)) set_error(ctl, kErrInhibitory);
            if (nw != old_w) mark_bit(d.ch_rec, static_cast<uint32_t>(slot));
            d.p.rec_weight[slot] = nw;
        }
    }
    if (!(sp.flags & kStepFrozen)) {
        const float N = static_cast<float>(cfg.neuron_count);
        const float pop_err = static_cast<float>(A) / N - cfg.target_activity;
        const uint32_t touched = ctl->tick_touched[tick & 1];
        for (uint32_t i = c.gtid; i < touched; i += c.gstride) {
            uint32_t n = d.touched_list[i];
            float local = d.activation[n] > 0.0f ? 1.0f : 0.0f;
            float local_err = local - cfg.target_activity;
            float delta = cfg.threshold_homeostasis_rate * (local_err + pop_err);
            float old_t = d.p.threshold[n];
            float nt = clampf(old_t + delta, 0.05f, 2.0f);
            if (nt != old_t) mark_bit(d.ch_threshold, n);
            d.p.threshold[n] = nt;
        }
    }
}

// Phase profiler: workgroup 0 of each lane timestamps the end of its own work
// and the end of the barrier wait of every phase (wall_clock64, constant rate).
struct PhaseClock {
    unsigned long long last = 0;
    unsigned long long* out = nullptr;
    __device__ void start(unsigned long long* profile) {
        out = profile;
        last = wall_clock64();
    }
    __device__ void arrive(uint32_t phase, unsigned long long& arrived) {
        arrived = wall_clock64();
        out[phase] += arrived - last;
    }
    __device__ void release(uint32_t phase, unsigned long long arrived) {
        last = wall_clock64();
        out[kPhases + phase] += last - arrived;
    }
};

template <bool kProfile>
__device__ __forceinline__ bool phase_barrier(const StepCtx& c, uint32_t& target, uint32_t spin_limit,
                                              PhaseClock& clock, uint32_t phase) {
    unsigned long long arrived = 0;
    const bool timer = kProfile && c.part == 0 && threadIdx.x == 0;
    if (timer) clock.arrive(phase, arrived);
    bool ok = lane_barrier(c.ctl, c.P, target, spin_limit);
    if (timer) clock.release(phase, arrived);
    return ok;
}

template <bool kProfile>
__device__ void lane_steps(const KernelArgs& args) {
    __shared__ uint64_t s_keys[kMaxBlockNeurons];
    __shared__ float s_f[kOutStride + 4];
    __shared__ float s_f2[kOutStride + kThreads + 4];
    __shared__ uint32_t s_u32[kThreads];
    const uint32_t L = args.lane_count, P = args.wgs_per_lane;
    const uint32_t lane = blockIdx.x % L;
    StepCtx c;
    c.a = &args;
    c.d = &args.lanes[lane];
    c.ctl = c.d->ctl;
    c.part = blockIdx.x / L;
    c.P = P;
    c.gtid = c.part * kThreads + threadIdx.x;
    c.gstride = P * kThreads;
    c.tick = c.ctl->tick;
    c.parity = c.ctl->parity;
    c.dest_epoch = c.ctl->dest_epoch;
    uint32_t target = 0;
    const uint32_t steps = c.d->step_count;
    const bool redundant = args.redundant_global != 0;
    const uint32_t spin = args.spin_limit;
    PhaseClock clock;
    if (kProfile && c.part == 0 && threadIdx.x == 0) clock.start(c.d->phase_profile);
    bool ok = true;
    for (uint32_t s = 0; s < steps && ok; ++s) {
        const StepParams sp = c.d->steps[s];
        const bool trace = (sp.flags & kStepLearnTrace) != 0;
        phase_deliver(c, sp, s);
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 0))) break;
        phase_fold(c, sp);
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 1))) break;
        phase_select(c, s_keys, s_u32);
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 2))) break;
        if (redundant) {
            if (c.part == 0) build_active(c, s_keys, s_u32);
            if (trace) phase_eligibility(c);
        } else {
            if (c.part == 0) build_active(c, s_keys, s_u32);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 7))) break;
            const uint32_t touched = c.ctl->tick_touched[c.tick & 1];
            const uint32_t nb = args.cfg.neurons_per_block;
            for (uint32_t i = c.gtid; i < touched; i += c.gstride) {
                uint32_t n = c.d->touched_list[i];
                surrogate_for(c, n, c.d->block_cutoff[n / nb], c.ctl->pop_cutoff);
            }
            if (trace) {
                if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 7))) break;
                phase_eligibility(c);
            }
        }
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 3))) break;
        if (trace) c.parity ^= 1;
        phase_post(c, sp, s, s_f, s_f2, s_u32);
        const bool learn = (sp.flags & kStepLearn) != 0;
        if (learn || !(sp.flags & kStepFrozen)) {
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 4))) break;
            if (learn && sp.plasticity_scale > 0.0f) {
                c.dest_epoch += 1;
                phase_signals(c, s_f);
                if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 5))) break;
            }
            phase_learn(c, sp, s_f, s_f2);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 6))) break;
        } else {
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 4))) break;
        }
        c.tick += 1;
    }
    if (ok && c.part == 0 && threadIdx.x == 0) {
        if (steps > 0) finalize_record(*c.d, c.ctl, steps - 1, c.tick - 1);
        c.ctl->tick = c.tick;
        c.ctl->parity = c.parity;
        c.ctl->dest_epoch = c.dest_epoch;
    }
}

__global__ void __launch_bounds__(kThreads) leo_lane_steps(KernelArgs args) { lane_steps<false>(args); }
__global__ void __launch_bounds__(kThreads) leo_lane_steps_profiled(KernelArgs args) { lane_steps<true>(args); }

// ---------------------------------------------------------------------------
// reset_transient_state (runtime.rs:365-425) for every lane in args.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) leo_reset_lanes(KernelArgs args, uint32_t set_tick, uint32_t new_tick) {
    const LeoConfig& cfg = args.cfg;
    const uint32_t L = args.lane_count;
    const uint32_t lane = blockIdx.x % L;
    const uint32_t part = blockIdx.x / L, parts = gridDim.x / L;
    const LaneDesc& d = args.lanes[lane];
    const uint32_t tick = set_tick ? new_tick : d.ctl->tick;
    const uint64_t N = cfg.neuron_count, S = cfg.synapses_per_neuron;
    const uint64_t NS = N * S, NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint64_t t0 = static_cast<uint64_t>(part) * kThreads + threadIdx.x, ts = static_cast<uint64_t>(parts) * kThreads;
    for (uint64_t i = t0; i < N; i += ts) {
        d.membrane[i] = 0.0f;
        d.activation[i] = 0.0f;
        d.fatigue[i] = 0.0f;
        d.refractory_until[i] = 0;
        d.branches[4 * i] = 0.0f;
        d.branches[4 * i + 1] = 0.0f;
        d.branches[4 * i + 2] = 0.0f;
        d.branches[4 * i + 3] = 0.0f;
        d.adapt[i] = 0.0f;
        d.adapt[N + i] = 0.0f;
        d.adapt[2 * N + i] = 0.0f;
        d.last_tick[i] = tick;
        d.touched_epoch[i] = 0;
        d.selected_epoch[i] = 0;
        d.surrogate[i] = 0.0f;
        d.bucket_count[i] = 0;
    }
    for (uint64_t i = t0; i < 7 * NS; i += ts) d.rec_trace[i] = 0.0f;
    for (uint64_t i = t0; i < NS; i += ts) {
        d.rec_last[i] = tick;
        d.rec_mark[i] = 0;
    }
    for (uint64_t i = t0; i < 7 * NI; i += ts) d.in_trace[i] = 0.0f;
    for (uint64_t i = t0; i < NI; i += ts) {
        d.in_last[i] = tick;
        d.in_mark[i] = 0;
    }
    for (uint64_t i = t0; i < cfg.context_embedding_dim; i += ts) d.ctx_latent[i] = 0.0f;
    if (part == 0 && threadIdx.x == 0) {
        LaneControl* ctl = d.ctl;
        ctl->tick = tick;
        ctl->population_inhibition = 0.0f;
        ctl->parity = 0;
        ctl->rec_count[0] = ctl->rec_count[1] = 0;
        ctl->in_count[0] = ctl->in_count[1] = 0;
        ctl->history_len = 0;
        ctl->ctx_count = 0;
        ctl->ctx_probes = 0;
        ctl->ctx_applied = 0;
        ctl->block_selected = 0;
        ctl->clipped = 0;
        ctl->pop_cutoff = 0.0f;
        ctl->active_count = 0;
        ctl->error_code = 0;
        ctl->barrier = 0;
        ctl->abort = 0;
        for (uint32_t k = 0; k < kRing; ++k) {
            ctl->ring_tick[k] = 0xffffffffu;
            ctl->ring_count[k] = 0;
        }
        for (int k = 0; k < 2; ++k) {
            ctl->tick_touched[k] = ctl->tick_supra[k] = ctl->tick_events[k] = 0;
            ctl->tick_dest[k] = ctl->tick_ainh[k] = ctl->tick_scan_rec[k] = ctl->tick_scan_in[k] = 0;
        }
    }
}

// ---------------------------------------------------------------------------
// Batch-end mean of one fixed-parameter tensor over `lanes` story lanes
// (parallel.rs:975-1022 apply_sparse_scaled: canonical += f32(Σ_lanes f64(lane-base) / L),
// only where some lane changed it), then the projection of parallel.rs:1169-1246
// and the bound checks of parallel.rs:1248-1345.
// ---------------------------------------------------------------------------


__global__ void __launch_bounds__(kThreads) leo_merge_fixed(MergeArgs m) {
    unsigned long long local = 0;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < m.count;
         i += static_cast<uint64_t>(gridDim.x) * kThreads) {
        uint64_t at = m.row ? (i / m.row) * m.stride + (i % m.row) : i;
        const float base = m.canonical[at];
        double sum = 0.0;
        bool any = false;
        for (uint32_t l = 0; l < m.lane_count; ++l) {
            float delta = m.lanes[l][at] - base;
            if (delta != 0.0f) {
                any = true;
                if (!finitef(delta)) atomicCAS(m.error, 0u, 1u);
                sum += static_cast<double>(delta);
            }
        }
        if (!any) continue;
        float v = base + static_cast<float>(sum / static_cast<double>(m.lane_count));
        if (!finitef(v)) atomicCAS(m.error, 0u, 2u);
        switch (m.kind) {
            case kMergeThreshold: v = clampf(v, 0.05f, 2.0f); break;
            case kMergeRecurrent:
                v = clampf(v, m.weight_min, m.weight_max);
                v = m.neuron_type[i / m.synapses_per_neuron] == 0 ? maxnum(v, 0.0f) : fminf(v, 0.0f);
                break;
            case kMergeInput: v = clampf(v, 0.0f, m.weight_max); break;
            case kMergeOutput:
            case kMergeContextOut: v = clampf(v, m.weight_min, m.weight_max); break;
            default: break;
        }
        if (!finitef(v)) atomicCAS(m.error, 0u, 3u);
        m.canonical[at] = v;
        local += 1;
    }
    if (local) atomicAdd(m.updates, local);
}

}  // namespace leo
