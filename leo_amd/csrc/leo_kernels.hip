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

#include <type_traits>

#include "glibc_expf.h"
#define LEO_KERNEL_TRANSLATION_UNIT  // global-address-space descriptor pointers
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
// Rust's w.max(0.0) / w.min(0.0), the sign projections of runtime.rs:1475-1479
// and parallel.rs:1202-1206, as rustc lowers them on x86_64 (maxss/minss with
// the constant second operand, which wins on equal values and on NaN): -0.0
// and NaN project to +0.0.
__device__ __forceinline__ float max_zero(float v) { return v > 0.0f ? v : 0.0f; }
__device__ __forceinline__ float min_zero(float v) { return v < 0.0f ? v : 0.0f; }
// (a + b) mod n for a, b < n
__device__ __forceinline__ uint32_t add_mod(uint32_t a, uint32_t b, uint32_t n) {
    const uint32_t v = a + b;
    return v >= n ? v - n : v;
}
__device__ __forceinline__ bool finitef(float v) { return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u; }

// decay_for_elapsed (runtime.rs:78-85: 1 for 0 ticks, the base for 1, else
// Rust's f32::powi, i.e. compiler-rt's powisf2 square-and-multiply) of the six
// state decays (branch, membrane, fatigue, fast, medium and slow adaptation)
// for one elapsed count, in one loop over the exponent's bits: each base sees
// exactly powisf2's sequence of multiplications.
struct StateDecays {
    float branch, membrane, fatigue, fast, medium, slow;
};
__device__ __forceinline__ StateDecays state_decays(const LeoConfig& cfg, uint32_t elapsed) {
    float a0 = cfg.branch_decay, a1 = cfg.membrane_decay, a2 = cfg.fatigue_decay;
    float a3 = cfg.adaptation_fast_decay, a4 = cfg.adaptation_medium_decay, a5 = cfg.adaptation_slow_decay;
    if (elapsed == 0) return {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
    if (elapsed == 1) return {a0, a1, a2, a3, a4, a5};
    float r0 = 1.0f, r1 = 1.0f, r2 = 1.0f, r3 = 1.0f, r4 = 1.0f, r5 = 1.0f;
    int b = static_cast<int>(elapsed > 0x7fffffffu ? 0x7fffffffu : elapsed);
    while (true) {
        if (b & 1) {
            r0 *= a0;
            r1 *= a1;
            r2 *= a2;
            r3 *= a3;
            r4 *= a4;
            r5 *= a5;
        }
        b /= 2;
        if (b == 0) break;
        a0 *= a0;
        a1 *= a1;
        a2 *= a2;
        a3 *= a3;
        a4 *= a4;
        a5 *= a5;
    }
    return {r0, r1, r2, r3, r4, r5};
}
// The decays of elapsed counts below kDecayTable, computed by state_decays
// at each step-kernel launch into LDS (the same function, so the same
// values): a touched neuron's decay is then one table read instead of a loop
// over the count's bits. Larger counts take the loop.
constexpr uint32_t kDecayTable = 512;
__shared__ float decay_table[kDecayTable * 6];
__device__ __forceinline__ void fill_decay_table(const LeoConfig& cfg) {
    for (uint32_t e = threadIdx.x; e < kDecayTable; e += blockDim.x) {
        const StateDecays k = state_decays(cfg, e);
        float* t = &decay_table[e * 6];
        t[0] = k.branch;
        t[1] = k.membrane;
        t[2] = k.fatigue;
        t[3] = k.fast;
        t[4] = k.medium;
        t[5] = k.slow;
    }
}
__device__ __forceinline__ StateDecays decays_at(const LeoConfig& cfg, uint32_t elapsed) {
    if (elapsed >= kDecayTable) return state_decays(cfg, elapsed);
    const float* t = &decay_table[elapsed * 6];
    return {t[0], t[1], t[2], t[3], t[4], t[5]};
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
// A numerical guard of schedule step `step`: the first code set wins and
// records its step (the lane stops after that step).
__device__ __forceinline__ void set_step_error(LaneControl* ctl, uint32_t code, uint32_t step) {
    if (atomicCAS(&ctl->error_code, 0u, code) == 0u) ctl->error_step = step;
}
__device__ __forceinline__ void mark_bit(uint32_t* bits, uint32_t index) { atomicOr(&bits[index >> 5], 1u << (index & 31)); }

// Wave-aggregated append: one atomic per wave instead of one per lane. Must be
// reached by every active lane of the wave (wave-uniform control flow).
__device__ __forceinline__ uint32_t wave_append(uint32_t* counter, bool pred) {
    const unsigned long long mask = __ballot(pred);
    if (mask == 0) return 0;
    const uint32_t lane = __lane_id();
    const uint32_t leader = static_cast<uint32_t>(__ffsll(static_cast<long long>(mask)) - 1);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(counter, static_cast<uint32_t>(__popcll(mask)));
    base = __builtin_amdgcn_readlane(base, static_cast<int>(leader));
    return base + static_cast<uint32_t>(__popcll(mask & ((1ULL << lane) - 1ULL)));
}

// Inclusive prefix sum over the wave by DPP row shifts (within 16-lane rows)
// and row broadcasts (lane 15 into rows 1 and 3, lane 31 into rows 2 and 3):
// VALU data movement without an LDS round trip. Every lane must be active.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xf, true));
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    v += dpp_u32<0x111, 0xf>(v);  // row_shr:1
    v += dpp_u32<0x112, 0xf>(v);  // row_shr:2
    v += dpp_u32<0x114, 0xf>(v);  // row_shr:4
    v += dpp_u32<0x118, 0xf>(v);  // row_shr:8
    v += dpp_u32<0x142, 0xa>(v);  // row_bcast:15
    v += dpp_u32<0x143, 0xc>(v);  // row_bcast:31
    return v;
}
// Sum over the wave (every lane must be active), uniform.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    return __builtin_amdgcn_readlane(wave_incl_scan_u32(v), kWaveSize - 1);
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_xor(v, off);
        v = o < v ? o : v;
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_xor(v, off);
        v = o > v ? o : v;
    }
    return v;
}
// Index of the calling wave in its workgroup, known to the compiler as uniform
// (values derived from it live in scalar registers).
__device__ __forceinline__ uint32_t wave_index() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
}

// Orders LDS traffic between lanes of one wave (the wave executes in lockstep;
// this keeps the compiler from moving LDS accesses across the point).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Loads of lane state written by other workgroups of the lane. A relaxed
// agent-scope atomic load is a device-scope load (global_load ... sc1): it
// misses the CU's L1 and reads the L2, so it never returns a line another CU
// has since rewritten. Read-only topology uses plain loads.
template <class T>
__device__ __forceinline__ T ld(const T* p) {
    // lane state is device memory: the global address space avoids flat loads
    const auto g = (const __attribute__((address_space(1))) T*)(p);
    return __hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A word of neuron n's state record.
__device__ __forceinline__ float LEO_GLOBAL* nf(const LaneDesc& d, uint64_t n, uint32_t field) {
    return reinterpret_cast<float LEO_GLOBAL*>(d.neuron) + n * kNeuronWords + field;
}
__device__ __forceinline__ uint32_t LEO_GLOBAL* nu(const LaneDesc& d, uint64_t n, uint32_t field) {
    return d.neuron + n * kNeuronWords + field;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Coherent (device-scope, L1-bypassing) buffer loads of lane state written by
// other workgroups, 16 or 4 bytes at a time.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 16));
}
// Records of `stride` bytes through a buffer resource in index mode: the
// address is base + index * stride + offset, computed in 64 bits, and the
// range check counts records, so arrays of up to 2^32 records (beyond 4 GiB)
// are addressed with 32-bit indices. Device scope (sc1), like ld16.
__device__ f32x4 struct_buffer_load_b128(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v4f32");
__device__ float struct_buffer_load_b32(__amdgpu_buffer_rsrc_t rsrc, int vindex, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.f32");
__device__ __forceinline__ __amdgpu_buffer_rsrc_t record_rsrc(const void* base, uint32_t stride, uint32_t records) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(stride), static_cast<int>(records),
                                             0x00020000);
}
__device__ __forceinline__ f32x4 ld16_record(__amdgpu_buffer_rsrc_t r, uint32_t index, uint32_t byte_offset) {
    return struct_buffer_load_b128(r, static_cast<int>(index), static_cast<int>(byte_offset), 0, 16);
}
__device__ __forceinline__ float ld4_record(__amdgpu_buffer_rsrc_t r, uint32_t index, uint32_t byte_offset) {
    return struct_buffer_load_b32(r, static_cast<int>(index), static_cast<int>(byte_offset), 0, 16);
}
__device__ __forceinline__ float ld4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, 16));
}

// The four 16-byte quarters of neuron n's record (the host limits N * 64
// bytes to below 2^31).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t neuron_rsrc(const LaneDesc& d, uint32_t neurons) {
    return coherent_rsrc(d.neuron, neurons * kNeuronWords * 4);
}
__device__ __forceinline__ f32x4 ld_quarter(__amdgpu_buffer_rsrc_t r, uint32_t n, uint32_t quarter) {
    return ld16(r, n * (kNeuronWords * 4) + quarter * 16);
}

// XCD (accelerator complex die) this wave runs on.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    return v;
}

// Barrier of the P workgroups of one lane; false when the lane aborted
// (another workgroup's wait timed out or the host's spin limit ran out).
// Workgroups on one XCD (`local`) share its L2: each stores its arrival word
// to its own 128-byte line, and the first wave polls the P lines, one lane
// per line, so that arrivals and polls spread over the L2 channels (a shared
// counter queues every arrival atomic and every poll on one channel:
// measured, a frozen step at 32 workgroups took 10% longer). A lane spread
// over several XCDs counts arrivals with a device-scope atomic counter
// between release and acquire fences.
//
// An arrival word is (epoch << 16) | carry, where epoch is the barrier's
// number modulo 2^16 and carry the sum of `carries` (LDS, one value per wave,
// 16 bits in all). Each workgroup has two words, used by the epoch's parity:
// a workgroup can be at most one barrier ahead of a poller (it passes a
// barrier only once every workgroup has arrived), so the word of the polled
// parity holds the polled epoch or the one two before it, and the carry read
// with the epoch is that barrier's. With `sums` (LDS, 1 + kWavesPerGroup
// words, read after the barrier), the polling wave writes the sum of every
// workgroup's carry to sums[0] and, for wave k of this workgroup, the sum of
// the carries before it in lane order (the workgroups before this one, then
// this one's waves before k) to sums[1 + k].
//
// Visibility. With `local` (all workgroups of the lane verified to run on one
// XCD, and every cross-workgroup read done with ld()), waiting until this
// workgroup's stores have completed to L2 is the whole release and nothing
// needs invalidating. Otherwise agent-scope fences write back and invalidate
// the L2 so other XCDs see the data. The wait is bounded: on timeout the lane
// is aborted, so every workgroup leaves the step loop and the grid drains.
__device__ __forceinline__ bool lane_barrier(const LaneDesc& d, uint32_t part, uint32_t P, uint32_t& target,
                                             uint32_t spin_limit, bool local, const uint32_t* carries = nullptr,
                                             uint32_t* sums = nullptr) {
    __shared__ uint32_t s_abort;
    LaneControl* ctl = d.ctl;
    LaunchWords LEO_GLOBAL* words = d.launch;
    if (P == 1) {
        __syncthreads();
        return true;
    }
    if (local) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        target += P;  // every thread keeps the count (the polling wave compares against it)
        const uint32_t epoch = __builtin_amdgcn_readfirstlane(target / P) & 0xffffu, parity = epoch & 1u;
        if (threadIdx.x < kWaveSize) {
            const uint32_t lane = threadIdx.x;
            uint32_t LEO_GLOBAL* flags = d.barrier_flags;
            uint32_t carry = 0;
            if (carries) {
#pragma unroll
                for (uint32_t k = 0; k < kWavesPerGroup; ++k) carry += carries[k];
            }
            if (lane == 0)
                __hip_atomic_store(&flags[part * kFlagWords + parity], (epoch << 16) | (carry & 0xffffu),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uint32_t spins = 0, aborted = 0;
            for (;;) {
                bool arrived = true;
                uint32_t all = 0, before = 0;
                for (uint32_t w = lane; w < P; w += kWaveSize) {
                    const uint32_t v = ld(&flags[w * kFlagWords + parity]);
                    arrived &= (v >> 16) == epoch;
                    all += v & 0xffffu;
                    before += w < part ? v & 0xffffu : 0u;
                }
                if (__all(arrived)) {
                    if (sums) {
                        all = wave_sum_u32(all);
                        before = wave_sum_u32(before);
                        if (lane == 0) {
                            sums[0] = all;
#pragma unroll
                            for (uint32_t k = 0; k < kWavesPerGroup; ++k) {
                                sums[1 + k] = before;
                                before += carries[k];
                            }
                        }
                    }
                    break;
                }
                if ((spins & 15) == 15 && ld(&words->abort) != 0) {
                    aborted = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (++spins > spin_limit) {
                    if (lane == 0) {
                        __hip_atomic_store(&words->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        set_error(ctl, kErrBarrier);
                    }
                    aborted = 1;
                    break;
                }
            }
            if (lane == 0) s_abort = aborted;
        }
        __syncthreads();
        return s_abort == 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    target += P;
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(&words->barrier, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        uint32_t aborted = 0;
        for (;;) {
            // one poll in flight per workgroup; the abort flag every 16th
            const uint32_t arrived = __hip_atomic_load(&words->barrier, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
            if (arrived >= target) break;
            if ((spins & 15) == 15 && ld(&words->abort) != 0) {
                aborted = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (++spins > spin_limit) {
                __hip_atomic_store(&words->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                set_error(ctl, kErrBarrier);
                aborted = 1;
                break;
            }
        }
        s_abort = aborted;
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
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

// Window key of a neuron whose deep bucket the wave folds after the others
// (above every selection key, whose high word is at most 0xfffffffe).
constexpr uint64_t kDeepPending = ~1ULL;

// Selection key: ascending order == (activation desc, rotated tie key asc)
// (runtime.rs:987-1009); activation > 0 so its bit pattern is monotone.
__device__ __forceinline__ uint64_t selection_key(float act, uint32_t tie) {
    return (static_cast<uint64_t>(~__float_as_uint(act)) << 32) | tie;
}
__device__ __forceinline__ float key_activation(uint64_t key) { return __uint_as_float(~static_cast<uint32_t>(key >> 32)); }

// Steps whose parameters one load round brings into LDS.
constexpr uint32_t kStepChunk = 64;

// Shared memory of the step kernel, reused phase by phase.
struct alignas(16) StepShared {
    float err[kOutStride];                                      // errors / logits
    float aux[kOutStride + kThreads];                           // exps, latent, gradient
    uint32_t queue[kWavesPerGroup][2 * kWaveSize];              // per-wave destination queue
    uint32_t scan[kThreads];
    unsigned long long red[kWavesPerGroup];
    float redf[kWavesPerGroup];
    // context resolution (one thread per order)
    uint32_t hist[kMaxOrder];
    int64_t ctx_slot[kMaxOrder];
    float ctx_scale[kMaxOrder];
    uint32_t ctx_probes[kMaxOrder];
    uint32_t hist_len;
    // this workgroup's copy of the emission ring bookkeeping (LaneControl ring_*)
    uint32_t ring_tick[kRing];
    uint32_t ring_count[kRing];
    uint32_t ring_early[kRing];
    // each selecting wave's winner count and first 64 winners (phase 2 to 3)
    uint32_t win_count[kWavesPerGroup];
    uint32_t tally[kWavesPerGroup][kTWaveWords];  // a tally launch's per-wave totals
    unsigned long long tally_rec[4];               // and the recording wave's (active, cells, kept)
    uint32_t win_n[kWavesPerGroup][kWaveSize];
    float win_act[kWavesPerGroup][kWaveSize];
    // the winner totals a one-barrier step's barrier carries: every wave's,
    // and those of the workgroups before this one (lane_barrier)
    uint32_t lane_sums[1 + kWavesPerGroup];
    // the step parameters of kStepChunk + 1 steps from a multiple of
    // kStepChunk on (the last one is the next chunk's first)
    uint32_t step_chunk[(kStepChunk + 1) * (sizeof(StepParams) / 4)];
};

// Dynamic LDS (step_lds_bytes): one phase-2 window per wave (Window below);
// the binding-cap global sort reuses the front.
extern __shared__ __align__(16) unsigned char step_lds[];

struct StepCtx {
    const KernelArgs* a;
    LaneDesc d;
    LaneControl LEO_GLOBAL* ctl;
    uint32_t tick;
    uint32_t part;     // workgroup index within the lane group
    uint32_t P;
    uint32_t gtid;
    uint32_t gstride;
    uint32_t parity;   // current eligible list
    uint32_t dest_epoch;
    bool local;        // workgroups of the lane share one L2 (see lane_barrier)
    bool carried;      // a one-barrier step's barrier carries the waves' winner totals
    uint32_t* tally;   // a tally launch: this wave's totals in LDS (kTally* words); else null
};

// This thread's item index when a phase's items are dealt 64 at a time to the
// first `parts` workgroups of the lane in turn (chunk wave * parts + part)
// rather than by thread id: a list shorter than the threads then spreads its
// memory traffic over every workgroup's CU instead of the first few, whose
// stores would drain before their barrier arrivals.
__device__ __forceinline__ uint32_t dealt_index(const StepCtx& c, uint32_t parts) {
    return (wave_index() * parts + c.part) * kWaveSize + __lane_id();
}

// Waves that own selection blocks: with several workgroups per lane the last
// one owns none (it resolves the context and takes deliveries instead).
__device__ __forceinline__ uint32_t selecting_waves(const StepCtx& c) {
    return (c.P > 1 ? c.P - 1 : 1) * kWavesPerGroup;
}

// ---------------------------------------------------------------------------
// Phase 1: start_tick (runtime.rs:537-561), event delivery scatter
// (runtime.rs:605-625) and injection (runtime.rs:627-639). Trace activation
// (runtime.rs:710-766) is slot-local; branch adds go to per-target buckets
// keyed by CPU delivery order and are folded in phase 2.
// ---------------------------------------------------------------------------
// Coherent loads of a trace record's two quarters (the host limits the trace
// arrays to below 2^32 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t trace_rsrc(const float LEO_GLOBAL* trace, uint64_t slots) {
    return record_rsrc(trace, kTraceWords * 4, static_cast<uint32_t>(slots));
}

// Brings one trace slot to `tick` and adds `activation` to its branch
// sensitivity (runtime.rs:710-766).
// With the slot's two record quarters already loaded (q0, q1).
__device__ __forceinline__ void activate_loaded_trace(float LEO_GLOBAL* trace, uint32_t slot, uint32_t tick,
                                                      float activation, const LeoConfig& cfg, f32x4 q0, f32x4 q1) {
    static_assert(kTBranch == 0 && kTAdapt0 == 3 && kTEligibility == 6 && kTLast == 7, "trace layout");
    f32x4 LEO_GLOBAL* rec = reinterpret_cast<f32x4 LEO_GLOBAL*>(trace + static_cast<uint64_t>(slot) * kTraceWords);
    const uint32_t e = tick - __float_as_uint(q1.w);
    if (e == 0) {
        trace[static_cast<uint64_t>(slot) * kTraceWords + kTBranch] = q0.x + activation;
        return;
    }
    const StateDecays k = decays_at(cfg, e);
    const float bs = q0.x * k.branch;
    rec[0] = f32x4{bs + activation, q0.y * k.membrane, q0.z * k.fatigue, q0.w * k.fast};
    rec[1] = f32x4{q1.x * k.medium, q1.y * k.slow, q1.z, __uint_as_float(tick)};
}

// Late fields of a step record: work counters complete only after the step's
// last barrier, so the record is finished by the next step (or kernel end).
struct LateCounters {
    uint32_t events, touched, scanned_rec, scanned_in, destinations, inhibitory, learning, deep;
};

__device__ __forceinline__ uint32_t LEO_GLOBAL* counter_word(const StepCtx& c, uint32_t part, uint32_t kind,
                                                          uint32_t tick) {
    return c.d.wg_counts + part * kFlagWords + 2 * kind + (tick & 1);
}

// Adds a wave's count to its workgroup's counter (every lane of the wave calls).
__device__ __forceinline__ void count_wave(const StepCtx& c, uint32_t kind, uint32_t tick, uint32_t local) {
    const uint32_t total = wave_sum_u32(local);
    if (__lane_id() == 0 && total) {
        if (c.tally) {
            if (kind == kCInhibitory) c.tally[kTInhibitory] += total;
        } else {
            atomicAdd(counter_word(c, c.part, kind, tick), total);
        }
    }
}

// One counter of `tick` summed over the lane's workgroups by a whole wave, uniform.
__device__ __forceinline__ uint32_t counter_total(const StepCtx& c, uint32_t kind, uint32_t tick) {
    uint32_t v = 0;
    for (uint32_t w = __lane_id(); w < c.P; w += kWaveSize) v += ld(counter_word(c, w, kind, tick));
    return wave_sum_u32(v);
}

// The late counters of `tick` by a whole wave (all loads in one round), uniform.
__device__ __forceinline__ LateCounters load_late_counters(const StepCtx& c, uint32_t tick) {
    uint32_t v[kCounterKinds];
#pragma unroll
    for (uint32_t k = 0; k < kCounterKinds; ++k) v[k] = 0;
    for (uint32_t w = __lane_id(); w < c.P; w += kWaveSize) {
#pragma unroll
        for (uint32_t k = 0; k < kCounterKinds; ++k) v[k] += ld(counter_word(c, w, k, tick));
    }
    LateCounters out;
    // the fold counted every entry it folded, the tick's F injections too
    const uint32_t folded = wave_sum_u32(v[kCEvents]), F = c.a->cfg.input_fanout;
    out.events = folded > F ? folded - F : 0u;
    out.touched = wave_sum_u32(v[kCTouched]);
    out.scanned_rec = wave_sum_u32(v[kCScanRec]);
    out.scanned_in = wave_sum_u32(v[kCScanIn]);
    out.destinations = wave_sum_u32(v[kCDest]);
    out.inhibitory = wave_sum_u32(v[kCInhibitory]);
    out.learning = wave_sum_u32(v[kCLearn]);
    out.deep = wave_sum_u32(v[kCDeep]);
    return out;
}

__device__ __forceinline__ void store_late_record(const LaneDesc& d, uint32_t step_index, const LateCounters& v) {
    StepRecord LEO_GLOBAL& rec = d.records[step_index];
    rec.events = v.events;
    rec.touched = v.touched;
    rec.scanned_rec = v.scanned_rec;
    rec.scanned_in = v.scanned_in;
    rec.destinations = v.destinations;
    rec.active_inhibitory = v.inhibitory;
    rec.learning_slots = v.learning;
    rec.deep_folds = v.deep;
}

// By a whole wave: all loads first (one round trip), then the stores.
__device__ __forceinline__ void finalize_record(const StepCtx& c, uint32_t step_index, uint32_t tick) {
    const LateCounters v = load_late_counters(c, tick);
    if (__lane_id() == 0) store_late_record(c.d, step_index, v);
}

// Clears the per-tick counters that tick+1 reuses, by a whole wave (after its
// loads of tick-1's counters, which share the words).
__device__ __forceinline__ void clear_counters(const StepCtx& c, uint32_t tick) {
    for (uint32_t w = __lane_id(); w < c.P; w += kWaveSize) {
#pragma unroll
        for (uint32_t k = 0; k < kCounterKinds; ++k) *counter_word(c, w, k, tick + 1) = 0u;
    }
}
// Once tick-1 is complete (by one wave): its record is finished and its
// per-tick counters, which tick+1 reuses, are cleared.
__device__ __forceinline__ void roll_counters(const StepCtx& c, uint32_t step_index) {
    if (step_index > 0) finalize_record(c, step_index - 1, c.tick - 1);
    clear_counters(c, c.tick);
}

// The selecting waves' winner totals of one tick: `all`, and `before` those of
// the waves below wv, by a whole wave (uniform). Up to 256 waves' totals are
// loaded in one round, and each lane's partial sums are reduced once.
__device__ __forceinline__ void sum_totals(const uint32_t LEO_GLOBAL* totals, uint32_t nwaves, uint32_t wv,
                                           uint32_t& all, uint32_t& before) {
    constexpr uint32_t kAtOnce = 4;
    const uint32_t lane = __lane_id();
    all = before = 0;
    for (uint32_t base = 0; base < nwaves; base += kAtOnce * kWaveSize) {
        uint32_t v[kAtOnce];
#pragma unroll
        for (uint32_t k = 0; k < kAtOnce; ++k) {
            const uint32_t w = base + k * kWaveSize + lane;
            v[k] = w < nwaves ? ld(&totals[w]) : 0u;
        }
        uint32_t a = 0, b = 0;
#pragma unroll
        for (uint32_t k = 0; k < kAtOnce; ++k) {
            a += v[k];
            b += base + k * kWaveSize + lane < wv ? v[k] : 0u;
        }
        all += wave_sum_u32(a);
        before += wave_sum_u32(b);
    }
}

// The bucket set of the deliveries of `tick` (LaneDesc::bucket_sets).
__device__ __forceinline__ uint32_t set_of(const LaneDesc& d, uint32_t tick) {
    return d.bucket_sets == 1 ? 0u : tick % kBucketSets;
}
__device__ __forceinline__ uint64_t LEO_GLOBAL* set_bucket(const LaneDesc& d, uint32_t set) {
    return d.bucket + set * d.bucket_stride;
}
__device__ __forceinline__ uint32_t LEO_GLOBAL* set_counts(const LaneDesc& d, uint32_t set, uint32_t N) {
    return d.bucket_count + static_cast<uint64_t>(set) * N;
}
__device__ __forceinline__ uint32_t LEO_GLOBAL* set_touched(const LaneDesc& d, uint32_t set) {
    return d.touched_bits + static_cast<uint64_t>(set) * d.touched_stride;
}
// This tick's per-wave winner totals (two buffers by tick parity).
__device__ __forceinline__ uint32_t LEO_GLOBAL* wave_totals(const LaneDesc& d, uint32_t tick) {
    return d.wave_total + (tick & 1u) * kMaxWaves;
}

// Entry p of target n's delivery bucket: the first kFixedEntries at fixed
// places (kFixedEntries*n + p), the rest in the target's overflow range.
__device__ __forceinline__ uint64_t bucket_entry(uint64_t overflow, uint32_t n, uint32_t p) {
    return p < kFixedEntries ? static_cast<uint64_t>(kFixedEntries) * n + p : overflow + (p - kFixedEntries);
}

// One delivery into target's bucket of `set` (the fold of phase 2 orders the
// bucket by key), in two parts so that a thread can claim several entries in
// one round: the claim of an entry (the counter increment) and its write.
// An entry past the target's fixed ones reads the target's overflow offset
// first (rare: the fixed entries hold nearly every target of a sparse tick).
// The write tells whether it is the target's first delivery of the tick.
struct EntryClaim {
    uint32_t p;
};
__device__ __forceinline__ EntryClaim claim_entry(const StepCtx& c, uint32_t set, uint32_t target) {
    EntryClaim k;
    k.p = atomicAdd(set_counts(c.d, set, c.a->cfg.neuron_count) + target, 1u);
    return k;
}
__device__ __forceinline__ bool write_entry(const StepCtx& c, uint32_t set, uint32_t target, const EntryClaim& k,
                                            uint64_t key, float value) {
    const uint64_t overflow = k.p < kFixedEntries ? 0 : c.a->m.bucket_offset[target];
    const uint64_t at = bucket_entry(overflow, target, k.p);
    uint64_t LEO_GLOBAL* bucket = set_bucket(c.d, set);
    // the 16-byte entry (key, value) in one store
    *reinterpret_cast<uint4 LEO_GLOBAL*>(bucket + 2 * at) =
        make_uint4(static_cast<uint32_t>(key), static_cast<uint32_t>(key >> 32), __float_as_uint(value), 0u);
    return k.p == 0;
}
__device__ __forceinline__ bool scatter_event(const StepCtx& c, uint32_t set, uint32_t target, uint64_t key,
                                              float value) {
    return write_entry(c, set, target, claim_entry(c, set, target), key, value);
}

// Touched mark of neuron n at `tick`: the block's bitmap bit in the tick's
// set, read by phase 2 (which writes the touched epoch when it folds n). A
// delivery marks its target only when it is the target's first of the tick
// (bucket count 0); setting a bit is idempotent, so a neuron also marked as
// previously active is marked twice harmlessly.
__device__ __forceinline__ void touch_neuron(const StepCtx& c, uint32_t n, uint32_t tick) {
    const uint32_t nb = c.a->cfg.neurons_per_block;
    const uint32_t blk = fast_div(n, c.a->div_block), off = n - blk * nb;
    atomicOr(&set_touched(c.d, set_of(c.d, tick))[blk * block_words(nb) + off / 32], 1u << (off & 31));
}

// The items of one tick's delivery: the previous active set, the ring
// snapshots of delay classes 8, 4, 2, 1 (all S synapses of each source,
// kept when the synapse's delay matches) and the symbol's F input edges.
// `ahead`: the next tick's delivery, run in the current tick's last phase
// (a frozen step after a fused one). The selecting waves handle the current
// tick's winners there (activation reset, touch, delay-1 events), so only
// delay classes 8, 4, 2 and the injection remain.
struct DeliverPlan {
    uint32_t tick, prev_slot, prev_count, off4, off2, off1, off_in, total;
    uint32_t rs8, rs4, rs2, rs1;
    uint32_t stride;  // items per round over the delivering workgroups
    bool delivers;    // this workgroup takes deliveries
};

__device__ __forceinline__ DeliverPlan deliver_plan(const StepCtx& c, const StepShared& sh, bool ahead) {
    const uint32_t S = c.a->cfg.synapses_per_neuron, F = c.a->cfg.input_fanout;
    DeliverPlan p;
    const uint32_t tick = p.tick = c.tick + (ahead ? 1u : 0u);
    // previous active set (runtime.rs:544-555)
    p.prev_slot = (tick + kRing - 1) % kRing;
    p.prev_count = (!ahead && tick > 0 && sh.ring_tick[p.prev_slot] == tick - 1) ? sh.ring_count[p.prev_slot] : 0;
    // delivery classes: delay 8, 4, 2, 1 in that order (chronological by emission tick)
    // (a class whose events the emitting tick delivered itself has none left)
    auto class_items = [&](uint32_t delay, uint32_t& rs) {
        rs = (tick + kRing - delay) % kRing;
        const bool valid = tick >= delay && sh.ring_tick[rs] == tick - delay && (sh.ring_early[rs] & delay) == 0;
        return (valid ? sh.ring_count[rs] : 0) * S;
    };
    p.rs1 = 0;
    p.off4 = p.prev_count + class_items(8, p.rs8);
    p.off2 = p.off4 + class_items(4, p.rs4);
    p.off1 = p.off2 + class_items(2, p.rs2);
    p.off_in = p.off1 + (ahead ? 0u : class_items(1, p.rs1));
    p.total = p.off_in + F;
    // with several workgroups the last one resolves the context meanwhile and
    // takes no deliveries, except ahead (the context then waits for phase 2)
    p.stride = (ahead || c.P == 1 ? c.P : c.P - 1) * kThreads;
    p.delivers = ahead || c.P == 1 || c.part < c.P - 1;
    return p;
}

// One delivery item of this thread, between its loads and its scatter.
struct DeliverItem {
    uint32_t touch_n, target;
    uint64_t key, rbase, slot;
    float value;
    uint32_t edge;
    uint32_t cls;      // delay class of a ring item (0..3 for delay 8, 4, 2, 1)
    bool ring, inj;
    // trace steps: a ring item's source and activation, an injection's trace
    // record quarters and list mark, loaded with the item
    uint32_t src;
    float act;
    f32x4 tq0, tq1;
    uint32_t mark;
};

// The item's loads (no dependent load: the emission snapshot holds the
// synapse with its value).
__device__ __forceinline__ DeliverItem deliver_fetch(const StepCtx& c, const StepParams& sp, const DeliverPlan& p,
                                                     uint32_t item) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const uint32_t S = a.cfg.synapses_per_neuron, F = a.cfg.input_fanout, cap = a.cfg.max_active_global;
    DeliverItem it;
    it.touch_n = 0xffffffffu;
    it.target = 0;
    it.key = it.rbase = it.slot = 0;
    it.value = 0.0f;
    it.edge = 0;
    it.cls = 0;
    it.ring = it.inj = false;
    it.src = 0;
    it.act = 0.0f;
    it.tq0 = it.tq1 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    it.mark = 0;
    const bool trace = (sp.flags & kStepLearnTrace) != 0;
    if (item < p.prev_count) {
        it.touch_n = ld(&d.ring_active[static_cast<uint64_t>(p.prev_slot) * cap + item]);
    } else if (item < p.off_in) {
        // the class's first item and ring slot as sums of masked steps: a
        // select among the plan's fields becomes a load from private memory
        const uint32_t c4 = item >= p.off4 ? 1u : 0u, c2 = item >= p.off2 ? 1u : 0u, c1 = item >= p.off1 ? 1u : 0u;
        const uint32_t k = c4 + c2 + c1;
        const uint32_t lo = p.prev_count + c4 * (p.off4 - p.prev_count) + c2 * (p.off2 - p.off4) + c1 * (p.off1 - p.off2);
        const uint32_t rsk = p.rs8 + c4 * (p.rs4 - p.rs8) + c2 * (p.rs2 - p.rs4) + c1 * (p.rs1 - p.rs2);
        const uint32_t local = item - lo;
        const uint32_t r = fast_div(local, a.div_synapses), j = local - r * S;
        it.rbase = static_cast<uint64_t>(rsk) * cap + r;
        it.edge = ld(&d.ring_edge[it.rbase * S + j]);
        it.value = ld(&d.ring_value[it.rbase * S + j]);
        it.cls = k;
        it.slot = j;  // completed with the source at the trace activation
        it.key = (static_cast<uint64_t>(k) << 61) | (static_cast<uint64_t>(r) << 32) | (static_cast<uint64_t>(j) << 2);
        it.ring = true;
        if (trace) {
            it.src = ld(&d.ring_active[it.rbase]);
            it.act = ld(&d.ring_act[it.rbase]);
        }
    } else if (item < p.total) {
        const uint32_t i = item - p.off_in;
        it.slot = static_cast<uint64_t>(sp.symbol) * F + i;
        const uint32_t edge = a.m.in_edge[it.slot];  // target and branch in one load
        it.target = edge_target(edge);
        it.key = (4ULL << 61) | (static_cast<uint64_t>(i) << 2) | edge_branch(edge);
        it.value = ld(&d.p.in_weight[it.slot]);
        it.inj = true;
        if (trace) {
            const uint64_t NI = static_cast<uint64_t>(kSymbols) * F;
            const __amdgpu_buffer_rsrc_t rsrc = trace_rsrc(d.in_trace, NI);
            it.tq0 = ld16_record(rsrc, static_cast<uint32_t>(it.slot), 0);
            it.tq1 = ld16_record(rsrc, static_cast<uint32_t>(it.slot), 16);
            it.mark = ld(&d.in_mark[it.slot]);
        }
    }
    return it;
}

// The item's scatter and touch, and for trace steps the trace activation of
// the delivering slot (runtime.rs:710-766) with its eligible-list append.
// Every lane of the wave calls (the appends are wave-aggregated).
__device__ __forceinline__ void deliver_commit(const StepCtx& c, const StepParams& sp, const DeliverPlan& p,
                                               DeliverItem& it, uint32_t& delivered) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    LaneControl* ctl = c.ctl;
    const uint32_t S = cfg.synapses_per_neuron;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * S;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const bool trace = (sp.flags & kStepLearnTrace) != 0;
    bool scatter = it.inj;
    if (it.ring) {
        it.ring = edge_delay(it.edge) == (8u >> it.cls);
        if (it.ring) {
            delivered += 1;
            it.target = edge_target(it.edge);
            it.key |= edge_branch(it.edge);
            scatter = true;
        }
    } else if (it.touch_n != 0xffffffffu) {
        (*nf(d, it.touch_n, kNActivation)) = 0.0f;
    }
    // a delivering recurrent slot's trace record and mark go out before the
    // bucket claim (in the same round)
    uint64_t rslot = 0;
    if (trace && it.ring) {
        rslot = it.slot + static_cast<uint64_t>(it.src) * S;
        const __amdgpu_buffer_rsrc_t rsrc = trace_rsrc(d.rec_trace, NS);
        it.tq0 = ld16_record(rsrc, static_cast<uint32_t>(rslot), 0);
        it.tq1 = ld16_record(rsrc, static_cast<uint32_t>(rslot), 16);
        it.mark = ld(&d.rec_mark[rslot]);
    }
    if (scatter && scatter_event(c, set_of(d, p.tick), it.target, it.key, it.value)) it.touch_n = it.target;
    if (it.touch_n != 0xffffffffu) touch_neuron(c, it.touch_n, p.tick);
    // frozen steps skip the appends below: their wave-uniform counter read
    // would wait for this item's stores before the next item's loads
    if (!trace) return;
    // the slot's list mark through one selected pointer (two stores into
    // different arrays would be merged through a private pointer table)
    const bool fresh = (it.ring || it.inj) && it.mark != kMarkListed;
    const uint32_t eslot = static_cast<uint32_t>(it.ring ? rslot : it.slot);
    if (it.ring) activate_loaded_trace(d.rec_trace, eslot, p.tick, it.act, cfg, it.tq0, it.tq1);
    else if (it.inj) activate_loaded_trace(d.in_trace, eslot, p.tick, 1.0f, cfg, it.tq0, it.tq1);
    uint8_t LEO_GLOBAL* mark = it.ring ? d.rec_mark + rslot : d.in_mark + it.slot;
    if (fresh) *mark = kMarkListed;
    const bool new_rec = fresh && it.ring, new_in = fresh && !it.ring;
    uint32_t pos = wave_append(&ctl->rec_count[c.parity], new_rec);
    if (new_rec) d.rec_list[static_cast<uint64_t>(c.parity) * NS + pos] = eslot;
    pos = wave_append(&ctl->in_count[c.parity], new_in);
    if (new_in) d.in_list[static_cast<uint64_t>(c.parity) * NI + pos] = eslot;
}

// Items from `first` on, one per thread per round.
__device__ __forceinline__ void deliver_items(const StepCtx& c, const StepParams& sp, const DeliverPlan& p,
                                              uint32_t first, uint32_t& delivered) {
    const uint32_t lane = __lane_id();
    for (uint32_t base = first - lane; p.delivers && base < p.total; base += p.stride) {
        DeliverItem it = deliver_fetch(c, sp, p, base + lane);
        deliver_commit(c, sp, p, it, delivered);
    }
}

// Reset of this step's next eligible lists (trace steps append to them).
__device__ __forceinline__ void reset_next_lists(const StepCtx& c) {
    if (c.part == 0 && threadIdx.x == 0) {
        c.ctl->rec_count[c.parity ^ 1] = 0;
        c.ctl->in_count[c.parity ^ 1] = 0;
    }
}

__device__ __forceinline__ void phase_deliver(const StepCtx& c, const StepParams& sp, const StepShared& sh) {
    reset_next_lists(c);
    const DeliverPlan p = deliver_plan(c, sh, false);
    uint32_t delivered = 0;  // counted by the fold instead (it folds every delivered entry)
    deliver_items(c, sp, p, dealt_index(c, p.stride / kThreads), delivered);
}

// ---------------------------------------------------------------------------
// Context resolution (runtime.rs:641-677, model.rs:173-221), one thread per
// order on the last workgroup during phase 1; phase 2 is the per-block fold,
// drive and top-k on one wave per block (runtime.rs:576-603, 701-708,
// 940-1011, 787-803).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void context_resolve(const StepCtx& c, const StepParams& sp, StepShared& sh) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = c.d;
    LaneControl* ctl = c.ctl;
    const uint32_t max_order = cfg.context_max_order, E = cfg.context_embedding_dim;
    const bool enabled = (sp.flags & kStepContext) != 0;
    const bool allocate = (sp.flags & kStepAllocate) != 0;
    // the history entries and its length are loaded in one round
    if (threadIdx.x < kMaxOrder) sh.hist[threadIdx.x] = ld(&ctl->history[threadIdx.x]);
    if (threadIdx.x == kMaxOrder) sh.hist_len = ld(&ctl->history_len);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t len = sh.hist_len;
        if (len == max_order) {
            for (uint32_t i = 1; i < len; ++i) sh.hist[i - 1] = sh.hist[i];
            len -= 1;
        }
        sh.hist[len++] = sp.symbol;
        sh.hist_len = len;
        for (uint32_t i = 0; i < len; ++i) ctl->history[i] = sh.hist[i];
        ctl->history_len = len;
    }
    __syncthreads();
    const uint32_t len = sh.hist_len;
    if (threadIdx.x < len && enabled) {
        const uint32_t order = threadIdx.x + 1;
        const uint64_t key = context_key(sh.hist, len, order);
        const uint64_t spo = cfg.context_slots_per_order;
        // slots per order is uniform; a power of two needs no 64-bit division
        const uint64_t base = static_cast<uint64_t>(order - 1) * spo;
        const uint64_t start = (spo & (spo - 1)) == 0 ? key & (spo - 1) : key % spo;
        // probe_limit <= slots_per_order (config.rs:457): one wrap at most
        auto probe_slot = [&](uint32_t off) {
            const uint64_t at = start + off;
            return base + (at >= spo ? at - spo : at);
        };
        int64_t found = -1, empty = -1;
        uint64_t weakest = base + start;
        uint32_t weakest_obs = 0xffffffffu, probes = 0, found_obs = 0;
        // the probe window is loaded at once when it is short
        constexpr uint32_t kWindow = 8;
        const uint32_t limit = cfg.context_probe_limit;
        uint64_t keys[kWindow];
        uint32_t obs_w[kWindow];
#pragma unroll
        for (uint32_t off = 0; off < kWindow; ++off) {
            const uint64_t slot = probe_slot(off);
            keys[off] = off < limit ? ld(&d.p.ctx_keys[slot]) : 0;
            obs_w[off] = off < limit ? ld(&d.p.ctx_obs[slot]) : 0;
        }
        bool done = false;
        for (uint32_t off = 0; !done && off < limit; ++off) {
            const uint64_t slot = probe_slot(off);
            uint64_t existing = 0;
            uint32_t obs = 0;
            if (off < kWindow) {
#pragma unroll
                for (uint32_t w = 0; w < kWindow; ++w)  // select from registers without indexing
                    if (w == off) {
                        existing = keys[w];
                        obs = obs_w[w];
                    }
            } else {
                existing = ld(&d.p.ctx_keys[slot]);
                obs = ld(&d.p.ctx_obs[slot]);
            }
            probes += 1;
            if (existing == key) {
                found = static_cast<int64_t>(slot);
                found_obs = obs;
                done = true;
            } else {
                if (existing == 0 && empty < 0) empty = static_cast<int64_t>(slot);
                if (obs < weakest_obs) {
                    weakest_obs = obs;
                    weakest = slot;
                }
            }
        }
        if (found < 0 && allocate) {
            const uint64_t slot = empty >= 0 ? static_cast<uint64_t>(empty) : weakest;
            d.p.ctx_keys[slot] = key;
            d.p.ctx_obs[slot] = 0;
            for (uint32_t e = 0; e < E; ++e) d.p.ctx_emb[slot * E + e] = 0.0f;
            found = static_cast<int64_t>(slot);
            found_obs = 0;
        }
        float scale = 0.0f;
        if (found >= 0) {
            const float obs = static_cast<float>(found_obs);
            const float confidence = obs / (obs + static_cast<float>(cfg.context_confidence_observations));
            scale = confidence * static_cast<float>(order);
        }
        sh.ctx_slot[threadIdx.x] = found;
        sh.ctx_scale[threadIdx.x] = scale;
        sh.ctx_probes[threadIdx.x] = probes;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t count = 0, probes = 0;
        float scale_sum = 0.0f;
        float scales[kMaxOrder];
        if (enabled) {
            for (uint32_t t = 0; t < len; ++t) {
                probes += sh.ctx_probes[t];
                if (sh.ctx_slot[t] < 0) continue;
                ctl->ctx_slots[count] = static_cast<uint32_t>(sh.ctx_slot[t]);
                scales[count] = sh.ctx_scale[t];
                scale_sum += sh.ctx_scale[t];
                count += 1;
            }
            for (uint32_t i = 0; i < count; ++i)
                ctl->ctx_scales[i] = scale_sum > 0.0f ? scales[i] / scale_sum : scales[i];
        }
        ctl->ctx_applied = enabled ? 1u : 0u;
        ctl->ctx_count = count;
        ctl->ctx_probes = probes;
    }
}

// Sorts n <= 8 (key, value) pairs ascending by key with a fixed network
// (entries n..7 hold ~0 keys and stay last).
__device__ __forceinline__ void sort8(uint64_t (&k)[8], uint32_t (&v)[8]) {
    auto cx = [&](int i, int j) {
        if (k[j] < k[i]) {
            const uint64_t tk = k[i];
            k[i] = k[j];
            k[j] = tk;
            const uint32_t tv = v[i];
            v[i] = v[j];
            v[j] = tv;
        }
    };
    cx(0, 2); cx(1, 3); cx(4, 6); cx(5, 7);
    cx(0, 4); cx(1, 5); cx(2, 6); cx(3, 7);
    cx(0, 1); cx(2, 3); cx(4, 5); cx(6, 7);
    cx(2, 4); cx(3, 5);
    cx(1, 4); cx(3, 6);
    cx(1, 2); cx(3, 4); cx(5, 6);
}

// Brings touched neuron n to the current tick (runtime.rs:576-603), folds its
// delivered values in CPU delivery order (runtime.rs:605-639, 701-708), and,
// unless refractory, applies the drive (runtime.rs:940-975). Returns the
// margin membrane - threshold; *refractory tells whether the neuron skipped.
// A neuron with more than 8 deliveries this tick is left untouched and
// *deferred set: the wave folds it with deep_fold. *entries is the bucket's
// entry count (its deliveries of the tick, folded here or by deep_fold).
//
// `post_pending`: the previous tick was a one-barrier frozen step, which
// left its winners' post-fire updates (runtime.rs:920-938, 1084-1106) and
// activation reset (runtime.rs:544-555) to this fold: a record whose
// activation is nonzero belongs to such a winner (an activation is nonzero
// only from a neuron's selection to the next tick's reset), and every
// winner is touched at the next tick. They are applied here before the
// decay, in the order and with the values the post phase would have used
// (the threshold does not change in a frozen step).
__device__ __forceinline__ void apply_post_fire(const LeoConfig& cfg, uint32_t fired_tick, float threshold,
                                                float& act, float& mem, float& fat, float& ad0, float& ad1,
                                                float& ad2, uint32_t& refractory_until) {
    fat = fat + cfg.fatigue_gain * act;
    ad0 = ad0 + cfg.adaptation_fast_gain * act;
    ad1 = ad1 + cfg.adaptation_medium_gain * act;
    ad2 = ad2 + cfg.adaptation_slow_gain * act;
    mem = mem - threshold * cfg.membrane_reset_fraction;
    refractory_until = fired_tick + cfg.refractory_ticks + 1;
    act = 0.0f;
}

__device__ __forceinline__ float fold_drive(const StepCtx& c, uint32_t n, float pi, uint32_t set, bool post_pending,
                                            bool* refractory, bool* deferred, uint32_t* entries) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, tick = c.tick;
    // the record in three 16-byte loads (membrane .. refractory tick)
    static_assert(kNMembrane == 0 && kNFatigue == 2 && kNAdapt0 == 3 && kNBranch0 == 6 && kNLastTick == 10 &&
                      kNRefractory == 11 && kNTouched == 12,
                  "record layout");
    const __amdgpu_buffer_rsrc_t rec = neuron_rsrc(d, N);
    const f32x4 q0 = ld_quarter(rec, n, 0), q1 = ld_quarter(rec, n, 1), q2 = ld_quarter(rec, n, 2);
    uint32_t LEO_GLOBAL* counts = set_counts(d, set, N);
    const uint64_t LEO_GLOBAL* bucket = set_bucket(d, set);
    float mem = q0.x, fat = q0.z, ad0 = q0.w, ad1 = q1.x, ad2 = q1.y;
    float b0 = q1.z, b1 = q1.w, b2 = q2.x, b3 = q2.y;
    const uint32_t last = __float_as_uint(q2.z);
    const uint32_t cnt = ld(&counts[n]);
    *entries = cnt;

    // the fixed bucket entries (one 64-byte run, 16 bytes each: key, value)
    // are read with the state; N * 64 bytes fits a buffer like the records
    static_assert(kFixedEntries == 4, "the fold reads four fixed entries");
    const __amdgpu_buffer_rsrc_t fixed = coherent_rsrc(bucket, N * kFixedEntries * 16);
    f32x4 fe[kFixedEntries];
#pragma unroll
    for (uint32_t x = 0; x < kFixedEntries; ++x) fe[x] = ld16(fixed, (n * kFixedEntries + x) * 16);
    auto entry_key = [](const f32x4& e) {
        return (static_cast<uint64_t>(__float_as_uint(e.y)) << 32) | __float_as_uint(e.x);
    };
    const uint64_t k0 = entry_key(fe[0]), k1 = entry_key(fe[1]);
    const uint32_t v0 = __float_as_uint(fe[0].z), v1 = __float_as_uint(fe[1].z);
    const float threshold = ld(&d.p.threshold[n]);
    const float excitability = a.m.excitability[n];  // in the same round, though a refractory neuron skips it
    *deferred = cnt > 8;
    if (cnt > 8) return 0.0f;  // every load above is in flight together; nothing written yet
    float act = q0.y;
    uint32_t refractory_until = __float_as_uint(q2.w);
    if (post_pending && act > 0.0f)
        apply_post_fire(cfg, tick - 1, threshold, act, mem, fat, ad0, ad1, ad2, refractory_until);
    const bool refr = refractory_until > tick;
    const uint32_t e = tick - last;
    if (e > 0) {
        const StateDecays k = decays_at(cfg, e);
        b0 *= k.branch;
        b1 *= k.branch;
        b2 *= k.branch;
        b3 *= k.branch;
        mem *= k.membrane;
        fat *= k.fatigue;
        ad0 *= k.fast;
        ad1 *= k.medium;
        ad2 *= k.slow;
    }
    if (cnt > 0) {
        // selects, not an indexed array (which would live in scratch)
        auto add = [&](uint64_t key, uint32_t bits) {
            const float v = __uint_as_float(bits);
            const uint32_t br = static_cast<uint32_t>(key) & 3u;
            b0 = br == 0 ? b0 + v : b0;
            b1 = br == 1 ? b1 + v : b1;
            b2 = br == 2 ? b2 + v : b2;
            b3 = br == 3 ? b3 + v : b3;
        };
        if (cnt == 1) {
            add(k0, v0);
        } else if (cnt == 2) {
            if (k1 < k0) {
                add(k1, v1);
                add(k0, v0);
            } else {
                add(k0, v0);
                add(k1, v1);
            }
        } else {
            uint64_t k[8];
            uint32_t v[8];
#pragma unroll
            for (uint32_t x = 0; x < kFixedEntries; ++x) {
                k[x] = x < cnt ? entry_key(fe[x]) : ~0ULL;
                v[x] = x < cnt ? __float_as_uint(fe[x].z) : 0u;
            }
            const uint64_t LEO_GLOBAL* over = bucket + 2 * a.m.bucket_offset[n];
#pragma unroll
            for (uint32_t x = kFixedEntries; x < 8; ++x) {
                k[x] = x < cnt ? ld(&over[2 * (x - kFixedEntries)]) : ~0ULL;
                v[x] = x < cnt ? static_cast<uint32_t>(ld(&over[2 * (x - kFixedEntries) + 1])) : 0u;
            }
            sort8(k, v);
#pragma unroll
            for (uint32_t x = 0; x < 8; ++x)
                if (x < cnt) add(k[x], v[x]);
        }
        counts[n] = 0;
    }
    *refractory = refr;
    if (!refr) {
        const float gate = clampf(b3, 0.0f, 1.0f);
        const float net = b0 + b2 * gate + b1;
        const float adaptation = ad0 + ad1 + ad2;
        const float drive = excitability * net - fat - adaptation - pi;
        mem = mem + drive;
    }
    // quarters 0-2 written whole (the wave owns the neuron during this
    // phase; the activation and refractory tick are written back unchanged)
    f32x4 LEO_GLOBAL* rq = reinterpret_cast<f32x4 LEO_GLOBAL*>(nf(d, n, 0));
    rq[0] = f32x4{mem, act, fat, ad0};
    rq[1] = f32x4{ad1, ad2, b0, b1};
    rq[2] = f32x4{b2, b3, __uint_as_float(e > 0 ? tick : last), __uint_as_float(refractory_until)};
    (*nu(d, n, kNTouched)) = tick + 1;
    return mem - threshold;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, uint32_t lane) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), static_cast<int>(lane));
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(v >> 32), static_cast<int>(lane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One entry (key, value bits) of a deep bucket in its current array: the
// target's bucket (entries by bucket_entry) or its shadow range.
struct DeepArray {
    uint64_t LEO_GLOBAL* base;
    uint64_t overflow;   // the bucket's overflow offset (bucket) or the shadow range's start (shadow)
    uint32_t n;
    bool bucket;
    __device__ __forceinline__ uint64_t at(uint32_t p) const {
        return bucket ? bucket_entry(overflow, n, p) : overflow + p;
    }
};

constexpr uint32_t kDeepTiles = 8;  // 64-entry tiles a lane has in flight

// fold_drive of a neuron with more than 8 deliveries, by the whole wave (all
// lanes active, n uniform): the bucket is sorted by delivery key -- ranked in
// registers up to kDeepRegisterEntries entries, else by an LSD radix sort
// between the bucket and the target's shadow range with the histogram in
// `hist` (256 words of LDS) -- and every lane adds the entries in that order
// (uniform values, so every lane holds the same sums). Lane 0 writes the
// state.
__device__ float deep_fold(const StepCtx& c, uint32_t n, float pi, uint32_t set, bool post_pending, bool* refractory,
                           uint32_t* hist) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, tick = c.tick, lane = __lane_id();
    const __amdgpu_buffer_rsrc_t rec = neuron_rsrc(d, N);
    const f32x4 q0 = ld_quarter(rec, n, 0), q1 = ld_quarter(rec, n, 1), q2 = ld_quarter(rec, n, 2);
    uint32_t LEO_GLOBAL* counts = set_counts(d, set, N);
    uint64_t LEO_GLOBAL* const set_base = set_bucket(d, set);
    const uint64_t overflow = a.m.bucket_offset[n];
    const float threshold = ld(&d.p.threshold[n]);
    float mem = q0.x, fat = q0.z, ad0 = q0.w, ad1 = q1.x, ad2 = q1.y;
    float b0 = q1.z, b1 = q1.w, b2 = q2.x, b3 = q2.y;
    // every lane read the same count: it is uniform
    const uint32_t last = __float_as_uint(q2.z), cnt = __builtin_amdgcn_readfirstlane(ld(&counts[n]));
    float act = q0.y;
    uint32_t refractory_until = __float_as_uint(q2.w);
    const bool fired = post_pending && act > 0.0f;
    if (fired) apply_post_fire(cfg, tick - 1, threshold, act, mem, fat, ad0, ad1, ad2, refractory_until);
    const bool refr = refractory_until > tick;
    const uint32_t e = tick - last;
    if (e > 0) {
        const StateDecays k = decays_at(cfg, e);
        b0 *= k.branch;
        b1 *= k.branch;
        b2 *= k.branch;
        b3 *= k.branch;
        mem *= k.membrane;
        fat *= k.fatigue;
        ad0 *= k.fast;
        ad1 *= k.medium;
        ad2 *= k.slow;
    }
    auto add = [&](uint32_t key_lo, uint32_t bits) {
        const float v = __uint_as_float(bits);
        const uint32_t br = key_lo & 3u;
        b0 = br == 0 ? b0 + v : b0;
        b1 = br == 1 ? b1 + v : b1;
        b2 = br == 2 ? b2 + v : b2;
        b3 = br == 3 ? b3 + v : b3;
    };
    DeepArray bucket{set_base, overflow, n, true};
    if (cnt <= kDeepRegisterEntries) {
        // two entries per lane; rank = number of smaller keys (keys unique)
        uint64_t k0 = ~0ULL, k1 = ~0ULL;
        uint32_t v0 = 0, v1 = 0;
        if (lane < cnt) {
            const uint64_t at = bucket.at(lane);
            k0 = ld(&set_base[2 * at]);
            v0 = static_cast<uint32_t>(ld(&set_base[2 * at + 1]));
        }
        if (lane + kWaveSize < cnt) {
            const uint64_t at = bucket.at(lane + kWaveSize);
            k1 = ld(&set_base[2 * at]);
            v1 = static_cast<uint32_t>(ld(&set_base[2 * at + 1]));
        }
        uint32_t r0 = 0, r1 = 0;
        for (uint32_t q = 0; q < cnt; ++q) {
            const uint64_t kq = readlane_u64(q < kWaveSize ? k0 : k1, q & (kWaveSize - 1));
            r0 += kq < k0 ? 1u : 0u;
            r1 += kq < k1 ? 1u : 0u;
        }
        for (uint32_t r = 0; r < cnt; ++r) {
            const uint64_t m0 = __ballot(lane < cnt && r0 == r);
            const uint64_t m1 = __ballot(lane + kWaveSize < cnt && r1 == r);
            const bool first = m0 != 0;
            const uint32_t src = static_cast<uint32_t>(__ffsll(static_cast<long long>(first ? m0 : m1)) - 1);
            const uint32_t key_lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(first ? k0 : k1), static_cast<int>(src));
            const uint32_t bits = __builtin_amdgcn_readlane(first ? v0 : v1, static_cast<int>(src));
            add(key_lo, bits);
        }
    } else {
        // LSD radix sort, 8-bit digits; each pass reads its source in order
        // (kDeepTiles tiles of 64 entries in flight per lane), counts the
        // next digit while scattering the current one stably
        const DeepSortPlan& plan = a.deep;
        const DeepArray shadow{d.shadow, a.m.shadow_offset[n], n, false};
        auto digit_of = [&](uint64_t key, uint32_t pass) {
            const uint64_t sk = deep_sort_key(key, plan.rank_bits, plan.slot_bits);
            return static_cast<uint32_t>(sk >> plan.shift[pass]) & ((1u << plan.bits[pass]) - 1u);
        };
        auto zero_hist = [&]() {
            for (uint32_t b = lane; b < 256; b += kWaveSize) hist[b] = 0u;
            wave_sync();
        };
        auto exclusive_scan_hist = [&]() {
            uint32_t h[4];
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) h[k] = hist[4 * lane + k];
            const uint32_t local = h[0] + h[1] + h[2] + h[3];
            uint32_t run = wave_incl_scan_u32(local) - local;
            wave_sync();
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                hist[4 * lane + k] = run;
                run += h[k];
            }
            wave_sync();
        };
        // counts of the first digit
        zero_hist();
        for (uint32_t t0 = 0; t0 < cnt; t0 += kDeepTiles * kWaveSize) {
            uint64_t keys[kDeepTiles];
#pragma unroll
            for (uint32_t k = 0; k < kDeepTiles; ++k) {
                const uint32_t p = t0 + k * kWaveSize + lane;
                keys[k] = p < cnt ? ld(&set_base[2 * bucket.at(p)]) : 0ULL;
            }
#pragma unroll
            for (uint32_t k = 0; k < kDeepTiles; ++k)
                if (t0 + k * kWaveSize + lane < cnt) atomicAdd(&hist[digit_of(keys[k], 0)], 1u);
        }
        wave_sync();
        for (uint32_t pass = 0; pass < plan.passes; ++pass) {
            // selects, not an indexed pair (which would live in scratch)
            const DeepArray src = (pass & 1) ? shadow : bucket;
            const DeepArray dst = (pass & 1) ? bucket : shadow;
            const bool more = pass + 1 < plan.passes;
            exclusive_scan_hist();
            // the next pass's counts go to the second half of the stage: the
            // scatter offsets stay in the first
            uint32_t* next = hist + 256;
            if (more) {
                for (uint32_t b = lane; b < 256; b += kWaveSize) next[b] = 0u;
                wave_sync();
            }
            const uint32_t bits = plan.bits[pass];
            const uint64_t below = (1ULL << lane) - 1ULL;
            for (uint32_t t0 = 0; t0 < cnt; t0 += kDeepTiles * kWaveSize) {
                uint64_t keys[kDeepTiles];
                uint32_t vals[kDeepTiles];
#pragma unroll
                for (uint32_t k = 0; k < kDeepTiles; ++k) {
                    const uint32_t p = t0 + k * kWaveSize + lane;
                    const uint64_t at = p < cnt ? src.at(p) : 0u;
                    keys[k] = p < cnt ? ld(&src.base[2 * at]) : 0ULL;
                    vals[k] = p < cnt ? static_cast<uint32_t>(ld(&src.base[2 * at + 1])) : 0u;
                }
#pragma unroll
                for (uint32_t k = 0; k < kDeepTiles; ++k) {
                    const bool tile = t0 + k * kWaveSize < cnt;  // uniform
                    const bool valid = t0 + k * kWaveSize + lane < cnt;
                    const uint32_t dig = valid ? digit_of(keys[k], pass) : 0u;
                    uint64_t peers = __ballot(valid);
                    for (uint32_t b = 0; b < bits; ++b) {
                        const bool bit = ((dig >> b) & 1u) != 0;
                        const uint64_t ones = __ballot(bit);
                        peers &= bit ? ones : ~ones;
                    }
                    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & below));
                    const uint32_t group = static_cast<uint32_t>(__popcll(peers));
                    const uint32_t pos = tile ? hist[dig] + rank : 0u;
                    wave_sync();
                    if (valid) {
                        const uint64_t at = dst.at(pos);
                        dst.base[2 * at] = keys[k];
                        dst.base[2 * at + 1] = vals[k];
                        if (rank + 1 == group) hist[dig] += group;
                        if (more) atomicAdd(&next[digit_of(keys[k], pass + 1)], 1u);
                    }
                    wave_sync();
                }
            }
            // the stores are complete before the next pass reads them
            __builtin_amdgcn_s_waitcnt(0);
            wave_sync();
            if (more) {
                for (uint32_t b = lane; b < 256; b += kWaveSize) hist[b] = next[b];
                wave_sync();
            }
        }
        // fold in sorted order, tile by tile
        const DeepArray sorted = (plan.passes & 1) ? shadow : bucket;
        for (uint32_t t0 = 0; t0 < cnt; t0 += kWaveSize) {
            const uint32_t p = t0 + lane;
            const uint64_t at = p < cnt ? sorted.at(p) : 0u;
            const uint32_t key_lo = p < cnt ? static_cast<uint32_t>(ld(&sorted.base[2 * at])) : 0u;
            const uint32_t val = p < cnt ? static_cast<uint32_t>(ld(&sorted.base[2 * at + 1])) : 0u;
            const uint32_t m = min(kWaveSize, cnt - t0);
            for (uint32_t j = 0; j < m; ++j)
                add(__builtin_amdgcn_readlane(key_lo, static_cast<int>(j)), __builtin_amdgcn_readlane(val, static_cast<int>(j)));
        }
    }
    *refractory = refr;
    if (!refr) {
        const float gate = clampf(b3, 0.0f, 1.0f);
        const float net = b0 + b2 * gate + b1;
        const float adaptation = ad0 + ad1 + ad2;
        const float drive = a.m.excitability[n] * net - fat - adaptation - pi;
        mem = mem + drive;
    }
    if (lane == 0) {
        if (c.tally)
            c.tally[cnt <= kDeepRegisterEntries ? kTDeepRegister : kTDeepRadix] += 1u;
        else
            atomicAdd(counter_word(c, c.part, kCDeep, tick), cnt <= kDeepRegisterEntries ? 1u : 0x10000u);
        if (e > 0) {
            (*nf(d, n, kNFatigue)) = fat;
            (*nf(d, n, kNAdapt0)) = ad0;
            (*nf(d, n, kNAdapt0 + 1)) = ad1;
            (*nf(d, n, kNAdapt0 + 2)) = ad2;
            (*nu(d, n, kNLastTick)) = tick;
        }
        counts[n] = 0;
        (*nu(d, n, kNTouched)) = tick + 1;
        if (fired) {
            (*nf(d, n, kNActivation)) = 0.0f;
            (*nu(d, n, kNRefractory)) = refractory_until;
        }
        (*nf(d, n, kNBranch0)) = b0;
        (*nf(d, n, kNBranch0 + 1)) = b1;
        (*nf(d, n, kNBranch0 + 2)) = b2;
        (*nf(d, n, kNBranch0 + 3)) = b3;
        if (e > 0 || !refr) (*nf(d, n, kNMembrane)) = mem;
    }
    return mem - threshold;
}

// analog_rank_surrogate of a touched neuron (runtime.rs:787-803).
__device__ __forceinline__ float surrogate_value(const LeoConfig& cfg, bool refractory, float margin, float cutoff,
                                                 bool selected) {
    if (refractory) return 0.0f;
    return analog_rank_surrogate(margin, cutoff, selected, cfg.surrogate_width, cfg.surrogate_gain);
}

// Phase-2 window of one wave in dynamic LDS (window_bytes per wave): the
// touched neurons of a group of blocks in neuron order, their selection keys,
// and per group block its first list position, candidate count and the key of
// rank `limit`; plus the group's bitmap words and their list positions.
struct Window {
    uint64_t* key;     // capacity: selection key, ~0 for a non-candidate
    uint64_t* cut;     // kGroupBlocks
    uint32_t* entry;   // capacity: (group block << 16) | offset in the block
    uint32_t* start;   // kGroupBlocks + 1
    uint32_t* cands;   // kGroupBlocks
    uint32_t* woff;    // kGroupBlocks: first staged winner position of each group block
    uint32_t* bits;    // kWaveSize * kWordsPerLane: bitmap words of the group
    uint32_t* pos;     // kWaveSize * kWordsPerLane: list position of each word's first bit
};

static_assert(kGroupBlocks == kWaveSize, "one lane per group block");
static_assert(kMaxBlockNeurons <= 0x10000u, "window entries hold a 16-bit offset in the block");

__device__ __forceinline__ Window wave_window(uint32_t wave, uint32_t nb) {
    unsigned char* base = step_lds + static_cast<size_t>(wave) * wave_lds_bytes(nb);
    const uint32_t cap = window_capacity(nb);
    Window w;
    w.key = reinterpret_cast<uint64_t*>(base);
    w.cut = w.key + cap;
    w.entry = reinterpret_cast<uint32_t*>(w.cut + kGroupBlocks);
    w.start = w.entry + cap;
    w.cands = w.start + kGroupBlocks + 1;
    w.woff = w.cands + kGroupBlocks;
    w.bits = w.woff + kGroupBlocks;
    w.pos = w.bits + kWaveSize * kWordsPerLane;
    return w;
}

// Phase 2: each wave owns a range of blocks and takes it in groups of up to
// kGroupBlocks blocks. Per group it loads (and clears) the group's touched
// bitmap in one round of coalesced loads, lists the touched neurons in neuron
// order, folds and drives them one lane each, and ranks every candidate within
// its block: a candidate's rank is the number of smaller (activation desc, tie
// asc) keys of its block, i.e. its position in the reference's sorted order
// (runtime.rs:987-1011; keys are unique); rank `limit` gives the block cutoff.
// The winners of the wave's range are staged in block order (runtime.rs:
// 1010-1013), compacted from the range's first block row, so that phase 3
// reads them in one round. A group with more touched neurons than the window
// holds is taken in windows of whole blocks.
// `keep_bits`: a trace step leaves the bitmap words set for its eligibility
// update (the learning phase clears them from the touched list). `pi` is the
// population inhibition the previous tick left; `post_pending` that the
// previous tick's winners still await their post-fire updates (fold_drive).
// The fold counts the tick's delivered entries (kCEvents: the F injections
// included, which the record takes off).
__device__ __forceinline__ void phase_fold_select(const StepCtx& c, StepShared& sh, bool keep_bits, float pi,
                                                  bool post_pending) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, nb = cfg.neurons_per_block, limit = cfg.max_active_per_block;
    const uint32_t tick = c.tick, rot = tick % N;
    const uint32_t wave = wave_index(), lane = __lane_id();
    const uint32_t nwaves = selecting_waves(c);
    const uint32_t wv = c.part * kWavesPerGroup + wave;
    const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
    const uint32_t b0 = min(cfg.block_count, wv * range), b1 = min(cfg.block_count, b0 + range);
    const uint32_t wpb = block_words(nb);
    const uint32_t group = min(kGroupBlocks, kWaveSize * kWordsPerLane / wpb);
    const uint32_t cap = window_capacity(nb);
    const uint32_t set = set_of(d, tick);
    const FastDiv block_div = a.div_block_words;
    const Window w = wave_window(wave, nb);
    w.cands[lane] = 0;
    w.cut[lane] = ~0ULL;
    const uint64_t row0 = static_cast<uint64_t>(b0) * limit;
    // this wave's touched neurons are listed from its range's first neuron on
    // (no shared counter to wait for)
    const uint32_t first_listed = b0 * nb;
    uint32_t supra = 0, staged = 0, listed_before = 0, entries = 0;
    for (uint32_t gb = b0; gb < b1; gb += group) {
        const uint32_t gn = min(group, b1 - gb), gw = gn * wpb;
        uint32_t* bits = set_touched(d, set) + static_cast<uint64_t>(gb) * wpb;
        uint32_t word[kWordsPerLane];
#pragma unroll
        for (uint32_t k = 0; k < kWordsPerLane; ++k) {
            const uint32_t at = k * kWaveSize + lane;
            word[k] = at < gw ? ld(&bits[at]) : 0u;
        }
        // list positions in word order (row k holds words k*64 .. k*64+63);
        // each row's neurons are listed as soon as its positions are known
        // (the words are in registers), at positions below the window
        // capacity: a group that fits the window is then fully listed
        uint32_t total = 0;
#pragma unroll
        for (uint32_t k = 0; k < kWordsPerLane; ++k) {
            const uint32_t at = k * kWaveSize + lane;
            if (k * kWaveSize < gw) {
                const uint32_t cnt = __popc(word[k]);
                const uint32_t incl = wave_incl_scan_u32(cnt);
                uint32_t p = total + incl - cnt;
                w.bits[at] = word[k];
                w.pos[at] = p;
                uint32_t v = word[k];
                if (v != 0 && p < cap) {
                    const uint32_t g = fast_div(at, block_div), base = (at - g * wpb) * 32;
                    while (v) {
                        const uint32_t bit = __ffs(v) - 1;
                        v &= v - 1;
                        if (p < cap) w.entry[p] = (g << 16) | (base + bit);
                        ++p;
                    }
                }
                total += __builtin_amdgcn_readlane(incl, kWaveSize - 1);
            }
        }
        // the words are cleared after the scan: a store issued between the
        // rows would be waited for together with the next row's words
#pragma unroll
        for (uint32_t k = 0; k < kWordsPerLane; ++k) {
            const uint32_t at = k * kWaveSize + lane;
            if (!keep_bits && at < gw && word[k]) bits[at] = 0u;
        }
        // block starts: the list position of each block's first word
        wave_sync();
        if (lane < gn) w.start[lane] = w.pos[lane * wpb];
        if (lane == 0) w.start[gn] = total;
        wave_sync();
        for (uint32_t lo = 0; lo < total;) {
            uint32_t hi = total;
            if (total - lo > cap) {
                // the last block boundary within the window (a block holds at most nb <= cap)
                uint32_t best = lo;
                for (uint32_t g = lane; g <= gn; g += kWaveSize) {
                    const uint32_t st = w.start[g];
                    if (st <= lo + cap && st > best) best = st;
                }
                hi = static_cast<uint32_t>(wave_max_u64(best));
            }
            for (uint32_t k = 0; total > cap && k < kWordsPerLane; ++k) {  // else listed in the scan
                const uint32_t at = k * kWaveSize + lane;
                if (at >= gw) break;
                uint32_t v = w.bits[at], p = w.pos[at];
                if (p >= hi || p + __popc(v) <= lo) continue;
                const uint32_t g = fast_div(at, block_div), base = (at - g * wpb) * 32;
                while (v) {
                    const uint32_t bit = __ffs(v) - 1;
                    v &= v - 1;
                    if (p >= lo && p < hi) w.entry[p - lo] = (g << 16) | (base + bit);
                    ++p;
                }
            }
            wave_sync();
            const uint32_t cnt = hi - lo;
            const uint32_t listed = first_listed + listed_before + lo;
            bool any_deep = false;
            for (uint32_t i = lane; i < cnt; i += kWaveSize) {
                const uint32_t e = w.entry[i];
                const uint32_t g = e >> 16;
                const uint32_t n = (gb + g) * nb + (e & 0xffffu);
                bool refractory = false, deep = false;
                uint32_t folded = 0;
                const float act = clampf(fold_drive(c, n, pi, set, post_pending, &refractory, &deep, &folded), 0.0f, 1.0f);
                entries += folded;
                const bool candidate = !deep && !refractory && act > 0.0f;
                w.key[i] = deep ? kDeepPending : candidate ? selection_key(act, add_mod(n, N - rot, N)) : ~0ULL;
                any_deep |= deep;
                if (candidate) atomicAdd(&w.cands[g], 1u);
                if (keep_bits) d.touched_list[listed + i] = n;  // read by a trace step's homeostasis only
            }
            wave_sync();
            if (__ballot(any_deep)) {
                // neurons with more than 8 deliveries: the whole wave folds each
                uint32_t* hist = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned char*>(w.key) +
                                                             wave_window_bytes(nb));
                for (uint32_t i0 = 0; i0 < cnt; i0 += kWaveSize) {
                    uint64_t pending = __ballot(i0 + lane < cnt && w.key[i0 + lane] == kDeepPending);
                    while (pending) {
                        const uint32_t i = i0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(pending)) - 1);
                        pending &= pending - 1;
                        const uint32_t e = __builtin_amdgcn_readfirstlane(w.entry[i]);
                        const uint32_t g = e >> 16;
                        const uint32_t n = (gb + g) * nb + (e & 0xffffu);
                        bool refractory = false;
                        const float act = clampf(deep_fold(c, n, pi, set, post_pending, &refractory, hist), 0.0f, 1.0f);
                        const bool candidate = !refractory && act > 0.0f;
                        if (lane == 0) {
                            w.key[i] = candidate ? selection_key(act, add_mod(n, N - rot, N)) : ~0ULL;
                            if (candidate) atomicAdd(&w.cands[g], 1u);
                        }
                        wave_sync();
                    }
                }
            }
            {
                // staged positions of this window's blocks (block order)
                const bool in = lane < gn && w.start[lane] >= lo && w.start[lane] < hi;
                const uint32_t win = in ? min(w.cands[lane], limit) : 0u;
                const uint32_t incl = wave_incl_scan_u32(win);
                if (in) w.woff[lane] = staged + incl - win;
                staged += __builtin_amdgcn_readlane(incl, kWaveSize - 1);
            }
            wave_sync();
            for (uint32_t i = lane; i < cnt; i += kWaveSize) {
                const uint64_t mine = w.key[i];
                if (mine == ~0ULL) continue;
                const uint32_t g = w.entry[i] >> 16;
                const uint32_t s0 = w.start[g] - lo, s1 = w.start[g + 1] - lo;
                uint32_t rank = 0;
                // eight independent LDS reads in flight per round (one read
                // at a time waits out the LDS latency on every key)
                uint32_t j = s0;
                for (; j + 8 <= s1; j += 8) {
                    uint64_t k[8];
#pragma unroll
                    for (uint32_t x = 0; x < 8; ++x) k[x] = w.key[j + x];
#pragma unroll
                    for (uint32_t x = 0; x < 8; ++x) rank += k[x] < mine ? 1u : 0u;
                }
                for (; j < s1; ++j) rank += w.key[j] < mine ? 1u : 0u;
                if (rank < limit) {
                    const uint32_t n = add_mod(static_cast<uint32_t>(mine), rot, N);
                    const float act = key_activation(mine);
                    const uint32_t k = w.woff[g] + rank;  // staged position in the wave's range
                    const uint64_t at = row0 + k;
                    d.range_winners[at] = n;
                    d.range_winner_act[at] = act;
                    if (k < kWaveSize) {  // kept for phase 3 in the wave's LDS
                        sh.win_n[wave][k] = n;
                        sh.win_act[wave][k] = act;
                    }
                    if (a.redundant_global) {  // the global cap cannot bind (runtime.rs:1060-1067)
                        (*nf(d, n, kNActivation)) = act;
                        (*nu(d, n, kNSelected)) = tick + 1;
                    }
                } else if (rank == limit) {
                    w.cut[g] = mine;
                }
            }
            wave_sync();
            lo = hi;
        }
        // block results, read only by a trace step's eligibility update (as
        // this tick's, by epoch); a block without touched neurons keeps a
        // stale epoch (no winners, cutoff 0)
        if (lane < gn && w.start[lane + 1] > w.start[lane]) {
            const uint32_t b = gb + lane;
            if (keep_bits) {
                d.block_cutoff[b] = w.cut[lane] != ~0ULL ? key_activation(w.cut[lane]) : 0.0f;
                d.block_epoch[b] = tick + 1;
            }
            supra += w.cands[lane];
        }
        w.cands[lane] = 0;
        w.cut[lane] = ~0ULL;
        listed_before += total;
        wave_sync();
    }
    supra = wave_sum_u32(supra);
    entries = wave_sum_u32(entries);
    if (lane == 0) {
        if (c.tally) {
            // no counter atomics mid-step: each would hold up the wave's later
            // load waits (memory operations retire in order)
            c.tally[kTEvents] += entries;
            c.tally[kTTouched] += listed_before;
        } else {
            if (supra) atomicAdd(counter_word(c, c.part, kCSupra, tick), supra);
            if (entries) atomicAdd(counter_word(c, c.part, kCEvents, tick), entries);
            if (listed_before) atomicAdd(counter_word(c, c.part, kCTouched, tick), listed_before);
        }
        sh.win_count[wave] = staged;
        wave_totals(d, tick)[wv] = staged;
        d.wave_touched[wv] = listed_before;
    }
}

// ---------------------------------------------------------------------------
// Phase 3: the active list of this tick (block winners concatenated in block
// order, runtime.rs:1010-1013), population inhibition (runtime.rs:1076-1082)
// and the forward eligibilities (runtime.rs:805-918).
// ---------------------------------------------------------------------------
// With `ahead` (a fused step followed by a frozen one, `next`) the next
// tick's delivery runs here too: each wave starts the next tick for its own
// winners (activation reset and touch, runtime.rs:544-555, and the delivery
// of their delay-1 events, which the next tick would otherwise read back
// from the ring), and the delivering workgroups take the remaining items.
// The memory operations are grouped into three rounds: the winners with the
// first next-tick item; the winners' state and synapses with that item's
// bucket increment; the delay-1 bucket increments.
__device__ __forceinline__ void write_active(const StepCtx& c, const StepParams& sp, uint32_t step_index,
                                             StepShared& sh, bool fuse_post, bool ahead, const StepParams& next,
                                             bool late_done) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = c.d;
    const uint32_t cap = cfg.max_active_global, limit = cfg.max_active_per_block;
    const uint32_t wave = wave_index(), lane = __lane_id();
    const uint32_t nwaves = selecting_waves(c);
    const uint32_t wv = c.part * kWavesPerGroup + wave;
    const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
    const uint32_t rs = c.tick % kRing;
    const uint32_t b0 = min(cfg.block_count, wv * range);
    const uint64_t row0 = static_cast<uint64_t>(b0) * limit;
    // first memory round: the per-wave totals, this wave's winners' state and first
    // synapses, and this thread's first item of the next tick
    // the recording wave's loads go out in the same round; it runs on the
    // workgroup that selects nothing (the least work in this phase)
    const bool rec_wave = c.part == c.P - 1 && wave == 0;
    const bool recorder = rec_wave && lane == 0;
    float pi_old = 0.0f;
    uint32_t supra = 0, rec_n = 0, in_n = 0, cells = 0, probes = 0, applied = 0;
    LateCounters late{};
    if (rec_wave && !c.tally) {
        if (fuse_post) supra = counter_total(c, kCSupra, c.tick);
        if (step_index > 0 && !late_done) late = load_late_counters(c, c.tick - 1);
    }
    if (recorder) {
        pi_old = ld(&c.ctl->population_inhibition);
        if (fuse_post) {
            rec_n = ld(&c.ctl->rec_count[c.parity]);
            in_n = ld(&c.ctl->in_count[c.parity]);
            // the context of this step is resolved (phase 1 or 2); the next
            // step's resolution runs after these loads (phase 2 of the next
            // step, or below on the same workgroup)
            cells = ld(&c.ctl->ctx_count);
            probes = ld(&c.ctl->ctx_probes);
            applied = ld(&c.ctl->ctx_applied);
        }
    }
    const DeliverPlan np = deliver_plan(c, sh, true);
    const bool deliver_next = ahead && np.delivers;
    // the next tick's items are dealt to the workgroups in turn (by thread
    // id, the first 16 of 32 workgroups at D took them all)
    const uint32_t dealt = dealt_index(c, c.P);
    DeliverItem item0 = deliver_fetch(c, next, np, deliver_next ? dealt : np.total);
    if (ahead) reset_next_lists(c);
    // this wave's winners are in its LDS since phase 2: their state and
    // synapses are loaded in the same round as the totals
    const uint32_t mine = sh.win_count[wave];
    const uint32_t first_n = lane < mine ? sh.win_n[wave][lane] : 0u;
    const float first_act = lane < mine ? sh.win_act[wave][lane] : 0.0f;
    const uint32_t S = cfg.synapses_per_neuron, N = cfg.neuron_count;
    const uint32_t items = mine * S;
    const bool pf = fuse_post && lane < mine, sn = fuse_post && lane < items;
    float fat = 0.0f, ad0 = 0.0f, ad1 = 0.0f, ad2 = 0.0f, mem = 0.0f, thr = 0.0f;
    uint8_t type = 0;
    if (pf) {
        // quarters 0 and 1 of the record: membrane, fatigue, adaptations
        const __amdgpu_buffer_rsrc_t rec = neuron_rsrc(d, N);
        const f32x4 q0 = ld_quarter(rec, first_n, 0), q1 = ld_quarter(rec, first_n, 1);
        mem = q0.x;
        fat = q0.z;
        ad0 = q0.w;
        ad1 = q1.x;
        ad2 = q1.y;
        thr = ld(&d.p.threshold[first_n]);
        type = c.a->m.neuron_type[first_n];
    }
    uint32_t r0 = 0, j0 = 0, edge0 = 0;
    float act0 = 0.0f, weight0 = 0.0f;
    if (sn) {
        r0 = fast_div(lane, c.a->div_synapses);
        j0 = lane - r0 * S;
        const uint32_t n = sh.win_n[wave][r0];
        act0 = sh.win_act[wave][r0];
        const uint64_t slot = static_cast<uint64_t>(n) * S + j0;
        weight0 = ld(&d.p.rec_weight[slot]);
        edge0 = c.a->m.rec_edge[slot];
    }
    uint32_t before = 0, all = 0;
    sum_totals(wave_totals(d, c.tick), nwaves, wv, all, before);
    uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap + before;
    float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap + before;
    for (uint32_t i = lane; i < mine; i += kWaveSize) {
        const bool pre = i == lane;
        act_list[i] = pre ? first_n : ld(&d.range_winners[row0 + i]);
        act_val[i] = pre ? first_act : ld(&d.range_winner_act[row0 + i]);
    }
    const float activity = static_cast<float>(all) / static_cast<float>(cfg.neuron_count);
    if (recorder) {
        // tick-1's record is finished (tick-1 is complete); the recording
        // wave then clears its counters, which tick+1 reuses
        LaneControl LEO_GLOBAL* ctl = c.ctl;
        if (step_index > 0 && !late_done && !c.tally) store_late_record(d, step_index - 1, late);
        ctl->active_count = all;
        ctl->block_selected = all;
        ctl->clipped = 0;
        ctl->pop_cutoff = 0.0f;
        ctl->ring_tick[rs] = c.tick;
        ctl->ring_count[rs] = all;
        ctl->ring_early[rs] = 0;
        const float pi = clampf(pi_old + cfg.population_inhibition_rate * (activity - cfg.target_activity), 0.0f,
                                cfg.population_inhibition_max);
        ctl->population_inhibition = pi;
        if (fuse_post && c.tally) {
            sh.tally_rec[0] += all;
            sh.tally_rec[1] += cells;
            sh.tally_rec[2] += rec_n;
            sh.tally_rec[3] += in_n;
        } else if (fuse_post) {
            // the step record the post phase would write (no readout this step)
            StepRecord LEO_GLOBAL& rec = d.records[step_index];
            rec.p_target = 0.0f;
            rec.predicted = 0;
            rec.population_inhibition = pi;
            rec.active = all;
            rec.suprathreshold = supra;
            rec.block_selected = all;
            rec.clipped = 0;
            rec.context_cells = cells;
            rec.context_probes = probes;
            rec.context_applied = applied;
            rec.eligible_rec = rec_n;
            rec.eligible_in = in_n;
            rec.error_code = 0;
        }
    }
    if (rec_wave && !c.tally) clear_counters(c, c.tick);  // after its loads of tick-1's counters
    if (!fuse_post) return;
    // Post-fire updates of this wave's winners and their emission snapshots
    // (the post phase, runtime.rs:920-938, 1084-1106), folded in here when no
    // eligibility update or readout of this step reads the state in between.
    // The wave's first 64 winners are in its LDS since phase 2.
    const uint32_t refractory = c.tick + cfg.refractory_ticks + 1;
    const uint32_t next_set = set_of(d, c.tick + 1);
    uint32_t inhibitory = 0, delivered = 0;
    auto post_fire = [&](uint32_t n, float act, float fat, float ad0, float ad1, float ad2, float mem, float thr,
                         uint8_t type) {
        inhibitory += type != 0 ? 1u : 0u;
        (*nf(d, n, kNFatigue)) = fat + cfg.fatigue_gain * act;
        (*nf(d, n, kNAdapt0)) = ad0 + cfg.adaptation_fast_gain * act;
        (*nf(d, n, kNAdapt0 + 1)) = ad1 + cfg.adaptation_medium_gain * act;
        (*nf(d, n, kNAdapt0 + 2)) = ad2 + cfg.adaptation_slow_gain * act;
        (*nf(d, n, kNMembrane)) = mem - thr * cfg.membrane_reset_fraction;
        (*nu(d, n, kNRefractory)) = refractory;
        if (ahead) {
            (*nf(d, n, kNActivation)) = 0.0f;
            touch_neuron(c, n, c.tick + 1);
        }
    };
    auto snapshot = [&](uint32_t r, uint32_t j, float act, float weight, uint32_t edge) {
        const uint64_t at = (static_cast<uint64_t>(rs) * cap + before + r) * S + j;
        const float value = act * weight;
        d.ring_value[at] = value;
        d.ring_edge[at] = edge;
        if (ahead && edge_delay(edge) == 1) {
            // delay class 1 of the next tick, keyed by active rank as its
            // delivery from the ring would be
            const uint64_t key = (3ull << 61) | (static_cast<uint64_t>(before + r) << 32) |
                                 (static_cast<uint64_t>(j) << 2) | edge_branch(edge);
            if (scatter_event(c, next_set, edge_target(edge), key, value)) touch_neuron(c, edge_target(edge), c.tick + 1);
            delivered += 1;
        }
    };
    // second memory round: the bucket increment of this thread's first next-tick item
    // (the winners' state and first synapses are loaded with the totals)
    if (deliver_next) deliver_commit(c, next, np, item0, delivered);
    // third memory round: the delay-1 bucket increments
    if (pf) post_fire(first_n, first_act, fat, ad0, ad1, ad2, mem, thr, type);
    if (sn) snapshot(r0, j0, act0, weight0, edge0);
    // further rounds: more than 64 winners or synapses in this wave, more
    // next-tick items than delivering threads
    for (uint32_t r = lane + kWaveSize; r < mine; r += kWaveSize) {
        const uint32_t n = ld(&d.range_winners[row0 + r]);
        post_fire(n, ld(&d.range_winner_act[row0 + r]), ld(nf(d, n, kNFatigue)), ld(nf(d, n, kNAdapt0)), ld(nf(d, n, kNAdapt0 + 1)),
                  ld(nf(d, n, kNAdapt0 + 2)), ld(nf(d, n, kNMembrane)), ld(&d.p.threshold[n]), c.a->m.neuron_type[n]);
    }
    for (uint32_t item = lane + kWaveSize; item < items; item += kWaveSize) {
        const uint32_t r = fast_div(item, c.a->div_synapses), j = item - r * S;
        const uint32_t n = r < kWaveSize ? sh.win_n[wave][r] : ld(&d.range_winners[row0 + r]);
        const float act = r < kWaveSize ? sh.win_act[wave][r] : ld(&d.range_winner_act[row0 + r]);
        const uint64_t slot = static_cast<uint64_t>(n) * S + j;
        snapshot(r, j, act, ld(&d.p.rec_weight[slot]), c.a->m.rec_edge[slot]);
    }
    if (ahead) deliver_items(c, next, np, dealt + np.stride, delivered);
    count_wave(c, kCInhibitory, c.tick, inhibitory);
    if (threadIdx.x == 0) {  // the next deliveries read this tick's ring entry from LDS
        sh.ring_tick[rs] = c.tick;
        sh.ring_count[rs] = all;
        sh.ring_early[rs] = 0;
    }
}

// ---------------------------------------------------------------------------
// One-barrier frozen steps. On a lane with kBucketSets bucket sets, a frozen
// step whose next step is frozen too (neither reads eligibilities or the
// readout) runs as a single phase: the fold and selection of its tick t,
// then, with no barrier between, every event its winners emit, each into the
// bucket set of its arrival tick t + delay (up to 8 ticks ahead, a set no
// other wave folds in this phase), and tick t+1's other deliveries (the
// input injection, the ring classes of earlier two-phase ticks). No wave
// waits for another: an event is keyed by its winner's staged position in
// its wave's block range (row0 + k) instead of its active-list rank. The
// active list is the waves' staged winners in wave order, so both keys order
// a tick's events alike and the fold sums them in the reference's order
// (runtime.rs:605-639). What needs every wave's winners waits for the next
// phase: the winners' post-fire updates and activation reset for their fold
// at t+1 (fold_drive), the population inhibition and the step record for
// frozen_prologue. The ring keeps no entries for tick t (its readers find a
// stale tick there and deliver nothing from it: every event of t is
// already in its bucket).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void frozen_emit(const StepCtx& c, StepShared& sh, uint32_t early, const StepParams& next) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = c.d;
    const uint32_t wave = wave_index(), lane = __lane_id();
    const uint32_t nwaves = selecting_waves(c);
    const uint32_t wv = c.part * kWavesPerGroup + wave;
    const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
    const uint32_t b0 = min(cfg.block_count, wv * range);
    const uint64_t row0 = static_cast<uint64_t>(b0) * cfg.max_active_per_block;
    const uint32_t S = cfg.synapses_per_neuron;
    // tick t+1's other deliveries, dealt over every workgroup: this thread's
    // first item's loads go out before the winners' work
    const DeliverPlan np = deliver_plan(c, sh, true);
    const uint32_t dealt = dealt_index(c, c.P);
    DeliverItem item0 = deliver_fetch(c, next, np, np.delivers ? dealt : np.total);
    reset_next_lists(c);
    const uint32_t mine = sh.win_count[wave];
    // staged winners past the wave's LDS copy are read back from memory the
    // wave has just written
    if (mine > kWaveSize) __builtin_amdgcn_s_waitcnt(0);
    auto winner = [&](uint32_t r, uint32_t& n, float& act) {
        if (r < kWaveSize) {
            n = sh.win_n[wave][r];
            act = sh.win_act[wave][r];
        } else {
            n = ld(&d.range_winners[row0 + r]);
            act = ld(&d.range_winner_act[row0 + r]);
        }
    };
    // the winners are touched at t+1, whose fold applies their post-fire
    // updates; the inhibitory ones count for this tick's record
    uint32_t inhibitory = 0;
    for (uint32_t r = lane; r < mine; r += kWaveSize) {
        uint32_t n;
        float act;
        winner(r, n, act);
        inhibitory += c.a->m.neuron_type[n] != 0 ? 1u : 0u;
        touch_neuron(c, n, c.tick + 1);
    }
    // every synapse of every winner whose delay is early (runtime.rs:1084-1106
    // emits them into the ring; the value is the snapshot the ring would
    // hold); the other delays' events stay for the ring, which the next
    // phase's prologue fills. A lane takes up to kEmitBatch events per round
    // of memory operations (their synapse loads, then their bucket claims,
    // then their entry writes), and the first round also claims the bucket
    // entry of its next-tick injection, whose loads went out above.
    constexpr uint32_t kEmitBatch = 4;
    const uint32_t items = early ? mine * S : 0u;
    const bool inj0 = np.delivers && item0.inj;
    const uint32_t inj_set = set_of(d, c.tick + 1);
    const uint32_t rounds = items > 0 ? (items + kEmitBatch * kWaveSize - 1) / (kEmitBatch * kWaveSize) : 1u;
    for (uint32_t round = 0; round < rounds; ++round) {
        const uint32_t base = round * kEmitBatch * kWaveSize;
        uint32_t edge[kEmitBatch], rj[kEmitBatch];
        float value[kEmitBatch];
        bool live[kEmitBatch];
#pragma unroll
        for (uint32_t k = 0; k < kEmitBatch; ++k) {
            const uint32_t item = base + k * kWaveSize + lane;
            live[k] = item < items;
            edge[k] = 0;
            value[k] = 0.0f;
            rj[k] = 0;
            if (live[k]) {
                const uint32_t r = fast_div(item, c.a->div_synapses), j = item - r * S;
                uint32_t n;
                float act;
                winner(r, n, act);
                const uint64_t slot = static_cast<uint64_t>(n) * S + j;
                value[k] = act * ld(&d.p.rec_weight[slot]);
                edge[k] = c.a->m.rec_edge[slot];
                rj[k] = item;
            }
        }
        EntryClaim claim[kEmitBatch];
        uint32_t set[kEmitBatch];
#pragma unroll
        for (uint32_t k = 0; k < kEmitBatch; ++k) {
            const uint32_t dl = (edge[k] >> kEdgeTargetBits) & 3u;  // delay 1 << dl, delivery class 3 - dl
            live[k] = live[k] && (early & (1u << dl)) != 0;
            set[k] = set_of(d, c.tick + (1u << dl));
            if (live[k]) claim[k] = claim_entry(c, set[k], edge_target(edge[k]));
        }
        EntryClaim inj{};
        const bool inj_here = round == 0 && inj0;
        if (inj_here) inj = claim_entry(c, inj_set, item0.target);
#pragma unroll
        for (uint32_t k = 0; k < kEmitBatch; ++k) {
            if (!live[k]) continue;
            const uint32_t dl = (edge[k] >> kEdgeTargetBits) & 3u;
            const uint32_t r = fast_div(rj[k], c.a->div_synapses), j = rj[k] - r * S;
            const uint64_t key = (static_cast<uint64_t>(3u - dl) << 61) | ((row0 + r) << 32) |
                                 (static_cast<uint64_t>(j) << 2) | edge_branch(edge[k]);
            if (write_entry(c, set[k], edge_target(edge[k]), claim[k], key, value[k]))
                touch_neuron(c, edge_target(edge[k]), c.tick + (1u << dl));
        }
        if (inj_here && write_entry(c, inj_set, item0.target, inj, item0.key, item0.value))
            touch_neuron(c, item0.target, c.tick + 1);
    }
    uint32_t delivered = 0;  // counted by the fold
    item0.inj = item0.inj && !inj0;  // an injection claimed above is done
    if (np.delivers) deliver_commit(c, next, np, item0, delivered);
    deliver_items(c, next, np, dealt + np.stride, delivered);
    count_wave(c, kCInhibitory, c.tick, inhibitory);
}

// The start of the phase after a one-barrier frozen step (tick t-1, step
// step_index-1): every wave sums that tick's winners from the waves' totals
// and takes the population inhibition forward from the value the previous
// fold read (runtime.rs:1076-1082; every wave computes the same value);
// the recording wave writes the step's record and clears the counters that
// tick t+1 reuses. Returns tick t-1's population inhibition, which the fold
// of t reads.
__device__ __forceinline__ float frozen_prologue(const StepCtx& c, StepShared& sh, uint32_t step_index,
                                                float pi_before, uint32_t early) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = c.d;
    const uint32_t prev = c.tick - 1, nwaves = selecting_waves(c), lane = __lane_id(), wave = wave_index();
    const uint32_t wv = c.part * kWavesPerGroup + wave;
    uint32_t all = 0, before = 0;
    if (c.carried) {
        // from the barrier: the lane's total and the waves before this one
        all = sh.lane_sums[0];
        before = sh.lane_sums[1 + wave];
    } else {
        sum_totals(wave_totals(d, prev), nwaves, wv, all, before);
    }
    const uint32_t rs = prev % kRing;
    if (early != 0xfu && wv < nwaves) {
        // some delays' events go through the ring: the tick's active list
        // (runtime.rs:1010-1013) and emission snapshots, at active-list
        // positions (the wave's winners of tick t-1 are still in its LDS:
        // this tick's fold has not run yet)
        const uint32_t cap = cfg.max_active_global, S = cfg.synapses_per_neuron;
        const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
        const uint64_t row0 = static_cast<uint64_t>(min(cfg.block_count, wv * range)) * cfg.max_active_per_block;
        const uint32_t mine = sh.win_count[wave];
        auto winner = [&](uint32_t r, uint32_t& n, float& act) {
            if (r < kWaveSize) {
                n = sh.win_n[wave][r];
                act = sh.win_act[wave][r];
            } else {
                n = ld(&d.range_winners[row0 + r]);
                act = ld(&d.range_winner_act[row0 + r]);
            }
        };
        const uint64_t first = static_cast<uint64_t>(rs) * cap + before;
        for (uint32_t r = lane; r < mine; r += kWaveSize) {
            uint32_t n;
            float act;
            winner(r, n, act);
            d.ring_active[first + r] = n;
            d.ring_act[first + r] = act;
        }
        for (uint32_t item = lane; item < mine * S; item += kWaveSize) {
            const uint32_t r = fast_div(item, c.a->div_synapses), j = item - r * S;
            uint32_t n;
            float act;
            winner(r, n, act);
            const uint64_t slot = static_cast<uint64_t>(n) * S + j;
            const uint64_t at = (first + r) * S + j;
            d.ring_value[at] = act * ld(&d.p.rec_weight[slot]);
            d.ring_edge[at] = c.a->m.rec_edge[slot];
        }
    }
    if (threadIdx.x == 0) {  // this workgroup's deliveries read the slot from LDS
        sh.ring_tick[rs] = prev;
        sh.ring_count[rs] = all;
        sh.ring_early[rs] = early;
    }
    const float activity = static_cast<float>(all) / static_cast<float>(cfg.neuron_count);
    const float pi = clampf(pi_before + cfg.population_inhibition_rate * (activity - cfg.target_activity), 0.0f,
                            cfg.population_inhibition_max);
    if (c.part == c.P - 1 && wave_index() == 0) {
        LateCounters late{};
        uint32_t supra = 0;
        if (!c.tally) {
            late = load_late_counters(c, prev);
            supra = counter_total(c, kCSupra, prev);
        }
        if (lane == 0) {
            LaneControl LEO_GLOBAL* ctl = c.ctl;
            const uint32_t rec_n = ld(&ctl->rec_count[c.parity]), in_n = ld(&ctl->in_count[c.parity]);
            const uint32_t cells = ld(&ctl->ctx_count), probes = ld(&ctl->ctx_probes);
            const uint32_t applied = ld(&ctl->ctx_applied);
            if (c.tally) {
                sh.tally_rec[0] += all;
                sh.tally_rec[1] += cells;
                sh.tally_rec[2] += rec_n;
                sh.tally_rec[3] += in_n;
            } else {
                StepRecord LEO_GLOBAL& rec = d.records[step_index - 1];
                rec.p_target = 0.0f;
                rec.predicted = 0;
                rec.population_inhibition = pi;
                rec.active = all;
                rec.suprathreshold = supra;
                rec.block_selected = all;
                rec.clipped = 0;
                rec.context_cells = cells;
                rec.context_probes = probes;
                rec.context_applied = applied;
                rec.eligible_rec = rec_n;
                rec.eligible_in = in_n;
                rec.error_code = 0;
                store_late_record(d, step_index - 1, late);
            }
            ctl->active_count = all;
            ctl->block_selected = all;
            ctl->clipped = 0;
            ctl->pop_cutoff = 0.0f;
            ctl->population_inhibition = pi;
            ctl->ring_tick[rs] = prev;
            ctl->ring_count[rs] = all;
            ctl->ring_early[rs] = early;
        }
        if (!c.tally) clear_counters(c, c.tick);  // after the loads of tick t-1's counters, whose words t+1 reuses
    }
    return pi;
}

// First active-list position of each selecting wave's winners (block order,
// runtime.rs:1010-1013) into starts[0..nwaves], starts[nwaves] = the total;
// by the whole workgroup (the running scan uses sh.scan).
__device__ __forceinline__ uint32_t wave_starts(const StepCtx& c, StepShared& sh, uint32_t* starts, uint32_t nwaves) {
    uint32_t running = 0;
    for (uint32_t base = 0; base < nwaves; base += kThreads) {
        const uint32_t wv = base + threadIdx.x;
        const uint32_t v = wv < nwaves ? ld(&wave_totals(c.d, c.tick)[wv]) : 0;
        sh.scan[threadIdx.x] = v;
        __syncthreads();
        for (uint32_t off = 1; off < kThreads; off <<= 1) {
            const uint32_t add = threadIdx.x >= off ? sh.scan[threadIdx.x - off] : 0;
            __syncthreads();
            sh.scan[threadIdx.x] += add;
            __syncthreads();
        }
        if (wv < nwaves) starts[wv] = running + sh.scan[threadIdx.x] - v;
        const uint32_t chunk_total = sh.scan[kThreads - 1];
        __syncthreads();
        running += chunk_total;
    }
    if (threadIdx.x == 0) starts[nwaves] = running;
    __syncthreads();
    return running;
}

// Binding global cap: every block winner by selection key ascending
// (activation desc, tie asc); the first max_active_global form the active list
// (runtime.rs:1029-1057). Every workgroup lists the selecting waves' first
// winner positions in LDS; up to kMaxBlockNeurons winners are then sorted in
// workgroup 0's LDS. Beyond that every workgroup ranks its share of the
// winners by counting the smaller keys (the keys are distinct: they hold the
// rotated neuron index), with all keys streamed through LDS in tiles, and
// places each kept winner at its rank.
__device__ __forceinline__ uint64_t winner_key(const LaneDesc& d, const uint32_t* starts, uint32_t nwaves,
                                               uint32_t range, uint32_t block_count, uint32_t limit, uint32_t flat,
                                               uint32_t N, uint32_t rot, uint32_t* n_out, float* act_out) {
    // the last wave whose first position is <= flat (empty waves come before it)
    uint32_t lo = 0, hi = nwaves;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (starts[mid] <= flat) lo = mid;
        else hi = mid;
    }
    const uint64_t at = static_cast<uint64_t>(min(block_count, lo * range)) * limit + (flat - starts[lo]);
    const uint32_t n = ld(&d.range_winners[at]);
    const float act = ld(&d.range_winner_act[at]);
    *n_out = n;
    *act_out = act;
    return selection_key(act, add_mod(n, N - rot, N));
}

__device__ __forceinline__ void global_select(const StepCtx& c, StepShared& sh, uint32_t step_index) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t N = cfg.neuron_count, limit = cfg.max_active_per_block, cap = cfg.max_active_global;
    const uint32_t tick = c.tick, rot = tick % N;
    const uint32_t rs = tick % kRing;
    uint32_t* starts = reinterpret_cast<uint32_t*>(step_lds);
    uint64_t* keys = reinterpret_cast<uint64_t*>(step_lds + kSelectStartsBytes);
    const uint32_t nwaves = selecting_waves(c);
    const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
    const uint32_t running = wave_starts(c, sh, starts, nwaves);
    const uint32_t active = running < cap ? running : cap;
    uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    float pop_cutoff = 0.0f;
    // the first winner not kept sets the population cutoff from its margin,
    // clamped to population_inhibition_max, not from its activation (which
    // is clamped to 1) (runtime.rs:1045-1050)
    auto cutoff_of = [&](uint32_t n) {
        return clampf(ld(nf(d, n, kNMembrane)) - ld(&d.p.threshold[n]), 0.0f, cfg.population_inhibition_max);
    };
    auto keep = [&](uint32_t rank, uint32_t n, float act) {
        act_list[rank] = n;
        act_val[rank] = act;
        (*nf(d, n, kNActivation)) = act;
        (*nu(d, n, kNSelected)) = tick + 1;
    };
    if (running <= kMaxBlockNeurons) {
        if (c.part != 0) return;
        for (uint32_t f = threadIdx.x; f < running; f += kThreads) {
            uint32_t n;
            float act;
            keys[f] = winner_key(d, starts, nwaves, range, cfg.block_count, limit, f, N, rot, &n, &act);
        }
        const uint32_t M = next_pow2(running < 2 ? 2 : running);
        for (uint32_t i = running + threadIdx.x; i < M; i += kThreads) keys[i] = ~0ULL;
        __syncthreads();
        bitonic_sort_lds(keys, M);
        if (running > cap) pop_cutoff = cutoff_of(add_mod(static_cast<uint32_t>(keys[cap]), rot, N));
        for (uint32_t i = threadIdx.x; i < active; i += kThreads) {
            const uint64_t key = keys[i];
            keep(i, add_mod(static_cast<uint32_t>(key), rot, N), key_activation(key));
        }
    } else {
        // this workgroup's share of the winners, a thread's key at a time
        const uint32_t tile = a.select_tile;
        const uint32_t per = (running + c.P - 1) / c.P;
        const uint32_t mine_lo = min(running, c.part * per), mine_hi = min(running, mine_lo + per);
        for (uint32_t base = mine_lo; base < mine_hi; base += kThreads) {
            const uint32_t f = base + threadIdx.x;
            const bool has = f < mine_hi;
            uint32_t my_n = 0;
            float my_act = 0.0f;
            uint64_t my_key = ~0ULL;
            if (has) my_key = winner_key(d, starts, nwaves, range, cfg.block_count, limit, f, N, rot, &my_n, &my_act);
            uint32_t rank = 0;
            for (uint32_t t0 = 0; t0 < running; t0 += tile) {
                const uint32_t tn = min(tile, running - t0);
                __syncthreads();  // the previous tile is consumed
                for (uint32_t i = threadIdx.x; i < tn; i += kThreads) {
                    uint32_t n;
                    float act;
                    keys[i] = winner_key(d, starts, nwaves, range, cfg.block_count, limit, t0 + i, N, rot, &n, &act);
                }
                __syncthreads();
                if (has)
                    for (uint32_t i = 0; i < tn; ++i) rank += keys[i] < my_key ? 1u : 0u;
            }
            if (has) {
                if (rank < cap) keep(rank, my_n, my_act);
                else if (rank == cap) c.ctl->pop_cutoff = cutoff_of(my_n);
            }
        }
        if (c.part != 0) return;
    }
    __syncthreads();
    if (threadIdx.x < kWaveSize) roll_counters(c, step_index);
    if (threadIdx.x == 0) {
        LaneControl* ctl = c.ctl;
        ctl->active_count = active;
        ctl->block_selected = running;
        ctl->clipped = running - active;
        // beyond kMaxBlockNeurons winners the workgroup that ranks the first
        // winner not kept stores the cutoff
        if (running <= kMaxBlockNeurons || running <= cap) ctl->pop_cutoff = pop_cutoff;
        ctl->ring_tick[rs] = tick;
        ctl->ring_count[rs] = active;
        ctl->ring_early[rs] = 0;
        const float activity = static_cast<float>(active) / static_cast<float>(N);
        ctl->population_inhibition = clampf(
            ld(&ctl->population_inhibition) + cfg.population_inhibition_rate * (activity - cfg.target_activity), 0.0f,
            cfg.population_inhibition_max);
    }
}

// One eligible slot's update (runtime.rs:805-918) in parts, so that a lane
// can keep the loads of two slots in flight together: the slot's trace record
// (two 16-byte loads) with the destination's touched and selected epochs,
// then -- only for a destination touched this tick (a few percent of the
// eligible slots of a large model) -- the rest of the destination's state,
// then the update and its two 16-byte stores.
struct SlotInputs {
    float bs, ms, fs, as0, as1, as2, e;
    uint32_t last;
    uint32_t touched_epoch, selected_epoch, refractory_until, block_epoch;
    float temporal, gate_acc, block_cut, membrane, threshold, excitability;
};

__device__ __forceinline__ void load_slot(SlotInputs& in, __amdgpu_buffer_rsrc_t rsrc, uint32_t slot) {
    const f32x4 q0 = ld16_record(rsrc, slot, 0), q1 = ld16_record(rsrc, slot, 16);
    in.bs = q0.x;
    in.ms = q0.y;
    in.fs = q0.z;
    in.as0 = q0.w;
    in.as1 = q1.x;
    in.as2 = q1.y;
    in.e = q1.z;
    in.last = __float_as_uint(q1.w);
}

// Whether the destination was touched this tick: its bit in the touched
// bitmap, which a trace step keeps until its learning phase (a 4-byte read
// from a cache-resident array instead of a line of the destination's record).
__device__ __forceinline__ void load_touched(SlotInputs& in, const StepCtx& c, uint32_t dst) {
    const uint32_t nb = c.a->cfg.neurons_per_block;
    const uint32_t blk = fast_div(dst, c.a->div_block), off = dst - blk * nb;
    const uint32_t word = ld(&set_touched(c.d, set_of(c.d, c.tick))[blk * block_words(nb) + off / 32]);
    in.touched_epoch = (word >> (off & 31)) & 1u ? c.tick + 1 : 0u;
}

// The destination's state: quarters 0, 2 and 3 of its record (membrane,
// branches, refractory tick, selected epoch), its block's selection and its
// threshold and excitability.
__device__ __forceinline__ void load_destination(SlotInputs& in, const StepCtx& c, uint32_t dst) {
    static_assert(kNMembrane == 0 && kNBranch0 + BR_TEMP == 8 && kNBranch0 + BR_GATE == 9 && kNRefractory == 11 &&
                      kNSelected == 13,
                  "record layout");
    const LaneDesc& d = c.d;
    const uint32_t blk = fast_div(dst, c.a->div_block);
    const __amdgpu_buffer_rsrc_t rec = neuron_rsrc(d, c.a->cfg.neuron_count);
    const f32x4 q0 = ld_quarter(rec, dst, 0), q2 = ld_quarter(rec, dst, 2), q3 = ld_quarter(rec, dst, 3);
    in.selected_epoch = __float_as_uint(q3.y);
    in.refractory_until = __float_as_uint(q2.w);
    in.temporal = q2.x;
    in.gate_acc = q2.y;
    in.block_epoch = ld(&d.block_epoch[blk]);
    in.block_cut = ld(&d.block_cutoff[blk]);
    in.membrane = q0.x;
    in.threshold = ld(&d.p.threshold[dst]);
    in.excitability = c.a->m.excitability[dst];
}

__device__ __forceinline__ bool finish_slot(const StepCtx& c, const SlotInputs& in, float LEO_GLOBAL* trace,
                                            uint32_t slot, uint8_t br, float pop_cutoff, float& eligibility) {
    const LeoConfig& cfg = c.a->cfg;
    const uint32_t tick = c.tick;
    float bs = in.bs, ms = in.ms, fs = in.fs, as0 = in.as0, as1 = in.as1, as2 = in.as2;
    const uint32_t el = tick - in.last;
    if (el > 0) {
        const StateDecays k = decays_at(cfg, el);
        bs *= k.branch;
        ms *= k.membrane;
        fs *= k.fatigue;
        as0 *= k.fast;
        as1 *= k.medium;
        as2 *= k.slow;
    }
    const bool touched = in.touched_epoch == tick + 1;
    const bool selected = in.selected_epoch == tick + 1;
    float elig;
    if (!touched || in.refractory_until > tick) {
        elig = in.e * cfg.eligibility_decay;
    } else {
        const float jac = branch_jacobian(br, in.excitability, in.temporal, in.gate_acc);
        // the destination's selection surrogate (runtime.rs:787-803), a pure
        // function of its state after selection, evaluated where it is used
        const float block_cutoff = in.block_epoch == tick + 1 ? in.block_cut : 0.0f;
        const float sur =
            surrogate_value(cfg, false, in.membrane - in.threshold, maxnum(block_cutoff, pop_cutoff), selected);
        const float asum = as0 + as1 + as2;
        ms = ms + jac * bs - fs - asum;
        elig = sur * ms;
    }
    if (touched && selected) {
        fs += cfg.fatigue_gain * elig;
        as0 += cfg.adaptation_fast_gain * elig;
        as1 += cfg.adaptation_medium_gain * elig;
        as2 += cfg.adaptation_slow_gain * elig;
    }
    // the record in two 16-byte stores (the last tick moves only when it was behind)
    f32x4 LEO_GLOBAL* rec = reinterpret_cast<f32x4 LEO_GLOBAL*>(trace + static_cast<uint64_t>(slot) * kTraceWords);
    rec[0] = f32x4{bs, ms, fs, as0};
    rec[1] = f32x4{as1, as2, elig, __uint_as_float(el > 0 ? tick : in.last)};
    float mag = maxnum(maxnum(maxnum(fabsf(bs), fabsf(ms)), fabsf(fs)), fabsf(elig));
    mag = maxnum(mag, fabsf(as0));
    mag = maxnum(mag, fabsf(as1));
    mag = maxnum(mag, fabsf(as2));
    eligibility = elig;
    return mag > cfg.eligibility_epsilon;
}

// Where a plasticity step lists its learning slots and claims their
// destinations (runtime.rs:1214-1243).
struct LearnOut {
    uint32_t LEO_GLOBAL* list;   // learning slots of this list
    uint32_t LEO_GLOBAL* count;
    bool plastic;                // the step commits recurrent/input plasticity
    uint32_t claimed;            // this thread's destinations claimed
    uint32_t listed;             // this thread's learning slots listed
};

// Wave-aggregated append of K predicates per lane (every lane active): one
// atomic for the wave; lane order within each predicate, predicate k's
// entries before predicate k+1's.
template <uint32_t K>
__device__ __forceinline__ void wave_append_k(uint32_t LEO_GLOBAL* counter, const bool (&p)[K], uint32_t (&pos)[K]) {
    unsigned long long m[K];
    uint32_t total = 0;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        m[k] = __ballot(p[k]);
        total += static_cast<uint32_t>(__popcll(m[k]));
    }
    uint32_t base = 0;
    if (total != 0 && __lane_id() == 0) base = atomicAdd(counter, total);
    base = __builtin_amdgcn_readfirstlane(base);
    const unsigned long long below = (1ULL << __lane_id()) - 1ULL;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        pos[k] = base + static_cast<uint32_t>(__popcll(m[k] & below));
        base += static_cast<uint32_t>(__popcll(m[k]));
    }
}

// Eligible slots of one list, K per lane per iteration (their loads in
// flight together: 2 when the list gives each thread a few slots, more when
// it gives each many, as on story lanes with few workgroups); kept slots are
// compacted into the next list. On a
// plasticity step the kept slots whose update can change their weight
// (nonzero eligibility; every kept slot when skip_zero_eligibility is off) are
// listed as learning slots, and their destinations are claimed once each
// with an epoch exchange: the learning signal is computed for exactly those.
// The reference also computes signals for the other destinations (the
// targets of zero-eligibility slots and the active neurons); no update reads
// them.
// Each slot's packed synapse (`edges`) gives its destination and branch in
// one load.
template <uint32_t K>
__device__ __forceinline__ void eligibility_list(const StepCtx& c, float LEO_GLOBAL* trace, uint64_t slots,
                                                 uint8_t LEO_GLOBAL* marks,
                                                 const uint32_t LEO_GLOBAL* cur, uint32_t cur_n,
                                                 uint32_t LEO_GLOBAL* next, uint32_t LEO_GLOBAL* next_count,
                                                 const uint32_t* edges, float pop_cutoff, LearnOut& learn,
                                                 uint32_t gstride) {
    const bool skip_zero = c.a->skip_zero_eligibility != 0;
    const uint32_t lane = __lane_id();
    const __amdgpu_buffer_rsrc_t rsrc = trace_rsrc(trace, slots);
    for (uint32_t base = dealt_index(c, gstride / kThreads) - lane; base < cur_n; base += K * gstride) {
        bool v[K];
        uint32_t sl[K], t[K];
        uint8_t r[K];
        SlotInputs in[K];
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t i = base + k * gstride + lane;
            v[k] = i < cur_n;
            sl[k] = v[k] ? ld(&cur[i]) : 0u;
            t[k] = 0;
            r[k] = 0;
            in[k] = SlotInputs{};
        }
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            if (v[k]) {
                const uint32_t edge = edges[sl[k]];
                t[k] = edge_target(edge);
                r[k] = static_cast<uint8_t>(edge_branch(edge));
                load_slot(in[k], rsrc, sl[k]);
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (v[k]) load_touched(in[k], c, t[k]);
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (v[k] && in[k].touched_epoch == c.tick + 1) load_destination(in[k], c, t[k]);
        float e[K];
        bool kept[K];
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            e[k] = 0.0f;
            kept[k] = v[k] && finish_slot(c, in[k], trace, sl[k], r[k], pop_cutoff, e[k]);
        }
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (v[k] && !kept[k]) marks[sl[k]] = kMarkDropped;
        uint32_t pos[K];
        wave_append_k<K>(next_count, kept, pos);
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (kept[k]) next[pos[k]] = sl[k];
        if (learn.plastic) {  // wave-uniform
            bool l[K];
#pragma unroll
            for (uint32_t k = 0; k < K; ++k) l[k] = kept[k] && (e[k] != 0.0f || !skip_zero);
            wave_append_k<K>(learn.count, l, pos);
#pragma unroll
            for (uint32_t k = 0; k < K; ++k)
                if (l[k]) learn.list[pos[k]] = sl[k];
            bool w[K];
#pragma unroll
            for (uint32_t k = 0; k < K; ++k)
                w[k] = l[k] && atomicExch(nu(c.d, t[k], kNDestEpoch), c.dest_epoch) != c.dest_epoch;
            wave_append_k<K>(&c.ctl->dest_count, w, pos);
#pragma unroll
            for (uint32_t k = 0; k < K; ++k) {
                if (w[k]) c.d.dest_list[pos[k]] = t[k];
                learn.listed += l[k] ? 1u : 0u;
                learn.claimed += w[k] ? 1u : 0u;
            }
        }
    }
}

// Slots per lane and iteration for a list of n slots over gstride threads:
// four once every thread has at least eight slots (two iterations of four
// instead of four of two), else two (wider iterations cost a lane with only a
// few slots more than they save: +0.5 us per supervised canonical step).
template <class F>
__device__ __forceinline__ void eligibility_width(uint32_t n, uint32_t gstride, F&& walk) {
    if (n >= 8u * gstride) walk(std::integral_constant<uint32_t, 4>{});
    else walk(std::integral_constant<uint32_t, 2>{});
}

// The slots are dealt over the threads of the first gstride / kThreads
// workgroups (all of them, or all but the readout workgroup).
__device__ __forceinline__ void phase_eligibility(const StepCtx& c, bool plastic, uint32_t gstride) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * cfg.synapses_per_neuron;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint32_t p = c.parity, q = c.parity ^ 1;
    const uint32_t rec_n = ld(&c.ctl->rec_count[p]), in_n = ld(&c.ctl->in_count[p]);
    if (c.part == 0 && threadIdx.x == 0) {
        *counter_word(c, 0, kCScanRec, c.tick) = rec_n;
        *counter_word(c, 0, kCScanIn, c.tick) = in_n;
    }
    const float pop_cutoff = a.redundant_global ? 0.0f : ld(&c.ctl->pop_cutoff);
    LearnOut rec{d.rec_learn, &c.ctl->rec_learn_count, plastic, 0, 0};
    eligibility_width(rec_n, gstride, [&](auto width) {
        eligibility_list<decltype(width)::value>(c, d.rec_trace, NS, d.rec_mark, d.rec_list + p * NS, rec_n,
                                                 d.rec_list + q * NS, &c.ctl->rec_count[q], a.m.rec_edge,
                                                 pop_cutoff, rec, gstride);
    });
    LearnOut in{d.in_learn, &c.ctl->in_learn_count, plastic, rec.claimed, rec.listed};
    eligibility_width(in_n, gstride, [&](auto width) {
        eligibility_list<decltype(width)::value>(c, d.in_trace, NI, d.in_mark, d.in_list + p * NI, in_n,
                                                 d.in_list + q * NI, &c.ctl->in_count[q], a.m.in_edge,
                                                 pop_cutoff, in, gstride);
    });
    if (plastic) {
        count_wave(c, kCDest, c.tick, in.claimed);
        count_wave(c, kCLearn, c.tick, in.listed);
    }
}

// The serial sum of kOutputs values in LDS (runtime.rs:1175-1180 order),
// read sixteen at a time in 16-byte loads (one read at a time would wait out
// the LDS latency on every term).
__device__ __forceinline__ float serial_sum_outputs(const float* v) {
    static_assert(kOutputs == 257, "256 values in sixteen-value groups, then the last");
    const f32x4* v4 = reinterpret_cast<const f32x4*>(v);
    float sum = 0.0f;
    for (uint32_t g = 0; g < 64; g += 4) {
        const f32x4 a = v4[g], b = v4[g + 1], c = v4[g + 2], e = v4[g + 3];
        sum += a.x; sum += a.y; sum += a.z; sum += a.w;
        sum += b.x; sum += b.y; sum += b.z; sum += b.w;
        sum += c.x; sum += c.y; sum += c.z; sum += c.w;
        sum += e.x; sum += e.y; sum += e.z; sum += e.w;
    }
    return sum + v[256];
}

// ---------------------------------------------------------------------------
// Phase 4: post-activation dynamics (runtime.rs:920-938), emission snapshot
// (runtime.rs:1084-1106), and on the last workgroup the readout, softmax and
// errors (runtime.rs:1108-1197, 1205-1206).
// ---------------------------------------------------------------------------
// The readout runs in phase 3, beside the eligibility update, on the last
// workgroup (which selects no blocks); the post phase leaves its record
// fields alone. With a non-binding global cap the active list is still being
// written in that phase, so the readout takes it from the selecting waves'
// winners (block order: the same list); otherwise the global selection has
// written it before the phase's first barrier.
__device__ __forceinline__ void readout(const StepCtx& c, const StepParams& sp, StepShared& sh, uint32_t step_index) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    LaneControl* ctl = c.ctl;
    const uint32_t cap = cfg.max_active_global, E = cfg.context_embedding_dim;
    const uint32_t rs = c.tick % kRing;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const uint32_t wave = wave_index(), lane = __lane_id();
    const uint32_t o1 = threadIdx.x, o2 = threadIdx.x + kThreads;
    const bool has2 = o2 < kOutputs;
    float* lat = sh.aux;
    // Memory rounds: (1) the context count, slots and scales, the bias and
    // the waves' winner totals; (2) the context embeddings; (3) the first 256
    // active ids and activations (into LDS) with this thread's first 16
    // context-projection weights; (4) rows of 32 active neurons at a time.
    // (A load's wait also waits for every load issued before it, so the
    // projection weights, needed last, go out after the embeddings.)
    const bool from_waves = a.redundant_global != 0;
    uint32_t* starts = reinterpret_cast<uint32_t*>(step_lds + 2 * kThreads * 4);
    const uint32_t nwaves = selecting_waves(c);
    const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
    const uint32_t N = cfg.neuron_count, rot = c.tick % N;
    if (threadIdx.x == 0) {
        d.records[step_index].p_target = 0.0f;
        d.records[step_index].predicted = 0;
    }
    // the slots past the count are loaded too (and not used), so that the
    // slots do not wait for the count
    const uint32_t ctx_count = ld(&ctl->ctx_count);
    uint32_t slot[kMaxOrder];
    float scale[kMaxOrder];
#pragma unroll
    for (uint32_t i = 0; i < kMaxOrder; ++i) {
        slot[i] = threadIdx.x < E ? ld(&ctl->ctx_slots[i]) : 0u;
        scale[i] = threadIdx.x < E ? ld(&ctl->ctx_scales[i]) : 0.0f;
    }
    float l1 = ld(&d.p.bias[o1]), l2 = has2 ? ld(&d.p.bias[o2]) : 0.0f;
    const float bias1 = l1, bias2 = l2;
    const uint32_t A = from_waves ? wave_starts(c, sh, starts, nwaves) : ld(&ctl->active_count);
    // context latent (runtime.rs:1120-1136): serial over active slots per
    // dimension
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        float emb[kMaxOrder];
#pragma unroll
        for (uint32_t i = 0; i < kMaxOrder; ++i)
            emb[i] = i < ctx_count && scale[i] > 0.0f ? ld(&d.p.ctx_emb[static_cast<uint64_t>(slot[i]) * E + e]) : 0.0f;
        float v = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < kMaxOrder; ++i)
            if (i < ctx_count && scale[i] > 0.0f) v += emb[i] * scale[i];
        lat[e] = v;
        d.ctx_latent[e] = v;
    }
    constexpr uint32_t kDims = 16;
    float x1[kDims], x2[kDims];
#pragma unroll
    for (uint32_t k = 0; k < kDims; ++k) {
        x1[k] = k < E ? ld(&d.p.ctx_out[o1 * E + k]) : 0.0f;
        x2[k] = k < E && has2 ? ld(&d.p.ctx_out[o2 * E + k]) : 0.0f;
    }
    // logits[o] = bias[o] + sum over active in order of W[n][o]*a_n (+ context
    // once): thread t owns outputs t and t+256; the active ids and
    // activations are staged in LDS 256 at a time, then the rows of 32
    // neurons go out together ahead of the serial adds
    // (ids past the block's end read row 0 and are not added, so the row
    // loads carry no conditions and go out back to back)
    uint32_t* ids = reinterpret_cast<uint32_t*>(step_lds);
    float* acts = reinterpret_cast<float*>(step_lds) + kThreads;
    constexpr uint32_t kRows = 32;
    static_assert(kThreads % kRows == 0, "whole row chunks per block of ids");
    for (uint32_t b0 = 0; b0 < A; b0 += kThreads) {
        const uint32_t bn = min(kThreads, A - b0);
        __syncthreads();  // the previous block's ids are consumed (and the latent is written)
        if (from_waves) {
            uint32_t n = 0;
            float act = 0.0f;
            if (threadIdx.x < bn)
                (void)winner_key(d, starts, nwaves, range, cfg.block_count, cfg.max_active_per_block,
                                 b0 + threadIdx.x, N, rot, &n, &act);
            ids[threadIdx.x] = n;
            if (threadIdx.x < bn) acts[threadIdx.x] = act;
        } else {
            ids[threadIdx.x] = threadIdx.x < bn ? ld(&act_list[b0 + threadIdx.x]) : 0u;
            if (threadIdx.x < bn) acts[threadIdx.x] = ld(&act_val[b0 + threadIdx.x]);
        }
        __syncthreads();
        for (uint32_t r0 = 0; r0 < bn; r0 += kRows) {
            float w1[kRows], w2[kRows];
            uint32_t n[kRows];
            const uint4* ids4 = reinterpret_cast<const uint4*>(ids + r0);
#pragma unroll
            for (uint32_t k = 0; k < kRows / 4; ++k) {
                const uint4 q = ids4[k];
                n[4 * k] = q.x;
                n[4 * k + 1] = q.y;
                n[4 * k + 2] = q.z;
                n[4 * k + 3] = q.w;
            }
#pragma unroll
            for (uint32_t k = 0; k < kRows; ++k) {
                const float* row = d.p.out_w + static_cast<uint64_t>(n[k]) * kOutStride;
                w1[k] = ld(&row[o1]);
                w2[k] = has2 ? ld(&row[o2]) : 0.0f;
            }
            float av[kRows];
            const f32x4* acts4 = reinterpret_cast<const f32x4*>(acts + r0);
#pragma unroll
            for (uint32_t k = 0; k < kRows / 4; ++k) {
                const f32x4 q = acts4[k];
                av[4 * k] = q.x;
                av[4 * k + 1] = q.y;
                av[4 * k + 2] = q.z;
                av[4 * k + 3] = q.w;
            }
#pragma unroll
            for (uint32_t k = 0; k < kRows; ++k) {
                if (r0 + k < bn) {  // rows in order, the ragged last chunk stops at A
                    l1 += w1[k] * av[k];
                    l2 += w2[k] * av[k];
                }
            }
        }
    }
    __syncthreads();  // the latent is visible (A = 0 skips the loop's barriers)
    // the context contribution (read from the latent in sh.aux) is computed
    // before the neural-loss pass reuses sh.aux, and added after it
    float c1 = 0.0f, c2 = 0.0f;
    if (ctx_count > 0) {
        for (uint32_t e0 = 0; e0 < E; e0 += kDims) {
            if (e0 > 0) {
#pragma unroll
                for (uint32_t k = 0; k < kDims; ++k) {
                    x1[k] = e0 + k < E ? ld(&d.p.ctx_out[o1 * E + e0 + k]) : 0.0f;
                    x2[k] = e0 + k < E && has2 ? ld(&d.p.ctx_out[o2 * E + e0 + k]) : 0.0f;
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < kDims; ++k) {
                if (e0 + k >= E) break;
                c1 += x1[k] * lat[e0 + k];
                c2 += x2[k] * lat[e0 + k];
            }
        }
    }
    if (sp.flags & kStepNeuralLoss) {
        // loss_from_logits on the neural logits, before the context is added
        // (runtime.rs:1119, 1151-1167): f32::max fold, exp, serial sum
        float nm = has2 ? maxnum(l1, l2) : l1;
        for (int off = 32; off > 0; off >>= 1) nm = maxnum(nm, __shfl_xor(nm, off));
        if (lane == 0) sh.redf[wave] = nm;
        __syncthreads();
        nm = sh.redf[0];
        for (uint32_t w = 1; w < kWavesPerGroup; ++w) nm = maxnum(nm, sh.redf[w]);
        sh.aux[o1] = glibc_expf_nonpositive(l1 - nm);
        if (has2) sh.aux[o2] = glibc_expf_nonpositive(l2 - nm);
        __syncthreads();
        StepRecord LEO_GLOBAL& rec = d.records[step_index];
        if (threadIdx.x == 0) {
            const float sum = serial_sum_outputs(sh.aux);
            rec.neural_max = nm;
            rec.neural_sum = sum;
        }
        if (sp.target_index >= 0 && static_cast<uint32_t>(sp.target_index) == o1) rec.neural_target = l1;
        if (sp.target_index >= 0 && has2 && static_cast<uint32_t>(sp.target_index) == o2) rec.neural_target = l2;
        __syncthreads();
    }
    if (ctx_count > 0) {
        l1 += c1;
        l2 += c2;
    }
    sh.err[o1] = l1;
    d.logits[o1] = l1;
    if (has2) {
        sh.err[o2] = l2;
        d.logits[o2] = l2;
    }
    // maximum: order-independent, reduced across the workgroup
    float mx = has2 ? maxnum(l1, l2) : l1;
    for (int off = 32; off > 0; off >>= 1) mx = maxnum(mx, __shfl_xor(mx, off));
    if (lane == 0) sh.redf[wave] = mx;
    __syncthreads();
    mx = sh.redf[0];
    for (uint32_t w = 1; w < kWavesPerGroup; ++w) mx = maxnum(mx, sh.redf[w]);
    // exp in parallel (glibc expf), then the serial sum of runtime.rs:1175-1180
    sh.aux[o1] = glibc_expf_nonpositive(l1 - mx);
    if (has2) sh.aux[o2] = glibc_expf_nonpositive(l2 - mx);
    __syncthreads();
    if (threadIdx.x == 0) sh.redf[0] = serial_sum_outputs(sh.aux);
    __syncthreads();
    const float sum = sh.redf[0];
    const bool uniform = !finitef(sum) || sum <= 0.0f;
    const float p1 = uniform ? 1.0f / static_cast<float>(kOutputs) : sh.aux[o1] / sum;
    const float p2 = has2 ? (uniform ? 1.0f / static_cast<float>(kOutputs) : sh.aux[o2] / sum) : 0.0f;
    d.probs[o1] = p1;
    d.errors[o1] = static_cast<int32_t>(o1) == sp.target_index ? p1 - 1.0f : p1;
    if (has2) {
        d.probs[o2] = p2;
        d.errors[o2] = static_cast<int32_t>(o2) == sp.target_index ? p2 - 1.0f : p2;
    }
    // argmax: largest probability, first index among equals (runtime.rs:1190-1197);
    // probabilities are non-negative, so their bit patterns order them
    unsigned long long best = (static_cast<unsigned long long>(__float_as_uint(p1)) << 32) | (0xffffffffu - o1);
    if (has2) {
        const unsigned long long k2 = (static_cast<unsigned long long>(__float_as_uint(p2)) << 32) | (0xffffffffu - o2);
        best = k2 > best ? k2 : best;
    }
    best = wave_max_u64(best);
    __syncthreads();
    if (lane == 0) sh.red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < kWavesPerGroup; ++w) best = sh.red[w] > best ? sh.red[w] : best;
        best = sh.red[0] > best ? sh.red[0] : best;
        StepRecord& rec = d.records[step_index];
        rec.predicted = 0xffffffffu - static_cast<uint32_t>(best);
    }
    if (sp.target_index >= 0 && (threadIdx.x == static_cast<uint32_t>(sp.target_index) ||
                                 (has2 && o2 == static_cast<uint32_t>(sp.target_index))))
        d.records[step_index].p_target = threadIdx.x == static_cast<uint32_t>(sp.target_index) ? p1 : p2;
    __syncthreads();  // thread 0 has read the argmax partials in sh.red
    if (sp.flags & kStepLearn) {
        // The learning phase's bias update (runtime.rs:1290-1298), checked
        // ahead: the reference adds the outputs' deltas in order and stops at
        // the first bias that becomes non-finite (after writing it), before
        // the context, synapse and homeostasis updates. The learning phase
        // reads the first such output from the control word.
        const float olr = cfg.output_learning_rate, ss = sp.supervised_strength, mu = cfg.max_update;
        const float e1 = static_cast<int32_t>(o1) == sp.target_index ? p1 - 1.0f : p1;
        const float e2 = static_cast<int32_t>(o2) == sp.target_index ? p2 - 1.0f : p2;
        uint32_t fail = kNoFail;
        if (!finitef(bias1 + bounded(-olr * ss * e1, mu))) fail = o1;
        else if (has2 && !finitef(bias2 + bounded(-olr * ss * e2, mu))) fail = o2;
        for (int off = 32; off > 0; off >>= 1) fail = min(fail, static_cast<uint32_t>(__shfl_xor(static_cast<int>(fail), off)));
        if (lane == 0) sh.red[wave] = fail;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (uint32_t w = 1; w < kWavesPerGroup; ++w) fail = min(fail, static_cast<uint32_t>(sh.red[w]));
            ctl->bias_fail = fail;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void phase_post(const StepCtx& c, const StepParams& sp, uint32_t step_index, StepShared& sh) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    const uint32_t S = cfg.synapses_per_neuron, cap = cfg.max_active_global;
    const uint32_t rs = c.tick % kRing;
    const uint32_t A = ld(&c.ctl->active_count);
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const uint32_t total = A + A * S;
    const uint32_t refractory = c.tick + cfg.refractory_ticks + 1;
    uint32_t inhibitory = 0;
    for (uint32_t item = dealt_index(c, c.P); item < total; item += c.gstride) {
        if (item < A) {
            const uint32_t n = ld(&act_list[item]);
            const float act = ld(nf(d, n, kNActivation));
            inhibitory += a.m.neuron_type[n] != 0 ? 1u : 0u;
            (*nf(d, n, kNFatigue)) = ld(nf(d, n, kNFatigue)) + cfg.fatigue_gain * act;
            (*nf(d, n, kNAdapt0)) = ld(nf(d, n, kNAdapt0)) + cfg.adaptation_fast_gain * act;
            (*nf(d, n, kNAdapt0 + 1)) = ld(nf(d, n, kNAdapt0 + 1)) + cfg.adaptation_medium_gain * act;
            (*nf(d, n, kNAdapt0 + 2)) = ld(nf(d, n, kNAdapt0 + 2)) + cfg.adaptation_slow_gain * act;
            (*nf(d, n, kNMembrane)) = ld(nf(d, n, kNMembrane)) - ld(&d.p.threshold[n]) * cfg.membrane_reset_fraction;
            (*nu(d, n, kNRefractory)) = refractory;
        } else {
            const uint32_t local = item - A;
            const uint32_t r = fast_div(local, a.div_synapses), j = local - r * S;
            const uint64_t rb = static_cast<uint64_t>(rs) * cap + r;
            const uint64_t slot = static_cast<uint64_t>(ld(&act_list[r])) * S + j;
            d.ring_value[rb * S + j] = ld(&act_val[r]) * ld(&d.p.rec_weight[slot]);
            d.ring_edge[rb * S + j] = a.m.rec_edge[slot];
        }
    }
    count_wave(c, kCInhibitory, c.tick, inhibitory);
    if (threadIdx.x == 0) {  // the next deliveries read this tick's ring entry from LDS
        sh.ring_tick[rs] = c.tick;
        sh.ring_count[rs] = A;
        sh.ring_early[rs] = 0;
    }
    const uint32_t readout_wg = c.P - 1;
    if (c.part == readout_wg) {
        const uint32_t supra = threadIdx.x < kWaveSize ? counter_total(c, kCSupra, c.tick) : 0u;
        if (threadIdx.x == 0) {
            LaneControl LEO_GLOBAL* ctl = c.ctl;
            // the loads go out together, before any store
            const float pi = ld(&ctl->population_inhibition);
            const uint32_t selected = ld(&ctl->block_selected);
            const uint32_t clipped = ld(&ctl->clipped), cells = ld(&ctl->ctx_count);
            const uint32_t probes = ld(&ctl->ctx_probes), applied = ld(&ctl->ctx_applied);
            const uint32_t rec_n = ld(&ctl->rec_count[c.parity]), in_n = ld(&ctl->in_count[c.parity]);
            StepRecord LEO_GLOBAL& rec = d.records[step_index];
            if (!(sp.flags & kStepOutput)) {  // an output step's readout has set them
                rec.p_target = 0.0f;
                rec.predicted = 0;
            }
            rec.population_inhibition = pi;
            rec.active = A;
            rec.suprathreshold = supra;
            rec.block_selected = selected;
            rec.clipped = clipped;
            rec.context_cells = cells;
            rec.context_probes = probes;
            rec.context_applied = applied;
            rec.eligible_rec = rec_n;
            rec.eligible_in = in_n;
            rec.error_code = 0;
        }
    }
}

// ---------------------------------------------------------------------------
// Phase 5: learning destinations and signals (runtime.rs:1214-1263). Each wave
// claims destinations, queues them, and computes their serial 257-term dot
// products 64 at a time from output rows staged through LDS (coalesced row
// loads).
// ---------------------------------------------------------------------------
// Device-scope 16-byte loads through a buffer resource (cache policy sc1: the
// load misses the CU's L1 like ld()); the resource is wave-uniform and covers
// `bytes` from `base` (loads beyond it return 0).
// Serial 257-term dot of one output row with the errors, in output order
// (runtime.rs:1245-1250).
// Learning signals of up to 64 destinations, one per lane (`dst` on lanes
// below `count`; every lane of the wave calls): the output rows are streamed
// through the wave's LDS stage one 128-byte line at a time, 8 whole lines per
// load instruction, with the next two lines in flight while the current one
// is summed; each lane then adds its row's 257 products in the reference's
// order (runtime.rs:1214-1263).
__device__ __forceinline__ float signal_rows(__amdgpu_buffer_rsrc_t rows, uint32_t dst, uint32_t count, const float* err,
                                             float* stage) {
    constexpr uint32_t kLines = kEndIndex / 32;  // 128-byte lines before the end-class weight
    const uint32_t lane = __lane_id();
    const uint32_t seg = lane & 7, sub = lane >> 3;
    // this lane loads 16 bytes of rows sub, 8 + sub, ..., 56 + sub
    uint32_t row_of[8];
    bool live[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t row = 8 * k + sub;
        live[k] = row < count;
        row_of[k] = static_cast<uint32_t>(__shfl(static_cast<int>(dst), static_cast<int>(row)));
    }
    const float tail = lane < count ? ld4_record(rows, dst, 4 * kEndIndex) : 0.0f;
    // two lines in flight (even lines in v, odd lines in w; the unrolled loop
    // names the buffers statically, so no register copy waits for a load)
    static_assert(kLines % 2 == 0, "lines are taken in pairs");
    f32x4 v[8], w[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        v[k] = live[k] ? ld16_record(rows, row_of[k], seg * 16) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        w[k] = live[k] ? ld16_record(rows, row_of[k], seg * 16 + 128) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float acc = 0.0f;
#pragma unroll
    for (uint32_t line = 0; line < kLines; ++line) {
        f32x4(&cur)[8] = (line & 1) ? w : v;
        wave_sync();
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            float* st = stage + (8 * k + sub) * kStageRowFloats + seg * 4;
            st[0] = cur[k].x;
            st[1] = cur[k].y;
            st[2] = cur[k].z;
            st[3] = cur[k].w;
        }
        wave_sync();
        if (line + 2 < kLines) {
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k)
                cur[k] = live[k] ? ld16_record(rows, row_of[k], seg * 16 + (line + 2) * 128)
                                 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (lane < count) {
            const float* r = stage + lane * kStageRowFloats;
            const float* e = err + line * 32;
#pragma unroll
            for (uint32_t o = 0; o < 32; ++o) acc += r[o] * e[o];
        }
    }
    acc += tail * err[kEndIndex];
    return acc;
}

// The listed destinations' signals (runtime.rs:1245-1250), 64 at a time per
// wave, the batches dealt round-robin over every wave of the lane.
__device__ __forceinline__ void phase_signals(const StepCtx& c, StepShared& sh) {
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = c.a->cfg;
    // one round: the errors, the destination count and this wave's first
    // batch of the list (read before the count is known; entries past it are
    // masked below)
    const uint32_t wave = wave_index(), lane = __lane_id();
    // batches of 64 destinations dealt to the workgroups in turn
    const uint32_t waves = c.P * kWavesPerGroup, b0 = wave * c.P + c.part;
    const uint32_t N = cfg.neuron_count;
    const uint32_t count = ld(&c.ctl->dest_count);
    const uint32_t first_at = b0 * kWaveSize + lane;
    const uint32_t first_dst = first_at < N ? ld(&d.dest_list[first_at]) : 0u;
    for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) sh.err[o] = ld(&d.errors[o]);
    __syncthreads();
    // rows addressed by index (N records of kOutStride floats)
    const __amdgpu_buffer_rsrc_t rows = record_rsrc(d.p.out_w, kOutStride * 4, N);
    float* stage = reinterpret_cast<float*>(step_lds + static_cast<size_t>(wave) * wave_lds_bytes(cfg.neurons_per_block));
    for (uint32_t b = b0; b * kWaveSize < count; b += waves) {
        const uint32_t n = min(kWaveSize, count - b * kWaveSize);
        const uint32_t dst = lane < n ? (b == b0 ? first_dst : ld(&d.dest_list[b * kWaveSize + lane])) : 0u;
        const float sig = signal_rows(rows, dst, n, sh.err, stage);
        if (lane < n) d.learning_signal[dst] = sig;
    }
}

// ---------------------------------------------------------------------------
// Phase 6: output/bias/context updates (runtime.rs:1265-1303, 1318-1384),
// recurrent and input synapses (runtime.rs:1451-1523), inhibitory
// homeostasis (runtime.rs:1525-1565) and threshold homeostasis
// (runtime.rs:1567-1593).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float inhibitory_step(const LeoConfig& cfg, float w, float src_act, float tgt_act, float strength) {
    const float err = tgt_act - cfg.target_activity;
    const float delta = bounded(-cfg.inhibitory_learning_rate * strength * src_act * err, cfg.max_update);
    return clampf(w + delta, cfg.weight_min, 0.0f);
}

__device__ __forceinline__ void context_update(const StepCtx& c, const StepParams& sp, StepShared& sh,
                                               uint32_t step_index) {
    const LeoConfig& cfg = c.a->cfg;
    const LaneDesc& d = c.d;
    LaneControl* ctl = c.ctl;
    const uint32_t E = cfg.context_embedding_dim, count = ld(&ctl->ctx_count);
    const float lr = cfg.context_learning_rate, mu = cfg.max_update, wmin = cfg.weight_min, wmax = cfg.weight_max;
    const float strength = sp.supervised_strength;
    float* grad = sh.aux;
    // serial in output order; the weights of 32 outputs are loaded at a time
    constexpr uint32_t kChunk = 32;
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        float g = 0.0f;
        for (uint32_t o0 = 0; o0 < kOutputs; o0 += kChunk) {
            float w[kChunk];
#pragma unroll
            for (uint32_t k = 0; k < kChunk; ++k) w[k] = o0 + k < kOutputs ? ld(&d.p.ctx_out[(o0 + k) * E + e]) : 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < kChunk; ++k)
                if (o0 + k < kOutputs) g += w[k] * sh.err[o0 + k];
        }
        grad[e] = g;
    }
    __syncthreads();
    if (threadIdx.x == 0) ctl->ctx_out_dirty = 1;
    // four elements per thread at a time, their loads together
    constexpr uint32_t kBatch = 4;
    for (uint32_t i0 = threadIdx.x; i0 < kOutputs * E; i0 += kBatch * kThreads) {
        float old[kBatch], latent[kBatch];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) {
            const uint32_t i = i0 + k * kThreads;
            old[k] = i < kOutputs * E ? ld(&d.p.ctx_out[i]) : 0.0f;
            latent[k] = i < kOutputs * E ? ld(&d.ctx_latent[i % E]) : 0.0f;
        }
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) {
            const uint32_t i = i0 + k * kThreads;
            if (i >= kOutputs * E) continue;
            const float gradient = sh.err[i / E] * latent[k];
            const float delta = bounded(-lr * strength * gradient, mu);
            const float updated = clampf(old[k] + delta, wmin, wmax);
            if (!finitef(updated)) set_step_error(ctl, kErrContextProjection, step_index);
            d.p.ctx_out[i] = updated;
        }
    }
    for (uint32_t i = threadIdx.x; i < count * E; i += kThreads) {
        const uint32_t k = i / E, e = i % E;
        const uint64_t slot = ld(&ctl->ctx_slots[k]);
        const float gradient = ld(&ctl->ctx_scales[k]) * grad[e];
        const float delta = bounded(-lr * strength * gradient, mu);
        const float updated = clampf(ld(&d.p.ctx_emb[slot * E + e]) + delta, wmin, wmax);
        if (!finitef(updated)) set_step_error(ctl, kErrContextEmbedding, step_index);
        d.p.ctx_emb[slot * E + e] = updated;
    }
    for (uint32_t k = threadIdx.x; k < count; k += kThreads) {
        const uint32_t slot = ld(&ctl->ctx_slots[k]);
        mark_bit(d.ch_ctx, slot);
        const uint32_t obs = ld(&d.p.ctx_obs[slot]);
        d.p.ctx_obs[slot] = obs == 0xffffffffu ? obs : obs + 1;
    }
    __syncthreads();
}

__device__ __forceinline__ void phase_learn(const StepCtx& c, const StepParams& sp, StepShared& sh,
                                            uint32_t step_index) {
    const KernelArgs& a = *c.a;
    const LaneDesc& d = c.d;
    const LeoConfig& cfg = a.cfg;
    LaneControl* ctl = c.ctl;
    const uint32_t S = cfg.synapses_per_neuron, cap = cfg.max_active_global;
    const uint64_t NS = static_cast<uint64_t>(cfg.neuron_count) * S;
    const uint64_t NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint32_t tick = c.tick;
    const bool learn = (sp.flags & kStepLearn) != 0;
    const bool plastic = learn && sp.plasticity_scale > 0.0f;
    const uint32_t A = ld(&ctl->active_count);
    const uint32_t rs = tick % kRing;
    const uint32_t* act_list = d.ring_active + static_cast<uint64_t>(rs) * cap;
    const float* act_val = d.ring_act + static_cast<uint64_t>(rs) * cap;
    const float mu = cfg.max_update, wmin = cfg.weight_min, wmax = cfg.weight_max;
    uint32_t bias_fail = kNoFail;
    if (learn) {
        // the readout workgroup updates the bias and the context projection;
        // the other workgroups share the output rows and the synapse slots
        const uint32_t sharers = c.P > 1 ? c.P - 1 : 1;
        const uint32_t first = c.part < sharers ? dealt_index(c, sharers) : ~0u, stride = sharers * kThreads;
        // the learning-slot list lengths and this thread's first learning
        // slots go out with the errors (slots read before the lengths are
        // known are masked by the loops below)
        const uint32_t* rec_cur = d.rec_learn;
        const uint32_t* in_cur = d.in_learn;
        const uint32_t rec_n = plastic ? ld(&ctl->rec_learn_count) : 0u;
        const uint32_t in_n = plastic ? ld(&ctl->in_learn_count) : 0u;
        const uint32_t rec_first = plastic && first < NS ? ld(&rec_cur[first]) : 0u;
        const uint32_t in_first = plastic && first < NI ? ld(&in_cur[first]) : 0u;
        for (uint32_t o = threadIdx.x; o < kOutputs; o += kThreads) sh.err[o] = ld(&d.errors[o]);
        // an output whose bias becomes non-finite ends the step's learning
        // after the output rows and the bias up to it (runtime.rs:1296-1300)
        bias_fail = ld(&ctl->bias_fail);
        __syncthreads();
        const float ss = sp.supervised_strength;
        const float olr = cfg.output_learning_rate;
        // output rows of active neurons
        const uint32_t out_items = A * kOutputs;
        for (uint32_t item = first; item < out_items; item += stride) {
            const uint32_t r = item / kOutputs, o = item % kOutputs;
            const uint32_t n = ld(&act_list[r]);
            const float act = ld(&act_val[r]);
            if (o == 0) mark_bit(d.ch_out, n);
            const float raw = -olr * ss * sh.err[o] * act;
            float* w = d.p.out_w + static_cast<uint64_t>(n) * kOutStride + o;
            *w = clampf(ld(w) + bounded(raw, mu), wmin, wmax);
        }
        // bias and context projection on the readout workgroup
        if (c.part == c.P - 1) {
            for (uint32_t o = threadIdx.x; o <= min(bias_fail, kOutputs - 1); o += kThreads) {
                const float raw = -olr * ss * sh.err[o];
                const float b = ld(&d.p.bias[o]) + bounded(raw, mu);
                d.p.bias[o] = b;
            }
            if (threadIdx.x == 0) {
                ctl->bias_dirty = 1;
                if (bias_fail != kNoFail) set_step_error(ctl, kErrBias, step_index);
            }
            if (bias_fail == kNoFail && ld(&ctl->ctx_applied) && ld(&ctl->ctx_count) > 0)
                context_update(c, sp, sh, step_index);
        }
        if (plastic && bias_fail == kNoFail) {
            const float cs = ss * sp.plasticity_scale;
            const float lr = cfg.recurrent_learning_rate;
            for (uint32_t i = first; i < rec_n; i += stride) {
                const uint32_t slot = i == first ? rec_first : ld(&rec_cur[i]);
                const uint32_t dst = a.m.rec_target[slot];
                const uint32_t src = fast_div(slot, a.div_synapses);
                const float e = ld(&d.rec_trace[static_cast<uint64_t>(slot) * kTraceWords + kTEligibility]);
                const float gradient = ld(&d.learning_signal[dst]) * e;
                const float delta = bounded(-lr * cs * gradient, mu);
                const float old_w = ld(&d.p.rec_weight[slot]);
                float nw = clampf(old_w + delta, wmin, wmax);
                const bool excitatory = a.m.neuron_type[src] == 0;
                nw = excitatory ? max_zero(nw) : min_zero(nw);
                if (!finitef(nw)) set_step_error(ctl, kErrRecurrent, step_index);
                bool changed = nw != old_w;
                if (!excitatory && ld(nu(d, src, kNSelected)) == tick + 1) {
                    const float tgt_act = ld(nf(d, dst, kNActivation)) > 0.0f ? 1.0f : 0.0f;
                    const float nw2 = inhibitory_step(cfg, nw, ld(nf(d, src, kNActivation)), tgt_act, sp.strength);
                    if (!finitef(nw2)) set_step_error(ctl, kErrInhibitory, step_index);
                    changed = changed || nw2 != nw;
                    nw = nw2;
                }
                if (changed) mark_bit(d.ch_rec, slot);
                d.p.rec_weight[slot] = nw;
            }
            for (uint32_t i = first; i < in_n; i += stride) {
                const uint32_t slot = i == first ? in_first : ld(&in_cur[i]);
                const uint32_t dst = a.m.in_target[slot];
                const float e = ld(&d.in_trace[static_cast<uint64_t>(slot) * kTraceWords + kTEligibility]);
                const float gradient = ld(&d.learning_signal[dst]) * e;
                const float delta = bounded(-lr * cs * gradient, mu);
                const float old_w = ld(&d.p.in_weight[slot]);
                const float nw = clampf(old_w + delta, 0.0f, wmax);
                if (!finitef(nw)) set_step_error(ctl, kErrInput, step_index);
                if (nw != old_w) mark_bit(d.ch_in, slot);
                d.p.in_weight[slot] = nw;
            }
        }
        // inhibitory homeostasis on the rows of active inhibitory sources not
        // already handled with their learning slot above (a kept eligible
        // slot with nonzero eligibility, or any kept slot without the zero
        // skip)
        const uint32_t inh_items = bias_fail == kNoFail ? A * S : 0u;
        const bool skip_zero = a.skip_zero_eligibility != 0;
        for (uint32_t item = first; item < inh_items; item += stride) {
            const uint32_t r = fast_div(item, a.div_synapses), j = item - r * S;
            const uint32_t src = ld(&act_list[r]);
            if (a.m.neuron_type[src] == 0) continue;
            const uint64_t slot = static_cast<uint64_t>(src) * S + j;
            if (plastic && ld(&d.rec_mark[slot]) == kMarkListed &&
                (!skip_zero || ld(&d.rec_trace[slot * kTraceWords + kTEligibility]) != 0.0f))
                continue;
            const uint32_t dst = a.m.rec_target[slot];
            const float tgt_act = ld(nf(d, dst, kNActivation)) > 0.0f ? 1.0f : 0.0f;
            const float old_w = ld(&d.p.rec_weight[slot]);
            const float nw = inhibitory_step(cfg, old_w, ld(nf(d, src, kNActivation)), tgt_act, sp.strength);
            if (!finitef(nw)) set_step_error(ctl, kErrInhibitory, step_index);
            if (nw != old_w) mark_bit(d.ch_rec, static_cast<uint32_t>(slot));
            d.p.rec_weight[slot] = nw;
        }
    }
    if (!(sp.flags & kStepFrozen)) {
        const float N = static_cast<float>(cfg.neuron_count);
        const float pop_err = static_cast<float>(A) / N - cfg.target_activity;
        // the touched list is kept in one segment per selecting wave (at the
        // first neuron of its block range): one wave per segment
        const uint32_t nwaves = selecting_waves(c), lane = __lane_id();
        const uint32_t range = (cfg.block_count + nwaves - 1) / nwaves;
        for (uint32_t w = c.part * kWavesPerGroup + wave_index(); w < nwaves; w += c.P * kWavesPerGroup) {
            const uint32_t count = ld(&d.wave_touched[w]);
            const uint32_t first = min(cfg.block_count, w * range) * cfg.neurons_per_block;
            for (uint32_t i = lane; i < count; i += kWaveSize) {
                const uint32_t n = ld(&d.touched_list[first + i]);
                {  // the bitmap word this trace step kept for its eligibility update
                    const uint32_t nb = cfg.neurons_per_block;
                    const uint32_t blk = fast_div(n, a.div_block), off = n - blk * nb;
                    set_touched(d, set_of(d, c.tick))[blk * block_words(nb) + off / 32] = 0u;
                }
                if (bias_fail != kNoFail) continue;  // the failed step ends before homeostasis
                const float local = ld(nf(d, n, kNActivation)) > 0.0f ? 1.0f : 0.0f;
                const float local_err = local - cfg.target_activity;
                const float delta = cfg.threshold_homeostasis_rate * (local_err + pop_err);
                const float old_t = ld(&d.p.threshold[n]);
                const float nt = clampf(old_t + delta, 0.05f, 2.0f);
                if (nt != old_t) mark_bit(d.ch_threshold, n);
                d.p.threshold[n] = nt;
            }
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
    // a section inside a phase, [from, to), added to slot `slot`
    __device__ void section(uint32_t slot, unsigned long long from, unsigned long long to) { out[slot] += to - from; }
};

template <bool kProfile>
__device__ __forceinline__ bool phase_barrier(const StepCtx& c, uint32_t& target, uint32_t spin_limit,
                                              PhaseClock& clock, uint32_t phase, const uint32_t* carries = nullptr,
                                              uint32_t* sums = nullptr) {
    unsigned long long arrived = 0;
    const bool timer = kProfile && c.part == c.a->profile_part && threadIdx.x == 0;
    if (timer) clock.arrive(phase, arrived);
    const bool ok = lane_barrier(c.d, c.part, c.P, target, spin_limit, c.local, carries, sums);
    if (timer) clock.release(phase, arrived);
    return ok;
}

// Step loop. Phases (barriers): deliver (+context) | fold+select | active list +
// eligibility + readout (on the last workgroup) | post (+ signals on a
// plasticity step) | learning. Frozen steps stop after the post phase; a
// binding global cap inserts the global sort before the eligibility update
// and the readout.
//
// Workgroup b serves lane b % lane_stride (lane_stride is a multiple of the 8
// XCDs, and workgroups are dealt to XCDs round-robin, so a lane's workgroups
// normally share one XCD); workgroups of padding lanes exit at once. Before the
// first step the lane checks where its workgroups actually run and uses the
// cheap XCD-local barrier only if they all share one XCD.
// Copies a workgroup-uniform descriptor word by word into scalar registers.
__device__ __forceinline__ LaneDesc load_uniform(const LaneDesc* p) {
    static_assert(sizeof(LaneDesc) % 4 == 0, "descriptor is made of 32-bit words");
    uint32_t w[sizeof(LaneDesc) / 4];
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(LaneDesc) / 4; ++i) w[i] = __builtin_amdgcn_readfirstlane(src[i]);
    LaneDesc out;
    __builtin_memcpy(&out, w, sizeof(LaneDesc));
    return out;
}

// kFrozenOnly: every step of the launch is a frozen step without output and
// the global cap cannot bind (the host checks both); the steps' flags say so
// at compile time, so the kernel carries none of the learning, readout,
// eligibility and global-selection code (a smaller program and register set
// for the serial replay prefix).
template <bool kProfile, bool kFrozenOnly>
__device__ __forceinline__ void lane_steps(const KernelArgs& args) {
    __shared__ StepShared sh;
    const uint32_t stride = args.lane_stride, P = args.wgs_per_lane;
    const uint32_t lane = blockIdx.x % stride;
    if (lane >= args.lane_count) return;
    StepCtx c;
    c.a = &args;
    c.d = load_uniform(&args.lanes[lane]);  // a private copy: its pointers stay in scalar registers
    c.ctl = c.d.ctl;
    c.part = blockIdx.x / stride;
    c.P = P;
    c.gtid = c.part * kThreads + threadIdx.x;
    c.gstride = P * kThreads;
    // the previous launch's outcome: no workgroup passes this launch's first
    // barrier before this one has arrived there, so no step has changed it
    if (c.d.outcome && c.part == 0 && threadIdx.x == 0) {
        c.d.outcome[0] = ld(&c.ctl->error_code);
        c.d.outcome[1] = ld(&c.ctl->error_step);
        c.d.outcome[2] = ld(&c.ctl->bias_fail);
        c.d.outcome[3] = ld(&c.ctl->tick);
    }
    // A tally launch: its totals start at zero (the global words are cleared
    // by the first workgroup before its first barrier, which every other
    // workgroup passes only after), and each workgroup clears its own
    // per-step counter words, which the launch leaves untouched, for the
    // lane's next launch.
    c.tally = nullptr;
    if (kFrozenOnly && args.tally) {
        c.tally = &sh.tally[wave_index()][0];
        if (threadIdx.x < kWavesPerGroup * kTWaveWords) (&sh.tally[0][0])[threadIdx.x] = 0u;
        if (threadIdx.x < 4) sh.tally_rec[threadIdx.x] = 0ull;
        if (threadIdx.x < 2 * kCounterKinds) c.d.wg_counts[c.part * kFlagWords + threadIdx.x] = 0u;
        if (c.part == 0 && threadIdx.x < kTallyWords) args.tally[threadIdx.x] = 0u;
        __syncthreads();
    }
    // a lane whose guard tripped in an earlier launch runs nothing until the
    // host has read the code (every workgroup reads it before its first
    // barrier, and no step of this launch can set it before then)
    if (ld(&c.ctl->error_code) != 0) return;
    c.tick = ld(&c.ctl->tick);
    c.parity = ld(&c.ctl->parity);
    c.dest_epoch = ld(&c.ctl->dest_epoch);
    c.local = false;
    uint32_t target = 0;
    const uint32_t steps = c.d.step_count;
    const bool redundant = kFrozenOnly || args.redundant_global != 0;
    const uint32_t spin = args.spin_limit;
    if (P > 1 && args.local_sync) {
        // each workgroup clears its arrival words (last launch's epochs)
        // before the launch's first barrier, which counts arrivals instead
        if (threadIdx.x == 0) atomicOr(&c.d.launch->xcc_mask, 1u << xcc_id());
        if (threadIdx.x < 2) c.d.barrier_flags[c.part * kFlagWords + threadIdx.x] = 0u;
        if (!lane_barrier(c.d, c.part, P, target, spin, false)) return;
        c.local = __popc(ld(&c.d.launch->xcc_mask)) == 1;
    }
    {
        // a workgroup's winners fit the 16 bits its arrival word carries
        const uint32_t range = (args.cfg.block_count + selecting_waves(c) - 1) / selecting_waves(c);
        c.carried = c.local && P > 1 &&
                    static_cast<uint64_t>(range) * args.cfg.max_active_per_block * kWavesPerGroup <= 0xffffu;
    }
    if (threadIdx.x < kRing) {
        sh.ring_tick[threadIdx.x] = ld(&c.ctl->ring_tick[threadIdx.x]);
        sh.ring_count[threadIdx.x] = ld(&c.ctl->ring_count[threadIdx.x]);
        sh.ring_early[threadIdx.x] = ld(&c.ctl->ring_early[threadIdx.x]);
    }
    fill_decay_table(args.cfg);
    __syncthreads();
    PhaseClock clock;
    if (kProfile && c.part == args.profile_part && threadIdx.x == 0) clock.start(c.d.phase_profile);
    bool ok = true;
    // the step parameters come kStepChunk steps at a time, with one round
    // of coalesced loads into LDS: a load per step, even issued a step
    // ahead, would be waited for by the step's first wait on its own loads
    // (the vector memory counter drains in order)
    constexpr uint32_t kStepWords = sizeof(StepParams) / 4;
    static_assert(sizeof(StepParams) % 4 == 0, "step parameters are 32-bit words");
    uint32_t chunk_base = 0;
    auto load_chunk = [&](uint32_t first) {
        chunk_base = first;
        const uint32_t LEO_GLOBAL* src = reinterpret_cast<const uint32_t LEO_GLOBAL*>(c.d.steps + first);
        const uint32_t words = min(kStepChunk + 1, steps - first) * kStepWords;
        for (uint32_t i = threadIdx.x; i < words; i += kThreads) sh.step_chunk[i] = ld(&src[i]);
        __syncthreads();
    };
    auto params = [&](uint32_t index) {  // a step of the current chunk (or the next chunk's first)
        StepParams p;
        uint32_t w[kStepWords];
        const uint32_t at = (index - chunk_base) * kStepWords;
#pragma unroll
        for (uint32_t i = 0; i < kStepWords; ++i) w[i] = __builtin_amdgcn_readfirstlane(sh.step_chunk[at + i]);
        __builtin_memcpy(&p, w, sizeof(StepParams));
        if (kFrozenOnly) {
            p.flags = (p.flags & ~static_cast<uint32_t>(kStepLearnTrace | kStepAllocate | kStepLearn | kStepOutput)) |
                      kStepFrozen;
            p.plasticity_scale = 0.0f;
        }
        return p;
    };
    // a step whose delivery ran in the previous step's last phase; a step
    // after a one-barrier frozen step (frozen_emit), and the population
    // inhibition the last fold read
    bool delivered_ahead = false, stopped = false, after_one_barrier = false;
    float pi_read = 0.0f;
    uint32_t early_prev = 0;  // kStepEarly delays of the one-barrier step before
    const bool one_barrier_lane = c.d.bucket_sets != 1 && c.P > 1 && redundant;
    for (uint32_t s = 0; s < steps && ok; ++s) {
        if (s % kStepChunk == 0) load_chunk(s);
        const StepParams sp = params(s);
        const bool trace = (sp.flags & kStepLearnTrace) != 0;
        const bool learn = (sp.flags & kStepLearn) != 0;
        // steps without eligibility updates or readout fold the post phase
        // into the active-list write (one barrier fewer)
        const bool fused = redundant && !trace && !(sp.flags & kStepOutput);
        if (!delivered_ahead) {
            // the context (runtime.rs:641-677) is first read by the readout
            if (c.part == c.P - 1) context_resolve(c, sp, sh);
            phase_deliver(c, sp, sh);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 0))) break;
        }
        // this step's destination and learning-slot lists start empty (filled
        // by the eligibility phase) under a new claim epoch
        const bool plastic = learn && sp.plasticity_scale > 0.0f;
        if (plastic) {
            c.dest_epoch += 1;
            if (c.part == 0 && threadIdx.x == 0) {
                c.ctl->dest_count = 0;
                c.ctl->rec_learn_count = 0;
                c.ctl->in_learn_count = 0;
            }
        }
        // the previous tick's record and population inhibition after a
        // one-barrier frozen step (before this step's context replaces the
        // context fields that record reads)
        // the profiling build times a one-barrier step's prologue, context
        // and fold in the slots of the phases such a step does not run
        const bool timer = kProfile && c.part == args.profile_part && threadIdx.x == 0;
        const unsigned long long t_start = timer ? wall_clock64() : 0;
        const float pi =
            after_one_barrier ? frozen_prologue(c, sh, s, pi_read, early_prev) : ld(&c.ctl->population_inhibition);
        pi_read = pi;
        const unsigned long long t_prologue = timer ? wall_clock64() : 0;
        // the context of a step delivered ahead: on the workgroup that owns no
        // selection blocks, beside the fold (first read by the readout)
        if (delivered_ahead && c.P > 1 && c.part == c.P - 1) context_resolve(c, sp, sh);
        const unsigned long long t_context = timer ? wall_clock64() : 0;
        phase_fold_select(c, sh, trace, pi, after_one_barrier);
        const unsigned long long t_fold = timer ? wall_clock64() : 0;
        // a fused step followed by a frozen one starts the next tick in its
        // last phase: the next delivery runs before this step's closing
        // barrier (one barrier fewer again)
        StepParams next{};
        bool pipeline = false;
        if (fused && !learn && s + 1 < steps) {
            next = params(s + 1);
            pipeline = (next.flags & kStepLearnTrace) == 0;
        }
        // and with the bucket sets, a frozen step followed by a fused frozen
        // one takes a single phase (its delay-1 events are early: the host
        // marks the delays of every launched step)
        if (one_barrier_lane && pipeline && !(next.flags & kStepOutput) && (sp.flags & (1u << kStepEarlyShift))) {
            early_prev = (sp.flags & kStepEarlyMask) >> kStepEarlyShift;
            if (timer) {
                clock.section(3, t_start, t_prologue);
                clock.section(4, t_prologue, t_context);
                clock.section(5, t_context, t_fold);
            }
            frozen_emit(c, sh, early_prev, next);
            // after a two-phase step, the roll its successor's active-list
            // phase would make: that step's record is finished and the
            // counters tick+1 reuses are cleared (a one-barrier step's
            // prologue did both)
            if (!after_one_barrier && !c.tally && c.part == c.P - 1 && wave_index() == 0) roll_counters(c, s);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 6, c.carried ? sh.win_count : nullptr,
                                               c.carried ? sh.lane_sums : nullptr)))
                break;
            delivered_ahead = true;
            after_one_barrier = true;
            c.tick += 1;
            continue;
        }
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 1))) break;
        // An output step's readout runs on the last workgroup beside the
        // eligibility update, which the other workgroups share (a lane of one
        // workgroup runs both), so a plasticity step computes its signals in
        // the post phase (one barrier fewer). The post phase's state updates
        // are read by neither the readout nor the signals.
        const bool output = (sp.flags & kStepOutput) != 0;
        const bool reader = output && c.part == c.P - 1;
        const uint32_t elig_stride = output && c.P > 1 ? (c.P - 1) * kThreads : c.gstride;
        if (redundant) {
            write_active(c, sp, s, sh, fused, pipeline, next, after_one_barrier);
            if (trace && !(reader && c.P > 1)) phase_eligibility(c, plastic, elig_stride);
            if (pipeline && c.P == 1) context_resolve(c, next, sh);
        } else {
            global_select(c, sh, s);
            if (trace || output) {  // the readout reads the global selection's list
                if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 7))) break;
                if (trace && !(reader && c.P > 1)) phase_eligibility(c, plastic, elig_stride);
            }
        }
        if (__builtin_expect(reader, 0)) readout(c, sp, sh, s);  // laid out off the frozen path
        if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 2))) break;
        if (!fused) {
            if (trace) c.parity ^= 1;
            phase_post(c, sp, s, sh);
            if (!plastic && !(ok = phase_barrier<kProfile>(c, target, spin, clock, 3))) break;
        }
        if (plastic) {
            phase_signals(c, sh);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 4))) break;
        }
        if (learn || !(sp.flags & kStepFrozen)) {
            phase_learn(c, sp, sh, s);
            if (!(ok = phase_barrier<kProfile>(c, target, spin, clock, 5))) break;
            // a numerical guard of this step ends the lane here, as the
            // reference's step returns its error (every workgroup reads the
            // word after the barrier that follows the guards)
            if (learn && ld(&c.ctl->error_code) != 0) {
                stopped = true;
                c.tick += 1;
                break;
            }
        }
        delivered_ahead = pipeline;
        after_one_barrier = false;
        c.tick += 1;
    }
    if (ok && !stopped && !c.tally && c.part == 0 && threadIdx.x < kWaveSize && steps > 0)
        finalize_record(c, steps - 1, c.tick - 1);
    if (ok && c.tally && __lane_id() == 0) {
        // each wave's totals; the recording wave's 64-bit sums (it is the
        // only writer of those words after the launch's first barrier)
        const uint32_t wave = wave_index();
#pragma unroll
        for (uint32_t k = 0; k < kTWaveWords; ++k)
            if (sh.tally[wave][k]) atomicAdd(&args.tally[k], sh.tally[wave][k]);
        if (c.part == c.P - 1 && wave == 0) {
            unsigned long long LEO_GLOBAL* sums = reinterpret_cast<unsigned long long LEO_GLOBAL*>(args.tally + kTActive);
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) sums[k] = sh.tally_rec[k];
        }
    }
    if (ok && c.part == 0 && threadIdx.x == 0) {
        c.ctl->tick = c.tick;
        c.ctl->parity = c.parity;
        c.ctl->dest_epoch = c.dest_epoch;
    }
}

// The arguments live in device memory (read with scalar loads): a by-value
// argument whose address is taken is copied to scratch.
__global__ void __launch_bounds__(kThreads) leo_lane_steps(const KernelArgs* __restrict__ args) {
    lane_steps<false, false>(*args);
}
__global__ void __launch_bounds__(kThreads) leo_lane_steps_profiled(const KernelArgs* __restrict__ args) {
    lane_steps<true, false>(*args);
}
__global__ void __launch_bounds__(kThreads) leo_lane_steps_frozen(const KernelArgs* __restrict__ args) {
    lane_steps<false, true>(*args);
}

// Each lane's outcome of the launch before this kernel on the stream (error
// code, error step, bias fail, tick): four words per lane, gathered next to
// the launch's step records so that one download brings both.
__global__ void __launch_bounds__(kThreads) leo_lane_outcomes(const KernelArgs* __restrict__ args,
                                                            uint32_t* __restrict__ out) {
    const uint32_t l = blockIdx.x * kThreads + threadIdx.x;
    if (l >= args->lane_count) return;
    const LaneControl* ctl = args->lanes[l].ctl;
    out[4 * l + 0] = ctl->error_code;
    out[4 * l + 1] = ctl->error_step;
    out[4 * l + 2] = ctl->bias_fail;
    out[4 * l + 3] = ctl->tick;
}

// Clears the lanes' parameter-change bitmaps and dirty words
// (enable_parameter_tracking) in one pass for a whole group of lanes.
__global__ void __launch_bounds__(kThreads) leo_clear_changes(KernelArgs args, ChangeWords w) {
    const uint32_t L = args.lane_count;
    const uint32_t lane = blockIdx.x % L;
    const uint32_t part = blockIdx.x / L, parts = gridDim.x / L;
    const LaneDesc& d = args.lanes[lane];
    const uint64_t t0 = static_cast<uint64_t>(part) * kThreads + threadIdx.x, ts = static_cast<uint64_t>(parts) * kThreads;
    for (uint64_t i = t0; i < w.neurons; i += ts) {
        d.ch_threshold[i] = 0u;
        d.ch_out[i] = 0u;
    }
    for (uint64_t i = t0; i < w.recurrent; i += ts) d.ch_rec[i] = 0u;
    for (uint64_t i = t0; i < w.input; i += ts) d.ch_in[i] = 0u;
    for (uint64_t i = t0; i < w.slots; i += ts) d.ch_ctx[i] = 0u;
    if (part == 0 && threadIdx.x == 0) {
        d.ctl->bias_dirty = 0u;
        d.ctl->ctx_out_dirty = 0u;
    }
}

// A story group's fork of the canonical parameters (parallel.rs: each worker
// starts from base.clone()): every 16-byte vector of one canonical tensor is
// read once and stored to each lane's copy.
__global__ void __launch_bounds__(kThreads) leo_broadcast(Broadcast b) {
    const uint64_t t0 = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t ts = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = t0; i < b.vectors; i += ts) {
        const uint4 v = b.src[i];
        for (uint32_t l = 0; l < b.count; ++l) b.dst[l][i] = v;
    }
}

// ---------------------------------------------------------------------------
// reset_transient_state (runtime.rs:365-425) for every lane in args.
//
// Recurrent trace slots are cleared from their marks: a slot whose mark is 0
// has not been written since the last reset, so its seven values are still
// zero (1 = listed as eligible, 2 = dropped from the list with its values
// kept). Every group of 16 slots with a nonzero mark has its 16 trace
// records (512 contiguous bytes) rewritten; a clean slot keeps its last tick,
// also when the reset sets a new tick below it. Its values are zero, so its
// next activation at tick t leaves (activation, 0, ..., 0, t) whatever the
// old tick was: the elapsed ticks t - last wrap to a large count when last
// > t, and the decays of a large count are finite (every decay lies in
// [0, 1), config.rs:318-334), so they scale the zeros to zeros; with last == t
// only the branch sensitivity is added to. Lane state starts zero-filled
// (tick 0), so the first reset finds every slot clean.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void fill_u32(uint32_t LEO_GLOBAL* p, uint64_t n, uint32_t v, uint64_t t0, uint64_t ts) {
    // p is 256-byte aligned (lane-state layout)
    const uint64_t n4 = n / 4;
    uint4 LEO_GLOBAL* q = reinterpret_cast<uint4 LEO_GLOBAL*>(p);
    const uint4 w = make_uint4(v, v, v, v);
    for (uint64_t i = t0; i < n4; i += ts) q[i] = w;
    for (uint64_t i = 4 * n4 + t0; i < n; i += ts) p[i] = v;
}

__device__ __forceinline__ void fill_f32(float LEO_GLOBAL* p, uint64_t n, uint64_t t0, uint64_t ts) {
    fill_u32(reinterpret_cast<uint32_t LEO_GLOBAL*>(p), n, 0u, t0, ts);
}

// Group g of 16 slots, whose marks `m` the caller has loaded (a launch of its
// own: plain loads see the previous kernels' stores).
__device__ __forceinline__ void clear_trace_group(const LaneDesc& d, uint64_t g, uint4 m, uint32_t tick) {
    uint4 LEO_GLOBAL* marks = reinterpret_cast<uint4 LEO_GLOBAL*>(d.rec_mark);
    const bool dirty = (m.x | m.y | m.z | m.w) != 0u;
    if (!dirty) return;
    // 16 records of 32 bytes: zero sensitivities, last tick = tick
    uint4 LEO_GLOBAL* rec = reinterpret_cast<uint4 LEO_GLOBAL*>(d.rec_trace + 16 * g * kTraceWords);
    const uint4 zero = make_uint4(0u, 0u, 0u, 0u), with_tick = make_uint4(0u, 0u, 0u, tick);
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) {
        rec[2 * k] = zero;
        rec[2 * k + 1] = with_tick;
    }
    marks[g] = zero;
}

__global__ void __launch_bounds__(kThreads) leo_reset_lanes(KernelArgs args, uint32_t set_tick, uint32_t new_tick) {
    const LeoConfig& cfg = args.cfg;
    const uint32_t L = args.lane_count;
    const uint32_t lane = blockIdx.x % L;
    const uint32_t part = blockIdx.x / L, parts = gridDim.x / L;
    const LaneDesc& d = args.lanes[lane];
    // a lane stopped by a guard keeps the state the guard left until the
    // host has read the code and cleared it (a reset queued behind the
    // failing launch does nothing)
    if (d.ctl->error_code != 0) return;
    const uint32_t tick = set_tick ? new_tick : d.ctl->tick;
    const uint64_t N = cfg.neuron_count, S = cfg.synapses_per_neuron;
    const uint64_t NS = N * S, NI = static_cast<uint64_t>(kSymbols) * cfg.input_fanout;
    const uint64_t t0 = static_cast<uint64_t>(part) * kThreads + threadIdx.x, ts = static_cast<uint64_t>(parts) * kThreads;
    // neuron records: zero state, last tick = tick, epochs and claims 0
    // (claim epochs in use are >= 1)
    static_assert(kNeuronWords == 16 && kNLastTick == 10, "record layout");
    {
        uint4 LEO_GLOBAL* rec = reinterpret_cast<uint4 LEO_GLOBAL*>(d.neuron);
        // a select of the word, not of two vectors (which becomes an indexed
        // private array)
        for (uint64_t i = t0; i < 4 * N; i += ts) rec[i] = make_uint4(0u, 0u, (i & 3) == 2 ? tick : 0u, 0u);
    }
    const uint64_t groups = NS / 16;
    {
        // four groups' marks in flight per thread before any is cleared
        const uint4 LEO_GLOBAL* marks = reinterpret_cast<const uint4 LEO_GLOBAL*>(d.rec_mark);
        constexpr uint32_t kAhead = 4;
        for (uint64_t g = t0; g < groups; g += kAhead * ts) {
            uint4 m[kAhead];
#pragma unroll
            for (uint32_t k = 0; k < kAhead; ++k) {
                const uint64_t gk = g + k * ts;
                m[k] = make_uint4(0u, 0u, 0u, 0u);
                if (gk < groups) m[k] = marks[gk];
            }
#pragma unroll
            for (uint32_t k = 0; k < kAhead; ++k)
                if (g + k * ts < groups) clear_trace_group(d, g + k * ts, m[k], tick);
        }
    }
    auto clear_record = [&](float LEO_GLOBAL* trace, uint64_t i) {
        uint4 LEO_GLOBAL* rec = reinterpret_cast<uint4 LEO_GLOBAL*>(trace + i * kTraceWords);
        rec[0] = make_uint4(0u, 0u, 0u, 0u);
        rec[1] = make_uint4(0u, 0u, 0u, tick);
    };
    for (uint64_t i = 16 * groups + t0; i < NS; i += ts) {
        if (d.rec_mark[i] != 0) {
            clear_record(d.rec_trace, i);
            d.rec_mark[i] = 0;
        }
    }
    for (uint64_t i = t0; i < NI; i += ts) clear_record(d.in_trace, i);
    for (uint64_t i = t0; i < NI; i += ts) d.in_mark[i] = 0;
    for (uint64_t i = t0; i < cfg.context_embedding_dim; i += ts) d.ctx_latent[i] = 0.0f;
    fill_u32(d.block_epoch, cfg.block_count, 0u, t0, ts);
    {
        // bucket counts and touched bits of every set (deliveries pending for
        // later ticks are dropped): a nonzero count always has its target's
        // bit set, as a tick's first delivery to a target touches it, so the
        // set bits name every count to clear
        const uint32_t nb = cfg.neurons_per_block, wpb = block_words(nb);
        const uint64_t words = static_cast<uint64_t>(cfg.block_count) * wpb;
        for (uint32_t set = 0; set < d.bucket_sets; ++set) {
            uint32_t LEO_GLOBAL* bits = set_touched(d, set);
            uint32_t LEO_GLOBAL* counts = set_counts(d, set, cfg.neuron_count);
            for (uint64_t w = t0; w < words; w += ts) {
                uint32_t v = bits[w];
                if (v == 0) continue;
                const uint64_t blk = w / wpb, base = blk * nb + (w - blk * wpb) * 32;
                while (v) {
                    const uint32_t b = __ffs(v) - 1;
                    v &= v - 1;
                    counts[base + b] = 0u;
                }
                bits[w] = 0u;
            }
        }
    }
    for (uint64_t i = t0; i < kMaxWaves; i += ts) {
        d.wave_total[i] = 0;
        d.wave_total[kMaxWaves + i] = 0;
        d.wave_touched[i] = 0;
    }
    for (uint64_t i = t0; i < kMaxLaneWgs * kFlagWords; i += ts) d.wg_counts[i] = 0;
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
        ctl->dest_count = 0;
        ctl->rec_learn_count = 0;
        ctl->in_learn_count = 0;
        ctl->barrier = 0;
        ctl->abort = 0;
        for (uint32_t k = 0; k < kRing; ++k) {
            ctl->ring_tick[k] = 0xffffffffu;
            ctl->ring_count[k] = 0;
            ctl->ring_early[k] = 0;
        }
    }
}

// ---------------------------------------------------------------------------
// Batch-end mean of one fixed-parameter tensor over `lanes` story lanes
// (parallel.rs:975-1022 apply_sparse_scaled: canonical += f32(Σ_lanes f64(lane-base) / L),
// only where some lane changed it), then the projection of parallel.rs:1169-1246
// and the bound checks of parallel.rs:1248-1345.
// ---------------------------------------------------------------------------


__device__ __forceinline__ float merge_project(const MergeArgs& m, uint64_t i, float v) {
    switch (m.kind) {
        case kMergeThreshold: return clampf(v, 0.05f, 2.0f);
        case kMergeRecurrent:
            v = clampf(v, m.weight_min, m.weight_max);
            return m.neuron_type[i / m.synapses_per_neuron] == 0 ? max_zero(v) : min_zero(v);
        case kMergeInput: return clampf(v, 0.0f, m.weight_max);
        case kMergeOutput:
        case kMergeContextOut: return clampf(v, m.weight_min, m.weight_max);
        default: return v;
    }
}

// Host-stale mark of a merged element: its bit (its neuron row's for the
// output projection), or the tensor's flag word.
__device__ __forceinline__ void mark_stale(const MergeArgs& m, uint64_t i) {
    if (!m.stale) return;
    if (m.stale_flag) {
        m.stale[0] = 1u;
        return;
    }
    const uint64_t bit = m.kind == kMergeOutput ? i / m.row : i;
    atomicOr(&m.stale[bit >> 5], 1u << (bit & 31));
}

// One bitmap word per thread: the OR over the group's lanes, its set
// positions appended to the list (one atomic per wave; the list's order does
// not matter, every element is merged on its own).
__global__ void __launch_bounds__(kThreads) leo_merge_candidates(MergeCandidates mc) {
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads; base < mc.words;
         base += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t w = base + threadIdx.x;
        uint32_t word = 0;
        if (w < mc.words) {
            for (uint32_t l = 0; l < mc.lane_count; ++l) word |= mc.bits[l][w];
            const uint64_t tail = mc.positions - w * 32;  // positions in this word
            if (tail < 32) word &= (1u << tail) - 1u;
        }
        const uint32_t n = static_cast<uint32_t>(__popc(word));
        const uint32_t incl = wave_incl_scan_u32(n);
        const uint32_t total = __builtin_amdgcn_readlane(incl, kWaveSize - 1);
        unsigned long long at = 0;
        if (__lane_id() == kWaveSize - 1 && total) at = atomicAdd(mc.count, static_cast<unsigned long long>(total));
        at = static_cast<unsigned long long>(__builtin_amdgcn_readlane(static_cast<uint32_t>(at), kWaveSize - 1)) |
             (static_cast<unsigned long long>(__builtin_amdgcn_readlane(static_cast<uint32_t>(at >> 32), kWaveSize - 1))
              << 32);
        at += incl - n;
        while (word) {
            const uint32_t bit = __ffs(word) - 1;
            word &= word - 1;
            mc.list[at++] = static_cast<uint32_t>(w * 32 + bit);
        }
    }
}

// One lane per blockIdx.y: the lane's changed context slots (one bitmap word
// per thread) packed into its region, appended with one atomic per wave (the
// host orders the records by key).
__global__ void __launch_bounds__(kThreads) leo_context_changes(ContextChanges g) {
    const uint32_t l = blockIdx.y;
    const uint32_t rec_words = 4 + g.E;
    const uint32_t* bits = g.bits[l];
    const uint64_t* keys = g.keys[l];
    const uint32_t* obs = g.obs[l];
    const float* emb = g.emb[l];
    uint32_t LEO_GLOBAL* out = g.out + static_cast<uint64_t>(l) * g.stride;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads; base < g.words;
         base += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t w = base + threadIdx.x;
        uint32_t word = 0;
        if (w < g.words) {
            word = bits[w];
            const uint64_t tail = g.slots - w * 32;  // slots in this word
            if (tail < 32) word &= (1u << tail) - 1u;
        }
        const uint32_t n = static_cast<uint32_t>(__popc(word));
        const uint32_t incl = wave_incl_scan_u32(n);
        const uint32_t total = __builtin_amdgcn_readlane(incl, kWaveSize - 1);
        unsigned long long at = 0;
        if (__lane_id() == kWaveSize - 1 && total) at = atomicAdd(&g.counts[l], static_cast<unsigned long long>(total));
        at = static_cast<unsigned long long>(__builtin_amdgcn_readlane(static_cast<uint32_t>(at), kWaveSize - 1)) |
             (static_cast<unsigned long long>(__builtin_amdgcn_readlane(static_cast<uint32_t>(at >> 32), kWaveSize - 1))
              << 32);
        at += incl - n;
        while (word) {
            const uint32_t bit = __ffs(word) - 1;
            word &= word - 1;
            const uint64_t slot = w * 32 + bit;
            uint32_t LEO_GLOBAL* rec = out + at * rec_words;
            const uint64_t key = keys[slot];
            rec[0] = static_cast<uint32_t>(slot);
            rec[1] = static_cast<uint32_t>(key);
            rec[2] = static_cast<uint32_t>(key >> 32);
            rec[3] = obs[slot];
            for (uint32_t e = 0; e < g.E; ++e) rec[4 + e] = __float_as_uint(emb[slot * g.E + e]);
            at += 1;
        }
    }
}

__global__ void __launch_bounds__(kThreads) leo_merge_fixed(MergeArgs m) {
    unsigned long long local = 0, changes = 0;
    // visited elements: all of them, or the listed positions' elements
    const uint64_t per = m.row ? m.row : 1u;
    const uint64_t visits = m.list ? *m.list_count * per : m.count;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; k < visits;
         k += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t i = m.list ? static_cast<uint64_t>(m.list[k / per]) * per + k % per : k;
        uint64_t at = m.row ? (i / m.row) * m.stride + (i % m.row) : i;
        const float base = m.canonical[at];
        if (m.mode == kMergeFinalize) {
            if (!m.any[i]) continue;
            float v = base + static_cast<float>(m.acc[i] / static_cast<double>(m.total_lanes));
            if (!finitef(v)) atomicCAS(m.error, 0u, 2u);
            v = merge_project(m, i, v);
            if (!finitef(v)) atomicCAS(m.error, 0u, 3u);
            m.canonical[at] = v;
            mark_stale(m, i);
            local += 1;
            continue;
        }
        double sum = 0.0;
        bool any = false;
        if (m.mode == kMergeAccumulate && (m.list || !m.first)) {
            // with a list the flags were cleared before the first group, so an
            // element first listed in a later group starts from zero
            any = m.any[i] != 0;
            sum = any || !m.list ? m.acc[i] : 0.0;
        }
        for (uint32_t l = 0; l < m.lane_count; ++l) {
            float delta = m.lanes[l][at] - base;
            if (delta != 0.0f) {
                any = true;
                changes += 1;
                if (!finitef(delta)) atomicCAS(m.error, 0u, 1u);
                sum += static_cast<double>(delta);
            }
        }
        if (m.mode == kMergeAccumulate) {
            m.acc[i] = sum;
            m.any[i] = any ? 1 : 0;
            continue;
        }
        if (!any) continue;
        float v = base + static_cast<float>(sum / static_cast<double>(m.lane_count));
        if (!finitef(v)) atomicCAS(m.error, 0u, 2u);
        v = merge_project(m, i, v);
        if (!finitef(v)) atomicCAS(m.error, 0u, 3u);
        m.canonical[at] = v;
        mark_stale(m, i);
        local += 1;
    }
    if (local) atomicAdd(m.updates, local);
    if (changes) atomicAdd(m.lane_changes, changes);
}

// ---------------------------------------------------------------------------
// Host synchronisation of the canonical image (cuda.rs:5657-5760) and packed
// sparse updates (parallel.rs:186-302, cuda.rs:2869-3080).
// ---------------------------------------------------------------------------
// One tensor's elements (or rows) between the canonical image and a packed
// buffer, one element per thread.
__global__ void __launch_bounds__(kThreads) leo_sparse_move(SparseMove mv) {
    const uint64_t per = mv.row ? mv.row : 1u;
    const uint64_t total = mv.count * per;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t k = i / per, e = i - k * per;
        const uint64_t at = mv.row ? static_cast<uint64_t>(mv.index[k]) * mv.stride + e : mv.index[k];
        if (mv.to_tensor) mv.tensor[at] = mv.packed[i];
        else mv.packed[i] = mv.tensor[at];
    }
}

// stale |= changes, changes = 0, for each bitmap (and the dirty-flag words).
__global__ void __launch_bounds__(kThreads) leo_fold_changes(FoldArgs f) {
    for (uint32_t b = 0; b < 6; ++b) {
        for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < f.words[b];
             i += static_cast<uint64_t>(gridDim.x) * kThreads) {
            const uint32_t v = f.changes[b][i];
            if (v) {
                f.stale[b][i] |= v;
                f.changes[b][i] = 0u;
            }
        }
    }
}

}  // namespace leo
