// TEST INFRASTRUCTURE ONLY: CPU restatement of Leo's reference executor.
// Each function cites the reference file:line it follows (paths relative to
// the saravanaspar/Leo tree). Built with -ffp-contract=off so every FP32
// operation rounds exactly where the Rust source rounds. exp/ln call glibc
// expf/logf, which is what Rust's f32::exp/f32::ln lower to on x86_64 Linux;
// f32::powi lowers to compiler-rt __powisf2, restated in powisf2() below.

#include "leo_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <limits>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <utility>
#include <vector>

namespace {

constexpr uint32_t BYTE_SYMBOLS = 256;
constexpr uint32_t BEGIN_DOCUMENT = 256;
constexpr uint32_t END_DOCUMENT = 257;
constexpr size_t SYMBOL_COUNT = 258;
constexpr size_t OUTPUT_CLASSES = 257;
constexpr size_t END_INDEX = 256;
constexpr uint8_t BR_EXC = 0, BR_INH = 1, BR_TEMP = 2, BR_GATE = 3;

thread_local std::string g_last_error;

struct LeoError : std::runtime_error {
    int32_t code;
    LeoError(int32_t c, const std::string& m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] void internal(const std::string& m) { throw LeoError(ORACLE_ERR_INTERNAL, m); }
[[noreturn]] void numerical(const std::string& m) { throw LeoError(ORACLE_ERR_NUMERICAL, m); }

template <class F>
int32_t guard(F&& f) {
    try {
        f();
        return ORACLE_OK;
    } catch (const LeoError& e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return ORACLE_ERR_INTERNAL;
    }
}

inline uint64_t sat_add(uint64_t a, uint64_t b) { return (a > UINT64_MAX - b) ? UINT64_MAX : a + b; }
inline uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }
inline uint32_t sat_add32(uint32_t a, uint32_t b) { return (a > UINT32_MAX - b) ? UINT32_MAX : a + b; }
inline float clampf(float v, float lo, float hi) {  // Rust f32::clamp
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}
// Rust's w.max(0.0) / w.min(0.0) (the sign projections, runtime.rs:1475-1479,
// parallel.rs:1202-1206) as rustc lowers them on x86_64: maxss/minss with the
// constant as the second operand, and that operand wins when the values
// compare equal or one is NaN. So -0.0 and NaN both project to +0.0.
inline float max_zero(float v) { return v > 0.0f ? v : 0.0f; }
inline float min_zero(float v) { return v < 0.0f ? v : 0.0f; }
inline float maxf(float a, float b) {  // Rust f32::max (maxNum)
    if (std::isnan(a)) return b;
    if (std::isnan(b)) return a;
    return a > b ? a : b;
}
// Rust f32::total_cmp ordering key.
inline int32_t total_key(float v) {
    int32_t bits;
    std::memcpy(&bits, &v, 4);
    return bits ^ static_cast<int32_t>(static_cast<uint32_t>(bits >> 31) >> 1);
}
inline int total_cmp(float a, float b) {
    int32_t x = total_key(a), y = total_key(b);
    return (x < y) ? -1 : (x > y ? 1 : 0);
}

// compiler-rt lib/builtins/powisf2.c (Rust f32::powi with a runtime exponent).
float powisf2(float a, int b) {
    const bool recip = b < 0;
    float r = 1.0f;
    while (true) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

// runtime.rs:78-85
float decay_for_elapsed(float base, uint64_t elapsed) {
    if (elapsed == 0) return 1.0f;
    if (elapsed == 1) return base;
    uint64_t e = std::min<uint64_t>(elapsed, static_cast<uint64_t>(INT32_MAX));
    return powisf2(base, static_cast<int>(e));
}

// learning.rs:7-24
float analog_rank_surrogate(float margin, float cutoff, bool selected, float width, float gain) {
    float direct = (selected && margin > 0.0f && margin < 1.0f) ? 1.0f : 0.0f;
    if (width <= 0.0f || gain <= 0.0f) return direct;
    float boundary = clampf(1.0f - std::fabs(margin - cutoff) / width, 0.0f, 1.0f);
    return direct + gain * boundary;
}

// learning.rs:29-51
float branch_jacobian(uint8_t branch, float excitability, float temporal, float gate_acc) {
    float gate = clampf(gate_acc, 0.0f, 1.0f);
    switch (branch) {
        case BR_EXC: return excitability;
        case BR_TEMP: return excitability * gate;
        case BR_INH: return excitability;
        case BR_GATE: {
            float d = (gate_acc > 0.0f && gate_acc < 1.0f) ? 1.0f : 0.0f;
            return excitability * temporal * d;
        }
        default: return 0.0f;
    }
}

// learning.rs:54-56
inline float bounded_delta(float v, float m) { return clampf(v, -m, m); }

// learning.rs:60-71
float inhibitory_homeostasis_delta(float src, float tgt, float desired, float lr, float strength,
                                   float max_update) {
    float err = tgt - desired;
    return bounded_delta(-lr * strength * src * err, max_update);
}

// runtime.rs:103-116
bool context_survives_dropout(uint64_t seed, uint64_t tick, uint32_t symbol, float rate) {
    if (rate <= 0.0f) return true;
    uint64_t v = seed ^ (tick * 0x9e3779b97f4a7c15ULL) ^ (static_cast<uint64_t>(symbol) * 0xbf58476d1ce4e5b9ULL);
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
    v ^= v >> 31;
    float draw = static_cast<float>(static_cast<uint32_t>(v >> 40)) / static_cast<float>(1u << 24);
    return draw >= rate;
}

// runtime.rs:679-690
uint64_t context_key(const uint32_t* history, size_t len, size_t order) {
    const uint64_t prime = 0x100000001b3ULL;
    uint64_t h = 0xcbf29ce484222325ULL ^ static_cast<uint64_t>(order);
    for (size_t i = len - order; i < len; ++i) {
        uint32_t s = history[i];
        for (int b = 0; b < 4; ++b) {
            h ^= static_cast<uint64_t>((s >> (8 * b)) & 0xffu);
            h *= prime;
        }
    }
    return h < 1 ? 1 : h;
}

struct Config {
    OracleConfig c;
    // config.rs:137-145
    std::pair<float, size_t> plasticity_step(size_t phase, bool end_document) const {
        size_t window = std::max<size_t>(c.plasticity_window, 1);
        size_t step = std::min(phase, window - 1) + 1;
        if (step == window || end_document) return {static_cast<float>(step), 0};
        return {0.0f, step};
    }
    float strength(int32_t permission) const {  // permission.rs:24-31
        switch (permission) {
            case ORACLE_FROZEN: return 0.0f;
            case ORACLE_PROVISIONAL: return c.provisional_strength;
            case ORACLE_TRAINING: return c.training_strength;
            case ORACLE_VERIFIED: return c.verified_strength;
            default: internal("unknown permission");
        }
    }
};

struct Model {
    Config cfg;
    uint64_t generation = 0;
    uint64_t parameter_revision = 0;
    std::vector<float> threshold, excitability;
    std::vector<uint8_t> neuron_type;
    std::vector<uint32_t> rec_target;
    std::vector<uint8_t> rec_branch, rec_delay;
    std::vector<float> rec_weight;
    std::vector<uint32_t> in_target;
    std::vector<uint8_t> in_branch;
    std::vector<float> in_weight;
    std::vector<float> out_weight;  // output-major [257][N]
    std::vector<float> bias;
    std::vector<uint64_t> ctx_keys;
    std::vector<float> ctx_emb;
    std::vector<uint32_t> ctx_obs;
    std::vector<float> ctx_out;  // output-major [257][E]
    OracleStatistics stats{};

    size_t N() const { return cfg.c.neuron_count; }
    size_t S() const { return cfg.c.synapses_per_neuron; }
    size_t F() const { return cfg.c.input_fanout; }
    size_t E() const { return cfg.c.context_embedding_dim; }
    size_t slots() const { return static_cast<size_t>(cfg.c.context_max_order) * cfg.c.context_slots_per_order; }

    void load(const OracleConfig& config, const OracleModelView& v) {
        cfg.c = config;
        const size_t n = N(), ns = n * S(), ni = SYMBOL_COUNT * F(), sl = slots(), e = E();
        auto cp = [](auto& dst, const auto* src, size_t count) {
            if (!src) internal("null model array");
            dst.assign(src, src + count);
        };
        cp(threshold, v.threshold, n);
        cp(excitability, v.excitability, n);
        cp(neuron_type, v.neuron_type, n);
        cp(rec_target, v.rec_target, ns);
        cp(rec_branch, v.rec_branch, ns);
        cp(rec_delay, v.rec_delay, ns);
        cp(rec_weight, v.rec_weight, ns);
        cp(in_target, v.in_target, ni);
        cp(in_branch, v.in_branch, ni);
        cp(in_weight, v.in_weight, ni);
        cp(out_weight, v.out_weight, OUTPUT_CLASSES * n);
        cp(bias, v.bias, OUTPUT_CLASSES);
        cp(ctx_keys, v.ctx_keys, sl);
        cp(ctx_emb, v.ctx_emb, sl * e);
        cp(ctx_obs, v.ctx_obs, sl);
        cp(ctx_out, v.ctx_out, OUTPUT_CLASSES * e);
        generation = v.generation;
        parameter_revision = v.parameter_revision;
        stats = v.statistics;
    }
    void store(OracleModelView& v) const {
        auto cp = [](auto* dst, const auto& src) {
            if (dst) std::copy(src.begin(), src.end(), dst);
        };
        cp(v.threshold, threshold);
        cp(v.excitability, excitability);
        cp(v.neuron_type, neuron_type);
        cp(v.rec_target, rec_target);
        cp(v.rec_branch, rec_branch);
        cp(v.rec_delay, rec_delay);
        cp(v.rec_weight, rec_weight);
        cp(v.in_target, in_target);
        cp(v.in_branch, in_branch);
        cp(v.in_weight, in_weight);
        cp(v.out_weight, out_weight);
        cp(v.bias, bias);
        cp(v.ctx_keys, ctx_keys);
        cp(v.ctx_emb, ctx_emb);
        cp(v.ctx_obs, ctx_obs);
        cp(v.ctx_out, ctx_out);
        v.generation = generation;
        v.parameter_revision = parameter_revision;
        v.statistics = stats;
    }

    // model.rs:173-221
    std::pair<int64_t, size_t> resolve_context_slot(size_t order, uint64_t key, bool allocate) {
        if (order == 0 || order > cfg.c.context_max_order || key == 0)
            internal("invalid context order or fingerprint");
        const size_t spo = cfg.c.context_slots_per_order;
        const size_t probe_limit = cfg.c.context_probe_limit;
        const size_t base = (order - 1) * spo;
        const size_t start = static_cast<size_t>(key % spo);
        int64_t empty_slot = -1;
        size_t weakest_slot = base + start;
        uint32_t weakest_obs = UINT32_MAX;
        size_t probes = 0;
        for (size_t off = 0; off < probe_limit; ++off) {
            size_t slot = base + (start + off) % spo;
            probes += 1;
            uint64_t existing = ctx_keys[slot];
            if (existing == key) return {static_cast<int64_t>(slot), probes};
            if (existing == 0 && empty_slot < 0) empty_slot = static_cast<int64_t>(slot);
            uint32_t obs = ctx_obs[slot];
            if (obs < weakest_obs) {
                weakest_obs = obs;
                weakest_slot = slot;
            }
        }
        if (!allocate) return {-1, probes};
        size_t slot = empty_slot >= 0 ? static_cast<size_t>(empty_slot) : weakest_slot;
        if (ctx_keys[slot] != key) {
            ctx_keys[slot] = key;
            ctx_obs[slot] = 0;
            std::fill(ctx_emb.begin() + slot * E(), ctx_emb.begin() + (slot + 1) * E(), 0.0f);
        }
        return {static_cast<int64_t>(slot), probes};
    }

    // model.rs:223-396 (the subset of invariants the executor relies on).
    void validate() const {
        const size_t n = N(), s = S();
        if (n == 0 || cfg.c.block_count * cfg.c.neurons_per_block != n) internal("model dimensions are incompatible");
        if (cfg.c.branches_per_neuron != 4) internal("Leo requires exactly four dendritic branches per neuron");
        for (size_t src = 0; src < n; ++src) {
            if (neuron_type[src] > 1) internal("neuron types must be excitatory or inhibitory");
            for (size_t slot = src * s; slot < (src + 1) * s; ++slot) {
                if (rec_target[slot] >= n) internal("recurrent slot targets a neuron outside the model");
                uint8_t br = rec_branch[slot], d = rec_delay[slot];
                if (br > BR_GATE || !(d == 1 || d == 2 || d == 4 || d == 8)) internal("recurrent slot has invalid branch or delay");
                float w = rec_weight[slot];
                if (!(w >= cfg.c.weight_min && w <= cfg.c.weight_max)) internal("recurrent slot has invalid weight");
                if (neuron_type[src] == 0) {
                    if (w < 0.0f || br == BR_INH) internal("excitatory source has incompatible slot");
                } else if (w > 0.0f || br != BR_INH) {
                    internal("inhibitory source has incompatible slot");
                }
            }
        }
        for (size_t i = 0; i < in_target.size(); ++i) {
            if (in_target[i] >= n || in_branch[i] == BR_INH || in_branch[i] > BR_GATE || in_weight[i] < 0.0f ||
                in_weight[i] > cfg.c.weight_max)
                internal("input projection slot has invalid state");
        }
        for (float t : threshold)
            if (!std::isfinite(t) || t < 0.05f || t > 2.0f) internal("neuron thresholds violate canonical parameter bounds");
        for (float x : excitability)
            if (!std::isfinite(x) || x < 0.1f || x > 4.0f) internal("neuron excitability violates canonical parameter bounds");
        auto bounded = [&](const std::vector<float>& v) {
            for (float x : v)
                if (!std::isfinite(x) || x < cfg.c.weight_min || x > cfg.c.weight_max)
                    internal("learned projection weights violate canonical parameter bounds");
        };
        bounded(out_weight);
        bounded(ctx_emb);
        bounded(ctx_out);
        for (float b : bias)
            if (!std::isfinite(b)) internal("model contains NaN or infinite values");
        for (size_t i = 0; i < ctx_keys.size(); ++i)
            if (ctx_keys[i] == 0 && ctx_obs[i] != 0) internal("empty context slots cannot contain observations");
    }
};

struct Event {
    uint32_t target_neuron;
    uint8_t target_branch;
    float value;
    uint32_t synapse_slot;
    float presynaptic_activation;
};

struct Selection {
    size_t suprathreshold = 0, block_selected = 0, global_clipped = 0;
};

struct LearnMetrics {
    double abs_sum = 0.0;
    size_t count = 0;
    float mean() const { return count == 0 ? 0.0f : static_cast<float>(abs_sum / static_cast<double>(count)); }
};

struct ParameterChanges {
    std::vector<size_t> threshold, recurrent_weight, input_weight, output_neurons, context_slots;
    bool output_bias_dirty = false, context_output_dirty = false;
};

// runtime.rs:118-190
struct Runtime {
    Model model;
    // WorkerState (runtime.rs:48-67)
    std::vector<float> membrane, activation, fatigue;
    std::vector<uint64_t> refractory_until;
    std::vector<float> branches;
    std::vector<std::vector<Event>> delay_ring;
    std::vector<Event> due_events;
    uint64_t current_tick = 0;
    size_t plasticity_phase = 0;
    std::vector<size_t> touched;
    std::vector<uint8_t> touched_mark;
    std::vector<size_t> active, previous_active;
    std::vector<uint8_t> selected_mark;
    std::vector<float> selection_surrogate;
    std::vector<uint64_t> branch_last_tick, neuron_last_tick;
    std::vector<float> adaptation[3];
    std::vector<float> rbs, rms, rfs, ras[3], elig;
    std::vector<uint64_t> elig_last;
    std::vector<size_t> elig_rec;
    std::vector<uint8_t> elig_rec_mark;
    std::vector<float> ibs, ims, ifs, ias[3], ielig;
    std::vector<uint64_t> ielig_last;
    std::vector<size_t> elig_in;
    std::vector<uint8_t> elig_in_mark;
    std::vector<float> logits, probabilities, errors, learning_signal;
    std::vector<size_t> learning_destinations;
    std::vector<uint8_t> learning_destination_mark;
    std::vector<float> out_by_neuron;  // neuron-major [N][257]
    bool output_cache_dirty = false;
    std::vector<std::vector<std::pair<size_t, float>>> block_candidates;
    std::vector<float> block_cutoff;
    float population_cutoff = 0.0f;
    std::vector<uint32_t> context_history;
    std::vector<size_t> active_context_slots;
    std::vector<float> active_context_scales;
    std::vector<float> context_latent, context_latent_gradient;
    size_t active_context_probes = 0;
    bool context_applied = false;
    float population_inhibition = 0.0f;
    bool track = false;
    std::vector<size_t> ch_threshold, ch_rec, ch_in, ch_out, ch_ctx;
    std::vector<uint8_t> ch_threshold_mark, ch_rec_mark, ch_in_mark, ch_out_mark, ch_ctx_mark;
    bool output_bias_dirty = false, context_output_dirty = false;
    bool persistent_document_activity = false;
    bool learning_trace_enabled = false;

    // runtime.rs:87-97
    void transpose_output() {
        const size_t n = model.N();
        out_by_neuron.assign(n * OUTPUT_CLASSES, 0.0f);
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o)
            for (size_t i = 0; i < n; ++i) out_by_neuron[i * OUTPUT_CLASSES + o] = model.out_weight[o * n + i];
    }

    // runtime.rs:192-296
    explicit Runtime(Model m) : model(std::move(m)) {
        model.validate();
        const size_t n = model.N(), ns = model.rec_weight.size(), ni = model.in_weight.size();
        uint8_t max_delay = 8;
        for (uint8_t d : model.rec_delay) max_delay = std::max(max_delay, d);
        delay_ring.assign(static_cast<size_t>(max_delay) + 1, {});
        membrane.assign(n, 0.0f);
        activation.assign(n, 0.0f);
        fatigue.assign(n, 0.0f);
        refractory_until.assign(n, 0);
        branches.assign(n * 4, 0.0f);
        touched_mark.assign(n, 0);
        selected_mark.assign(n, 0);
        selection_surrogate.assign(n, 0.0f);
        branch_last_tick.assign(n, 0);
        neuron_last_tick.assign(n, 0);
        for (auto& a : adaptation) a.assign(n, 0.0f);
        rbs.assign(ns, 0.0f); rms.assign(ns, 0.0f); rfs.assign(ns, 0.0f);
        for (auto& a : ras) a.assign(ns, 0.0f);
        elig.assign(ns, 0.0f);
        elig_last.assign(ns, 0);
        elig_rec_mark.assign(ns, 0);
        ibs.assign(ni, 0.0f); ims.assign(ni, 0.0f); ifs.assign(ni, 0.0f);
        for (auto& a : ias) a.assign(ni, 0.0f);
        ielig.assign(ni, 0.0f);
        ielig_last.assign(ni, 0);
        elig_in_mark.assign(ni, 0);
        logits.assign(OUTPUT_CLASSES, 0.0f);
        probabilities.assign(OUTPUT_CLASSES, 0.0f);
        errors.assign(OUTPUT_CLASSES, 0.0f);
        learning_signal.assign(n, 0.0f);
        learning_destination_mark.assign(n, 0);
        transpose_output();
        block_candidates.assign(model.cfg.c.block_count, {});
        block_cutoff.assign(model.cfg.c.block_count, 0.0f);
        context_latent.assign(model.E(), 0.0f);
        context_latent_gradient.assign(model.E(), 0.0f);
    }

    void ensure_output_cache() {
        if (output_cache_dirty) {
            transpose_output();
            output_cache_dirty = false;
        }
    }

    // runtime.rs:310-320
    void enable_parameter_tracking() {
        if (track) return;
        track = true;
        ch_threshold_mark.assign(model.N(), 0);
        ch_rec_mark.assign(model.rec_weight.size(), 0);
        ch_in_mark.assign(model.in_weight.size(), 0);
        ch_out_mark.assign(model.N(), 0);
        ch_ctx_mark.assign(model.ctx_keys.size(), 0);
    }

    // The GPU adapter's enable_parameter_tracking (cuda.rs:2827-2837): a fresh
    // change set and clean dirty flags on every call, also when tracking is on.
    void restart_parameter_tracking() {
        track = false;
        enable_parameter_tracking();
        ch_threshold.clear();
        ch_rec.clear();
        ch_in.clear();
        ch_out.clear();
        ch_ctx.clear();
        output_bias_dirty = false;
        context_output_dirty = false;
    }

    ParameterChanges parameter_changes() const {
        ParameterChanges c;
        c.threshold = ch_threshold;
        c.recurrent_weight = ch_rec;
        c.input_weight = ch_in;
        c.output_neurons = ch_out;
        c.context_slots = ch_ctx;
        c.output_bias_dirty = output_bias_dirty;
        c.context_output_dirty = context_output_dirty;
        return c;
    }

    // runtime.rs:357-363
    void finish_document() {
        if (persistent_document_activity) model.stats.processed_stories = sat_add(model.stats.processed_stories, 1);
        reset_transient_state();
    }

    // runtime.rs:365-425
    void reset_transient_state() {
        std::fill(membrane.begin(), membrane.end(), 0.0f);
        std::fill(activation.begin(), activation.end(), 0.0f);
        std::fill(fatigue.begin(), fatigue.end(), 0.0f);
        std::fill(refractory_until.begin(), refractory_until.end(), 0);
        std::fill(branches.begin(), branches.end(), 0.0f);
        for (auto& a : adaptation) std::fill(a.begin(), a.end(), 0.0f);
        for (auto& b : delay_ring) b.clear();
        due_events.clear();
        for (auto* v : {&rbs, &rms, &rfs, &ras[0], &ras[1], &ras[2], &elig}) std::fill(v->begin(), v->end(), 0.0f);
        std::fill(elig_last.begin(), elig_last.end(), current_tick);
        std::fill(elig_rec_mark.begin(), elig_rec_mark.end(), 0);
        elig_rec.clear();
        for (auto* v : {&ibs, &ims, &ifs, &ias[0], &ias[1], &ias[2], &ielig}) std::fill(v->begin(), v->end(), 0.0f);
        std::fill(ielig_last.begin(), ielig_last.end(), current_tick);
        std::fill(elig_in_mark.begin(), elig_in_mark.end(), 0);
        elig_in.clear();
        std::fill(branch_last_tick.begin(), branch_last_tick.end(), current_tick);
        std::fill(neuron_last_tick.begin(), neuron_last_tick.end(), current_tick);
        std::fill(touched_mark.begin(), touched_mark.end(), 0);
        std::fill(selected_mark.begin(), selected_mark.end(), 0);
        std::fill(selection_surrogate.begin(), selection_surrogate.end(), 0.0f);
        touched.clear();
        active.clear();
        previous_active.clear();
        for (auto& b : block_candidates) b.clear();
        std::fill(block_cutoff.begin(), block_cutoff.end(), 0.0f);
        population_cutoff = 0.0f;
        context_history.clear();
        active_context_slots.clear();
        active_context_scales.clear();
        std::fill(context_latent.begin(), context_latent.end(), 0.0f);
        std::fill(context_latent_gradient.begin(), context_latent_gradient.end(), 0.0f);
        active_context_probes = 0;
        context_applied = false;
        population_inhibition = 0.0f;
        persistent_document_activity = false;
        learning_trace_enabled = false;
        plasticity_phase = 0;
    }

    // runtime.rs:427-535
    OracleStepMetrics step(uint32_t symbol, int32_t target, int32_t permission) {
        if (symbol >= SYMBOL_COUNT) internal("invalid input symbol");
        int64_t target_index = -1;
        if (target >= 0) {
            uint32_t t = static_cast<uint32_t>(target);
            if (t < BYTE_SYMBOLS) target_index = t;
            else if (t == END_DOCUMENT) target_index = END_INDEX;
            else internal("invalid output target");
        }
        ensure_output_cache();
        const bool frozen = permission == ORACLE_FROZEN;
        learning_trace_enabled = !frozen;

        start_tick();
        deliver_due_events();
        inject_symbol(symbol);
        bool context_enabled = frozen || context_survives_dropout(model.cfg.c.seed, current_tick, symbol,
                                                                  model.cfg.c.context_dropout_rate);
        activate_context(symbol, !frozen && context_enabled, context_enabled);
        Selection sel = select_active_neurons();
        if (learning_trace_enabled) update_forward_eligibilities();
        apply_post_activation_dynamics();
        size_t emitted = emit_recurrent_events();
        bool has_neural = false;
        float neural_loss = compute_output_probabilities(target_index, &has_neural);
        uint32_t predicted = argmax_probability();
        predicted = predicted < BYTE_SYMBOLS ? predicted : END_DOCUMENT;
        bool has_loss = target_index >= 0;
        float loss = has_loss ? -std::log(maxf(probabilities[target_index], 1.0e-12f)) : NAN;
        float context_loss_gain = (has_neural && has_loss) ? neural_loss - loss : 0.0f;

        LearnMetrics lm;
        if (target_index >= 0) {
            float strength = model.cfg.strength(permission);
            float target_weight = (static_cast<size_t>(target_index) == END_INDEX) ? model.cfg.c.end_document_weight : 1.0f;
            if (strength > 0.0f) {
                lm = apply_learning(static_cast<size_t>(target_index), strength, target_weight);
                model.parameter_revision = sat_add(model.parameter_revision, 1);
            }
        }
        const size_t active_neurons = active.size();
        if (!frozen) {
            persistent_document_activity = true;
            update_homeostasis(active_neurons);
            update_statistics(symbol, has_loss, loss, emitted);
        }
        current_tick = sat_add(current_tick, 1);  // finish_tick runtime.rs:563-565

        const size_t E = model.E();
        OracleStepMetrics m{};
        m.loss = loss;
        m.has_loss = has_loss ? 1 : 0;
        m.predicted_symbol = predicted;
        m.active_neurons = static_cast<uint32_t>(active_neurons);
        m.emitted_events = static_cast<uint32_t>(emitted);
        m.suprathreshold_neurons = static_cast<uint32_t>(sel.suprathreshold);
        m.block_selected_neurons = static_cast<uint32_t>(sel.block_selected);
        m.global_cap_clipped_neurons = static_cast<uint32_t>(sel.global_clipped);
        m.population_inhibition = population_inhibition;
        m.context_cells = static_cast<uint32_t>(active_context_slots.size());
        m.context_probes = static_cast<uint32_t>(active_context_probes);
        m.context_applied = context_applied ? 1 : 0;
        m.context_loss_gain = context_loss_gain;
        m.output_madds = static_cast<uint32_t>(active_neurons * OUTPUT_CLASSES + active_context_slots.size() * E +
                                               (active_context_slots.empty() ? 0 : E * OUTPUT_CLASSES));
        m.eligible_recurrent_synapses = static_cast<uint32_t>(elig_rec.size());
        m.eligible_input_synapses = static_cast<uint32_t>(elig_in.size());
        m.mean_abs_eligibility = lm.mean();
        m.target_probability = has_loss ? probabilities[target_index] : NAN;
        return m;
    }

    // runtime.rs:537-561
    void start_tick() {
        for (size_t n : touched) {
            touched_mark[n] = 0;
            selection_surrogate[n] = 0.0f;
        }
        touched.clear();
        std::swap(active, previous_active);
        active.clear();
        for (size_t n : previous_active) {
            activation[n] = 0.0f;
            selected_mark[n] = 0;
        }
        for (size_t i = 0; i < previous_active.size(); ++i) mark_touched(previous_active[i]);
        for (auto& b : block_candidates) b.clear();
        std::fill(block_cutoff.begin(), block_cutoff.end(), 0.0f);
        population_cutoff = 0.0f;
    }

    // runtime.rs:567-574
    void mark_touched(size_t n) {
        if (touched_mark[n]) return;
        bring_neuron_to_current_tick(n);
        touched_mark[n] = 1;
        touched.push_back(n);
    }

    // runtime.rs:576-603
    void bring_neuron_to_current_tick(size_t n) {
        const auto& d = model.cfg.c;
        uint64_t be = sat_sub(current_tick, branch_last_tick[n]);
        if (be > 0) {
            float decay = decay_for_elapsed(d.branch_decay, be);
            for (size_t b = 0; b < 4; ++b) branches[n * 4 + b] *= decay;
            branch_last_tick[n] = current_tick;
        }
        uint64_t ne = sat_sub(current_tick, neuron_last_tick[n]);
        if (ne > 0) {
            membrane[n] *= decay_for_elapsed(d.membrane_decay, ne);
            fatigue[n] *= decay_for_elapsed(d.fatigue_decay, ne);
            for (int k = 0; k < 3; ++k) adaptation[k][n] *= decay_for_elapsed(d.adaptation_decay[k], ne);
            neuron_last_tick[n] = current_tick;
        }
    }

    // runtime.rs:605-625
    void deliver_due_events() {
        size_t bucket = static_cast<size_t>(current_tick % delay_ring.size());
        std::swap(due_events, delay_ring[bucket]);
        for (size_t i = 0; i < due_events.size(); ++i) {
            Event ev = due_events[i];
            if (learning_trace_enabled) activate_recurrent_trace(ev.synapse_slot, ev.presynaptic_activation);
            add_to_branch(ev.target_neuron, ev.target_branch, ev.value);
        }
        due_events.clear();
    }

    // runtime.rs:627-639
    void inject_symbol(uint32_t symbol) {
        const size_t F = model.F();
        const size_t start = static_cast<size_t>(symbol) * F;
        for (size_t off = start; off < start + F; ++off) {
            size_t target = model.in_target[off];
            uint8_t br = model.in_branch[off];
            float value = model.in_weight[off];
            if (learning_trace_enabled) activate_input_trace(off, 1.0f);
            add_to_branch(target, br, value);
        }
    }

    // runtime.rs:641-677
    void activate_context(uint32_t symbol, bool allocate, bool enabled) {
        const size_t max_order = model.cfg.c.context_max_order;
        if (context_history.size() == max_order) context_history.erase(context_history.begin());
        context_history.push_back(symbol);
        active_context_slots.clear();
        active_context_scales.clear();
        std::fill(context_latent.begin(), context_latent.end(), 0.0f);
        std::fill(context_latent_gradient.begin(), context_latent_gradient.end(), 0.0f);
        active_context_probes = 0;
        context_applied = enabled;
        if (!enabled) return;
        const size_t available = std::min(context_history.size(), max_order);
        const float confidence_target = static_cast<float>(model.cfg.c.context_confidence_observations);
        float scale_sum = 0.0f;
        for (size_t order = 1; order <= available; ++order) {
            uint64_t key = context_key(context_history.data(), context_history.size(), order);
            auto [slot, probes] = model.resolve_context_slot(order, key, allocate);
            active_context_probes += probes;
            if (slot < 0) continue;
            float obs = static_cast<float>(model.ctx_obs[static_cast<size_t>(slot)]);
            float confidence = obs / (obs + confidence_target);
            float scale = confidence * static_cast<float>(order);
            active_context_slots.push_back(static_cast<size_t>(slot));
            active_context_scales.push_back(scale);
            scale_sum += scale;
        }
        if (scale_sum > 0.0f)
            for (float& s : active_context_scales) s /= scale_sum;
    }

    // runtime.rs:701-708
    void add_to_branch(size_t n, uint8_t br, float value) {
        if (n >= model.N() || br > BR_GATE) return;
        mark_touched(n);
        branches[n * 4 + br] += value;
    }

    // runtime.rs:710-726
    void activate_recurrent_trace(size_t slot, float pre) {
        advance_recurrent_trace(slot);
        rbs[slot] += pre;
        if (!elig_rec_mark[slot]) {
            elig_rec_mark[slot] = 1;
            elig_rec.push_back(slot);
        }
    }
    void activate_input_trace(size_t slot, float act) {
        advance_input_trace(slot);
        ibs[slot] += act;
        if (!elig_in_mark[slot]) {
            elig_in_mark[slot] = 1;
            elig_in.push_back(slot);
        }
    }

    // runtime.rs:728-766
    void advance_trace(size_t slot, std::vector<uint64_t>& last, std::vector<float>& bs, std::vector<float>& ms,
                       std::vector<float>& fs, std::vector<float>* as) {
        uint64_t e = sat_sub(current_tick, last[slot]);
        if (e == 0) return;
        const auto& d = model.cfg.c;
        bs[slot] *= decay_for_elapsed(d.branch_decay, e);
        ms[slot] *= decay_for_elapsed(d.membrane_decay, e);
        fs[slot] *= decay_for_elapsed(d.fatigue_decay, e);
        for (int k = 0; k < 3; ++k) as[k][slot] *= decay_for_elapsed(d.adaptation_decay[k], e);
        last[slot] = current_tick;
    }
    void advance_recurrent_trace(size_t slot) { advance_trace(slot, elig_last, rbs, rms, rfs, ras); }
    void advance_input_trace(size_t slot) { advance_trace(slot, ielig_last, ibs, ims, ifs, ias); }

    bool refractory(size_t n) const { return refractory_until[n] > current_tick; }

    float destination_jacobian(size_t dst, uint8_t br) const {
        return branch_jacobian(br, model.excitability[dst], branches[dst * 4 + BR_TEMP], branches[dst * 4 + BR_GATE]);
    }

    // runtime.rs:787-803
    void cache_selection_surrogates() {
        const size_t bs = model.cfg.c.neurons_per_block;
        const float width = model.cfg.c.surrogate_width, gain = model.cfg.c.surrogate_gain;
        for (size_t dst : touched) {
            if (refractory(dst)) {
                selection_surrogate[dst] = 0.0f;
                continue;
            }
            float margin = membrane[dst] - model.threshold[dst];
            float cutoff = maxf(block_cutoff[dst / bs], population_cutoff);
            selection_surrogate[dst] = analog_rank_surrogate(margin, cutoff, selected_mark[dst] != 0, width, gain);
        }
    }

    // runtime.rs:805-830
    void update_forward_eligibilities() {
        const float eps = model.cfg.c.eligibility_epsilon;
        size_t i = 0;
        while (i < elig_rec.size()) {
            size_t slot = elig_rec[i];
            if (update_slot(slot, eps, model.rec_target[slot], model.rec_branch[slot], rbs, rms, rfs, ras, elig,
                            elig_last)) {
                ++i;
            } else {
                elig_rec_mark[slot] = 0;
                elig_rec[i] = elig_rec.back();  // Vec::swap_remove
                elig_rec.pop_back();
            }
        }
        i = 0;
        while (i < elig_in.size()) {
            size_t slot = elig_in[i];
            if (update_slot(slot, eps, model.in_target[slot], model.in_branch[slot], ibs, ims, ifs, ias, ielig,
                            ielig_last)) {
                ++i;
            } else {
                elig_in_mark[slot] = 0;
                elig_in[i] = elig_in.back();
                elig_in.pop_back();
            }
        }
    }

    // runtime.rs:832-918 (recurrent and input slots share this rule)
    bool update_slot(size_t slot, float eps, size_t dst, uint8_t br, std::vector<float>& bs, std::vector<float>& ms,
                     std::vector<float>& fs, std::vector<float>* as, std::vector<float>& e,
                     std::vector<uint64_t>& last) {
        advance_trace(slot, last, bs, ms, fs, as);
        const auto& d = model.cfg.c;
        float eligibility;
        if (!touched_mark[dst] || refractory(dst)) {
            eligibility = e[slot] * d.eligibility_decay;
        } else {
            float jac = destination_jacobian(dst, br);
            float sur = selection_surrogate[dst];
            float asum = as[0][slot] + as[1][slot] + as[2][slot];
            float msv = ms[slot] + jac * bs[slot] - fs[slot] - asum;
            ms[slot] = msv;
            eligibility = sur * msv;
        }
        e[slot] = eligibility;
        if (touched_mark[dst] && selected_mark[dst]) {
            fs[slot] += d.fatigue_gain * eligibility;
            for (int k = 0; k < 3; ++k) as[k][slot] += d.adaptation_gain[k] * eligibility;
        }
        float mag = maxf(maxf(maxf(std::fabs(bs[slot]), std::fabs(ms[slot])), std::fabs(fs[slot])), std::fabs(eligibility));
        for (int k = 0; k < 3; ++k) mag = maxf(mag, std::fabs(as[k][slot]));
        return mag > eps;
    }

    // runtime.rs:920-938
    void apply_post_activation_dynamics() {
        const auto& d = model.cfg.c;
        for (size_t n : active) {
            float a = activation[n];
            fatigue[n] += d.fatigue_gain * a;
            for (int k = 0; k < 3; ++k) adaptation[k][n] += d.adaptation_gain[k] * a;
            membrane[n] -= model.threshold[n] * d.membrane_reset_fraction;
            refractory_until[n] = sat_add(sat_add(current_tick, d.refractory_ticks), 1);
        }
    }

    static size_t rotated_tie_key(size_t n, size_t rot, size_t count) { return (n + count - rot) % count; }  // runtime.rs:99-101

    // runtime.rs:940-1074
    Selection select_active_neurons() {
        const auto& d = model.cfg.c;
        const size_t bs = d.neurons_per_block;
        const size_t count = std::max<size_t>(model.N(), 1);
        const size_t rot = static_cast<size_t>(current_tick % count);
        for (size_t ti = 0; ti < touched.size(); ++ti) {
            size_t n = touched[ti];
            if (refractory(n)) continue;
            const size_t base = n * 4;
            float gate = clampf(branches[base + BR_GATE], 0.0f, 1.0f);
            float inhibitory = branches[base + BR_INH];
            float net = branches[base + BR_EXC] + branches[base + BR_TEMP] * gate + inhibitory;
            float adapt = adaptation[0][n] + adaptation[1][n] + adaptation[2][n];
            float drive = model.excitability[n] * net - fatigue[n] - adapt - population_inhibition;
            membrane[n] += drive;
            float act = clampf(membrane[n] - model.threshold[n], 0.0f, 1.0f);
            if (act > 0.0f) block_candidates[n / bs].push_back({n, act});
        }
        Selection sel;
        for (auto& b : block_candidates) sel.suprathreshold += b.size();

        const size_t limit = d.max_active_per_block;
        auto cmp = [&](const std::pair<size_t, float>& l, const std::pair<size_t, float>& r) {
            int c = total_cmp(r.second, l.second);
            if (c != 0) return c < 0;
            return rotated_tie_key(l.first, rot, count) < rotated_tie_key(r.first, rot, count);
        };
        for (size_t bi = 0; bi < block_candidates.size(); ++bi) {
            auto& block = block_candidates[bi];
            if (block.size() > limit) {
                // select_nth_unstable_by + truncate: the order is strict (tie keys are
                // unique), so the k smallest under cmp and the (k+1)-th are unique.
                std::nth_element(block.begin(), block.begin() + static_cast<long>(limit), block.end(), cmp);
                block_cutoff[bi] = block[limit].second;
                block.resize(limit);
            }
            std::sort(block.begin(), block.end(), cmp);
            for (auto& p : block) active.push_back(p.first);
        }
        sel.block_selected = active.size();
        const size_t cap = d.max_active_global;
        const size_t capacity = static_cast<size_t>(d.block_count) * limit;
        if (cap >= capacity) {
            population_cutoff = 0.0f;
            sel.global_clipped = 0;
        } else {
            auto act_of = [&](size_t n) { return clampf(membrane[n] - model.threshold[n], 0.0f, 1.0f); };
            std::sort(active.begin(), active.end(), [&](size_t l, size_t r) {
                int c = total_cmp(act_of(r), act_of(l));
                if (c != 0) return c < 0;
                return rotated_tie_key(l, rot, count) < rotated_tie_key(r, rot, count);
            });
            if (active.size() > cap) {
                size_t cn = active[cap];
                population_cutoff = clampf(membrane[cn] - model.threshold[cn], 0.0f, d.population_inhibition_max);
            } else {
                population_cutoff = 0.0f;
            }
            size_t clipped = active.size() > cap ? active.size() - cap : 0;
            if (clipped > 0) active.resize(cap);
            sel.global_clipped = clipped;
        }
        update_population_inhibition(active.size());
        for (size_t n : active) {
            float margin = membrane[n] - model.threshold[n];
            activation[n] = clampf(margin, 0.0f, 1.0f);
            selected_mark[n] = 1;
        }
        cache_selection_surrogates();
        return sel;
    }

    // runtime.rs:1076-1082
    void update_population_inhibition(size_t active_count) {
        const auto& d = model.cfg.c;
        float activity = static_cast<float>(active_count) / static_cast<float>(std::max<size_t>(model.N(), 1));
        float err = activity - d.target_activity;
        population_inhibition = clampf(population_inhibition + d.population_inhibition_rate * err, 0.0f,
                                       d.population_inhibition_max);
    }

    // runtime.rs:1084-1106
    size_t emit_recurrent_events() {
        size_t emitted = 0;
        const size_t S = model.S();
        for (size_t ai = 0; ai < active.size(); ++ai) {
            size_t src = active[ai];
            float a = activation[src];
            for (size_t slot = src * S; slot < (src + 1) * S; ++slot) {
                size_t delay = std::max<uint8_t>(model.rec_delay[slot], 1);
                size_t bucket = static_cast<size_t>((current_tick + delay) % delay_ring.size());
                delay_ring[bucket].push_back(
                    Event{model.rec_target[slot], model.rec_branch[slot], a * model.rec_weight[slot],
                          static_cast<uint32_t>(slot), a});
                ++emitted;
            }
        }
        return emitted;
    }

    // runtime.rs:1108-1149
    float compute_output_probabilities(int64_t target_index, bool* has_neural) {
        std::copy(model.bias.begin(), model.bias.end(), logits.begin());
        for (size_t n : active) {
            float a = activation[n];
            const size_t row = n * OUTPUT_CLASSES;
            for (size_t o = 0; o < OUTPUT_CLASSES; ++o) logits[o] += out_by_neuron[row + o] * a;
        }
        float neural = 0.0f;
        *has_neural = target_index >= 0;
        if (*has_neural) neural = loss_from_logits(static_cast<size_t>(target_index));
        std::fill(context_latent.begin(), context_latent.end(), 0.0f);
        const size_t E = model.E();
        if (!active_context_slots.empty()) {
            for (size_t i = 0; i < active_context_slots.size(); ++i) {
                size_t slot = active_context_slots[i];
                float scale = active_context_scales[i];
                if (scale <= 0.0f) continue;
                for (size_t dd = 0; dd < E; ++dd) context_latent[dd] += model.ctx_emb[slot * E + dd] * scale;
            }
            for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
                float contribution = 0.0f;
                for (size_t dd = 0; dd < E; ++dd) contribution += model.ctx_out[o * E + dd] * context_latent[dd];
                logits[o] += contribution;
            }
        }
        normalize_probabilities();
        return neural;
    }

    // runtime.rs:1151-1167
    float loss_from_logits(size_t target) const {
        float maximum = -INFINITY;
        for (float l : logits) maximum = maxf(maximum, l);
        float sum = 0.0f;  // Sum<f32>: fold from -0.0; -0.0 + x == x for every x
        bool first = true;
        for (float l : logits) {
            float v = std::exp(l - maximum);
            sum = first ? v : sum + v;
            first = false;
        }
        if (!std::isfinite(sum) || sum <= 0.0f) return std::log(static_cast<float>(OUTPUT_CLASSES));
        return maximum + std::log(sum) - logits[target];
    }

    // runtime.rs:1169-1188
    void normalize_probabilities() {
        float maximum = -INFINITY;
        for (float l : logits) maximum = maxf(maximum, l);
        float sum = 0.0f;
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
            float v = std::exp(logits[o] - maximum);
            probabilities[o] = v;
            sum += v;
        }
        if (!std::isfinite(sum) || sum <= 0.0f) {
            std::fill(probabilities.begin(), probabilities.end(), 1.0f / static_cast<float>(OUTPUT_CLASSES));
        } else {
            for (float& p : probabilities) p /= sum;
        }
    }

    // runtime.rs:1190-1197: maximum by total order, first index among equals.
    uint32_t argmax_probability() const {
        size_t best = 0;
        for (size_t o = 1; o < OUTPUT_CLASSES; ++o)
            if (total_cmp(probabilities[o], probabilities[best]) > 0) best = o;
        return static_cast<uint32_t>(best);
    }

    void mark(size_t idx, std::vector<uint8_t>& marks, std::vector<size_t>& list) {
        if (!track) return;
        if (!marks[idx]) {
            marks[idx] = 1;
            list.push_back(idx);
        }
    }

    void add_learning_destination(size_t dst) {
        if (learning_destination_mark[dst]) return;
        learning_destination_mark[dst] = 1;
        learning_destinations.push_back(dst);
    }

    // runtime.rs:1199-1316
    LearnMetrics apply_learning(size_t target, float strength, float target_weight) {
        const auto& d = model.cfg.c;
        std::copy(probabilities.begin(), probabilities.end(), errors.begin());
        errors[target] -= 1.0f;
        const float ss = strength * target_weight;
        auto [plasticity_scale, next_phase] = model.cfg.plasticity_step(plasticity_phase, target == END_INDEX);
        const size_t n_count = model.N();
        for (size_t n : learning_destinations) {
            learning_signal[n] = 0.0f;
            learning_destination_mark[n] = 0;
        }
        learning_destinations.clear();
        if (plasticity_scale > 0.0f) {
            for (size_t i = 0; i < elig_rec.size(); ++i) add_learning_destination(model.rec_target[elig_rec[i]]);
            for (size_t i = 0; i < elig_in.size(); ++i) add_learning_destination(model.in_target[elig_in[i]]);
            for (size_t i = 0; i < active.size(); ++i) add_learning_destination(active[i]);
            for (size_t n : learning_destinations) {
                const size_t row = n * OUTPUT_CLASSES;
                float signal = 0.0f;
                for (size_t o = 0; o < OUTPUT_CLASSES; ++o) signal += out_by_neuron[row + o] * errors[o];
                learning_signal[n] = signal;
            }
        }
        const float olr = d.output_learning_rate, mu = d.max_update, wmin = d.weight_min, wmax = d.weight_max;
        for (size_t n : active) {
            float a = activation[n];
            const size_t row = n * OUTPUT_CLASSES;
            mark(n, ch_out_mark, ch_out);
            for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
                float raw = -olr * ss * errors[o] * a;
                float delta = bounded_delta(raw, mu);
                float updated = clampf(model.out_weight[o * n_count + n] + delta, wmin, wmax);
                model.out_weight[o * n_count + n] = updated;
                out_by_neuron[row + o] = updated;
            }
        }
        if (track) output_bias_dirty = true;
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
            float raw = -olr * ss * errors[o];
            model.bias[o] += bounded_delta(raw, mu);
            if (!std::isfinite(model.bias[o])) numerical("output bias " + std::to_string(o) + " became non-finite");
        }
        if (context_applied) update_context_projection(ss);
        LearnMetrics lm;
        if (plasticity_scale > 0.0f) {
            float cs = ss * plasticity_scale;
            update_recurrent_synapses(cs, lm);
            update_input_synapses(cs, lm);
        }
        apply_inhibitory_homeostasis(strength);
        plasticity_phase = next_phase;
        return lm;
    }

    // runtime.rs:1318-1384
    void update_context_projection(float strength) {
        if (active_context_slots.empty()) return;
        const auto& d = model.cfg.c;
        const float lr = d.context_learning_rate, mu = d.max_update, wmin = d.weight_min, wmax = d.weight_max;
        const size_t E = model.E();
        std::fill(context_latent_gradient.begin(), context_latent_gradient.end(), 0.0f);
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o)
            for (size_t dd = 0; dd < E; ++dd) context_latent_gradient[dd] += model.ctx_out[o * E + dd] * errors[o];
        if (track) context_output_dirty = true;
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
            for (size_t dd = 0; dd < E; ++dd) {
                float g = errors[o] * context_latent[dd];
                float delta = bounded_delta(-lr * strength * g, mu);
                float updated = clampf(model.ctx_out[o * E + dd] + delta, wmin, wmax);
                if (!std::isfinite(updated)) numerical("non-finite context output update rejected");
                model.ctx_out[o * E + dd] = updated;
            }
        }
        for (size_t i = 0; i < active_context_slots.size(); ++i) {
            size_t slot = active_context_slots[i];
            float ls = active_context_scales[i];
            for (size_t dd = 0; dd < E; ++dd) {
                float g = ls * context_latent_gradient[dd];
                float delta = bounded_delta(-lr * strength * g, mu);
                float updated = clampf(model.ctx_emb[slot * E + dd] + delta, wmin, wmax);
                if (!std::isfinite(updated)) internal("non-finite context embedding update rejected");
                model.ctx_emb[slot * E + dd] = updated;
            }
            mark(slot, ch_ctx_mark, ch_ctx);
            model.ctx_obs[slot] = sat_add32(model.ctx_obs[slot], 1);
        }
    }

    // runtime.rs:1451-1491
    void update_recurrent_synapses(float strength, LearnMetrics& lm) {
        const auto& d = model.cfg.c;
        const float lr = d.recurrent_learning_rate, mu = d.max_update, wmin = d.weight_min, wmax = d.weight_max;
        const size_t S = model.S();
        for (size_t i = 0; i < elig_rec.size(); ++i) {
            size_t slot = elig_rec[i];
            size_t dst = model.rec_target[slot];
            float e = elig[slot];
            lm.abs_sum += static_cast<double>(std::fabs(e));
            lm.count += 1;
            float g = learning_signal[dst] * e;
            float delta = bounded_delta(-lr * strength * g, mu);
            float old_w = model.rec_weight[slot];
            float nw = clampf(old_w + delta, wmin, wmax);
            nw = model.neuron_type[slot / S] == 0 ? max_zero(nw) : min_zero(nw);
            if (!std::isfinite(nw)) {
                model.stats.numerical_rejections = sat_add(model.stats.numerical_rejections, 1);
                numerical("non-finite recurrent update rejected");
            }
            if (nw != old_w) mark(slot, ch_rec_mark, ch_rec);
            model.rec_weight[slot] = nw;
        }
    }

    // runtime.rs:1493-1523
    void update_input_synapses(float strength, LearnMetrics& lm) {
        const auto& d = model.cfg.c;
        const float lr = d.recurrent_learning_rate, mu = d.max_update, wmax = d.weight_max;
        for (size_t i = 0; i < elig_in.size(); ++i) {
            size_t slot = elig_in[i];
            size_t dst = model.in_target[slot];
            float e = ielig[slot];
            lm.abs_sum += static_cast<double>(std::fabs(e));
            lm.count += 1;
            float g = learning_signal[dst] * e;
            float delta = bounded_delta(-lr * strength * g, mu);
            float old_w = model.in_weight[slot];
            float nw = clampf(old_w + delta, 0.0f, wmax);
            if (!std::isfinite(nw)) numerical("non-finite input update rejected");
            if (nw != old_w) mark(slot, ch_in_mark, ch_in);
            model.in_weight[slot] = nw;
        }
    }

    // runtime.rs:1525-1565
    void apply_inhibitory_homeostasis(float strength) {
        const auto& d = model.cfg.c;
        const size_t S = model.S();
        for (size_t ai = 0; ai < active.size(); ++ai) {
            size_t src = active[ai];
            if (model.neuron_type[src] == 0) continue;
            float sa = activation[src];
            for (size_t slot = src * S; slot < (src + 1) * S; ++slot) {
                size_t tgt = model.rec_target[slot];
                float delta = inhibitory_homeostasis_delta(sa, activation[tgt] > 0.0f ? 1.0f : 0.0f, d.target_activity,
                                                           d.inhibitory_learning_rate, strength, d.max_update);
                float old_w = model.rec_weight[slot];
                float nw = clampf(old_w + delta, d.weight_min, 0.0f);
                if (!std::isfinite(nw)) numerical("non-finite inhibitory update rejected");
                if (nw != old_w) mark(slot, ch_rec_mark, ch_rec);
                model.rec_weight[slot] = nw;
            }
        }
    }

    // runtime.rs:1567-1593
    void update_homeostasis(size_t active_count) {
        const auto& d = model.cfg.c;
        float pop_activity = static_cast<float>(active_count) / static_cast<float>(std::max<size_t>(model.N(), 1));
        float pop_err = pop_activity - d.target_activity;
        for (size_t n : touched) {
            float local = activation[n] > 0.0f ? 1.0f : 0.0f;
            float local_err = local - d.target_activity;
            float delta = d.threshold_homeostasis_rate * (local_err + pop_err);
            float old_t = model.threshold[n];
            float nt = clampf(old_t + delta, 0.05f, 2.0f);
            if (nt != old_t) mark(n, ch_threshold_mark, ch_threshold);
            model.threshold[n] = nt;
        }
    }

    // runtime.rs:1595-1622
    void update_statistics(uint32_t symbol, bool has_loss, float loss, size_t emitted) {
        auto& s = model.stats;
        if (symbol < 256) s.processed_bytes = sat_add(s.processed_bytes, 1);
        if (has_loss) {
            s.training_loss_sum += static_cast<double>(loss);
            s.training_targets = sat_add(s.training_targets, 1);
        }
        s.active_neurons_sum = sat_add(s.active_neurons_sum, active.size());
        s.active_neurons_peak = std::max<uint64_t>(s.active_neurons_peak, active.size());
        s.synaptic_events = sat_add(s.synaptic_events, emitted);
        s.persistent_ticks = sat_add(s.persistent_ticks, 1);
    }
};

// ---------------------------------------------------------------------------
// parallel.rs: sparse deltas and the batch-end mean
// ---------------------------------------------------------------------------
struct SparseF32 {
    size_t index;
    float delta;
    bool operator==(const SparseF32& o) const {
        return index == o.index && std::memcmp(&delta, &o.delta, 4) == 0;
    }
};
struct ContextKeyDelta {
    size_t order;
    uint64_t key;
    std::vector<float> embedding_delta;
    uint32_t observation_increment;
    bool operator==(const ContextKeyDelta& o) const {
        return order == o.order && key == o.key && observation_increment == o.observation_increment &&
               embedding_delta.size() == o.embedding_delta.size() &&
               std::memcmp(embedding_delta.data(), o.embedding_delta.data(), 4 * embedding_delta.size()) == 0;
    }
};
struct StatsDelta {
    uint64_t processed_bytes = 0, processed_stories = 0;
    double training_loss_sum = 0.0;
    uint64_t training_targets = 0, active_neurons_sum = 0, active_neurons_peak = 0, synaptic_events = 0,
             numerical_rejections = 0, persistent_ticks = 0;
    bool operator==(const StatsDelta& o) const {
        return processed_bytes == o.processed_bytes && processed_stories == o.processed_stories &&
               std::memcmp(&training_loss_sum, &o.training_loss_sum, 8) == 0 && training_targets == o.training_targets &&
               active_neurons_sum == o.active_neurons_sum && active_neurons_peak == o.active_neurons_peak &&
               synaptic_events == o.synaptic_events && numerical_rejections == o.numerical_rejections &&
               persistent_ticks == o.persistent_ticks;
    }
};

std::string config_fingerprint(const Config& c) {
    return std::string(reinterpret_cast<const char*>(&c.c), sizeof(OracleConfig));
}

}  // namespace

struct OracleDelta {
    std::string fingerprint;
    uint64_t base_revision = 0, revision_increment = 0;
    std::vector<SparseF32> threshold, excitability, recurrent_weight, input_weight, output_weight, output_bias,
        context_output_weight;
    std::vector<ContextKeyDelta> context;
    StatsDelta statistics;
    bool operator==(const OracleDelta& o) const {
        return fingerprint == o.fingerprint && base_revision == o.base_revision &&
               revision_increment == o.revision_increment && threshold == o.threshold &&
               excitability == o.excitability && recurrent_weight == o.recurrent_weight &&
               input_weight == o.input_weight && output_weight == o.output_weight && output_bias == o.output_bias &&
               context_output_weight == o.context_output_weight && context == o.context && statistics == o.statistics;
    }
    // parallel.rs:676-691
    void canonicalize_order() {
        auto by_index = [](const SparseF32& a, const SparseF32& b) { return a.index < b.index; };
        for (auto* v : {&threshold, &excitability, &recurrent_weight, &input_weight, &output_weight, &output_bias,
                        &context_output_weight})
            std::sort(v->begin(), v->end(), by_index);
        std::sort(context.begin(), context.end(), [](const ContextKeyDelta& a, const ContextKeyDelta& b) {
            return std::make_pair(a.order, a.key) < std::make_pair(b.order, b.key);
        });
    }
};

struct OracleRuntime {
    std::unique_ptr<Runtime> rt;
};

namespace {

void ensure_aligned(const Model& base, const Model& trained) {  // parallel.rs:868-882
    if (config_fingerprint(base.cfg) != config_fingerprint(trained.cfg) || base.rec_target != trained.rec_target ||
        base.rec_branch != trained.rec_branch || base.rec_delay != trained.rec_delay ||
        base.in_target != trained.in_target || base.in_branch != trained.in_branch ||
        base.neuron_type != trained.neuron_type)
        internal("worker model topology is not aligned with the canonical checkpoint");
}

std::vector<SparseF32> diff_f32(const std::vector<float>& before, const std::vector<float>& after) {  // parallel.rs:884-894
    std::vector<SparseF32> out;
    for (size_t i = 0; i < before.size(); ++i) {
        float d = after[i] - before[i];
        if (d != 0.0f) out.push_back({i, d});
    }
    return out;
}

std::vector<SparseF32> diff_selected(const std::vector<float>& before, const std::vector<float>& after,
                                     const std::vector<size_t>& idx) {  // parallel.rs:896-914
    std::vector<SparseF32> out;
    for (size_t i : idx) {
        if (i >= before.size() || i >= after.size()) internal("tracked parameter index is outside the model");
        float d = after[i] - before[i];
        if (d != 0.0f) out.push_back({i, d});
    }
    return out;
}

int64_t find_context_slot(const Model& m, size_t order, uint64_t key) {  // parallel.rs:916-927
    const size_t spo = m.cfg.c.context_slots_per_order;
    const size_t base = (order - 1) * spo;
    const size_t start = static_cast<size_t>(key % spo);
    for (size_t off = 0; off < m.cfg.c.context_probe_limit; ++off) {
        size_t slot = base + (start + off) % spo;
        if (m.ctx_keys[slot] == key) return static_cast<int64_t>(slot);
    }
    return -1;
}

StatsDelta statistics_delta(const OracleStatistics& b, const OracleStatistics& a) {  // parallel.rs:1115-1137
    StatsDelta d;
    d.processed_bytes = sat_sub(a.processed_bytes, b.processed_bytes);
    d.processed_stories = sat_sub(a.processed_stories, b.processed_stories);
    d.training_loss_sum = a.training_loss_sum - b.training_loss_sum;
    d.training_targets = sat_sub(a.training_targets, b.training_targets);
    d.active_neurons_sum = sat_sub(a.active_neurons_sum, b.active_neurons_sum);
    d.active_neurons_peak = a.active_neurons_peak;
    d.synaptic_events = sat_sub(a.synaptic_events, b.synaptic_events);
    d.numerical_rejections = sat_sub(a.numerical_rejections, b.numerical_rejections);
    d.persistent_ticks = sat_sub(a.persistent_ticks, b.persistent_ticks);
    return d;
}

ContextKeyDelta context_delta_for(const Model& base, size_t order, uint64_t key, const float* trained_emb,
                                  uint32_t trained_obs, bool* keep) {
    const size_t E = base.E();
    int64_t bslot = find_context_slot(base, order, key);
    uint32_t bobs = bslot >= 0 ? base.ctx_obs[static_cast<size_t>(bslot)] : 0;
    ContextKeyDelta c{order, key, {}, 0};
    bool changed = false;
    for (size_t dd = 0; dd < E; ++dd) {
        float before = bslot >= 0 ? base.ctx_emb[static_cast<size_t>(bslot) * E + dd] : 0.0f;
        float delta = trained_emb[dd] - before;
        changed |= delta != 0.0f;
        c.embedding_delta.push_back(delta);
    }
    c.observation_increment = trained_obs > bobs ? trained_obs - bobs : 0;
    *keep = changed || c.observation_increment > 0;
    return c;
}

// parallel.rs:313-383
OracleDelta delta_between(const Model& base, const Model& trained) {
    ensure_aligned(base, trained);
    const size_t spo = base.cfg.c.context_slots_per_order, E = base.E();
    OracleDelta d;
    for (size_t slot = 0; slot < trained.ctx_keys.size(); ++slot) {
        uint64_t key = trained.ctx_keys[slot];
        if (key == 0) continue;
        size_t order = slot / spo + 1;
        // parallel.rs:317-322 keys the base by (order,key) across the whole partition;
        // a valid model stores each key once per order, so scanning the partition is equivalent.
        int64_t bslot = -1;
        for (size_t s = (order - 1) * spo; s < order * spo; ++s)
            if (base.ctx_keys[s] == key) { bslot = static_cast<int64_t>(s); break; }
        ContextKeyDelta c{order, key, {}, 0};
        bool changed = false;
        for (size_t dd = 0; dd < E; ++dd) {
            float before = bslot >= 0 ? base.ctx_emb[static_cast<size_t>(bslot) * E + dd] : 0.0f;
            float delta = trained.ctx_emb[slot * E + dd] - before;
            changed |= delta != 0.0f;
            c.embedding_delta.push_back(delta);
        }
        uint32_t bobs = bslot >= 0 ? base.ctx_obs[static_cast<size_t>(bslot)] : 0;
        c.observation_increment = trained.ctx_obs[slot] > bobs ? trained.ctx_obs[slot] - bobs : 0;
        if (changed || c.observation_increment > 0) d.context.push_back(std::move(c));
    }
    d.fingerprint = config_fingerprint(base.cfg);
    d.base_revision = base.parameter_revision;
    d.revision_increment = sat_sub(trained.parameter_revision, base.parameter_revision);
    d.threshold = diff_f32(base.threshold, trained.threshold);
    d.excitability = diff_f32(base.excitability, trained.excitability);
    d.recurrent_weight = diff_f32(base.rec_weight, trained.rec_weight);
    d.input_weight = diff_f32(base.in_weight, trained.in_weight);
    d.output_weight = diff_f32(base.out_weight, trained.out_weight);
    d.output_bias = diff_f32(base.bias, trained.bias);
    d.context_output_weight = diff_f32(base.ctx_out, trained.ctx_out);
    d.statistics = statistics_delta(base.stats, trained.stats);
    d.canonicalize_order();
    return d;
}

// parallel.rs:385-454
OracleDelta delta_between_tracked(const Model& base, const Model& trained, const ParameterChanges& ch) {
    ensure_aligned(base, trained);
    const size_t n = base.N();
    OracleDelta d;
    for (size_t neuron : ch.output_neurons) {
        if (neuron >= n) internal("tracked output neuron is outside the model");
        for (size_t o = 0; o < OUTPUT_CLASSES; ++o) {
            size_t idx = o * n + neuron;
            float delta = trained.out_weight[idx] - base.out_weight[idx];
            if (delta != 0.0f) d.output_weight.push_back({idx, delta});
        }
    }
    d.fingerprint = config_fingerprint(base.cfg);
    d.base_revision = base.parameter_revision;
    d.revision_increment = sat_sub(trained.parameter_revision, base.parameter_revision);
    d.threshold = diff_selected(base.threshold, trained.threshold, ch.threshold);
    d.recurrent_weight = diff_selected(base.rec_weight, trained.rec_weight, ch.recurrent_weight);
    d.input_weight = diff_selected(base.in_weight, trained.in_weight, ch.input_weight);
    if (ch.output_bias_dirty) d.output_bias = diff_f32(base.bias, trained.bias);
    if (ch.context_output_dirty) d.context_output_weight = diff_f32(base.ctx_out, trained.ctx_out);
    // parallel.rs:929-973 context_deltas_for_slots
    const size_t spo = base.cfg.c.context_slots_per_order, E = base.E();
    for (size_t slot : ch.context_slots) {
        if (slot >= trained.ctx_keys.size()) internal("tracked context slot is outside the model");
        uint64_t key = trained.ctx_keys[slot];
        if (key == 0) continue;
        size_t order = slot / spo + 1;
        bool keep = false;
        ContextKeyDelta c = context_delta_for(base, order, key, &trained.ctx_emb[slot * E], trained.ctx_obs[slot], &keep);
        if (keep) d.context.push_back(std::move(c));
    }
    d.statistics = statistics_delta(base.stats, trained.stats);
    d.canonicalize_order();
    return d;
}

// parallel.rs:975-1022
size_t apply_sparse_scaled(std::vector<float>& target, const std::vector<const std::vector<SparseF32>*>& groups,
                           size_t divisor) {
    std::vector<size_t> pos(groups.size(), 0);
    size_t updates = 0;
    while (true) {
        bool found = false;
        size_t index = 0;
        for (size_t g = 0; g < groups.size(); ++g) {
            if (pos[g] < groups[g]->size()) {
                size_t i = (*groups[g])[pos[g]].index;
                if (!found || i < index) { index = i; found = true; }
            }
        }
        if (!found) break;
        if (index >= target.size()) internal("invalid sparse worker parameter delta");
        double sum = 0.0;
        for (size_t g = 0; g < groups.size(); ++g) {
            if (pos[g] < groups[g]->size() && (*groups[g])[pos[g]].index == index) {
                float dv = (*groups[g])[pos[g]].delta;
                if (!std::isfinite(dv)) internal("invalid sparse worker parameter delta");
                sum += static_cast<double>(dv);
                pos[g] += 1;
            }
        }
        target[index] += static_cast<float>(sum / static_cast<double>(divisor));
        if (!std::isfinite(target[index])) internal("merged parameter became non-finite");
        updates += 1;
    }
    return updates;
}

// parallel.rs:1024-1113
size_t apply_context_deltas(Model& master, const std::vector<const OracleDelta*>& deltas, size_t divisor) {
    struct Merged {
        size_t order;
        uint64_t key;
        std::vector<double> sum;
        uint64_t observations;
    };
    const size_t E = master.E();
    std::vector<size_t> pos(deltas.size(), 0);
    std::vector<Merged> merged;
    while (true) {
        bool found = false;
        std::pair<size_t, uint64_t> next{0, 0};
        for (size_t g = 0; g < deltas.size(); ++g) {
            if (pos[g] < deltas[g]->context.size()) {
                const auto& u = deltas[g]->context[pos[g]];
                auto k = std::make_pair(u.order, u.key);
                if (!found || k < next) { next = k; found = true; }
            }
        }
        if (!found) break;
        Merged m{next.first, next.second, std::vector<double>(E, 0.0), 0};
        for (size_t g = 0; g < deltas.size(); ++g) {
            if (pos[g] < deltas[g]->context.size()) {
                const auto& u = deltas[g]->context[pos[g]];
                if (u.order == next.first && u.key == next.second) {
                    if (u.embedding_delta.size() != E || u.order == 0 || u.order > master.cfg.c.context_max_order ||
                        u.key == 0)
                        internal("invalid keyed context worker delta");
                    for (size_t dd = 0; dd < E; ++dd) {
                        if (!std::isfinite(u.embedding_delta[dd])) internal("invalid keyed context worker delta");
                        m.sum[dd] += static_cast<double>(u.embedding_delta[dd]);
                    }
                    m.observations = sat_add(m.observations, u.observation_increment);
                    pos[g] += 1;
                }
            }
        }
        merged.push_back(std::move(m));
    }
    // sort_unstable_by on a strict total order (keys unique) == any sort
    std::sort(merged.begin(), merged.end(), [](const Merged& l, const Merged& r) {
        if (l.observations != r.observations) return l.observations > r.observations;
        return std::make_pair(l.order, l.key) < std::make_pair(r.order, r.key);
    });
    for (const auto& u : merged) {
        auto [slot, probes] = master.resolve_context_slot(u.order, u.key, true);
        (void)probes;
        size_t s = static_cast<size_t>(slot);
        for (size_t dd = 0; dd < E; ++dd)
            master.ctx_emb[s * E + dd] += static_cast<float>(u.sum[dd] / static_cast<double>(divisor));
        uint32_t inc = static_cast<uint32_t>(std::min<uint64_t>(u.observations, UINT32_MAX));
        master.ctx_obs[s] = sat_add32(master.ctx_obs[s], inc);
    }
    return merged.size();
}

// parallel.rs:715-798 (+ projection 1169-1246 and validation 1248-1345)
std::pair<size_t, size_t> apply_deltas_with_divisor(Model& master, const std::vector<const OracleDelta*>& deltas,
                                                    size_t divisor) {
    if (deltas.empty()) internal("cannot merge an empty worker batch");
    if (divisor == 0) internal("worker merge divisor cannot be zero");
    std::string fp = config_fingerprint(master.cfg);
    for (auto* d : deltas)
        if (d->fingerprint != fp) internal("worker delta configuration does not match the canonical model");
    for (auto* d : deltas)
        if (d->base_revision != master.parameter_revision)
            internal("worker delta was not produced from the current canonical revision");
    auto groups = [&](std::vector<SparseF32> OracleDelta::*member) {
        std::vector<const std::vector<SparseF32>*> g;
        for (auto* d : deltas) g.push_back(&(d->*member));
        return g;
    };
    size_t fixed = 0;
    fixed += apply_sparse_scaled(master.threshold, groups(&OracleDelta::threshold), divisor);
    fixed += apply_sparse_scaled(master.excitability, groups(&OracleDelta::excitability), divisor);
    fixed += apply_sparse_scaled(master.rec_weight, groups(&OracleDelta::recurrent_weight), divisor);
    fixed += apply_sparse_scaled(master.in_weight, groups(&OracleDelta::input_weight), divisor);
    fixed += apply_sparse_scaled(master.out_weight, groups(&OracleDelta::output_weight), divisor);
    fixed += apply_sparse_scaled(master.bias, groups(&OracleDelta::output_bias), divisor);
    fixed += apply_sparse_scaled(master.ctx_out, groups(&OracleDelta::context_output_weight), divisor);
    size_t ctx = apply_context_deltas(master, deltas, divisor);
    for (auto* d : deltas) {  // parallel.rs:1139-1167
        auto& s = master.stats;
        const auto& x = d->statistics;
        s.processed_bytes = sat_add(s.processed_bytes, x.processed_bytes);
        s.processed_stories = sat_add(s.processed_stories, x.processed_stories);
        s.training_loss_sum += x.training_loss_sum;
        s.training_targets = sat_add(s.training_targets, x.training_targets);
        s.active_neurons_sum = sat_add(s.active_neurons_sum, x.active_neurons_sum);
        s.active_neurons_peak = std::max(s.active_neurons_peak, x.active_neurons_peak);
        s.synaptic_events = sat_add(s.synaptic_events, x.synaptic_events);
        s.numerical_rejections = sat_add(s.numerical_rejections, x.numerical_rejections);
        s.persistent_ticks = sat_add(s.persistent_ticks, x.persistent_ticks);
    }
    uint64_t inc = 0;
    for (auto* d : deltas) inc = sat_add(inc, d->revision_increment);
    master.parameter_revision = sat_add(master.parameter_revision, inc);
    // project_parameter_constraints_sparse (parallel.rs:1169-1246)
    const float wmin = master.cfg.c.weight_min, wmax = master.cfg.c.weight_max;
    const size_t S = master.S(), E = master.E();
    for (auto* d : deltas) {
        for (auto& u : d->threshold) master.threshold[u.index] = clampf(master.threshold[u.index], 0.05f, 2.0f);
        for (auto& u : d->excitability) master.excitability[u.index] = clampf(master.excitability[u.index], 0.1f, 4.0f);
        for (auto& u : d->recurrent_weight) {
            float w = clampf(master.rec_weight[u.index], wmin, wmax);
            w = master.neuron_type[u.index / S] == 0 ? max_zero(w) : min_zero(w);
            master.rec_weight[u.index] = w;
        }
        for (auto& u : d->input_weight) master.in_weight[u.index] = clampf(master.in_weight[u.index], 0.0f, wmax);
        for (auto& u : d->output_weight) master.out_weight[u.index] = clampf(master.out_weight[u.index], wmin, wmax);
        for (auto& u : d->context) {
            auto [slot, probes] = master.resolve_context_slot(u.order, u.key, false);
            (void)probes;
            if (slot >= 0)
                for (size_t dd = 0; dd < E; ++dd) {
                    float& w = master.ctx_emb[static_cast<size_t>(slot) * E + dd];
                    w = clampf(w, wmin, wmax);
                }
        }
        for (auto& u : d->context_output_weight) master.ctx_out[u.index] = clampf(master.ctx_out[u.index], wmin, wmax);
    }
    // validate_sparse_merge (parallel.rs:1248-1345)
    if (!std::isfinite(master.stats.training_loss_sum)) internal("merged model statistics contain a non-finite loss");
    for (auto* d : deltas) {
        for (auto& u : d->threshold) {
            float v = master.threshold[u.index];
            if (!std::isfinite(v) || v < 0.05f || v > 2.0f) internal("merged threshold violates canonical parameter bounds");
        }
        for (auto& u : d->excitability) {
            float v = master.excitability[u.index];
            if (!std::isfinite(v) || v < 0.1f || v > 4.0f)
                internal("merged excitability violates canonical parameter bounds");
        }
        for (auto& u : d->recurrent_weight) {
            float w = master.rec_weight[u.index];
            bool sign_ok = master.neuron_type[u.index / S] == 0 ? w >= 0.0f : w <= 0.0f;
            if (!std::isfinite(w) || w < wmin || w > wmax || !sign_ok) internal("merged recurrent parameter violates model constraints");
        }
        for (auto& u : d->input_weight) {
            float w = master.in_weight[u.index];
            if (!std::isfinite(w) || w < 0.0f || w > wmax) internal("merged input parameter violates model constraints");
        }
        for (auto& u : d->output_weight) {
            float w = master.out_weight[u.index];
            if (!std::isfinite(w) || w < wmin || w > wmax) internal("merged output weight violates canonical parameter bounds");
        }
        for (auto& u : d->output_bias)
            if (!std::isfinite(master.bias[u.index])) internal("merged output bias is non-finite");
        for (auto& u : d->context) {
            auto [slot, probes] = master.resolve_context_slot(u.order, u.key, false);
            (void)probes;
            if (slot < 0) continue;
            const size_t s = static_cast<size_t>(slot);
            if (master.ctx_keys[s] == 0 && master.ctx_obs[s] != 0)
                internal("merged context slot has observations without a key");
            for (size_t dd = 0; dd < E; ++dd) {
                float w = master.ctx_emb[s * E + dd];
                if (!std::isfinite(w) || w < wmin || w > wmax)
                    internal("merged context embedding violates canonical parameter bounds");
            }
        }
        for (auto& u : d->context_output_weight) {
            float w = master.ctx_out[u.index];
            if (!std::isfinite(w) || w < wmin || w > wmax) internal("merged context output weight violates canonical parameter bounds");
        }
    }
    return {fixed, ctx};
}

// ---------------------------------------------------------------------------
// training.rs: document pass, replay ranges, replay executors, story batch
// ---------------------------------------------------------------------------
struct DocPass {
    double mean_loss = 0.0;
    std::vector<float> losses;
    uint64_t steps = 0, active_sum = 0, events = 0;
};

// training.rs:1729-1768
DocPass train_document_pass(Runtime& rt, const uint8_t* story, size_t len, int32_t permission) {
    DocPass p;
    if (len == 0) return p;
    double loss_sum = 0.0;
    rt.reset_transient_state();  // begin_document
    std::vector<std::pair<uint32_t, int32_t>> steps;
    steps.push_back({BEGIN_DOCUMENT, story[0]});
    for (size_t i = 0; i + 1 < len; ++i) steps.push_back({story[i], story[i + 1]});
    steps.push_back({story[len - 1], static_cast<int32_t>(END_DOCUMENT)});
    for (auto [sym, tgt] : steps) {
        OracleStepMetrics m = rt.step(sym, tgt, permission);
        float loss = m.has_loss ? m.loss : 0.0f;  // record_training_step
        p.losses.push_back(loss);
        loss_sum += static_cast<double>(loss);
        p.steps += 1;
        p.active_sum += m.active_neurons;
        p.events += m.emitted_events;
    }
    rt.finish_document();
    p.mean_loss = loss_sum / static_cast<double>(std::max<size_t>(p.losses.size(), 1));
    return p;
}

// training.rs:1782-1830
std::vector<std::pair<size_t, size_t>> select_replay_ranges(const float* losses, size_t n, float fraction,
                                                            size_t segment) {
    std::vector<std::pair<size_t, size_t>> selected;
    if (n == 0 || !std::isfinite(fraction) || fraction <= 0.0f || segment == 0) return selected;
    size_t budget = static_cast<size_t>(std::max(1.0, std::ceil(static_cast<double>(n) * static_cast<double>(std::min(fraction, 1.0f)))));
    std::vector<std::pair<size_t, float>> pos;
    for (size_t i = 0; i < n; ++i) pos.push_back({i, losses[i]});
    std::sort(pos.begin(), pos.end(), [](const auto& l, const auto& r) {
        int c = total_cmp(r.second, l.second);
        if (c != 0) return c < 0;
        return l.first < r.first;
    });
    size_t chosen = 0;
    for (auto [p, loss] : pos) {
        if (chosen >= budget) break;
        if (!std::isfinite(loss) || loss <= 0.0f) continue;
        size_t remaining = budget - chosen;
        size_t width = std::min(std::min(segment, remaining), n);
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

struct ReplayCounts {
    uint64_t replay_steps = 0, prefix_steps = 0, active_sum = 0, events = 0, steps = 0;
};

// training.rs:1848-1954
void replay_target_range(Runtime& rt, const uint8_t* story, size_t len, size_t rs, size_t re, int32_t permission,
                         bool cleanup, ReplayCounts& rc) {
    if (len == 0 || rs >= re || rs > len) return;
    size_t end = std::min(re, len + 1);
    rt.reset_transient_state();  // begin_document_deferred_for_replay == begin_document on CPU
    size_t next = rs;
    if (next > 0) {
        rt.step(BEGIN_DOCUMENT, -1, ORACLE_FROZEN);
        for (size_t i = 0; i + 1 < next; ++i) rt.step(story[i], -1, ORACLE_FROZEN);
        rc.prefix_steps += next;
    }
    std::vector<std::pair<uint32_t, int32_t>> batch;
    if (next == 0) {
        batch.push_back({BEGIN_DOCUMENT, story[0]});
        next = 1;
    }
    for (size_t p = next; p < end; ++p)
        batch.push_back({story[p - 1], p < len ? static_cast<int32_t>(story[p]) : static_cast<int32_t>(END_DOCUMENT)});
    for (auto [s, t] : batch) {
        OracleStepMetrics m = rt.step(s, t, permission);
        rc.replay_steps += 1;
        rc.steps += 1;
        rc.active_sum += m.active_neurons;
        rc.events += m.emitted_events;
    }
    if (cleanup) rt.reset_transient_state();
}

// training.rs:162-255
void replay_ranges_streaming(Runtime& rt, const uint8_t* story, size_t len,
                             const std::vector<std::pair<size_t, size_t>>& ranges, int32_t permission,
                             ReplayCounts& rc) {
    if (len == 0 || ranges.empty()) return;
    rt.reset_transient_state();
    const size_t terminal = len + 1;
    size_t cursor = 0;
    auto step_at = [&](size_t position, bool supervised) {
        uint32_t input = position == 0 ? BEGIN_DOCUMENT : story[position - 1];
        int32_t target = -1;
        if (supervised) target = position < len ? story[position] : static_cast<int32_t>(END_DOCUMENT);
        return std::make_pair(input, target);
    };
    for (auto [rs, re] : ranges) {
        size_t start = std::max(std::min(rs, terminal), cursor);
        size_t end = std::max(std::min(re, terminal), start);
        for (size_t p = cursor; p < start; ++p) {
            auto [s, t] = step_at(p, false);
            rt.step(s, t, ORACLE_FROZEN);
            rc.prefix_steps += 1;
        }
        for (size_t p = start; p < end; ++p) {
            auto [s, t] = step_at(p, true);
            OracleStepMetrics m = rt.step(s, t, permission);
            rc.replay_steps += 1;
            rc.steps += 1;
            rc.active_sum += m.active_neurons;
            rc.events += m.emitted_events;
        }
        cursor = end;
    }
    rt.reset_transient_state();
}

// training.rs:394-470 (replay_streaming_enabled: config replay.stateful_batch)
void execute_replay_ranges(Runtime& rt, const uint8_t* story, size_t len,
                           const std::vector<std::pair<size_t, size_t>>& ranges, int32_t permission,
                           ReplayCounts& rc) {
    if (rt.model.cfg.c.replay_stateful_batch && !ranges.empty()) {
        replay_ranges_streaming(rt, story, len, ranges, permission, rc);
        return;
    }
    for (size_t i = 0; i < ranges.size(); ++i)
        replay_target_range(rt, story, len, ranges[i].first, ranges[i].second, permission, i + 1 == ranges.size(), rc);
}

void apply_replay_policy(Runtime& rt, const uint8_t* story, size_t len, const std::vector<float>& losses,
                         int32_t permission, ReplayCounts& rc, uint64_t* segments) {  // training.rs:257-379
    auto ranges = select_replay_ranges(losses.data(), losses.size(), rt.model.cfg.c.replay_fraction,
                                       rt.model.cfg.c.replay_segment_bytes);
    *segments += ranges.size();
    execute_replay_ranges(rt, story, len, ranges, permission, rc);
}

}  // namespace

// ---------------------------------------------------------------------------
// C API
// ---------------------------------------------------------------------------
extern "C" {

int32_t oracle_last_error(char* buffer, size_t capacity) {
    if (!buffer || capacity == 0) return ORACLE_ERR_ARGUMENT;
    std::snprintf(buffer, capacity, "%s", g_last_error.c_str());
    return ORACLE_OK;
}

int32_t oracle_runtime_new(const OracleConfig* config, const OracleModelView* model, OracleRuntime** out) {
    return guard([&] {
        if (!config || !model || !out) internal("null argument");
        Model m;
        m.load(*config, *model);
        auto h = std::make_unique<OracleRuntime>();
        h->rt = std::make_unique<Runtime>(std::move(m));
        *out = h.release();
    });
}

void oracle_runtime_free(OracleRuntime* runtime) { delete runtime; }

int32_t oracle_runtime_read_model(const OracleRuntime* runtime, OracleModelView* out) {
    return guard([&] { runtime->rt->model.store(*out); });
}

int32_t oracle_runtime_write_model(OracleRuntime* runtime, const OracleModelView* model) {
    return guard([&] {
        runtime->rt->model.load(runtime->rt->model.cfg.c, *model);
        runtime->rt->output_cache_dirty = true;
    });
}

int32_t oracle_begin_document(OracleRuntime* r) { return guard([&] { r->rt->reset_transient_state(); }); }
int32_t oracle_finish_document(OracleRuntime* r) { return guard([&] { r->rt->finish_document(); }); }
int32_t oracle_reset_transient_state(OracleRuntime* r) { return guard([&] { r->rt->reset_transient_state(); }); }
int32_t oracle_enable_parameter_tracking(OracleRuntime* r) { return guard([&] { r->rt->enable_parameter_tracking(); }); }
int32_t oracle_restart_parameter_tracking(OracleRuntime* r) { return guard([&] { r->rt->restart_parameter_tracking(); }); }
int32_t oracle_changes_flags(const OracleRuntime* r, uint32_t* bias_dirty, uint32_t* ctx_dirty) {
    *bias_dirty = r->rt->output_bias_dirty;
    *ctx_dirty = r->rt->context_output_dirty;
    return ORACLE_OK;
}

int32_t oracle_step(OracleRuntime* r, uint32_t symbol, int32_t target, int32_t permission, OracleStepMetrics* out) {
    return guard([&] {
        OracleStepMetrics m = r->rt->step(symbol, target, permission);
        if (out) *out = m;
    });
}

uint64_t oracle_current_tick(const OracleRuntime* r) { return r->rt->current_tick; }
float oracle_population_inhibition(const OracleRuntime* r) { return r->rt->population_inhibition; }

int64_t oracle_read_list(const OracleRuntime* r, int32_t which, uint64_t* out, size_t capacity) {
    const Runtime& rt = *r->rt;
    std::vector<size_t> v;
    bool sorted = true;
    switch (which) {
        case ORACLE_L_ACTIVE: v = rt.active; sorted = false; break;
        case ORACLE_L_TOUCHED: v = rt.touched; break;
        case ORACLE_L_ELIGIBLE_REC: v = rt.elig_rec; break;
        case ORACLE_L_ELIGIBLE_IN: v = rt.elig_in; break;
        case ORACLE_L_LEARNING_DESTINATIONS: v = rt.learning_destinations; break;
        case ORACLE_L_CHANGED_THRESHOLD: v = rt.ch_threshold; break;
        case ORACLE_L_CHANGED_REC: v = rt.ch_rec; break;
        case ORACLE_L_CHANGED_IN: v = rt.ch_in; break;
        case ORACLE_L_CHANGED_OUTPUT: v = rt.ch_out; break;
        case ORACLE_L_CHANGED_CONTEXT: v = rt.ch_ctx; break;
        case ORACLE_L_ACTIVE_CONTEXT_SLOTS: v = rt.active_context_slots; sorted = false; break;
        default: return -1;
    }
    if (sorted) std::sort(v.begin(), v.end());
    if (out)
        for (size_t i = 0; i < std::min(capacity, v.size()); ++i) out[i] = v[i];
    return static_cast<int64_t>(v.size());
}

int32_t oracle_read_f32(const OracleRuntime* r, int32_t which, float* out, size_t count) {
    const Runtime& rt = *r->rt;
    const std::vector<float>* v = nullptr;
    switch (which) {
        case ORACLE_F_MEMBRANE: v = &rt.membrane; break;
        case ORACLE_F_ACTIVATION: v = &rt.activation; break;
        case ORACLE_F_FATIGUE: v = &rt.fatigue; break;
        case ORACLE_F_BRANCHES: v = &rt.branches; break;
        case ORACLE_F_ADAPT0: v = &rt.adaptation[0]; break;
        case ORACLE_F_ADAPT1: v = &rt.adaptation[1]; break;
        case ORACLE_F_ADAPT2: v = &rt.adaptation[2]; break;
        case ORACLE_F_SURROGATE: v = &rt.selection_surrogate; break;
        case ORACLE_F_REC_BS: v = &rt.rbs; break;
        case ORACLE_F_REC_MS: v = &rt.rms; break;
        case ORACLE_F_REC_FS: v = &rt.rfs; break;
        case ORACLE_F_REC_AS0: v = &rt.ras[0]; break;
        case ORACLE_F_REC_AS1: v = &rt.ras[1]; break;
        case ORACLE_F_REC_AS2: v = &rt.ras[2]; break;
        case ORACLE_F_REC_E: v = &rt.elig; break;
        case ORACLE_F_IN_BS: v = &rt.ibs; break;
        case ORACLE_F_IN_MS: v = &rt.ims; break;
        case ORACLE_F_IN_FS: v = &rt.ifs; break;
        case ORACLE_F_IN_AS0: v = &rt.ias[0]; break;
        case ORACLE_F_IN_AS1: v = &rt.ias[1]; break;
        case ORACLE_F_IN_AS2: v = &rt.ias[2]; break;
        case ORACLE_F_IN_E: v = &rt.ielig; break;
        case ORACLE_F_LOGITS: v = &rt.logits; break;
        case ORACLE_F_PROBABILITIES: v = &rt.probabilities; break;
        case ORACLE_F_ERRORS: v = &rt.errors; break;
        case ORACLE_F_LEARNING_SIGNAL: v = &rt.learning_signal; break;
        case ORACLE_F_BLOCK_CUTOFF: v = &rt.block_cutoff; break;
        case ORACLE_F_CONTEXT_LATENT: v = &rt.context_latent; break;
        default: return ORACLE_ERR_ARGUMENT;
    }
    if (count != v->size()) return ORACLE_ERR_ARGUMENT;
    std::copy(v->begin(), v->end(), out);
    return ORACLE_OK;
}

int32_t oracle_read_u64(const OracleRuntime* r, int32_t which, uint64_t* out, size_t count) {
    const Runtime& rt = *r->rt;
    const std::vector<uint64_t>* v = nullptr;
    switch (which) {
        case ORACLE_U_REFRACTORY: v = &rt.refractory_until; break;
        case ORACLE_U_NEURON_LAST_TICK: v = &rt.neuron_last_tick; break;
        case ORACLE_U_REC_LAST_TICK: v = &rt.elig_last; break;
        case ORACLE_U_IN_LAST_TICK: v = &rt.ielig_last; break;
        default: return ORACLE_ERR_ARGUMENT;
    }
    if (count != v->size()) return ORACLE_ERR_ARGUMENT;
    std::copy(v->begin(), v->end(), out);
    return ORACLE_OK;
}

int32_t oracle_train_document_pass(OracleRuntime* r, const uint8_t* story, uint64_t length, int32_t permission,
                                   float* losses_out) {
    return guard([&] {
        DocPass p = train_document_pass(*r->rt, story, length, permission);
        if (losses_out) std::copy(p.losses.begin(), p.losses.end(), losses_out);
    });
}

int32_t oracle_execute_replay_ranges(OracleRuntime* r, const uint8_t* story, uint64_t length, const uint64_t* ranges,
                                     uint32_t count, int32_t permission, uint64_t* replay_steps,
                                     uint64_t* prefix_steps) {
    return guard([&] {
        std::vector<std::pair<size_t, size_t>> rr;
        for (uint32_t i = 0; i < count; ++i) rr.push_back({ranges[2 * i], ranges[2 * i + 1]});
        ReplayCounts rc;
        execute_replay_ranges(*r->rt, story, length, rr, permission, rc);
        if (replay_steps) *replay_steps = rc.replay_steps;
        if (prefix_steps) *prefix_steps = rc.prefix_steps;
    });
}

// training.rs:1539-1727 (CPU backend path)
int32_t oracle_train_story_batch(OracleRuntime* r, const uint8_t* bytes, const uint64_t* offsets, uint32_t count,
                                 int32_t permission, uint32_t replay_enabled, float* losses_out,
                                 OracleBatchReport* report) {
    return guard([&] {
        if (count == 0) internal("training batch cannot be empty");
        Runtime& canonical = *r->rt;
        OracleBatchReport rep{};
        auto story = [&](uint32_t i) { return bytes + offsets[i]; };
        auto slen = [&](uint32_t i) { return static_cast<size_t>(offsets[i + 1] - offsets[i]); };
        size_t loss_cursor = 0;
        if (count == 1) {
            DocPass p = train_document_pass(canonical, story(0), slen(0), permission);
            if (losses_out) std::copy(p.losses.begin(), p.losses.end(), losses_out);
            ReplayCounts rc;
            uint64_t segments = 0;
            if (replay_enabled) apply_replay_policy(canonical, story(0), slen(0), p.losses, permission, rc, &segments);
            rep.mean_loss = p.mean_loss;
            rep.targets = p.losses.size();
            rep.stories = 1;
            rep.replay_segments = segments;
            rep.replay_steps = rc.replay_steps;
            rep.replay_prefix_steps = rc.prefix_steps;
            rep.merge_workers = 1;
            rep.activity_steps = p.steps + rc.steps;
            rep.active_neurons_sum = p.active_sum + rc.active_sum;
            rep.emitted_events = p.events + rc.events;
            if (report) *report = rep;
            return;
        }
        const Model base = canonical.model;  // synchronize_model + clone
        struct WorkerResult {
            OracleDelta delta;
            DocPass pass;
            std::string error;
            int32_t code = 0;
        };
        std::vector<WorkerResult> results(count);
        std::vector<std::thread> threads;
        threads.reserve(count);
        for (uint32_t i = 0; i < count; ++i) {
            threads.emplace_back([&, i] {
                try {
                    Runtime worker(base);  // fork: Runtime::new(base.clone()), tick 0
                    worker.enable_parameter_tracking();
                    results[i].pass = train_document_pass(worker, story(i), slen(i), permission);
                    results[i].delta = delta_between_tracked(base, worker.model, worker.parameter_changes());
                } catch (const LeoError& e) {
                    results[i].error = e.what();
                    results[i].code = e.code;
                } catch (const std::exception& e) {
                    results[i].error = e.what();
                    results[i].code = ORACLE_ERR_INTERNAL;
                }
            });
        }
        for (auto& t : threads) t.join();
        for (auto& w : results)
            if (w.code != 0) throw LeoError(w.code, w.error);
        std::vector<const OracleDelta*> deltas;
        for (auto& w : results) deltas.push_back(&w.delta);
        auto [fixed, ctx] = apply_deltas_with_divisor(canonical.model, deltas, deltas.size());
        canonical.output_cache_dirty = true;  // model_mut()
        canonical.reset_transient_state();
        double weighted = 0.0;
        uint64_t targets = 0;
        for (auto& w : results) {
            weighted += w.pass.mean_loss * static_cast<double>(w.pass.losses.size());
            targets += w.pass.losses.size();
            rep.activity_steps += w.pass.steps;
            rep.active_neurons_sum += w.pass.active_sum;
            rep.emitted_events += w.pass.events;
            if (losses_out) {
                std::copy(w.pass.losses.begin(), w.pass.losses.end(), losses_out + loss_cursor);
                loss_cursor += w.pass.losses.size();
            }
        }
        ReplayCounts rc;
        uint64_t segments = 0;
        if (replay_enabled)
            for (uint32_t i = 0; i < count; ++i)
                apply_replay_policy(canonical, story(i), slen(i), results[i].pass.losses, permission, rc, &segments);
        rep.mean_loss = weighted / static_cast<double>(std::max<uint64_t>(targets, 1));
        rep.targets = targets;
        rep.stories = count;
        rep.replay_segments = segments;
        rep.replay_steps = rc.replay_steps;
        rep.replay_prefix_steps = rc.prefix_steps;
        rep.merge_workers = count;
        rep.merge_fixed_parameter_updates = fixed;
        rep.merge_context_keys = ctx;
        rep.activity_steps += rc.steps;
        rep.active_neurons_sum += rc.active_sum;
        rep.emitted_events += rc.events;
        if (report) *report = rep;
    });
}

int64_t oracle_select_replay_ranges(const float* losses, uint64_t count, float fraction, uint64_t segment,
                                    uint64_t* out, size_t capacity) {
    auto r = select_replay_ranges(losses, count, fraction, segment);
    for (size_t i = 0; i < std::min(capacity, r.size()); ++i) {
        out[2 * i] = r[i].first;
        out[2 * i + 1] = r[i].second;
    }
    return static_cast<int64_t>(r.size());
}

int32_t oracle_delta_between(const OracleConfig* config, const OracleModelView* base, const OracleModelView* trained,
                             OracleDelta** out) {
    return guard([&] {
        Model b, t;
        b.load(*config, *base);
        t.load(*config, *trained);
        *out = new OracleDelta(delta_between(b, t));
    });
}

int32_t oracle_delta_between_tracked(const OracleModelView* base, const OracleRuntime* trained, OracleDelta** out) {
    return guard([&] {
        Model b;
        b.load(trained->rt->model.cfg.c, *base);
        *out = new OracleDelta(delta_between_tracked(b, trained->rt->model, trained->rt->parameter_changes()));
    });
}

void oracle_delta_free(OracleDelta* d) { delete d; }

int64_t oracle_delta_count(const OracleDelta* d, int32_t which) {
    switch (which) {
        case 0: return static_cast<int64_t>(d->threshold.size());
        case 1: return static_cast<int64_t>(d->recurrent_weight.size());
        case 2: return static_cast<int64_t>(d->input_weight.size());
        case 3: return static_cast<int64_t>(d->output_weight.size());
        case 4: return static_cast<int64_t>(d->output_bias.size());
        case 5: return static_cast<int64_t>(d->context_output_weight.size());
        case 6: return static_cast<int64_t>(d->context.size());
        case 7: return static_cast<int64_t>(d->revision_increment);
        default: return -1;
    }
}

int32_t oracle_delta_equal(const OracleDelta* l, const OracleDelta* r) { return (*l == *r) ? 1 : 0; }

int32_t oracle_apply_deltas(OracleRuntime* master, OracleDelta* const* deltas, uint32_t count, int32_t mode,
                            uint64_t* fixed_updates, uint64_t* context_keys) {
    return guard([&] {
        std::vector<const OracleDelta*> d(deltas, deltas + count);
        auto [fixed, ctx] = apply_deltas_with_divisor(master->rt->model, d, mode == 0 ? d.size() : 1);
        master->rt->output_cache_dirty = true;
        if (fixed_updates) *fixed_updates = fixed;
        if (context_keys) *context_keys = ctx;
    });
}

float oracle_analog_rank_surrogate(float margin, float cutoff, int32_t selected, float width, float gain) {
    return analog_rank_surrogate(margin, cutoff, selected != 0, width, gain);
}
float oracle_branch_jacobian(uint8_t branch, float excitability, float temporal, float gate) {
    return branch_jacobian(branch, excitability, temporal, gate);
}
float oracle_bounded_delta(float value, float maximum) { return bounded_delta(value, maximum); }
float oracle_inhibitory_homeostasis_delta(float s, float t, float d, float lr, float st, float mu) {
    return inhibitory_homeostasis_delta(s, t, d, lr, st, mu);
}
int32_t oracle_context_survives_dropout(uint64_t seed, uint64_t tick, uint32_t symbol, float rate) {
    return context_survives_dropout(seed, tick, symbol, rate) ? 1 : 0;
}
uint64_t oracle_context_key(const uint32_t* history, size_t len, size_t order) {
    if (order == 0 || order > len) return 0;
    return context_key(history, len, order);
}
float oracle_decay_for_elapsed(float base, uint64_t elapsed) { return decay_for_elapsed(base, elapsed); }

int32_t oracle_resolve_context_slot(OracleRuntime* r, uint64_t order, uint64_t key, int32_t allocate, int64_t* slot,
                                    uint64_t* probes) {
    return guard([&] {
        auto [s, p] = r->rt->model.resolve_context_slot(order, key, allocate != 0);
        *slot = s;
        *probes = p;
    });
}

int32_t oracle_test_update_context_projection(OracleRuntime* r, const uint64_t* slots, const float* scales,
                                              uint32_t count, const float* errors, float strength) {
    return guard([&] {
        Runtime& rt = *r->rt;
        rt.active_context_slots.assign(slots, slots + count);
        rt.active_context_scales.assign(scales, scales + count);
        std::copy(errors, errors + OUTPUT_CLASSES, rt.errors.begin());
        rt.update_context_projection(strength);
    });
}

int32_t oracle_plasticity_step(uint32_t window, uint64_t phase, int32_t end_document, float* scale,
                               uint64_t* next_phase) {
    Config c{};
    c.c.plasticity_window = window;
    auto [s, n] = c.plasticity_step(phase, end_document != 0);
    *scale = s;
    *next_phase = n;
    return ORACLE_OK;
}

}  // extern "C"
