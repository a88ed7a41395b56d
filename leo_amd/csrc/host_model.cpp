// Host-side model code of the MI355X backend: Leo's seeded initialisation,
// model validation, and the seeded synthetic workloads the benchmark trains.
// None of this runs on the GPU; it produces the canonical host image that
// leo_hip_create uploads.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "leo_hip.h"
#include "leo_host.h"

namespace leo {

namespace {

// crates/leo-core/src/rng.rs:3-42 (SplitMix64).
struct SplitMix64 {
    uint64_t state;
    explicit SplitMix64(uint64_t seed) : state(seed) {}
    uint64_t next_u64() {
        state += 0x9E3779B97F4A7C15ULL;
        uint64_t v = state;
        v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ULL;
        v = (v ^ (v >> 27)) * 0x94D049BB133111EBULL;
        return v ^ (v >> 31);
    }
    float next_f32() {  // (u64 >> 40) / (2^24 - 1)
        uint32_t v = static_cast<uint32_t>(next_u64() >> 40);
        return static_cast<float>(v) / static_cast<float>((1u << 24) - 1u);
    }
    size_t range_usize(size_t upper) {
        if (upper <= 1) return 0;
        return static_cast<size_t>(next_u64() % static_cast<uint64_t>(upper));
    }
    float range_f32(float low, float high) { return low + (high - low) * next_f32(); }
    // The i-th output depends only on seed + i * increment, so a generator
    // can be positioned anywhere in the stream.
    static constexpr uint64_t kIncrement = 0x9E3779B97F4A7C15ULL;
    void skip(uint64_t outputs) { state += outputs * kIncrement; }
    template <class T>
    void shuffle(std::vector<T>& v) {
        for (size_t i = v.size(); i-- > 1;) {
            size_t other = range_usize(i + 1);
            std::swap(v[i], v[other]);
        }
    }
    double next_unit_open() {  // (0,1), for the synthetic generators only
        return (static_cast<double>(next_u64() >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    }
    double normal() {  // Box-Muller, synthetic generators only
        double u1 = next_unit_open(), u2 = next_unit_open();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

// Fills out[i] = range_f32(low, high) for i < count with the generator's next
// `count` outputs, in parallel chunks (each positioned with skip), and leaves
// the generator where the sequential loop would: the values are the ones the
// sequential loop draws.
void fill_range_f32(SplitMix64& rng, float* out, size_t count, float low, float high) {
    const size_t kChunk = size_t(1) << 22;
    const unsigned threads = static_cast<unsigned>(
        std::min<size_t>({std::max(1u, std::thread::hardware_concurrency()), 16u, (count + kChunk - 1) / kChunk}));
    auto work = [&](size_t begin, size_t end) {
        SplitMix64 local = rng;
        local.skip(begin);
        for (size_t i = begin; i < end; ++i) out[i] = local.range_f32(low, high);
    };
    if (threads <= 1) {
        work(0, count);
    } else {
        std::vector<std::thread> pool;
        const size_t per = (count + threads - 1) / threads;
        for (unsigned t = 0; t < threads; ++t) {
            const size_t begin = std::min(count, t * per), end = std::min(count, begin + per);
            pool.emplace_back(work, begin, end);
        }
        for (auto& th : pool) th.join();
    }
    rng.skip(count);
}

constexpr uint8_t BR_EXC = 0, BR_INH = 1, BR_TEMP = 2, BR_GATE = 3;

// model.rs:498-505
uint8_t sample_delay(SplitMix64& rng) {
    size_t r = rng.range_usize(100);
    if (r <= 49) return 1;
    if (r <= 74) return 2;
    if (r <= 89) return 4;
    return 8;
}

struct Sizes {
    size_t n, s, f, slots, e;
};

Sizes sizes_of(const LeoHostConfig& c) {
    Sizes z;
    z.n = c.device.neuron_count;
    z.s = c.device.synapses_per_neuron;
    z.f = c.device.input_fanout;
    z.slots = static_cast<size_t>(c.device.context_max_order) * c.device.context_slots_per_order;
    z.e = c.device.context_embedding_dim;
    return z;
}

void require_arrays(const LeoModelView& m) {
    if (!m.threshold || !m.excitability || !m.neuron_type || !m.rec_target || !m.rec_branch || !m.rec_delay ||
        !m.rec_weight || !m.in_target || !m.in_branch || !m.in_weight || !m.out_weight || !m.bias || !m.ctx_keys ||
        !m.ctx_emb || !m.ctx_obs || !m.ctx_out)
        throw Error(LEO_ERR_INVALID_ARGUMENT, "model view has a null array");
}

// model.rs:97-111: neuron types by shuffled ids, then thresholds.
void init_neurons(const LeoHostConfig& c, SplitMix64& rng, LeoModelView& m) {
    const size_t n = c.device.neuron_count;
    std::fill(m.neuron_type, m.neuron_type + n, 0);
    size_t inhibitory = static_cast<size_t>(std::max(0.0f, std::round((1.0f - c.excitatory_fraction) * static_cast<float>(n))));
    std::vector<size_t> ids(n);
    for (size_t i = 0; i < n; ++i) ids[i] = i;
    rng.shuffle(ids);
    for (size_t i = 0; i < std::min(inhibitory, n); ++i) m.neuron_type[ids[i]] = 1;
    for (size_t i = 0; i < n; ++i) m.excitability[i] = 1.0f;
    for (size_t i = 0; i < n; ++i) m.threshold[i] = rng.range_f32(0.45f, 0.55f);
}

// model.rs:461-496
void init_input(const LeoHostConfig& c, SplitMix64& rng, LeoModelView& m) {
    const size_t f = c.device.input_fanout, n = c.device.neuron_count;
    std::vector<size_t> used;
    for (size_t symbol = 0; symbol < 258; ++symbol) {
        used.clear();
        for (size_t index = 0; index < f; ++index) {
            size_t target;
            while (true) {
                target = rng.range_usize(n);
                if (std::find(used.begin(), used.end(), target) == used.end()) {
                    used.push_back(target);
                    break;
                }
            }
            size_t off = symbol * f + index;
            m.in_target[off] = static_cast<uint32_t>(target);
            m.in_branch[off] = (index % 8 == 6) ? BR_TEMP : (index % 8 == 7 ? BR_GATE : BR_EXC);
            m.in_weight[off] = rng.range_f32(0.05f, 0.20f);
        }
    }
}

// model.rs:126-157: output, context projection, empty context memory.
void init_projections(const LeoHostConfig& c, SplitMix64& rng, LeoModelView& m) {
    const Sizes z = sizes_of(c);
    fill_range_f32(rng, m.out_weight, 257 * z.n, -0.005f, 0.005f);
    fill_range_f32(rng, m.ctx_out, 257 * z.e, -0.005f, 0.005f);
    std::fill(m.bias, m.bias + 257, 0.0f);
    std::fill(m.ctx_keys, m.ctx_keys + z.slots, 0);
    std::fill(m.ctx_emb, m.ctx_emb + z.slots * z.e, 0.0f);
    std::fill(m.ctx_obs, m.ctx_obs + z.slots, 0);
    m.generation = 0;
    m.parameter_revision = 0;
    std::memset(&m.statistics, 0, sizeof(m.statistics));
}

}  // namespace

// model.rs:79-158 + initialize_recurrent (model.rs:399-459)
void model_initialize(const LeoHostConfig& c, LeoModelView& m) {
    validate_config(c);
    require_arrays(m);
    SplitMix64 rng(c.seed);
    init_neurons(c, rng, m);
    const size_t n = c.device.neuron_count, s = c.device.synapses_per_neuron, bs = c.device.neurons_per_block;
    const size_t blocks = c.device.block_count;
    const size_t local_count = (s * 3) / 4;
    std::vector<std::pair<size_t, uint8_t>> used;
    for (size_t src = 0; src < n; ++src) {
        const uint8_t type = m.neuron_type[src];
        const size_t src_block = src / bs;
        used.clear();
        for (size_t local = 0; local < s; ++local) {
            const size_t slot = src * s + local;
            const bool prefer_local = local < local_count;
            bool ok = false;
            size_t target = 0;
            uint8_t branch = 0;
            for (int attempt = 0; attempt < 128; ++attempt) {
                if (prefer_local) {
                    long delta = static_cast<long>(rng.range_usize(3)) - 1;
                    long b = std::min<long>(std::max<long>(static_cast<long>(src_block) + delta, 0), static_cast<long>(blocks) - 1);
                    target = static_cast<size_t>(b) * bs + rng.range_usize(bs);
                } else {
                    target = rng.range_usize(n);
                }
                if (type == 0) {
                    size_t r = rng.range_usize(3);
                    branch = r == 0 ? BR_EXC : (r == 1 ? BR_TEMP : BR_GATE);
                } else {
                    branch = BR_INH;
                }
                if (target == src && branch != BR_TEMP) continue;
                auto key = std::make_pair(target, branch);
                if (std::find(used.begin(), used.end(), key) == used.end()) {
                    used.push_back(key);
                    ok = true;
                    break;
                }
            }
            if (!ok) throw Error(LEO_ERR_INTERNAL, "could not initialize unique synapse for neuron " + std::to_string(src));
            m.rec_target[slot] = static_cast<uint32_t>(target);
            m.rec_branch[slot] = branch;
            m.rec_delay[slot] = sample_delay(rng);
            m.rec_weight[slot] = type == 0 ? rng.range_f32(0.01f, 0.08f) : rng.range_f32(-0.08f, -0.01f);
        }
    }
    init_input(c, rng, m);
    init_projections(c, rng, m);
}

// Synthetic benchmark topologies. Rows stay Leo-valid (unique (target,branch)
// per source, self-edges only on TEMPORAL, inhibitory sources on INHIBITORY).
void model_initialize_synthetic(const LeoHostConfig& c, uint32_t topology, float exponent, uint32_t cap,
                                float sigma, LeoModelView& m) {
    validate_config(c);
    require_arrays(m);
    if (topology > LEO_TOPOLOGY_HEAVY_TAIL) throw Error(LEO_ERR_INVALID_ARGUMENT, "unknown synthetic topology");
    if (!(sigma > 0.0f)) throw Error(LEO_ERR_INVALID_ARGUMENT, "weight_sigma must be positive");
    SplitMix64 rng(c.seed);
    init_neurons(c, rng, m);
    const size_t n = c.device.neuron_count, s = c.device.synapses_per_neuron;
    // Target sampler: uniform, or Zipf(exponent) over a seeded permutation of the
    // neurons (inverse CDF by binary search), so in-degree is heavy-tailed while
    // every row keeps its fixed capacity S.
    // A guide table narrows each search: with K a power of two, u*K is exact,
    // so j = floor(u*K) gives j/K <= u < (j+1)/K and the lower bound of u lies
    // in [guide[j], guide[j+1]], guide[j] being the lower bound of j/K.
    std::vector<double> cdf;
    std::vector<uint32_t> perm, guide;
    size_t guide_size = 1;
    if (topology != LEO_TOPOLOGY_UNIFORM) {
        if (!(exponent > 0.0f)) throw Error(LEO_ERR_INVALID_ARGUMENT, "power-law exponent must be positive");
        cdf.resize(n);
        double acc = 0.0;
        for (size_t i = 0; i < n; ++i) {
            acc += std::pow(static_cast<double>(i + 1), -static_cast<double>(exponent));
            cdf[i] = acc;
        }
        for (double& x : cdf) x /= acc;
        perm.resize(n);
        for (size_t i = 0; i < n; ++i) perm[i] = static_cast<uint32_t>(i);
        rng.shuffle(perm);
        while (guide_size < n && guide_size < (size_t(1) << 24)) guide_size <<= 1;
        guide.resize(guide_size + 1);
        size_t at = 0;
        for (size_t j = 0; j <= guide_size; ++j) {
            const double bound = static_cast<double>(j) / static_cast<double>(guide_size);
            while (at < n && cdf[at] < bound) ++at;
            guide[j] = static_cast<uint32_t>(at);
        }
    }
    std::vector<uint32_t> in_degree(cap ? n : 0, 0);
    auto draw_target = [&]() -> size_t {
        if (topology == LEO_TOPOLOGY_UNIFORM) return rng.range_usize(n);
        double u = rng.next_unit_open();
        const size_t j = static_cast<size_t>(u * static_cast<double>(guide_size));
        size_t rank = static_cast<size_t>(
            std::lower_bound(cdf.begin() + guide[j], cdf.begin() + guide[j + 1], u) - cdf.begin());
        return perm[std::min(rank, n - 1)];
    };
    std::vector<std::pair<size_t, uint8_t>> used;
    for (size_t src = 0; src < n; ++src) {
        const uint8_t type = m.neuron_type[src];
        used.clear();
        for (size_t local = 0; local < s; ++local) {
            const size_t slot = src * s + local;
            bool ok = false;
            size_t target = 0;
            uint8_t branch = BR_INH;
            for (int attempt = 0; attempt < 4096; ++attempt) {
                target = attempt < 256 ? draw_target() : rng.range_usize(n);
                if (cap && in_degree[target] >= cap) continue;
                if (type == 0) {
                    size_t r = rng.range_usize(3);
                    branch = r == 0 ? BR_EXC : (r == 1 ? BR_TEMP : BR_GATE);
                }
                if (target == src && branch != BR_TEMP) continue;
                auto key = std::make_pair(target, branch);
                if (std::find(used.begin(), used.end(), key) == used.end()) {
                    used.push_back(key);
                    ok = true;
                    break;
                }
            }
            if (!ok) throw Error(LEO_ERR_INTERNAL, "synthetic topology could not place a unique synapse");
            if (cap) in_degree[target] += 1;
            m.rec_target[slot] = static_cast<uint32_t>(target);
            m.rec_branch[slot] = branch;
            m.rec_delay[slot] = sample_delay(rng);
            float w = std::fabs(static_cast<float>(rng.normal() * sigma));
            w = std::min(w, c.device.weight_max);
            m.rec_weight[slot] = type == 0 ? w : std::max(-w, c.device.weight_min);
        }
    }
    init_input(c, rng, m);
    init_projections(c, rng, m);
}

void splitmix64_stream(uint64_t seed, uint64_t* out, uint64_t count) {
    SplitMix64 rng(seed);
    for (uint64_t i = 0; i < count; ++i) out[i] = rng.next_u64();
}

// config.rs:250-519 (the rules the executor and the device layout depend on).
void validate_config(const LeoHostConfig& c) {
    const LeoConfig& d = c.device;
    auto fail = [](const char* msg) { throw Error(LEO_ERR_INVALID_ARGUMENT, msg); };
    if (d.neuron_count == 0 || d.block_count == 0 || d.neurons_per_block == 0) fail("model dimensions must be positive");
    if (static_cast<uint64_t>(d.block_count) * d.neurons_per_block != d.neuron_count)
        fail("block_count * neurons_per_block must equal neuron_count without overflow");
    if (d.branches_per_neuron != 4) fail("Leo requires exactly four dendritic branches per neuron");
    if (!std::isfinite(c.excitatory_fraction) || !(c.excitatory_fraction >= 0.0f && c.excitatory_fraction < 1.0f))
        fail("excitatory_fraction must be finite and strictly between 0 and 1");
    if (d.synapses_per_neuron == 0 || d.input_fanout == 0) fail("synapses_per_neuron and input_fanout must be positive");
    if (d.synapses_per_neuron > d.neuron_count) fail("synapses_per_neuron cannot exceed neuron_count");
    if (d.input_fanout > d.neuron_count) fail("input_fanout cannot exceed neuron_count");
    if (d.max_active_per_block == 0 || d.max_active_per_block > d.neurons_per_block)
        fail("max_active_per_block must be in 1..=neurons_per_block");
    if (d.max_active_global == 0 || d.max_active_global > d.neuron_count) fail("max_active_global must be in 1..=neuron_count");
    if (d.refractory_ticks == 0) fail("refractory_ticks must be positive in the integrated architecture");
    const float decays[] = {d.branch_decay, d.membrane_decay, d.fatigue_decay, d.adaptation_fast_decay,
                            d.adaptation_medium_decay, d.adaptation_slow_decay, d.eligibility_decay};
    for (float v : decays)
        if (!std::isfinite(v) || !(v >= 0.0f && v < 1.0f)) fail("decays must be finite and strictly between 0 and 1");
    const float positives[] = {d.fatigue_gain, d.adaptation_fast_gain, d.adaptation_medium_gain, d.adaptation_slow_gain,
                               d.threshold_homeostasis_rate, d.population_inhibition_rate, d.output_learning_rate,
                               d.recurrent_learning_rate, d.inhibitory_learning_rate, d.eligibility_epsilon,
                               d.surrogate_width, d.surrogate_gain, d.max_update};
    for (float v : positives)
        if (!std::isfinite(v) || v <= 0.0f) fail("gains, rates and limits must be finite and positive");
    if (!std::isfinite(d.target_activity) || !(d.target_activity > 0.0f && d.target_activity <= 1.0f))
        fail("target_activity must be finite and in (0, 1]");
    if (!std::isfinite(d.population_inhibition_max) || d.population_inhibition_max <= 0.0f)
        fail("population_inhibition_max must be finite and positive");
    if (!std::isfinite(d.membrane_reset_fraction) || !(d.membrane_reset_fraction > 0.0f && d.membrane_reset_fraction <= 1.0f))
        fail("membrane_reset_fraction must be finite and in (0, 1]");
    if (static_cast<size_t>(std::ceil(d.target_activity * static_cast<float>(d.neuron_count))) > d.max_active_global)
        fail("target_activity requires more neurons than max_active_global permits");
    if (d.weight_min >= 0.0f || d.weight_max <= 0.0f || d.weight_min >= d.weight_max)
        fail("weight_min must be negative and weight_max must be positive");
    if (c.plasticity_window == 0 || c.plasticity_window > 64) fail("learning.plasticity_window must be in 1..=64");
    if (!std::isfinite(c.end_document_weight) || !(c.end_document_weight >= 1.0f && c.end_document_weight <= 16.0f))
        fail("end_document_weight must be finite and in [1, 16]");
    for (float v : {c.provisional_strength, c.training_strength, c.verified_strength})
        if (!std::isfinite(v) || !(v > 0.0f && v <= 1.0f)) fail("strengths must be finite and in (0, 1]");
    if (d.context_max_order == 0 || d.context_embedding_dim == 0 || d.context_slots_per_order == 0 ||
        d.context_probe_limit == 0 || d.context_confidence_observations == 0)
        fail("all context-memory dimensions must be positive");
    if (d.context_embedding_dim > 256) fail("context.embedding_dim cannot exceed 256");
    if (d.context_max_order > 16) fail("context.max_order cannot exceed 16");
    if (d.context_probe_limit > d.context_slots_per_order) fail("context.probe_limit cannot exceed slots_per_order");
    if (!std::isfinite(c.context_dropout_rate) || !(c.context_dropout_rate >= 0.0f && c.context_dropout_rate < 1.0f))
        fail("context.dropout_rate must be finite and in [0, 1)");
    if (!std::isfinite(d.context_learning_rate) || d.context_learning_rate <= 0.0f)
        fail("context.learning_rate must be finite and positive");
    if (!std::isfinite(c.replay_fraction) || c.replay_fraction < 0.0f || c.replay_fraction > 1.0f)
        fail("replay.fraction must be finite and in the interval [0, 1]");
    if (c.replay_segment_bytes == 0) fail("all replay limits must be positive");
}

// model.rs:223-396
void model_validate(const LeoHostConfig& c, const LeoModelView& m) {
    validate_config(c);
    require_arrays(m);
    const Sizes z = sizes_of(c);
    const float wmin = c.device.weight_min, wmax = c.device.weight_max;
    auto fail = [](const std::string& msg) { throw Error(LEO_ERR_INVALID_ARGUMENT, msg); };
    auto finite = [&](const float* v, size_t count) {
        for (size_t i = 0; i < count; ++i)
            if (!std::isfinite(v[i])) fail("model contains NaN or infinite values");
    };
    finite(m.threshold, z.n);
    finite(m.excitability, z.n);
    finite(m.rec_weight, z.n * z.s);
    finite(m.in_weight, 258 * z.f);
    finite(m.out_weight, 257 * z.n);
    finite(m.bias, 257);
    finite(m.ctx_emb, z.slots * z.e);
    finite(m.ctx_out, 257 * z.e);
    if (!std::isfinite(m.statistics.training_loss_sum)) fail("model contains NaN or infinite values");
    for (size_t i = 0; i < z.n; ++i)
        if (m.threshold[i] < 0.05f || m.threshold[i] > 2.0f) fail("neuron thresholds violate canonical parameter bounds");
    for (size_t i = 0; i < z.n; ++i)
        if (m.excitability[i] < 0.1f || m.excitability[i] > 4.0f) fail("neuron excitability violates canonical parameter bounds");
    auto bounded = [&](const float* v, size_t count) {
        for (size_t i = 0; i < count; ++i)
            if (v[i] < wmin || v[i] > wmax) fail("learned projection weights violate canonical parameter bounds");
    };
    bounded(m.out_weight, 257 * z.n);
    bounded(m.ctx_emb, z.slots * z.e);
    bounded(m.ctx_out, 257 * z.e);
    for (size_t i = 0; i < z.slots; ++i)
        if (m.ctx_keys[i] == 0 && m.ctx_obs[i] != 0) fail("empty context slots cannot contain observations");
    for (size_t i = 0; i < z.n; ++i)
        if (m.neuron_type[i] > 1) fail("neuron types must be excitatory or inhibitory");
    for (size_t src = 0; src < z.n; ++src) {
        for (size_t slot = src * z.s; slot < (src + 1) * z.s; ++slot) {
            uint32_t t = m.rec_target[slot];
            uint8_t br = m.rec_branch[slot], d = m.rec_delay[slot];
            float w = m.rec_weight[slot];
            if (t >= z.n) fail("recurrent slot " + std::to_string(slot) + " targets a neuron outside the model");
            if (br > BR_GATE || !(d == 1 || d == 2 || d == 4 || d == 8))
                fail("recurrent slot " + std::to_string(slot) + " has invalid branch or delay");
            if (w < wmin || w > wmax) fail("recurrent slot " + std::to_string(slot) + " has invalid weight");
            if (m.neuron_type[src] == 0) {
                if (w < 0.0f || br == BR_INH) fail("excitatory source " + std::to_string(src) + " has incompatible slot");
            } else if (w > 0.0f || br != BR_INH) {
                fail("inhibitory source " + std::to_string(src) + " has incompatible slot");
            }
        }
    }
    for (size_t i = 0; i < 258 * z.f; ++i)
        if (m.in_target[i] >= z.n || m.in_branch[i] == BR_INH || m.in_branch[i] > BR_GATE || m.in_weight[i] < 0.0f ||
            m.in_weight[i] > wmax)
            fail("input projection slot " + std::to_string(i) + " has invalid state");
}

// Seeded Zipf-ASCII stories: a 2,000-word lowercase vocabulary (2-9 letters),
// Zipf(1.1) word ranks, spaces, ", " / ". " punctuation, '\n' terminator.
void synthetic_stories(uint64_t seed, uint32_t count, double mean, double stddev, uint32_t min_len, uint32_t max_len,
                       uint8_t* bytes, uint64_t capacity, uint64_t* offsets) {
    if (min_len < 2 || max_len < min_len) throw Error(LEO_ERR_INVALID_ARGUMENT, "story lengths must satisfy 2 <= min <= max");
    SplitMix64 rng(seed);
    const size_t vocab = 2000;
    std::vector<std::string> words(vocab);
    for (auto& w : words) {
        size_t len = 2 + rng.range_usize(8);
        for (size_t i = 0; i < len; ++i) w.push_back(static_cast<char>('a' + rng.range_usize(26)));
    }
    std::vector<double> cdf(vocab);
    double acc = 0.0;
    for (size_t i = 0; i < vocab; ++i) {
        acc += std::pow(static_cast<double>(i + 1), -1.1);
        cdf[i] = acc;
    }
    for (double& x : cdf) x /= acc;
    uint64_t cursor = 0;
    offsets[0] = 0;
    for (uint32_t s = 0; s < count; ++s) {
        double target_len = stddev < 0.0 ? static_cast<double>(min_len) + rng.next_unit_open() * static_cast<double>(max_len - min_len + 1)
                                         : mean + stddev * rng.normal();
        size_t len = static_cast<size_t>(std::llround(std::floor(target_len)));
        len = std::min<size_t>(std::max<size_t>(len, min_len), max_len);
        if (cursor + len > capacity) throw Error(LEO_ERR_INVALID_ARGUMENT, "story buffer capacity exceeded");
        size_t written = 0;
        while (written + 1 < len) {
            double u = rng.next_unit_open();
            const std::string& w = words[static_cast<size_t>(std::lower_bound(cdf.begin(), cdf.end(), u) - cdf.begin())];
            for (char ch : w) {
                if (written + 1 >= len) break;
                bytes[cursor + written++] = static_cast<uint8_t>(ch);
            }
            size_t p = rng.range_usize(100);
            const char* sep = p < 4 ? ", " : (p < 10 ? ". " : " ");
            for (const char* q = sep; *q; ++q) {
                if (written + 1 >= len) break;
                bytes[cursor + written++] = static_cast<uint8_t>(*q);
            }
        }
        bytes[cursor + written++] = static_cast<uint8_t>('\n');
        cursor += written;
        offsets[s + 1] = cursor;
    }
}

}  // namespace leo
