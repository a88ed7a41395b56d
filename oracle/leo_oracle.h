/*
 * TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of Leo's reference executor (saravanaspar/Leo v1.0.41),
 * written from the Rust sources read as text:
 *   crates/leo-core/src/runtime.rs    Runtime::step and every phase it calls
 *   crates/leo-core/src/learning.rs   surrogate, branch Jacobian, clip, inhibitory delta
 *   crates/leo-core/src/model.rs      resolve_context_slot, validate
 *   crates/leo-core/src/config.rs     plasticity_step
 *   crates/leo-core/src/parallel.rs   SparseModelDelta, apply_mean_deltas, merged_parameter_changes
 *   crates/leo-cli/src/training.rs    train_story_batch (CPU path), train_document_pass,
 *                                     select_replay_ranges, replay executors
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker or the CPU baseline. The product
 * (leo_amd/) never links or calls it.
 *
 * Pins (tests/test_oracle_reference.py, tests/test_known_answers.py): the
 * reference's own unit tests of runtime.rs, runtime_smoke.rs, learning.rs,
 * parallel.rs and main.rs restated against this library; brute force for
 * block selection order and replay range selection; published SplitMix64 and
 * FNV-1a vectors for the dropout hash and the context key.
 *
 * Parity unpinned (no reference-held vector covers them; the reference is Rust
 * and cannot run here): multi-step Runtime::step trajectories on random
 * models, context-slot eviction under collisions in the keyed context merge,
 * and end-to-end train_story_batch + replay state. exp/ln are glibc expf/logf,
 * the functions Rust's f32::exp/ln call on x86_64 Linux.
 */
#ifndef LEO_ORACLE_H
#define LEO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OracleConfig {
    uint64_t seed;
    uint64_t refractory_ticks;
    uint32_t neuron_count;
    uint32_t block_count;
    uint32_t neurons_per_block;
    uint32_t branches_per_neuron;
    uint32_t synapses_per_neuron;
    uint32_t input_fanout;
    uint32_t max_active_per_block;
    uint32_t max_active_global;
    float excitatory_fraction;
    float branch_decay;
    float membrane_decay;
    float fatigue_decay;
    float fatigue_gain;
    float target_activity;
    float threshold_homeostasis_rate;
    float population_inhibition_rate;
    float population_inhibition_max;
    float adaptation_decay[3];
    float adaptation_gain[3];
    float membrane_reset_fraction;
    float output_learning_rate;
    float recurrent_learning_rate;
    float inhibitory_learning_rate;
    float eligibility_decay;
    float eligibility_epsilon;
    float surrogate_width;
    float surrogate_gain;
    float max_update;
    float weight_min;
    float weight_max;
    float provisional_strength;
    float training_strength;
    float verified_strength;
    float end_document_weight;
    uint32_t plasticity_window;
    uint32_t context_max_order;
    uint32_t context_embedding_dim;
    uint32_t context_slots_per_order;
    uint32_t context_probe_limit;
    uint32_t context_confidence_observations;
    float context_learning_rate;
    float context_dropout_rate;
    float replay_fraction;
    uint32_t replay_segment_bytes;
    uint32_t replay_stateful_batch;
    uint32_t reserved;
} OracleConfig;

typedef struct OracleStatistics {
    uint64_t processed_bytes;
    uint64_t processed_stories;
    double training_loss_sum;
    uint64_t training_targets;
    uint64_t active_neurons_sum;
    uint64_t active_neurons_peak;
    uint64_t synaptic_events;
    uint64_t numerical_rejections;
    uint64_t persistent_ticks;
} OracleStatistics;

/* Host model image in the reference's host layouts: output weights and the
 * context output projection are output-major ([257][N], [257][E]). */
typedef struct OracleModelView {
    float* threshold;
    float* excitability;
    uint8_t* neuron_type;
    uint32_t* rec_target;
    uint8_t* rec_branch;
    uint8_t* rec_delay;
    float* rec_weight;
    uint32_t* in_target;
    uint8_t* in_branch;
    float* in_weight;
    float* out_weight;
    float* bias;
    uint64_t* ctx_keys;
    float* ctx_emb;
    uint32_t* ctx_obs;
    float* ctx_out;
    uint64_t generation;
    uint64_t parameter_revision;
    OracleStatistics statistics;
} OracleModelView;

typedef struct OracleStepMetrics {
    float loss;            /* NaN when the step had no target */
    uint32_t has_loss;
    uint32_t predicted_symbol;
    uint32_t active_neurons;
    uint32_t emitted_events;
    uint32_t suprathreshold_neurons;
    uint32_t block_selected_neurons;
    uint32_t global_cap_clipped_neurons;
    float population_inhibition;
    uint32_t context_cells;
    uint32_t context_probes;
    uint32_t context_applied;
    float context_loss_gain;
    uint32_t output_madds;
    uint32_t eligible_recurrent_synapses;
    uint32_t eligible_input_synapses;
    float mean_abs_eligibility;
    float target_probability;
} OracleStepMetrics;

typedef struct OracleBatchReport {
    double mean_loss;
    uint64_t targets;
    uint64_t stories;
    uint64_t replay_segments;
    uint64_t replay_steps;
    uint64_t replay_prefix_steps;
    uint64_t merge_workers;
    uint64_t merge_fixed_parameter_updates;
    uint64_t merge_context_keys;
    uint64_t activity_steps;
    uint64_t active_neurons_sum;
    uint64_t emitted_events;
} OracleBatchReport;

enum {
    ORACLE_OK = 0,
    ORACLE_ERR_INTERNAL = 1,
    ORACLE_ERR_NUMERICAL = 2,
    ORACLE_ERR_ARGUMENT = 3,
};

enum { ORACLE_FROZEN = 0, ORACLE_PROVISIONAL = 1, ORACLE_TRAINING = 2, ORACLE_VERIFIED = 3 };

/* Dense state selectors for oracle_read_f32 / oracle_read_u64. */
enum {
    ORACLE_F_MEMBRANE = 0, ORACLE_F_ACTIVATION, ORACLE_F_FATIGUE, ORACLE_F_BRANCHES,
    ORACLE_F_ADAPT0, ORACLE_F_ADAPT1, ORACLE_F_ADAPT2, ORACLE_F_SURROGATE,
    ORACLE_F_REC_BS, ORACLE_F_REC_MS, ORACLE_F_REC_FS, ORACLE_F_REC_AS0, ORACLE_F_REC_AS1,
    ORACLE_F_REC_AS2, ORACLE_F_REC_E,
    ORACLE_F_IN_BS, ORACLE_F_IN_MS, ORACLE_F_IN_FS, ORACLE_F_IN_AS0, ORACLE_F_IN_AS1,
    ORACLE_F_IN_AS2, ORACLE_F_IN_E,
    ORACLE_F_LOGITS, ORACLE_F_PROBABILITIES, ORACLE_F_ERRORS, ORACLE_F_LEARNING_SIGNAL,
    ORACLE_F_BLOCK_CUTOFF, ORACLE_F_CONTEXT_LATENT,
    ORACLE_F_COUNT
};
enum {
    ORACLE_U_REFRACTORY = 0, ORACLE_U_NEURON_LAST_TICK, ORACLE_U_REC_LAST_TICK,
    ORACLE_U_IN_LAST_TICK, ORACLE_U_COUNT
};
/* Index lists for oracle_read_list (sets are returned sorted ascending, the
 * active list in selection order). */
enum {
    ORACLE_L_ACTIVE = 0, ORACLE_L_TOUCHED, ORACLE_L_ELIGIBLE_REC, ORACLE_L_ELIGIBLE_IN,
    ORACLE_L_LEARNING_DESTINATIONS, ORACLE_L_CHANGED_THRESHOLD, ORACLE_L_CHANGED_REC,
    ORACLE_L_CHANGED_IN, ORACLE_L_CHANGED_OUTPUT, ORACLE_L_CHANGED_CONTEXT,
    ORACLE_L_ACTIVE_CONTEXT_SLOTS, ORACLE_L_COUNT
};

typedef struct OracleRuntime OracleRuntime;

int32_t oracle_last_error(char* buffer, size_t capacity);

int32_t oracle_runtime_new(const OracleConfig* config, const OracleModelView* model,
                           OracleRuntime** out);
void oracle_runtime_free(OracleRuntime* runtime);
int32_t oracle_runtime_read_model(const OracleRuntime* runtime, OracleModelView* out);
/* model_mut(): replace the learned image and mark the neuron-major cache dirty. */
int32_t oracle_runtime_write_model(OracleRuntime* runtime, const OracleModelView* model);
int32_t oracle_begin_document(OracleRuntime* runtime);
int32_t oracle_finish_document(OracleRuntime* runtime);
int32_t oracle_reset_transient_state(OracleRuntime* runtime);
int32_t oracle_enable_parameter_tracking(OracleRuntime* runtime);
/* The GPU adapter's tracking restart (cuda.rs:2827-2837): empty change sets
 * and clean dirty flags on every call. */
int32_t oracle_restart_parameter_tracking(OracleRuntime* runtime);
int32_t oracle_changes_flags(const OracleRuntime* runtime, uint32_t* bias_dirty,
                             uint32_t* context_output_dirty);
int32_t oracle_step(OracleRuntime* runtime, uint32_t symbol, int32_t target, int32_t permission,
                    OracleStepMetrics* out);
uint64_t oracle_current_tick(const OracleRuntime* runtime);
float oracle_population_inhibition(const OracleRuntime* runtime);
int64_t oracle_read_list(const OracleRuntime* runtime, int32_t which, uint64_t* out,
                         size_t capacity);
int32_t oracle_read_f32(const OracleRuntime* runtime, int32_t which, float* out, size_t count);
int32_t oracle_read_u64(const OracleRuntime* runtime, int32_t which, uint64_t* out, size_t count);

/* Training coordinator (training.rs:1539 train_story_batch, CPU path). One OS
 * thread per story when more than one story is given. Per-story losses are
 * written to losses_out (story order, story_len+1 entries each) when given. */
int32_t oracle_train_story_batch(OracleRuntime* runtime, const uint8_t* bytes,
                                 const uint64_t* offsets, uint32_t story_count,
                                 int32_t permission, uint32_t replay_enabled,
                                 float* losses_out, OracleBatchReport* report);

/* One document pass (training.rs:1729) on this runtime. */
int32_t oracle_train_document_pass(OracleRuntime* runtime, const uint8_t* story, uint64_t length,
                                   int32_t permission, float* losses_out);

/* Replay executor over explicit ranges (training.rs:394 execute_replay_ranges). */
int32_t oracle_execute_replay_ranges(OracleRuntime* runtime, const uint8_t* story,
                                     uint64_t length, const uint64_t* ranges, uint32_t count,
                                     int32_t permission, uint64_t* replay_steps,
                                     uint64_t* prefix_steps);

/* training.rs:1782. ranges_out holds (start,end) pairs; returns the count or -1. */
int64_t oracle_select_replay_ranges(const float* losses, uint64_t count, float fraction,
                                    uint64_t segment_targets, uint64_t* ranges_out,
                                    size_t capacity);

/* Sparse deltas and batch merge (parallel.rs). Deltas are opaque handles. */
typedef struct OracleDelta OracleDelta;
int32_t oracle_delta_between(const OracleConfig* config, const OracleModelView* base,
                             const OracleModelView* trained, OracleDelta** out);
int32_t oracle_delta_between_tracked(const OracleModelView* base, const OracleRuntime* trained,
                                     OracleDelta** out);
void oracle_delta_free(OracleDelta* delta);
int64_t oracle_delta_count(const OracleDelta* delta, int32_t which);
int32_t oracle_delta_equal(const OracleDelta* left, const OracleDelta* right);
/* Merge into `master` (a runtime used as the canonical model owner).
 * divisor_mode 0 = mean (apply_mean_deltas), 1 = sum (apply_sum_deltas). */
int32_t oracle_apply_deltas(OracleRuntime* master, OracleDelta* const* deltas, uint32_t count,
                            int32_t divisor_mode, uint64_t* fixed_updates,
                            uint64_t* context_keys);

/* Helpers from learning.rs / runtime.rs / model.rs exposed for known-answer tests. */
float oracle_analog_rank_surrogate(float margin, float cutoff, int32_t selected, float width,
                                   float gain);
float oracle_branch_jacobian(uint8_t branch, float excitability, float temporal, float gate);
float oracle_bounded_delta(float value, float maximum);
float oracle_inhibitory_homeostasis_delta(float source_activation, float target_activity,
                                          float desired_activity, float learning_rate,
                                          float strength, float maximum_update);
int32_t oracle_context_survives_dropout(uint64_t seed, uint64_t tick, uint32_t symbol,
                                        float rate);
uint64_t oracle_context_key(const uint32_t* history, size_t history_len, size_t order);
float oracle_decay_for_elapsed(float base, uint64_t elapsed);
int32_t oracle_resolve_context_slot(OracleRuntime* runtime, uint64_t order, uint64_t key,
                                    int32_t allocate, int64_t* slot, uint64_t* probes);
/* runtime.rs:1757 test hook: run update_context_projection with explicit
 * active slots, scales and errors. */
int32_t oracle_test_update_context_projection(OracleRuntime* runtime, const uint64_t* slots,
                                              const float* scales, uint32_t count,
                                              const float* errors, float strength);
int32_t oracle_plasticity_step(uint32_t window, uint64_t phase, int32_t end_document,
                               float* scale, uint64_t* next_phase);

#ifdef __cplusplus
}
#endif

#endif
