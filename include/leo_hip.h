/*
 * leo_hip.h -- C-ABI of the MI355X (gfx950) execution backend for Leo's
 * per-byte training step.
 *
 * The boundary mirrors the reference's execution-backend trait
 * `RuntimeBackend` (crates/leo-core/src/backend.rs:351-475) and its GPU
 * adapter `GpuRuntime` (backend.rs:547-794): a Rust `HipRuntime:
 * RuntimeBackend` binds these functions one-for-one.
 * Plain pointers and sizes only; every call returns an int32 status (0 = ok)
 * and leo_hip_last_error() returns the message of the last failure on the
 * calling thread. A handle is single-threaded (RuntimeBackend is Send, not
 * Sync: backend.rs:351); concurrent calls on one handle are rejected.
 * An explicit GPU request never falls back to the CPU
 * (docs/ADR-0001-EXECUTION-BACKENDS.md:9): without a usable gfx950 device,
 * leo_hip_create fails with LEO_ERR_DEVICE.
 */
#ifndef LEO_HIP_H
#define LEO_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "leo_hip_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (LeoErrorKind, crates/leo-core/src/lib.rs:41-128). */
enum {
    LEO_OK = 0,
    LEO_ERR_INVALID_ARGUMENT = 1,
    LEO_ERR_OUT_OF_MEMORY = 2,
    LEO_ERR_DEVICE = 3,
    LEO_ERR_NUMERICAL = 4, /* device guard tripped; sub-code in LeoStepMetrics.error_code */
    LEO_ERR_UNSUPPORTED = 5,
    LEO_ERR_INTERNAL = 6,
    LEO_ERR_BUSY = 7
};

/* Permission (crates/leo-core/src/permission.rs:6-11). */
enum { LEO_FROZEN = 0, LEO_PROVISIONAL = 1, LEO_TRAINING = 2, LEO_VERIFIED = 3 };

/* Synthetic topologies for leo_model_initialize_synthetic. */
enum { LEO_TOPOLOGY_UNIFORM = 0, LEO_TOPOLOGY_POWER_LAW = 1, LEO_TOPOLOGY_HEAVY_TAIL = 2 };

/* Host-side configuration: the 160-byte device block plus the fields that
 * only the host reads (config.rs:10-156). */
typedef struct LeoHostConfig {
    LeoConfig device;
    uint64_t seed;
    float excitatory_fraction;
    uint32_t plasticity_window;
    float end_document_weight;
    float provisional_strength;
    float training_strength;
    float verified_strength;
    float context_dropout_rate;
    float replay_fraction;
    uint32_t replay_segment_bytes;
    uint32_t replay_stateful_batch;
} LeoHostConfig;

/* TrainingStatistics (crates/leo-core/src/metrics.rs:4-15). */
typedef struct LeoStatistics {
    uint64_t processed_bytes;
    uint64_t processed_stories;
    double training_loss_sum;
    uint64_t training_targets;
    uint64_t active_neurons_sum;
    uint64_t active_neurons_peak;
    uint64_t synaptic_events;
    uint64_t numerical_rejections;
    uint64_t persistent_ticks;
} LeoStatistics;

/* Host model image in the reference's host layouts (model.rs:19-76): output
 * weights [257][N] and context output projection [257][E] are output-major.
 * Arrays are caller-owned; sizes follow from the config: N, N*S, 258*F,
 * max_order*slots_per_order, E. */
typedef struct LeoModelView {
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
    LeoStatistics statistics;
} LeoModelView;

/* StepMetrics (metrics.rs:39-66), the fields the device path produces. */
typedef struct LeoStepMetrics {
    float loss;
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
    uint32_t eligible_recurrent_synapses;
    uint32_t eligible_input_synapses;
    float target_probability;
    uint32_t error_code;
} LeoStepMetrics;

/* MergeMetrics (parallel.rs:305-310) + BatchTrainingReport (training.rs). */
typedef struct LeoBatchReport {
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
    double story_seconds;
    double merge_seconds;
    double replay_seconds;
} LeoBatchReport;

/* EvaluationMetrics with its ActivityDiagnostics
 * (crates/leo-cli/src/training/metrics.rs:6-24, 182-191). */
typedef struct LeoEvaluationReport {
    double loss;                       /* mean loss over targets */
    double bits_per_byte;              /* loss / ln 2 */
    double accuracy;                   /* predicted == target, over targets */
    uint64_t targets;
    uint64_t processed_stories;
    uint64_t processed_bytes;
    uint64_t neuron_count;
    uint64_t steps;
    uint64_t active_neurons_sum;
    uint64_t active_neurons_peak;
    uint64_t emitted_events;
    uint64_t suprathreshold_sum;
    uint64_t block_selected_sum;
    uint64_t cap_clipped_sum;
    uint64_t cap_hit_steps;
    double population_inhibition_sum;
    float population_inhibition_peak;
    uint32_t pad0;
    double eligibility_sum;
    uint64_t eligibility_count;
    uint64_t context_cells_sum;
    uint64_t context_probes_sum;
    uint64_t context_applied_steps;
    double context_loss_gain_sum;      /* neural-only loss minus loss, summed */
    uint64_t output_madds_sum;
} LeoEvaluationReport;

/* Device telemetry of the step kernel (the role of the reference's sampled
 * batch telemetry, cuda_plan.rs:67-103 / cuda.rs:8671-9022). kernel_ms is the
 * summed HIP-event time of the step-kernel launches on the runtime's stream;
 * algorithmic_bytes applies a per-lane-step byte model to the device's work
 * counters (events, touched neurons, eligible slots, destinations, ...). */
typedef struct LeoKernelStats {
    uint64_t launches;
    uint64_t lane_steps;
    double kernel_ms;
    double algorithmic_bytes;
    uint64_t events;
    uint64_t touched;
    uint64_t active;
    uint64_t scanned_rec;
    uint64_t scanned_in;
    uint64_t kept_rec;
    uint64_t kept_in;
    uint64_t destinations;
    uint64_t active_inhibitory;
    uint64_t merge_launches;
    double merge_ms;
    /* With LEO_HIP_PHASE_PROFILE=1 at creation: per step phase (deliver,
     * fold+select, active list+eligibility, post/readout, signals, learn, unused,
     * binding-cap global selection), the microseconds workgroup 0 of the first
     * lane spent working and waiting at the phase barrier. */
    double phase_work_us[8];
    double phase_wait_us[8];
    /* Story lanes resident on the device at once; larger batches run in
     * groups of this many lanes (sized from free device memory at creation). */
    uint64_t resident_lanes;
    /* The step-kernel figures above split by the lanes a launch served:
     * [0] story lanes of a logical batch, [1] the canonical runtime (replay,
     * in-place single-story passes and single steps). */
    uint64_t section_launches[2];
    uint64_t section_lane_steps[2];
    double section_kernel_ms[2];
    double section_bytes[2];
    /* Batch-end mean: (element, lane) pairs whose lane value differs from the
     * base, merged elements, and the algorithmic bytes they imply (24 B per
     * changed lane value -- lane value, base and the f64 accumulator
     * read-modify-write -- plus 4 (L+1) B per merged element for the
     * canonical write and the lane scatters). */
    uint64_t merge_lane_changes;
    uint64_t merge_elements;
    double merge_bytes;
    /* Eligible slots whose weight update a plasticity step applied: the kept
     * slots with nonzero eligibility (with zero eligibility the update leaves
     * the weight unchanged, bit for bit). */
    uint64_t learning_slots;
    /* Delivery buckets of more than 8 entries in one tick, folded by a whole
     * wave after a sort: ranked in registers (up to 128 entries) or radix
     * sorted through the target's shadow range. */
    uint64_t deep_register_folds;
    uint64_t deep_radix_folds;
} LeoKernelStats;

/* Selectors for leo_hip_parameter_changes (ParameterChanges, runtime.rs:37-46). */
enum {
    LEO_CHANGED_THRESHOLD = 0,
    LEO_CHANGED_RECURRENT = 1,
    LEO_CHANGED_INPUT = 2,
    LEO_CHANGED_OUTPUT_NEURONS = 3,
    LEO_CHANGED_CONTEXT_SLOTS = 4
};

/* Selectors for leo_hip_read_state (transient state of the canonical runtime). */
enum {
    LEO_STATE_MEMBRANE = 0, LEO_STATE_ACTIVATION, LEO_STATE_FATIGUE, LEO_STATE_BRANCHES,
    LEO_STATE_ADAPT0, LEO_STATE_ADAPT1, LEO_STATE_ADAPT2, LEO_STATE_SURROGATE,
    LEO_STATE_REC_BS, LEO_STATE_REC_MS, LEO_STATE_REC_FS, LEO_STATE_REC_AS0, LEO_STATE_REC_AS1,
    LEO_STATE_REC_AS2, LEO_STATE_REC_E,
    LEO_STATE_IN_BS, LEO_STATE_IN_MS, LEO_STATE_IN_FS, LEO_STATE_IN_AS0, LEO_STATE_IN_AS1,
    LEO_STATE_IN_AS2, LEO_STATE_IN_E,
    LEO_STATE_LOGITS, LEO_STATE_PROBABILITIES, LEO_STATE_ERRORS, LEO_STATE_LEARNING_SIGNAL,
    LEO_STATE_F32_COUNT
};
/* Index sets for leo_hip_read_list (sorted ascending; ACTIVE in selection order). */
enum {
    LEO_LIST_ACTIVE = 0, LEO_LIST_TOUCHED = 1, LEO_LIST_ELIGIBLE_REC = 2, LEO_LIST_ELIGIBLE_IN = 3
};

typedef struct LeoHipRuntime LeoHipRuntime;

/* Message of the last failed call on this thread. */
int32_t leo_hip_last_error(char* buffer, size_t capacity);
/* LEO_HIP_ABI_VERSION of the loaded library (cuda_abi.def:1 `abi_version`). */
int32_t leo_hip_abi_version(void);

/* SplitMix64 stream of crates/leo-core/src/rng.rs:13-19 (the generator every seeded
 * initialisation draws from): writes `count` successive next_u64() values. */
int32_t leo_splitmix64(uint64_t seed, uint64_t* out, uint64_t count);

/* Model::initialize (crates/leo-core/src/model.rs:79-158): seeded SplitMix64
 * (rng.rs:13-42) initialisation into caller-owned arrays. */
int32_t leo_model_initialize(const LeoHostConfig* config, LeoModelView* out);
/* Seeded synthetic topology for the benchmark workloads: Leo-valid fixed-S rows,
 * targets drawn uniform / power-law / heavy-tailed (in-degree capped at
 * `in_degree_cap` when nonzero), weights |N(0,weight_sigma)| signed by source
 * type; thresholds, input, output and context follow model.rs:116-137, 461-496. */
int32_t leo_model_initialize_synthetic(const LeoHostConfig* config, uint32_t topology,
                                       float exponent, uint32_t in_degree_cap,
                                       float weight_sigma, LeoModelView* out);
/* Model::validate (model.rs:223-396). */
int32_t leo_model_validate(const LeoHostConfig* config, const LeoModelView* model);
/* Seeded Zipf-ASCII stories: `count` stories written back to back into `bytes`
 * (capacity bytes), offsets[count+1]. Length ~ N(mean,stddev) clipped to
 * [min_len,max_len], or uniform in [min_len,max_len] when stddev < 0. */
int32_t leo_synthetic_stories(uint64_t seed, uint32_t count, double mean, double stddev,
                              uint32_t min_len, uint32_t max_len, uint8_t* bytes,
                              uint64_t capacity, uint64_t* offsets);

/* BackendRuntime::new(model, BackendKind::Gpu) -> GpuRuntime::new
 * (backend.rs:555-566, cuda.rs:1894 CudaRuntime::new_on_device): upload the
 * canonical model to `device` and size story lanes for up to `max_lanes`
 * logical workers. */
int32_t leo_hip_create(const LeoHostConfig* config, const LeoModelView* model, int32_t device,
                       uint32_t max_lanes, LeoHipRuntime** out);
void leo_hip_destroy(LeoHipRuntime* runtime);

/* RuntimeBackend::begin_document / finish_document / reset_transient_state
 * (backend.rs:391-402). */
int32_t leo_hip_begin_document(LeoHipRuntime* runtime);
int32_t leo_hip_finish_document(LeoHipRuntime* runtime);
int32_t leo_hip_reset_transient_state(LeoHipRuntime* runtime);
/* RuntimeBackend::enable_parameter_tracking (backend.rs:358). */
int32_t leo_hip_enable_parameter_tracking(LeoHipRuntime* runtime);

/* RuntimeBackend::step (backend.rs:403-408); target < 0 means None. */
int32_t leo_hip_step(LeoHipRuntime* runtime, uint32_t symbol, int32_t target,
                     int32_t permission, LeoStepMetrics* out);
/* RuntimeBackend::training_step_batch (backend.rs:413-422): `count` dependent
 * steps in one device launch; targets[i] < 0 means None. */
int32_t leo_hip_training_step_batch(LeoHipRuntime* runtime, const uint32_t* symbols,
                                    const int32_t* targets, uint32_t count, int32_t permission,
                                    LeoStepMetrics* out);
/* RuntimeBackend::advance_frozen_batch (backend.rs:428-431). */
int32_t leo_hip_advance_frozen_batch(LeoHipRuntime* runtime, const uint32_t* symbols,
                                     uint32_t count);
/* RuntimeBackend::replay_streaming_batch (backend.rs:439-453): one mixed
 * timeline without resets; targets[i] >= 0 positions are supervised with
 * `permission`, targets[i] < 0 positions advance frozen state. Metrics are
 * written to out[] for supervised positions only (*supervised of them). */
int32_t leo_hip_replay_streaming_batch(LeoHipRuntime* runtime, const uint32_t* symbols,
                                       const int32_t* targets, uint32_t count, int32_t permission,
                                       LeoStepMetrics* out, uint32_t* supervised);
/* RuntimeBackend::training_story_batch (backend.rs:457-463): one device lane
 * per story, each forked from the canonical revision at tick 0, followed by
 * the batch-end lane-ordered mean (parallel.rs:694-798). The canonical model
 * is merged when the call returns. losses_out (optional) receives, story by
 * story, the story_len+1 per-step losses. */
int32_t leo_hip_training_story_batch(LeoHipRuntime* runtime, const uint8_t* bytes,
                                     const uint64_t* offsets, uint32_t count,
                                     int32_t permission, float* losses_out,
                                     LeoBatchReport* report);
/* TrainingEngine::train_batch -> train_story_batch (crates/leo-cli/src/training.rs:1539-1727):
 * the story batch (or the in-place single-story pass) followed, when
 * replay_enabled, by bounded-surprise replay on the canonical runtime. */
int32_t leo_hip_train_batch(LeoHipRuntime* runtime, const uint8_t* bytes, const uint64_t* offsets,
                            uint32_t count, int32_t permission, uint32_t replay_enabled,
                            float* losses_out, LeoBatchReport* report);

/* evaluate_model_shard (crates/leo-cli/src/training/validation.rs:65-135):
 * every non-empty story scored frozen -- begin_document, its document steps
 * (training.rs:1747-1757) with Permission::Frozen and their targets, then
 * finish_document -- with no learning and no statistics, accumulated as
 * record_evaluation_step does (validation.rs:137-154). Stories run on story
 * lanes that read the canonical image (frozen steps write no parameter), lane
 * i starting at the tick the sequential loop would reach, so every loss,
 * prediction and worklist equals one runtime scoring the stories in order;
 * the canonical runtime ends reset, its tick advanced past every step.
 * losses_out (optional) receives each non-empty story's len+1 step losses. */
int32_t leo_hip_evaluate(LeoHipRuntime* runtime, const uint8_t* bytes, const uint64_t* offsets,
                         uint32_t count, float* losses_out, LeoEvaluationReport* report);

/* RuntimeBackend::synchronize_model + model() (backend.rs:355-356): copy the
 * canonical model into caller-owned arrays (host layouts). */
int32_t leo_hip_download_model(LeoHipRuntime* runtime, LeoModelView* out);
/* RuntimeBackend::synchronize_model (backend.rs:356) as the GPU adapter does
 * it (cuda.rs:2817-2825 -> sync_changed_model_to_host, cuda.rs:5657-5760):
 * `mirror` is the caller's host model, current as of its last synchronisation
 * (leo_hip_download_model, this call, or the model the runtime was created or
 * uploaded with); only the elements of the canonical model changed since then
 * -- by steps, the batch-end mean, the keyed context merge -- are written into
 * it, plus the whole bias / context output projection when they changed, and
 * the generation, revision and statistics. The Rust adapter calls it in
 * parameter_changes() before returning, so that
 * PackedSparseModelUpdate::from_model reads current values (training.rs:1558-1562,
 * 1644-1648). */
int32_t leo_hip_synchronize_model(LeoHipRuntime* runtime, LeoModelView* mirror);

/* PackedSparseModelUpdate (crates/leo-core/src/parallel.rs:79-97): canonical
 * values of changed elements in packed layouts -- output rows neuron by
 * neuron (257 values each), context rows slot by slot (E values each). The
 * bias (257 values) and the context output projection (257*E, output-major)
 * are whole or NULL. */
typedef struct LeoPackedUpdate {
    const uint32_t* threshold_indices;
    const float* threshold_values;
    uint64_t threshold_count;
    const uint32_t* recurrent_indices;
    const float* recurrent_values;
    uint64_t recurrent_count;
    const uint32_t* input_indices;
    const float* input_values;
    uint64_t input_count;
    const uint32_t* output_neurons;
    const float* output_values_by_neuron;
    uint64_t output_count;
    const uint32_t* context_slots;
    const uint64_t* context_keys;
    const uint32_t* context_observations;
    const float* context_embeddings;
    uint64_t context_count;
    const float* output_bias;
    const float* context_output_weights;
    uint64_t generation;
    uint64_t parameter_revision;
    LeoStatistics statistics;
} LeoPackedUpdate;

/* RuntimeBackend::synchronize_packed_model (backend.rs:374-376, GPU adapter
 * cuda.rs:2844-2857 -> 2869-3080): scatter the packed rows into the canonical
 * device image (PackedSparseModelUpdate::apply_to_model, parallel.rs:186-302,
 * with its index and size checks) and take the update's generation, revision
 * and statistics; parameter tracking ends. Story lanes need no scatter: each
 * logical batch forks its lanes from the canonical image. */
int32_t leo_hip_synchronize_packed_model(LeoHipRuntime* runtime, const LeoPackedUpdate* update);
/* RuntimeBackend::commit_packed_host_model (backend.rs:378-387, cuda.rs:2859-2868):
 * the same scatter, keeping parameter tracking as it is. */
int32_t leo_hip_commit_packed_host_model(LeoHipRuntime* runtime, const LeoPackedUpdate* update);
/* No counterpart in the reference: leo_hip_commit_packed_host_model for
 * callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). It stages the packed rows
 * in a fixed 8 MiB device scratch array per GPU instead of the runtime's
 * growable buffer, and calls no device allocation. An update one of whose
 * tensors needs more than 8 MiB of staging (indices and values, e.g. more
 * than about 8,100 output rows or 1M recurrent elements) is refused with
 * LEO_ERR_INVALID_ARGUMENT before anything is written. All runtimes on a GPU
 * share its scratch, so overlapping calls on one GPU are serialised by a
 * per-device lock held until the commit's copies and kernels are done. */
int32_t leo_hip_commit_packed_host_model_no_alloc(LeoHipRuntime* runtime, const LeoPackedUpdate* update);
/* RuntimeBackend::model_mut (backend.rs:357): replace the canonical model. */
int32_t leo_hip_upload_model(LeoHipRuntime* runtime, const LeoModelView* model);
/* RuntimeBackend::parameter_changes (backend.rs:359): the tracked index set
 * `which` of the canonical runtime, sorted ascending. Returns the count in
 * *count; writes up to `capacity` indices when out is non-null. */
int32_t leo_hip_parameter_changes(LeoHipRuntime* runtime, int32_t which, uint64_t* out,
                                  uint64_t capacity, uint64_t* count, uint32_t* bias_dirty,
                                  uint32_t* context_output_dirty);
/* RuntimeBackend::probabilities / active_neurons (backend.rs:388-389). */
int32_t leo_hip_probabilities(LeoHipRuntime* runtime, float* out257);
int32_t leo_hip_read_list(LeoHipRuntime* runtime, int32_t which, uint64_t* out,
                          uint64_t capacity, uint64_t* count);
/* RuntimeBackend::active_neurons + activation (backend.rs:388-390, which the
 * GPU adapter serves from its host mirror, cuda.rs:3086-3092, refreshed with
 * the device's active list and values after each step, cuda.rs:5213-5229):
 * the last step's active neurons in selection order with their activations
 * (every other neuron's activation is 0). Returns the count in *count; writes
 * up to `capacity` entries of each array that is non-null. */
int32_t leo_hip_read_active(LeoHipRuntime* runtime, uint64_t* neurons, float* activations,
                            uint64_t capacity, uint64_t* count);
/* Transient state of the canonical runtime for parity checks; `count` must
 * equal the state's element count. */
int32_t leo_hip_read_state(LeoHipRuntime* runtime, int32_t which, float* out, uint64_t count);
uint64_t leo_hip_current_tick(const LeoHipRuntime* runtime);
/* Accumulated device telemetry since creation or the last reset (reset != 0
 * clears it after copying). */
int32_t leo_hip_kernel_stats(LeoHipRuntime* runtime, LeoKernelStats* out, int32_t reset);

#ifdef __cplusplus
}
#endif

#endif
