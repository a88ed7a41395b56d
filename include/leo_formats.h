/* Persistent artifacts on the host side of the MI355X backend: PSCLS100 model
 * checkpoints (crates/leo-format/src/lib.rs), LEODATA1 prepared datasets
 * (crates/leo-data/src/lib.rs) and their SHA-256 identities
 * (crates/leo-core/src/artifact.rs). Plain host code in libleo_hip.so; none of
 * it touches the GPU. Every entry returns a LEO_OK / LEO_ERR_* status and
 * leaves the message for leo_hip_last_error. */
#ifndef LEO_FORMATS_H
#define LEO_FORMATS_H

#include <stddef.h>
#include <stdint.h>

#include "leo_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the artifact layer (LeoError::checkpoint_corrupt,
 * checkpoint_incompatible and io in crates/leo-core/src/lib.rs:41-128). */
enum { LEO_ERR_CORRUPT = 8, LEO_ERR_INCOMPATIBLE = 9, LEO_ERR_IO = 10 };

/* ArtifactDigest (artifact.rs): 32 SHA-256 bytes. */
typedef struct LeoDigest {
    uint8_t bytes[32];
} LeoDigest;

/* digest_bytes / digest_file (artifact.rs). */
int32_t leo_sha256(const uint8_t* data, uint64_t length, LeoDigest* out);
int32_t leo_sha256_file(const char* path, LeoDigest* out);

/* ---- PSCLS100 checkpoints ------------------------------------------------ */

/* What a checkpoint holds before it is decoded: the header's generation, the
 * CONFIG section (the model's TOML configuration text) as a range of the
 * checkpoint bytes, and the tensor shapes the configuration must agree with. */
typedef struct LeoCheckpointInfo {
    uint64_t generation;
    uint64_t parameter_revision;
    uint64_t config_offset;
    uint64_t config_length;
    uint64_t neuron_count;
    uint64_t synapses_per_neuron;
    uint64_t input_fanout;
    uint64_t context_slots;
    uint64_t context_embedding_dim;
} LeoCheckpointInfo;

/* Size of encode_model's output (lib.rs:289-444) for this configuration and
 * configuration text. */
int32_t leo_checkpoint_encoded_size(const LeoHostConfig* config, uint64_t config_length, uint64_t* bytes_out);

/* encode_model (lib.rs:289-444): the model is validated first
 * (save_model_atomic, lib.rs:149); `config_toml` is Config::to_toml's text of
 * `config`. Writes exactly leo_checkpoint_encoded_size bytes. */
int32_t leo_checkpoint_encode(const LeoHostConfig* config, const LeoModelView* model, const char* config_toml,
                              uint64_t config_length, uint8_t* out, uint64_t capacity);

/* The structural half of decode_model (lib.rs:446-620): header, descriptor
 * table, ranges, per-section SHA-256, the required section set, the CONFIG
 * pointer and the semantics contract. On success `info` locates the CONFIG
 * text and the stored shapes. */
int32_t leo_checkpoint_inspect(const uint8_t* bytes, uint64_t length, LeoCheckpointInfo* info);

/* decode_model (lib.rs:446-620) into caller-owned arrays sized for `config`
 * (the configuration parsed from the CONFIG text): every check of
 * leo_checkpoint_inspect, the section payloads, the generation metadata,
 * Model::validate and the shape table (validate_shapes, lib.rs:718-800). */
int32_t leo_checkpoint_decode(const uint8_t* bytes, uint64_t length, const LeoHostConfig* config,
                              LeoModelView* model);

/* save_model_atomic (lib.rs:144-175): encode, write `path`.tmp, fsync, rename
 * over `path`, fsync the directory. With retain_previous and an existing
 * checkpoint at `path`, that checkpoint is first copied to
 * `path`.genNNNNNN (its own generation) unless that file exists. */
int32_t leo_checkpoint_save_atomic(const char* path, const LeoHostConfig* config, const LeoModelView* model,
                                   const char* config_toml, uint64_t config_length, uint32_t retain_previous);

/* read_generation (lib.rs:258-264): the generation of a checkpoint file's
 * validated header. */
int32_t leo_checkpoint_read_generation(const char* path, uint64_t* generation);

/* prune_generations (lib.rs:201-239): keeps the `keep_previous` newest
 * `path`.genNNNNNN files beside `path`. */
int32_t leo_checkpoint_prune_generations(const char* path, uint64_t keep_previous);

/* ---- LEODATA1 prepared datasets ------------------------------------------ */

/* StoryIndex (lib.rs:22-27), the index's 16-byte record. */
typedef struct LeoStoryIndex {
    uint64_t offset;
    uint32_t length;
    uint32_t split_flags;
} LeoStoryIndex;

/* DatasetIdentity (lib.rs:29-38). */
typedef struct LeoDatasetIdentity {
    uint32_t schema_version;
    uint32_t reserved;
    uint64_t record_count;
    uint64_t bytes_length;
    LeoDigest bytes_digest;
    LeoDigest records_digest;
    LeoDigest provenance_digest;
    LeoDigest dataset_id;
} LeoDatasetIdentity;

typedef struct LeoDataset LeoDataset;

/* compute_dataset_id (lib.rs:237-253). */
int32_t leo_dataset_compute_id(uint32_t schema_version, uint64_t record_count, uint64_t bytes_length,
                               const LeoDigest* bytes_digest, const LeoDigest* records_digest,
                               const LeoDigest* provenance_digest, LeoDigest* out);

/* write_index (lib.rs:255-323); `identity` may be null. */
int32_t leo_dataset_write_index(const char* index_path, const char* bytes_path, const LeoStoryIndex* entries,
                                uint64_t count, const LeoDigest* provenance, LeoDatasetIdentity* identity);

/* PreparedDataset::open (lib.rs:46-185): validates the whole artifact pair
 * (header digest, byte length and digest, record-table digest, dataset ID,
 * every record range) before returning a handle. */
int32_t leo_dataset_open(const char* bytes_path, const char* index_path, LeoDataset** out);
void leo_dataset_close(LeoDataset* dataset);
int32_t leo_dataset_identity(const LeoDataset* dataset, LeoDatasetIdentity* out);
uint64_t leo_dataset_len(const LeoDataset* dataset);
int32_t leo_dataset_entry(const LeoDataset* dataset, uint64_t index, LeoStoryIndex* out);

/* PreparedDataset::story (lib.rs:205-228): the story's bytes, checked to be
 * UTF-8; `length` receives its size (also when `capacity` is too small, which
 * fails with LEO_ERR_INVALID_ARGUMENT and writes nothing). */
int32_t leo_dataset_story(LeoDataset* dataset, uint64_t index, uint8_t* out, uint64_t capacity, uint64_t* length);

/* Stories [first, first + count) packed for leo_hip_train_batch /
 * leo_hip_evaluate: bytes back to back, offsets[0..count] (offsets[0] = 0).
 * With `bytes` null only offsets are written (to size the buffer). Each story
 * is checked to be UTF-8 as by leo_dataset_story. */
int32_t leo_dataset_pack(LeoDataset* dataset, uint64_t first, uint64_t count, uint8_t* bytes, uint64_t capacity,
                         uint64_t* offsets);

#ifdef __cplusplus
}
#endif

#endif
