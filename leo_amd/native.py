"""ctypes binding of the C-ABI in include/leo_hip.h (libleo_hip.so).

The library is built in-tree by ``python -m leo_amd.build``. Loading fails
loudly when it is missing: there is no CPU fallback behind this module.
"""
from __future__ import annotations

import ctypes
import pathlib
from typing import Optional

from ._abi import LeoConfig

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libleo_hip.so"

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_OUT_OF_MEMORY = 2
ERR_DEVICE = 3
ERR_NUMERICAL = 4
ERR_UNSUPPORTED = 5
ERR_INTERNAL = 6
ERR_BUSY = 7
ERR_CORRUPT = 8        # include/leo_formats.h: checkpoint / dataset artifact damaged
ERR_INCOMPATIBLE = 9   # artifact of another format version or semantics
ERR_IO = 10

FROZEN, PROVISIONAL, TRAINING, VERIFIED = 0, 1, 2, 3
TOPOLOGY_UNIFORM, TOPOLOGY_POWER_LAW, TOPOLOGY_HEAVY_TAIL = 0, 1, 2

CHANGED_THRESHOLD, CHANGED_RECURRENT, CHANGED_INPUT, CHANGED_OUTPUT_NEURONS, CHANGED_CONTEXT_SLOTS = range(5)
LIST_ACTIVE, LIST_TOUCHED, LIST_ELIGIBLE_REC, LIST_ELIGIBLE_IN = range(4)
STATE_NAMES = [
    "membrane", "activation", "fatigue", "branches", "adapt0", "adapt1", "adapt2", "surrogate",
    "rec_bs", "rec_ms", "rec_fs", "rec_as0", "rec_as1", "rec_as2", "rec_e",
    "in_bs", "in_ms", "in_fs", "in_as0", "in_as1", "in_as2", "in_e",
    "logits", "probabilities", "errors", "learning_signal",
]
STATE = {name: i for i, name in enumerate(STATE_NAMES)}


class LeoError(RuntimeError):
    """A failed C-ABI call: ``code`` is the LEO_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class LeoHostConfig(ctypes.Structure):
    _fields_ = [
        ("device", LeoConfig),
        ("seed", ctypes.c_uint64),
        ("excitatory_fraction", ctypes.c_float),
        ("plasticity_window", ctypes.c_uint32),
        ("end_document_weight", ctypes.c_float),
        ("provisional_strength", ctypes.c_float),
        ("training_strength", ctypes.c_float),
        ("verified_strength", ctypes.c_float),
        ("context_dropout_rate", ctypes.c_float),
        ("replay_fraction", ctypes.c_float),
        ("replay_segment_bytes", ctypes.c_uint32),
        ("replay_stateful_batch", ctypes.c_uint32),
    ]


class LeoStatistics(ctypes.Structure):
    _fields_ = [
        ("processed_bytes", ctypes.c_uint64),
        ("processed_stories", ctypes.c_uint64),
        ("training_loss_sum", ctypes.c_double),
        ("training_targets", ctypes.c_uint64),
        ("active_neurons_sum", ctypes.c_uint64),
        ("active_neurons_peak", ctypes.c_uint64),
        ("synaptic_events", ctypes.c_uint64),
        ("numerical_rejections", ctypes.c_uint64),
        ("persistent_ticks", ctypes.c_uint64),
    ]


_P = ctypes.c_void_p


class LeoModelView(ctypes.Structure):
    _fields_ = [
        ("threshold", _P), ("excitability", _P), ("neuron_type", _P), ("rec_target", _P), ("rec_branch", _P),
        ("rec_delay", _P), ("rec_weight", _P), ("in_target", _P), ("in_branch", _P), ("in_weight", _P),
        ("out_weight", _P), ("bias", _P), ("ctx_keys", _P), ("ctx_emb", _P), ("ctx_obs", _P), ("ctx_out", _P),
        ("generation", ctypes.c_uint64),
        ("parameter_revision", ctypes.c_uint64),
        ("statistics", LeoStatistics),
    ]


class LeoStepMetrics(ctypes.Structure):
    _fields_ = [
        ("loss", ctypes.c_float), ("has_loss", ctypes.c_uint32), ("predicted_symbol", ctypes.c_uint32),
        ("active_neurons", ctypes.c_uint32), ("emitted_events", ctypes.c_uint32),
        ("suprathreshold_neurons", ctypes.c_uint32), ("block_selected_neurons", ctypes.c_uint32),
        ("global_cap_clipped_neurons", ctypes.c_uint32), ("population_inhibition", ctypes.c_float),
        ("context_cells", ctypes.c_uint32), ("context_probes", ctypes.c_uint32),
        ("context_applied", ctypes.c_uint32), ("eligible_recurrent_synapses", ctypes.c_uint32),
        ("eligible_input_synapses", ctypes.c_uint32), ("target_probability", ctypes.c_float),
        ("error_code", ctypes.c_uint32),
    ]


class LeoBatchReport(ctypes.Structure):
    _fields_ = [
        ("mean_loss", ctypes.c_double), ("targets", ctypes.c_uint64), ("stories", ctypes.c_uint64),
        ("replay_segments", ctypes.c_uint64), ("replay_steps", ctypes.c_uint64),
        ("replay_prefix_steps", ctypes.c_uint64), ("merge_workers", ctypes.c_uint64),
        ("merge_fixed_parameter_updates", ctypes.c_uint64), ("merge_context_keys", ctypes.c_uint64),
        ("activity_steps", ctypes.c_uint64), ("active_neurons_sum", ctypes.c_uint64),
        ("emitted_events", ctypes.c_uint64), ("story_seconds", ctypes.c_double),
        ("merge_seconds", ctypes.c_double), ("replay_seconds", ctypes.c_double),
    ]


class LeoEvaluationReport(ctypes.Structure):
    _fields_ = [
        ("loss", ctypes.c_double), ("bits_per_byte", ctypes.c_double), ("accuracy", ctypes.c_double),
        ("targets", ctypes.c_uint64), ("processed_stories", ctypes.c_uint64), ("processed_bytes", ctypes.c_uint64),
        ("neuron_count", ctypes.c_uint64), ("steps", ctypes.c_uint64), ("active_neurons_sum", ctypes.c_uint64),
        ("active_neurons_peak", ctypes.c_uint64), ("emitted_events", ctypes.c_uint64),
        ("suprathreshold_sum", ctypes.c_uint64), ("block_selected_sum", ctypes.c_uint64),
        ("cap_clipped_sum", ctypes.c_uint64), ("cap_hit_steps", ctypes.c_uint64),
        ("population_inhibition_sum", ctypes.c_double), ("population_inhibition_peak", ctypes.c_float),
        ("pad0", ctypes.c_uint32), ("eligibility_sum", ctypes.c_double), ("eligibility_count", ctypes.c_uint64),
        ("context_cells_sum", ctypes.c_uint64), ("context_probes_sum", ctypes.c_uint64),
        ("context_applied_steps", ctypes.c_uint64), ("context_loss_gain_sum", ctypes.c_double),
        ("output_madds_sum", ctypes.c_uint64),
    ]


class LeoKernelStats(ctypes.Structure):
    _fields_ = [
        ("launches", ctypes.c_uint64), ("lane_steps", ctypes.c_uint64), ("kernel_ms", ctypes.c_double),
        ("algorithmic_bytes", ctypes.c_double), ("events", ctypes.c_uint64), ("touched", ctypes.c_uint64),
        ("active", ctypes.c_uint64), ("scanned_rec", ctypes.c_uint64), ("scanned_in", ctypes.c_uint64),
        ("kept_rec", ctypes.c_uint64), ("kept_in", ctypes.c_uint64), ("destinations", ctypes.c_uint64),
        ("active_inhibitory", ctypes.c_uint64), ("merge_launches", ctypes.c_uint64), ("merge_ms", ctypes.c_double),
        ("phase_work_us", ctypes.c_double * 8), ("phase_wait_us", ctypes.c_double * 8),
        ("resident_lanes", ctypes.c_uint64),
        ("section_launches", ctypes.c_uint64 * 2), ("section_lane_steps", ctypes.c_uint64 * 2),
        ("section_kernel_ms", ctypes.c_double * 2), ("section_bytes", ctypes.c_double * 2),
        ("merge_lane_changes", ctypes.c_uint64), ("merge_elements", ctypes.c_uint64),
        ("merge_bytes", ctypes.c_double), ("learning_slots", ctypes.c_uint64),
        ("deep_register_folds", ctypes.c_uint64), ("deep_radix_folds", ctypes.c_uint64),
    ]


class LeoPackedUpdate(ctypes.Structure):
    _fields_ = [
        ("threshold_indices", _P), ("threshold_values", _P), ("threshold_count", ctypes.c_uint64),
        ("recurrent_indices", _P), ("recurrent_values", _P), ("recurrent_count", ctypes.c_uint64),
        ("input_indices", _P), ("input_values", _P), ("input_count", ctypes.c_uint64),
        ("output_neurons", _P), ("output_values_by_neuron", _P), ("output_count", ctypes.c_uint64),
        ("context_slots", _P), ("context_keys", _P), ("context_observations", _P), ("context_embeddings", _P),
        ("context_count", ctypes.c_uint64),
        ("output_bias", _P), ("context_output_weights", _P),
        ("generation", ctypes.c_uint64), ("parameter_revision", ctypes.c_uint64),
        ("statistics", LeoStatistics),
    ]


# Every symbol include/leo_hip.h declares, with its ctypes signature.
_I32, _U32, _U64, _F32, _F64, _SZ = ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_double, ctypes.c_size_t
SIGNATURES = {
    "leo_hip_last_error": (_I32, [ctypes.c_char_p, _SZ]),
    "leo_hip_abi_version": (_I32, []),
    "leo_splitmix64": (_I32, [_U64, _P, _U64]),
    "leo_model_initialize": (_I32, [_P, _P]),
    "leo_model_initialize_synthetic": (_I32, [_P, _U32, _F32, _U32, _F32, _P]),
    "leo_model_validate": (_I32, [_P, _P]),
    "leo_synthetic_stories": (_I32, [_U64, _U32, _F64, _F64, _U32, _U32, _P, _U64, _P]),
    "leo_hip_create": (_I32, [_P, _P, _I32, _U32, _P]),
    "leo_hip_destroy": (None, [_P]),
    "leo_hip_begin_document": (_I32, [_P]),
    "leo_hip_finish_document": (_I32, [_P]),
    "leo_hip_reset_transient_state": (_I32, [_P]),
    "leo_hip_enable_parameter_tracking": (_I32, [_P]),
    "leo_hip_step": (_I32, [_P, _U32, _I32, _I32, _P]),
    "leo_hip_training_step_batch": (_I32, [_P, _P, _P, _U32, _I32, _P]),
    "leo_hip_advance_frozen_batch": (_I32, [_P, _P, _U32]),
    "leo_hip_replay_streaming_batch": (_I32, [_P, _P, _P, _U32, _I32, _P, _P]),
    "leo_hip_training_story_batch": (_I32, [_P, _P, _P, _U32, _I32, _P, _P]),
    "leo_hip_train_batch": (_I32, [_P, _P, _P, _U32, _I32, _U32, _P, _P]),
    "leo_hip_evaluate": (_I32, [_P, _P, _P, _U32, _P, _P]),
    "leo_hip_download_model": (_I32, [_P, _P]),
    "leo_hip_upload_model": (_I32, [_P, _P]),
    "leo_hip_synchronize_model": (_I32, [_P, _P]),
    "leo_hip_synchronize_packed_model": (_I32, [_P, _P]),
    "leo_hip_commit_packed_host_model": (_I32, [_P, _P]),
    "leo_hip_commit_packed_host_model_no_alloc": (_I32, [_P, _P]),
    "leo_hip_parameter_changes": (_I32, [_P, _I32, _P, _U64, _P, _P, _P]),
    "leo_hip_probabilities": (_I32, [_P, _P]),
    "leo_hip_read_list": (_I32, [_P, _I32, _P, _U64, _P]),
    "leo_hip_read_active": (_I32, [_P, _P, _P, _U64, _P]),
    "leo_hip_read_state": (_I32, [_P, _I32, _P, _U64]),
    "leo_hip_current_tick": (_U64, [_P]),
    "leo_hip_kernel_stats": (_I32, [_P, _P, _I32]),
}

_lib: Optional[ctypes.CDLL] = None


def load(path: Optional[pathlib.Path] = None) -> ctypes.CDLL:
    """Load libleo_hip.so (raises when it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = pathlib.Path(path) if path else LIB_PATH
    if not target.exists():
        raise RuntimeError(f"{target} is missing: build it with `python -m leo_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in {**SIGNATURES, **FORMAT_SIGNATURES}.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.leo_hip_abi_version() != 1:
        raise RuntimeError("libleo_hip.so ABI version mismatch")
    if path is None:
        _lib = lib
    return lib



# Every symbol include/leo_formats.h declares (the host artifact layer).
class LeoDigest(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint8 * 32)]


class LeoCheckpointInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "generation", "parameter_revision", "config_offset", "config_length", "neuron_count",
        "synapses_per_neuron", "input_fanout", "context_slots", "context_embedding_dim")]


class LeoStoryIndex(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint64), ("length", ctypes.c_uint32), ("split_flags", ctypes.c_uint32)]


class LeoDatasetIdentity(ctypes.Structure):
    _fields_ = [("schema_version", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("record_count", ctypes.c_uint64), ("bytes_length", ctypes.c_uint64),
                ("bytes_digest", LeoDigest), ("records_digest", LeoDigest),
                ("provenance_digest", LeoDigest), ("dataset_id", LeoDigest)]


FORMAT_SIGNATURES = {
    "leo_sha256": (_I32, [_P, _U64, _P]),
    "leo_sha256_file": (_I32, [ctypes.c_char_p, _P]),
    "leo_checkpoint_encoded_size": (_I32, [_P, _U64, _P]),
    "leo_checkpoint_encode": (_I32, [_P, _P, _P, _U64, _P, _U64]),
    "leo_checkpoint_inspect": (_I32, [_P, _U64, _P]),
    "leo_checkpoint_decode": (_I32, [_P, _U64, _P, _P]),
    "leo_checkpoint_save_atomic": (_I32, [ctypes.c_char_p, _P, _P, _P, _U64, _U32]),
    "leo_checkpoint_read_generation": (_I32, [ctypes.c_char_p, _P]),
    "leo_checkpoint_prune_generations": (_I32, [ctypes.c_char_p, _U64]),
    "leo_dataset_compute_id": (_I32, [_U32, _U64, _U64, _P, _P, _P, _P]),
    "leo_dataset_write_index": (_I32, [ctypes.c_char_p, ctypes.c_char_p, _P, _U64, _P, _P]),
    "leo_dataset_open": (_I32, [ctypes.c_char_p, ctypes.c_char_p, _P]),
    "leo_dataset_close": (None, [_P]),
    "leo_dataset_identity": (_I32, [_P, _P]),
    "leo_dataset_len": (_U64, [_P]),
    "leo_dataset_entry": (_I32, [_P, _U64, _P]),
    "leo_dataset_story": (_I32, [_P, _U64, _P, _U64, _P]),
    "leo_dataset_pack": (_I32, [_P, _U64, _U64, _P, _U64, _P]),
}


def last_error(lib: ctypes.CDLL) -> str:
    buf = ctypes.create_string_buffer(4096)
    lib.leo_hip_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(lib: ctypes.CDLL, status: int) -> None:
    if status != OK:
        raise LeoError(status, last_error(lib))
