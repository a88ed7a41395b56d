"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (oracle/liboracle.so).

The oracle restates Leo's CPU reference executor (see leo_oracle.h for the
reference files it follows). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

FROZEN, PROVISIONAL, TRAINING, VERIFIED = 0, 1, 2, 3
ERR_INTERNAL, ERR_NUMERICAL, ERR_ARGUMENT = 1, 2, 3  # ORACLE_ERR_* (leo_oracle.h)
F_NAMES = ["membrane", "activation", "fatigue", "branches", "adapt0", "adapt1", "adapt2", "surrogate",
           "rec_bs", "rec_ms", "rec_fs", "rec_as0", "rec_as1", "rec_as2", "rec_e",
           "in_bs", "in_ms", "in_fs", "in_as0", "in_as1", "in_as2", "in_e",
           "logits", "probabilities", "errors", "learning_signal", "block_cutoff", "context_latent"]
U_NAMES = ["refractory", "neuron_last_tick", "rec_last_tick", "in_last_tick"]
L_NAMES = ["active", "touched", "eligible_rec", "eligible_in", "learning_destinations", "changed_threshold",
           "changed_rec", "changed_in", "changed_output", "changed_context", "active_context_slots"]


class OracleConfig(ctypes.Structure):
    _fields_ = [
        ("seed", ctypes.c_uint64), ("refractory_ticks", ctypes.c_uint64),
        ("neuron_count", ctypes.c_uint32), ("block_count", ctypes.c_uint32), ("neurons_per_block", ctypes.c_uint32),
        ("branches_per_neuron", ctypes.c_uint32), ("synapses_per_neuron", ctypes.c_uint32),
        ("input_fanout", ctypes.c_uint32), ("max_active_per_block", ctypes.c_uint32),
        ("max_active_global", ctypes.c_uint32), ("excitatory_fraction", ctypes.c_float),
        ("branch_decay", ctypes.c_float), ("membrane_decay", ctypes.c_float), ("fatigue_decay", ctypes.c_float),
        ("fatigue_gain", ctypes.c_float), ("target_activity", ctypes.c_float),
        ("threshold_homeostasis_rate", ctypes.c_float), ("population_inhibition_rate", ctypes.c_float),
        ("population_inhibition_max", ctypes.c_float), ("adaptation_decay", ctypes.c_float * 3),
        ("adaptation_gain", ctypes.c_float * 3), ("membrane_reset_fraction", ctypes.c_float),
        ("output_learning_rate", ctypes.c_float), ("recurrent_learning_rate", ctypes.c_float),
        ("inhibitory_learning_rate", ctypes.c_float), ("eligibility_decay", ctypes.c_float),
        ("eligibility_epsilon", ctypes.c_float), ("surrogate_width", ctypes.c_float),
        ("surrogate_gain", ctypes.c_float), ("max_update", ctypes.c_float), ("weight_min", ctypes.c_float),
        ("weight_max", ctypes.c_float), ("provisional_strength", ctypes.c_float),
        ("training_strength", ctypes.c_float), ("verified_strength", ctypes.c_float),
        ("end_document_weight", ctypes.c_float), ("plasticity_window", ctypes.c_uint32),
        ("context_max_order", ctypes.c_uint32), ("context_embedding_dim", ctypes.c_uint32),
        ("context_slots_per_order", ctypes.c_uint32), ("context_probe_limit", ctypes.c_uint32),
        ("context_confidence_observations", ctypes.c_uint32), ("context_learning_rate", ctypes.c_float),
        ("context_dropout_rate", ctypes.c_float), ("replay_fraction", ctypes.c_float),
        ("replay_segment_bytes", ctypes.c_uint32), ("replay_stateful_batch", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class OracleStatistics(ctypes.Structure):
    _fields_ = [(n, t) for n, t in [
        ("processed_bytes", ctypes.c_uint64), ("processed_stories", ctypes.c_uint64),
        ("training_loss_sum", ctypes.c_double), ("training_targets", ctypes.c_uint64),
        ("active_neurons_sum", ctypes.c_uint64), ("active_neurons_peak", ctypes.c_uint64),
        ("synaptic_events", ctypes.c_uint64), ("numerical_rejections", ctypes.c_uint64),
        ("persistent_ticks", ctypes.c_uint64)]]


_P = ctypes.c_void_p
ARRAYS = ("threshold", "excitability", "neuron_type", "rec_target", "rec_branch", "rec_delay", "rec_weight",
          "in_target", "in_branch", "in_weight", "out_weight", "bias", "ctx_keys", "ctx_emb", "ctx_obs", "ctx_out")


class OracleModelView(ctypes.Structure):
    _fields_ = [(n, _P) for n in ARRAYS] + [
        ("generation", ctypes.c_uint64), ("parameter_revision", ctypes.c_uint64), ("statistics", OracleStatistics)]


class OracleStepMetrics(ctypes.Structure):
    _fields_ = [
        ("loss", ctypes.c_float), ("has_loss", ctypes.c_uint32), ("predicted_symbol", ctypes.c_uint32),
        ("active_neurons", ctypes.c_uint32), ("emitted_events", ctypes.c_uint32),
        ("suprathreshold_neurons", ctypes.c_uint32), ("block_selected_neurons", ctypes.c_uint32),
        ("global_cap_clipped_neurons", ctypes.c_uint32), ("population_inhibition", ctypes.c_float),
        ("context_cells", ctypes.c_uint32), ("context_probes", ctypes.c_uint32), ("context_applied", ctypes.c_uint32),
        ("context_loss_gain", ctypes.c_float), ("output_madds", ctypes.c_uint32),
        ("eligible_recurrent_synapses", ctypes.c_uint32), ("eligible_input_synapses", ctypes.c_uint32),
        ("mean_abs_eligibility", ctypes.c_float), ("target_probability", ctypes.c_float),
    ]


class OracleBatchReport(ctypes.Structure):
    _fields_ = [("mean_loss", ctypes.c_double)] + [(n, ctypes.c_uint64) for n in (
        "targets", "stories", "replay_segments", "replay_steps", "replay_prefix_steps", "merge_workers",
        "merge_fixed_parameter_updates", "merge_context_keys", "activity_steps", "active_neurons_sum",
        "emitted_events")]


class OracleError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


_lib: Optional[ctypes.CDLL] = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "oracle_last_error": (ctypes.c_int32, [ctypes.c_char_p, ctypes.c_size_t]),
        "oracle_runtime_new": (ctypes.c_int32, [_P, _P, _P]),
        "oracle_runtime_free": (None, [_P]),
        "oracle_runtime_read_model": (ctypes.c_int32, [_P, _P]),
        "oracle_runtime_write_model": (ctypes.c_int32, [_P, _P]),
        "oracle_begin_document": (ctypes.c_int32, [_P]),
        "oracle_finish_document": (ctypes.c_int32, [_P]),
        "oracle_reset_transient_state": (ctypes.c_int32, [_P]),
        "oracle_enable_parameter_tracking": (ctypes.c_int32, [_P]),
        "oracle_restart_parameter_tracking": (ctypes.c_int32, [_P]),
        "oracle_changes_flags": (ctypes.c_int32, [_P, _P, _P]),
        "oracle_step": (ctypes.c_int32, [_P, ctypes.c_uint32, ctypes.c_int32, ctypes.c_int32, _P]),
        "oracle_current_tick": (ctypes.c_uint64, [_P]),
        "oracle_population_inhibition": (ctypes.c_float, [_P]),
        "oracle_read_list": (ctypes.c_int64, [_P, ctypes.c_int32, _P, ctypes.c_size_t]),
        "oracle_read_f32": (ctypes.c_int32, [_P, ctypes.c_int32, _P, ctypes.c_size_t]),
        "oracle_read_u64": (ctypes.c_int32, [_P, ctypes.c_int32, _P, ctypes.c_size_t]),
        "oracle_train_story_batch": (ctypes.c_int32, [_P, _P, _P, ctypes.c_uint32, ctypes.c_int32,
                                                      ctypes.c_uint32, _P, _P]),
        "oracle_train_document_pass": (ctypes.c_int32, [_P, _P, ctypes.c_uint64, ctypes.c_int32, _P]),
        "oracle_execute_replay_ranges": (ctypes.c_int32, [_P, _P, ctypes.c_uint64, _P, ctypes.c_uint32,
                                                          ctypes.c_int32, _P, _P]),
        "oracle_select_replay_ranges": (ctypes.c_int64, [_P, ctypes.c_uint64, ctypes.c_float, ctypes.c_uint64,
                                                         _P, ctypes.c_size_t]),
        "oracle_delta_between": (ctypes.c_int32, [_P, _P, _P, _P]),
        "oracle_delta_between_tracked": (ctypes.c_int32, [_P, _P, _P]),
        "oracle_delta_free": (None, [_P]),
        "oracle_delta_count": (ctypes.c_int64, [_P, ctypes.c_int32]),
        "oracle_delta_equal": (ctypes.c_int32, [_P, _P]),
        "oracle_apply_deltas": (ctypes.c_int32, [_P, _P, ctypes.c_uint32, ctypes.c_int32, _P, _P]),
        "oracle_analog_rank_surrogate": (ctypes.c_float, [ctypes.c_float, ctypes.c_float, ctypes.c_int32,
                                                          ctypes.c_float, ctypes.c_float]),
        "oracle_branch_jacobian": (ctypes.c_float, [ctypes.c_uint8, ctypes.c_float, ctypes.c_float, ctypes.c_float]),
        "oracle_bounded_delta": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
        "oracle_inhibitory_homeostasis_delta": (ctypes.c_float, [ctypes.c_float] * 6),
        "oracle_context_survives_dropout": (ctypes.c_int32, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                                             ctypes.c_float]),
        "oracle_context_key": (ctypes.c_uint64, [_P, ctypes.c_size_t, ctypes.c_size_t]),
        "oracle_decay_for_elapsed": (ctypes.c_float, [ctypes.c_float, ctypes.c_uint64]),
        "oracle_resolve_context_slot": (ctypes.c_int32, [_P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32,
                                                         _P, _P]),
        "oracle_test_update_context_projection": (ctypes.c_int32, [_P, _P, _P, ctypes.c_uint32, _P, ctypes.c_float]),
        "oracle_plasticity_step": (ctypes.c_int32, [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, _P, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        lib = load()
        buf = ctypes.create_string_buffer(4096)
        lib.oracle_last_error(buf, len(buf))
        raise OracleError(status, buf.value.decode(errors="replace"))


def oracle_config(config) -> OracleConfig:
    """OracleConfig from a leo_amd.Config."""
    m, d, l, c, r = config.model, config.dynamics, config.learning, config.context, config.replay
    o = OracleConfig()
    o.seed = m.seed
    o.refractory_ticks = d.refractory_ticks
    for name in ("neuron_count", "block_count", "neurons_per_block", "branches_per_neuron", "synapses_per_neuron",
                 "input_fanout", "max_active_per_block", "max_active_global", "excitatory_fraction"):
        setattr(o, name, getattr(m, name))
    for name in ("branch_decay", "membrane_decay", "fatigue_decay", "fatigue_gain", "target_activity",
                 "threshold_homeostasis_rate", "population_inhibition_rate", "population_inhibition_max",
                 "membrane_reset_fraction"):
        setattr(o, name, getattr(d, name))
    o.adaptation_decay[:] = [d.adaptation_fast_decay, d.adaptation_medium_decay, d.adaptation_slow_decay]
    o.adaptation_gain[:] = [d.adaptation_fast_gain, d.adaptation_medium_gain, d.adaptation_slow_gain]
    for name in ("output_learning_rate", "recurrent_learning_rate", "inhibitory_learning_rate", "eligibility_decay",
                 "eligibility_epsilon", "surrogate_width", "surrogate_gain", "max_update", "weight_min",
                 "weight_max", "provisional_strength", "training_strength", "verified_strength",
                 "end_document_weight", "plasticity_window"):
        setattr(o, name, getattr(l, name))
    o.context_max_order = c.max_order
    o.context_embedding_dim = c.embedding_dim
    o.context_slots_per_order = c.slots_per_order
    o.context_probe_limit = c.probe_limit
    o.context_confidence_observations = c.confidence_observations
    o.context_learning_rate = c.learning_rate
    o.context_dropout_rate = c.dropout_rate
    o.replay_fraction = r.fraction
    o.replay_segment_bytes = r.segment_bytes
    o.replay_stateful_batch = 1 if r.stateful_batch else 0
    return o


def model_view(model) -> OracleModelView:
    """View of a leo_amd.Model (host layouts are identical)."""
    v = OracleModelView()
    for name in ARRAYS:
        arr = getattr(model, name)
        assert arr.flags.c_contiguous
        setattr(v, name, arr.ctypes.data)
    v.generation = model.generation
    v.parameter_revision = model.parameter_revision
    for k, _ in OracleStatistics._fields_:
        setattr(v.statistics, k, model.statistics[k])
    return v


def absorb(model, v: OracleModelView) -> None:
    model.generation = int(v.generation)
    model.parameter_revision = int(v.parameter_revision)
    model.statistics = {k: getattr(v.statistics, k) for k, _ in OracleStatistics._fields_}


class OracleRuntime:
    """Runtime (runtime.rs:118-190) restated in C++; owns a copy of the model."""

    def __init__(self, model):
        self.lib = load()
        self.config = model.config
        self._template = model
        self.handle = ctypes.c_void_p()
        self._cfg = oracle_config(model.config)
        view = model_view(model)
        _check(self.lib.oracle_runtime_new(ctypes.byref(self._cfg), ctypes.byref(view), ctypes.byref(self.handle)))

    def __del__(self):
        try:
            if self.handle:
                self.lib.oracle_runtime_free(self.handle)
        except Exception:
            pass

    def model(self):
        out = self._template.copy()
        view = model_view(out)
        _check(self.lib.oracle_runtime_read_model(self.handle, ctypes.byref(view)))
        absorb(out, view)
        return out

    def set_model(self, model) -> None:
        view = model_view(model)
        _check(self.lib.oracle_runtime_write_model(self.handle, ctypes.byref(view)))

    def begin_document(self):
        _check(self.lib.oracle_begin_document(self.handle))

    def finish_document(self):
        _check(self.lib.oracle_finish_document(self.handle))

    def reset_transient_state(self):
        _check(self.lib.oracle_reset_transient_state(self.handle))

    def enable_parameter_tracking(self):
        _check(self.lib.oracle_enable_parameter_tracking(self.handle))

    def restart_parameter_tracking(self):
        """The GPU adapter's enable_parameter_tracking: fresh change sets on every call."""
        _check(self.lib.oracle_restart_parameter_tracking(self.handle))

    def step(self, symbol: int, target: Optional[int], permission: int) -> OracleStepMetrics:
        m = OracleStepMetrics()
        _check(self.lib.oracle_step(self.handle, symbol, -1 if target is None else target, permission,
                                    ctypes.byref(m)))
        return m

    @property
    def current_tick(self) -> int:
        return int(self.lib.oracle_current_tick(self.handle))

    @property
    def population_inhibition(self) -> float:
        return float(self.lib.oracle_population_inhibition(self.handle))

    def read_list(self, name: str) -> np.ndarray:
        which = L_NAMES.index(name)
        n = self.lib.oracle_read_list(self.handle, which, None, 0)
        buf = np.zeros(max(n, 1), dtype=np.uint64)
        self.lib.oracle_read_list(self.handle, which, buf.ctypes.data, buf.size)
        return buf[:n].astype(np.int64)

    def read_f32(self, name: str) -> np.ndarray:
        n = self.config.model.neuron_count
        sizes = {"branches": 4 * n, "logits": 257, "probabilities": 257, "errors": 257,
                 "block_cutoff": self.config.model.block_count, "context_latent": self.config.context.embedding_dim}
        if name.startswith("rec_"):
            size = self.config.synapse_count
        elif name.startswith("in_"):
            size = self.config.input_count
        else:
            size = sizes.get(name, n)
        out = np.zeros(size, dtype=np.float32)
        _check(self.lib.oracle_read_f32(self.handle, F_NAMES.index(name), out.ctypes.data, size))
        return out

    def read_u64(self, name: str) -> np.ndarray:
        size = {"refractory": self.config.model.neuron_count, "neuron_last_tick": self.config.model.neuron_count,
                "rec_last_tick": self.config.synapse_count, "in_last_tick": self.config.input_count}[name]
        out = np.zeros(size, dtype=np.uint64)
        _check(self.lib.oracle_read_u64(self.handle, U_NAMES.index(name), out.ctypes.data, size))
        return out

    def changes(self) -> Dict[str, object]:
        out: Dict[str, object] = {
            "threshold": self.read_list("changed_threshold"), "recurrent_weight": self.read_list("changed_rec"),
            "input_weight": self.read_list("changed_in"), "output_neurons": self.read_list("changed_output"),
            "context_slots": self.read_list("changed_context")}
        b, c = ctypes.c_uint32(), ctypes.c_uint32()
        self.lib.oracle_changes_flags(self.handle, ctypes.byref(b), ctypes.byref(c))
        out["output_bias_dirty"] = bool(b.value)
        out["context_output_dirty"] = bool(c.value)
        return out

    def train_story_batch(self, stories: Sequence[bytes], permission: int = TRAINING, replay: bool = True
                          ) -> Tuple[OracleBatchReport, List[np.ndarray]]:
        offsets = np.zeros(len(stories) + 1, dtype=np.uint64)
        for i, s in enumerate(stories):
            offsets[i + 1] = offsets[i] + len(s)
        data = np.frombuffer(b"".join(stories) or b"\0", dtype=np.uint8).copy()
        losses = np.zeros(int(offsets[-1]) + len(stories), dtype=np.float32)
        rep = OracleBatchReport()
        _check(self.lib.oracle_train_story_batch(self.handle, data.ctypes.data, offsets.ctypes.data, len(stories),
                                                 permission, 1 if replay else 0, losses.ctypes.data,
                                                 ctypes.byref(rep)))
        out, cursor = [], 0
        for s in stories:
            n = len(s) + 1 if len(s) else 0
            out.append(losses[cursor:cursor + n].copy())
            cursor += n
        return rep, out

    def train_document_pass(self, story: bytes, permission: int = TRAINING) -> np.ndarray:
        data = np.frombuffer(story, dtype=np.uint8).copy()
        losses = np.zeros(len(story) + 1, dtype=np.float32)
        _check(self.lib.oracle_train_document_pass(self.handle, data.ctypes.data, len(story), permission,
                                                   losses.ctypes.data))
        return losses

    def execute_replay_ranges(self, story: bytes, ranges: Sequence[Tuple[int, int]], permission: int = TRAINING
                              ) -> Tuple[int, int]:
        data = np.frombuffer(story, dtype=np.uint8).copy()
        r = np.array([x for pair in ranges for x in pair] or [0], dtype=np.uint64)
        rs, ps = ctypes.c_uint64(), ctypes.c_uint64()
        _check(self.lib.oracle_execute_replay_ranges(self.handle, data.ctypes.data, len(story), r.ctypes.data,
                                                     len(ranges), permission, ctypes.byref(rs), ctypes.byref(ps)))
        return int(rs.value), int(ps.value)

    def resolve_context_slot(self, order: int, key: int, allocate: bool) -> Tuple[Optional[int], int]:
        slot, probes = ctypes.c_int64(), ctypes.c_uint64()
        _check(self.lib.oracle_resolve_context_slot(self.handle, order, key, 1 if allocate else 0,
                                                    ctypes.byref(slot), ctypes.byref(probes)))
        return (None if slot.value < 0 else int(slot.value)), int(probes.value)

    def test_update_context_projection(self, slots, scales, errors, strength: float) -> None:
        s = np.asarray(slots, dtype=np.uint64)
        sc = np.asarray(scales, dtype=np.float32)
        e = np.asarray(errors, dtype=np.float32)
        _check(self.lib.oracle_test_update_context_projection(self.handle, s.ctypes.data, sc.ctypes.data, len(s),
                                                              e.ctypes.data, strength))


class Delta:
    """SparseModelDelta handle (parallel.rs:41-55)."""

    def __init__(self, handle):
        self.lib = load()
        self.handle = handle

    def __del__(self):
        try:
            self.lib.oracle_delta_free(self.handle)
        except Exception:
            pass

    @classmethod
    def between(cls, base, trained) -> "Delta":
        lib = load()
        h = ctypes.c_void_p()
        cfg = oracle_config(base.config)
        vb, vt = model_view(base), model_view(trained)
        _check(lib.oracle_delta_between(ctypes.byref(cfg), ctypes.byref(vb), ctypes.byref(vt), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def between_tracked(cls, base, runtime: OracleRuntime) -> "Delta":
        lib = load()
        h = ctypes.c_void_p()
        vb = model_view(base)
        _check(lib.oracle_delta_between_tracked(ctypes.byref(vb), runtime.handle, ctypes.byref(h)))
        return cls(h)

    def count(self, which: str) -> int:
        idx = ["threshold", "recurrent_weight", "input_weight", "output_weight", "output_bias",
               "context_output_weight", "context", "revision_increment"].index(which)
        return int(self.lib.oracle_delta_count(self.handle, idx))

    def __eq__(self, other) -> bool:
        return bool(self.lib.oracle_delta_equal(self.handle, other.handle))


def apply_deltas(master: OracleRuntime, deltas: Sequence[Delta], mean: bool = True) -> Tuple[int, int]:
    """apply_mean_deltas / apply_sum_deltas (parallel.rs:694-713) into the master runtime's model."""
    lib = load()
    arr = (ctypes.c_void_p * len(deltas))(*[d.handle for d in deltas])
    fixed, ctx = ctypes.c_uint64(), ctypes.c_uint64()
    _check(lib.oracle_apply_deltas(master.handle, arr, len(deltas), 0 if mean else 1, ctypes.byref(fixed),
                                   ctypes.byref(ctx)))
    return int(fixed.value), int(ctx.value)


def select_replay_ranges(losses: Sequence[float], fraction: float, segment: int) -> List[Tuple[int, int]]:
    lib = load()
    arr = np.asarray(losses, dtype=np.float32)
    out = np.zeros(2 * max(len(arr), 1), dtype=np.uint64)
    n = lib.oracle_select_replay_ranges(arr.ctypes.data, len(arr), fraction, segment, out.ctypes.data, len(arr))
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]


def context_key(history: Sequence[int], order: int) -> int:
    lib = load()
    h = np.asarray(history, dtype=np.uint32)
    return int(lib.oracle_context_key(h.ctypes.data, len(h), order))
