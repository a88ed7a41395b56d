"""HipRuntime: the RuntimeBackend of crates/leo-core/src/backend.rs:351-475 on MI355X.

Method names and argument meaning follow the reference trait; every call goes
through the C-ABI (include/leo_hip.h) into libleo_hip.so. There is no CPU
fallback: without a gfx950 device, construction raises ``LeoError`` with
``code == native.ERR_DEVICE`` (docs/ADR-0001-EXECUTION-BACKENDS.md:9).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import native
from .config import Config
from .model import Model, host_config


@dataclass
class StepMetrics:
    """StepMetrics (metrics.rs:39-66), the fields the device path produces."""

    loss: Optional[float]
    predicted_symbol: int
    active_neurons: int
    emitted_events: int
    suprathreshold_neurons: int
    block_selected_neurons: int
    global_cap_clipped_neurons: int
    population_inhibition: float
    context_cells: int
    context_probes: int
    context_applied: bool
    eligible_recurrent_synapses: int
    eligible_input_synapses: int
    target_probability: Optional[float]

    @classmethod
    def from_c(cls, m: native.LeoStepMetrics) -> "StepMetrics":
        return cls(
            loss=float(m.loss) if m.has_loss else None,
            predicted_symbol=int(m.predicted_symbol), active_neurons=int(m.active_neurons),
            emitted_events=int(m.emitted_events), suprathreshold_neurons=int(m.suprathreshold_neurons),
            block_selected_neurons=int(m.block_selected_neurons),
            global_cap_clipped_neurons=int(m.global_cap_clipped_neurons),
            population_inhibition=float(m.population_inhibition), context_cells=int(m.context_cells),
            context_probes=int(m.context_probes), context_applied=bool(m.context_applied),
            eligible_recurrent_synapses=int(m.eligible_recurrent_synapses),
            eligible_input_synapses=int(m.eligible_input_synapses),
            target_probability=float(m.target_probability) if m.has_loss else None,
        )


@dataclass
class BatchReport:
    """BatchTrainingReport (training.rs) + MergeMetrics (parallel.rs:305-310)."""

    mean_loss: float
    targets: int
    stories: int
    replay_segments: int
    replay_steps: int
    replay_prefix_steps: int
    merge_workers: int
    merge_fixed_parameter_updates: int
    merge_context_keys: int
    activity_steps: int
    active_neurons_sum: int
    emitted_events: int
    story_seconds: float
    merge_seconds: float
    replay_seconds: float

    @classmethod
    def from_c(cls, r: native.LeoBatchReport) -> "BatchReport":
        return cls(**{name: getattr(r, name) for name, _ in native.LeoBatchReport._fields_})


class PackedUpdate:
    """PackedSparseModelUpdate (crates/leo-core/src/parallel.rs:79-183): the
    canonical values of a change set, packed once per logical batch."""

    def __init__(self, model: Model, changes: Dict[str, object]):
        n = model.neuron_count
        dim = model.config.context.embedding_dim
        self.threshold_indices = np.asarray(changes["threshold"], dtype=np.uint32)
        self.threshold_values = model.threshold[self.threshold_indices].astype(np.float32)
        self.recurrent_indices = np.asarray(changes["recurrent_weight"], dtype=np.uint32)
        self.recurrent_values = model.rec_weight[self.recurrent_indices].astype(np.float32)
        self.input_indices = np.asarray(changes["input_weight"], dtype=np.uint32)
        self.input_values = model.in_weight[self.input_indices].astype(np.float32)
        self.output_neurons = np.asarray(changes["output_neurons"], dtype=np.uint32)
        # one contiguous row of the 257 outputs per changed neuron
        out = model.out_weight.reshape(257, n)
        self.output_values_by_neuron = np.ascontiguousarray(out[:, self.output_neurons].T).reshape(-1)
        self.context_slots = np.asarray(changes["context_slots"], dtype=np.uint32)
        self.context_keys = model.ctx_keys[self.context_slots].astype(np.uint64)
        self.context_observations = model.ctx_obs[self.context_slots].astype(np.uint32)
        emb = model.ctx_emb.reshape(-1, dim)
        self.context_embeddings = np.ascontiguousarray(emb[self.context_slots]).reshape(-1)
        self.output_bias = model.bias.copy() if changes["output_bias_dirty"] else None
        self.context_output_weights = model.ctx_out.copy() if changes["context_output_dirty"] else None
        self.generation = model.generation
        self.parameter_revision = model.parameter_revision
        self.statistics = dict(model.statistics)

    @classmethod
    def from_model(cls, model: Model, changes: Dict[str, object]) -> "PackedUpdate":
        return cls(model, changes)

    def to_c(self) -> native.LeoPackedUpdate:
        u = native.LeoPackedUpdate()
        for name in ("threshold", "recurrent", "input"):
            idx, val = getattr(self, f"{name}_indices"), getattr(self, f"{name}_values")
            setattr(u, f"{name}_indices", idx.ctypes.data)
            setattr(u, f"{name}_values", val.ctypes.data)
            setattr(u, f"{name}_count", idx.size)
        u.output_neurons = self.output_neurons.ctypes.data
        u.output_values_by_neuron = self.output_values_by_neuron.ctypes.data
        u.output_count = self.output_neurons.size
        u.context_slots = self.context_slots.ctypes.data
        u.context_keys = self.context_keys.ctypes.data
        u.context_observations = self.context_observations.ctypes.data
        u.context_embeddings = self.context_embeddings.ctypes.data
        u.context_count = self.context_slots.size
        u.output_bias = self.output_bias.ctypes.data if self.output_bias is not None else None
        u.context_output_weights = (self.context_output_weights.ctypes.data
                                    if self.context_output_weights is not None else None)
        u.generation = self.generation
        u.parameter_revision = self.parameter_revision
        for k, v in self.statistics.items():
            setattr(u.statistics, k, v)
        return u


def pack_stories(stories: Sequence[bytes]) -> Tuple[np.ndarray, np.ndarray]:
    """Concatenate stories into (bytes, offsets[count+1])."""
    offsets = np.zeros(len(stories) + 1, dtype=np.uint64)
    for i, s in enumerate(stories):
        offsets[i + 1] = offsets[i] + len(s)
    data = np.frombuffer(b"".join(bytes(s) for s in stories), dtype=np.uint8).copy()
    if data.size == 0:
        data = np.zeros(1, dtype=np.uint8)
    return data, offsets


class HipRuntime:
    """BackendRuntime::new(model, BackendKind::Gpu) (backend.rs:796-820) on a gfx950 device."""

    def __init__(self, model: Model, device: int = 0, max_lanes: int = 64):
        self._lib = native.load()
        self.config: Config = model.config
        self._hc = host_config(model.config)
        self._handle = ctypes.c_void_p()
        view = model.view()
        native.check(self._lib, self._lib.leo_hip_create(ctypes.byref(self._hc), ctypes.byref(view), device,
                                                          max_lanes, ctypes.byref(self._handle)))
        self._template = model
        self.device = device

    def fork(self, model: Model) -> "HipRuntime":
        """RuntimeBackend::fork (backend.rs:623-633 -> cuda.rs:2347-2356): a
        runtime for `model` on this runtime's device, with the whole model
        uploaded and its transient state reset (one story lane: a fork trains
        one worker story)."""
        return HipRuntime(model, device=self.device, max_lanes=1)

    def close(self) -> None:
        if self._handle:
            self._lib.leo_hip_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __enter__(self) -> "HipRuntime":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def _call(self, name: str, *args) -> None:
        native.check(self._lib, getattr(self._lib, name)(self._handle, *args))

    # --- RuntimeBackend -------------------------------------------------------
    def model(self) -> Model:
        """synchronize_model() + model() (backend.rs:355-356)."""
        out = Model.empty(self.config)
        view = out.view()
        self._call("leo_hip_download_model", ctypes.byref(view))
        out._absorb(view)
        return out

    def set_model(self, model: Model) -> None:
        """model_mut() replacement: upload a whole model (backend.rs:357)."""
        view = model.view()
        self._call("leo_hip_upload_model", ctypes.byref(view))

    def synchronize_model(self, mirror: Model) -> None:
        """synchronize_model() on a host mirror (cuda.rs:2817-2825): only the
        elements changed since the mirror's last synchronisation are copied."""
        view = mirror.view()
        self._call("leo_hip_synchronize_model", ctypes.byref(view))
        mirror._absorb(view)

    def synchronize_packed_model(self, update: PackedUpdate) -> None:
        """backend.rs:374-376 / cuda.rs:2844-2857: scatter; tracking ends."""
        u = update.to_c()
        self._call("leo_hip_synchronize_packed_model", ctypes.byref(u))

    def commit_packed_host_model(self, update: PackedUpdate) -> None:
        """backend.rs:378-387 / cuda.rs:2859-2868: scatter; tracking kept."""
        u = update.to_c()
        self._call("leo_hip_commit_packed_host_model", ctypes.byref(u))

    def begin_document(self) -> None:
        self._call("leo_hip_begin_document")

    def finish_document(self) -> None:
        self._call("leo_hip_finish_document")

    def reset_transient_state(self) -> None:
        self._call("leo_hip_reset_transient_state")

    def enable_parameter_tracking(self) -> None:
        self._call("leo_hip_enable_parameter_tracking")

    def step(self, symbol: int, target: Optional[int], permission: int) -> StepMetrics:
        m = native.LeoStepMetrics()
        self._call("leo_hip_step", symbol, -1 if target is None else target, permission, ctypes.byref(m))
        return StepMetrics.from_c(m)

    def training_step_batch(self, steps: Sequence[Tuple[int, Optional[int]]], permission: int) -> List[StepMetrics]:
        n = len(steps)
        if n == 0:
            return []
        symbols = np.array([s for s, _ in steps], dtype=np.uint32)
        targets = np.array([-1 if t is None else t for _, t in steps], dtype=np.int32)
        out = (native.LeoStepMetrics * n)()
        self._call("leo_hip_training_step_batch", symbols.ctypes.data, targets.ctypes.data, n, permission, out)
        return [StepMetrics.from_c(m) for m in out]

    def advance_frozen_batch(self, steps: Sequence[Tuple[int, Optional[int]]]) -> None:
        symbols = np.array([s for s, _ in steps], dtype=np.uint32)
        if symbols.size:
            self._call("leo_hip_advance_frozen_batch", symbols.ctypes.data, symbols.size)

    def replay_streaming_batch(self, steps: Sequence[Tuple[int, Optional[int]]], permission: int
                               ) -> List[StepMetrics]:
        """backend.rs:439-453: a mixed timeline; metrics for supervised positions only."""
        n = len(steps)
        if n == 0:
            return []
        symbols = np.array([s for s, _ in steps], dtype=np.uint32)
        targets = np.array([-1 if t is None else t for _, t in steps], dtype=np.int32)
        out = (native.LeoStepMetrics * n)()
        supervised = ctypes.c_uint32()
        self._call("leo_hip_replay_streaming_batch", symbols.ctypes.data, targets.ctypes.data, n, permission, out,
                   ctypes.byref(supervised))
        return [StepMetrics.from_c(out[i]) for i in range(supervised.value)]

    def training_story_batch(self, stories: Sequence[bytes], permission: int) -> Tuple[BatchReport, List[np.ndarray]]:
        """backend.rs:457-463: device lanes + the batch-end mean; returns per-story losses."""
        data, offsets = pack_stories(stories)
        losses = np.zeros(int(offsets[-1]) + len(stories), dtype=np.float32)
        rep = native.LeoBatchReport()
        self._call("leo_hip_training_story_batch", data.ctypes.data, offsets.ctypes.data, len(stories), permission,
                   losses.ctypes.data, ctypes.byref(rep))
        return BatchReport.from_c(rep), _split_losses(losses, stories)

    def train_batch(self, stories: Sequence[bytes], permission: int, replay: bool = True
                    ) -> Tuple[BatchReport, List[np.ndarray]]:
        """TrainingEngine::train_batch -> train_story_batch (training.rs:1539-1727)."""
        data, offsets = pack_stories(stories)
        losses = np.zeros(int(offsets[-1]) + len(stories), dtype=np.float32)
        rep = native.LeoBatchReport()
        self._call("leo_hip_train_batch", data.ctypes.data, offsets.ctypes.data, len(stories), permission,
                   1 if replay else 0, losses.ctypes.data, ctypes.byref(rep))
        return BatchReport.from_c(rep), _split_losses(losses, stories)

    def evaluate(self, stories: Sequence[bytes]) -> Tuple[Dict[str, float], List[np.ndarray]]:
        """evaluate_model_shard (crates/leo-cli/src/training/validation.rs:65-135): frozen
        scoring of the stories; returns EvaluationMetrics (+ ActivityDiagnostics) and each
        non-empty story's step losses."""
        data, offsets = pack_stories(stories)
        losses = np.zeros(int(offsets[-1]) + len(stories), dtype=np.float32)
        rep = native.LeoEvaluationReport()
        self._call("leo_hip_evaluate", data.ctypes.data, offsets.ctypes.data, len(stories), losses.ctypes.data,
                   ctypes.byref(rep))
        report = {name: getattr(rep, name) for name, _ in native.LeoEvaluationReport._fields_ if name != "pad0"}
        return report, [l for l in _split_losses(losses, stories) if l.size]

    def train_batch_packed(self, data: np.ndarray, offsets: np.ndarray, permission: int, replay: bool = True
                           ) -> BatchReport:
        """train_batch over pre-packed stories (no per-story loss copy-out)."""
        rep = native.LeoBatchReport()
        self._call("leo_hip_train_batch", data.ctypes.data, offsets.ctypes.data, len(offsets) - 1, permission,
                   1 if replay else 0, None, ctypes.byref(rep))
        return BatchReport.from_c(rep)

    def parameter_changes(self) -> Dict[str, object]:
        """parameter_changes() (backend.rs:359): sorted index sets + dirty flags."""
        out: Dict[str, object] = {}
        names = ["threshold", "recurrent_weight", "input_weight", "output_neurons", "context_slots"]
        bias = ctypes.c_uint32()
        ctx = ctypes.c_uint32()
        for which, name in enumerate(names):
            count = ctypes.c_uint64()
            self._call("leo_hip_parameter_changes", which, None, 0, ctypes.byref(count), None, None)
            buf = np.zeros(max(int(count.value), 1), dtype=np.uint64)
            self._call("leo_hip_parameter_changes", which, buf.ctypes.data, buf.size, ctypes.byref(count),
                       ctypes.byref(bias), ctypes.byref(ctx))
            out[name] = buf[: int(count.value)].astype(np.int64)
        out["output_bias_dirty"] = bool(bias.value)
        out["context_output_dirty"] = bool(ctx.value)
        return out

    def probabilities(self) -> np.ndarray:
        out = np.zeros(257, dtype=np.float32)
        self._call("leo_hip_probabilities", out.ctypes.data)
        return out

    def read_list(self, which: int) -> np.ndarray:
        count = ctypes.c_uint64()
        self._call("leo_hip_read_list", which, None, 0, ctypes.byref(count))
        buf = np.zeros(max(int(count.value), 1), dtype=np.uint64)
        self._call("leo_hip_read_list", which, buf.ctypes.data, buf.size, ctypes.byref(count))
        return buf[: int(count.value)].astype(np.int64)

    def _read_active(self) -> Tuple[np.ndarray, np.ndarray]:
        count = ctypes.c_uint64()
        self._call("leo_hip_read_active", None, None, 0, ctypes.byref(count))
        n = int(count.value)
        ids = np.zeros(max(n, 1), dtype=np.uint64)
        values = np.zeros(max(n, 1), dtype=np.float32)
        self._call("leo_hip_read_active", ids.ctypes.data, values.ctypes.data, ids.size, ctypes.byref(count))
        return ids[:n].astype(np.int64), values[:n]

    def active_neurons(self) -> np.ndarray:
        """RuntimeBackend::active_neurons (backend.rs:389): the last step's
        active neurons in selection order."""
        return self._read_active()[0]

    def activation(self, neuron: int) -> float:
        """RuntimeBackend::activation (backend.rs:390): the neuron's activation
        after the last step (0 unless it is active)."""
        ids, values = self._read_active()
        hit = np.nonzero(ids == neuron)[0]
        return float(values[hit[0]]) if hit.size else 0.0

    def read_state(self, name: str) -> np.ndarray:
        n = self.config.model.neuron_count
        sizes = {"branches": 4 * n, "logits": 257, "probabilities": 257, "errors": 257}
        if name.startswith("rec_"):
            size = self.config.synapse_count
        elif name.startswith("in_"):
            size = self.config.input_count
        else:
            size = sizes.get(name, n)
        out = np.zeros(size, dtype=np.float32)
        self._call("leo_hip_read_state", native.STATE[name], out.ctypes.data, size)
        return out

    def kernel_stats(self, reset: bool = False) -> Dict[str, float]:
        """Device telemetry of the step kernel (HIP-event time, work counters, byte model)."""
        st = native.LeoKernelStats()
        self._call("leo_hip_kernel_stats", ctypes.byref(st), 1 if reset else 0)
        out = {}
        for name, _ in native.LeoKernelStats._fields_:
            v = getattr(st, name)
            out[name] = list(v) if isinstance(v, ctypes.Array) else v
        return out

    @property
    def resident_lanes(self) -> int:
        """Story lanes held on the device at once (larger batches run in groups)."""
        return int(self.kernel_stats()["resident_lanes"])

    @property
    def current_tick(self) -> int:
        return int(self._lib.leo_hip_current_tick(self._handle))


def _split_losses(losses: np.ndarray, stories: Sequence[bytes]) -> List[np.ndarray]:
    out, cursor = [], 0
    for s in stories:
        n = len(s) + 1 if len(s) else 0
        out.append(losses[cursor:cursor + n].copy())
        cursor += n
    return out
