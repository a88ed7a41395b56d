"""Leo's persistent model (crates/leo-core/src/model.rs:19-76) as numpy arrays.

Layouts are the reference's host layouts: recurrent rows are source-major
(slot = src*S + j), output weights are output-major [257][N], the context
output projection is output-major [257][E]. ``Model.initialize`` runs the
reference's seeded SplitMix64 initialisation (model.rs:79-158) in native code.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict

import numpy as np

from . import native
from .config import Config

OUTPUT_CLASSES = 257
SYMBOL_COUNT = 258
BEGIN_DOCUMENT = 256
END_DOCUMENT = 257
BRANCH_EXCITATORY, BRANCH_INHIBITORY, BRANCH_TEMPORAL, BRANCH_CONTEXT_GATE = 0, 1, 2, 3

STAT_FIELDS = ("processed_bytes", "processed_stories", "training_loss_sum", "training_targets",
               "active_neurons_sum", "active_neurons_peak", "synaptic_events", "numerical_rejections",
               "persistent_ticks")

ARRAY_FIELDS = ("threshold", "excitability", "neuron_type", "rec_target", "rec_branch", "rec_delay",
                "rec_weight", "in_target", "in_branch", "in_weight", "out_weight", "bias", "ctx_keys",
                "ctx_emb", "ctx_obs", "ctx_out")

_DTYPES = {
    "threshold": np.float32, "excitability": np.float32, "neuron_type": np.uint8, "rec_target": np.uint32,
    "rec_branch": np.uint8, "rec_delay": np.uint8, "rec_weight": np.float32, "in_target": np.uint32,
    "in_branch": np.uint8, "in_weight": np.float32, "out_weight": np.float32, "bias": np.float32,
    "ctx_keys": np.uint64, "ctx_emb": np.float32, "ctx_obs": np.uint32, "ctx_out": np.float32,
}


def host_config(config: Config) -> native.LeoHostConfig:
    """Fill the C-ABI config (LeoConfig field order of cuda_abi.def, CudaConfig::from_model cuda.rs:276-328)."""
    m, d, l, c, r = config.model, config.dynamics, config.learning, config.context, config.replay
    h = native.LeoHostConfig()
    dev = h.device
    dev.neuron_count = m.neuron_count
    dev.block_count = m.block_count
    dev.neurons_per_block = m.neurons_per_block
    dev.branches_per_neuron = m.branches_per_neuron
    dev.synapses_per_neuron = m.synapses_per_neuron
    dev.input_fanout = m.input_fanout
    dev.max_active_per_block = m.max_active_per_block
    dev.max_active_global = m.max_active_global
    dev.context_max_order = c.max_order
    dev.context_embedding_dim = c.embedding_dim
    dev.context_slots_per_order = c.slots_per_order
    dev.context_probe_limit = c.probe_limit
    dev.context_confidence_observations = c.confidence_observations
    dev.refractory_ticks = d.refractory_ticks
    for name in ("branch_decay", "membrane_decay", "fatigue_decay", "fatigue_gain", "target_activity",
                 "threshold_homeostasis_rate", "population_inhibition_rate", "population_inhibition_max",
                 "adaptation_fast_decay", "adaptation_medium_decay", "adaptation_slow_decay",
                 "adaptation_fast_gain", "adaptation_medium_gain", "adaptation_slow_gain",
                 "membrane_reset_fraction"):
        setattr(dev, name, getattr(d, name))
    for name in ("output_learning_rate", "recurrent_learning_rate", "inhibitory_learning_rate", "eligibility_decay",
                 "eligibility_epsilon", "surrogate_width", "surrogate_gain", "max_update", "weight_min",
                 "weight_max"):
        setattr(dev, name, getattr(l, name))
    dev.context_learning_rate = c.learning_rate
    h.seed = m.seed
    h.excitatory_fraction = m.excitatory_fraction
    h.plasticity_window = l.plasticity_window
    h.end_document_weight = l.end_document_weight
    h.provisional_strength = l.provisional_strength
    h.training_strength = l.training_strength
    h.verified_strength = l.verified_strength
    h.context_dropout_rate = c.dropout_rate
    h.replay_fraction = r.fraction
    h.replay_segment_bytes = r.segment_bytes
    h.replay_stateful_batch = 1 if r.stateful_batch else 0
    return h


@dataclass
class Model:
    config: Config
    threshold: np.ndarray
    excitability: np.ndarray
    neuron_type: np.ndarray
    rec_target: np.ndarray
    rec_branch: np.ndarray
    rec_delay: np.ndarray
    rec_weight: np.ndarray
    in_target: np.ndarray
    in_branch: np.ndarray
    in_weight: np.ndarray
    out_weight: np.ndarray
    bias: np.ndarray
    ctx_keys: np.ndarray
    ctx_emb: np.ndarray
    ctx_obs: np.ndarray
    ctx_out: np.ndarray
    generation: int = 0
    parameter_revision: int = 0
    statistics: Dict[str, float] = field(default_factory=lambda: {k: 0 for k in STAT_FIELDS})

    @staticmethod
    def shapes(config: Config) -> Dict[str, int]:
        n, e = config.model.neuron_count, config.context.embedding_dim
        return {
            "threshold": n, "excitability": n, "neuron_type": n, "rec_target": config.synapse_count,
            "rec_branch": config.synapse_count, "rec_delay": config.synapse_count,
            "rec_weight": config.synapse_count, "in_target": config.input_count, "in_branch": config.input_count,
            "in_weight": config.input_count, "out_weight": OUTPUT_CLASSES * n, "bias": OUTPUT_CLASSES,
            "ctx_keys": config.context_slots, "ctx_emb": config.context_slots * e, "ctx_obs": config.context_slots,
            "ctx_out": OUTPUT_CLASSES * e,
        }

    @classmethod
    def empty(cls, config: Config) -> "Model":
        shapes = cls.shapes(config)
        arrays = {k: np.zeros(shapes[k], dtype=_DTYPES[k]) for k in ARRAY_FIELDS}
        return cls(config=config, **arrays)

    @classmethod
    def initialize(cls, config: Config) -> "Model":
        """Model::initialize (model.rs:79-158)."""
        config.validate()
        model = cls.empty(config)
        lib = native.load()
        hc = host_config(config)
        view = model.view()
        native.check(lib, lib.leo_model_initialize(ctypes.byref(hc), ctypes.byref(view)))
        model._absorb(view)
        return model

    @classmethod
    def synthetic(cls, config: Config, topology: int = native.TOPOLOGY_UNIFORM, exponent: float = 0.0,
                  in_degree_cap: int = 0, weight_sigma: float = 0.05) -> "Model":
        """Seeded synthetic benchmark model (include/leo_hip.h leo_model_initialize_synthetic)."""
        config.validate()
        model = cls.empty(config)
        lib = native.load()
        hc = host_config(config)
        view = model.view()
        native.check(lib, lib.leo_model_initialize_synthetic(ctypes.byref(hc), topology, exponent, in_degree_cap,
                                                              weight_sigma, ctypes.byref(view)))
        model._absorb(view)
        return model

    def validate(self) -> None:
        """Model::validate (model.rs:223-396); raises native.LeoError."""
        lib = native.load()
        hc = host_config(self.config)
        view = self.view()
        native.check(lib, lib.leo_model_validate(ctypes.byref(hc), ctypes.byref(view)))

    def view(self) -> native.LeoModelView:
        """C view of the arrays (valid while this Model is alive and unresized)."""
        v = native.LeoModelView()
        shapes = self.shapes(self.config)
        for k in ARRAY_FIELDS:
            arr = getattr(self, k)
            if arr.dtype != _DTYPES[k] or arr.size != shapes[k] or not arr.flags.c_contiguous:
                raise ValueError(f"model array {k} has the wrong dtype, size or layout")
            setattr(v, k, arr.ctypes.data)
        v.generation = self.generation
        v.parameter_revision = self.parameter_revision
        for k in STAT_FIELDS:
            setattr(v.statistics, k, self.statistics[k])
        return v

    def _absorb(self, view: native.LeoModelView) -> None:
        self.generation = int(view.generation)
        self.parameter_revision = int(view.parameter_revision)
        self.statistics = {k: getattr(view.statistics, k) for k in STAT_FIELDS}

    def copy(self) -> "Model":
        arrays = {k: getattr(self, k).copy() for k in ARRAY_FIELDS}
        return Model(config=self.config, generation=self.generation, parameter_revision=self.parameter_revision,
                     statistics=dict(self.statistics), **arrays)

    def synapse_slot_range(self, neuron: int) -> range:
        s = self.config.model.synapses_per_neuron
        return range(neuron * s, (neuron + 1) * s)

    @property
    def neuron_count(self) -> int:
        return self.config.model.neuron_count

    def bits_per_byte(self) -> float:
        """TrainingStatistics::bits_per_byte (metrics.rs:26-28)."""
        import math

        t = self.statistics["training_targets"]
        return 0.0 if t == 0 else self.statistics["training_loss_sum"] / t / math.log(2.0)
