"""Leo configuration (crates/leo-core/src/config.rs:10-156) and its validation.

Field names, nesting and defaults follow the reference's strict TOML schema so a
Leo config file loads unchanged (``Config.from_toml``). ``validate`` restates
config.rs:250-519 and raises ``ConfigError`` with the reference's messages.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field
from typing import Any, Dict


class ConfigError(ValueError):
    """LeoErrorKind::Configuration (lib.rs)."""


@dataclass
class ModelConfig:
    name: str = "Leo"
    seed: int = 1337
    neuron_count: int = 32_768
    block_count: int = 128
    neurons_per_block: int = 256
    branches_per_neuron: int = 4
    excitatory_fraction: float = 0.80
    synapses_per_neuron: int = 48
    input_fanout: int = 128
    max_active_per_block: int = 8
    max_active_global: int = 1_024


@dataclass
class DynamicsConfig:
    branch_decay: float = 0.85
    membrane_decay: float = 0.90
    fatigue_decay: float = 0.97
    fatigue_gain: float = 0.02
    refractory_ticks: int = 1
    target_activity: float = 0.02
    threshold_homeostasis_rate: float = 0.0001
    population_inhibition_rate: float = 0.05
    population_inhibition_max: float = 2.0
    adaptation_fast_decay: float = 0.95
    adaptation_medium_decay: float = 0.99
    adaptation_slow_decay: float = 0.999
    adaptation_fast_gain: float = 0.005
    adaptation_medium_gain: float = 0.001
    adaptation_slow_gain: float = 0.0002
    membrane_reset_fraction: float = 0.10


@dataclass
class LearningConfig:
    output_learning_rate: float = 0.001
    recurrent_learning_rate: float = 0.0002
    inhibitory_learning_rate: float = 0.00002
    eligibility_decay: float = 0.95
    eligibility_epsilon: float = 1.0e-5
    surrogate_width: float = 0.25
    surrogate_gain: float = 0.10
    max_update: float = 0.01
    weight_min: float = -1.0
    weight_max: float = 1.0
    provisional_strength: float = 0.20
    training_strength: float = 1.00
    verified_strength: float = 1.00
    plasticity_window: int = 1
    end_document_weight: float = 4.0


@dataclass
class ContextConfig:
    max_order: int = 8
    embedding_dim: int = 32
    slots_per_order: int = 8192
    probe_limit: int = 4
    learning_rate: float = 0.05
    confidence_observations: int = 4
    dropout_rate: float = 0.5


@dataclass
class ReplayConfig:
    fraction: float = 0.30
    segment_bytes: int = 64
    stateful_batch: bool = False
    teaching_replays: int = 1
    max_verified_replays: int = 4


@dataclass
class TrainingConfig:
    max_dataset_passes: int = 3
    validate_every_bytes: int = 25_000_000
    checkpoint_every_bytes: int = 50_000_000
    early_stop_checks: int = 3
    minimum_relative_improvement: float = 0.005


def _toml_value(value: Any, default: Any) -> str:
    if isinstance(value, bool):
        return "true" if value else "false"
    if isinstance(default, float) or isinstance(value, float):
        v = float(value)
        if not math.isfinite(v):
            raise ConfigError("configuration floats must be finite")
        text = repr(v)
        return text if any(ch in text for ch in ".eE") else text + ".0"
    if isinstance(value, int):
        return str(value)
    if isinstance(value, str):
        escaped = []
        for ch in value:
            if ch == "\\" or ch == '"':
                escaped.append("\\" + ch)
            elif ord(ch) < 0x20 or ord(ch) == 0x7F:
                escaped.append(f"\\u{ord(ch):04X}")
            else:
                escaped.append(ch)
        return '"' + "".join(escaped) + '"'
    raise ConfigError(f"cannot write {type(value).__name__} to TOML")


def _f32(value: float) -> float:
    import numpy as np

    return float(np.float32(value))


@dataclass
class Config:
    """Config::default() (config.rs:158-235) unless overridden."""

    model: ModelConfig = field(default_factory=ModelConfig)
    dynamics: DynamicsConfig = field(default_factory=DynamicsConfig)
    learning: LearningConfig = field(default_factory=LearningConfig)
    context: ContextConfig = field(default_factory=ContextConfig)
    replay: ReplayConfig = field(default_factory=ReplayConfig)
    training: TrainingConfig = field(default_factory=TrainingConfig)

    _SECTIONS = ("model", "dynamics", "learning", "context", "replay", "training")

    @classmethod
    def from_dict(cls, data: Dict[str, Any]) -> "Config":
        """Strict: unknown sections or fields are rejected (serde deny_unknown_fields)."""
        config = cls()
        for section, values in data.items():
            if section not in cls._SECTIONS:
                raise ConfigError(f"invalid TOML configuration: unknown section `{section}`")
            target = getattr(config, section)
            known = {f.name for f in dataclasses.fields(target)}
            for key, value in values.items():
                if key not in known:
                    raise ConfigError(f"invalid TOML configuration: unknown field `{key}`")
                setattr(target, key, value)
        config.validate()
        return config

    @classmethod
    def from_toml(cls, text: str) -> "Config":
        try:
            import tomllib  # type: ignore[import-not-found]
        except ModuleNotFoundError:  # Python 3.10
            import tomli as tomllib  # type: ignore[no-redef]
        return cls.from_dict(tomllib.loads(text))

    def to_dict(self) -> Dict[str, Any]:
        return {s: dataclasses.asdict(getattr(self, s)) for s in self._SECTIONS}

    def to_toml(self) -> str:
        """Config::to_toml (config.rs:521-523): every section and field in
        declaration order. Floats are written so that they parse back to the
        same value (as f64 here, and as f32 where the reference stores f32);
        the text is not byte-identical to the reference's serializer, and no
        reader depends on that."""
        lines = []
        for section in self._SECTIONS:
            if lines:
                lines.append("")
            lines.append(f"[{section}]")
            target = getattr(self, section)
            for f in dataclasses.fields(target):
                lines.append(f"{f.name} = {_toml_value(getattr(target, f.name), f.default)}")
        return "\n".join(lines) + "\n"

    def copy(self) -> "Config":
        return Config.from_dict(self.to_dict()) if self.is_valid() else dataclasses.replace(self)

    def is_valid(self) -> bool:
        try:
            self.validate()
            return True
        except ConfigError:
            return False

    # config.rs:250-519
    def validate(self) -> None:
        m, d, l, c, r, t = self.model, self.dynamics, self.learning, self.context, self.replay, self.training
        if not m.name.strip():
            raise ConfigError("model.name must not be empty")
        if m.neuron_count == 0 or m.block_count == 0 or m.neurons_per_block == 0:
            raise ConfigError("model dimensions must be positive")
        if m.block_count * m.neurons_per_block != m.neuron_count:
            raise ConfigError("block_count * neurons_per_block must equal neuron_count without overflow")
        if m.branches_per_neuron != 4:
            raise ConfigError("Leo requires exactly four dendritic branches per neuron")
        if not math.isfinite(m.excitatory_fraction) or not (0.0 <= m.excitatory_fraction < 1.0):
            raise ConfigError("excitatory_fraction must be finite and strictly between 0 and 1")
        if m.synapses_per_neuron == 0 or m.input_fanout == 0:
            raise ConfigError("synapses_per_neuron and input_fanout must be positive")
        if m.synapses_per_neuron > m.neuron_count:
            raise ConfigError("synapses_per_neuron cannot exceed neuron_count")
        if m.input_fanout > m.neuron_count:
            raise ConfigError("input_fanout cannot exceed neuron_count")
        if m.max_active_per_block == 0 or m.max_active_per_block > m.neurons_per_block:
            raise ConfigError("max_active_per_block must be in 1..=neurons_per_block")
        if m.max_active_global == 0 or m.max_active_global > m.neuron_count:
            raise ConfigError("max_active_global must be in 1..=neuron_count")
        if d.refractory_ticks == 0:
            raise ConfigError("refractory_ticks must be positive in the integrated architecture")
        for name in ("branch_decay", "membrane_decay", "fatigue_decay", "adaptation_fast_decay",
                     "adaptation_medium_decay", "adaptation_slow_decay"):
            v = getattr(d, name)
            if not math.isfinite(v) or not (0.0 <= v < 1.0):
                raise ConfigError(f"{name} must be finite and strictly between 0 and 1")
        if not math.isfinite(l.eligibility_decay) or not (0.0 <= l.eligibility_decay < 1.0):
            raise ConfigError("eligibility_decay must be finite and strictly between 0 and 1")
        positives = [
            ("fatigue_gain", d.fatigue_gain), ("adaptation_fast_gain", d.adaptation_fast_gain),
            ("adaptation_medium_gain", d.adaptation_medium_gain), ("adaptation_slow_gain", d.adaptation_slow_gain),
            ("threshold_homeostasis_rate", d.threshold_homeostasis_rate),
            ("population_inhibition_rate", d.population_inhibition_rate),
            ("output_learning_rate", l.output_learning_rate), ("recurrent_learning_rate", l.recurrent_learning_rate),
            ("inhibitory_learning_rate", l.inhibitory_learning_rate), ("eligibility_epsilon", l.eligibility_epsilon),
            ("surrogate_width", l.surrogate_width), ("surrogate_gain", l.surrogate_gain), ("max_update", l.max_update),
        ]
        for name, v in positives:
            if not math.isfinite(v) or v <= 0.0:
                raise ConfigError(f"{name} must be finite and positive")
        if not math.isfinite(d.target_activity) or not (0.0 < d.target_activity <= 1.0):
            raise ConfigError("target_activity must be finite and in (0, 1]")
        if not math.isfinite(d.population_inhibition_max) or d.population_inhibition_max <= 0.0:
            raise ConfigError("population_inhibition_max must be finite and positive")
        if not math.isfinite(d.membrane_reset_fraction) or not (0.0 < d.membrane_reset_fraction <= 1.0):
            raise ConfigError("membrane_reset_fraction must be finite and in (0, 1]")
        target_active = math.ceil(_f32(_f32(d.target_activity) * _f32(m.neuron_count)))
        if target_active > m.max_active_global:
            raise ConfigError("target_activity requires more neurons than max_active_global permits")
        if l.weight_min >= 0.0 or l.weight_max <= 0.0 or l.weight_min >= l.weight_max:
            raise ConfigError("weight_min must be negative and weight_max must be positive")
        if l.plasticity_window == 0 or l.plasticity_window > 64:
            raise ConfigError("learning.plasticity_window must be in 1..=64")
        if not math.isfinite(l.end_document_weight) or not (1.0 <= l.end_document_weight <= 16.0):
            raise ConfigError("end_document_weight must be finite and in [1, 16]")
        for name in ("provisional_strength", "training_strength", "verified_strength"):
            v = getattr(l, name)
            if not math.isfinite(v) or not (0.0 < v <= 1.0):
                raise ConfigError(f"{name} must be finite and in (0, 1]")
        if (c.max_order == 0 or c.embedding_dim == 0 or c.slots_per_order == 0 or c.probe_limit == 0
                or c.confidence_observations == 0):
            raise ConfigError("all context-memory dimensions must be positive")
        if c.embedding_dim > 256:
            raise ConfigError("context.embedding_dim cannot exceed 256")
        if c.max_order > 16:
            raise ConfigError("context.max_order cannot exceed 16")
        if c.probe_limit > c.slots_per_order:
            raise ConfigError("context.probe_limit cannot exceed slots_per_order")
        if not math.isfinite(c.dropout_rate) or not (0.0 <= c.dropout_rate < 1.0):
            raise ConfigError("context.dropout_rate must be finite and in [0, 1)")
        if not math.isfinite(c.learning_rate) or c.learning_rate <= 0.0:
            raise ConfigError("context.learning_rate must be finite and positive")
        if not math.isfinite(r.fraction) or r.fraction < 0.0 or r.fraction > 1.0:
            raise ConfigError("replay.fraction must be finite and in the interval [0, 1]")
        if r.segment_bytes == 0 or r.teaching_replays == 0 or r.max_verified_replays == 0:
            raise ConfigError("all replay limits must be positive")
        if (t.max_dataset_passes == 0 or t.validate_every_bytes == 0 or t.checkpoint_every_bytes == 0
                or t.early_stop_checks == 0):
            raise ConfigError("all training limits must be positive")
        if not math.isfinite(t.minimum_relative_improvement) or t.minimum_relative_improvement < 0.0:
            raise ConfigError("minimum_relative_improvement must be finite and nonnegative")

    # sizes
    @property
    def synapse_count(self) -> int:
        return self.model.neuron_count * self.model.synapses_per_neuron

    @property
    def input_count(self) -> int:
        return 258 * self.model.input_fanout

    @property
    def context_slots(self) -> int:
        return self.context.max_order * self.context.slots_per_order

    def strength(self, permission: int) -> float:
        """Permission::strength (permission.rs:24-31)."""
        from .native import FROZEN, PROVISIONAL, TRAINING, VERIFIED

        return {FROZEN: 0.0, PROVISIONAL: self.learning.provisional_strength,
                TRAINING: self.learning.training_strength, VERIFIED: self.learning.verified_strength}[permission]


def test_toml_values() -> Dict[str, Dict[str, Any]]:
    """The reference's configs/test.toml (128 neurons), as data."""
    return {
        "model": dict(name="Leo-test", seed=1337, neuron_count=128, block_count=8, neurons_per_block=16,
                      branches_per_neuron=4, excitatory_fraction=0.8, synapses_per_neuron=8, input_fanout=8,
                      max_active_per_block=2, max_active_global=8),
        "dynamics": dict(branch_decay=0.85, membrane_decay=0.90, fatigue_decay=0.97, fatigue_gain=0.02,
                         refractory_ticks=1, target_activity=0.04, threshold_homeostasis_rate=0.0001,
                         population_inhibition_rate=0.05, population_inhibition_max=2.0,
                         adaptation_fast_decay=0.95, adaptation_medium_decay=0.99, adaptation_slow_decay=0.999,
                         adaptation_fast_gain=0.005, adaptation_medium_gain=0.001, adaptation_slow_gain=0.0002,
                         membrane_reset_fraction=0.10),
        "learning": dict(output_learning_rate=0.002, recurrent_learning_rate=0.0005,
                         inhibitory_learning_rate=0.00005, eligibility_decay=0.95, eligibility_epsilon=0.00001,
                         surrogate_width=0.25, surrogate_gain=0.10, max_update=0.01, weight_min=-1.0,
                         weight_max=1.0, provisional_strength=0.20, training_strength=1.0, verified_strength=1.0,
                         plasticity_window=1, end_document_weight=4.0),
        "context": dict(embedding_dim=8, max_order=4, slots_per_order=128, probe_limit=4, learning_rate=0.08,
                        confidence_observations=2, dropout_rate=0.0),
        "replay": dict(fraction=0.30, segment_bytes=8, stateful_batch=False, teaching_replays=1,
                       max_verified_replays=2),
        "training": dict(max_dataset_passes=2, validate_every_bytes=512, checkpoint_every_bytes=1024,
                         early_stop_checks=3, minimum_relative_improvement=0.005),
    }
