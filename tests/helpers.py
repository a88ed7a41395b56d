"""Shared fixtures for the parity tests: configs and hand-wired models mirroring
the reference's own test fixtures (runtime.rs:1632-1692, configs/test.toml)."""
from __future__ import annotations

import numpy as np

from leo_amd.config import Config, test_toml_values
from leo_amd.model import Model

BRANCH_EXCITATORY, BRANCH_INHIBITORY, BRANCH_TEMPORAL, BRANCH_CONTEXT_GATE = 0, 1, 2, 3


def toml_test_config() -> Config:
    """configs/test.toml."""
    return Config.from_dict(test_toml_values())


def integrated_config() -> Config:
    """runtime.rs:1632-1660 integrated_config()."""
    c = Config()
    c.model.name = "integrated-runtime-test"
    c.model.neuron_count = 8
    c.model.block_count = 1
    c.model.neurons_per_block = 8
    c.model.synapses_per_neuron = 1
    c.model.input_fanout = 1
    c.model.max_active_per_block = 8
    c.model.max_active_global = 8
    c.dynamics.fatigue_gain = 1.0e-6
    c.dynamics.refractory_ticks = 1
    c.dynamics.target_activity = 0.5
    c.dynamics.threshold_homeostasis_rate = 1.0e-8
    c.learning.output_learning_rate = 1.0e-8
    c.learning.recurrent_learning_rate = 0.1
    c.learning.inhibitory_learning_rate = 1.0e-8
    c.learning.eligibility_epsilon = 1.0e-7
    c.learning.surrogate_width = 0.25
    c.learning.surrogate_gain = 0.1
    c.learning.max_update = 0.1
    c.context.max_order = 3
    c.context.slots_per_order = 1024
    c.context.learning_rate = 0.1
    c.context.confidence_observations = 1
    c.context.dropout_rate = 0.0
    c.validate()
    return c


def causal_model(delay: int) -> Model:
    """runtime.rs:1662-1692 causal_model()."""
    m = Model.initialize(integrated_config())
    m.threshold[:] = 0.1
    m.excitability[:] = 1.0
    m.rec_weight[:] = 0.0
    m.neuron_type[0] = 0
    for slot in m.synapse_slot_range(0):
        m.rec_branch[slot] = BRANCH_EXCITATORY
    m.in_weight[:] = 0.0
    m.in_branch[:] = BRANCH_EXCITATORY
    m.out_weight[:] = 0.0
    m.bias[:] = 0.0
    m.rec_target[0] = 1
    m.rec_branch[0] = BRANCH_EXCITATORY
    m.rec_delay[0] = delay
    m.rec_weight[0] = 0.5
    fan = m.config.model.input_fanout
    m.in_target[ord("A") * fan] = 0
    m.in_weight[ord("A") * fan] = 1.0
    m.in_target[ord("B") * fan] = 7
    m.in_weight[ord("B") * fan] = 0.0
    n = m.neuron_count
    m.out_weight[ord("Z") * n + 1] = 1.0
    return m


def small_redundant_config(neurons: int = 1024, synapses: int = 16, fanout: int = 64, per_block: int = 8,
                           seed: int = 1337, dropout: float = 0.5) -> Config:
    """A config-A-shaped model (blocks of 256, non-binding global cap) small enough for the oracle."""
    values = test_toml_values()
    values["model"].update(name="Leo-small", seed=seed, neuron_count=neurons, block_count=neurons // 256,
                           neurons_per_block=256, synapses_per_neuron=synapses, input_fanout=fanout,
                           max_active_per_block=per_block, max_active_global=(neurons // 256) * per_block)
    values["dynamics"].update(target_activity=0.02)
    values["context"].update(max_order=6, embedding_dim=16, slots_per_order=4096, probe_limit=4, learning_rate=0.02,
                             confidence_observations=8, dropout_rate=dropout)
    values["replay"].update(fraction=0.30, segment_bytes=32)
    return Config.from_dict(values)


def story(seed: int, length: int) -> bytes:
    """Deterministic lowercase ASCII story with a newline terminator."""
    rng = np.random.default_rng(seed)
    words = ["once", "upon", "a", "time", "the", "cat", "sat", "on", "mat", "and", "ran", "far", "away", "home"]
    out = []
    while sum(len(w) + 1 for w in out) < length:
        out.append(words[int(rng.integers(len(words)))])
    text = " ".join(out)[: length - 1] + "\n"
    return text.encode()


MODEL_ARRAYS = ("threshold", "rec_weight", "in_weight", "out_weight", "bias", "ctx_keys", "ctx_emb", "ctx_obs",
                "ctx_out")


def assert_models_equal(a: Model, b: Model, label: str = "") -> None:
    for name in MODEL_ARRAYS:
        x, y = getattr(a, name), getattr(b, name)
        if not np.array_equal(x, y):
            diff = np.nonzero(x != y)[0]
            raise AssertionError(f"{label}: {name} differs at {diff.size} entries, first {diff[:5]}: "
                                 f"{x[diff[:5]]} vs {y[diff[:5]]}")
    assert a.parameter_revision == b.parameter_revision, (label, a.parameter_revision, b.parameter_revision)
    for k, v in a.statistics.items():
        assert b.statistics[k] == v, (label, k, v, b.statistics[k])
