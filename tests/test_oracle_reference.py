"""Pins the CPU oracle to the known answers the reference's own tests hold.

Each test cites the reference test it restates; expected values are the
reference's literals (learning.rs:80-107, runtime.rs:1694-2150,
runtime_smoke.rs, parallel.rs:1365-1629, main.rs:1744-1752). A plausible slip
in the oracle -- a delay off by one tick, a dropped decay, a wrong sign in the
context gradient, a merge in the wrong order -- fails one of them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import (BRANCH_CONTEXT_GATE, BRANCH_EXCITATORY, BRANCH_INHIBITORY, BRANCH_TEMPORAL,
                           causal_model, integrated_config, toml_test_config)


# --- learning.rs:80-107 -----------------------------------------------------------
def test_analog_surrogate_preserves_selected_unsaturated_gradient(oracle):
    lib = oracle.load()
    assert abs(lib.oracle_analog_rank_surrogate(0.5, 0.4, 1, 0.25, 0.1) - 1.06) <= 1e-6
    assert lib.oracle_analog_rank_surrogate(1.0, 0.4, 1, 0.25, 0.1) == 0.0


def test_branch_jacobian_matches_integrated_branch_semantics(oracle):
    lib = oracle.load()
    assert lib.oracle_branch_jacobian(BRANCH_EXCITATORY, 1.0, 0.5, 0.5) == 1.0
    assert lib.oracle_branch_jacobian(BRANCH_TEMPORAL, 1.0, 0.5, 0.5) == 0.5
    assert lib.oracle_branch_jacobian(BRANCH_INHIBITORY, 1.0, 0.5, 0.5) == 1.0
    assert lib.oracle_branch_jacobian(BRANCH_CONTEXT_GATE, 1.0, 0.5, 0.5) == 0.5


def test_inhibitory_homeostasis_pushes_in_the_correct_direction(oracle):
    lib = oracle.load()
    assert lib.oracle_inhibitory_homeostasis_delta(1.0, 0.10, 0.02, 0.01, 1.0, 0.1) < 0.0
    assert lib.oracle_inhibitory_homeostasis_delta(1.0, 0.00, 0.02, 0.01, 1.0, 0.1) > 0.0


def test_update_clipping_is_symmetric(oracle):
    lib = oracle.load()
    assert lib.oracle_bounded_delta(1.0, 0.1) == np.float32(0.1)
    assert lib.oracle_bounded_delta(-1.0, 0.1) == np.float32(-0.1)


def test_decay_is_square_and_multiply_powi(oracle):
    """runtime.rs:78-85: 0 -> 1, 1 -> base, else f32::powi; powi(b, 2^k) is k exact squarings."""
    lib = oracle.load()
    base = np.float32(0.85)
    assert lib.oracle_decay_for_elapsed(base, 0) == 1.0
    assert lib.oracle_decay_for_elapsed(base, 1) == base
    sq = base
    for k in range(1, 6):
        sq = np.float32(sq * sq)
        assert lib.oracle_decay_for_elapsed(base, 2 ** k) == sq
    # 3 = 1 + 2: r = base; then r *= base^2
    assert lib.oracle_decay_for_elapsed(base, 3) == np.float32(base * np.float32(base * base))


def test_plasticity_window_schedule(oracle):
    """config.rs:137-145: window 1 consolidates every step; window 4 every 4th or at END."""
    import ctypes

    lib = oracle.load()
    scale, nxt = ctypes.c_float(), ctypes.c_uint64()
    lib.oracle_plasticity_step(1, 0, 0, ctypes.byref(scale), ctypes.byref(nxt))
    assert (scale.value, nxt.value) == (1.0, 0)
    seq, phase = [], 0
    for _ in range(5):
        lib.oracle_plasticity_step(4, phase, 0, ctypes.byref(scale), ctypes.byref(nxt))
        seq.append(scale.value)
        phase = nxt.value
    assert seq == [0.0, 0.0, 0.0, 4.0, 0.0]
    lib.oracle_plasticity_step(4, 1, 1, ctypes.byref(scale), ctypes.byref(nxt))
    assert (scale.value, nxt.value) == (2.0, 0)


# --- runtime.rs tests ------------------------------------------------------------
def test_frozen_execution_is_read_only(oracle):  # runtime.rs:1694-1708
    model = causal_model(2)
    rt = oracle.OracleRuntime(model)
    rt.begin_document()
    for sym in b"ABBA":
        rt.step(sym, None, oracle.FROZEN)
    assert rt.model().rec_weight[0] == model.rec_weight[0]
    assert rt.read_list("eligible_rec").size == 0
    assert rt.read_list("eligible_in").size == 0


@pytest.mark.parametrize("delay", [1, 2, 4, 8])
def test_recurrent_credit_arrives_on_the_configured_delay(oracle, delay):  # runtime.rs:1710-1732
    rt = oracle.OracleRuntime(causal_model(delay))
    rt.begin_document()
    initial = rt.model().rec_weight[0]
    rt.step(ord("A"), ord("Y"), oracle.TRAINING)
    assert rt.model().rec_weight[0] == initial
    for _ in range(1, delay):
        rt.step(ord("B"), ord("Y"), oracle.TRAINING)
        assert rt.model().rec_weight[0] == initial
    rt.step(ord("B"), ord("Y"), oracle.TRAINING)
    assert rt.model().rec_weight[0] != initial


def test_input_trace_survives_refractory_tick_and_receives_later_error(oracle):  # runtime.rs:1734-1754
    model = causal_model(1)
    slot = ord("A") * model.config.model.input_fanout
    model.in_weight[slot] = 0.5
    n = model.neuron_count
    model.out_weight[:] = 0.0
    model.out_weight[ord("Z") * n] = 1.0
    rt = oracle.OracleRuntime(model)
    rt.begin_document()
    rt.step(ord("A"), None, oracle.TRAINING)
    before = rt.model().in_weight[slot]
    rt.step(ord("B"), ord("Y"), oracle.TRAINING)
    assert rt.read_f32("in_e")[slot] > 0.0
    assert rt.model().in_weight[slot] < before


def test_context_embedding_gradient_uses_the_exact_forward_scale(oracle):  # runtime.rs:1756-1781
    c = integrated_config()
    c.context.embedding_dim = 1
    c.context.learning_rate = 0.1
    c.learning.max_update = 1.0
    c.validate()
    model = Model.initialize(c)
    model.ctx_emb[:] = 0.0
    model.ctx_out[:] = 0.0
    model.ctx_keys[0] = 1
    model.ctx_keys[1] = 2
    model.ctx_out[ord("X")] = 1.0
    rt = oracle.OracleRuntime(model)
    errors = np.zeros(257, dtype=np.float32)
    errors[ord("X")] = 1.0
    rt.test_update_context_projection([0, 1], [0.25, 0.75], errors, 1.0)
    emb = rt.model().ctx_emb
    assert abs(emb[0] + 0.025) < 1e-6
    assert abs(emb[1] + 0.075) < 1e-6


def test_activity_target_does_not_force_winners_without_evidence(oracle):  # runtime.rs:1783-1794
    model = Model.initialize(integrated_config())
    model.rec_weight[:] = 0.0
    model.in_weight[:] = 0.0
    model.threshold[:] = 0.5
    rt = oracle.OracleRuntime(model)
    rt.begin_document()
    m = rt.step(ord("A"), None, oracle.FROZEN)
    assert m.active_neurons == 0
    assert m.suprathreshold_neurons == 0


def _recurrent_memory_model() -> Model:  # runtime.rs:1796-1828
    c = integrated_config()
    c.model.neuron_count = 64
    c.model.block_count = 1
    c.model.neurons_per_block = 64
    c.model.synapses_per_neuron = 1
    c.model.input_fanout = 1
    c.model.max_active_per_block = 64
    c.model.max_active_global = 64
    c.dynamics.target_activity = 0.01
    c.dynamics.membrane_reset_fraction = 1.0
    c.dynamics.fatigue_gain = 1.0e-6
    c.dynamics.adaptation_fast_gain = 1.0e-8
    c.dynamics.adaptation_medium_gain = 1.0e-8
    c.dynamics.adaptation_slow_gain = 1.0e-8
    c.context.max_order = 8
    c.context.embedding_dim = 8
    c.context.slots_per_order = 64
    c.context.probe_limit = 4
    c.validate()
    m = Model.initialize(c)
    m.threshold[:] = 0.9
    m.excitability[:] = 2.0
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.out_weight[:] = 0.0
    m.bias[:] = 0.0
    m.ctx_emb[:] = 0.0
    m.ctx_out[:] = 0.0
    return m


def _configure_chain(m: Model, source: int, links: int, delay: int) -> int:  # runtime.rs:1830-1847
    for off in range(links):
        n = source + off
        slot = m.synapse_slot_range(n).start
        m.neuron_type[n] = 0
        m.rec_target[slot] = n + 1
        m.rec_branch[slot] = BRANCH_EXCITATORY
        m.rec_delay[slot] = delay
        m.rec_weight[slot] = 1.0
    end = source + links
    m.neuron_type[end] = 0
    es = m.synapse_slot_range(end).start
    m.rec_branch[es] = BRANCH_EXCITATORY
    m.rec_delay[es] = 1
    m.rec_weight[es] = 0.0
    return end


def _wire_chain_inputs(m: Model):
    fan = m.config.model.input_fanout
    a, b = ord("A") * fan, ord("B") * fan
    m.in_target[a], m.in_target[b] = 0, 32
    m.in_branch[a] = m.in_branch[b] = BRANCH_EXCITATORY
    m.in_weight[a] = m.in_weight[b] = 1.0


@pytest.mark.parametrize("distance", [16, 32, 64, 128])
def test_recurrent_only_state_preserves_branch_information(oracle, distance):  # runtime.rs:1849-1897
    m = _recurrent_memory_model()
    links = distance // 8
    end_a = _configure_chain(m, 0, links, 8)
    end_b = _configure_chain(m, 32, links, 8)
    _wire_chain_inputs(m)
    n = m.neuron_count
    m.out_weight[ord("X") * n + end_a] = 1.0
    m.out_weight[ord("Y") * n + end_b] = 1.0
    m.validate()
    rt = oracle.OracleRuntime(m)

    def predict(prefix):
        rt.begin_document()
        rt.step(prefix, None, oracle.FROZEN)
        pred = 0
        for _ in range(distance):
            pred = rt.step(ord("."), None, oracle.FROZEN).predicted_symbol
        return pred

    assert predict(ord("A")) == ord("X")
    assert predict(ord("B")) == ord("Y")


@pytest.mark.parametrize("distance", [16, 32])
def test_recurrent_only_readout_learns_delayed_branches(oracle, distance):  # runtime.rs:1899-1950
    m = _recurrent_memory_model()
    m.config.learning.output_learning_rate = 0.05
    m.config.learning.max_update = 0.05
    links = distance // 8
    _configure_chain(m, 0, links, 8)
    _configure_chain(m, 32, links, 8)
    _wire_chain_inputs(m)
    m.validate()
    rt = oracle.OracleRuntime(m)
    for _ in range(64):
        for prefix, target in ((ord("A"), ord("X")), (ord("B"), ord("Y"))):
            rt.begin_document()
            rt.step(prefix, None, oracle.FROZEN)
            for _ in range(distance - 1):
                rt.step(ord("."), None, oracle.FROZEN)
            rt.step(ord("."), target, oracle.TRAINING)
            rt.finish_document()
    for prefix, expected in ((ord("A"), ord("X")), (ord("B"), ord("Y"))):
        rt.begin_document()
        rt.step(prefix, None, oracle.FROZEN)
        pred = 0
        for _ in range(distance):
            pred = rt.step(ord("."), None, oracle.FROZEN).predicted_symbol
        assert pred == expected


def test_recurrent_only_ring_maintains_a_period(oracle):  # runtime.rs:1952-1993
    m = _recurrent_memory_model()
    period = 16
    n = m.neuron_count
    for neuron in range(period):
        slot = m.synapse_slot_range(neuron).start
        m.neuron_type[neuron] = 0
        m.rec_target[slot] = (neuron + 1) % period
        m.rec_branch[slot] = BRANCH_EXCITATORY
        m.rec_delay[slot] = 1
        m.rec_weight[slot] = 1.0
        m.out_weight[(ord("A") + neuron) * n + neuron] = 1.0
    fan = m.config.model.input_fanout
    m.in_target[ord("!") * fan] = 0
    m.in_branch[ord("!") * fan] = BRANCH_EXCITATORY
    m.in_weight[ord("!") * fan] = 1.0
    m.validate()
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    preds = [rt.step(ord("!"), None, oracle.FROZEN).predicted_symbol]
    for _ in range(1, period * 2):
        preds.append(rt.step(ord("."), None, oracle.FROZEN).predicted_symbol)
    assert preds[:period] == preds[period:]
    assert all(a != b for a, b in zip(preds[:period], preds[1:period]))


def test_context_fingerprints_separate_colliding_buckets(oracle):  # runtime.rs:1995-2011
    c = integrated_config()
    c.context.max_order = 1
    c.context.slots_per_order = 4
    c.context.probe_limit = 4
    c.validate()
    rt = oracle.OracleRuntime(Model.initialize(c))
    first, _ = rt.resolve_context_slot(1, 1, True)
    second, _ = rt.resolve_context_slot(1, 5, True)
    assert first != second
    keys = rt.model().ctx_keys
    assert keys[first] == 1 and keys[second] == 5


def test_temporal_context_learns_branching_prefixes(oracle):  # runtime.rs:2013-2076
    c = integrated_config()
    c.learning.output_learning_rate = 1.0e-8
    c.context.learning_rate = 0.5
    c.learning.max_update = 0.1
    c.validate()
    m = Model.initialize(c)
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.out_weight[:] = 0.0
    m.bias[:] = 0.0
    m.threshold[:] = 2.0
    rt = oracle.OracleRuntime(m)
    for _ in range(128):
        for s in (b"ABX", b"CBY"):
            rt.begin_document()
            rt.step(BEGIN_DOCUMENT, s[0], oracle.TRAINING)
            rt.step(s[0], s[1], oracle.TRAINING)
            rt.step(s[1], s[2], oracle.TRAINING)
            rt.step(s[2], END_DOCUMENT, oracle.TRAINING)
            rt.finish_document()

    def predict(prefix):
        rt.begin_document()
        rt.step(BEGIN_DOCUMENT, None, oracle.FROZEN)
        pred = END_DOCUMENT
        for b in prefix:
            pred = rt.step(b, None, oracle.FROZEN).predicted_symbol
        return pred

    assert predict(b"AB") == ord("X")
    assert predict(b"CB") == ord("Y")
    assert rt.model().rec_weight.size == m.rec_weight.size


def test_context_dropout_is_deterministic_and_exposes_neural_steps(oracle):  # runtime.rs:2078-2089
    lib = oracle.load()
    first = sum(lib.oracle_context_survives_dropout(1337, t, ord("A"), 0.5) for t in range(1024))
    second = sum(lib.oracle_context_survives_dropout(1337, t, ord("A"), 0.5) for t in range(1024))
    assert first == second
    assert 400 <= first <= 624
    assert all(lib.oracle_context_survives_dropout(1337, t, ord("A"), 0.0) for t in range(32))


def test_end_document_target_receives_extra_bounded_weight(oracle):  # runtime.rs:2091-2116
    c = integrated_config()
    c.learning.output_learning_rate = 0.01
    c.learning.end_document_weight = 4.0
    c.learning.max_update = 0.02
    c.context.dropout_rate = 0.0
    m = Model.initialize(c)
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.out_weight[:] = 0.0
    m.bias[:] = 0.0
    m.threshold[:] = 2.0
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, END_DOCUMENT, oracle.TRAINING)
    bias = rt.model().bias[256]
    assert 0.019 <= bias <= 0.02 + np.finfo(np.float32).eps


def test_initialization_enforces_excitatory_and_inhibitory_routes():  # runtime.rs:2118-2132
    m = Model.initialize(integrated_config())
    for src in range(m.neuron_count):
        for slot in m.synapse_slot_range(src):
            if m.neuron_type[src] == 0:
                assert m.rec_weight[slot] >= 0.0 and m.rec_branch[slot] != BRANCH_INHIBITORY
            else:
                assert m.rec_weight[slot] <= 0.0 and m.rec_branch[slot] == BRANCH_INHIBITORY


def test_adaptation_and_reset_are_part_of_every_runtime(oracle):  # runtime.rs:2134-2150
    m = Model.initialize(integrated_config())
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.threshold[:] = 0.1
    slot = ord("A") * m.config.model.input_fanout
    m.in_target[slot] = 0
    m.in_branch[slot] = BRANCH_EXCITATORY
    m.in_weight[slot] = 1.0
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    metrics = rt.step(ord("A"), None, oracle.FROZEN)
    assert metrics.active_neurons > 0
    assert rt.read_f32("membrane")[0] < 1.0
    assert any(rt.read_f32(f"adapt{k}")[0] > 0.0 for k in range(3))


# --- runtime_smoke.rs --------------------------------------------------------------
def test_frozen_document_is_read_only(oracle):  # runtime_smoke.rs:38-71
    m = Model.initialize(toml_test_config())
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, ord("A"), oracle.FROZEN)
    rt.step(ord("A"), END_DOCUMENT, oracle.FROZEN)
    rt.finish_document()
    out = rt.model()
    for name in ("rec_weight", "in_weight", "out_weight", "bias", "ctx_keys", "ctx_emb", "ctx_out", "ctx_obs"):
        assert np.array_equal(getattr(out, name), getattr(m, name)), name
    assert out.statistics["processed_bytes"] == 0 and out.statistics["processed_stories"] == 0


def test_training_document_updates_persistent_statistics(oracle):  # runtime_smoke.rs:73-90
    rt = oracle.OracleRuntime(Model.initialize(toml_test_config()))
    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, ord("A"), oracle.TRAINING)
    rt.step(ord("A"), END_DOCUMENT, oracle.TRAINING)
    rt.finish_document()
    s = rt.model().statistics
    assert (s["processed_bytes"], s["processed_stories"], s["training_targets"], s["persistent_ticks"]) == (1, 1, 2, 2)


def test_sparse_selection_respects_the_global_cap(oracle):  # runtime_smoke.rs:92-121
    c = toml_test_config()
    c.model.neuron_count = 64
    c.model.block_count = 1
    c.model.neurons_per_block = 64
    c.model.input_fanout = 64
    c.model.max_active_per_block = 64
    c.model.max_active_global = 8
    c.dynamics.target_activity = 0.02
    c.validate()
    m = Model.initialize(c)
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.threshold[:] = 0.1
    start = ord("A") * 64
    for neuron in range(64):
        m.in_target[start + neuron] = neuron
        m.in_branch[start + neuron] = BRANCH_EXCITATORY
        m.in_weight[start + neuron] = 1.0
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    metrics = rt.step(ord("A"), None, oracle.FROZEN)
    assert 0 < metrics.active_neurons <= 8


def test_output_cache_matches_checkpoint_layout(oracle):  # runtime_smoke.rs:9-36, 123-155
    m = Model.initialize(toml_test_config())
    m.threshold[:] = 0.1
    m.in_branch[:] = BRANCH_EXCITATORY
    m.in_weight[:] = 1.0
    rt = oracle.OracleRuntime(m)

    def manual(model):
        n = model.neuron_count
        logits = model.bias.astype(np.float32).copy()
        act = rt.read_f32("activation")
        for neuron in rt.read_list("active"):
            for o in range(257):
                logits[o] = np.float32(logits[o] + np.float32(model.out_weight[o * n + neuron] * act[neuron]))
        mx = logits.max()
        p = np.exp((logits - mx).astype(np.float64)).astype(np.float32)
        return p / p.sum(dtype=np.float32)

    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, None, oracle.FROZEN)
    assert rt.read_list("active").size > 0
    assert np.all(np.abs(rt.read_f32("probabilities") - manual(rt.model())) <= 1e-6)
    mut = rt.model()
    mut.out_weight[: mut.neuron_count] += np.float32(0.25)
    rt.set_model(mut)
    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, None, oracle.FROZEN)
    assert np.all(np.abs(rt.read_f32("probabilities") - manual(rt.model())) <= 1e-6)


# --- parallel.rs tests --------------------------------------------------------------
def test_fixed_parameters_merge_as_a_synchronous_mean_delta(oracle):  # parallel.rs:1365-1383
    base = Model.initialize(toml_test_config())
    first, second = base.copy(), base.copy()
    first.bias[0] += np.float32(0.2)
    second.bias[0] += np.float32(0.4)
    first.statistics["processed_stories"] += 1
    second.statistics["processed_stories"] += 1
    deltas = [oracle.Delta.between(base, first), oracle.Delta.between(base, second)]
    master = oracle.OracleRuntime(base)
    fixed, _ = oracle.apply_deltas(master, deltas)
    out = master.model()
    assert abs(out.bias[0] - (base.bias[0] + 0.3)) < 1e-6
    assert out.statistics["processed_stories"] == 2
    assert fixed == 1


def test_tracked_delta_matches_full_delta_for_one_worker_story(oracle):  # parallel.rs:1385-1404
    base = Model.initialize(toml_test_config())
    rt = oracle.OracleRuntime(base)
    rt.enable_parameter_tracking()
    rt.begin_document()
    rt.step(BEGIN_DOCUMENT, ord("A"), oracle.TRAINING)
    rt.step(ord("A"), END_DOCUMENT, oracle.TRAINING)
    rt.finish_document()
    full = oracle.Delta.between(base, rt.model())
    tracked = oracle.Delta.between_tracked(base, rt)
    assert tracked == full


def test_output_weights_merge_in_logical_worker_order(oracle):  # parallel.rs:1482-1504
    base = Model.initialize(toml_test_config())
    index = 7 * base.neuron_count + 3
    first, second = base.copy(), base.copy()
    first.out_weight[index] += np.float32(0.2)
    second.out_weight[index] -= np.float32(0.1)
    deltas = [oracle.Delta.between(base, first), oracle.Delta.between(base, second)]
    assert deltas[0].count("output_weight") == 1 and deltas[1].count("output_weight") == 1
    master = oracle.OracleRuntime(base)
    oracle.apply_deltas(master, deltas)
    assert abs(master.model().out_weight[index] - (base.out_weight[index] + 0.05)) < 1e-6


def test_additive_delta_merge_preserves_local_trajectory_magnitude(oracle):  # parallel.rs:1506-1524
    base = Model.initialize(toml_test_config())
    first, second = base.copy(), base.copy()
    first.bias[0] += np.float32(0.2)
    second.bias[0] -= np.float32(0.05)
    first.parameter_revision += 2
    second.parameter_revision += 3
    deltas = [oracle.Delta.between(base, first), oracle.Delta.between(base, second)]
    master = oracle.OracleRuntime(base)
    oracle.apply_deltas(master, deltas, mean=False)
    out = master.model()
    assert abs(out.bias[0] - (base.bias[0] + 0.15)) < 1e-6
    assert out.parameter_revision == base.parameter_revision + 5


def test_stale_worker_deltas_are_rejected(oracle):  # parallel.rs:1585-1595
    base = Model.initialize(toml_test_config())
    trained = base.copy()
    trained.bias[0] += np.float32(0.1)
    delta = oracle.Delta.between(base, trained)
    advanced = base.copy()
    advanced.parameter_revision += 1
    master = oracle.OracleRuntime(advanced)
    with pytest.raises(oracle.OracleError, match="current canonical revision"):
        oracle.apply_deltas(master, [delta])


def test_context_entries_merge_by_fingerprint_not_collision_slot(oracle):  # parallel.rs:1597-1629
    base = Model.initialize(toml_test_config())
    slots = base.config.context.slots_per_order
    k1, k2 = 1, 1 + slots
    r1, r2 = oracle.OracleRuntime(base), oracle.OracleRuntime(base)
    s1, _ = r1.resolve_context_slot(1, k1, True)
    s2, _ = r2.resolve_context_slot(1, k2, True)
    first, second = r1.model(), r2.model()
    dim = base.config.context.embedding_dim
    first.ctx_emb[s1 * dim] = 0.4
    second.ctx_emb[s2 * dim] = -0.2
    first.ctx_obs[s1] = 1
    second.ctx_obs[s2] = 1
    deltas = [oracle.Delta.between(base, first), oracle.Delta.between(base, second)]
    master = oracle.OracleRuntime(base)
    oracle.apply_deltas(master, deltas)
    keys = master.model().ctx_keys[:slots]
    assert k1 in keys and k2 in keys


# --- training.rs / main.rs ------------------------------------------------------------
def test_replay_selects_high_loss_non_overlapping_segments(oracle):  # main.rs:1744-1752
    ranges = oracle.select_replay_ranges([0.1, 4.0, 0.2, 0.1, 0.2, 5.0, 0.1, 0.1], 0.50, 3)
    assert len(ranges) == 2
    (a0, a1), (b0, b1) = ranges
    assert not (a0 < b1 and b0 < a1)
    assert any(s <= 1 < e for s, e in ranges)
    assert any(s <= 5 < e for s, e in ranges)


def _brute_force_replay(losses, fraction, segment):
    """Independent statement of training.rs:1782-1830 for the property check."""
    n = len(losses)
    if n == 0 or fraction <= 0 or segment == 0:
        return []
    budget = max(1, math.ceil(n * float(min(np.float32(fraction), np.float32(1.0)))))  # f64 product
    order = sorted(range(n), key=lambda i: (-losses[i], i))
    chosen, used = [], 0
    for p in order:
        if used >= budget:
            break
        if not math.isfinite(losses[p]) or losses[p] <= 0:
            continue
        width = min(segment, budget - used, n)
        start = max(p - width // 2, 0)
        end = min(start + width, n)
        start = max(end - width, 0)
        if any(s < end and start < e for s, e in chosen):
            continue
        used += end - start
        chosen.append((start, end))
    return sorted(chosen)


def test_replay_selection_matches_brute_force(oracle):
    rng = np.random.default_rng(9001)
    for trial in range(300):
        n = int(rng.integers(1, 40))
        losses = rng.choice([0.0, 0.5, 1.0, 2.0, 3.5], size=n).astype(np.float32)
        if trial % 3 == 0:
            losses = rng.random(n).astype(np.float32) * 5
        frac = float(rng.choice([0.1, 0.3, 0.5, 1.0]))
        seg = int(rng.integers(1, 9))
        assert oracle.select_replay_ranges(losses, frac, seg) == _brute_force_replay(
            [float(x) for x in losses], np.float32(frac), seg)


# --- block selection order (runtime.rs:940-1074) pinned by brute force ---------------------
@pytest.mark.parametrize("tick_offset", [0, 1, 5])
def test_block_selection_order_matches_brute_force(oracle, tick_offset):
    """Winners are the top-k by (activation desc, rotated tie key asc) with ties broken
    by (neuron + N - tick % N) % N; the cutoff is the (k+1)-th value."""
    c = toml_test_config()
    c.model.neuron_count = 64
    c.model.block_count = 1
    c.model.neurons_per_block = 64
    c.model.input_fanout = 64
    c.model.max_active_per_block = 6
    c.model.max_active_global = 6
    c.dynamics.target_activity = 0.02
    c.validate()
    m = Model.initialize(c)
    m.rec_weight[:] = 0.0
    m.in_weight[:] = 0.0
    m.threshold[:] = 0.1
    rng = np.random.default_rng(424242 + tick_offset)
    levels = np.array([0.3, 0.35, 0.35, 0.5, 0.5, 0.5, 0.7], dtype=np.float32)
    start = ord("A") * 64
    weights = rng.choice(levels, size=64)
    for neuron in range(64):
        m.in_target[start + neuron] = neuron
        m.in_branch[start + neuron] = BRANCH_EXCITATORY
        m.in_weight[start + neuron] = weights[neuron]
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    for _ in range(tick_offset):  # advance the tick with an input that touches nothing active
        rt.reset_transient_state()
        rt.step(ord("b"), None, oracle.FROZEN)
    rt.reset_transient_state()
    tick = rt.current_tick
    rt.step(ord("A"), None, oracle.FROZEN)
    acts = [np.float32(np.clip(np.float32(weights[n] - np.float32(0.1)), 0, 1)) for n in range(64)]
    key = lambda n: (-float(acts[n]), (n + 64 - tick % 64) % 64)
    expected = sorted(range(64), key=key)[:6]
    assert list(rt.read_list("active")) == expected
    cutoff = rt.read_f32("block_cutoff")[0]
    assert cutoff == acts[sorted(range(64), key=key)[6]]


# --- model.rs / config.rs --------------------------------------------------------------
def test_initialized_model_satisfies_canonical_parameter_bounds():  # model.rs:528-534
    Model.initialize(toml_test_config()).validate()


def test_validation_rejects_out_of_bounds_values():  # model.rs:517-526
    from leo_amd.native import LeoError

    m = Model.initialize(toml_test_config())
    m.threshold[0] = 2.01
    with pytest.raises(LeoError):
        m.validate()
    m = Model.initialize(toml_test_config())
    m.out_weight[0] = m.config.learning.weight_max + 0.01
    with pytest.raises(LeoError):
        m.validate()
