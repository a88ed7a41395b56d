"""GPU parity: the HIP path (through the C-ABI) against the CPU oracle on the
same seeded inputs. Worklists, masks and model tensors are compared bit for
bit; the HIP kernels reproduce the CPU executor's FP32 operation order."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import (assert_models_equal, causal_model, small_redundant_config, story, toml_test_config)

pytestmark = pytest.mark.gpu


def _runtime(model, max_lanes=8):
    from leo_amd.runtime import HipRuntime

    return HipRuntime(model, device=0, max_lanes=max_lanes)


def _document_steps(text: bytes):
    steps = [(BEGIN_DOCUMENT, text[0])]
    steps += [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    return steps


STATE_COMPARE = ["membrane", "activation", "fatigue", "branches", "adapt0", "adapt1", "adapt2",
                 "rec_bs", "rec_ms", "rec_fs", "rec_as0", "rec_as1", "rec_as2", "rec_e",
                 "in_bs", "in_ms", "in_fs", "in_as0", "in_as1", "in_as2", "in_e", "probabilities"]


def _compare_step_state(gpu, cpu, label):
    for lst, name in ((native.LIST_ACTIVE, "active"), (native.LIST_TOUCHED, "touched"),
                      (native.LIST_ELIGIBLE_REC, "eligible_rec"), (native.LIST_ELIGIBLE_IN, "eligible_in")):
        g = gpu.read_list(lst)
        c = cpu.read_list(name)
        assert np.array_equal(g, c), f"{label}: {name} list differs: gpu {g[:16]} cpu {c[:16]}"
    for name in STATE_COMPARE:
        g = gpu.read_state(name)
        c = cpu.read_f32(name)
        assert np.array_equal(g, c), f"{label}: {name} differs at {np.nonzero(g != c)[0][:8]}"


@pytest.mark.parametrize("make", ["test_toml", "small_redundant"])
def test_step_by_step_parity(require_gpu, oracle, make):
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config()
    model = Model.initialize(cfg)
    if make == "test_toml":
        model.threshold[:] = 0.12  # make the tiny model active from the first bytes
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    cpu.begin_document()
    gpu.begin_document()
    text = story(7, 40)
    for i, (sym, tgt) in enumerate(_document_steps(text)):
        print(f"step {i} symbol {sym} target {tgt}", flush=True)
        cm = cpu.step(sym, tgt, oracle.TRAINING)
        gm = gpu.step(sym, tgt, native.TRAINING)
        assert gm.active_neurons == cm.active_neurons, (i, gm.active_neurons, cm.active_neurons)
        assert gm.predicted_symbol == cm.predicted_symbol, i
        assert gm.loss == cm.loss, (i, gm.loss, cm.loss)
        assert gm.eligible_recurrent_synapses == cm.eligible_recurrent_synapses, i
        assert gm.context_cells == cm.context_cells and gm.context_probes == cm.context_probes, i
        assert gm.population_inhibition == cm.population_inhibition, i
        _compare_step_state(gpu, cpu, f"step {i}")
    assert_models_equal(gpu.model(), cpu.model(), "after document")
    gpu.close()


def test_reset_after_dropped_slots_parity(require_gpu, oracle):
    # slots that left the eligible list keep sub-epsilon values; the reset
    # between documents clears them from their marks, and the second
    # document's traces match the oracle's dense reset step by step (a large
    # epsilon makes slots leave the list within the first document)
    cfg = small_redundant_config()
    cfg = dataclasses.replace(cfg, learning=dataclasses.replace(cfg.learning, eligibility_epsilon=0.03))
    model = Model.initialize(cfg)
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    dropped = False
    for doc, (seed, n) in enumerate(((41, 60), (42, 40))):
        cpu.begin_document()
        gpu.begin_document()
        previous = 0
        for i, (sym, tgt) in enumerate(_document_steps(story(seed, n))):
            print(f"document {doc} step {i}", flush=True)
            cm = cpu.step(sym, tgt, oracle.TRAINING)
            gm = gpu.step(sym, tgt, native.TRAINING)
            assert gm.loss == cm.loss, (doc, i)
            dropped |= doc == 0 and gm.eligible_recurrent_synapses < previous
            previous = gm.eligible_recurrent_synapses
            if doc == 1:
                _compare_step_state(gpu, cpu, f"document {doc} step {i}")
        cpu.finish_document()
        gpu.finish_document()
    assert dropped, "the first document never dropped an eligible slot"
    assert_models_equal(gpu.model(), cpu.model(), "after two documents")
    gpu.close()


def test_causal_model_delay_credit(require_gpu, oracle):
    for delay in (1, 2, 4, 8):
        model = causal_model(delay)
        cpu = oracle.OracleRuntime(model)
        gpu = _runtime(model)
        for rt in (cpu, gpu):
            rt.begin_document()
        steps = [(ord("A"), ord("Y"))] + [(ord("B"), ord("Y"))] * delay
        for sym, tgt in steps:
            cpu.step(sym, tgt, oracle.TRAINING)
        gpu.training_step_batch(steps, native.TRAINING)
        g, c = gpu.model(), cpu.model()
        assert g.rec_weight[0] == c.rec_weight[0] != 0.5
        assert_models_equal(g, c, f"delay {delay}")
        gpu.close()


@pytest.mark.parametrize("make", ["test_toml", "small_redundant"])
def test_document_batch_parity(require_gpu, oracle, make):
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config()
    model = Model.initialize(cfg)
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    for k in range(3):
        text = story(100 + k, 120)
        cpu.begin_document()
        gpu.begin_document()
        steps = _document_steps(text)
        cms = [cpu.step(s, t, oracle.TRAINING) for s, t in steps]
        gms = gpu.training_step_batch(steps, native.TRAINING)
        assert [m.loss for m in gms] == [m.loss for m in cms]
        assert [m.active_neurons for m in gms] == [m.active_neurons for m in cms]
        cpu.finish_document()
        gpu.finish_document()
    assert_models_equal(gpu.model(), cpu.model(), make)
    gpu.close()


@pytest.mark.parametrize("make", ["test_toml", "small_redundant"])
def test_story_batch_merge_parity(require_gpu, oracle, make):
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config()
    model = Model.initialize(cfg)
    stories = [story(200 + k, 60 + 17 * k) for k in range(4)]
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=False)
    grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=False)
    for a, b in zip(gloss, closs):
        assert np.array_equal(a, b)
    assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
    assert grep.merge_context_keys == crep.merge_context_keys
    assert grep.mean_loss == crep.mean_loss
    assert_models_equal(gpu.model(), cpu.model(), make)
    gpu.close()


@pytest.mark.parametrize("make", ["test_toml", "small_redundant"])
def test_train_batch_with_replay_parity(require_gpu, oracle, make):
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config()
    model = Model.initialize(cfg)
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    batches = [[story(300, 90)], [story(301 + k, 50 + 11 * k) for k in range(3)]]
    for batch in batches:
        crep, _ = cpu.train_story_batch(batch, oracle.TRAINING, replay=True)
        grep, _ = gpu.train_batch(batch, native.TRAINING, replay=True)
        assert grep.replay_segments == crep.replay_segments
        assert grep.replay_steps == crep.replay_steps
        assert grep.replay_prefix_steps == crep.replay_prefix_steps
    assert_models_equal(gpu.model(), cpu.model(), make)
    gpu.close()


@pytest.mark.parametrize("make,resident", [("test_toml", 2), ("small_redundant", 2), ("small_redundant", 4)])
def test_story_batch_in_lane_groups_parity(require_gpu, oracle, make, resident, monkeypatch):
    # 5 stories with 2 resident lanes: groups 2+2+1 accumulate the lane-ordered
    # f64 mean and the keyed context merge across groups; with 4, the two
    # groups the capacity needs take 3+2 stories (split evenly, not 4+1)
    monkeypatch.setenv("LEO_HIP_RESIDENT_LANES", str(resident))
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config()
    model = Model.initialize(cfg)
    stories = [story(500 + k, 40 + 13 * k) for k in range(5)]
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    assert gpu.resident_lanes == resident
    for replay in (False, True):
        crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=replay)
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=replay)
        for a, b in zip(gloss, closs):
            assert np.array_equal(a, b)
        assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
        assert grep.merge_context_keys == crep.merge_context_keys
        assert grep.mean_loss == crep.mean_loss
    assert_models_equal(gpu.model(), cpu.model(), make)
    gpu.close()


def test_chunked_launches_and_agent_barriers_parity(require_gpu, oracle, monkeypatch):
    # schedules split into launches of 7 steps, and the agent-scope barrier
    # fallback, give the same bits as one launch with XCD-local barriers
    monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", "7")
    monkeypatch.setenv("LEO_HIP_AGENT_SYNC", "1")
    cfg = small_redundant_config()
    model = Model.initialize(cfg)
    stories = [story(600 + k, 50 + 9 * k) for k in range(3)]
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
    for a, b in zip(gloss, closs):
        assert np.array_equal(a, b)
    assert grep.replay_steps == crep.replay_steps
    assert_models_equal(gpu.model(), cpu.model(), "chunked")
    assert gpu.kernel_stats()["launches"] > 10
    gpu.close()


@pytest.mark.parametrize("wgs", ["1", "2"])
def test_replay_with_few_workgroups_parity(require_gpu, oracle, monkeypatch, wgs):
    # one workgroup per lane (selection, context and readout on the same
    # workgroup) and two (one selecting, one resolving the context): the
    # frozen replay prefixes run the fused steps that start the next tick
    # early on both layouts
    monkeypatch.setenv("LEO_HIP_WGS_PER_LANE", wgs)
    model = Model.initialize(small_redundant_config())
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    stories = [story(700 + k, 60 + 13 * k) for k in range(3)]
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
    for a, b in zip(gloss, closs):
        assert np.array_equal(a, b)
    assert grep.replay_prefix_steps == crep.replay_prefix_steps > 0
    assert grep.mean_loss == crep.mean_loss
    assert_models_equal(gpu.model(), cpu.model(), f"{wgs} workgroups")
    gpu.close()


@pytest.mark.parametrize("wgs", ["1", "2"])
def test_dense_touch_multi_window_parity(require_gpu, oracle, monkeypatch, wgs):
    # one or two workgroups per lane make every selecting wave own several
    # blocks, and an input fan-out of three quarters of the units touches well
    # over a window's 256 entries per wave and step: the phase-2 fold and block
    # ranking run in several windows of whole blocks
    monkeypatch.setenv("LEO_HIP_WGS_PER_LANE", wgs)
    cfg = small_redundant_config(neurons=4096, synapses=16, fanout=3072, per_block=8)
    model = Model.initialize(cfg)
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    cpu.begin_document()
    gpu.begin_document()
    text = story(31, 24)
    for i, (sym, tgt) in enumerate(_document_steps(text)):
        print(f"wgs {wgs} step {i} symbol {sym} target {tgt}", flush=True)
        cm = cpu.step(sym, tgt, oracle.TRAINING)
        gm = gpu.step(sym, tgt, native.TRAINING)
        assert gm.active_neurons == cm.active_neurons, (i, gm.active_neurons, cm.active_neurons)
        assert gm.loss == cm.loss, (i, gm.loss, cm.loss)
        _compare_step_state(gpu, cpu, f"step {i}")
    stats = gpu.kernel_stats()
    # more touched neurons per wave than one window holds
    assert stats["touched"] / max(stats["lane_steps"], 1) > int(wgs) * 4 * 256
    assert_models_equal(gpu.model(), cpu.model(), "after document")
    gpu.close()


def _bitwise_weights_equal(got, want, label):
    # np.array_equal treats -0.0 and +0.0 alike; the bit patterns must match too
    for name in ("rec_weight", "in_weight"):
        g = getattr(got, name).view(np.uint32)
        c = getattr(want, name).view(np.uint32)
        assert np.array_equal(g, c), f"{label}: {name} bits differ at {np.nonzero(g != c)[0][:8]}"


@pytest.mark.parametrize("negative_zero", [False, True])
def test_learning_slots_and_negative_zero_weights(require_gpu, oracle, negative_zero):
    # Learning slots are the kept eligible slots with nonzero eligibility;
    # a -0.0 recurrent or input weight switches every kept slot back to a
    # learning slot, and the weights must then match the oracle bit for bit
    # (an update with zero eligibility turns an excitatory -0.0 into +0.0).
    cfg = small_redundant_config()
    model = Model.initialize(cfg)
    if negative_zero:
        S = cfg.model.synapses_per_neuron
        excitatory = np.nonzero(model.neuron_type == 0)[0][:64]
        for n in excitatory:
            model.rec_weight[n * S:(n + 1) * S] = np.float32(-0.0)
        model.in_weight[::3] = np.float32(-0.0)
        model.validate()
    cpu = oracle.OracleRuntime(model)
    gpu = _runtime(model)
    try:
        for batch in ([story(700, 120)], [story(701 + k, 60 + 9 * k) for k in range(3)]):
            crep, closs = cpu.train_story_batch(batch, oracle.TRAINING, replay=True)
            grep, gloss = gpu.train_batch(batch, native.TRAINING, replay=True)
            for a, b in zip(gloss, closs):
                assert np.array_equal(a, b)
            assert grep.replay_steps == crep.replay_steps
        got, want = gpu.model(), cpu.model()
        assert_models_equal(got, want, f"negative zero {negative_zero}")
        _bitwise_weights_equal(got, want, f"negative zero {negative_zero}")
        stats = gpu.kernel_stats()
        assert stats["learning_slots"] > 0
        if not negative_zero:
            # far fewer learning slots than kept eligible slots
            assert stats["learning_slots"] < stats["kept_rec"] + stats["kept_in"]
    finally:
        gpu.close()
