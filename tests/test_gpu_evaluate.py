"""Frozen evaluation (leo_hip_evaluate, validation.rs:65-154) against the
oracle: one CPU runtime scoring the stories in order -- begin_document, the
document steps frozen with their targets, finish_document -- accumulated as
record_evaluation_step and ActivityDiagnostics::record do (validation.rs:137-154,
metrics.rs:27-69). The HIP path scores the stories on parallel lanes; every
step loss, the f64 sums (loss, population inhibition, context loss gain), the
counters and accuracy must be identical, the model untouched, and the
canonical runtime's tick advanced exactly as the sequential loop advances it
(checked by training a document afterwards on both)."""
from __future__ import annotations

import math

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import assert_models_equal, small_redundant_config, story, toml_test_config

pytestmark = pytest.mark.gpu


def _document_steps(text: bytes):
    steps = [(BEGIN_DOCUMENT, text[0])]
    steps += [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    return steps


def _oracle_evaluate(cpu, oracle, stories):
    rep = dict(targets=0, processed_stories=0, processed_bytes=0, steps=0, active_neurons_sum=0,
               active_neurons_peak=0, emitted_events=0, suprathreshold_sum=0, block_selected_sum=0,
               cap_clipped_sum=0, cap_hit_steps=0, population_inhibition_sum=0.0,
               population_inhibition_peak=np.float32(0.0), eligibility_sum=0.0, eligibility_count=0,
               context_cells_sum=0, context_probes_sum=0, context_applied_steps=0, context_loss_gain_sum=0.0,
               output_madds_sum=0)
    loss_sum, correct, losses = 0.0, 0, []
    for text in stories:
        if not text:
            continue
        cpu.begin_document()
        story_losses = []
        for symbol, target in _document_steps(text):
            m = cpu.step(symbol, target, oracle.FROZEN)
            story_losses.append(np.float32(m.loss))
            loss_sum += float(np.float32(m.loss))
            rep["targets"] += 1
            correct += 1 if m.predicted_symbol == target else 0
            rep["steps"] += 1
            rep["active_neurons_sum"] += m.active_neurons
            rep["active_neurons_peak"] = max(rep["active_neurons_peak"], m.active_neurons)
            rep["emitted_events"] += m.emitted_events
            rep["suprathreshold_sum"] += m.suprathreshold_neurons
            rep["block_selected_sum"] += m.block_selected_neurons
            rep["cap_clipped_sum"] += m.global_cap_clipped_neurons
            rep["cap_hit_steps"] += 1 if m.global_cap_clipped_neurons > 0 else 0
            rep["population_inhibition_sum"] += float(np.float32(m.population_inhibition))
            rep["population_inhibition_peak"] = max(rep["population_inhibition_peak"],
                                                    np.float32(m.population_inhibition))
            eligible = m.eligible_recurrent_synapses + m.eligible_input_synapses
            rep["eligibility_sum"] += float(np.float32(m.mean_abs_eligibility)) * eligible
            rep["eligibility_count"] += eligible
            rep["context_cells_sum"] += m.context_cells
            rep["context_probes_sum"] += m.context_probes
            rep["context_applied_steps"] += 1 if m.context_applied else 0
            rep["context_loss_gain_sum"] += float(np.float32(m.context_loss_gain))
            rep["output_madds_sum"] += m.output_madds
        cpu.finish_document()
        losses.append(np.array(story_losses, dtype=np.float32))
        rep["processed_stories"] += 1
        rep["processed_bytes"] += len(text)
    rep["loss"] = loss_sum / max(rep["targets"], 1)
    rep["bits_per_byte"] = rep["loss"] / math.log(2.0)
    rep["accuracy"] = correct / max(rep["targets"], 1)
    return rep, losses


@pytest.mark.parametrize("make", ["test_toml", "small_redundant"])
def test_frozen_evaluation_matches_sequential_oracle(require_gpu, oracle, make, monkeypatch):
    from leo_amd.runtime import HipRuntime

    # 2 resident lanes: the stories run in groups, each lane at its own tick
    monkeypatch.setenv("LEO_HIP_RESIDENT_LANES", "2")
    cfg = toml_test_config() if make == "test_toml" else small_redundant_config(dropout=0.5)
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_UNIFORM, weight_sigma=0.05) if make != "test_toml" \
        else Model.initialize(cfg)
    if make == "test_toml":
        model.threshold[:] = 0.12
    cpu = oracle.OracleRuntime(model)
    gpu = HipRuntime(model, device=0, max_lanes=4)
    try:
        # a trained model first (context slots to score against), then evaluate
        warm = [story(900, 110), story(901, 70)]
        cpu.train_story_batch(warm, oracle.TRAINING, replay=False)
        gpu.train_batch(warm, native.TRAINING, replay=False)
        trained = cpu.model()
        stories = [story(910 + k, 40 + 17 * k) for k in range(5)]
        stories.insert(2, b"")  # skipped, as validation.rs:86-88
        print(f"evaluate {make}: {len(stories)} stories", flush=True)
        want, want_losses = _oracle_evaluate(cpu, oracle, stories)
        got, got_losses = gpu.evaluate(stories)
        assert len(got_losses) == len(want_losses) == 5
        for i, (g, c) in enumerate(zip(got_losses, want_losses)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        for key, value in want.items():
            if key == "population_inhibition_peak":
                assert np.float32(got[key]) == value, key
            else:
                assert got[key] == value, (key, got[key], value)
        assert got["neuron_count"] == cfg.model.neuron_count
        assert got["context_applied_steps"] > 0 and got["context_loss_gain_sum"] != 0.0
        # evaluation is read-only
        assert_models_equal(gpu.model(), trained, "after evaluation")
        # the tick advanced as the sequential loop's: a document trained next agrees
        after = story(950, 60)
        cpu.train_story_batch([after], oracle.TRAINING, replay=False)
        gpu.train_batch([after], native.TRAINING, replay=False)
        assert_models_equal(gpu.model(), cpu.model(), "document after evaluation")
    finally:
        gpu.close()
