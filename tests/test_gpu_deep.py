"""Deep delivery buckets -- targets receiving more than 8 deliveries in one
tick, folded by the whole wave after a sort by delivery key -- against the
oracle, whose CPU executor delivers events one by one in order
(runtime.rs:605-639): power-law targets put hubs in the model, so buckets of
9-128 entries (ranked in registers) and of hundreds of entries (radix-sorted
through the shadow range) occur every tick. Story batches with replay and a
step-by-step document are compared bit for bit, and the telemetry shows both
sort paths ran."""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import assert_models_equal, small_redundant_config, story

pytestmark = pytest.mark.gpu


def _hub_model():
    # 2,048 units, fan-in 32 with power-law targets (exponent 1.6), up to 32
    # winners per block: the largest hubs take thousands of in-edges
    cfg = small_redundant_config(neurons=2048, synapses=32, fanout=64, per_block=32, dropout=0.0)
    cfg.dynamics.target_activity = 0.1
    cfg.validate()
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_POWER_LAW, exponent=1.6, weight_sigma=0.05)
    model.threshold[:] = np.float32(0.08)
    model.validate()
    indegree = np.bincount(model.rec_target.astype(np.int64), minlength=cfg.model.neuron_count)
    assert indegree.max() > 1000
    return model


def test_deep_buckets_match_oracle(require_gpu, oracle):
    from leo_amd.runtime import HipRuntime

    model = _hub_model()
    cpu = oracle.OracleRuntime(model)
    gpu = HipRuntime(model, device=0, max_lanes=4)
    try:
        print("deep buckets: document step by step", flush=True)
        text = story(71, 90)
        steps = [(BEGIN_DOCUMENT, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
        steps.append((text[-1], END_DOCUMENT))
        cpu.begin_document()
        gpu.begin_document()
        for i, (s, t) in enumerate(steps):
            c = cpu.step(s, t, oracle.TRAINING)
            g = gpu.step(s, t, native.TRAINING)
            assert g.loss == c.loss and g.active_neurons == c.active_neurons, f"step {i}"
        assert np.array_equal(gpu.read_state("branches"), cpu.read_f32("branches"))
        assert np.array_equal(gpu.read_state("membrane"), cpu.read_f32("membrane"))
        cpu.finish_document()
        gpu.finish_document()
        print("deep buckets: story batch with replay", flush=True)
        stories = [story(80 + k, 60 + 20 * k) for k in range(4)]
        crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert grep.replay_steps == crep.replay_steps
        assert_models_equal(gpu.model(), cpu.model(), "deep buckets")
        ks = gpu.kernel_stats()
        print(f"register folds {ks['deep_register_folds']}, radix folds {ks['deep_radix_folds']}", flush=True)
        assert ks["deep_register_folds"] > 0 and ks["deep_radix_folds"] > 0
    finally:
        gpu.close()
