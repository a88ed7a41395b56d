"""GPU checks at the benchmark's own workload (B: 16,384 units, S 32, F 128,
8 story lanes) and of the streaming replay entry point:

* one logical batch with replay against the CPU oracle, bit for bit;
* determinism: two fresh runtimes produce identical models;
* 8 lanes of one story (fully overlapping changed sets) against the oracle;
* replay_streaming_batch against the oracle stepped position by position.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from leo_amd.workload import WORKLOADS, synthetic_stories, workload_model
from tests.helpers import assert_models_equal, story, toml_test_config

pytestmark = pytest.mark.gpu

def _stories(count, offset=0):
    data, offsets = synthetic_stories(WORKLOADS["B"], count, offset)
    return [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(count)]


def _runtime(model, lanes):
    from leo_amd.runtime import HipRuntime

    return HipRuntime(model, device=0, max_lanes=lanes)


def test_workload_b_batch_with_replay_matches_oracle(require_gpu, oracle):
    model = workload_model(WORKLOADS["B"])
    stories = _stories(8)
    print(f"workload B: 8 stories, {sum(map(len, stories))} bytes, replay on", flush=True)
    cpu = oracle.OracleRuntime(model)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    gpu = _runtime(model, 8)
    try:
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert (grep.replay_segments, grep.replay_steps, grep.replay_prefix_steps) == \
            (crep.replay_segments, crep.replay_steps, crep.replay_prefix_steps)
        assert grep.mean_loss == crep.mean_loss
        assert_models_equal(gpu.model(), cpu.model(), "workload B batch")
    finally:
        gpu.close()


def test_workload_b_is_deterministic(require_gpu):
    model = workload_model(WORKLOADS["B"])
    stories = _stories(8, offset=8)
    finals = []
    for run in range(2):
        print(f"workload B determinism run {run}", flush=True)
        rt = _runtime(model, 8)
        try:
            rt.train_batch(stories, native.TRAINING, replay=True)
            finals.append(rt.model())
        finally:
            rt.close()
    assert_models_equal(finals[0], finals[1], "two runs")


def test_workload_b_identical_lanes_match_oracle(require_gpu, oracle):
    # every lane changes the same parameters: the merge's changed sets overlap fully
    model = workload_model(WORKLOADS["B"])
    stories = _stories(1, offset=16) * 8
    print("workload B: 8 lanes of one story, replay off", flush=True)
    cpu = oracle.OracleRuntime(model)
    crep, _ = cpu.train_story_batch(stories, oracle.TRAINING, replay=False)
    gpu = _runtime(model, 8)
    try:
        grep, _ = gpu.train_batch(stories, native.TRAINING, replay=False)
        assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
        assert grep.merge_context_keys == crep.merge_context_keys
        assert_models_equal(gpu.model(), cpu.model(), "identical lanes")
    finally:
        gpu.close()


def test_replay_streaming_batch_matches_stepwise_oracle(require_gpu, oracle):
    cfg = toml_test_config()
    model = Model.initialize(cfg)
    model.threshold[:] = 0.12
    text = story(11, 60)
    steps = [(BEGIN_DOCUMENT, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    # supervise positions 20..29 and 45..52, advance the rest frozen
    timeline = [(s, t if (20 <= i < 30 or 45 <= i < 53) else None) for i, (s, t) in enumerate(steps)]
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    want = []
    for s, t in timeline:
        m = cpu.step(s, t, oracle.TRAINING if t is not None else oracle.FROZEN)
        if t is not None:
            want.append(m)
    gpu = _runtime(model, 1)
    try:
        gpu.begin_document()
        got = gpu.replay_streaming_batch(timeline, native.TRAINING)
        assert len(got) == len(want) == 18
        for g, c in zip(got, want):
            assert g.loss == c.loss and g.active_neurons == c.active_neurons
            assert g.predicted_symbol == c.predicted_symbol
        assert_models_equal(gpu.model(), cpu.model(), "streaming replay")
    finally:
        gpu.close()
