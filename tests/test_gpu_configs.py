"""GPU checks at the large benchmark configurations:

* C (131,072 units, fan-in 64 with power-law targets, 32 story lanes): one
  32-story batch cut to 48 bytes per story, replay on, against the oracle bit
  for bit; and a full-length 32-story batch run twice: identical and valid;

* D (1,048,576 units, fan-in 64, 64 story lanes): the bench's bounded CPU
  sample -- the batch's first 8 stories cut to 128 bytes, replay on -- against
  the CPU oracle bit for bit; and one full-size 64-story batch with replay
  (two resident lane groups, the grouped mean) run twice from the same model:
  identical models, a valid model, and the batch's counters consistent.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from leo_amd.workload import WORKLOADS, story_list, synthetic_stories, workload_model
from tests.helpers import assert_models_equal

pytestmark = pytest.mark.gpu


def _runtime(model, lanes):
    from leo_amd.runtime import HipRuntime

    return HipRuntime(model, device=0, max_lanes=lanes)


@pytest.fixture(scope="module")
def model_d():
    print("building the workload D model (1,048,576 units)", flush=True)
    return workload_model(WORKLOADS["D"])


@pytest.fixture(scope="module")
def stories_d():
    w = WORKLOADS["D"]
    data, offsets = synthetic_stories(w, w.lanes)
    return story_list(data, offsets)


def test_workload_d_bounded_sample_matches_oracle(require_gpu, oracle, model_d, stories_d):
    stories = [s[:128] for s in stories_d[:8]]
    print(f"workload D: 8 stories cut to 128 bytes ({sum(map(len, stories))} bytes), replay on", flush=True)
    cpu = oracle.OracleRuntime(model_d)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    print("oracle done", flush=True)
    gpu = _runtime(model_d, 8)
    try:
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert (grep.replay_segments, grep.replay_steps, grep.replay_prefix_steps) == \
            (crep.replay_segments, crep.replay_steps, crep.replay_prefix_steps)
        assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
        assert grep.merge_context_keys == crep.merge_context_keys
        assert grep.mean_loss == crep.mean_loss
        got = gpu.model()
    finally:
        gpu.close()
    assert_models_equal(got, cpu.model(), "workload D bounded sample")


def test_workload_d_full_batch_is_deterministic_and_valid(require_gpu, model_d, stories_d):
    stories = stories_d[:64]
    trained = sum(map(len, stories))
    finals, reports = [], []
    for run in range(2):
        print(f"workload D: 64-story batch ({trained} bytes) with replay, run {run}", flush=True)
        rt = _runtime(model_d, 64)
        try:
            resident = rt.resident_lanes
            rep, losses = rt.train_batch(stories, native.TRAINING, replay=True)
            finals.append(rt.model())
            reports.append(rep)
        finally:
            rt.close()
        print(f"run {run}: {resident} resident lanes, story {rep.story_seconds:.2f} s, merge "
              f"{rep.merge_seconds:.2f} s, replay {rep.replay_seconds:.2f} s", flush=True)
        assert len(losses) == 64 and all(len(l) == len(s) + 1 for l, s in zip(losses, stories))
        assert all(np.isfinite(l).all() and (l > 0).all() for l in losses)
    assert_models_equal(finals[0], finals[1], "two runs of the workload D batch")
    a, b = reports
    for field in ("mean_loss", "targets", "replay_segments", "replay_steps", "replay_prefix_steps",
                  "merge_fixed_parameter_updates", "merge_context_keys", "active_neurons_sum", "emitted_events"):
        assert getattr(a, field) == getattr(b, field), field
    assert a.stories == 64 and a.merge_workers == 64 and a.targets == trained + 64
    assert a.replay_steps > 0 and a.replay_prefix_steps > 0 and a.merge_fixed_parameter_updates > 0
    m = finals[0]
    m.validate()
    assert m.statistics["processed_bytes"] - model_d.statistics["processed_bytes"] >= trained
    assert m.parameter_revision > model_d.parameter_revision


# --- C: 131,072 units, fan-in 64 with power-law targets, 32 story lanes ----------------
@pytest.fixture(scope="module")
def model_c():
    print("building the workload C model (131,072 units, power-law targets)", flush=True)
    return workload_model(WORKLOADS["C"])


@pytest.fixture(scope="module")
def stories_c():
    w = WORKLOADS["C"]
    data, offsets = synthetic_stories(w, w.lanes)
    return story_list(data, offsets)


def test_workload_c_bounded_batch_matches_oracle(require_gpu, oracle, model_c, stories_c):
    stories = [s[:48] for s in stories_c[:32]]
    print(f"workload C: 32 stories cut to 48 bytes ({sum(map(len, stories))} bytes), replay on", flush=True)
    cpu = oracle.OracleRuntime(model_c)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    print("oracle done", flush=True)
    gpu = _runtime(model_c, 32)
    try:
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert (grep.replay_segments, grep.replay_steps, grep.replay_prefix_steps) == \
            (crep.replay_segments, crep.replay_steps, crep.replay_prefix_steps)
        assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
        assert grep.merge_context_keys == crep.merge_context_keys
        got = gpu.model()
    finally:
        gpu.close()
    assert_models_equal(got, cpu.model(), "workload C bounded batch")


def test_workload_c_full_batch_is_deterministic_and_valid(require_gpu, model_c, stories_c):
    stories = stories_c[:32]
    trained = sum(map(len, stories))
    finals, reports = [], []
    for run in range(2):
        print(f"workload C: 32-story batch ({trained} bytes) with replay, run {run}", flush=True)
        rt = _runtime(model_c, 32)
        try:
            rep, losses = rt.train_batch(stories, native.TRAINING, replay=True)
            finals.append(rt.model())
            reports.append(rep)
        finally:
            rt.close()
        assert all(np.isfinite(l).all() and (l > 0).all() for l in losses)
    assert_models_equal(finals[0], finals[1], "two runs of the workload C batch")
    for field in ("mean_loss", "targets", "replay_steps", "replay_prefix_steps", "merge_fixed_parameter_updates",
                  "merge_context_keys", "active_neurons_sum"):
        assert getattr(reports[0], field) == getattr(reports[1], field), field
    assert reports[0].replay_steps > 0 and reports[0].targets == trained + 32
    finals[0].validate()
