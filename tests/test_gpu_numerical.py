"""The numerical-rejection path on the device against the oracle, through the
C-ABI (runtime.rs:1290-1300: the bias guard; the GPU adapter turns sticky
device codes into errors, cuda.rs:9093-9103).

A finite but huge output learning rate and max_update with the bias near the
f32 maximum (tests/test_oracle_numerical.py pins what the reference does
then) make one bias update overflow. Each case compares the status
(LEO_ERR_NUMERICAL and the reference's message), numerical_rejections, the
statistics, the revision and every learned tensor after the error with the
oracle:

* one lane, a training step batch: the END step overflows, in one launch and
  with the schedule cut into launches of 8 steps;
* the first supervised step overflows at output 97 (the bias up to it is
  written, the rest of the step is skipped), then the runtime takes new
  frozen steps after a reset exactly as the oracle does;
* a story batch whose lanes fail in the story pass: the canonical model is
  untouched;
* a failure inside the replay after the batch-end mean (one story in place
  and two story lanes), with replay launches of 4 steps so that launches are
  queued behind the failing one: they must change nothing.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from tests.helpers import assert_models_equal
from tests.test_oracle_numerical import document, overflow_model

pytestmark = pytest.mark.gpu

A_STORY = b"a" * 30 + b"\n"


def _runtime(model, lanes=1):
    from leo_amd.runtime import HipRuntime

    return HipRuntime(model, device=0, max_lanes=lanes)


def _expect_numerical(call, message):
    with pytest.raises(native.LeoError) as err:
        call()
    assert err.value.code == native.ERR_NUMERICAL, err.value
    assert message in err.value.message, err.value.message


@pytest.mark.parametrize("launch_steps", [None, 8])
def test_step_batch_end_overflow_matches_oracle(require_gpu, oracle, monkeypatch, launch_steps):
    if launch_steps:
        monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", str(launch_steps))
    model = overflow_model(0.05e38, 3.3e38, 3.25e38)
    steps = document(A_STORY)
    print(f"numerical: END overflow in a {len(steps)}-step batch, launches of {launch_steps or 'any'} steps",
          flush=True)
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
        for s, t in steps:
            cpu.step(s, t, oracle.TRAINING)
    gpu = _runtime(model)
    try:
        gpu.begin_document()
        _expect_numerical(lambda: gpu.training_step_batch(steps, native.TRAINING), "output bias 256 became non-finite")
        got = gpu.model()
        assert_models_equal(got, cpu.model(), "after the END overflow")
        assert got.statistics["numerical_rejections"] == 0
        assert np.isinf(got.bias[256])
    finally:
        gpu.close()


def test_first_step_overflow_then_frozen_steps_match_oracle(require_gpu, oracle):
    model = overflow_model(0.2e38, 3.3e38, 3.3e38)
    print("numerical: overflow at output 97 on the first supervised step, then frozen steps", flush=True)
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    with pytest.raises(oracle.OracleError, match="output bias 97 became non-finite"):
        cpu.step(256, ord("a"), oracle.TRAINING)
    gpu = _runtime(model)
    try:
        gpu.begin_document()
        _expect_numerical(lambda: gpu.training_step_batch([(256, ord("a"))], native.TRAINING),
                          "output bias 97 became non-finite")
        assert_models_equal(gpu.model(), cpu.model(), "after the overflow at output 97")
        # the runtime is usable again after a reset: the sticky word was reported
        cpu.begin_document()
        gpu.begin_document()
        for s in b"abc":
            cpu.step(s, None, oracle.FROZEN)
            gpu.step(s, None, native.FROZEN)
            assert np.array_equal(gpu.probabilities(), cpu.read_f32("probabilities"))
            assert np.array_equal(np.sort(gpu.active_neurons()), np.sort(cpu.read_list("active")))
    finally:
        gpu.close()


def test_story_batch_lane_overflow_leaves_canonical(require_gpu, oracle):
    model = overflow_model(0.05e38, 3.3e38, 3.25e38)
    stories = [A_STORY, b"b" * 20 + b"\n"]
    print("numerical: both story lanes overflow at END", flush=True)
    cpu = oracle.OracleRuntime(model)
    with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
        cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    gpu = _runtime(model, lanes=2)
    try:
        _expect_numerical(lambda: gpu.train_batch(stories, native.TRAINING, replay=True),
                          "output bias 256 became non-finite")
        assert_models_equal(gpu.model(), cpu.model(), "story batch")
        assert_models_equal(gpu.model(), model, "story batch vs the model before it")
    finally:
        gpu.close()


@pytest.mark.parametrize("stories", [[A_STORY], [A_STORY, b"a" * 20 + b"\n"]], ids=["in_place", "two_lanes"])
def test_replay_overflow_matches_oracle(require_gpu, oracle, monkeypatch, stories):
    monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", "4")
    model = overflow_model(0.05e38, 3.3e38, 3.05e38)
    print(f"numerical: replay overflow after the merge, {len(stories)} stories, replay launches of 4 steps",
          flush=True)
    cpu = oracle.OracleRuntime(model)
    with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
        cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    gpu = _runtime(model, lanes=len(stories))
    try:
        _expect_numerical(lambda: gpu.train_batch(stories, native.TRAINING, replay=True),
                          "output bias 256 became non-finite")
        got, want = gpu.model(), cpu.model()
        assert want.statistics["training_targets"] > sum(len(s) + 1 for s in stories)
        assert_models_equal(got, want, "after the replay overflow")
    finally:
        gpu.close()
