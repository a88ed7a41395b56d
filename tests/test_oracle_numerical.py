"""The numerical-rejection path of Runtime::step (crates/leo-core/src/runtime.rs:
apply_learning :1199-1316, the bias guard :1290-1300), pinned on the oracle.

A config with a finite but huge output learning rate and max_update (both
valid: config.rs:350-370 only asks for finite and positive) and a model whose
bias sits near the f32 maximum makes one bias update overflow. The reference
then writes the non-finite bias, returns its error, and skips everything
after it in that step: the later outputs' biases, the context projection,
the recurrent/input/inhibitory updates, the revision increment, homeostasis
and the statistics (runtime.rs:476-494). These tests check each of those
against a runtime that stopped one step earlier.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd.model import Model
from leo_amd.workload import WORKLOADS, workload_config

F32 = np.float32
TENSORS = ("threshold", "rec_weight", "in_weight", "out_weight", "ctx_keys", "ctx_emb", "ctx_obs", "ctx_out")


def overflow_model(olr: float, bias: float, end_bias: float):
    """Workload A's model with output_learning_rate = olr, max_update = 1e38,
    end_document_weight 4 and every byte output's bias at `bias` (END at
    end_bias)."""
    w = WORKLOADS["A"]
    cfg = workload_config(w)
    cfg.learning.output_learning_rate = olr
    cfg.learning.max_update = 1.0e38
    cfg.learning.end_document_weight = 4.0
    cfg.validate()
    m = Model.synthetic(cfg, topology=w.topology, weight_sigma=0.05)
    m.bias[:] = F32(bias)
    m.bias[256] = F32(end_bias)
    return m


def document(story: bytes):
    return [(256, story[0])] + [(story[i], story[i + 1]) for i in range(len(story) - 1)] + [(story[-1], 257)]


def test_bias_overflow_stops_the_step_after_writing_the_failing_bias(oracle):
    # olr 0.2e38: the first target ('a' = 97) has p = 1/257, so its bias gains
    # ~0.2e38 and overflows from 3.3e38 at the first supervised step
    m = overflow_model(0.2e38, 3.3e38, 3.3e38)
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    with pytest.raises(oracle.OracleError) as err:
        rt.step(256, ord("a"), oracle.TRAINING)
    assert err.value.code == oracle.ERR_NUMERICAL and err.value.message == "output bias 97 became non-finite"
    out = rt.model()
    p = rt.read_f32("probabilities")
    errors = p.copy()
    errors[97] -= F32(1.0)
    # outputs before the failing one learned, the failing one is +inf, the rest untouched
    for o in range(97):
        raw = F32(-F32(0.2e38) * F32(1.0) * errors[o])
        assert out.bias[o] == F32(m.bias[o] + np.clip(raw, F32(-1e38), F32(1e38)))
    assert np.isinf(out.bias[97]) and out.bias[97] > 0
    assert np.array_equal(out.bias[98:], m.bias[98:])
    # nothing after the bias: thresholds (homeostasis), synapses, the context
    # projection and embeddings, revision, statistics (the step's context slot
    # keys are allocated before learning, runtime.rs:641-677)
    for name in ("threshold", "rec_weight", "in_weight", "ctx_emb", "ctx_obs", "ctx_out"):
        assert np.array_equal(getattr(out, name), getattr(m, name)), name
    assert out.parameter_revision == m.parameter_revision
    assert out.statistics == m.statistics
    # only the output rows of the step's active neurons learned (they precede the bias)
    n = m.neuron_count
    changed = np.nonzero((out.out_weight != m.out_weight).reshape(257, n).any(axis=0))[0]
    assert set(changed.tolist()) <= set(rt.read_list("active").tolist())


def test_end_step_overflow_keeps_the_earlier_steps(oracle):
    # the END target learns with end_document_weight 4: 3.25e38 + 4 * 0.05e38 overflows,
    # while every byte target's +0.05e38 from 3.3e38 stays finite
    story = b"a" * 30 + b"\n"
    m = overflow_model(0.05e38, 3.3e38, 3.25e38)
    steps = document(story)
    before = oracle.OracleRuntime(m)
    before.begin_document()
    for s, t in steps[:-1]:
        before.step(s, t, oracle.TRAINING)
    rt = oracle.OracleRuntime(m)
    rt.begin_document()
    for s, t in steps[:-1]:
        rt.step(s, t, oracle.TRAINING)
    with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
        rt.step(*steps[-1], oracle.TRAINING)
    got, want = rt.model(), before.model()
    assert np.isinf(got.bias[256])
    for name in ("threshold", "rec_weight", "in_weight", "ctx_keys", "ctx_emb", "ctx_obs", "ctx_out"):
        assert np.array_equal(getattr(got, name), getattr(want, name)), name
    assert got.parameter_revision == want.parameter_revision
    assert got.statistics == want.statistics
    assert got.statistics["numerical_rejections"] == 0


def test_a_failing_story_lane_leaves_the_canonical_model(oracle):
    """training.rs:1669-1692: the lanes are forks; the first failing lane's
    error returns before the batch-end mean."""
    m = overflow_model(0.05e38, 3.3e38, 3.25e38)
    rt = oracle.OracleRuntime(m)
    with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
        rt.train_story_batch([b"a" * 30 + b"\n", b"b" * 20 + b"\n"], oracle.TRAINING, replay=True)
    out = rt.model()
    for name in TENSORS + ("bias",):
        assert np.array_equal(getattr(out, name), getattr(m, name)), name
    assert out.parameter_revision == m.parameter_revision and out.statistics == m.statistics


def test_replay_overflow_after_the_merge(oracle):
    """With END at 3.05e38 one END update (+0.2e38) stays finite in the story
    pass; the replay of the END range adds a second one on the merged model
    and overflows there: the merge and the replay steps before it stay."""
    m = overflow_model(0.05e38, 3.3e38, 3.05e38)
    for stories in ([b"a" * 30 + b"\n"], [b"a" * 30 + b"\n", b"a" * 20 + b"\n"]):
        rt = oracle.OracleRuntime(m)
        with pytest.raises(oracle.OracleError, match="output bias 256 became non-finite"):
            rt.train_story_batch(stories, oracle.TRAINING, replay=True)
        out = rt.model()
        story_targets = sum(len(s) + 1 for s in stories)
        assert out.statistics["training_targets"] > story_targets  # replay steps ran before the error
        assert np.isinf(out.bias[256])
