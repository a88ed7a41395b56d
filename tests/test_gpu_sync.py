"""The Rust coordinator's synchronisation sequences, replayed through the C-ABI
against the oracle's train_story_batch:

* single story (training.rs:1548-1563): tracking on, the in-place document
  pass and its replay through the step primitives, then parameter_changes,
  synchronize_model on the host mirror, PackedSparseModelUpdate::from_model
  on the mirror and synchronize_packed_model;
* logical batch (training.rs:1585-1649): training_story_batch (merged on
  return), tracking restarted, the batch's replay, then the same packing.

After each sequence the host mirror -- updated only through the sparse
synchronisation -- and the device model both equal the oracle's model bit for
bit. The packed entries are also checked for their tracking semantics and
index checks.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import assert_models_equal, small_redundant_config, story

pytestmark = pytest.mark.gpu


def _document_steps(text: bytes):
    steps = [(BEGIN_DOCUMENT, text[0])]
    steps += [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    return steps


def _replay_classic(gpu, text: bytes, ranges, permission):
    """Classic bounded-surprise replay of one story through the step primitives
    (training.rs:162-255): per range a reset, the frozen prefix, the supervised
    targets; a reset after the last range."""
    n = len(text)
    ranges = list(ranges)
    for i, (rs, re) in enumerate(ranges):
        if rs >= re or rs > n:
            continue
        end = min(re, n + 1)
        gpu.begin_document()
        nxt = rs
        if nxt > 0:
            gpu.advance_frozen_batch([(BEGIN_DOCUMENT, None)] + [(text[k], None) for k in range(nxt - 1)])
        supervised = []
        if nxt == 0:
            supervised.append((BEGIN_DOCUMENT, text[0]))
            nxt = 1
        for p in range(nxt, end):
            supervised.append((text[p - 1], text[p] if p < n else END_DOCUMENT))
        gpu.training_step_batch(supervised, permission)
        if i + 1 == len(ranges):
            gpu.reset_transient_state()


def _pack_and_sync(gpu, mirror):
    from leo_amd.runtime import PackedUpdate

    changes = gpu.parameter_changes()
    gpu.synchronize_model(mirror)
    update = PackedUpdate.from_model(mirror, changes)
    gpu.synchronize_packed_model(update)
    return changes


def test_coordinator_sync_sequences_match_oracle(require_gpu, oracle):
    from leo_amd.runtime import HipRuntime

    cfg = small_redundant_config()
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_UNIFORM, weight_sigma=0.05)
    fraction, segment = cfg.replay.fraction, cfg.replay.segment_bytes
    cpu = oracle.OracleRuntime(model)
    gpu = HipRuntime(model, device=0, max_lanes=4)
    mirror = model.copy()
    try:
        # single story: the canonical runtime trains in place
        text = story(41, 150)
        print("sync: single-story sequence", flush=True)
        cpu.train_story_batch([text], oracle.TRAINING, replay=True)
        gpu.enable_parameter_tracking()
        gpu.begin_document()
        metrics = gpu.training_step_batch(_document_steps(text), native.TRAINING)
        gpu.finish_document()
        losses = [m.loss for m in metrics]
        _replay_classic(gpu, text, oracle.select_replay_ranges(losses, fraction, segment), native.TRAINING)
        changes = _pack_and_sync(gpu, mirror)
        assert changes["recurrent_weight"].size > 0
        assert_models_equal(mirror, cpu.model(), "mirror after the single-story sequence")
        assert_models_equal(gpu.model(), cpu.model(), "device after the single-story sequence")
        # tracking ended with the packed synchronisation
        assert all(gpu.parameter_changes()[k].size == 0 for k in ("threshold", "recurrent_weight"))

        # logical batch: merged on return, then replay with tracking
        stories = [story(50 + k, 70 + 15 * k) for k in range(4)]
        print("sync: logical-batch sequence", flush=True)
        cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
        _, per_story = gpu.training_story_batch(stories, native.TRAINING)
        gpu.enable_parameter_tracking()
        for text, story_losses in zip(stories, per_story):
            ranges = oracle.select_replay_ranges(list(story_losses), fraction, segment)
            _replay_classic(gpu, text, ranges, native.TRAINING)
        _pack_and_sync(gpu, mirror)
        want = cpu.model()
        assert_models_equal(mirror, want, "mirror after the batch sequence")
        assert_models_equal(gpu.model(), want, "device after the batch sequence")
    finally:
        gpu.close()


def test_packed_entries_tracking_and_checks(require_gpu):
    from leo_amd.runtime import HipRuntime, PackedUpdate

    cfg = small_redundant_config()
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_UNIFORM, weight_sigma=0.05)
    gpu = HipRuntime(model, device=0, max_lanes=2)
    try:
        gpu.enable_parameter_tracking()
        gpu.begin_document()
        gpu.training_step_batch(_document_steps(story(60, 80)), native.TRAINING)
        mirror = model.copy()
        changes = gpu.parameter_changes()
        gpu.synchronize_model(mirror)
        # a hand-made change to the mirror, committed: the device takes it and
        # tracking stays on
        slot = int(changes["recurrent_weight"][0])
        mirror.rec_weight[slot] = np.float32(0.0) if model.neuron_type[slot // cfg.model.synapses_per_neuron] else \
            np.float32(0.0625)
        update = PackedUpdate.from_model(mirror, changes)
        gpu.commit_packed_host_model(update)
        assert gpu.model().rec_weight[slot] == mirror.rec_weight[slot]
        assert gpu.parameter_changes()["recurrent_weight"].size == changes["recurrent_weight"].size
        # an index outside the model is refused before anything is written
        bad = PackedUpdate.from_model(mirror, changes)
        bad.threshold_indices = np.array([cfg.model.neuron_count], dtype=np.uint32)
        bad.threshold_values = np.array([0.5], dtype=np.float32)
        with pytest.raises(native.LeoError) as err:
            gpu.synchronize_packed_model(bad)
        assert err.value.code == native.ERR_INVALID_ARGUMENT
        # synchronize_packed_model ends tracking
        gpu.synchronize_packed_model(update)
        assert gpu.parameter_changes()["recurrent_weight"].size == 0
        assert_models_equal(gpu.model(), mirror, "after the packed synchronisation")
    finally:
        gpu.close()
