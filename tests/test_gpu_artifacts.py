"""End to end through the persistent artifacts on the GPU: stories come from a
LEODATA1 dataset, the trained model goes through a PSCLS100 checkpoint, and a
fresh runtime resumes from the checkpoint -- each stage against the CPU
oracle bit for bit (the flow of `leo train` with checkpoints,
crates/leo-cli/src/training.rs, over crates/leo-data and crates/leo-format).
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import formats, native
from leo_amd.workload import WORKLOADS, synthetic_stories, workload_model
from tests.helpers import assert_models_equal

pytestmark = pytest.mark.gpu


def _write_dataset(tmp_path, count):
    data, offsets = synthetic_stories(WORKLOADS["A"], count)
    b, idx = tmp_path / "train.bytes", tmp_path / "train.idx"
    b.write_bytes(data.tobytes())
    entries = [formats.StoryIndex(int(offsets[i]), int(offsets[i + 1] - offsets[i])) for i in range(count)]
    formats.write_index(idx, b, entries, formats.digest_bytes(b"synthetic workload A"))
    return b, idx


def test_dataset_checkpoint_resume_matches_oracle(require_gpu, oracle, tmp_path):
    from leo_amd.runtime import HipRuntime

    b, idx = _write_dataset(tmp_path, 12)
    ds = formats.PreparedDataset.open(b, idx)
    batches = [ds.stories(4 * k, 4) for k in range(3)]
    ckpt = tmp_path / "model.pscls"
    initial = workload_model(WORKLOADS["A"])
    print("two batches from the dataset, then a checkpoint", flush=True)
    gpu = HipRuntime(initial, device=0, max_lanes=4)
    cpu = oracle.OracleRuntime(initial)
    try:
        for batch in batches[:2]:
            grep, gloss = gpu.train_batch(batch, native.TRAINING, replay=True)
            crep, closs = cpu.train_story_batch(batch, oracle.TRAINING, replay=True)
            for g, c in zip(gloss, closs):
                assert np.array_equal(g, c)
        trained = gpu.model()
    finally:
        gpu.close()
    assert_models_equal(trained, cpu.model(), "after two dataset batches")
    formats.commit_model_rolling(ckpt, trained, 1)
    loaded = formats.load_model(ckpt)
    assert loaded.generation == 1 and loaded.parameter_revision == trained.parameter_revision
    assert loaded.statistics == trained.statistics
    assert_models_equal(loaded, trained, "checkpoint round trip")
    print("a fresh runtime resumes from the checkpoint", flush=True)
    gpu = HipRuntime(loaded, device=0, max_lanes=4)
    cpu = oracle.OracleRuntime(loaded)
    try:
        grep, gloss = gpu.train_batch(batches[2], native.TRAINING, replay=True)
        crep, closs = cpu.train_story_batch(batches[2], oracle.TRAINING, replay=True)
        for g, c in zip(gloss, closs):
            assert np.array_equal(g, c)
        assert grep.mean_loss == crep.mean_loss
        resumed = gpu.model()
    finally:
        gpu.close()
    assert_models_equal(resumed, cpu.model(), "resumed from the checkpoint")
    assert resumed.generation == 1
    formats.commit_model_rolling(ckpt, resumed, 1)
    assert formats.read_generation(ckpt) == 2
    assert formats.load_model(formats.generation_path(ckpt, 1)).parameter_revision == trained.parameter_revision
    ds.close()
