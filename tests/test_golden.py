"""Committed fixture (tests/golden/make_golden.py): two logical batches of
workload A with 30% replay. The CPU test checks the oracle and the seeded model
generator still reproduce it; the GPU test checks the HIP path against it bit
for bit (per-step losses, replay schedule, every learned tensor)."""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np
import pytest

from leo_amd import native
from leo_amd.workload import WORKLOADS, workload_model

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
TENSORS = ("threshold", "rec_weight", "in_weight", "out_weight", "bias", "ctx_keys", "ctx_emb", "ctx_obs", "ctx_out")


def _fixture():
    arrays = np.load(GOLDEN / "workloadA_batches.npz")
    record = json.loads((GOLDEN / "workloadA_batches.json").read_text())
    data = arrays["story_bytes"].tobytes()
    stories, cursor = [], 0
    for n in arrays["story_lengths"]:
        stories.append(data[cursor:cursor + int(n)])
        cursor += int(n)
    return arrays, record, stories


def _digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _check_model(model, expected, label):
    for name in TENSORS:
        assert _digest(getattr(model, name)) == expected["digests"][name], f"{label}: {name}"
    assert int(model.parameter_revision) == expected["parameter_revision"], label
    for k, v in expected["statistics"].items():
        assert model.statistics[k] == v, f"{label}: statistics {k}"


def _run(runtime, train, record, stories):
    losses = []
    for (lo, hi), want in zip(record["batches"], record["reports"]):
        rep, per_story = train(runtime, stories[lo:hi])
        losses.extend(per_story)
        assert int(rep.replay_segments) == want["replay_segments"]
        assert int(rep.replay_steps) == want["replay_steps"]
        assert int(rep.replay_prefix_steps) == want["replay_prefix_steps"]
        assert int(rep.merge_fixed_parameter_updates) == want["merge_fixed_parameter_updates"]
        assert int(rep.merge_context_keys) == want["merge_context_keys"]
        assert float(rep.mean_loss) == want["mean_loss"]
    return np.concatenate(losses).astype(np.float32)


def test_seeded_model_generator_matches_fixture():
    _, record, _ = _fixture()
    _check_model(workload_model(WORKLOADS["A"]), record["initial"], "initial model")


def test_oracle_reproduces_fixture(oracle):
    arrays, record, stories = _fixture()
    rt = oracle.OracleRuntime(workload_model(WORKLOADS["A"]))
    losses = _run(rt, lambda r, s: r.train_story_batch(s, oracle.TRAINING, replay=True), record, stories)
    assert np.array_equal(losses, arrays["losses"])
    final = rt.model()
    assert np.array_equal(final.threshold, arrays["threshold"]) and np.array_equal(final.bias, arrays["bias"])
    _check_model(final, record["final"], "oracle")


@pytest.mark.gpu
def test_hip_path_matches_fixture(require_gpu):
    from leo_amd.runtime import HipRuntime

    arrays, record, stories = _fixture()
    rt = HipRuntime(workload_model(WORKLOADS["A"]), device=0, max_lanes=2)
    try:
        print("golden: workload A, 2 batches, replay on", flush=True)
        losses = _run(rt, lambda r, s: r.train_batch(s, native.TRAINING, replay=True), record, stories)
        assert np.array_equal(losses, arrays["losses"])
        final = rt.model()
        assert np.array_equal(final.threshold, arrays["threshold"]) and np.array_equal(final.bias, arrays["bias"])
        _check_model(final, record["final"], "hip")
    finally:
        rt.close()


# --- the long run (tests/golden/make_golden.py --long) -----------------------------------
def _long_fixture():
    return json.loads((GOLDEN / "workloadA_1M.json").read_text())


def _check_long_record(got, want, label):
    assert got["stories"] == want["stories"] and got["trained_bytes"] == want["trained_bytes"], label
    assert got["digests"] == want["digests"], f"{label}: tensor digests"
    assert got["statistics"] == want["statistics"], f"{label}: statistics"
    assert got["parameter_revision"] == want["parameter_revision"], label
    assert got["context_slots_taken"] == want["context_slots_taken"], label
    # the north star's criterion is running bits per byte within 1e-3; the
    # path is bit-exact, so the figure is identical
    assert abs(got["bits_per_byte"] - want["bits_per_byte"]) <= 1e-3, label
    assert got["bits_per_byte"] == want["bits_per_byte"], label


def test_long_fixture_fills_the_context_tables():
    record = _long_fixture()
    last = record["records"][-1]
    assert last["trained_bytes"] >= 1 << 20
    spo = 4096
    # orders 4-6 are full from the second checkpoint on: their allocations evict
    for rec in record["records"][1:]:
        assert all(taken == spo for taken in rec["context_slots_taken"][3:]), rec["context_slots_taken"]


def test_oracle_reproduces_long_fixture_first_checkpoint(oracle):
    import sys

    sys.path.insert(0, str(GOLDEN))
    import make_golden

    record = _long_fixture()
    w, stories = make_golden.long_stories()
    rt = oracle.OracleRuntime(workload_model(w))
    got = make_golden.long_run(rt, lambda r, s: r.train_story_batch([s], oracle.TRAINING, replay=True), stories,
                               checkpoints=record["checkpoints"][:1])
    _check_long_record(got[0], record["records"][0], "oracle, first checkpoint")


@pytest.mark.gpu
def test_hip_path_matches_long_fixture(require_gpu):
    import sys

    from leo_amd.runtime import HipRuntime

    sys.path.insert(0, str(GOLDEN))
    import make_golden

    record = _long_fixture()
    w, stories = make_golden.long_stories()
    # a run of a few minutes: progress goes to the terminal even when pytest
    # captures output
    say = lambda *a: print(*a, file=sys.__stderr__, flush=True)  # noqa: E731
    done = [0]

    def train(r, s):
        out = r.train_batch([s], native.TRAINING, replay=True)
        done[0] += 1
        if done[0] % 200 == 0:
            say(f"golden long run: {done[0]} stories trained")
        return out

    rt = HipRuntime(workload_model(w), device=0, max_lanes=1)
    try:
        say("golden: workload A, one story per batch with replay, past 2^20 trained bytes")
        got = make_golden.long_run(rt, train, stories, checkpoints=record["checkpoints"],
                                   on_checkpoint=lambda rec: say("checkpoint", rec["trained_bytes"],
                                                                 rec["bits_per_byte"]))
    finally:
        rt.close()
    assert len(got) == len(record["records"])
    for g, want in zip(got, record["records"]):
        _check_long_record(g, want, f"hip at {want['trained_bytes']} bytes")


# --- workload B past 2^20 trained bytes (tests/golden/make_golden.py --long-b) -----------
# 8 story lanes per logical batch: the lane-ordered batch-end mean
# (parallel.rs:694-798) and the keyed context merge (parallel.rs:1024-1113)
# run every batch, then 30% replay on the merged model (training.rs:1585-1727).
def _long_b_fixture():
    return json.loads((GOLDEN / "workloadB_1M.json").read_text())


def _check_long_b_record(got, want, label):
    _check_long_record(got, want, label)
    assert got["batch_report"] == want["batch_report"], f"{label}: batch report"


def test_long_b_fixture_passes_a_mebibyte():
    record = _long_b_fixture()
    assert record["lanes"] == 8 and record["records"][-1]["trained_bytes"] >= 1 << 20
    # the mean merges changes of many lanes and keys every batch
    assert all(r["batch_report"]["merge_context_keys"] > 0 for r in record["records"])


def test_oracle_reproduces_long_b_fixture_first_checkpoint(oracle):
    import sys

    sys.path.insert(0, str(GOLDEN))
    import make_golden

    record = _long_b_fixture()
    w, stories = make_golden.long_b_stories()
    rt = oracle.OracleRuntime(workload_model(w))

    def train(r, batch):
        report, _ = r.train_story_batch(batch, oracle.TRAINING, replay=True)
        return report

    got = make_golden.long_run_batches(rt, train, stories, record["lanes"], checkpoints=record["checkpoints"][:1])
    _check_long_b_record(got[0], record["records"][0], "oracle, first checkpoint")


@pytest.mark.gpu
def test_hip_path_matches_long_b_fixture(require_gpu):
    import sys

    from leo_amd.runtime import HipRuntime

    sys.path.insert(0, str(GOLDEN))
    import make_golden

    record = _long_b_fixture()
    w, stories = make_golden.long_b_stories()
    say = lambda *a: print(*a, file=sys.__stderr__, flush=True)  # noqa: E731
    done = [0]

    def train(r, batch):
        report, _ = r.train_batch(batch, native.TRAINING, replay=True)
        done[0] += 1
        if done[0] % 20 == 0:
            say(f"golden B long run: {done[0]} batches trained")
        return report

    rt = HipRuntime(workload_model(w), device=0, max_lanes=record["lanes"])
    try:
        say("golden: workload B, 8 story lanes per batch with replay, past 2^20 trained bytes")
        got = make_golden.long_run_batches(rt, train, stories, record["lanes"], checkpoints=record["checkpoints"],
                                           on_checkpoint=lambda rec: say("checkpoint", rec["trained_bytes"],
                                                                         rec["bits_per_byte"]))
    finally:
        rt.close()
    assert len(got) == len(record["records"])
    for g, want in zip(got, record["records"]):
        _check_long_b_record(g, want, f"hip at {want['trained_bytes']} bytes")
