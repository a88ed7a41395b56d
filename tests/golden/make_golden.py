"""Writes the CPU oracle's golden fixtures for workload A (1,024 units, one
logical worker, 30% replay), from the seeded synthetic model and seeded
stories:

    python tests/golden/make_golden.py          # workloadA_batches.npz / .json
    python tests/golden/make_golden.py --long   # workloadA_1M.json
    python tests/golden/make_golden.py --long-b # workloadB_1M.json (~35 minutes of oracle time)

workloadA_batches holds two logical batches: the inputs (story bytes,
offsets), every per-step loss, the replay schedule counts, the full threshold
and bias vectors, and SHA-256 digests of every learned tensor.

workloadA_1M holds a run over the first stories of the workload until more
than 2^20 bytes are trained, one story per logical batch (the workload's single
worker trains in place, training.rs:1548-1582) with replay: at checkpoints
after 2^16, 2^18, 2^19 and 2^20 trained bytes, the running bits per byte, the
statistics, the parameter revision, the digests of every learned tensor and
how many slots of each context order are taken. Context orders 4 to 6
(4,096 slots each) are full by the second checkpoint, so from there on every
allocation at those orders evicts the weakest slot of its probe window.

workloadB_1M holds workload B (16,384 units, 8 story lanes per logical
batch, 30% replay) trained batch by batch until more than 2^20 bytes are
trained: the same checkpoint records (after 2^14, 2^17, 2^19 and 2^20 bytes)
plus that batch's merge and replay report. Every batch runs the lane-ordered
batch-end mean and the keyed context merge.

tests/test_golden.py checks that the oracle still reproduces them (CPU; the
long runs up to their first checkpoint) and that the HIP path matches them
bit for bit (GPU).
"""
from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from leo_amd.workload import WORKLOADS, synthetic_stories, workload_model  # noqa: E402

TENSORS = ("threshold", "rec_weight", "in_weight", "out_weight", "bias", "ctx_keys", "ctx_emb", "ctx_obs", "ctx_out")
BATCHES = ((0, 1), (1, 3))  # story index ranges of the two logical batches


def digest(array: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


def model_record(model) -> dict:
    return {
        "digests": {name: digest(getattr(model, name)) for name in TENSORS},
        "statistics": {k: (float(v) if isinstance(v, float) else int(v)) for k, v in model.statistics.items()},
        "parameter_revision": int(model.parameter_revision),
    }


def inputs():
    w = WORKLOADS["A"]
    data, offsets = synthetic_stories(w, 3)
    stories = [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(3)]
    return w, stories


def main() -> None:
    from oracle import binding

    w, stories = inputs()
    model = workload_model(w)
    rt = binding.OracleRuntime(model)
    losses, reports = [], []
    for lo, hi in BATCHES:
        rep, per_story = rt.train_story_batch(stories[lo:hi], binding.TRAINING, replay=True)
        losses.extend(per_story)
        reports.append({"replay_segments": int(rep.replay_segments), "replay_steps": int(rep.replay_steps),
                        "replay_prefix_steps": int(rep.replay_prefix_steps),
                        "merge_fixed_parameter_updates": int(rep.merge_fixed_parameter_updates),
                        "merge_context_keys": int(rep.merge_context_keys), "mean_loss": float(rep.mean_loss)})
    final = rt.model()
    np.savez_compressed(HERE / "workloadA_batches.npz",
                        story_bytes=np.frombuffer(b"".join(stories), dtype=np.uint8),
                        story_lengths=np.array([len(s) for s in stories], dtype=np.uint64),
                        losses=np.concatenate(losses).astype(np.float32),
                        threshold=final.threshold.astype(np.float32), bias=final.bias.astype(np.float32))
    record = {"workload": "A", "batches": [list(b) for b in BATCHES], "reports": reports,
              "initial": model_record(model), "final": model_record(final)}
    (HERE / "workloadA_batches.json").write_text(json.dumps(record, indent=1, sort_keys=True) + "\n")
    print("wrote", HERE / "workloadA_batches.npz", "and .json")


LONG_CHECKPOINTS = (1 << 16, 1 << 18, 1 << 19, 1 << 20)
LONG_STORIES = 2000  # more than enough stories of U[256,1024] bytes for 2^20 bytes


def long_run(runtime, train, stories, checkpoints=LONG_CHECKPOINTS, on_checkpoint=None):
    """Trains one story per logical batch until the last checkpoint is passed;
    returns the checkpoint records (the first story boundary at or past each)."""
    records, trained, pending = [], 0, list(checkpoints)
    for index, story in enumerate(stories):
        train(runtime, story)
        trained += len(story)
        if pending and trained >= pending[0]:
            pending.pop(0)
            model = runtime.model()
            spo = model.config.context.slots_per_order
            rec = model_record(model)
            rec.update(stories=index + 1, trained_bytes=trained, bits_per_byte=float(model.bits_per_byte()),
                       context_slots_taken=[int((model.ctx_keys[o * spo:(o + 1) * spo] != 0).sum())
                                            for o in range(model.config.context.max_order)])
            records.append(rec)
            if on_checkpoint:
                on_checkpoint(rec)
            if not pending:
                break
    return records


def long_stories():
    w = WORKLOADS["A"]
    data, offsets = synthetic_stories(w, LONG_STORIES)
    return w, [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(LONG_STORIES)]


def main_long() -> None:
    from oracle import binding

    w, stories = long_stories()
    model = workload_model(w)
    rt = binding.OracleRuntime(model)
    records = long_run(rt, lambda r, s: r.train_story_batch([s], binding.TRAINING, replay=True), stories,
                       on_checkpoint=lambda rec: print("checkpoint", rec["trained_bytes"], rec["bits_per_byte"],
                                                       flush=True))
    out = {"workload": "A", "checkpoints": list(LONG_CHECKPOINTS), "initial": model_record(model),
           "records": records}
    (HERE / "workloadA_1M.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print("wrote", HERE / "workloadA_1M.json")


LONG_B_CHECKPOINTS = (1 << 14, 1 << 17, 1 << 19, 1 << 20)
LONG_B_STORIES = 1600  # N(800,250)-byte stories: ~1,310 of them pass 2^20 bytes


def long_run_batches(runtime, train_batch, stories, lanes, checkpoints=LONG_B_CHECKPOINTS, on_checkpoint=None):
    """Trains logical batches of `lanes` consecutive stories (story lanes, the
    lane-ordered batch-end mean and the keyed context merge, then replay:
    training.rs:1585-1727) until the last checkpoint is passed. Returns the
    checkpoint records, taken at the first batch boundary at or past each, with
    that batch's merge and replay report."""
    records, trained, pending = [], 0, list(checkpoints)
    for start in range(0, len(stories) - lanes + 1, lanes):
        report = train_batch(runtime, stories[start:start + lanes])
        trained += sum(len(s) for s in stories[start:start + lanes])
        if pending and trained >= pending[0]:
            pending.pop(0)
            model = runtime.model()
            spo = model.config.context.slots_per_order
            rec = model_record(model)
            rec.update(stories=start + lanes, trained_bytes=trained, bits_per_byte=float(model.bits_per_byte()),
                       context_slots_taken=[int((model.ctx_keys[o * spo:(o + 1) * spo] != 0).sum())
                                            for o in range(model.config.context.max_order)],
                       batch_report={"replay_segments": int(report.replay_segments),
                                     "replay_steps": int(report.replay_steps),
                                     "replay_prefix_steps": int(report.replay_prefix_steps),
                                     "merge_fixed_parameter_updates": int(report.merge_fixed_parameter_updates),
                                     "merge_context_keys": int(report.merge_context_keys),
                                     "mean_loss": float(report.mean_loss)})
            records.append(rec)
            if on_checkpoint:
                on_checkpoint(rec)
            if not pending:
                break
    return records


def long_b_stories():
    w = WORKLOADS["B"]
    data, offsets = synthetic_stories(w, LONG_B_STORIES)
    return w, [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(LONG_B_STORIES)]


def main_long_b() -> None:
    """workloadB_1M.json: workload B (16,384 units, 8 story lanes per logical
    batch, 30% replay) past 2^20 trained bytes."""
    from oracle import binding

    w, stories = long_b_stories()
    model = workload_model(w)
    rt = binding.OracleRuntime(model)

    def train(r, batch):
        report, _ = r.train_story_batch(batch, binding.TRAINING, replay=True)
        return report

    records = long_run_batches(rt, train, stories, w.lanes,
                               on_checkpoint=lambda rec: print("checkpoint", rec["trained_bytes"],
                                                               rec["bits_per_byte"], flush=True))
    out = {"workload": "B", "lanes": w.lanes, "checkpoints": list(LONG_B_CHECKPOINTS),
           "initial": model_record(model), "records": records}
    (HERE / "workloadB_1M.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print("wrote", HERE / "workloadB_1M.json")


if __name__ == "__main__":
    if "--long-b" in sys.argv[1:]:
        main_long_b()
    elif "--long" in sys.argv[1:]:
        main_long()
    else:
        main()
