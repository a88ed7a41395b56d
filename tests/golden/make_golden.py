"""Writes tests/golden/workloadA_batches.npz and .json: the CPU oracle's results
for two logical batches of workload A (1,024 units) with 30% replay, from the
seeded synthetic model and the first three seeded stories.

    python tests/golden/make_golden.py

The fixture holds the inputs (story bytes, offsets), every per-step loss, the
replay schedule counts, the full threshold and bias vectors, and SHA-256
digests of every learned tensor. tests/test_golden.py checks that the oracle
still reproduces it (CPU) and that the HIP path matches it bit for bit (GPU).
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


if __name__ == "__main__":
    main()
