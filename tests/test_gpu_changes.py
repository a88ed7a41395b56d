"""The sparse-sync masks (ParameterChanges, runtime.rs:37-46) of the HIP path
against the oracle, as sets, through the coordinator's sequence
(training.rs:1548-1563, 1585-1649):

* tracking restarted (the GPU adapter clears the change sets and dirty flags
  on every call, cuda.rs:2827-2837), then an in-place document pass;
* a story batch (merged on return), tracking restarted, then a replay range
  (frozen prefix, supervised targets) through the step primitives;
* a restart with nothing after it: empty sets and clean flags.

The oracle follows the CPU Runtime, whose enable is a no-op once tracking is on
(runtime.rs:310-320); its restart_parameter_tracking restates the adapter's
clearing for the comparison.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import small_redundant_config, story

pytestmark = pytest.mark.gpu

SETS = ("threshold", "recurrent_weight", "input_weight", "output_neurons", "context_slots")


def _document_steps(text: bytes):
    steps = [(BEGIN_DOCUMENT, text[0])]
    steps += [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    return steps


def _compare(gpu_changes, cpu_changes, label):
    for name in SETS:
        g = np.asarray(gpu_changes[name], dtype=np.int64)
        c = np.sort(np.asarray(cpu_changes[name], dtype=np.int64))
        assert np.array_equal(g, c), f"{label}: {name}: gpu {g.size} entries, cpu {c.size}; " \
                                     f"first differing {np.setxor1d(g, c)[:8]}"
    for flag in ("output_bias_dirty", "context_output_dirty"):
        assert gpu_changes[flag] == cpu_changes[flag], f"{label}: {flag}"


def test_parameter_changes_match_oracle_through_the_coordinator_sequence(require_gpu, oracle):
    from leo_amd.runtime import HipRuntime

    cfg = small_redundant_config(dropout=0.0)
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_UNIFORM, weight_sigma=0.05)
    cpu = oracle.OracleRuntime(model)
    gpu = HipRuntime(model, device=0, max_lanes=4)
    try:
        # 1) in-place document pass with tracking
        text = story(21, 120)
        print("changes: document pass", flush=True)
        cpu.restart_parameter_tracking()
        gpu.enable_parameter_tracking()
        cpu.begin_document()
        gpu.begin_document()
        steps = _document_steps(text)
        for s, t in steps:
            cpu.step(s, t, oracle.TRAINING)
        gpu.training_step_batch(steps, native.TRAINING)
        g1 = gpu.parameter_changes()
        _compare(g1, cpu.changes(), "document pass")
        assert g1["recurrent_weight"].size > 0 and g1["threshold"].size > 0 and g1["output_bias_dirty"]
        cpu.finish_document()
        gpu.finish_document()

        # 2) story batch, then a replay range with tracking restarted
        stories = [story(30 + i, 90) for i in range(4)]
        print("changes: story batch + replay range", flush=True)
        cpu.train_story_batch(stories, oracle.TRAINING, replay=False)
        gpu.training_story_batch(stories, native.TRAINING)
        cpu.restart_parameter_tracking()
        gpu.enable_parameter_tracking()
        replay = stories[1]
        start, end = 40, 72
        prefix = [(BEGIN_DOCUMENT, None)] + [(replay[i], None) for i in range(start - 1)]
        targets = [(replay[p - 1], replay[p]) for p in range(start, end)]
        cpu.begin_document()
        gpu.begin_document()
        for s, _ in prefix:
            cpu.step(s, None, oracle.FROZEN)
        gpu.advance_frozen_batch(prefix)
        for s, t in targets:
            cpu.step(s, t, oracle.TRAINING)
        gpu.training_step_batch(targets, native.TRAINING)
        g2 = gpu.parameter_changes()
        _compare(g2, cpu.changes(), "replay range")
        assert g2["recurrent_weight"].size > 0

        # 3) a restart leaves empty sets and clean flags
        cpu.restart_parameter_tracking()
        gpu.enable_parameter_tracking()
        g3 = gpu.parameter_changes()
        _compare(g3, cpu.changes(), "after restart")
        assert all(g3[name].size == 0 for name in SETS)
        assert not g3["output_bias_dirty"] and not g3["context_output_dirty"]
    finally:
        gpu.close()
