"""One-barrier frozen runs on the canonical lane.

With its kBucketSets delivery bucket sets, the canonical lane runs a frozen
step that is followed by a fused frozen step as a single phase: the winners'
events go into the bucket set of their arrival tick when they are emitted
(up to 8 ticks ahead), keyed by staged position instead of active-list rank,
their post-fire updates wait for the next fold, and the step record is
written by the next phase. Events whose arrival step runs a learning trace, or
lies past the launch, go through the ring as before.

Timelines of frozen runs of every length around the 1/2/4/8 delays, with
supervised steps between them and launches cut at several lengths, must give
the oracle's metrics, touched counts and model (runtime.rs:537-1106), and the
same work counters as the two-phase step loop (LEO_HIP_BUCKET_SETS=1)."""
from __future__ import annotations

import pytest

from leo_amd import native
from leo_amd.model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from tests.helpers import assert_models_equal, small_redundant_config, story

pytestmark = pytest.mark.gpu

# frozen run lengths between supervised pairs: each side of the 1, 2, 4 and 8
# tick delays, a lone frozen step, none, and a long run
FROZEN_RUNS = [1, 2, 3, 4, 5, 7, 8, 9, 16, 0, 1, 30]
COUNTERS = ("lane_steps", "events", "touched", "active", "scanned_rec", "scanned_in", "kept_rec", "kept_in",
            "destinations", "active_inhibitory", "learning_slots", "deep_register_folds", "deep_radix_folds")


def _timeline(text: bytes):
    steps = [(BEGIN_DOCUMENT, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
    steps.append((text[-1], END_DOCUMENT))
    timeline, at = [], 0
    for run in FROZEN_RUNS:
        for _ in range(run):
            if at < len(steps):
                timeline.append((steps[at][0], None))
                at += 1
        for _ in range(2):
            if at < len(steps):
                timeline.append(steps[at])
                at += 1
    timeline += [(s, None) for s, _ in steps[at:]]  # a frozen tail to the launch's end
    return timeline


@pytest.mark.parametrize("launch_steps", [None, 6, 13])
def test_one_barrier_frozen_runs_match_oracle_and_two_phase(require_gpu, oracle, monkeypatch, launch_steps):
    from leo_amd.runtime import HipRuntime

    model = Model.initialize(small_redundant_config())
    timeline = _timeline(story(5, 140))
    assert sum(1 for _, t in timeline if t is None) > 100
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    want, touched = [], 0
    for s, t in timeline:
        m = cpu.step(s, t, oracle.TRAINING if t is not None else oracle.FROZEN)
        touched += len(cpu.read_list("touched"))
        if t is not None:
            want.append(m)
    if launch_steps:
        monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", str(launch_steps))
    stats = {}
    for sets in ("9", "1"):
        monkeypatch.setenv("LEO_HIP_BUCKET_SETS", sets)
        print(f"{len(timeline)} steps, bucket sets {sets}, launches of {launch_steps or 'any'} steps", flush=True)
        gpu = HipRuntime(model, device=0, max_lanes=1)
        try:
            gpu.begin_document()
            gpu.kernel_stats(reset=True)
            got = gpu.replay_streaming_batch(timeline, native.TRAINING)
            assert len(got) == len(want)
            for i, (g, c) in enumerate(zip(got, want)):
                assert g.loss == c.loss and g.active_neurons == c.active_neurons, (sets, i)
                assert g.predicted_symbol == c.predicted_symbol, (sets, i)
                assert g.population_inhibition == c.population_inhibition, (sets, i)
            assert_models_equal(gpu.model(), cpu.model(), f"bucket sets {sets}")
            stats[sets] = gpu.kernel_stats()
        finally:
            gpu.close()
        assert stats[sets]["touched"] == touched, sets
    for key in COUNTERS:
        assert stats["9"][key] == stats["1"][key], key


@pytest.mark.parametrize("launch_steps", [None, 100])
def test_frozen_only_kernel_matches_oracle_and_general_kernel(require_gpu, oracle, monkeypatch, launch_steps):
    """A launch of frozen steps without output runs the step kernel built for
    them (no learning, readout or eligibility code; LEO_HIP_FROZEN_KERNEL=0
    keeps the general one). A long frozen prefix (advance_frozen_batch,
    backend.rs:428-431) followed by a mixed timeline must give the oracle's
    metrics, touched counts and model, and the same work counters as the
    general kernel."""
    from leo_amd.runtime import HipRuntime

    model = Model.initialize(small_redundant_config())
    text = story(9, 420)
    prefix = [(BEGIN_DOCUMENT, None)] + [(b, None) for b in text[:259]]
    rest = _timeline(text[259:])
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    want, touched = [], 0
    for s, t in prefix + rest:
        m = cpu.step(s, t, oracle.TRAINING if t is not None else oracle.FROZEN)
        touched += len(cpu.read_list("touched"))
        if t is not None:
            want.append(m)
    if launch_steps:
        monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", str(launch_steps))
    stats = {}
    for kernel in ("1", "0"):
        monkeypatch.setenv("LEO_HIP_FROZEN_KERNEL", kernel)
        print(f"frozen-only kernel {kernel}, launches of {launch_steps or 'any'} steps", flush=True)
        gpu = HipRuntime(model, device=0, max_lanes=1)
        try:
            gpu.begin_document()
            gpu.kernel_stats(reset=True)
            gpu.advance_frozen_batch(prefix)
            got = gpu.replay_streaming_batch(rest, native.TRAINING)
            assert len(got) == len(want)
            for i, (g, c) in enumerate(zip(got, want)):
                assert g.loss == c.loss and g.active_neurons == c.active_neurons, (kernel, i)
                assert g.predicted_symbol == c.predicted_symbol, (kernel, i)
                assert g.population_inhibition == c.population_inhibition, (kernel, i)
            assert_models_equal(gpu.model(), cpu.model(), f"frozen-only kernel {kernel}")
            stats[kernel] = gpu.kernel_stats()
        finally:
            gpu.close()
        assert stats[kernel]["touched"] == touched, kernel
    for key in COUNTERS:
        assert stats["1"][key] == stats["0"][key], key


@pytest.mark.parametrize("launch_steps", [None, 100])
def test_replay_tally_launches_match_oracle_and_recorded_launches(require_gpu, oracle, monkeypatch, launch_steps):
    """The replay's frozen prefixes of 64 steps or more run as tally launches
    of the frozen-only build (training.rs:1848-1954: the replay keeps no
    metrics of its frozen steps): no step records and no per-step work
    counters, the launch's totals summed on the device instead. A batch with
    replay must leave the oracle's model, and the same work counters and
    byte-model total as the same launches recording every step
    (LEO_HIP_TALLY=0); the general kernel (LEO_HIP_FROZEN_KERNEL=0) must leave
    the same model."""
    from leo_amd.runtime import HipRuntime

    model = Model.initialize(small_redundant_config())
    stories = [story(s, 420) for s in (3, 5)]
    cpu = oracle.OracleRuntime(model)
    cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    want = cpu.model()
    if launch_steps:
        monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", str(launch_steps))
    stats = {}
    for kernel, tally in (("1", "1"), ("1", "0"), ("0", "1")):
        monkeypatch.setenv("LEO_HIP_FROZEN_KERNEL", kernel)
        monkeypatch.setenv("LEO_HIP_TALLY", tally)
        print(f"replay: frozen-only kernel {kernel}, tally {tally}, launches of {launch_steps or 'any'} steps",
              flush=True)
        gpu = HipRuntime(model, device=0, max_lanes=len(stories))
        try:
            gpu.kernel_stats(reset=True)
            gpu.train_batch(stories, native.TRAINING, replay=True)
            assert_models_equal(gpu.model(), want, f"replay, frozen-only kernel {kernel}, tally {tally}")
            stats[kernel + tally] = gpu.kernel_stats()
        finally:
            gpu.close()
    assert stats["11"]["lane_steps"] > 0
    for key in COUNTERS:
        assert stats["11"][key] == stats["10"][key], key
    assert stats["11"]["algorithmic_bytes"] == pytest.approx(stats["10"]["algorithmic_bytes"], rel=1e-12)
    print("events: tally", stats["11"]["events"], "recorded", stats["10"]["events"], "general kernel",
          stats["01"]["events"], flush=True)
