"""GPU checks at the large benchmark configurations:

* C (131,072 units, fan-in 64 with power-law targets, 32 story lanes): one
  32-story batch cut to 48 bytes per story, replay on, against the oracle bit
  for bit; and a full-length 32-story batch run twice: identical and valid;

* D (1,048,576 units, fan-in 64, 64 story lanes): the bench's bounded CPU
  sample -- the batch's first 8 stories cut to 128 bytes, replay on -- against
  the CPU oracle bit for bit; and one full-size 64-story batch with replay
  (two resident lane groups, the grouped mean) run twice from the same model:
  identical models, a valid model, and the batch's counters consistent;

* E-shaped (E's configuration, heavy-tailed in-degree capped at 4096, 80
  winners per block, 30% target activity, on 65,536 units driven to the
  per-block cap): a 4-story batch cut to 40 bytes, replay on, against the
  oracle bit for bit, with the hub buckets folded by the radix path; and E
  at full size in the same regime: an 8-story batch run twice, identical and
  valid.
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


# --- E-shaped reduced model: heavy-tailed in-degree capped at 4096, 80 winners per
# block, 30% target activity (E's rules on 65,536 units) ---------------------------
E_REDUCED_NEURONS = 65_536
E_REDUCED_THRESHOLD = 0.05  # the lowest canonical threshold


def drive_to_e_regime(m):
    """Drives a synthetic model into workload E's high-activity regime:
    thresholds at 0.05, excitatory recurrent weights tripled and input weights
    doubled (clamped to weight_max). Without it the synthetic E model starts
    nearly silent (a handful of active units a step)."""
    wmax = np.float32(m.config.learning.weight_max)
    exc = m.rec_weight > 0
    m.rec_weight[exc] = np.minimum(m.rec_weight[exc] * np.float32(3.0), wmax)
    m.in_weight[:] = np.minimum(m.in_weight * np.float32(2.0), wmax)
    m.threshold[:] = np.float32(E_REDUCED_THRESHOLD)
    m.validate()
    return m


def e_reduced_model():
    """Workload E's configuration and topology generator on 65,536 units (256
    blocks, 80 winners each, max_active_global = blocks * 80 as in E), driven
    into E's regime, so that the blocks reach their 80-winner cap (31% of the
    units) within about 40 steps and the capped hubs receive hundreds of
    events a step."""
    from leo_amd.model import Model
    from leo_amd.workload import workload_config

    w = WORKLOADS["E"]
    cfg = workload_config(w)
    blocks = E_REDUCED_NEURONS // 256
    cfg.model.neuron_count = E_REDUCED_NEURONS
    cfg.model.block_count = blocks
    cfg.model.max_active_global = blocks * w.per_block
    m = Model.synthetic(cfg, topology=w.topology, exponent=w.exponent, in_degree_cap=w.in_degree_cap,
                        weight_sigma=0.05)
    return drive_to_e_regime(m)


@pytest.fixture(scope="module")
def model_e_reduced():
    print("building the E-shaped reduced model (65,536 units, heavy-tailed in-degree capped at 4096)", flush=True)
    return e_reduced_model()


def test_workload_e_shaped_batch_matches_oracle(require_gpu, oracle, model_e_reduced):
    w = WORKLOADS["E"]
    data, offsets = synthetic_stories(w, 4)
    stories = [s[:40] for s in story_list(data, offsets)]
    deg = np.bincount(model_e_reduced.rec_target.astype(np.int64), minlength=E_REDUCED_NEURONS)
    assert deg.max() == w.in_degree_cap and (deg > 1024).sum() > 100
    print(f"E-shaped: 4 stories cut to 40 bytes ({sum(map(len, stories))} bytes), replay on", flush=True)
    cpu = oracle.OracleRuntime(model_e_reduced)
    crep, closs = cpu.train_story_batch(stories, oracle.TRAINING, replay=True)
    print("oracle done", flush=True)
    gpu = _runtime(model_e_reduced, 4)
    try:
        gpu.kernel_stats(reset=True)
        grep, gloss = gpu.train_batch(stories, native.TRAINING, replay=True)
        stats = gpu.kernel_stats()
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert (grep.replay_segments, grep.replay_steps, grep.replay_prefix_steps) == \
            (crep.replay_segments, crep.replay_steps, crep.replay_prefix_steps)
        assert grep.merge_fixed_parameter_updates == crep.merge_fixed_parameter_updates
        assert grep.merge_context_keys == crep.merge_context_keys
        assert grep.active_neurons_sum == crep.active_neurons_sum
        got = gpu.model()
    finally:
        gpu.close()
    print(f"active per step {grep.active_neurons_sum / max(1, grep.activity_steps):.0f}; deep folds: register "
          f"{stats['deep_register_folds']}, radix {stats['deep_radix_folds']}", flush=True)
    # the batch reaches the per-block cap regime and folds hub buckets by radix sort
    assert grep.active_neurons_sum > 0.15 * E_REDUCED_NEURONS * grep.activity_steps
    assert stats["deep_radix_folds"] > 0
    assert_models_equal(got, cpu.model(), "E-shaped reduced batch")


@pytest.fixture(scope="module")
def model_e():
    print("building the workload E model (4,194,304 units)", flush=True)
    return drive_to_e_regime(workload_model(WORKLOADS["E"]))


def test_workload_e_full_size_batch_is_deterministic_and_valid(require_gpu, model_e):
    """Workload E at full size (4,194,304 units, 2^27 recurrent synapses,
    heavy-tailed in-degree capped at 4096) driven into its regime: an 8-story
    batch cut to 48 bytes with replay (about 400 lane steps and 120 replay
    steps), run twice from the same model."""
    w = WORKLOADS["E"]
    model = model_e
    data, offsets = synthetic_stories(w, 8)
    stories = [s[:48] for s in story_list(data, offsets)]
    trained = sum(map(len, stories))
    finals, reports, stats = [], [], []
    for run in range(2):
        print(f"workload E: 8-story batch ({trained} bytes) with replay, run {run}", flush=True)
        rt = _runtime(model, 8)
        try:
            rt.kernel_stats(reset=True)
            rep, losses = rt.train_batch(stories, native.TRAINING, replay=True)
            stats.append(rt.kernel_stats())
            finals.append(rt.model())
            reports.append(rep)
        finally:
            rt.close()
        print(f"run {run}: story {rep.story_seconds:.2f} s, replay {rep.replay_seconds:.2f} s, "
              f"{rep.active_neurons_sum / max(1, rep.activity_steps):.0f} active per step, "
              f"{rep.replay_steps} replay steps", flush=True)
        assert len(losses) == 8 and all(len(l) == len(s) + 1 for l, s in zip(losses, stories))
        assert all(np.isfinite(l).all() and (l >= 0).all() for l in losses)
    assert_models_equal(finals[0], finals[1], "two runs of the workload E batch")
    for field in ("mean_loss", "targets", "replay_steps", "replay_prefix_steps", "merge_fixed_parameter_updates",
                  "merge_context_keys", "active_neurons_sum", "emitted_events"):
        assert getattr(reports[0], field) == getattr(reports[1], field), field
    for key in ("lane_steps", "deep_register_folds", "deep_radix_folds", "learning_slots"):
        assert stats[0][key] == stats[1][key], key
    a = reports[0]
    assert a.targets == trained + 8 and a.replay_steps > 0
    assert stats[0]["deep_radix_folds"] > 0
    assert a.active_neurons_sum > 0.02 * w.neurons * a.activity_steps
    finals[0].validate()


def test_workload_e_lane_groups_and_multi_launch_story(require_gpu, model_e, monkeypatch):
    """E's batch shape at full size: more stories than resident lanes (two
    lane groups of two, joined by the grouped batch-end mean) and a story of
    160 bytes whose schedule is cut into launches of 32 steps (the reference
    carries long stories across chunks, cuda.rs:8555-8581). The same batch
    with all four lanes resident and the launches sized by the runtime must
    give the identical model, replay schedule and counters; the model stays
    valid."""
    w = WORKLOADS["E"]
    data, offsets = synthetic_stories(w, 4, 16)
    stories = [s[:160] if i == 0 else s[:48] for i, s in enumerate(story_list(data, offsets))]
    assert len(stories[0]) == 160
    trained = sum(map(len, stories))
    finals, reports, stats = [], [], []
    for resident, launch_steps in ((2, 32), (4, None)):
        monkeypatch.setenv("LEO_HIP_RESIDENT_LANES", str(resident))
        if launch_steps:
            monkeypatch.setenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", str(launch_steps))
        else:
            monkeypatch.delenv("LEO_HIP_MAX_STEPS_PER_LAUNCH", raising=False)
        print(f"workload E: 4 stories ({trained} bytes, the first 160) with replay, {resident} resident lanes, "
              f"launches of {launch_steps or 'any'} steps", flush=True)
        rt = _runtime(model_e, 4)
        try:
            assert rt.resident_lanes == resident
            rt.kernel_stats(reset=True)
            rep, losses = rt.train_batch(stories, native.TRAINING, replay=True)
            stats.append(rt.kernel_stats())
            finals.append(rt.model())
            reports.append(rep)
        finally:
            rt.close()
        print(f"  story {rep.story_seconds:.2f} s, replay {rep.replay_seconds:.2f} s, "
              f"{stats[-1]['launches']} launches, {rep.replay_steps} replay steps", flush=True)
        assert all(len(l) == len(s) + 1 and np.isfinite(l).all() for l, s in zip(losses, stories))
    assert_models_equal(finals[0], finals[1], "two lane groups with cut launches vs one group")
    for field in ("mean_loss", "targets", "replay_steps", "replay_prefix_steps", "merge_fixed_parameter_updates",
                  "merge_context_keys", "active_neurons_sum", "emitted_events"):
        assert getattr(reports[0], field) == getattr(reports[1], field), field
    for key in ("lane_steps", "events", "touched", "active", "learning_slots", "deep_radix_folds"):
        assert stats[0][key] == stats[1][key], key
    # the long story spans several launches in both runs, cut differently
    # (161 steps in launches of 32 take six; the runtime's own sizing differs)
    assert stats[0]["launches"] >= 6 and stats[1]["launches"] >= 6
    assert stats[0]["launches"] != stats[1]["launches"]
    assert reports[0].targets == trained + 4 and reports[0].replay_steps > 0
    finals[0].validate()


# --- binding global cap beyond 1,024 block winners: 256 blocks of 256 units,
# 16 winners each (up to 4,096 block winners) against a cap of 2,048 --------
BINDING_NEURONS = 65_536
BINDING_CAP = 2048


def binding_cap_model():
    """Workload D's configuration (uniform targets) on 65,536 units with fan-in
    32, 16 winners per block and max_active_global 2,048 (target_activity
    0.02), driven to high activity like E's regime (thresholds 0.05,
    excitatory recurrent weights x3, input weights x2): more than 2,048 of the
    up to 4,096 block winners compete within a few steps."""
    from leo_amd.model import Model
    from leo_amd.workload import workload_config

    w = WORKLOADS["D"]
    cfg = workload_config(w)
    cfg.model.neuron_count = BINDING_NEURONS
    cfg.model.block_count = BINDING_NEURONS // 256
    cfg.model.synapses_per_neuron = 32
    cfg.model.input_fanout = 256
    cfg.model.max_active_per_block = 16
    cfg.model.max_active_global = BINDING_CAP
    cfg.dynamics.target_activity = 0.02
    m = Model.synthetic(cfg, topology=w.topology, weight_sigma=0.05)
    return drive_to_e_regime(m)


def test_binding_global_cap_beyond_1024_winners_matches_oracle(require_gpu, oracle):
    from leo_amd.runtime import HipRuntime

    print("building a 65,536-unit model with 16 winners per block and max_active_global 2048", flush=True)
    model = binding_cap_model()
    w = WORKLOADS["D"]
    data, offsets = synthetic_stories(w, 4)
    stories = [s[:36] for s in story_list(data, offsets)]
    cpu = oracle.OracleRuntime(model)
    gpu = HipRuntime(model, device=0, max_lanes=4)
    try:
        # a document step by step: the step metrics of the global selection
        cpu.begin_document()
        gpu.begin_document()
        text = stories[0]
        steps = [(256, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
        widest = clipped = 0
        for i, (sym, tgt) in enumerate(steps):
            cm = cpu.step(sym, tgt, oracle.TRAINING)
            gm = gpu.step(sym, tgt, native.TRAINING)
            assert (gm.active_neurons, gm.block_selected_neurons, gm.global_cap_clipped_neurons) == \
                (cm.active_neurons, cm.block_selected_neurons, cm.global_cap_clipped_neurons), i
            assert gm.population_inhibition == cm.population_inhibition, i
            assert gm.loss == cm.loss and gm.eligible_recurrent_synapses == cm.eligible_recurrent_synapses, i
            widest = max(widest, gm.block_selected_neurons)
            clipped += gm.global_cap_clipped_neurons
        print(f"document: up to {widest} block winners, {clipped} clipped by the cap", flush=True)
        assert widest > 1024 and clipped > 0
        # then a story batch with replay from the trained state
        crep, closs = cpu.train_story_batch(stories[1:], oracle.TRAINING, replay=True)
        print("oracle batch done", flush=True)
        grep, gloss = gpu.train_batch(stories[1:], native.TRAINING, replay=True)
        for i, (g, c) in enumerate(zip(gloss, closs)):
            assert np.array_equal(g, c), f"story {i}: first differing step {np.nonzero(g != c)[0][:4]}"
        assert (grep.replay_steps, grep.replay_prefix_steps, grep.active_neurons_sum) == \
            (crep.replay_steps, crep.replay_prefix_steps, crep.active_neurons_sum)
        # frozen steps with targets: a readout after the global selection
        # with no eligibility update in the phase
        cpu.begin_document()
        gpu.begin_document()
        text = stories[2]
        frozen = [(256, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
        for i, (sym, tgt) in enumerate(frozen):
            cm = cpu.step(sym, tgt, oracle.FROZEN)
            gm = gpu.step(sym, tgt, native.FROZEN)
            assert (gm.active_neurons, gm.global_cap_clipped_neurons, gm.predicted_symbol) == \
                (cm.active_neurons, cm.global_cap_clipped_neurons, cm.predicted_symbol), i
            assert gm.loss == cm.loss and gm.population_inhibition == cm.population_inhibition, i
        assert np.array_equal(gpu.probabilities(), cpu.read_f32("probabilities"))
        got = gpu.model()
    finally:
        gpu.close()
    assert_models_equal(got, cpu.model(), "binding global cap")
