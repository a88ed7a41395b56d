"""The RuntimeBackend state accessors and fork through the C-ABI
(crates/leo-core/src/backend.rs:388-390 active_neurons / activation,
:623-633 fork), against the oracle.

* checkpoint.rs:64-84 restated: after a frozen BEGIN step the active list is
  non-empty (and equals the oracle's, in selection order, with the same
  activations); after save -> load -> a new runtime, the list is empty and
  every activation is 0.
* fork: a runtime for a given model on the parent's device, model uploaded
  and transient state reset (cuda.rs:2347-2356); its training equals the
  oracle's and leaves the parent untouched.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd import formats, native
from leo_amd.model import BEGIN_DOCUMENT, Model
from tests.helpers import assert_models_equal, story, toml_test_config

pytestmark = pytest.mark.gpu


def _runtime(model, lanes=1):
    from leo_amd.runtime import HipRuntime

    return HipRuntime(model, device=0, max_lanes=lanes)


def test_checkpoint_excludes_worker_local_runtime_state(require_gpu, oracle, tmp_path):
    model = Model.initialize(toml_test_config())
    model.threshold[:] = 0.1
    model.in_weight[:] = 1.0
    print("backend state: frozen BEGIN step, then save/load into a new runtime", flush=True)
    cpu = oracle.OracleRuntime(model)
    cpu.begin_document()
    cpu.step(BEGIN_DOCUMENT, None, oracle.FROZEN)
    gpu = _runtime(model)
    try:
        gpu.begin_document()
        gpu.step(BEGIN_DOCUMENT, None, native.FROZEN)
        active = gpu.active_neurons()
        assert active.size > 0
        assert np.array_equal(active, cpu.read_list("active"))
        want = cpu.read_f32("activation")
        got = np.array([gpu.activation(int(n)) for n in range(model.neuron_count)], dtype=np.float32)
        assert np.array_equal(got, want)
        assert np.array_equal(gpu.read_state("activation"), want)
        path = tmp_path / "worker-state.pscls"
        formats.save_model_atomic(path, gpu.model(), False)
        loaded = formats.load_model(path)
    finally:
        gpu.close()
    resumed = _runtime(loaded)
    try:
        assert resumed.active_neurons().size == 0
        assert all(resumed.activation(n) == 0.0 for n in range(loaded.neuron_count))
        assert not resumed.read_state("activation").any()
    finally:
        resumed.close()


def test_fork_trains_its_own_model_on_the_parent_device(require_gpu, oracle):
    model = Model.initialize(toml_test_config())
    text = story(3, 48)
    print("backend state: fork, then a document on the fork", flush=True)
    parent = _runtime(model)
    try:
        parent.begin_document()
        parent.step(BEGIN_DOCUMENT, None, native.FROZEN)
        worker_model = parent.model()
        fork = parent.fork(worker_model)
        try:
            assert fork.device == parent.device
            assert fork.active_neurons().size == 0  # transient state reset
            assert_models_equal(fork.model(), worker_model, "fork before training")
            cpu = oracle.OracleRuntime(worker_model)
            cpu.begin_document()
            fork.begin_document()
            steps = [(BEGIN_DOCUMENT, text[0])] + [(text[i], text[i + 1]) for i in range(len(text) - 1)]
            for s, t in steps:
                cpu.step(s, t, oracle.TRAINING)
            fork.training_step_batch(steps, native.TRAINING)
            assert_models_equal(fork.model(), cpu.model(), "fork after a document")
            assert np.array_equal(fork.active_neurons(), cpu.read_list("active"))
            assert np.array_equal(fork.probabilities(), cpu.read_f32("probabilities"))
        finally:
            fork.close()
        assert_models_equal(parent.model(), worker_model, "parent after the fork trained")
    finally:
        parent.close()
