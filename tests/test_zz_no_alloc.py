"""leo_hip_commit_packed_host_model_no_alloc (staging in the per-GPU static
scratch, no device allocation) against leo_hip_commit_packed_host_model on
the same packed updates: two calls in a row, the second smaller, leave both
runtimes with identical models bit for bit; an update whose staging exceeds
the scratch is refused before anything is written."""
from __future__ import annotations

import ctypes

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


def _bits_equal(a: Model, b: Model, label: str):
    assert_models_equal(a, b, label)
    for name in ("threshold", "rec_weight", "in_weight", "out_weight", "bias", "ctx_emb", "ctx_out"):
        x, y = getattr(a, name).view(np.uint32), getattr(b, name).view(np.uint32)
        assert np.array_equal(x, y), f"{label}: {name} bits differ"


def _commit_no_alloc(rt, update):
    u = update.to_c()
    native.check(rt._lib, rt._lib.leo_hip_commit_packed_host_model_no_alloc(rt._handle, ctypes.byref(u)))


def test_no_alloc_commit_matches_the_allocating_commit(require_gpu):
    from leo_amd.runtime import HipRuntime, PackedUpdate

    cfg = small_redundant_config()
    model = Model.synthetic(cfg, topology=native.TOPOLOGY_UNIFORM, weight_sigma=0.05)
    print("no-alloc: building a packed update from a trained runtime", flush=True)
    trainer = HipRuntime(model, device=0, max_lanes=1)
    try:
        trainer.enable_parameter_tracking()
        trainer.begin_document()
        trainer.training_step_batch(_document_steps(story(80, 160)), native.TRAINING)
        changes = trainer.parameter_changes()
        mirror = model.copy()
        trainer.synchronize_model(mirror)
    finally:
        trainer.close()
    first = PackedUpdate.from_model(mirror, changes)
    assert first.recurrent_indices.size > 8 and first.output_neurons.size > 2
    # a second, smaller update: every other changed element, new values, no
    # bias or context projection
    second = PackedUpdate.from_model(mirror, changes)
    for name in ("threshold", "recurrent", "input"):
        idx = getattr(second, f"{name}_indices")[::2].copy()
        setattr(second, f"{name}_indices", idx)
        setattr(second, f"{name}_values", getattr(second, f"{name}_values")[::2].copy())
    second.recurrent_values = np.where(second.recurrent_values > 0, second.recurrent_values * np.float32(0.5),
                                       second.recurrent_values).astype(np.float32)
    second.output_neurons = second.output_neurons[:1].copy()
    second.output_values_by_neuron = second.output_values_by_neuron[:257].copy()
    second.context_slots = second.context_slots[:1].copy()
    second.context_keys = second.context_keys[:1].copy()
    second.context_observations = second.context_observations[:1].copy()
    second.context_embeddings = second.context_embeddings[:cfg.context.embedding_dim].copy()
    second.output_bias = None
    second.context_output_weights = None
    second.parameter_revision += 1

    allocating = HipRuntime(model, device=0, max_lanes=1)
    fixed = HipRuntime(model, device=0, max_lanes=1)
    try:
        for label, update in (("first call", first), ("second, smaller call", second)):
            print(f"no-alloc: {label}", flush=True)
            allocating.commit_packed_host_model(update)
            _commit_no_alloc(fixed, update)
            _bits_equal(fixed.model(), allocating.model(), label)
        before = fixed.model()
        # one tensor's staging beyond the 8 MiB scratch: refused, nothing written
        too_big = PackedUpdate.from_model(mirror, changes)
        n = (8 << 20) // 8 + 1024
        too_big.recurrent_indices = np.resize(first.recurrent_indices, n).astype(np.uint32)
        too_big.recurrent_values = np.resize(first.recurrent_values, n).astype(np.float32)
        with pytest.raises(native.LeoError) as err:
            _commit_no_alloc(fixed, too_big)
        assert err.value.code == native.ERR_INVALID_ARGUMENT
        _bits_equal(fixed.model(), before, "after the refused update")
    finally:
        allocating.close()
        fixed.close()
