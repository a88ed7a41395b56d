"""The batch-end merge's constraint projection and validation
(project_parameter_constraints_sparse and validate_sparse_merge,
crates/leo-core/src/parallel.rs:1169-1345), pinned with hand-worked cases.

A mean of valid lane values stays inside every bound, so these cases use the
additive merge (apply_sum_deltas, parallel.rs:707-713: divisor 1) to push a
merged value past a bound: two workers each move a parameter by d, the merge
adds 2d, and the expected result is worked out by hand from the projection's
rules. Each case is chosen so that a plausible slip fails it:
  * recurrent weights: clamp to [weight_min, weight_max], then the sign of the
    SOURCE neuron's type (a slot whose target has the other type separates a
    source/target mix-up);
  * input weights: [0, weight_max], not [weight_min, weight_max];
  * thresholds [0.05, 2.0], excitability [0.1, 4.0];
  * output, context output and context embedding weights [weight_min, weight_max];
  * the output bias is not clamped;
  * a sign projection that lands on zero gives +0.0, never -0.0.
"""
from __future__ import annotations

import ctypes
import pathlib
import shutil
import subprocess

import numpy as np
import pytest

from leo_amd.model import Model
from tests.helpers import toml_test_config

F32 = np.float32


def _base():
    return Model.initialize(toml_test_config())


def _two_workers(base, edit):
    """Two trained copies of base, both edited by edit(model)."""
    first, second = base.copy(), base.copy()
    edit(first)
    edit(second)
    return first, second


def _merge(oracle, base, models, mean):
    deltas = [oracle.Delta.between(base, m) for m in models]
    master = oracle.OracleRuntime(base)
    fixed, ctx = oracle.apply_deltas(master, deltas, mean=mean)
    return master.model(), fixed, ctx


def _bits(x):
    return np.asarray(x, dtype=F32).view(np.uint32)


def _mixed_slot(model, source_type):
    """A recurrent slot whose source has source_type and whose target has the other type."""
    S = model.config.model.synapses_per_neuron
    for slot in range(model.rec_weight.size):
        src, dst = slot // S, int(model.rec_target[slot])
        if model.neuron_type[src] == source_type and model.neuron_type[dst] != source_type:
            return slot
    raise AssertionError("no mixed-type slot in the test model")


def test_recurrent_weights_clamp_then_take_the_source_sign(oracle):
    base = _base()
    exc_hi = _mixed_slot(base, 0)        # excitatory source, inhibitory target
    inh_hi = _mixed_slot(base, 1)        # inhibitory source, excitatory target
    S = base.config.model.synapses_per_neuron
    exc_lo = next(s for s in range(base.rec_weight.size)
                  if base.neuron_type[s // S] == 0 and s not in (exc_hi,))
    inh_lo = next(s for s in range(base.rec_weight.size)
                  if base.neuron_type[s // S] == 1 and s not in (inh_hi,))
    base.rec_weight[exc_hi] = F32(0.6)   # +0.3 twice: 1.2 -> clamp 1.0
    base.rec_weight[exc_lo] = F32(0.25)  # -0.25 twice: -0.25 -> clamp -0.25 -> excitatory max(., 0) = +0.0
    base.rec_weight[inh_hi] = F32(-0.25)  # +0.25 twice: 0.25 -> inhibitory min(., 0) = +0.0
    base.rec_weight[inh_lo] = F32(-0.6)  # -0.3 twice: -1.2 -> clamp -1.0

    def edit(m):
        m.rec_weight[exc_hi] = F32(0.9)
        m.rec_weight[exc_lo] = F32(0.0)
        m.rec_weight[inh_hi] = F32(0.0)
        m.rec_weight[inh_lo] = F32(-0.9)

    out, fixed, _ = _merge(oracle, base, _two_workers(base, edit), mean=False)
    assert out.rec_weight[exc_hi] == F32(1.0)
    assert out.rec_weight[inh_lo] == F32(-1.0)
    # zero from the sign projection is +0.0: a target-typed projection would
    # keep -0.25 / +0.25 here, a multiply-by-mask projection would give -0.0
    assert _bits(out.rec_weight[exc_lo]) == _bits(0.0)
    assert _bits(out.rec_weight[inh_hi]) == _bits(0.0)
    assert fixed == 4


def test_input_weights_clamp_to_zero_and_weight_max(oracle):
    base = _base()
    low, high = 3, 17
    base.in_weight[low] = F32(0.1)   # -0.1 twice: -0.1 -> [0, wmax] -> +0.0 ([wmin, wmax] would keep -0.1)
    base.in_weight[high] = F32(0.6)  # +0.3 twice: 1.2 -> 1.0

    def edit(m):
        m.in_weight[low] = F32(0.0)
        m.in_weight[high] = F32(0.9)

    out, _, _ = _merge(oracle, base, _two_workers(base, edit), mean=False)
    assert _bits(out.in_weight[low]) == _bits(0.0)
    assert out.in_weight[high] == F32(1.0)


def test_thresholds_and_excitability_clamp_to_their_ranges(oracle):
    base = _base()
    base.threshold[0] = F32(1.5)    # +0.4 twice: 2.3 -> 2.0
    base.threshold[1] = F32(0.1)    # -0.04 twice: 0.02 -> 0.05
    base.excitability[2] = F32(3.0)  # +0.8 twice: 4.6 -> 4.0
    base.excitability[3] = F32(0.3)  # -0.15 twice: 0.0 -> 0.1

    def edit(m):
        m.threshold[0] = F32(1.9)
        m.threshold[1] = F32(0.06)
        m.excitability[2] = F32(3.8)
        m.excitability[3] = F32(0.15)

    out, fixed, _ = _merge(oracle, base, _two_workers(base, edit), mean=False)
    assert out.threshold[0] == F32(2.0) and out.threshold[1] == F32(0.05)
    assert out.excitability[2] == F32(4.0) and out.excitability[3] == F32(0.1)
    assert fixed == 4


def test_output_and_context_output_weights_clamp_but_the_bias_does_not(oracle):
    base = _base()
    n = base.neuron_count
    hi, lo = 5 * n + 7, 9 * n + 2
    base.out_weight[hi] = F32(0.8)   # +0.15 twice: 1.1 -> 1.0
    base.out_weight[lo] = F32(-0.8)  # -0.15 twice: -1.1 -> -1.0
    base.ctx_out[4] = F32(0.7)       # +0.2 twice: 1.1 -> 1.0
    base.ctx_out[11] = F32(-0.7)     # -0.2 twice: -1.1 -> -1.0
    base.bias[3] = F32(0.5)          # +0.4 twice: 1.3, unclamped

    def edit(m):
        m.out_weight[hi] = F32(0.95)
        m.out_weight[lo] = F32(-0.95)
        m.ctx_out[4] = F32(0.9)
        m.ctx_out[11] = F32(-0.9)
        m.bias[3] = F32(0.9)

    out, _, _ = _merge(oracle, base, _two_workers(base, edit), mean=False)
    assert out.out_weight[hi] == F32(1.0) and out.out_weight[lo] == F32(-1.0)
    assert out.ctx_out[4] == F32(1.0) and out.ctx_out[11] == F32(-1.0)
    d = F32(F32(0.9) - F32(0.5))
    assert out.bias[3] == F32(F32(0.5) + F32(np.float64(d) + np.float64(d)))
    assert out.bias[3] > F32(1.0)


def test_context_embeddings_clamp_after_the_keyed_merge(oracle):
    base = _base()
    dim = base.config.context.embedding_dim
    key = 12345
    workers = []
    for _ in range(2):
        rt = oracle.OracleRuntime(base)
        slot, _ = rt.resolve_context_slot(2, key, True)
        m = rt.model()
        m.ctx_emb[slot * dim + 0] = F32(0.8)    # +0.8 twice: 1.6 -> 1.0
        m.ctx_emb[slot * dim + 1] = F32(-0.8)   # -0.8 twice: -1.6 -> -1.0
        m.ctx_emb[slot * dim + 2] = F32(0.25)   # +0.25 twice: 0.5, inside the bounds
        m.ctx_obs[slot] = 1
        workers.append(m)
    out, _, ctx = _merge(oracle, base, workers, mean=False)
    probe = oracle.OracleRuntime(out)
    slot, _ = probe.resolve_context_slot(2, key, False)
    assert slot is not None and ctx == 1
    row = out.ctx_emb[slot * dim:(slot + 1) * dim]
    assert row[0] == F32(1.0) and row[1] == F32(-1.0) and row[2] == F32(0.5)
    assert out.ctx_obs[slot] == 2


def test_mean_merge_of_valid_lanes_needs_no_projection(oracle):
    """Mean mode (the device path): with every lane's value inside the bounds
    the mean lands inside them, so the projection leaves it as computed."""
    base = _base()
    base.rec_weight[0] = F32(0.3)
    first, second = base.copy(), base.copy()
    first.rec_weight[0] = F32(1.0)
    second.rec_weight[0] = F32(0.5)
    out, _, _ = _merge(oracle, base, [first, second], mean=True)
    d1, d2 = np.float64(F32(F32(1.0) - F32(0.3))), np.float64(F32(F32(0.5) - F32(0.3)))
    assert out.rec_weight[0] == F32(F32(0.3) + F32((d1 + d2) / 2))


def test_mean_merge_writes_a_cancelled_update_and_clears_a_negative_zero(oracle):
    """An element whose lane deltas cancel is still merged (target += 0.0,
    parallel.rs:1014): a -0.0 output weight becomes +0.0. A merge that
    skipped zero sums would keep -0.0."""
    base = _base()
    n = base.neuron_count
    i = 2 * n + 5
    base.out_weight[i] = F32(-0.0)
    first, second = base.copy(), base.copy()
    first.out_weight[i] = F32(0.25)
    second.out_weight[i] = F32(-0.25)
    out, fixed, _ = _merge(oracle, base, [first, second], mean=True)
    assert _bits(out.out_weight[i]) == _bits(0.0)
    assert fixed == 1


def test_inhibitory_negative_zero_projects_to_positive_zero(oracle):
    """-0.0 on an inhibitory slot: clamp keeps -0.0 and the reference's
    weight.min(0.0) returns +0.0 (on x86_64 rustc lowers f32::min with a
    constant second operand to minss, which returns that operand when the
    values compare equal; see test_x86_minnum_lowering_of_a_constant_zero)."""
    base = _base()
    S = base.config.model.synapses_per_neuron
    slot = next(s for s in range(base.rec_weight.size) if base.neuron_type[s // S] == 1)
    base.rec_weight[slot] = F32(-0.0)
    tiny = np.array([1], dtype=np.uint32).view(F32)[0]  # 2^-149
    first, second = base.copy(), base.copy()
    first.rec_weight[slot] = -tiny      # delta -2^-149; the mean -2^-150 rounds to -0.0
    out, _, _ = _merge(oracle, base, [first, second], mean=True)
    assert _bits(out.rec_weight[slot]) == _bits(0.0)


def test_x86_minnum_lowering_of_a_constant_zero(tmp_path):
    """Pins the rule the oracle's sign projection follows: LLVM's x86-64
    lowering of minnum/maxnum(x, 0.0) (what rustc emits for f32::min/max)
    returns +0.0 for x = -0.0 and x = NaN."""
    clang = shutil.which("clang") or "/opt/rocm/llvm/bin/clang"
    if not pathlib.Path(clang).exists():
        pytest.skip("no clang to check the lowering")
    src = tmp_path / "m.c"
    src.write_text(
        "__attribute__((noinline)) float mn(float w){return __builtin_fminf(w,0.0f);}\n"
        "__attribute__((noinline)) float mx(float w){return __builtin_fmaxf(w,0.0f);}\n")
    lib = tmp_path / "m.so"
    subprocess.run([clang, "-O2", "-shared", "-fPIC", str(src), "-o", str(lib)], check=True)
    m = ctypes.CDLL(str(lib))
    for f in (m.mn, m.mx):
        f.restype, f.argtypes = ctypes.c_float, [ctypes.c_float]
    for fn in (m.mn, m.mx):
        for x in (-0.0, float("nan")):
            r = F32(fn(x))
            assert _bits(r) == _bits(0.0), (fn, x, r)
    assert F32(m.mn(-0.5)) == F32(-0.5) and F32(m.mx(0.5)) == F32(0.5)


def test_merge_validation_rejects_a_non_finite_loss_sum(oracle):
    base = _base()
    first = base.copy()
    first.statistics["training_loss_sum"] = float("inf")
    first.bias[0] += F32(0.1)
    with pytest.raises(oracle.OracleError, match="non-finite loss"):
        _merge(oracle, base, [first], mean=True)


def test_merge_rejects_a_parameter_that_overflows(oracle):
    """apply_sparse_scaled (parallel.rs:1014-1017): the additive sum of two
    finite bias deltas of 3e38 overflows and the merge fails."""
    base = _base()
    first, second = base.copy(), base.copy()
    first.bias[1] = F32(3.0e38)
    second.bias[1] = F32(3.0e38)
    with pytest.raises(oracle.OracleError, match="non-finite"):
        _merge(oracle, base, [first, second], mean=False)


def test_context_embedding_overflow_is_clamped_not_rejected(oracle):
    """The keyed context merge has no finiteness check of its own
    (parallel.rs:1024-1113): an embedding pushed to +inf by two 3e38 deltas is
    clamped to weight_max by the projection and passes validation."""
    base = _base()
    dim = base.config.context.embedding_dim
    workers = []
    for _ in range(2):
        rt = oracle.OracleRuntime(base)
        slot, _ = rt.resolve_context_slot(1, 77, True)
        m = rt.model()
        m.ctx_emb[slot * dim] = F32(3.0e38)
        m.ctx_obs[slot] = 1
        workers.append(m)
    # the workers' tables are outside the model bounds; only the delta is used
    deltas = [oracle.Delta.between(base, m) for m in workers]
    master = oracle.OracleRuntime(base)
    oracle.apply_deltas(master, deltas, mean=False)
    out = master.model()
    slot, _ = oracle.OracleRuntime(out).resolve_context_slot(1, 77, False)
    assert out.ctx_emb[slot * dim] == F32(1.0)
