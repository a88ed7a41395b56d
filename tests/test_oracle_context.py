"""Pins the oracle's context-slot resolution and the keyed merge's slot
replacement, the two parts the reference's own tests reach only with free
slots (runtime.rs:1995-2011, parallel.rs:1597-1629).

* ``Model::resolve_context_slot`` (model.rs:173-221) against a declarative
  statement on random tiny tables: the existing key anywhere in the probe
  window (even past an empty slot) wins; else, when allocating, the first
  empty slot in probe order; else the slot with the fewest observations,
  the earliest in probe order among equals. A replaced slot takes the key with
  zero observations and a zero embedding. Probes count up to the hit, else the
  whole window.
* ``apply_context_deltas`` (parallel.rs:1093-1111) on hand-worked cases where
  the merged entries evict each other, so that the final table depends on the
  replacement priority: observations descending, then (order, key)
  ascending. The expected tables are worked out by hand below.
"""
from __future__ import annotations

import numpy as np
import pytest

from leo_amd.model import Model
from tests.helpers import integrated_config

U32_MAX = 0xFFFFFFFF


def _context_config(max_order: int, slots: int, probe: int, dim: int = 4):
    c = integrated_config()
    c.context.max_order = max_order
    c.context.slots_per_order = slots
    c.context.probe_limit = probe
    c.context.embedding_dim = dim
    c.validate()
    return c


def _declarative_resolve(keys, obs, slots, probe, order, key, allocate):
    """(slot or None, probes, replaced) from the rules in the module docstring."""
    base = (order - 1) * slots
    start = key % slots
    window = [base + (start + o) % slots for o in range(probe)]
    hits = [i for i, s in enumerate(window) if keys[s] == key]
    if hits:
        return window[hits[0]], hits[0] + 1, False
    if not allocate:
        return None, probe, False
    empties = [s for s in window if keys[s] == 0]
    if empties:
        return empties[0], probe, True
    weakest = min(range(probe), key=lambda i: (int(obs[window[i]]), i))
    return window[weakest], probe, True


@pytest.mark.parametrize("seed", range(6))
def test_resolve_context_slot_matches_declarative_rules(oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    cases = 0
    for slots in (2, 3, 4, 5):
        for probe in range(1, slots + 1):
            for max_order in (1, 2):
                cfg = _context_config(max_order, slots, probe)
                dim = cfg.context.embedding_dim
                for _ in range(12):
                    model = Model.initialize(cfg)
                    total = max_order * slots
                    pool = rng.integers(1, 3 * slots + 1, size=4 * slots).astype(np.uint64)
                    keys = np.where(rng.random(total) < 0.25, 0, rng.choice(pool, size=total)).astype(np.uint64)
                    obs = rng.integers(0, 4, size=total).astype(np.uint32)
                    obs[rng.random(total) < 0.1] = U32_MAX  # saturated counters
                    obs[keys == 0] = 0  # a valid model holds no observations in empty slots
                    model.ctx_keys[:] = keys
                    model.ctx_obs[:] = obs
                    model.ctx_emb[:] = rng.uniform(-0.5, 0.5, total * dim).astype(np.float32)
                    order = int(rng.integers(1, max_order + 1))
                    key = int(rng.choice(pool))
                    allocate = bool(rng.random() < 0.8)
                    want_slot, want_probes, replaced = _declarative_resolve(keys, obs, slots, probe, order, key,
                                                                            allocate)
                    rt = oracle.OracleRuntime(model)
                    got_slot, got_probes = rt.resolve_context_slot(order, key, allocate)
                    label = (slots, probe, order, key, allocate, keys.tolist(), obs.tolist())
                    assert (got_slot, got_probes) == (want_slot, want_probes), label
                    after = rt.model()
                    want_keys, want_obs, want_emb = keys.copy(), obs.copy(), model.ctx_emb.copy()
                    if replaced and keys[want_slot] != key:
                        want_keys[want_slot] = key
                        want_obs[want_slot] = 0
                        want_emb[want_slot * dim:(want_slot + 1) * dim] = 0.0
                    assert np.array_equal(after.ctx_keys, want_keys), label
                    assert np.array_equal(after.ctx_obs, want_obs), label
                    assert np.array_equal(after.ctx_emb, want_emb), label
                    cases += 1
    assert cases == 14 * 2 * 12


def _lane_with_new_key(oracle, base, key, observations, embedding):
    """A worker model that allocated `key` (order 1) and observed it."""
    rt = oracle.OracleRuntime(base)
    slot, _ = rt.resolve_context_slot(1, key, True)
    lane = rt.model()
    dim = base.config.context.embedding_dim
    lane.ctx_obs[slot] = observations
    lane.ctx_emb[slot * dim:(slot + 1) * dim] = embedding
    return lane


def _full_base(oracle, k0, k1):
    """One order of two slots (probe 2), both taken: k0 with 3 and k1 with 5
    observations, zero embeddings."""
    cfg = _context_config(1, 2, 2)
    base = Model.initialize(cfg)
    s0, s1 = k0 % 2, k1 % 2
    assert s0 != s1
    base.ctx_keys[s0], base.ctx_obs[s0] = k0, 3
    base.ctx_keys[s1], base.ctx_obs[s1] = k1, 5
    base.ctx_emb[:] = 0.0
    return base, s0, s1


def test_keyed_merge_applies_heavier_observations_first(oracle):
    # K0 (slot 0, 3 observations) and K1 (slot 1, 5) fill the order. Worker 1
    # brings new key A with 1 observation, worker 2 new key B with 4. B goes
    # first: it evicts K0 (3 < 5) and ends with 4 observations; then A evicts
    # B (4 < 5) and ends with 1. With the opposite priority B would remain.
    k0, k1, a, b = 2, 3, 4, 6
    base, s0, s1 = _full_base(oracle, k0, k1)
    ea = np.array([0.4, 0.0, 0.0, 0.0], dtype=np.float32)
    eb = np.array([0.0, -0.2, 0.0, 0.0], dtype=np.float32)
    lanes = [_lane_with_new_key(oracle, base, a, 1, ea), _lane_with_new_key(oracle, base, b, 4, eb)]
    deltas = [oracle.Delta.between(base, lane) for lane in lanes]
    master = oracle.OracleRuntime(base)
    updates, context_keys = oracle.apply_deltas(master, deltas)
    assert context_keys == 2
    out = master.model()
    assert (int(out.ctx_keys[s0]), int(out.ctx_obs[s0])) == (a, 1)
    assert (int(out.ctx_keys[s1]), int(out.ctx_obs[s1])) == (k1, 5)
    # the slot was cleared when A replaced B: only A's mean delta remains
    assert np.array_equal(out.ctx_emb[s0 * 4:(s0 + 1) * 4], np.float32(ea / np.float32(2)))


def test_keyed_merge_breaks_equal_observations_by_key(oracle):
    # C < D, both new with 2 observations: C goes first and evicts K0 (3);
    # then D evicts C (2 < 5). Key-descending ties would leave C.
    k0, k1, c, d = 2, 3, 8, 10
    base, s0, s1 = _full_base(oracle, k0, k1)
    ec = np.array([0.0, 0.0, 0.3, 0.0], dtype=np.float32)
    ed = np.array([0.0, 0.0, 0.0, 0.1], dtype=np.float32)
    lanes = [_lane_with_new_key(oracle, base, d, 2, ed), _lane_with_new_key(oracle, base, c, 2, ec)]
    deltas = [oracle.Delta.between(base, lane) for lane in lanes]
    master = oracle.OracleRuntime(base)
    oracle.apply_deltas(master, deltas)
    out = master.model()
    assert (int(out.ctx_keys[s0]), int(out.ctx_obs[s0])) == (d, 2)
    assert (int(out.ctx_keys[s1]), int(out.ctx_obs[s1])) == (k1, 5)
    assert np.array_equal(out.ctx_emb[s0 * 4:(s0 + 1) * 4], np.float32(ed / np.float32(2)))


def test_keyed_merge_sums_one_key_across_workers_before_placing_it(oracle):
    # Both workers bring key A (1 + 1 observations): one merged entry with 2
    # observations evicts K0; its embedding is the lane-ordered mean.
    k0, k1, a = 2, 3, 4
    base, s0, s1 = _full_base(oracle, k0, k1)
    e1 = np.array([0.5, 0.25, 0.0, 0.0], dtype=np.float32)
    e2 = np.array([0.25, 0.0, 0.0, -0.5], dtype=np.float32)
    lanes = [_lane_with_new_key(oracle, base, a, 1, e1), _lane_with_new_key(oracle, base, a, 1, e2)]
    deltas = [oracle.Delta.between(base, lane) for lane in lanes]
    master = oracle.OracleRuntime(base)
    _, context_keys = oracle.apply_deltas(master, deltas)
    assert context_keys == 1
    out = master.model()
    assert (int(out.ctx_keys[s0]), int(out.ctx_obs[s0])) == (a, 2)
    want = ((e1.astype(np.float64) + e2.astype(np.float64)) / 2.0).astype(np.float32)
    assert np.array_equal(out.ctx_emb[s0 * 4:(s0 + 1) * 4], want)
