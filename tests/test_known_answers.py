"""Known-answer pins for the fixed functions of the model format, taken from
published test vectors rather than from the formulas themselves:

* SplitMix64 (crates/leo-core/src/rng.rs:13-19): the seed-0 output stream is
  the published reference sequence of Vigna's splitmix64.c.
* Dropout hash (runtime.rs:103-116): its finaliser is SplitMix64's mix, so with
  inputs chosen to make its pre-mix value equal the first SplitMix64 state, the
  draw is fixed by the same published stream.
* Context key (runtime.rs:679-690): FNV-1a 64 over the little-endian bytes of
  the history, from the offset basis xor order. Undoing the three zero-byte
  rounds of a one-symbol history leaves the published FNV-1a vector for "a".
"""
from __future__ import annotations

import ctypes

import numpy as np

from leo_amd import native

# splitmix64.c with seed 0: the first five outputs
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC,
                    0x1B39896A51A8749B]
GOLDEN_GAMMA = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1
FNV_PRIME = 0x100000001B3
FNV1A64_A = 0xAF63DC4C8601EC8C  # FNV-1a 64 of the one-byte string "a"


def test_splitmix64_seed0_stream():
    lib = native.load()
    out = np.zeros(5, dtype=np.uint64)
    native.check(lib, lib.leo_splitmix64(0, out.ctypes.data, 5))
    assert [int(v) for v in out] == SPLITMIX64_SEED0


def test_dropout_hash_finaliser_and_draw(oracle):
    lib = oracle.load()
    draw = (SPLITMIX64_SEED0[0] >> 40) / float(1 << 24)  # 0xe220a8 / 2^24, exact in f32
    below, above = np.float32(draw - 1e-6), np.float32(draw + 1e-6)
    # pre-mix value = seed ^ tick*gamma ^ symbol*0xbf58476d1ce4e5b9 = gamma, three ways
    cases = [(GOLDEN_GAMMA, 0, 0), (0, 1, 0), (GOLDEN_GAMMA ^ 0xBF58476D1CE4E5B9, 0, 1)]
    for seed, tick, symbol in cases:
        assert lib.oracle_context_survives_dropout(seed, tick, symbol, float(below)) == 1
        assert lib.oracle_context_survives_dropout(seed, tick, symbol, float(above)) == 0
    assert lib.oracle_context_survives_dropout(123, 4, 5, 0.0) == 1  # rate 0 always survives


def test_context_key_is_fnv1a_from_the_order_basis(oracle):
    # history [0x60], order 1: bytes 0x60,0,0,0 from basis^1, so the first round
    # xors 0x60^1 = 0x61 ('a') into the standard basis
    key = oracle.context_key([0x60], 1)
    inv = pow(FNV_PRIME, -1, 1 << 64)
    assert (key * inv * inv * inv) & M64 == FNV1A64_A
    # the key of a longer history only depends on its last `order` symbols
    assert oracle.context_key([9, 8, 0x60], 1) == key
    assert oracle.context_key([9, 8, 0x60], 2) == oracle.context_key([7, 8, 0x60], 2)
    assert oracle.context_key([9, 8, 0x60], 3) != oracle.context_key([7, 8, 0x60], 3)

