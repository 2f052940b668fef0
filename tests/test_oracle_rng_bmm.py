"""Pins the oracle's dropout (Philox-4x32-10 stream), causal mask and batched
products: the published Philox known-answer vectors, the properties the
reference's tests/python/test_dropout.py and test_bmm.py assert, closed forms,
and bit-exact agreement with oracle/_ref (the reference's own CPU build)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O

f32 = np.float32
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference tree)")

# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key, expected).
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    np.testing.assert_array_equal(O.philox4x32_10(ctr, key), np.array(want, np.uint32))


def test_philox_uniform_is_word0_scaled():
    # counter = (idx lo, idx hi, 0, 0), key = (seed lo, seed hi); word 0 * 2^-32
    for seed, idx in ((0, 0), (5, 1), (2**40 + 3, 2**33 + 7), (2**64 - 1, 2**64 - 1)):
        w = O.philox4x32_10([idx & 0xFFFFFFFF, idx >> 32, 0, 0], [seed & 0xFFFFFFFF, seed >> 32])
        # uint32 -> float rounds to nearest even, as C's conversion does
        assert O.philox_uniform(seed, idx) == f32(np.float32(w[0]) * f32(2.0 ** -32))


def test_dropout_reference_properties():
    # tests/python/test_dropout.py:16-64 restated on the oracle
    out, _ = O.dropout(np.ones(20000, f32), 0.3, 0)
    assert abs(float((out == 0).mean()) - 0.3) < 0.02
    out, _ = O.dropout(np.full(1000, 2.0, f32), 0.4, 1)
    np.testing.assert_allclose(out[out != 0], 2.0 / 0.6, atol=1e-5)
    x = np.random.default_rng(0).standard_normal(50).astype(f32)
    np.testing.assert_array_equal(O.dropout(x, 0.5, 123)[0], O.dropout(x, 0.5, 123)[0])
    assert not np.array_equal(O.dropout(np.ones(200, f32), 0.5, 7)[0], O.dropout(np.ones(200, f32), 0.5, 8)[0])
    x = np.random.default_rng(0).standard_normal(32).astype(f32)
    out, mask = O.dropout(x, 0.4, 42)
    np.testing.assert_array_equal(mask, np.where(out != 0, f32(1) / f32(0.6), 0).astype(f32))
    np.testing.assert_array_equal(out, x * mask)


def test_dropout_keep_rule_by_brute_force():
    # element i survives iff philox_uniform(seed, i) >= p
    x = np.arange(1, 301, dtype=f32)
    for p in (0.1, 0.5, 0.9):
        _, mask = O.dropout(x, p, 99)
        keep = np.array([O.philox_uniform(99, i) >= f32(p) for i in range(300)])
        np.testing.assert_array_equal(mask != 0, keep)


def test_causal_mask_closed_form():
    x = np.random.default_rng(0).standard_normal((3, 17, 17)).astype(f32)
    tri = np.tril(np.ones((17, 17), bool))
    np.testing.assert_array_equal(O.causal_mask(x), np.where(tri, x, -np.inf).astype(f32))
    np.testing.assert_array_equal(O.causal_mask(x, 0.0), np.where(tri, x, 0).astype(f32))


def test_bmm_closed_forms():
    # tests/python/test_bmm.py:15-37 (numpy products, float64 here)
    rng = np.random.default_rng(0)
    a = rng.standard_normal((6, 4, 5)).astype(f32)
    b = rng.standard_normal((6, 5, 7)).astype(f32)
    bt = rng.standard_normal((6, 7, 5)).astype(f32)
    at = rng.standard_normal((6, 5, 4)).astype(f32)
    a64 = a.astype(np.float64)
    np.testing.assert_allclose(O.bmm("bmm", a, b), a64 @ b, atol=1e-5)
    np.testing.assert_allclose(O.bmm("bmm_a_bt", a, bt), a64 @ bt.transpose(0, 2, 1), atol=1e-5)
    np.testing.assert_allclose(O.bmm("bmm_at_b", at, b), at.astype(np.float64).transpose(0, 2, 1) @ b, atol=1e-5)
    assert O.bmm("bmm", np.zeros((0, 4, 5), f32), np.zeros((0, 5, 7), f32)).shape == (0, 4, 7)


@needs_ref
def test_ref_bitexact_dropout_mask_bmm():
    rng = np.random.default_rng(3)
    for seed, idx in ((0, 0), (2026, 12345), (2**40 + 3, 2**33 + 5)):
        assert O.ref_philox_uniform(seed, idx) == O.philox_uniform(seed, idx)
    x = rng.standard_normal(1000).astype(f32)
    for p, seed in ((0.3, 2026), (0.5, 7), (0.9, 2**35 + 1)):
        y, dx = O.ref_dropout(x, p, seed, grad=True)
        out, mask = O.dropout(x, p, seed)
        np.testing.assert_array_equal(y, out)
        np.testing.assert_array_equal(dx, mask)
    s = rng.standard_normal((4, 9, 9)).astype(f32)
    g = rng.standard_normal((4, 9, 9)).astype(f32)
    y, dx = O.ref_causal_mask(s, g)
    np.testing.assert_array_equal(y, O.causal_mask(s))
    np.testing.assert_array_equal(dx, O.causal_mask(g, 0.0))
    a = rng.standard_normal((3, 13, 11)).astype(f32)
    b = rng.standard_normal((3, 11, 6)).astype(f32)
    bt = rng.standard_normal((3, 6, 11)).astype(f32)
    at = rng.standard_normal((3, 11, 13)).astype(f32)
    np.testing.assert_array_equal(O.ref_bmm("bmm", a, b), O.bmm("bmm", a, b))
    np.testing.assert_array_equal(O.ref_bmm("bmm_a_bt", a, bt), O.bmm("bmm_a_bt", a, bt))
    np.testing.assert_array_equal(O.ref_bmm("bmm_at_b", at, b), O.bmm("bmm_at_b", at, b))
