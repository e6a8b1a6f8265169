"""Pins of the fp8 oracle (oracle.floatops.e4m3fn_to_f64, matmul_fp8).

The reference has no fp8 type, so there are no golden vectors; the decode is
pinned by the OCP e4m3fn closed forms (1.0, the largest finite value, the
smallest normal and subnormal, negative zero, NaN) and by torch's own
float8_e4m3fn conversion of all 256 codes (a library routine); the matmul by a
brute-force triple loop on a tiny case, by exactly representable identities
(identity matrix, a constant row), and by planted mistakes (exponent bias 8,
subnormals as normals, a transposed operand) that each fail one of them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import rng

ALL_CODES = np.arange(256, dtype=np.uint8)


def random_codes(generator: np.random.Generator, shape: tuple[int, ...]) -> np.ndarray:
    """Finite e4m3fn codes (NaN codes 0x7F and 0xFF replaced by zero)."""
    codes = generator.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((codes & 0x7F) == 0x7F, np.uint8(0), codes)


def test_decode_closed_forms():
    d = oracle.e4m3fn_to_f64(ALL_CODES)
    assert d[0x38] == 1.0
    assert d[0x7E] == 448.0 and d[0xFE] == -448.0
    assert d[0x08] == 2.0**-6  # smallest normal
    assert d[0x01] == 2.0**-9  # smallest subnormal
    assert d[0x07] == 7 * 2.0**-9  # largest subnormal
    assert d[0x00] == 0.0 and d[0x80] == 0.0 and np.signbit(d[0x80])
    assert np.isnan(d[0x7F]) and np.isnan(d[0xFF])
    assert np.count_nonzero(np.isnan(d)) == 2
    finite = d[~np.isnan(d)]
    positive = np.sort(finite[finite > 0])
    assert len(positive) == 126 and np.all(np.diff(positive) > 0)


def test_decode_matches_torch_float8_e4m3fn():
    mine = oracle.e4m3fn_to_f64(ALL_CODES)
    theirs = torch.from_numpy(ALL_CODES.copy()).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    np.testing.assert_array_equal(np.isnan(mine), np.isnan(theirs))
    np.testing.assert_array_equal(mine[~np.isnan(mine)], theirs[~np.isnan(theirs)])


def test_matmul_matches_a_triple_loop():
    g = rng(801)
    x = random_codes(g, (3, 5))
    w = random_codes(g, (5, 4))
    dx = oracle.e4m3fn_to_f64(x)
    dw = oracle.e4m3fn_to_f64(w)
    expected = np.zeros((3, 4))
    for i in range(3):
        for j in range(4):
            expected[i, j] = 0.75 * sum(dx[i, k] * dw[k, j] for k in range(5))
    np.testing.assert_allclose(oracle.matmul_fp8(x, w, 0.75), expected, rtol=1e-15, atol=0)


def test_matmul_identities():
    g = rng(802)
    x = random_codes(g, (6, 16))
    eye = np.where(np.eye(16, dtype=bool), np.uint8(0x38), np.uint8(0))
    np.testing.assert_array_equal(oracle.matmul_fp8(x, eye, 1.0), oracle.e4m3fn_to_f64(x))
    ones = np.full((1, 16), 0x38, dtype=np.uint8)
    w = random_codes(g, (16, 3))
    np.testing.assert_array_equal(oracle.matmul_fp8(ones, w, 2.0)[0], 2.0 * oracle.e4m3fn_to_f64(w).sum(axis=0))


def _decode_bias8(codes):
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 0xF, c & 7
    v = np.where(e == 0, np.ldexp(m.astype(float), -10), np.ldexp(1 + m / 8, e - 8))
    return np.where(c & 0x80, -v, v)


def _decode_no_subnormals(codes):
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 0xF, c & 7
    v = np.ldexp(1 + m / 8, e - 7)
    return np.where(c & 0x80, -v, v)


@pytest.mark.parametrize("mistake", ["bias8", "no_subnormals", "transposed"])
def test_a_planted_fp8_mistake_is_caught(mistake):
    reference = torch.from_numpy(ALL_CODES.copy()).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    finite = ~np.isnan(reference)
    if mistake == "bias8":
        assert not np.array_equal(_decode_bias8(ALL_CODES)[finite], reference[finite])
    elif mistake == "no_subnormals":
        assert not np.array_equal(_decode_no_subnormals(ALL_CODES)[finite], reference[finite])
    else:
        g = rng(803)
        x = random_codes(g, (4, 4))
        w = random_codes(g, (4, 4))
        dx, dw = oracle.e4m3fn_to_f64(x), oracle.e4m3fn_to_f64(w)
        assert not np.array_equal(dx @ dw.T, oracle.matmul_fp8(x, w, 1.0))
