"""Pins of the oracle's batched projection (refcpu.ref_gemm_f16), CPU only.

The reference's GEMM harness ladder (gemm_harness/gemm_test.odin:1058-1067):
all-ones, identity, row-distinct and column-distinct operands have closed-form
products; random operands are checked against an independent numpy float64
product of the f16-rounded, dequantized rows (dequant_row itself is pinned
bit-exactly in test_oracle.py)."""
import numpy as np
import pytest

import refcpu
from gemm_blocks import gemm_blocks, q8_const_blocks, x16


def test_all_ones():
    m, k, n = 8, 64, 8
    c = refcpu.gemm_f16(q8_const_blocks(np.ones((m, k))), 8, m, k, x16(np.ones((n, k))))
    assert np.array_equal(c, np.full((n, m), float(k)))


def test_identity():
    k = 64
    rng = np.random.default_rng(1)
    x = rng.uniform(-1, 1, size=(5, k))
    c = refcpu.gemm_f16(q8_const_blocks(np.eye(k)), 8, k, k, x16(x))
    assert np.array_equal(c, x.astype(np.float16).astype(np.float64))


def test_row_and_column_distinct():
    m, k, n = 8, 96, 6
    rows = np.repeat(np.arange(1, m + 1)[:, None], k, axis=1)
    cols_x = np.repeat(np.arange(1, n + 1)[:, None], k, axis=1)
    c = refcpu.gemm_f16(q8_const_blocks(rows), 8, m, k, x16(np.ones((n, k))))
    assert np.array_equal(c, np.tile(k * np.arange(1, m + 1, dtype=np.float64), (n, 1)))
    c = refcpu.gemm_f16(q8_const_blocks(np.ones((m, k))), 8, m, k, x16(cols_x))
    assert np.array_equal(c, np.repeat(k * np.arange(1, n + 1, dtype=np.float64)[:, None], m, axis=1))


@pytest.mark.parametrize("kind,m,k,n", [(12, 16, 512, 9), (14, 8, 512, 5), (8, 12, 256, 7)])
def test_random_vs_numpy(kind, m, k, n):
    rng = np.random.default_rng(kind * 7 + n)
    w = gemm_blocks(kind, m, k, rng)
    x = x16(rng.uniform(-1, 1, size=(n, k)))
    a = refcpu.dequant_row(kind, w, m * k).reshape(m, k).astype(np.float16).astype(np.float64)
    want = x.view(np.float16).astype(np.float64) @ a.T
    got = refcpu.gemm_f16(w, kind, m, k, x)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    # a planted transpose (x against the wrong operand axis) is caught
    assert not np.allclose(got, (x.view(np.float16).astype(np.float64)[:, ::-1] @ a.T), rtol=1e-3)
