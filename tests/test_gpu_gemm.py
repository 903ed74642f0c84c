"""GPU parity of the batched projection on the matrix cores (oi_gemm, gemm.hip)
against the oracle (refcpu.gemm_f16: f16-rounded dequantized rows times f16
activations, summed in float64), on the reference GEMM harness's ladder and
shapes (gemm_harness/gemm_test.odin:1058-1110) with its tolerances: error
scaled by the output magnitude <= 2e-3 for small shapes, 5e-3 for 256x64x4096,
1e-2 for the full projection shapes.  Closed-form ladder cases must be exact."""
import numpy as np
import pytest

import refcpu
from gemm_blocks import gemm_blocks, q8_const_blocks, x16
from helpers import scaled_err
from oi import ggml

pytestmark = pytest.mark.gpu


def test_ladder_exact():
    m, k, n = 16, 64, 8
    c = ggml.gemm(8, q8_const_blocks(np.ones((m, k))), m, k, x16(np.ones((n, k))))
    assert np.array_equal(c, np.full((n, m), float(k), np.float32))
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, size=(5, 64))
    c = ggml.gemm(8, q8_const_blocks(np.eye(64)), 64, 64, x16(x))
    assert np.array_equal(c, x.astype(np.float16).astype(np.float32))
    rows = np.repeat(np.arange(1, 33)[:, None], 128, axis=1)
    c = ggml.gemm(8, q8_const_blocks(rows), 32, 128, x16(np.ones((3, 128))))
    assert np.array_equal(c, np.tile(128 * np.arange(1, 33, dtype=np.float32), (3, 1)))
    xc = np.repeat(np.arange(1, 71)[:, None] / 64.0, 128, axis=1)  # 70 tokens: two token tiles
    c = ggml.gemm(8, q8_const_blocks(np.ones((32, 128))), 32, 128, x16(xc))
    assert np.array_equal(c, np.repeat((2 * np.arange(1, 71, dtype=np.float32))[:, None], 32, axis=1))


CASES = [
    (12, 8, 8, 256, 2e-3), (12, 16, 16, 512, 2e-3), (12, 32, 32, 256, 2e-3), (12, 64, 64, 512, 2e-3),
    (12, 256, 64, 4096, 5e-3), (12, 4096, 64, 4096, 1e-2), (12, 12288, 64, 4096, 1e-2),
    (14, 8, 8, 256, 2e-3), (14, 64, 64, 512, 2e-3), (14, 256, 64, 4096, 5e-3), (14, 4096, 64, 12288, 1e-2),
    (8, 8, 8, 256, 2e-3), (8, 64, 64, 512, 2e-3), (8, 1024, 64, 3072, 1e-2),
    (12, 40, 1, 512, 2e-3), (12, 40, 65, 512, 2e-3), (14, 24, 130, 256, 2e-3),
]


@pytest.mark.parametrize("kind,m,n,k,tol", CASES)
def test_gemm_vs_oracle(kind, m, n, k, tol):
    rng = np.random.default_rng(m * 31 + n * 7 + k + kind)
    w = gemm_blocks(kind, m, k, rng)
    x = x16(rng.uniform(-1, 1, size=(n, k)))
    got = ggml.gemm(kind, w, m, k, x)
    ref = refcpu.gemm_f16(w, kind, m, k, x)
    err = scaled_err(got, ref)
    assert err <= tol, "%s %dx%dx%d scaled error %.3g" % (kind, m, n, k, err)


def test_gemm_rejects_bad_shapes():
    rng = np.random.default_rng(0)
    w = gemm_blocks(12, 8, 256, rng)
    with pytest.raises(Exception):
        ggml.gemm(12, w, 8, 256, np.zeros((0, 256), np.uint16))
