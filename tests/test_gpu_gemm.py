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
    m, k, n = 16, 256, 8
    c = ggml.gemm(8, q8_const_blocks(np.ones((m, k))), m, k, x16(np.ones((n, k))))
    assert np.array_equal(c, np.full((n, m), float(k), np.float32))
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, size=(5, 256))
    c = ggml.gemm(8, q8_const_blocks(np.eye(256)[:64]), 64, 256, x16(x))
    assert np.array_equal(c, x[:, :64].astype(np.float16).astype(np.float32))
    rows = np.repeat(np.arange(1, 33)[:, None], 256, axis=1)
    c = ggml.gemm(8, q8_const_blocks(rows), 32, 256, x16(np.ones((3, 256))))
    assert np.array_equal(c, np.tile(256 * np.arange(1, 33, dtype=np.float32), (3, 1)))
    xc = np.repeat(np.arange(1, 71)[:, None] / 64.0, 256, axis=1)  # 70 tokens: two token tiles
    c = ggml.gemm(8, q8_const_blocks(np.ones((32, 256))), 32, 256, x16(xc))
    assert np.array_equal(c, np.repeat((4 * np.arange(1, 71, dtype=np.float32))[:, None], 32, axis=1))


CASES = [
    (12, 8, 8, 256, 2e-3), (12, 16, 16, 512, 2e-3), (12, 32, 32, 256, 2e-3), (12, 64, 64, 512, 2e-3),
    (12, 256, 64, 4096, 5e-3), (12, 4096, 64, 4096, 1e-2), (12, 12288, 64, 4096, 1e-2),
    (14, 8, 8, 256, 2e-3), (14, 64, 64, 512, 2e-3), (14, 256, 64, 4096, 5e-3), (14, 4096, 64, 12288, 1e-2),
    (8, 8, 8, 256, 2e-3), (8, 64, 64, 512, 2e-3), (8, 1024, 64, 3072, 1e-2), (8, 130, 64, 1280, 2e-3),
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


def _q4k_wide_range_blocks(rows, rng):
    """Q4_K rows of one super-block with d in [0.5, 2) and dmin in [2^-16, 2^-12):
    d*sc*q - dmin*m then spans more than 24 bits, so the f32 dequantization
    rounds, and rounding that value to f16 differs from rounding the exact
    value to f16 once in about 1 of 8000 weights."""
    raw = rng.integers(0, 256, size=(rows, 144), dtype=np.uint8)
    raw[:, 0:2] = (0.5 + 1.5 * rng.random(rows)).astype(np.float16).view(np.uint8).reshape(rows, 2)
    raw[:, 2:4] = (2.0 ** rng.uniform(-16, -12, rows)).astype(np.float16).view(np.uint8).reshape(rows, 2)
    return raw


def _q4k_double_rounding_sensitive(raw):
    """Weights whose f16 value depends on rounding to f32 first (float64 stands in
    for the exact value, close enough to count them)."""
    d = raw[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    dmin = raw[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float64)
    n = 0
    for r in range(raw.shape[0]):
        q12 = raw[r, 4:16]
        for j in range(8):
            sc, mc = refcpu.get_scale_min_k4(j, q12)
            qs = raw[r, 16 + 32 * (j // 2):16 + 32 * (j // 2) + 32]
            q = (qs & 15) if j % 2 == 0 else (qs >> 4)
            d1, m = np.float32(d[r] * sc), np.float32(dmin[r] * mc)  # exact products
            x = float(d1) * q.astype(np.float64) - float(m)
            once = x.astype(np.float16)
            twice = x.astype(np.float32).astype(np.float16)
            n += int(np.count_nonzero(once != twice))
    return n


def test_gemm_staged_weights_bit_exact():
    """One-hot activations (token t has 1.0 at column t and zeros elsewhere) make
    C[t][r] the staged weight f16(dequant(W)[r][t]) itself: one exact product,
    every other term zero.  The staging (dequantize in f32 as ggml/quant.odin
    does, then round to f16) is compared bit for bit over 4096 Q4_K rows drawn
    so that the f32 dequantization rounds; the rows hold weights where rounding
    the exact value to f16 in one step (v_fma_mix*_f16) would differ."""
    rng = np.random.default_rng(2024)
    m, k = 4096, 256
    raw = _q4k_wide_range_blocks(m, rng)
    assert _q4k_double_rounding_sensitive(raw[:512]) >= 5  # the draw exercises the distinction
    x = x16(np.eye(k))
    got = ggml.gemm(12, raw.reshape(-1), m, k, x)
    ref = refcpu.gemm_f16(raw.reshape(-1), 12, m, k, x)
    bad = np.flatnonzero(got.astype(np.float64).ravel() != ref.ravel())
    assert bad.size == 0, "%d staged weights differ, first at %s" % (bad.size, np.unravel_index(bad[:4], got.shape))


def test_gemm_rejects_bad_shapes():
    rng = np.random.default_rng(0)
    w = gemm_blocks(12, 8, 256, rng)
    with pytest.raises(Exception):
        ggml.gemm(12, w, 8, 256, np.zeros((0, 256), np.uint16))
    w8 = gemm_blocks(8, 8, 128, rng)  # K must be a multiple of 256 (one chunk), as the reference's MMQ
    with pytest.raises(Exception):
        ggml.gemm(8, w8, 8, 128, np.zeros((4, 128), np.uint16))


class _Hip:
    """Device buffers from the HIP runtime the library is linked against."""

    def __init__(self):
        import ctypes
        self.ct = ctypes
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.bufs = []

    def alloc(self, nbytes):
        p = self.ct.c_void_p()
        assert self.lib.hipMalloc(self.ct.byref(p), self.ct.c_size_t(max(nbytes, 16))) == 0
        self.bufs.append(p)
        return p.value

    def put(self, arr):
        p = self.alloc(arr.nbytes)
        assert self.lib.hipMemcpy(self.ct.c_void_p(p), arr.ctypes.data_as(self.ct.c_void_p),
                                  self.ct.c_size_t(arr.nbytes), 1) == 0
        return p

    def get(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.lib.hipDeviceSynchronize() == 0
        assert self.lib.hipMemcpy(out.ctypes.data_as(self.ct.c_void_p), self.ct.c_void_p(p),
                                  self.ct.c_size_t(out.nbytes), 2) == 0
        return out

    def close(self):
        for p in self.bufs:
            self.lib.hipFree(p)


@pytest.mark.parametrize("kind,m,n,k", [(12, 4096, 64, 4096), (14, 1024, 40, 12288)])
def test_gemm_workspace_split(kind, m, n, k):
    """K split over workgroups (partial products in the caller's workspace,
    summed in slice order) and unsplit (no workspace) both match the oracle;
    the split result is bit-identical from run to run (no atomics)."""
    rng = np.random.default_rng(kind + m + n)
    wb = gemm_blocks(kind, m, k, rng)
    x = x16(rng.uniform(-1, 1, size=(n, k)))
    ref = refcpu.gemm_f16(wb, kind, m, k, x)
    w = ggml.DeviceWeights(kind, wb, m, k)
    hip = _Hip()
    try:
        wsb = w.gemm_workspace_bytes(n)
        assert wsb > 0, "this shape is expected to split K"
        xd, cd, ws = hip.put(np.ascontiguousarray(x)), hip.alloc(n * m * 4), hip.alloc(wsb)
        w.launch_gemm(xd, n, cd, ws, wsb)
        split1 = hip.get(cd, (n, m), np.float32)
        w.launch_gemm(xd, n, cd, ws, wsb)
        split2 = hip.get(cd, (n, m), np.float32)
        w.launch_gemm(xd, n, cd, None, 0)
        whole = hip.get(cd, (n, m), np.float32)
        w.launch_gemm(xd, n, cd, ws, wsb // 2)  # room for fewer slices
        fewer = hip.get(cd, (n, m), np.float32)
    finally:
        hip.close()
        w.free()
    assert np.array_equal(split1, split2)
    for got in (split1, whole, fewer):
        assert scaled_err(got, ref) <= 1e-2
