"""The allocation-free routed-expert FFN (oi_moe_ffn_launch_noalloc: the
library's own fixed device workspace, no hipMalloc) against the entry point
it varies (oi_moe_ffn_launch with a caller workspace), through the C ABI, on
two calls in a row -- the config-4 shape, then a smaller one -- so a stale
workspace from the first call would show in the second; outputs bit-equal,
and within the oracle's bar.  Oversized dims are rejected with OI_E_ARG."""
import ctypes
import numpy as np
import pytest

import refcpu
from oi import _native, ggml
from helpers import DeviceBuffer
from test_moe_oracle import make_moe

pytestmark = pytest.mark.gpu


def _run(E, k, dim, inter, etype, rtype, seed, norm=1):
    rng = np.random.default_rng(seed)
    rb, gb, ub, db = make_moe(rng, E, dim, inter, etype, rtype=rtype)
    x = rng.standard_normal(dim).astype(np.float32)
    w = [ggml.DeviceWeights(rtype, rb, E, dim), ggml.DeviceWeights(etype, gb, E * inter, dim),
         ggml.DeviceWeights(etype, ub, E * inter, dim), ggml.DeviceWeights(etype, db, E * dim, inter)]
    d = _native.MoeDims(E, k, dim, inter, norm)
    L = _native.hip()
    nan = np.full(dim, np.nan, np.float32)
    xd, y_ws, y_na = DeviceBuffer(dim * 4).from_host(x), DeviceBuffer(dim * 4).from_host(nan), \
        DeviceBuffer(dim * 4).from_host(nan)
    ws = DeviceBuffer(int(L.oi_moe_workspace_bytes(ctypes.byref(d))))
    try:
        _native.check(L.oi_moe_ffn_launch(ctypes.byref(d), *[ww.h for ww in w], xd.ptr, ws.ptr, y_ws.ptr, None))
        _native.check(L.oi_moe_ffn_launch_noalloc(ctypes.byref(d), *[ww.h for ww in w], xd.ptr, y_na.ptr, None))
        xd.sync()
        out_ws, out_na = y_ws.to_host().view(np.float32), y_na.to_host().view(np.float32)
    finally:
        for b in (xd, y_ws, y_na, ws):
            b.free()
        for ww in w:
            ww.free()
    ry, _, _ = refcpu.moe_ffn(E, k, dim, inter, norm, rtype, rb, etype, gb, ub, db, x)
    return out_ws, out_na, ry


def test_noalloc_equals_workspace_entry_two_calls():
    for case in [(128, 8, 2048, 768, 12, 12, 41), (16, 4, 256, 128, 8, 0, 42)]:
        print("case E=%d top_k=%d dim=%d inter=%d expert type %d router type %d" % case[:6], flush=True)
        y_ws, y_na, ry = _run(*case)
        assert np.all(np.isfinite(y_na))
        assert np.array_equal(y_ws.view(np.uint32), y_na.view(np.uint32))
        assert np.max(np.abs(np.float64(y_na) - ry)) / np.max(np.abs(ry)) <= 1e-4


def test_noalloc_rejects_dims_beyond_its_workspace():
    rng = np.random.default_rng(0)
    rb, gb, ub, db = make_moe(rng, 4, 128, 64, 8)
    w = [ggml.DeviceWeights(0, rb, 4, 128), ggml.DeviceWeights(8, gb, 4 * 64, 128),
         ggml.DeviceWeights(8, ub, 4 * 64, 128), ggml.DeviceWeights(8, db, 4 * 128, 64)]
    # 64 + 2 * 32 + 32 * 4160 floats > the 131072-float workspace
    d = _native.MoeDims(64, 32, 128, 4160, 1)
    rc = _native.hip().oi_moe_ffn_launch_noalloc(ctypes.byref(d), *[ww.h for ww in w], None, None, None)
    assert rc == -1  # OI_E_ARG
    assert b"exceeds" in _native.hip().oi_last_error()
    for ww in w:
        ww.free()
