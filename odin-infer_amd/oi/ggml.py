"""Quant codec, mirroring the reference's `ggml` package (ggml/quant.odin).

dequant_row runs the device decode (liboi_hip.so) and is bit-exact with the
reference's dequant_row; row_byte_size / block_info are the same tables.
"""
import ctypes
from enum import IntEnum

import numpy as np

from . import _native
from ._native import check


class GGML_Type(IntEnum):  # ggml/gguf.odin:27-42
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15


_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
          10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}

DEVICE_TYPES = (GGML_Type.F32, GGML_Type.F16, GGML_Type.Q8_0, GGML_Type.Q4_K, GGML_Type.Q6_K)


def ggml_block_info(kind):
    """ggml/quant.odin:10-42 -> (elems, bytes)."""
    return _BLOCK.get(int(kind), (1, 4))


def row_byte_size(kind, n):
    """ggml/quant.odin:44-47."""
    e, b = ggml_block_info(kind)
    return (n // e) * b


def is_supported_quant(kind):
    """ggml/quant.odin:49-55 (the reference's CPU set)."""
    return int(kind) in (0, 1, 2, 3, 6, 7, 8, 12, 14)


def dequant_row(kind, src, n):
    """Device dequant of n elements of `kind` blocks (host bytes) -> float32."""
    src = np.ascontiguousarray(src, np.uint8)
    out = np.empty(n, np.float32)
    check(_native.hip().oi_dequant(int(kind), src.ctypes.data, int(n), out.ctypes.data))
    return out


def gemv(kind, w_blocks, rows, cols, x):
    """y = W x on the device (host in, host out)."""
    w = np.ascontiguousarray(w_blocks, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    check(_native.hip().oi_gemv(int(kind), w.ctypes.data, int(rows), int(cols), x.ctypes.data, y.ctypes.data))
    return y


def gemm(kind, w_blocks, rows, cols, x16):
    """Batched projection on the matrix cores (host in, host out):
    c[t][r] = sum_k f16(dequant(W)[r][k]) * x16[t][k], f32 accumulation.
    x16: uint16 (f16 bits) [n][cols] -> float32 [n][rows]."""
    w = np.ascontiguousarray(w_blocks, np.uint8)
    x = np.ascontiguousarray(x16, np.uint16)
    n = x.shape[0]
    c = np.empty((n, rows), np.float32)
    check(_native.hip().oi_gemm(int(kind), w.ctypes.data, int(rows), int(cols), x.ctypes.data, int(n), c.ctypes.data))
    return c


class DeviceWeights:
    """A matrix resident in HBM in the GEMV layout (oi_weights_upload)."""

    def __init__(self, kind, w_blocks, rows, cols):
        w = np.ascontiguousarray(w_blocks, np.uint8)
        h = ctypes.c_void_p()
        check(_native.hip().oi_weights_upload(int(kind), w.ctypes.data, int(rows), int(cols), ctypes.byref(h)))
        self.h = h.value
        self.rows, self.cols, self.kind = rows, cols, kind
        self.nbytes = _native.hip().oi_weights_bytes(self.h)

    def launch(self, x_dev_ptr, y_dev_ptr, stream=None):
        check(_native.hip().oi_gemv_launch(self.h, x_dev_ptr, y_dev_ptr, stream))

    def gemm_workspace_bytes(self, n):
        return int(_native.hip().oi_gemm_workspace_bytes(self.h, int(n)))

    def launch_gemm(self, x_dev_ptr, n, c_dev_ptr, ws_dev_ptr=None, ws_bytes=0, stream=None):
        check(_native.hip().oi_gemm_launch(self.h, x_dev_ptr, int(n), c_dev_ptr, ws_dev_ptr, int(ws_bytes), stream))

    def free(self):
        if self.h:
            _native.hip().oi_weights_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
