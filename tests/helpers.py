"""Shared helpers for the tests."""
import numpy as np


def scaled_err(got, ref):
    """max|got-ref| / max|ref| -- the error measure of the reference's GEMM
    harness (gemm_harness/gemm_test.odin:885-888)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def random_blocks(kind, nblocks, rng):
    """Random bytes for `nblocks` blocks of `kind`, with the f16 scale fields
    set to finite values of assorted magnitude (any byte pattern is a valid
    block for dequant; finite scales keep comparisons free of inf/nan)."""
    e, b = {8: (32, 34), 12: (256, 144), 14: (256, 210), 1: (1, 2), 0: (1, 4), 2: (32, 18), 3: (32, 20),
            6: (32, 22), 7: (32, 24)}[kind]
    raw = rng.integers(0, 256, size=(nblocks, b), dtype=np.uint8)

    def f16_field(n):
        mag = rng.choice([1e-6, 1e-4, 1e-3, 0.01, 0.1, 1.0, 100.0], size=n)
        v = (rng.standard_normal(n) * mag).astype(np.float16)
        v[rng.random(n) < 0.05] = 0
        return v.view(np.uint16)

    if kind in (8, 2, 6):  # d
        raw[:, 0:2] = f16_field(nblocks).view(np.uint8).reshape(nblocks, 2)
    elif kind in (12, 3, 7):  # d, then dmin (K) or m (Q4_1 / Q5_1)
        raw[:, 0:2] = f16_field(nblocks).view(np.uint8).reshape(nblocks, 2)
        raw[:, 2:4] = f16_field(nblocks).view(np.uint8).reshape(nblocks, 2)
    elif kind == 14:
        raw[:, 208:210] = f16_field(nblocks).view(np.uint8).reshape(nblocks, 2)
    elif kind == 1:
        v = (rng.standard_normal(nblocks) * 3).astype(np.float16)
        raw = v.view(np.uint8).reshape(nblocks, 2)
    elif kind == 0:
        v = rng.standard_normal(nblocks).astype(np.float32)
        raw = v.view(np.uint8).reshape(nblocks, 4)
    return raw.reshape(-1)


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


class DeviceBuffer:
    """Device memory from the HIP runtime the library itself uses
    (libamdhip64), for tests that hand device pointers to the C ABI."""

    def __init__(self, nbytes):
        import ctypes
        self._hip = ctypes.CDLL("libamdhip64.so")
        self.nbytes = max(int(nbytes), 1)
        self.ptr = ctypes.c_void_p()
        if self._hip.hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(self.nbytes)) != 0:
            raise RuntimeError("hipMalloc failed")

    def from_host(self, a):
        import ctypes
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("host array larger than the buffer")
        if self._hip.hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1) != 0:
            raise RuntimeError("hipMemcpy failed")
        return self

    def sync(self):
        if self._hip.hipDeviceSynchronize() != 0:
            raise RuntimeError("hipDeviceSynchronize failed")

    def to_host(self, n=None):
        import ctypes
        out = np.empty(self.nbytes if n is None else n, np.uint8)
        if self._hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, ctypes.c_size_t(out.size), 2) != 0:
            raise RuntimeError("hipMemcpy failed")
        return out

    def free(self):
        if self.ptr:
            self._hip.hipFree(self.ptr)
            self.ptr = None
