"""Shared helpers for the tests."""
import struct

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


def gguf_fields(data):
    """Offsets of a GGUF v3 header's fields: a list of (name, offset, size)."""
    out = [("magic", 0, 4), ("version", 4, 4), ("n_tensors", 8, 8), ("n_meta", 16, 8)]
    n_tensors, n_meta = struct.unpack_from("<QQ", data, 8)
    pos = 24
    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def value(t, pos, name):
        if t in sizes:
            out.append((name + ".value", pos, sizes[t]))
            return pos + sizes[t]
        if t == 8:
            (n,) = struct.unpack_from("<Q", data, pos)
            out.append((name + ".strlen", pos, 8))
            return pos + 8 + n
        if t == 9:
            (et,) = struct.unpack_from("<I", data, pos)
            (cnt,) = struct.unpack_from("<Q", data, pos + 4)
            out.append((name + ".atype", pos, 4))
            out.append((name + ".count", pos + 4, 8))
            pos += 12
            for _ in range(cnt):
                pos = value(et, pos, name + "[]")
            return pos
        raise ValueError(t)

    for _ in range(n_meta):
        (kl,) = struct.unpack_from("<Q", data, pos)
        key = data[pos + 8:pos + 8 + kl].decode()
        out.append(("meta:%s.keylen" % key, pos, 8))
        pos += 8 + kl
        (t,) = struct.unpack_from("<I", data, pos)
        out.append(("meta:%s.type" % key, pos, 4))
        pos = value(t, pos + 4, "meta:" + key)
    for _ in range(n_tensors):
        (nl,) = struct.unpack_from("<Q", data, pos)
        name = data[pos + 8:pos + 8 + nl].decode()
        out.append(("tensor:%s.namelen" % name, pos, 8))
        pos += 8 + nl
        (nd,) = struct.unpack_from("<I", data, pos)
        out.append(("tensor:%s.n_dims" % name, pos, 4))
        pos += 4
        for d in range(nd):
            out.append(("tensor:%s.dim%d" % (name, d), pos, 8))
            pos += 8
        out.append(("tensor:%s.type" % name, pos, 4))
        out.append(("tensor:%s.offset" % name, pos + 4, 8))
        pos += 12
    out.append(("end", pos, 0))
    return out


def gguf_tensor_data(data):
    """{tensor name: (absolute byte offset of its data, GGML type)} of a GGUF v3
    file held in `data` (the data section starts at the first multiple of
    general.alignment, default 32, after the tensor infos)."""
    fields = gguf_fields(data)
    align = 32
    for name, off, size in fields:
        if name == "meta:general.alignment.value":
            align = int.from_bytes(data[off:off + size], "little")
    start = -(-fields[-1][1] // align) * align
    out = {}
    for name, off, size in fields:
        if name.startswith("tensor:") and name.endswith(".offset"):
            t = name[len("tensor:"):-len(".offset")]
            out[t] = (start + int.from_bytes(data[off:off + 8], "little"),
                      int.from_bytes(data[off - 4:off], "little"))
    return out
