"""Weight blocks and activations for the batched-projection (GEMM) tests, as
the reference's GEMM harness draws them (gemm_harness/gemm_test.odin:828-845,
1008-1016): Q4_K d in [0.02, 0.2], dmin in [0, 0.05], random scale and quant
bytes; Q6_K d in [0.02, 0.2], random ql/qh/scale bytes; activations uniform in
[-1, 1] as f16.  (Q8_0, which the harness does not cover, uses the same d
range and random int8 quants.)"""
import numpy as np

BLOCK = {8: (32, 34), 12: (256, 144), 14: (256, 210)}


def gemm_blocks(kind, rows, cols, rng):
    e, b = BLOCK[kind]
    n = rows * (cols // e)
    raw = rng.integers(0, 256, size=(n, b), dtype=np.uint8)
    d = (rng.random(n) * 0.18 + 0.02).astype(np.float16).view(np.uint8).reshape(n, 2)
    if kind == 12:
        raw[:, 0:2] = d
        raw[:, 2:4] = (rng.random(n) * 0.05).astype(np.float16).view(np.uint8).reshape(n, 2)
    elif kind == 14:
        raw[:, 208:210] = d
    else:
        raw[:, 0:2] = d
    return raw.reshape(-1)


def q8_const_blocks(qmat):
    """Q8_0 rows with d = 1.0 and the given int8 quants (rows x cols, cols % 32 == 0):
    the dequantized matrix is exactly qmat."""
    rows, cols = qmat.shape
    q = np.asarray(qmat, np.int8).reshape(rows, cols // 32, 32)
    out = np.zeros((rows, cols // 32, 34), np.uint8)
    out[:, :, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def x16(values):
    return np.asarray(values, np.float16).view(np.uint16)
