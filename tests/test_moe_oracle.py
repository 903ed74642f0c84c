"""The oracle's routed-expert FFN (refcpu.ref_moe_ffn; HF Qwen3-MoE
convention, the reference has no MoE code) pinned by a float64 brute force on
the same dequantized weights, a tie case (equal router logits pick the lower
id first), and the renormalization closed form; the float64 model without
renormalization must fail the bound."""
import numpy as np
import pytest

import refcpu
from oi import synth


def make_moe(rng, E, dim, inter, etype, tie=None, rtype=0):
    """Router (F32, or quantized to rtype), gate, up, down weights."""
    router = (rng.standard_normal((E, dim)) * 0.1).astype(np.float32)
    if tie is not None:  # experts tie[0] and tie[1] share the largest router row
        router[list(tie)] = router[0] * 0 + 0.5 / np.sqrt(dim)
    seed = int(rng.integers(1, 2 ** 31))  # expert matrices from the seeded C generator (fast at 512 experts)
    gate = synth.tensor_f32(seed, "gate", E * inter, dim, sigma=0.05)
    up = synth.tensor_f32(seed, "up", E * inter, dim, sigma=0.05)
    down = synth.tensor_f32(seed, "down", E * dim, inter, sigma=0.05)
    q = lambda m: synth.quantize_rows(etype, m)
    rb = router.view(np.uint8).reshape(-1) if rtype == 0 else synth.quantize_rows(rtype, router)
    return rb, q(gate), q(up), q(down)


def moe_f64(E, k, dim, inter, norm, rtype, rb, etype, gb, ub, db, x, renorm=True):
    deq = lambda kind, blocks, rows, cols: refcpu.dequant_row(kind, blocks, rows * cols).reshape(rows, cols).astype(
        np.float64)
    R = deq(rtype, rb, E, dim)
    G, U, D = deq(etype, gb, E * inter, dim), deq(etype, ub, E * inter, dim), deq(etype, db, E * dim, inter)
    x = np.float64(x)
    lg = R @ x
    p = np.exp(lg - lg.max())
    p /= p.sum()
    ids = sorted(range(E), key=lambda e: (-p[e], e))[:k]
    w = p[ids] / (p[ids].sum() if (norm and renorm) else 1.0)
    y = np.zeros(dim)
    for wk, e in zip(w, ids):
        g = G[e * inter:(e + 1) * inter] @ x
        u = U[e * inter:(e + 1) * inter] @ x
        y += wk * (D[e * dim:(e + 1) * dim] @ (g / (1 + np.exp(-g)) * u))
    return y, np.array(ids), w


@pytest.mark.parametrize("E,k,dim,inter,etype,rtype", [(16, 4, 256, 128, 8, 0), (8, 2, 256, 256, 12, 0),
                                                        (6, 6, 128, 64, 8, 0), (32, 8, 512, 256, 12, 12)])
def test_moe_vs_float64(E, k, dim, inter, etype, rtype):
    rng = np.random.default_rng(E * 13 + k)
    rb, gb, ub, db = make_moe(rng, E, dim, inter, etype, rtype=rtype)
    x = rng.standard_normal(dim).astype(np.float32)
    y, ids, w = refcpu.moe_ffn(E, k, dim, inter, 1, rtype, rb, etype, gb, ub, db, x)
    ry, rids, rw = moe_f64(E, k, dim, inter, 1, rtype, rb, etype, gb, ub, db, x)
    assert np.array_equal(ids, rids)
    assert np.allclose(w, rw, rtol=1e-5) and abs(w.sum() - 1.0) < 1e-5
    assert np.max(np.abs(y - ry)) / np.max(np.abs(ry)) <= 1e-5
    if k < E:  # without renormalization the result moves well past the bound
        bad, _, _ = moe_f64(E, k, dim, inter, 1, rtype, rb, etype, gb, ub, db, x, renorm=False)
        assert np.max(np.abs(y - bad)) / np.max(np.abs(ry)) > 100 * 1e-5


def test_moe_ties_pick_lower_id_and_plain_weights():
    rng = np.random.default_rng(3)
    E, k, dim, inter = 8, 3, 128, 64
    rb, gb, ub, db = make_moe(rng, E, dim, inter, 8, tie=(5, 2))
    x = np.ones(dim, np.float32)
    y, ids, w = refcpu.moe_ffn(E, k, dim, inter, 0, 0, rb, 8, gb, ub, db, x)
    assert list(ids[:2]) == [2, 5] and w[0] == w[1]
    ry, rids, rw = moe_f64(E, k, dim, inter, 0, 0, rb, 8, gb, ub, db, x)
    assert np.array_equal(ids, rids) and np.allclose(w, rw, rtol=1e-5)  # w = p when not renormalized
