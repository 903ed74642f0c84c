"""GPU parity of the routed-expert FFN (oi_moe_ffn, kernels.hip moe_*) against
the oracle (refcpu.ref_moe_ffn, pinned by a float64 brute force): the same
expert ids in the same order, outputs within a
scaled error of 1e-4 (weights within 1e-5: the router logits are summed in
another order), at the measurement-plan shape of config 4 (128 experts,
top 8, dim 2048, expert inner 768, Q4_K experts, F32 router) and small shapes
with Q8_0 / Q6_K experts, ties, and no renormalization."""
import numpy as np
import pytest

import refcpu
from oi import _native, moe
from test_moe_oracle import make_moe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k,dim,inter,etype,norm", [
    (128, 8, 2048, 768, 12, 1),   # config 4 shape
    (16, 4, 256, 128, 8, 1), (8, 8, 256, 256, 14, 0), (32, 10, 512, 512, 12, 1)])
def test_moe_vs_oracle(E, k, dim, inter, etype, norm):
    rng = np.random.default_rng(E + k + dim)
    rb, gb, ub, db = make_moe(rng, E, dim, inter, etype)
    x = rng.standard_normal(dim).astype(np.float32)
    y, ids, w = moe.moe_ffn(E, k, dim, inter, norm, 0, rb, etype, gb, ub, db, x)
    ry, rids, rw = refcpu.moe_ffn(E, k, dim, inter, norm, 0, rb, etype, gb, ub, db, x)
    assert np.array_equal(ids, rids), (ids, rids)
    assert np.allclose(w, rw, rtol=1e-5, atol=0)  # router logits summed in another order
    err = np.max(np.abs(np.float64(y) - ry)) / np.max(np.abs(ry))
    assert err <= 1e-4, err


@pytest.mark.parametrize("dim,inter", [(128, 64), (256, 256)])
def test_moe_ties(dim, inter):
    """Equal router rows 5 and 2: rank order puts the lower id first.  128/64
    runs the generic kernels (moe_topk_kernel), 256/256 the routing inside the
    gate/up GEMV and the columns-mode down GEMV."""
    rng = np.random.default_rng(3)
    E, k = 8, 3
    rb, gb, ub, db = make_moe(rng, E, dim, inter, 8, tie=(5, 2))
    x = np.ones(dim, np.float32)
    y, ids, w = moe.moe_ffn(E, k, dim, inter, 0, 0, rb, 8, gb, ub, db, x)
    assert list(ids[:2]) == [2, 5]
    ry, rids, rw = refcpu.moe_ffn(E, k, dim, inter, 0, 0, rb, 8, gb, ub, db, x)
    assert np.array_equal(ids, rids)
    assert np.allclose(w, rw, rtol=1e-5, atol=0)
    assert np.max(np.abs(np.float64(y) - ry)) / np.max(np.abs(ry)) <= 1e-4


def test_moe_rejects_bad_dims():
    rng = np.random.default_rng(0)
    rb, gb, ub, db = make_moe(rng, 4, 128, 64, 8)
    with pytest.raises(_native.OIError):
        moe.moe_ffn(4, 5, 128, 64, 1, 0, rb, 8, gb, ub, db, np.ones(128, np.float32))  # top_k > n_experts
