"""GPU parity of the routed-expert FFN (oi_moe_ffn, kernels.hip moe_*) against
the oracle (refcpu.ref_moe_ffn, pinned by a float64 brute force): the same
expert ids in the same order, outputs within a
scaled error of 1e-4 (weights within 1e-5: the router logits are summed in
another order), at the measurement-plan shapes of config 4 (128 experts,
top 8, dim 2048, expert inner 768) and config 5 (512 experts, top 10, dim
2048, inner 512), with F32 and Q4_K routers (config 4 and 5 quantize the
router Q4_K), and small shapes with Q8_0 / Q6_K experts, ties, and no
renormalization."""
import numpy as np
import pytest

import refcpu
from oi import _native, moe
from test_moe_oracle import make_moe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k,dim,inter,etype,norm,rtype", [
    (128, 8, 2048, 768, 12, 1, 0), (128, 8, 2048, 768, 12, 1, 12),    # config 4 shape, F32 / Q4_K router
    (512, 10, 2048, 512, 12, 1, 12),                                  # config 5 shape, Q4_K router
    (16, 4, 256, 128, 8, 1, 0), (8, 8, 256, 256, 14, 0, 0), (32, 10, 512, 512, 12, 1, 0),
    (64, 6, 1024, 256, 8, 1, 8)])
def test_moe_vs_oracle(E, k, dim, inter, etype, norm, rtype):
    rng = np.random.default_rng(E + k + dim)
    rb, gb, ub, db = make_moe(rng, E, dim, inter, etype, rtype=rtype)
    x = rng.standard_normal(dim).astype(np.float32)
    y, ids, w = moe.moe_ffn(E, k, dim, inter, norm, rtype, rb, etype, gb, ub, db, x)
    ry, rids, rw = refcpu.moe_ffn(E, k, dim, inter, norm, rtype, rb, etype, gb, ub, db, x)
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


@pytest.mark.parametrize("dim,inter", [(128, 64), (256, 256)])
def test_moe_nan_router_logit_leaves_defined_ids(dim, inter):
    """A NaN router logit makes every probability NaN, so no expert ranks
    below the first: the unfilled ranks must still name a valid expert (id 0,
    weight 0) rather than whatever an earlier call left.  128/64 runs the
    generic top-k kernel, 256/256 the routing inside the gate/up GEMV."""
    rng = np.random.default_rng(4)
    E, k = 8, 3
    rb, gb, ub, db = make_moe(rng, E, dim, inter, 8)
    x = rng.standard_normal(dim).astype(np.float32)
    moe.moe_ffn(E, k, dim, inter, 1, 0, rb, 8, gb, ub, db, x)  # a normal call first
    r = rb.view(np.float32).copy()
    r[3 * dim + 7] = np.nan
    y, ids, w = moe.moe_ffn(E, k, dim, inter, 1, 0, r.view(np.uint8), 8, gb, ub, db, x)
    assert np.all((ids >= 0) & (ids < E)), ids
    assert np.all(ids[1:] == 0), ids


def test_moe_rejects_bad_dims():
    rng = np.random.default_rng(0)
    rb, gb, ub, db = make_moe(rng, 4, 128, 64, 8)
    with pytest.raises(_native.OIError):
        moe.moe_ffn(4, 5, 128, 64, 1, 0, rb, 8, gb, ub, db, np.ones(128, np.float32))  # top_k > n_experts


def test_fused_router_matches_separate(make_model, monkeypatch):
    """The token loop's router inside the routed gate/up launch
    (OI_MOE_ROUTER=fused: each workgroup computes the 128 router logits of
    config 4's layer from its RMSNormed x) against the router as a launch of
    its own (the default): the same int8 products up to the order of the lane
    sums, so the same experts are chosen and 16 steps of logits agree within
    1e-5, on 4 layers of the Qwen3-30B-A3B shape; the device loop's greedy ids
    are equal."""
    import numpy as np
    from helpers import scaled_err
    from oi import infer
    path = make_model("qwen3-30b-a3b-4layer")
    out, ids = {}, {}
    for kind in ("separate", "fused"):
        if kind == "fused":
            monkeypatch.setenv("OI_MOE_ROUTER", "fused")
        e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
        assert ok
        try:
            toks = [int(t) for t in np.random.default_rng(9).integers(0, 151936, 16)]
            out[kind] = [infer.engine_forward(e, t, p).copy() for p, t in enumerate(toks)]
            infer.engine_reset_state(e)
            ids[kind] = list(infer.engine_decode_greedy(e, 0, 0, 24))
        finally:
            infer.engine_destroy(e)
    worst = max(scaled_err(a, b) for a, b in zip(out["fused"], out["separate"]))
    print("fused vs separate router, worst scaled logit difference %.3g" % worst)
    assert worst <= 1e-5
    assert ids["fused"] == ids["separate"]
