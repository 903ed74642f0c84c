"""The oracle's whole-model forward for the routed-expert ("qwen3moe") and
hybrid ("qwen35": full attention + gated DeltaNet, dense or routed FFN with a
shared expert) layouts, pinned by the float64 restatement
npref.forward_general_f64 on small synthetic models: per-token logits within a
scaled error of 3e-4.  The layer pieces are pinned on their own elsewhere
(ref_moe_ffn, ref_deltanet_steps, ref_qwen35_attn_steps); this pins their
composition -- layer order, which norm feeds which sublayer, residuals, the
attention output gate, the routed weights' renormalization and the shared
expert's gate; the 3:1 layer schedule (qwen3_5/model.odin:289-300) is fixed by
which tensors the file holds.  Each variant model with one of
those mistakes must miss by at least 10x the bound.  The reference has no MoE
code, so the routed-expert convention itself (HF Qwen3-MoE / Qwen3-Next) is
pinned only by these restatements."""
import os

import numpy as np
import pytest

import refcpu
from helpers import scaled_err
from npref import GGUFWeights, forward_general_f64

TOL = 3e-4
TOKENS = [0, 17, 3, 900, 5, 1234, 7, 64]


def _oracle_logits(path, tokens):
    r = refcpu.RefEngine(path, max_ctx=64, num_threads=min(8, os.cpu_count() or 1), kv_f16=True)
    try:
        return [np.array(r.forward(t, pos), np.float64) for pos, t in enumerate(tokens)]
    finally:
        r.close()


def _worst(a, b):
    return max(scaled_err(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("name,mistakes", [
    ("moe-tiny", [dict(moe_renorm=False), dict(ffn_norm=False)]),
    ("qwen35-tiny", [dict(attn_gate=False), dict(ffn_norm=False)]),
    ("qwen35-moe-tiny", [dict(moe_renorm=False), dict(shared_gate=False), dict(attn_gate=False)]),
])
def test_oracle_model_vs_float64(make_model, name, mistakes):
    path = make_model(name)
    W = GGUFWeights(path)
    got = _oracle_logits(path, TOKENS)
    ref = forward_general_f64(W, TOKENS)
    err = _worst(got, ref)
    assert err <= TOL, "%s: scaled error %.3g" % (name, err)
    for kw in mistakes:
        bad = forward_general_f64(W, TOKENS, **kw)
        assert _worst(got, bad) > 10 * TOL, (name, kw, _worst(got, bad))


def test_oracle_hybrid_layer_schedule(make_model):
    """Every 4th layer (index 3, 7, ...) is full attention: the tiny hybrid has
    layers 0-2 DeltaNet and layer 3 full attention, as its tensors say."""
    W = GGUFWeights(make_model("qwen35-tiny"))
    for l in range(4):
        full = "blk.%d.attn_q.weight" % l in W.tensors
        lin = "blk.%d.ssm_out.weight" % l in W.tensors
        assert (full, lin) == ((l + 1) % 4 == 0, (l + 1) % 4 != 0)


@pytest.mark.parametrize("name,mistake", [("moe-tiny", dict(moe_renorm=False)),
                                          ("qwen35-tiny", dict(attn_gate=False)),
                                          ("qwen35-moe-tiny", dict(shared_gate=False))])
def test_oracle_batched_prefill_vs_float64(make_model, name, mistake):
    """The oracle's batched prefill for these layouts (a chunk of 8 with the
    attention / DeltaNet / dense-MLP projections staged in f16, the routed
    experts exact; then 3 tokens per token) against the float64 model with the
    same positions staged.  The f16 rounding of the staged inputs makes this
    comparison noisy: a relative change of 1e-7 in the float64 model's inputs
    before the rounding (the size of the f32 / float64 difference) moves its
    chunk logits by 4.5e-4 (moe-tiny) to 6.2e-4 (qwen35-tiny), about as much
    as the staging itself; so the chunk is held to 1.5e-3 (which a staged
    model with a planted composition mistake misses by 10x), and the
    per-token tail after it to the per-token bound.  The staged product itself
    is pinned exactly by test_gemm_oracle."""
    path = make_model(name)
    W = GGUFWeights(path)
    tokens = TOKENS + [11, 250, 3]
    ref = forward_general_f64(W, tokens, staged=set(range(8)))
    bad = forward_general_f64(W, tokens[:8], staged=set(range(8)), **mistake)
    r = refcpu.RefEngine(path, max_ctx=64, num_threads=min(8, os.cpu_count() or 1), kv_f16=True)
    try:
        got8 = np.array(r.prefill(tokens[:8], 0), np.float64)
        err8 = scaled_err(got8, ref[7])
        print("%s: oracle vs staged float64 %.3g, vs a planted mistake %.3g" % (name, err8, scaled_err(got8, bad[7])))
        assert err8 <= 5 * TOL
        assert scaled_err(got8, bad[7]) > 10 * 5 * TOL
        got = np.array(r.prefill(tokens[8:], 8), np.float64)
        assert scaled_err(got, ref[-1]) <= 5 * TOL
    finally:
        r.close()
