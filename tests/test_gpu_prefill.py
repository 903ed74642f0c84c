"""GPU parity of batched prefill (oi_engine_prefill, engine_forward_batch of
qwen3_5/engine.odin:61-93) against the CPU oracle's restatement of the same
path (refcpu.ref_engine_prefill: chunks of a multiple of 8 up to 512 tokens
with f16-staged projections summed exactly, the trailing 1-7 tokens per
token).

Bars: last-token logits within a scaled error max|d|/max|ref| <= 1e-3 of the
oracle and the same argmax; greedy continuation after the prefill identical to
the oracle's.  The GPU sums the staged products in f32 (the reference's MMQ
accumulator), the oracle in float64, which the bar covers.
"""
import os

import numpy as np
import pytest

import refcpu
from helpers import scaled_err
from oi import _native, infer

pytestmark = pytest.mark.gpu
TOL = 1e-3
NTHREADS = min(16, os.cpu_count() or 1)


def _engines(path, max_ctx):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    return e, r


def _tokens(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


@pytest.mark.parametrize("name,n", [("tiny-q4_k", 40), ("tiny-q8_0", 40), ("small-q4_k", 64), ("tiny-q4_k", 13),
                                    ("tiny-q8_0", 5)])
def test_prefill_logits_vs_oracle(make_model, name, n):
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        toks = _tokens(n, n, r.vocab_size)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        assert err <= TOL, "%s n=%d scaled error %.3g" % (name, n, err)
        assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


def test_prefill_512_tokens_fused_gate_up(make_model):
    """512 batched tokens on small-q4_k: 24 row tiles x 8 token tiles of the
    gate/up GEMM need no K split, so the fused gate/up pass with the SwiGLU
    epilogue runs (the 8B-shape prefill's path); logits and argmax vs the
    oracle."""
    path = make_model("small-q4_k")
    e, r = _engines(path, 1024)
    try:
        toks = _tokens(512, 512, r.vocab_size)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        assert err <= TOL, "scaled error %.3g" % err
        assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


def test_prefill_fused_gate_up_equals_unfused_at_8b_shape(make_model, monkeypatch):
    """One layer of the Qwen3-8B shape (gate/up 12288 x 4096, 16 K chunks),
    512 tokens: the fused gate/up pass (SwiGLU in its epilogue) gives the same
    last-token logits as the two projections + SwiGLU kernel (OI_PREFILL_UNFUSED=1):
    both compute f16(silu(g) * u) from the same f32 accumulators."""
    path = make_model("8b-1layer-q4_k")
    toks = _tokens(3, 512, 4096)
    out = []
    for unfused in ("0", "1"):
        monkeypatch.setenv("OI_PREFILL_UNFUSED", unfused)
        e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=1024))
        assert ok
        try:
            out.append(infer.engine_forward_batch(e, toks, 0).copy())
        finally:
            infer.engine_destroy(e)
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32)), scaled_err(out[0], out[1])


def _greedy_ref(r, token, pos, n):
    out = []
    for i in range(n):
        token = refcpu.argmax(r.forward(token, pos + i))
        out.append(token)
    return np.array(out, np.int32)


@pytest.mark.parametrize("name", ["tiny-q4_k", "small-q4_k"])
def test_prefill_then_greedy_matches_oracle(make_model, name):
    """A prompt through the batched path leaves the KV cache the decode loop
    continues from: the greedy ids after it match the oracle's."""
    path = make_model(name)
    e, r = _engines(path, 512)
    try:
        toks = _tokens(5, 100, r.vocab_size)  # 96 batched + 4 per token
        first = int(np.argmax(infer.engine_forward_batch(e, toks, 0)))
        assert first == refcpu.argmax(r.prefill(toks, 0))
        got = infer.engine_decode_greedy(e, first, len(toks), 32)
        ref = _greedy_ref(r, first, len(toks), 32)
        assert np.array_equal(got, ref), (got, ref)
    finally:
        infer.engine_destroy(e)
        r.close()


def test_prefill_full_chunk_and_offset(make_model):
    """520 tokens (one chunk of 512, one of 8) at position 0, then 24 more at
    position 520 on top of the cache the first call left."""
    path = make_model("tiny-q4_k")
    e, r = _engines(path, 1024)
    try:
        toks = _tokens(9, 544, r.vocab_size)
        got = infer.engine_forward_batch(e, toks[:520], 0).copy()
        ref = r.prefill(toks[:520], 0)
        assert scaled_err(got, ref) <= TOL
        got = infer.engine_forward_batch(e, toks[520:], 520).copy()
        ref = r.prefill(toks[520:], 520)
        assert scaled_err(got, ref) <= TOL
    finally:
        infer.engine_destroy(e)
        r.close()


def test_prefill_split_calls_agree(make_model):
    """The same 48 tokens in one call and in two (24 + 24): the per-token math
    is independent of the chunk a token sits in, so the logits agree up to the
    summation order of the projections' K slices."""
    path = make_model("tiny-q8_0")
    toks = _tokens(11, 48, 2048)
    e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    try:
        whole = infer.engine_forward_batch(e, toks, 0).copy()
        infer.engine_forward_batch(e, toks[:24], 0)
        parts = infer.engine_forward_batch(e, toks[24:], 24).copy()
        assert scaled_err(parts, whole) <= 1e-4
    finally:
        infer.engine_destroy(e)


def test_prefill_unbatched_model_uses_token_path(make_model):
    """F32 projections have no batched kernel: every token runs the decode
    path, so the result equals the oracle's per-token forward."""
    path = make_model("tiny-f32")
    e, r = _engines(path, 64)
    try:
        toks = _tokens(2, 12, r.vocab_size)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        for p, t in enumerate(toks):
            ref = r.forward(int(t), p)
        assert scaled_err(got, ref) <= TOL
    finally:
        infer.engine_destroy(e)
        r.close()


def test_prefill_errors(make_model):
    path = make_model("tiny-q8_0")
    e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    try:
        with pytest.raises(_native.OIError) as ex:
            infer.engine_forward_batch(e, np.zeros(0, np.int32), 0)
        assert ex.value.code == -1
        with pytest.raises(_native.OIError) as ex:
            infer.engine_forward_batch(e, np.zeros(16, np.int32), 60)  # past seq_len 64
        assert ex.value.code == infer.OI_E_RANGE
        with pytest.raises(_native.OIError) as ex:
            infer.engine_forward_batch(e, np.array([1, 2, 99999], np.int32), 0)
        assert ex.value.code == infer.OI_E_RANGE
        # the engine still works after rejected calls
        assert np.isfinite(infer.engine_forward_batch(e, np.arange(8, dtype=np.int32), 0)).all()
    finally:
        infer.engine_destroy(e)
