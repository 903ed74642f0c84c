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


def test_prefill_with_token_kernel_decode(make_model, monkeypatch):
    """With the persistent token kernel (OI_STREAM=1) the batched prompt, its
    per-token tail and the decode after it share one KV cache: the greedy ids
    after a 45-token prompt (40 batched + 5 per token) match the oracle."""
    monkeypatch.setenv("OI_STREAM", "1")
    path = make_model("tiny-q4_k")
    e, r = _engines(path, 256)
    try:
        toks = _tokens(21, 45, r.vocab_size)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        assert scaled_err(got, ref) <= TOL
        first = int(np.argmax(got))
        dev = infer.engine_decode_greedy(e, first, len(toks), 16)
        assert np.array_equal(dev, _greedy_ref(r, first, len(toks), 16))
    finally:
        infer.engine_destroy(e)
        r.close()
