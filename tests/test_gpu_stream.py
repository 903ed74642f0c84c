"""GPU parity of the persistent token kernel (stream.hip, engines loaded with
OI_STREAM=1) against the CPU oracle, on the same bars as test_gpu_parity.py:
per-step logits within a scaled error of 1e-3 and identical greedy ids.

The multi-kernel path is covered by test_gpu_parity.py; the token kernel must
reach the same results through its own GEMV layout, producer-quantized
activations, grid barriers and split-L attention.
"""
import os

import numpy as np
import pytest

import refcpu
from helpers import scaled_err
from oi import infer, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3
NTHREADS = min(16, os.cpu_count() or 1)


@pytest.fixture
def stream_env(monkeypatch):
    monkeypatch.setenv("OI_STREAM", "1")


def _engines(path, max_ctx):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    return e, r


def _greedy_ref(r, token, pos, n):
    out = []
    for i in range(n):
        token = refcpu.argmax(r.forward(token, pos + i))
        out.append(token)
    return np.array(out, np.int32)


@pytest.mark.parametrize("name", ["tiny-q4_k", "tiny-q8_0", "small-q4_k"])
def test_stream_forward_logits(stream_env, make_model, name):
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        rng = np.random.default_rng(2)
        cfg = infer.engine_config(e)
        toks = rng.integers(0, cfg.vocab_size, size=70)
        toks[0] = 0
        for pos, t in enumerate(toks):
            got = infer.engine_forward(e, int(t), pos).copy()
            ref = r.forward(int(t), pos)
            err = scaled_err(got, ref)
            assert err <= TOL, "pos %d err %.3g" % (pos, err)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name", ["tiny-q4_k", "tiny-q8_0", "small-q4_k"])
def test_stream_greedy_matches_oracle(stream_env, make_model, name):
    path = make_model(name)
    e, r = _engines(path, 512)
    try:
        got = infer.engine_decode_greedy(e, 0, 0, 64)
        assert np.array_equal(got, _greedy_ref(r, 0, 0, 64))
    finally:
        infer.engine_destroy(e)
        r.close()


def test_stream_matches_multikernel_greedy(make_model, monkeypatch):
    """Both device paths pick the same ids (each is also pinned to the oracle)."""
    path = make_model("small-q4_k")
    monkeypatch.setenv("OI_STREAM", "0")
    e0, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=256))
    monkeypatch.setenv("OI_STREAM", "1")
    e1, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=256))
    try:
        a = infer.engine_decode_greedy(e0, 7, 0, 48)
        b = infer.engine_decode_greedy(e1, 7, 0, 48)
        assert np.array_equal(a, b)
    finally:
        infer.engine_destroy(e0)
        infer.engine_destroy(e1)


def test_stream_long_context(stream_env, make_model):
    """Many 64-position chunks per KV head, including more chunks than
    attention slots per head on small grids, over a pre-filled f16 cache."""
    path = make_model("small-q4_k")
    L = 1500
    e, r = _engines(path, 2048)
    try:
        cfg = infer.engine_config(e)
        k, v = synth.kv_prefill(99, cfg.n_layers, cfg.n_kv_heads, L, cfg.head_dim)
        infer.engine_kv_fill(e, 0, 0, k, v)
        for l in range(cfg.n_layers):
            r.kv_fill(l, 0, k[l], v[l])
        tok = 5
        for pos in range(L, L + 6):
            got = infer.engine_forward(e, tok, pos).copy()
            ref = r.forward(tok, pos)
            assert scaled_err(got, ref) <= TOL
            assert int(np.argmax(got)) == refcpu.argmax(ref)
            tok = refcpu.argmax(ref)
        ids = infer.engine_decode_greedy(e, tok, L + 6, 8)
        assert np.array_equal(ids, _greedy_ref(r, tok, L + 6, 8))
    finally:
        infer.engine_destroy(e)
        r.close()


def test_stream_qwen3_06b_shape(stream_env, make_model):
    """Qwen3-0.6B shape (Q8_0, tied classifier): the first greedy steps."""
    path = make_model("qwen3-0.6b-q8_0")
    e, r = _engines(path, 128)
    try:
        tok = 0
        for pos in range(6):
            got = infer.engine_forward(e, tok, pos).copy()
            ref = r.forward(tok, pos)
            assert scaled_err(got, ref) <= TOL
            tok = refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()
