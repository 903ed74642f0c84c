"""GPU parity of the HIP path against the CPU oracle (oracle/refcpu.c).

Bars: dequantized values bit-exact; GEMV and per-step logits within a scaled
error max|d|/max|ref| <= 1e-3; greedy ids identical.  The oracle runs with an
f16 KV cache (kv_f16=True), the cache precision of the HIP path.
"""
import os

import numpy as np
import pytest

import refcpu
from helpers import random_blocks, same_bits, scaled_err
from oi import ggml, infer, synth

pytestmark = pytest.mark.gpu
TOL = 1e-3
NTHREADS = min(16, os.cpu_count() or 1)
BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


@pytest.mark.parametrize("kind", [8, 12, 14, 1, 0])
def test_dequant_bit_exact_random(kind):
    rng = np.random.default_rng(100 + kind)
    n = 16384
    e, b = BLOCK[kind]
    blocks = random_blocks(kind, n // e, rng)
    got = ggml.dequant_row(kind, blocks, n)
    ref = refcpu.dequant_row(kind, blocks, n)
    assert same_bits(got, ref)


def test_dequant_f16_all_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = ggml.dequant_row(1, bits.view(np.uint8), 65536)
    ref = bits.view(np.float16).astype(np.float32)
    assert same_bits(got, ref)


def test_dequant_edge_blocks():
    # extreme scales: max f16, smallest subnormal, negative zero, all-max nibbles
    edge16 = [0x7BFF, 0x0001, 0x8000, 0x3C00, 0xFBFF, 0x0400, 0x03FF]
    q4 = []
    for d in edge16:
        for dm in edge16[:3]:
            blk = np.zeros(144, np.uint8)
            blk[0:2] = np.array([d], np.uint16).view(np.uint8)
            blk[2:4] = np.array([dm], np.uint16).view(np.uint8)
            blk[4:16] = 0xFF
            blk[16:] = np.arange(128, dtype=np.uint8) * 37
            q4.append(blk)
    q4 = np.concatenate(q4)
    n = 256 * (len(q4) // 144)
    assert same_bits(ggml.dequant_row(12, q4, n), refcpu.dequant_row(12, q4, n))
    q6 = []
    for d in edge16:
        blk = np.arange(210, dtype=np.uint8) * 91
        blk[192:208] = np.array([-128, 127, 0, -1, 1, 64, -64, 5] * 2, np.int8).view(np.uint8)
        blk[208:210] = np.array([d], np.uint16).view(np.uint8)
        q6.append(blk)
    q6 = np.concatenate(q6 + q6[:1])  # 8 super-blocks
    n = 256 * 8
    assert same_bits(ggml.dequant_row(14, q6, n), refcpu.dequant_row(14, q6, n))
    q8 = []
    for d in edge16 + [0x3555]:
        blk = np.zeros(34, np.uint8)
        blk[0:2] = np.array([d], np.uint16).view(np.uint8)
        blk[2:] = np.array([-128, 127, 0, -1] * 8, np.int8).view(np.uint8)
        q8.append(blk)
    q8 = np.concatenate(q8)
    assert same_bits(ggml.dequant_row(8, q8, 256), refcpu.dequant_row(8, q8, 256))


def _gemv_case(kind, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = synth.tensor_f32(seed, "gemv.%d" % kind, rows, cols, sigma=0.02)
    blocks = synth.quantize_rows(kind, w)
    x = rng.standard_normal(cols).astype(np.float32)
    return blocks, x


@pytest.mark.parametrize("kind", [12, 14, 8, 1, 0])
@pytest.mark.parametrize("rows,cols", [(512, 4096), (300, 1024), (64, 12288), (1000, 512), (7, 2048), (96, 1536),
                                       (130, 3072), (40, 768), (33, 5120)])
def test_gemv_small(kind, rows, cols):
    blocks, x = _gemv_case(kind, rows, cols, 5 + rows + cols)
    got = ggml.gemv(kind, blocks, rows, cols, x)
    ref = refcpu.matmul_t(blocks, kind, x, rows, NTHREADS)
    assert scaled_err(got, ref) <= TOL


@pytest.mark.parametrize("kind", [12, 14, 8])
@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 12288), (4096, 4096), (151936, 4096)])
def test_gemv_microbench_shapes(kind, rows, cols):
    """BASELINE config 2 shapes, outputs vs the oracle's matmul_t."""
    blocks, x = _gemv_case(kind, rows, cols, 17)
    got = ggml.gemv(kind, blocks, rows, cols, x)
    ref = refcpu.matmul_t(blocks, kind, x, rows, NTHREADS)
    assert scaled_err(got, ref) <= TOL


def _engines(path, max_ctx):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    return e, r


@pytest.mark.parametrize("name", ["tiny-q4_k", "tiny-q8_0", "tiny-f32"])
def test_forward_logits_teacher_forced(make_model, name):
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        cfg = infer.engine_config(e)
        assert (cfg.dim, cfg.n_layers, cfg.vocab_size, cfg.seq_len) == (r.dim, r.n_layers, r.vocab_size, r.seq_len)
        rng = np.random.default_rng(1)
        toks = rng.integers(0, cfg.vocab_size, size=80)
        toks[0] = 0
        for pos, t in enumerate(toks):
            got = infer.engine_forward(e, int(t), pos).copy()
            ref = r.forward(int(t), pos)
            err = scaled_err(got, ref)
            assert err <= TOL, "pos %d err %.3g" % (pos, err)
    finally:
        infer.engine_destroy(e)
        r.close()


def _greedy_ref(r, token, pos, n):
    out = []
    for i in range(n):
        logits = r.forward(token, pos + i)
        token = refcpu.argmax(logits)
        out.append(token)
    return np.array(out, np.int32)


@pytest.mark.parametrize("name,steps", [("tiny-q4_k", 64), ("tiny-q8_0", 64), ("small-q4_k", 64)])
def test_greedy_decode_matches_oracle(make_model, name, steps):
    path = make_model(name)
    e, r = _engines(path, 512)
    try:
        got = infer.engine_decode_greedy(e, 0, 0, steps)
        ref = _greedy_ref(r, 0, 0, steps)
        assert np.array_equal(got, ref), (got, ref)
    finally:
        infer.engine_destroy(e)
        r.close()


def test_decode_greedy_equals_forward_loop(make_model):
    path = make_model("tiny-q4_k")
    e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=256))
    try:
        dev = infer.engine_decode_greedy(e, 3, 0, 24)
        tok, host = 3, []
        for pos in range(24):
            tok = int(np.argmax(infer.engine_forward(e, tok, pos)))
            host.append(tok)
        assert np.array_equal(dev, np.array(host, np.int32))
    finally:
        infer.engine_destroy(e)


def test_long_context_prefilled_kv(make_model):
    """Split-L attention over a pre-filled f16 cache (many splits)."""
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
    finally:
        infer.engine_destroy(e)
        r.close()


def test_forward_range_errors(make_model):
    path = make_model("tiny-q8_0")
    e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    try:
        for tok, pos in [(-1, 0), (10 ** 6, 0), (0, -1), (0, 64)]:
            with pytest.raises(infer.OIError) as ei:
                infer.engine_forward(e, tok, pos)
            assert ei.value.code == infer.OI_E_RANGE
        infer.engine_forward(e, 0, 63)  # last valid position
    finally:
        infer.engine_destroy(e)


def greedy_tie_aware(e, r, token, pos, n, tie_rel=1e-4):
    """Walk the oracle's greedy path (both engines teacher-forced on it).  At
    every step the GPU's pick must equal the oracle's unless the oracle's own
    logits put the two within tie_rel * max|logit| (a near-tie that any f32
    reordering may flip).  Returns (steps, near-tie steps, max scaled error)."""
    ties, worst = 0, 0.0
    for i in range(n):
        got = infer.engine_forward(e, token, pos + i).copy()
        ref = r.forward(token, pos + i)
        worst = max(worst, scaled_err(got, ref))
        rt, gt = refcpu.argmax(ref), int(np.argmax(got))
        if gt != rt:
            margin = float(ref[rt] - ref[gt])
            assert margin <= tie_rel * float(np.max(np.abs(ref))), \
                "step %d: gpu %d vs oracle %d, oracle margin %.3g" % (i, gt, rt, margin)
            ties += 1
        token = rt
    return n, ties, worst


def test_qwen3_06b_q8_0_greedy(make_model):
    """BASELINE config 1 (Qwen3-0.6B shape, Q8_0, tied output): token 0 then
    greedy steps.  This seed has a near-tie at step 1 (oracle margin 4.0e-5 of
    max|logit| 2.9), so the greedy path is checked tie-aware; logits must stay
    within the scaled error bound at every step."""
    path = make_model("qwen3-0.6b-q8_0")
    e, r = _engines(path, 4096)
    try:
        n, ties, worst = greedy_tie_aware(e, r, 0, 0, 32)
        assert worst <= TOL
        assert ties <= 2, ties
        # the device-side loop equals the GPU's own forward + argmax loop
        dev = infer.engine_decode_greedy(e, 0, 0, 16)
        tok, host = 0, []
        for pos in range(16):
            tok = int(np.argmax(infer.engine_forward(e, tok, pos)))
            host.append(tok)
        assert np.array_equal(dev, np.array(host, np.int32))
    finally:
        infer.engine_destroy(e)
        r.close()
