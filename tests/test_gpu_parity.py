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
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144),
         14: (256, 210)}


@pytest.mark.parametrize("kind", [8, 12, 14, 1, 0, 2, 3, 6, 7])
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


@pytest.mark.parametrize("kind", [12, 14, 8, 1, 0, 2, 3, 6, 7])
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


def _outlier_x(rng, cols, mode):
    """N(0,1) activations with outliers: 'group' puts one element of every
    32-element group at 10^2..10^4 times the others; 'massive' makes four fixed
    channels 10^3..10^4 (the residual-stream pattern of Qwen models)."""
    x = rng.standard_normal(cols).astype(np.float32)
    if mode == "group":
        g = cols // 32
        pos = np.arange(g) * 32 + rng.integers(0, 32, size=g)
        x[pos] *= (10.0 ** rng.uniform(2, 4, size=g)).astype(np.float32)
    else:
        ch = np.array([3, 777, cols // 2 + 5, cols - 9])
        x[ch] = np.array([3.1e3, -8.7e3, 1.2e4, -1.5e3], np.float32)
    return x


@pytest.mark.parametrize("mode", ["group", "massive"])
@pytest.mark.parametrize("kind", [12, 14, 8])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (12288, 4096), (4096, 12288)])
def test_gemv_outlier_activations(kind, rows, cols, mode):
    """Config-2 shapes with activation outliers, vs the oracle's matmul_t."""
    blocks, _ = _gemv_case(kind, rows, cols, 31)
    x = _outlier_x(np.random.default_rng(rows + cols + kind), cols, mode)
    got = ggml.gemv(kind, blocks, rows, cols, x)
    ref = refcpu.matmul_t(blocks, kind, x, rows, NTHREADS)
    assert scaled_err(got, ref) <= TOL


@pytest.mark.parametrize("kind", [12, 14, 8])
def test_gemv_activation_quantization_bound(kind):
    """The GEMV multiplies the weights with x quantized per 32-element group:
    x_j -> rint(x_j * (2^21 - 1) / amax_g) * amax_g / (2^21 - 1), an error of at
    most half a step (plus the f32 rounding of the scaling, so 0.75 of a step
    is allowed).  Every output row must stay within the bound this implies,
    sum_j |w_rj| * 0.75 * amax_g(j) / (2^21 - 1), plus f32 accumulation noise.
    The adversarial input puts a 10^4 outlier in every group whose weights are
    zero in that column (Q8_0, Q6_K), so the row sums come entirely from the
    small elements quantized against the outlier: a scaled error above 1e-3
    that the bound must still cover (a wrong plane shift or scale breaks it).
    Real weights are not zero in the outlier channels; there the outlier's own
    term dominates the row (test_gemv_outlier_activations)."""
    rows, cols = 512, 4096
    rng = np.random.default_rng(5)
    x = rng.standard_normal(cols).astype(np.float32)
    pos = np.arange(cols // 32) * 32 + rng.integers(0, 32, size=cols // 32)
    x[pos] = (1e4 * np.sign(rng.standard_normal(pos.size))).astype(np.float32)
    w = synth.tensor_f32(77, "bound.%d" % kind, rows, cols, sigma=0.02)
    w[:, pos] = 0.0  # quantizes to exact zeros in every type
    blocks = synth.quantize_rows(kind, w)
    wd = refcpu.dequant_row(kind, blocks, rows * cols).reshape(rows, cols).astype(np.float64)
    if kind != 12:  # Q8_0 and Q6_K store 0 exactly; Q4_K's group minimum leaves a small value
        assert np.all(wd[:, pos] == 0)
    got = np.float64(ggml.gemv(kind, blocks, rows, cols, x))
    exact = wd @ np.float64(x)
    amax = np.abs(x).reshape(-1, 32).max(axis=1).repeat(32).astype(np.float64)
    bound = np.abs(wd) @ (0.75 * amax / 2097151.0) + 1e-6 * (np.abs(wd) @ np.abs(np.float64(x)))
    assert np.all(np.abs(got - exact) <= bound), float(np.max(np.abs(got - exact) / bound))
    print("adversarial scaled error %.3g (bound-limited)" % scaled_err(got, exact))


def _engines(path, max_ctx):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    return e, r


@pytest.mark.parametrize("name", ["tiny-q4_k", "tiny-q8_0", "tiny-f32", "tiny-legacy"])
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


@pytest.mark.parametrize("name,steps", [("tiny-q4_k", 64), ("tiny-q8_0", 64), ("small-q4_k", 64),
                                        ("tiny-legacy", 64)])
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
