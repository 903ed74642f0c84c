"""GPU parity of batched prefill for the Qwen3.5 hybrid and routed-expert
layouts (oi_engine_prefill: forward_gpu_batch of qwen3_5/metal.odin:1472-1654
for the full-attention and DeltaNet layers; the routed-expert FFN, which the
reference's batched path does not have, in f32 as the per-token path) against
the oracle's restatement (refcpu.ref_engine_prefill: staged attention /
DeltaNet / dense-MLP projections, the routed experts exact, the trailing 1-7
tokens per token).

Bars: last-token logits within a scaled error of 1e-3 and the same argmax;
the state the chunk leaves (K/V of the full-attention layers, conv and
recurrent states of the DeltaNet layers, compared through the .oikv file
both sides write) within 1e-3; greedy decoding after the prefill identical
to the oracle's; one call and two calls over the same tokens agree.
"""
import os
import struct

import numpy as np
import pytest

import refcpu
from helpers import gguf_tensor_data, scaled_err
from oi import infer

pytestmark = pytest.mark.gpu
TOL = 1e-3
NT = min(16, os.cpu_count() or 1)


def _engines(path, max_ctx):
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    return e, refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NT, kv_f16=True)


def _tokens(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


@pytest.mark.parametrize("name,n", [("qwen35-tiny", 40), ("qwen35-tiny", 13), ("qwen35-moe-tiny", 40),
                                    ("moe-tiny", 40), ("qwen35-moe-tiny", 200)])
def test_prefill_logits_vs_oracle(make_model, name, n):
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        toks = _tokens(n + 1, n, r.vocab_size)
        print("case %s n=%d" % (name, n), flush=True)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        print("%s n=%d: scaled error %.3g" % (name, n, err))
        assert err <= TOL, "%s n=%d scaled error %.3g" % (name, n, err)
        assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name,n", [("qwen35-hybrid-moe-2layer", 64), ("qwen35-hybrid-moe-2layer", 200),
                                    ("qwen3-30b-a3b-2layer", 64)])
def test_prefill_full_shapes_vs_oracle(make_model, name, n):
    """The per-layer shapes of configs 5 (a DeltaNet and a full-attention
    layer: 16 / 32 DeltaNet heads, head_dim 256 with 16 / 2 heads, 512 experts
    top 10 + the merged shared expert) and 4 (128 experts top 8, expert inner
    768), two layers each.  (Deeper stacks of these shapes are not compared
    against the staged oracle: the f16 staging rounds f32 and float64 inputs
    apart at half-way points, ~1e-4 per layer, and a top-10-of-512 routing
    step turns that into a different expert for some token a few layers on;
    the per-token path, without staging, is compared at four layers in
    test_gpu_models.)"""
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        toks = _tokens(7, n, r.vocab_size)
        print("case %s n=%d" % (name, n), flush=True)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        print("%s: scaled error %.3g" % (name, err))
        assert err <= TOL
        assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


def _oikv_sections(g, o, name):
    """Compare two .oikv files (GPU, oracle): header byte for byte, then the
    K/V, conv and recurrent sections by scaled difference."""
    assert len(g) == len(o) and g[:60] == o[:60]
    bg, bo = np.frombuffer(g[60:-4], np.float32), np.frombuffer(o[60:-4], np.float32)
    n, _, n_full, n_lin, kv_dim, conv_dim, kern, nv, hk, hv = struct.unpack_from("<10I", o, 20)
    off, errs = 0, {}
    for what, size in [("K/V", 2 * n_full * n * kv_dim), ("conv", n_lin * conv_dim * max(kern - 1, 0)),
                       ("recurrent", n_lin * nv * hk * hv)]:
        if size:
            errs[what] = scaled_err(bg[off:off + size], bo[off:off + size])
            print("%s: %s section, scaled difference GPU vs oracle %.3g" % (name, what, errs[what]), flush=True)
        off += size
    assert off == bo.size
    return errs


@pytest.mark.timeout(1200)
def test_c5_prompt_2048_in_64_token_chunks_then_decode(make_model, tmp_path):
    """BASELINE config 5 as configured, on two layers of its shapes (a
    DeltaNet layer, then a full-attention layer; 512 experts top 10 + the
    shared expert): a 2048-token random-id prompt in 64-token chunks (one
    engine_forward_batch call per chunk, qwen3_5/engine.odin:66-93), so the
    conv and recurrent states carry across 32 chunks and the key-split
    prefill attention runs at positions up to 2048; then greedy decoding
    from position 2048.  Against the oracle's staged prefill over the same
    prompt (qwen3_5/forward.odin:46-225 per token, projections staged in f16
    as qwen3_5/metal.odin:493-609): last logits within 1e-3 and the same
    argmax, the K/V, conv and recurrent state after the prompt within 1e-3
    (through the .oikv files both sides write), then 32 identical greedy ids."""
    path = make_model("qwen35-hybrid-moe-2layer")
    n, chunk, ndec = 2048, 64, 32
    e, r = _engines(path, n + ndec + 8)
    try:
        toks = _tokens(2048, n, r.vocab_size)
        for i in range(0, n, chunk):
            got = infer.engine_forward_batch(e, toks[i:i + chunk], i)
        got = got.copy()
        print("C5 GPU prompt done (%d chunks of %d)" % (n // chunk, chunk), flush=True)
        r.route_log(True)
        for i in range(0, n, 256):  # the oracle's result does not depend on its chunking
            ref = r.prefill(toks[i:i + 256], i)
            print("oracle prompt: %d / %d tokens" % (i + 256, n), flush=True)
        margins = r.route_margins()[:n, 0]  # layer 0's routing, which feeds layer 1's K/V
        r.route_log(False)
        err = scaled_err(got, ref)
        print("C5 last logits after the 2048-token prompt: scaled error %.3g" % err, flush=True)
        assert err <= TOL
        first = int(np.argmax(got))
        assert first == refcpu.argmax(ref)
        fg, fr = tmp_path / "gpu.oikv", tmp_path / "ref.oikv"
        assert infer.engine_save_kv(e, fg, n)
        r.save_kv(fr, n)
        g, o = fg.read_bytes(), fr.read_bytes()
        errs = _oikv_sections(g, o, "C5 after 2048 tokens")
        assert set(errs) == {"K/V", "conv", "recurrent"}
        assert errs["conv"] <= TOL and errs["recurrent"] <= TOL
        # K/V per position.  Layer 0's top-10-of-512 routing of a token whose
        # 10th and 11th experts are closer than the f16 staging noise of its
        # input (the staged projections round the GPU's f32 and the oracle's
        # float64-accumulated inputs apart at half-way points) may pick the
        # other expert on the GPU, which moves that one position's layer-1 K/V
        # by a few percent.  Such a position is accepted only where the
        # oracle's own routing margin there, log(p10 / p11), is below
        # ROUTE_TIE, and at most 1% of the positions may need it; every other
        # position must be within TOL.
        ROUTE_TIE = 3e-4
        n_full, kv_dim = struct.unpack_from("<I", o, 28)[0], struct.unpack_from("<I", o, 36)[0]
        assert n_full == 1
        bg = np.frombuffer(g[60:60 + 8 * n * kv_dim], np.float32).reshape(2, n, kv_dim).astype(np.float64)
        bo = np.frombuffer(o[60:60 + 8 * n * kv_dim], np.float32).reshape(2, n, kv_dim).astype(np.float64)
        per_pos = np.abs(bg - bo).max(axis=(0, 2)) / np.abs(bo).max()
        bad = np.nonzero(per_pos > TOL)[0]
        print("C5 K/V: positions over %.0e: %s; their layer-0 routing margins %s; positions with a margin "
              "below %.0e: %d; worst elsewhere %.3g" % (
                  TOL, list(bad), ["%.2g" % margins[p] for p in bad], ROUTE_TIE,
                  int(np.sum(margins < ROUTE_TIE)), float(np.delete(per_pos, bad).max())), flush=True)
        assert len(bad) <= n // 100
        assert all(margins[p] < ROUTE_TIE for p in bad), "a K/V difference at a position routed with a clear margin"
        got_g = infer.engine_decode_greedy(e, first, n, ndec)
        ref_g, tok = [], first
        for i in range(ndec):
            tok = refcpu.argmax(r.forward(tok, n + i))
            ref_g.append(tok)
        print("C5 greedy ids from %d: gpu %s oracle %s" % (n, list(got_g), ref_g), flush=True)
        assert np.array_equal(got_g, np.array(ref_g, np.int32))
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name", ["qwen35-tiny", "qwen35-moe-tiny"])
def test_prefill_state_vs_oracle(make_model, tmp_path, name):
    """The state after a 37-token prompt (32 batched + 5 per token) through
    the .oikv files both sides write: header byte for byte, K/V, conv and
    recurrent sections within 1e-3."""
    path = make_model(name)
    e, r = _engines(path, 64)
    try:
        toks = _tokens(3, 37, r.vocab_size)
        infer.engine_forward_batch(e, toks, 0)
        r.prefill(toks, 0)
        fg, fr = tmp_path / "gpu.oikv", tmp_path / "ref.oikv"
        assert infer.engine_save_kv(e, fg, len(toks))
        r.save_kv(fr, len(toks))
        for what, v in _oikv_sections(fg.read_bytes(), fr.read_bytes(), name).items():
            assert v <= TOL, what
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name", ["qwen35-tiny", "qwen35-moe-tiny", "moe-tiny"])
def test_prefill_then_greedy_matches_oracle(make_model, name):
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        toks = _tokens(5, 100, r.vocab_size)  # 96 batched + 4 per token
        first = int(np.argmax(infer.engine_forward_batch(e, toks, 0)))
        assert first == refcpu.argmax(r.prefill(toks, 0))
        got = infer.engine_decode_greedy(e, first, len(toks), 24)
        ref, tok = [], first
        for i in range(24):
            tok = refcpu.argmax(r.forward(tok, len(toks) + i))
            ref.append(tok)
        assert np.array_equal(got, np.array(ref, np.int32)), (got, ref)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("chunk,bar", [("0", 1e-4), (None, TOL)])
def test_prefill_split_calls_agree(make_model, monkeypatch, chunk, bar):
    """48 tokens in one call and in two (24 + 24) on the hybrid: the
    recurrent and conv states carry across chunks as across tokens.  With
    the delta rule token by token (OI_PREFILL_DN_CHUNK=0) both partitions do
    the same arithmetic (1e-4); in the default chunked form one 48-token
    chunk and two 24-token chunks sum in different orders, and the f16
    staging of the next projections turns those roundings into differences
    of the size of the oracle bar, which each partition also meets against
    the oracle (test_prefill_logits_vs_oracle)."""
    if chunk is not None:
        monkeypatch.setenv("OI_PREFILL_DN_CHUNK", chunk)
    path = make_model("qwen35-moe-tiny")
    toks = _tokens(11, 48, 2048)
    e, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    e2, _ = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    try:
        whole = infer.engine_forward_batch(e, toks, 0).copy()
        infer.engine_forward_batch(e2, toks[:24], 0)
        parts = infer.engine_forward_batch(e2, toks[24:], 24).copy()
        err = scaled_err(parts, whole)
        print("split calls, chunk %s: scaled difference %.3g" % (chunk or "default", err))
        assert err <= bar
    finally:
        infer.engine_destroy(e)
        infer.engine_destroy(e2)


@pytest.mark.parametrize("shape,n", [("c5", 200), ("c5", 64), ("c4", 200), ("c4", 48)])
def test_prefill_expert_kernels_agree(tmp_path, monkeypatch, shape, n):
    """The routed experts of a chunk on the expert kernels: items of up to 4
    pairs (the default when the chunk's pairs average at most 4 per expert:
    64 tokens at C5, 48 at C4) on int8 MFMA (x scaled per row to 28-bit
    integers in four planes; OI_PREFILL_EXPERTS=i8 forces it), on the decode
    GEMV's int8 dot4 arithmetic (x quantized to 22 bits per group of 32;
    dot4) or on f16 MFMA (fewmfma); Q4_K quants on f16 MFMA with the scales applied per 32 weights
    in f32 and x split hi + lo in items of up to 16 pairs (the default
    otherwise; OI_PREFILL_EXPERTS=wide), the
    decoded weights on f32 MFMA (OI_PREFILL_EXPERTS=f32, the default for
    Q6_K / Q8_0) and the multi-token GEMV (OI_PREFILL_EXPERTS=gemv): the same
    f32 arithmetic up to the order of the sums and x to ~2^-22.  One layer of
    the config 5 / config 4 shapes, so nothing staged in f16 follows the
    experts (a later staged projection would turn a 1e-7 difference into
    ~1e-4 at its rounding boundaries): the last logits agree within 1e-5."""
    from oi import synth
    spec = (synth._hybrid(2048, 512, 1, 16, 2, 256, 4096, 4096, 64, 16, 32, 128, experts=512, used=10, eff=512,
                          shared=512, interval=2, seed=47) if shape == "c5" else
            synth._moe(2048, 1, 32, 4, 4096, 4096, 128, 8, 768, seed=37))
    path = tmp_path / ("%s.gguf" % shape)
    synth.write_gguf(path, spec)
    toks = _tokens(13, n, 4096)
    out = {}
    for kind in ("default", "dot4", "i8", "fewmfma", "wide", "f32", "gemv"):
        monkeypatch.setenv("OI_PREFILL_EXPERTS", kind)
        e, ok = infer.engine_load(str(path), infer.Engine_Opts(max_ctx=256))
        assert ok
        try:
            out[kind] = infer.engine_forward_batch(e, toks, 0).copy()
        finally:
            infer.engine_destroy(e)
    for kind in ("dot4", "i8", "fewmfma", "wide", "f32", "gemv"):
        err = scaled_err(out["default"], out[kind])
        print("%s n=%d: default vs %s experts %.3g" % (shape, n, kind, err))
        assert err <= 1e-5, kind


@pytest.mark.parametrize("shape,n,kind", [("c5", 64, "default"), ("c5", 200, "i8"), ("c4", 48, "default"),
                                          ("c4", 200, "i8")])
def test_prefill_int8_rows_quantized_once_bit_identical(tmp_path, monkeypatch, shape, n, kind):
    """The int8 router and routed gate/up items take the chunk's normalized
    rows quantized once per row (qi_rows_kernel: planes, group sums, scale)
    instead of quantizing their pairs' rows in each item's prologue
    (OI_PREFILL_XQ=0).  The two are the same arithmetic (the same maximum,
    rounding and sum order), so the chunk's last logits are bit for bit the
    same, items with fewer than four pairs included."""
    from oi import synth
    spec = (synth._hybrid(2048, 512, 1, 16, 2, 256, 4096, 4096, 64, 16, 32, 128, experts=512, used=10, eff=512,
                          shared=512, interval=2, seed=59) if shape == "c5" else
            synth._moe(2048, 1, 32, 4, 4096, 4096, 128, 8, 768, seed=61))
    path = tmp_path / ("%s.gguf" % shape)
    synth.write_gguf(path, spec)
    toks = _tokens(23, n, 4096)
    monkeypatch.setenv("OI_PREFILL_EXPERTS", kind)
    out = {}
    for xq in ("1", "0"):
        monkeypatch.setenv("OI_PREFILL_XQ", xq)
        e, ok = infer.engine_load(str(path), infer.Engine_Opts(max_ctx=256))
        assert ok
        try:
            print("case %s n=%d experts %s OI_PREFILL_XQ=%s" % (shape, n, kind, xq), flush=True)
            out[xq] = infer.engine_forward_batch(e, toks, 0).copy()
        finally:
            infer.engine_destroy(e)
    assert np.all(np.isfinite(out["1"]))
    assert np.array_equal(out["1"], out["0"]), scaled_err(out["1"], out["0"])


@pytest.mark.parametrize("mode", ["massive", "group"])
def test_prefill_int8_experts_outlier_activations(tmp_path, mode):
    """The routed experts of a 64-token chunk on the int8 matrix cores (the
    default at config 5's shapes) scale each pair's x row once, by its
    largest element, into four 7-bit planes: 28 bits relative to the row's
    maximum, so a row holding a 10^3..10^4 outlier keeps far fewer bits for
    its small elements.  The FFN norm weight of a one-layer config-5-shape
    model (a DeltaNet layer, 512 experts top 10 + the shared expert) is
    patched so that every token's expert input carries outliers: four massive
    channels at 1.5e3..1.2e4 times the rest (the residual-stream pattern of
    Qwen models) or one element of every 32 at 10^2..10^4 times the rest.
    The last logits against the oracle's prefill (its routed experts in
    float64 from f32 x, qwen3_5/forward.odin:227-243): scaled error 1e-3 and
    the same argmax."""
    from oi import synth
    spec = synth._hybrid(2048, 512, 1, 16, 2, 256, 4096, 4096, 64, 16, 32, 128, experts=512, used=10, eff=512,
                         shared=512, interval=2, seed=53)
    path = tmp_path / "c5l1.gguf"
    synth.write_gguf(path, spec)
    data = bytearray(path.read_bytes())
    off, typ = gguf_tensor_data(bytes(data))["blk.0.post_attention_norm.weight"]
    assert typ == 0  # F32
    w = np.frombuffer(data, np.float32, 2048, off).copy()
    rng = np.random.default_rng(11)
    if mode == "massive":
        w[[3, 777, 1029, 2039]] *= np.array([3.1e3, -8.7e3, 1.2e4, -1.5e3], np.float32)
    else:
        pos = np.arange(64) * 32 + rng.integers(0, 32, size=64)
        w[pos] *= (10.0 ** rng.uniform(2, 4, size=64)).astype(np.float32)
    data[off:off + w.nbytes] = w.tobytes()
    path.write_bytes(bytes(data))
    e, r = _engines(str(path), 256)
    try:
        toks = _tokens(19, 64, r.vocab_size)
        print("case outliers %s" % mode, flush=True)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        print("outliers %s: scaled error %.3g" % (mode, err))
        assert err <= TOL
        assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("chunk", ["0", "16", "32"])
@pytest.mark.parametrize("name,n", [("qwen35-tiny", 40), ("qwen35-hybrid-moe-2layer", 200)])
def test_prefill_chunked_delta_vs_oracle(make_model, monkeypatch, chunk, name, n):
    """Prefill with the delta rule of the DeltaNet layers token by token
    (OI_PREFILL_DN_CHUNK=0) or in the lane-level chunked form over 16 / 32
    tokens, instead of the default 64-token chunks on the matrix cores,
    against the oracle's prefill (the delta rule token by token): the same
    bars as the default path, and the same greedy continuation on the tiny
    model."""
    monkeypatch.setenv("OI_PREFILL_DN_CHUNK", chunk)
    path = make_model(name)
    e, r = _engines(path, 256)
    try:
        toks = _tokens(n + 1, n, r.vocab_size)  # the inputs of test_prefill_logits_vs_oracle
        print("case %s n=%d chunk %s" % (name, n, chunk), flush=True)
        got = infer.engine_forward_batch(e, toks, 0).copy()
        ref = r.prefill(toks, 0)
        err = scaled_err(got, ref)
        print("%s n=%d chunk %s: scaled error %.3g" % (name, n, chunk, err))
        assert err <= TOL
        first = int(np.argmax(got))
        assert first == refcpu.argmax(ref)
        if name == "qwen35-tiny":
            got_g = infer.engine_decode_greedy(e, first, n, 8)
            ref_g, tok = [], first
            for i in range(8):
                tok = refcpu.argmax(r.forward(tok, n + i))
                ref_g.append(tok)
            assert np.array_equal(got_g, np.array(ref_g, np.int32))
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("n", [200, 40])
def test_prefill_attention_kernels_agree(make_model, monkeypatch, n):
    """The head_dim-256 causal attention on the matrix cores (f16 MFMA with q
    and p split hi + lo: one workgroup per 64 queries at 200 tokens, and at 40
    tokens, a short chunk, the keys split over workgroups and merged) and on
    the lane-per-position kernel (OI_PREFILL_ATTN=lanes): both f32
    arithmetic on the same f16 cache up to the order of the sums; through the
    following staged projections of a tiny hybrid model the last logits agree
    within 1e-4 (measured ~1e-6; the f16 rounding of the attention output can
    move at a half-way point), and each is within 1e-3 of the oracle (above)."""
    path = make_model("qwen35-moe-tiny")
    toks = _tokens(23, n, 2048)
    out = {}
    for kind in ("mfma", "lanes"):
        if kind == "lanes":
            monkeypatch.setenv("OI_PREFILL_ATTN", "lanes")
        e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=256))
        assert ok
        try:
            if n < 128:  # a short chunk after a longer prompt: several key blocks to split
                infer.engine_forward_batch(e, _tokens(29, 160, 2048), 0)
                out[kind] = infer.engine_forward_batch(e, toks, 160).copy()
            else:
                out[kind] = infer.engine_forward_batch(e, toks, 0).copy()
        finally:
            infer.engine_destroy(e)
    err = scaled_err(out["mfma"], out["lanes"])
    print("head_dim 256 attention: matrix cores vs lanes %.3g" % err)
    assert err <= 1e-4


@pytest.mark.parametrize("name,seed", [("tiny-q4_k", 31), ("moe-tiny", 43), ("qwen35-moe-tiny", 194)])
def test_verify_batch_vs_oracle(make_model, name, seed):
    """engine_verify_batch (qwen3_5/engine.odin:166-174): after a 20-token
    prompt, 11 draft tokens (a batched chunk of 8, then 3 through the token
    path) with every position's logits returned.  Each row within 1e-3 of the
    oracle's verify_batch with the same argmax; the last row equals
    engine_forward_batch's result for the same tokens on a second engine, bit
    for bit (the same kernels); the state afterwards is the prefill's: the
    next token's logits match the oracle's.  The tiny routed models choose 2
    of 8 experts, so one routing step whose 2nd and 3rd experts are closer
    than the f16 staging noise would move every later row by percents; the
    token seeds are ones whose routing margins log(p2 / p3) in the oracle are
    all above 5e-3, which the test checks first."""
    path = make_model(name)
    e, r = _engines(path, 128)
    e2, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    assert ok
    try:
        t = _tokens(seed, 31, r.vocab_size)
        prompt, draft = t[:20], t[20:]
        infer.engine_forward_batch(e, prompt, 0)
        r.route_log(True)
        r.prefill(prompt, 0)
        ref = r.verify_batch(draft, 20)
        if "moe" in name:
            assert np.nanmin(r.route_margins()[:31]) > 5e-3
        r.route_log(False)
        rows = infer.engine_verify_batch(e, draft, 20).copy()
        assert rows.shape == ref.shape == (11, r.vocab_size)
        errs = [scaled_err(rows[i], ref[i]) for i in range(11)]
        print("%s verify rows, scaled error: %s" % (name, " ".join("%.2g" % x for x in errs)), flush=True)
        assert max(errs) <= TOL
        assert [int(np.argmax(x)) for x in rows] == [refcpu.argmax(x) for x in ref]
        infer.engine_forward_batch(e2, prompt, 0)
        last = infer.engine_forward_batch(e2, draft, 20).copy()
        assert np.array_equal(last, rows[-1])
        got = infer.engine_forward(e, 5, 31).copy()
        assert scaled_err(got, r.forward(5, 31)) <= TOL
        with pytest.raises(infer.OIError):
            infer.engine_verify_batch(e, [], 0)
    finally:
        infer.engine_destroy(e)
        infer.engine_destroy(e2)
        r.close()
