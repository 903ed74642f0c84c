"""Whole-model GPU parity at the measured configurations, against the CPU
oracle (oracle/refcpu.c, the restated reference forward, infer/forward.odin:
17-146) on the same seeded synthetic GGUF:

  C1  Qwen3-0.6B shape, Q8_0, tied classifier: token 0 at position 0, then 64
      greedy steps;
  C3  Qwen3-8B shape, Q4_K with Q6_K attn_v and output: f16 KV pre-filled with
      N(0,1) to 4096 positions, token 0 at position 4096, then 64 greedy steps
      (the first steps of the bench's workload, same model and cache seeds);
  C4 / C5 layer shapes (4 layers each) and small models of the routed-expert
      and hybrid layouts: logits on the oracle's greedy path, then greedy ids.

Bars (the north star's): per-step logits within a scaled error
max|d|/max|ref| <= 1e-3, and greedy ids identical for 64 steps with ties to
the lowest id (sampler/sampler.odin:79-89).  The oracle runs with an f16 KV
cache, the cache precision of the GPU path.

One exception is allowed, and it must be proven, not assumed: where the GPU's
pick differs from the oracle's, the two logits must be so close that the
reference algorithm itself does not decide between them in f32 -- their
oracle margin must not exceed the amount by which a second, equally valid f32
summation order of the same oracle (refcpu.set_dot_order(1)) moves the
logits at that step.  The walk then continues teacher-forced on the oracle's
path.  Margins are printed for every step.
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


def _top2(logits):
    i = refcpu.argmax(logits)
    rest = np.array(logits, np.float64)
    rest[i] = -np.inf
    return i, float(logits[i] - rest.max())


def _oracle_path(r, token, pos, n, keep_logits):
    """The oracle's greedy walk: ids, top-1/top-2 margins, and the logits of
    the first keep_logits steps."""
    ids, margins, kept = [], [], []
    for i in range(n):
        lg = r.forward(token, pos + i)
        token, m = _top2(lg)
        ids.append(token)
        margins.append(m)
        if i < keep_logits:
            kept.append(lg.copy())
    return np.array(ids, np.int32), margins, kept


def _noise_at(path, max_ctx, prefill, start_token, pos, tokens, step):
    """max |logits(order 0) - logits(order 1)| of the oracle at `step` of the
    given token path (both orders teacher-forced on it from the start)."""
    out = []
    for order in (0, 1):
        refcpu.set_dot_order(order)
        try:
            r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
            try:
                if prefill is not None:
                    for l in range(r.n_layers):
                        r.kv_fill(l, 0, prefill[0][l], prefill[1][l])
                tok = start_token
                for i in range(step + 1):
                    lg = r.forward(tok, pos + i)
                    tok = int(tokens[i])
                out.append(np.array(lg, np.float64))
            finally:
                r.close()
        finally:
            refcpu.set_dot_order(0)
    return float(np.max(np.abs(out[0] - out[1])))


def _oracle_logits_at(path, max_ctx, prefill, token, pos, ref_ids, i):
    """The oracle's logits at step i of its own greedy path."""
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    try:
        if prefill is not None:
            for l in range(r.n_layers):
                r.kv_fill(l, 0, prefill[0][l], prefill[1][l])
        tok = token
        for j in range(i + 1):
            lg = r.forward(tok, pos + j)
            tok = int(ref_ids[j])
    finally:
        r.close()
    return lg


def _prove_tie(path, max_ctx, prefill, token, pos, ref_ids, i, gpu_pick):
    """Assert that the GPU's pick at step i (on the oracle's path up to it) is
    a proven f32 tie of the oracle's: its oracle margin does not exceed the
    oracle's own f32 reordering noise at that step."""
    lg = _oracle_logits_at(path, max_ctx, prefill, token, pos, ref_ids, i)
    margin = float(lg[ref_ids[i]] - lg[gpu_pick])
    noise = _noise_at(path, max_ctx, prefill, token, pos, ref_ids, i)
    print("step %d: gpu %d vs oracle %d, oracle margin %.3g, oracle f32 reordering noise %.3g"
          % (i, gpu_pick, ref_ids[i], margin, noise))
    assert margin <= noise, "step %d: gpu %d vs oracle %d, margin %.3g exceeds the oracle's f32 noise %.3g" % (
        i, gpu_pick, ref_ids[i], margin, noise)


def _check_greedy(e, path, max_ctx, prefill, token, pos, ref_ids, ref_margins):
    """GPU device-side greedy loop vs the oracle's ids; a differing step must
    be a proven f32 tie of the oracle (module docstring), after which the
    remaining steps are teacher-forced on the oracle's path, where every
    further difference needs the same proof."""
    n = len(ref_ids)
    got = infer.engine_decode_greedy(e, token, pos, n)
    ties = []
    i = 0
    while i < n:
        if got[i] == ref_ids[i]:
            i += 1
            continue
        # oracle and GPU agree on the path up to step i; the GPU picked got[i]
        _prove_tie(path, max_ctx, prefill, token, pos, ref_ids, i, int(got[i]))
        ties.append(i)
        # continue teacher-forced on the oracle's path from step i + 1; the
        # replay from a reset state covers models whose DeltaNet recurrence
        # cannot be rewound (a dense cache is simply overwritten)
        if prefill is None:
            infer.engine_reset_state(e)
            e_tok = token
            for j in range(i + 1):
                infer.engine_forward(e, e_tok, pos + j)
                e_tok = int(ref_ids[j])
        e_tok = int(ref_ids[i])
        for j in range(i + 1, n):
            lg = infer.engine_forward(e, e_tok, pos + j)
            got_j = int(np.argmax(lg))
            if got_j != ref_ids[j]:
                _prove_tie(path, max_ctx, prefill, token, pos, ref_ids, j, got_j)
                ties.append(j)
            e_tok = int(ref_ids[j])
        break
    return ties


def test_c1_qwen3_06b_q8_0_64_greedy_steps(make_model):
    """BASELINE config 1 shape: logits at every one of the 64 steps and the
    64 greedy ids of the device-side loop."""
    path = make_model("qwen3-0.6b-q8_0")
    max_ctx, n = 256, 64
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    try:
        ref_ids, margins, kept = _oracle_path(r, 0, 0, n, n)
        print("C1 oracle top-1/top-2 margins:", " ".join("%.2g" % m for m in margins))
        # logits, teacher-forced on the oracle's path
        tok, worst = 0, 0.0
        for i in range(n):
            got = infer.engine_forward(e, tok, i).copy()
            worst = max(worst, scaled_err(got, kept[i]))
            tok = int(ref_ids[i])
        print("C1 worst scaled logit error over %d steps: %.3g" % (n, worst))
        assert worst <= TOL
        ties = _check_greedy(e, path, max_ctx, None, 0, 0, ref_ids, margins)
        print("C1 proven f32 ties:", ties)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.timeout(900)
def test_c3_qwen3_8b_q4_k_m_decode_from_4096(make_model):
    """BASELINE config 3 (the bench's workload): f16 KV pre-filled with N(0,1)
    to 4096 (the bench's seed), token 0 at position 4096; logits of the first
    8 steps and the 64 greedy ids of the device-side loop."""
    path = make_model("qwen3-8b-q4_k_m")
    L, n, nlog = 4096, 64, 8
    max_ctx = L + n + 8
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    try:
        cfg = infer.engine_config(e)
        assert (cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.hidden_dim, cfg.vocab_size) == (
            4096, 36, 32, 8, 12288, 151936)
        k, v = synth.kv_prefill(4242, cfg.n_layers, cfg.n_kv_heads, L, cfg.head_dim)
        infer.engine_kv_fill(e, 0, 0, k, v)
        for l in range(cfg.n_layers):
            r.kv_fill(l, 0, k[l], v[l])
        ref_ids, margins, kept = _oracle_path(r, 0, L, n, nlog)
        print("C3 oracle top-1/top-2 margins:", " ".join("%.2g" % m for m in margins))
        tok, worst = 0, 0.0
        for i in range(nlog):
            got = infer.engine_forward(e, tok, L + i).copy()
            err = scaled_err(got, kept[i])
            worst = max(worst, err)
            assert err <= TOL, "step %d scaled error %.3g" % (i, err)
            tok = int(ref_ids[i])
        print("C3 worst scaled logit error over %d steps: %.3g" % (nlog, worst))
        ties = _check_greedy(e, path, max_ctx, (k, v), 0, L, ref_ids, margins)
        print("C3 proven f32 ties:", ties)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.timeout(900)
def test_c4_qwen3_moe_decode_from_2048(make_model):
    """BASELINE config 4 at its own context: the Qwen3-30B-A3B layer shapes
    (32 query / 4 KV heads, so the attention kernel serves 8 query heads per
    KV head; 128 experts top 8, expert inner 768) on 4 layers, f16 KV
    pre-filled with N(0,1) to 2048 positions, token 0 at position 2048: the
    split attention over 33 splits and their merge, the router and the routed
    experts against the oracle -- logits of the first 8 steps and the 64
    greedy ids of the device-side loop (infer/forward.odin:87-115 for the
    attention; the routed FFN restates the HF Qwen3-MoE convention)."""
    path = make_model("qwen3-30b-a3b-4layer")
    L, n, nlog = 2048, 64, 8
    max_ctx = L + n + 8
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    try:
        cfg = infer.engine_config(e)
        assert (cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.vocab_size) == (2048, 4, 32, 4, 151936)
        k, v = synth.kv_prefill(4343, cfg.n_layers, cfg.n_kv_heads, L, cfg.head_dim)
        infer.engine_kv_fill(e, 0, 0, k, v)
        for l in range(cfg.n_layers):
            r.kv_fill(l, 0, k[l], v[l])
        ref_ids, margins, kept = _oracle_path(r, 0, L, n, nlog)
        print("C4 oracle top-1/top-2 margins:", " ".join("%.2g" % m for m in margins), flush=True)
        tok, worst = 0, 0.0
        for i in range(nlog):
            got = infer.engine_forward(e, tok, L + i).copy()
            err = scaled_err(got, kept[i])
            worst = max(worst, err)
            assert err <= TOL, "step %d scaled error %.3g" % (i, err)
            tok = int(ref_ids[i])
        print("C4 worst scaled logit error over %d steps from position %d: %.3g" % (nlog, L, worst))
        ties = _check_greedy(e, path, max_ctx, (k, v), 0, L, ref_ids, margins)
        print("C4 proven f32 ties:", ties)
    finally:
        infer.engine_destroy(e)
        r.close()


def _walk_logits(e, r, n, token=0):
    """Teacher-forced on the oracle's greedy path from position 0: the worst
    scaled logit error over n steps and the oracle's ids and margins."""
    ids, margins, worst = [], [], 0.0
    for pos in range(n):
        got = infer.engine_forward(e, token, pos).copy()
        ref = r.forward(token, pos)
        worst = max(worst, scaled_err(got, ref))
        token, m = _top2(ref)
        ids.append(token)
        margins.append(m)
    return worst, np.array(ids, np.int32), margins


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name,steps", [
    ("moe-tiny", 48),                 # routed experts (Qwen3-MoE layout), small
    ("qwen35-tiny", 48),              # hybrid: 3 DeltaNet layers + 1 full-attention layer, dense FFN
    ("qwen35-moe-tiny", 48),          # hybrid + routed experts + shared expert
    ("qwen3-30b-a3b-4layer", 32),     # config 4's layer shapes: 128 experts top 8, inner 768, 32/4 heads
    ("qwen35-hybrid-moe-4layer", 32),  # config 5's layer shapes: 512 experts top 10 + shared, 16/2 heads of 256
])
def test_moe_and_hybrid_models_vs_oracle(make_model, name, steps):
    """Per-step logits within 1e-3 on the oracle's greedy path from token 0 at
    position 0, then the device-side greedy loop from a reset state against
    the oracle's ids (a differing step must be a proven f32 tie)."""
    path = make_model(name)
    max_ctx = 128
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=max_ctx))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=max_ctx, num_threads=NTHREADS, kv_f16=True)
    try:
        worst, ref_ids, margins = _walk_logits(e, r, steps)
        print("%s worst scaled logit error over %d steps: %.3g" % (name, steps, worst))
        assert worst <= TOL
        infer.engine_reset_state(e)  # the DeltaNet states cannot be rewound
        ties = _check_greedy(e, path, max_ctx, None, 0, 0, ref_ids, margins)
        print("%s proven f32 ties:" % name, ties)
    finally:
        infer.engine_destroy(e)
        r.close()


def test_reset_state_repeats_the_first_token(make_model):
    """engine_reset_state (qwen3_5/engine.odin:108-132) zeroes the DeltaNet
    states and the cache: the same prompt gives the same logits again."""
    path = make_model("qwen35-tiny")
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
    try:
        first = [infer.engine_forward(e, t, p).copy() for p, t in enumerate([3, 9, 27])]
        infer.engine_reset_state(e)
        again = [infer.engine_forward(e, t, p).copy() for p, t in enumerate([3, 9, 27])]
        for a, b in zip(first, again):
            assert np.array_equal(a, b)
    finally:
        infer.engine_destroy(e)


@pytest.mark.parametrize("name", ["qwen35-tiny", "qwen35-hybrid-moe-2layer"])
def test_split_deltanet_step_matches_fused(make_model, monkeypatch, name):
    """The token loop's DeltaNet step in its split form (the conv as the
    in_qkv GEMV's epilogue, the delta rule over (value head, 32 columns)
    workgroups, the gated norm as the output GEMV's prologue; the default)
    against the one-launch step (OI_DN_FUSED=1): the same f32 arithmetic up
    to the order of the sums.  Over 24 steps the logits agree within 2e-4,
    the scale of the f32 order noise on these models (each form is within
    ~5e-5 of the oracle; the recurrent state carries a step's rounding into
    every later step)."""
    path = make_model(name)
    toks = [int(t) for t in np.random.default_rng(3).integers(0, 2048, 24)]
    out = {}
    for fused in (False, True):
        if fused:
            monkeypatch.setenv("OI_DN_FUSED", "1")
        e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=64))
        assert ok
        try:
            out[fused] = [infer.engine_forward(e, t, p).copy() for p, t in enumerate(toks)]
        finally:
            infer.engine_destroy(e)
    worst = max(scaled_err(a, b) for a, b in zip(out[False], out[True]))
    print("%s: split vs fused DeltaNet step, worst scaled logit difference %.3g" % (name, worst))
    assert worst <= 2e-4


@pytest.mark.parametrize("overrides", [
    {"n_heads": 16, "n_kv_heads": 2, "head_dim": 256},  # groups of 8 query heads (8-wave workgroups)
    {"n_heads": 4, "n_kv_heads": 2, "head_dim": 256},   # groups of 2
])
def test_head_dim_256_decode_vs_oracle(make_model, overrides):
    """Dense decode attention at head_dim 256 (attn_kernel<256, G>: 4 values
    per lane in o, 32 16-byte chunks per K row): a two-layer model of the
    small shape with the head layout overridden, KV pre-filled with N(0,1) to
    300 positions (5 splits), logits of 4 steps within 1e-3 of the oracle
    (f16 KV) and the same argmax."""
    path = make_model("tiny-q4_k", **overrides)
    L = 300
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=L + 16))
    assert ok
    r = refcpu.RefEngine(path, max_ctx=L + 16, num_threads=NTHREADS, kv_f16=True)
    try:
        cfg = infer.engine_config(e)
        assert cfg.head_dim == 256
        k, v = synth.kv_prefill(91, cfg.n_layers, cfg.n_kv_heads, L, cfg.head_dim)
        infer.engine_kv_fill(e, 0, 0, k, v)
        for l in range(cfg.n_layers):
            r.kv_fill(l, 0, k[l], v[l])
        toks = [int(t) for t in np.random.default_rng(9).integers(0, cfg.vocab_size, 4)]
        for i, t in enumerate(toks):
            got = infer.engine_forward(e, t, L + i).copy()
            ref = r.forward(t, L + i)
            err = scaled_err(got, ref)
            print("head_dim 256, group %d, step %d: scaled error %.3g" % (cfg.n_heads // cfg.n_kv_heads, i, err))
            assert err <= TOL
            assert int(np.argmax(got)) == refcpu.argmax(ref)
    finally:
        infer.engine_destroy(e)
        r.close()


@pytest.mark.parametrize("name,overrides,L", [
    ("tiny-q4_k", {"n_heads": 2, "n_kv_heads": 2}, 700),  # 1 query head per KV head
    ("qwen3-0.6b-q8_0", {"n_layers": 2}, 1500),           # 2 (config 1's heads)
    ("small-q4_k", {}, 3000),                              # 4
    ("qwen3-30b-a3b-4layer", {}, 2048),                    # 8 (config 4's heads)
])
def test_decode_attention_kernels_agree(make_model, monkeypatch, name, overrides, L):
    """The head_dim-128 decode attention on the lane-per-position kernel over
    splits of 64 (the default, f32 q) against the matrix-core kernel
    (OI_ATTN=mfma: splits sized from pos, one 16-key tile per wave, q split
    into f16 + remainder, f32 sums): the same f32 arithmetic up to the order
    of the sums and q's ~2^-22 rounding.  8 steps from a KV cache pre-filled
    with N(0,1) to L positions, logits within 2e-5 (scaled) of each other
    (the matrix-core kernel without the remainder columns measured 4.1e-4 on
    small-q4_k); the default is within 1e-3 of the oracle in the tests above."""
    path = make_model(name, **overrides)
    out = {}
    for kind in ("default", "mfma"):
        if kind == "mfma":
            monkeypatch.setenv("OI_ATTN", "mfma")
        e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=L + 16))
        assert ok
        try:
            cfg = infer.engine_config(e)
            k, v = synth.kv_prefill(77, cfg.n_layers, cfg.n_kv_heads, L, cfg.head_dim)
            infer.engine_kv_fill(e, 0, 0, k, v)
            toks = [int(t) for t in np.random.default_rng(5).integers(0, cfg.vocab_size, 8)]
            out[kind] = [infer.engine_forward(e, t, L + i).copy() for i, t in enumerate(toks)]
        finally:
            infer.engine_destroy(e)
    worst = max(scaled_err(a, b) for a, b in zip(out["default"], out["mfma"]))
    print("%s (L=%d): matrix-core vs lane-per-position attention, worst scaled logit difference %.3g"
          % (name, L, worst))
    assert worst <= 2e-5
