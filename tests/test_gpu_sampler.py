"""The device sampler (sample.hip) against the oracle's restatement of
sampler/sampler.odin:141-199.

The device sums running probabilities exactly (64-bit fixed point), the
reference in sequential f32.  So:
  * temperature 0 (argmax after the penalty) and a zero coin (seed 0, the
    serve harness's setting) must give the oracle's pick exactly;
  * otherwise the device's pick must be the float64 pick (softmax and running
    sums in float64 on the same f32 tempered logits), except where the target
    lies within 1e-6 of a boundary (the device's probabilities carry an ulp
    or two of exp and of a tree-ordered f32 sum); how often the
    reference's f32 pick differs from exact arithmetic is pinned on the CPU
    (tests/test_sampler_oracle.py);
  * the xorshift state advances exactly as the reference's, one draw per
    sample, none at temperature 0.
"""
import os

import numpy as np
import pytest

import refcpu
from helpers import scaled_err
from oi import infer

pytestmark = pytest.mark.gpu
F32 = np.float32
NT = min(16, os.cpu_count() or 1)


def _penalised(logits, penalty, last):
    x = np.array(logits, F32, copy=True)
    seen = set()
    if penalty != 1.0:
        for t in last:
            if 0 <= t < x.size and t not in seen:
                seen.add(t)
                x[t] = x[t] / F32(penalty) if x[t] > 0 else x[t] * F32(penalty)
    return x


def exact_pick(logits, t, topp, coin, penalty=1.0, last=()):
    """The reference's algorithm in float64 (softmax and running sums) on the
    f32 penalised, tempered logits; also the distance of the target from the
    nearest boundary."""
    x = (_penalised(logits, penalty, last) / F32(t)).astype(F32).astype(np.float64)
    p = np.exp(x - x.max())
    p /= p.sum()  # exact-enough softmax: the f32 sequential sum of 150k terms is not
    n = p.size
    if topp <= 0 or topp >= 1:
        c = np.cumsum(p)
        i = int(np.searchsorted(c, coin, side="right"))
        return min(i, n - 1), float(np.min(np.abs(c - coin)))
    cutoff = F32(F32(1.0) - F32(topp)) / F32(n - 1)
    p32 = p.astype(F32)
    idx = np.nonzero(p32 >= cutoff)[0]
    order = idx[np.lexsort((idx, -p[idx]))]
    c = np.cumsum(p[order])
    k = int(np.searchsorted(c, float(F32(topp)), side="right"))
    last_i = min(k, order.size - 1)
    r = coin * c[last_i]
    j = min(int(np.searchsorted(c[:last_i + 1], r, side="right")), last_i)
    margin = min(float(np.min(np.abs(c - float(F32(topp))))), float(np.min(np.abs(c - r))))
    return int(order[j]), margin


@pytest.mark.parametrize("n", [2048, 151936])
def test_sampler_against_exact_picks(n):
    rng = np.random.default_rng(n)
    logits = (rng.standard_normal(n) * 3).astype(F32)
    near = total = 0
    for t in (0.6, 1.0, 1.7):
        for topp in (0.0, 0.5, 0.9, 0.95, 1.0):
            s = infer.Sampler(t, topp, rng_seed=1000 + n)
            for _ in range(10):
                coin, st_next = refcpu.random_f32(s.rng_state)
                got = infer.sample(s, logits)
                assert s.rng_state == st_next
                want, margin = exact_pick(logits, t, topp, coin)
                total += 1
                if got != want:
                    near += 1
                    assert margin <= 1e-6, (t, topp, got, want, margin)
    print("n=%d: %d of %d picks within 1e-6 of a boundary and different" % (n, near, total))
    assert near <= total // 50


def test_temperature_zero_and_penalty_match_the_oracle_exactly():
    rng = np.random.default_rng(1)
    for n in (3, 2048, 151936):
        logits = (rng.standard_normal(n) * 2).astype(F32)
        last = list(rng.integers(0, n, 40)) + [-1, n + 5]
        for penalty in (1.0, 1.3, 2.0):
            s = infer.Sampler(0.0, 0.9, rng_seed=55, repeat_penalty=penalty, last=last)
            got = infer.sample(s, logits)
            want, st = refcpu.sample(logits, 0.0, 0.9, penalty, last, rng_state=55)
            assert got == want and s.rng_state == st == 55
    # the penalty known answers of the oracle tests, on the device
    assert infer.sample(infer.Sampler(0.0, 0.0, repeat_penalty=2.0, last=[0, 0]), np.array([3, 0, 1.4], F32)) == 0
    assert infer.sample(infer.Sampler(0.0, 0.0, repeat_penalty=2.0, last=[0]), np.array([-1, -1.5], F32)) == 1


def test_penalty_below_one_is_clamped_at_the_c_abi():
    """enable_repeat_penalty clamps penalties below 1 to 1 (sampler.odin:42-44);
    a C caller that writes 0.5 or 0 into oi_sampler directly gets the same
    pick as the clamped reference (no division by 0, no inverted penalty)."""
    rng = np.random.default_rng(11)
    logits = (rng.standard_normal(2048) * 2).astype(F32)
    last = list(rng.integers(0, 2048, 30))
    for t, topp in ((0.0, 0.9), (0.7, 0.9)):
        for raw in (0.5, 0.0):
            s = infer.Sampler(t, topp, rng_seed=77, last=last)
            s.repeat_penalty = raw  # past the wrapper's clamp: the value reaches the C ABI
            got = infer.sample(s, logits)
            want, st = refcpu.sample(logits, t, topp, 1.0, last, rng_state=77)
            assert got == want and s.rng_state == st


def test_coin_near_one_matches_exact_picks():
    """Coins within 2^-24 of 1 (the largest the 24-bit coin takes): the pick is
    the float64 one, so rounding the fixed-point masses keeps the running
    total from falling short of the coin and the draw from falling through
    to the last vocabulary id."""
    from refcpu import random_f32
    rng = np.random.default_rng(12)
    logits = (rng.standard_normal(151936) * 0.5).astype(F32)  # flat: many small masses
    # xorshift64* states whose next coin is the largest, found by search on the CPU
    states, st = [], 1
    while len(states) < 3:
        coin, nxt = random_f32(st)
        if coin >= 1.0 - 2.0 ** -20:
            states.append(st)
        st = (st * 6364136223846793005 + 1442695040888963407) % 2 ** 64 or 1
    for st in states:
        coin, _ = random_f32(st)
        for t, topp in ((1.0, 0.0), (0.9, 0.95)):
            want, margin = exact_pick(logits, t, topp, coin)
            got = infer.sample(infer.Sampler(t, topp, rng_seed=st), logits)
            assert got == want or margin <= 1e-6, (st, coin, t, topp, got, want)


@pytest.mark.parametrize("topp", [0.9, 0.0])
def test_equal_probabilities_across_slices(topp):
    """A run of 12000 equal logits spanning several of the sampler's
    2048-logit workgroup slices: the top-p boundary and the coin fall inside
    the run, so the pick is the j-th equal probability in index order,
    counted across slices (top-p), or the first index past the coin's mass
    (multinomial)."""
    n = 20000
    logits = np.full(n, -2.0, F32)
    logits[3000:15000] = 1.0
    for seed in range(1, 13):
        coin, _ = refcpu.random_f32(seed)
        want, margin = exact_pick(logits, 1.0, topp, coin)
        got = infer.sample(infer.Sampler(1.0, topp, rng_seed=seed), logits)
        assert got == want or margin <= 1e-6, (seed, got, want)
        if topp:
            assert 3000 <= got < 15000


def test_zero_coin_matches_the_oracle_exactly():
    """seed 0 (serve.odin:1544): every coin is 0."""
    rng = np.random.default_rng(2)
    for n in (2048, 151936):
        logits = (rng.standard_normal(n) * 3).astype(F32)
        for t, topp in ((0.6, 0.95), (1.0, 0.0), (0.8, 0.5)):
            got = infer.sample(infer.Sampler(t, topp, rng_seed=0), logits)
            assert got == refcpu.sample(logits, t, topp, rng_state=0)[0]


def test_penalty_with_sampling_and_record_window():
    rng = np.random.default_rng(3)
    logits = (rng.standard_normal(4096) * 3).astype(F32)
    s = infer.Sampler(0.9, 0.9, rng_seed=7, repeat_penalty=1.5, record=True, last=list(range(60)))
    ref_last = list(range(60))
    for _ in range(8):
        coin, _ = refcpu.random_f32(s.rng_state)
        want, margin = exact_pick(logits, 0.9, 0.9, coin, 1.5, ref_last)
        got = infer.sample(s, logits)
        assert got == want or margin <= 1e-6
        ref_last = refcpu.record_token(ref_last, got, 1.5)
        assert s.last == ref_last
    assert len(s.last) == 64


@pytest.mark.parametrize("name", ["tiny-q8_0", "qwen35-tiny", "moe-tiny"])
def test_decode_sample_against_oracle_walk(make_model, name):
    """The device loop, step by step: a second engine and the oracle follow
    the device's picks; the second engine's logits (the same kernels) are
    within 1e-3 of the oracle's, and each pick is the float64 pick on those
    logits with the reference's coin (1e-6 boundary allowance)."""
    path = make_model(name)
    e, ok = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    e2, ok2 = infer.engine_load(path, infer.Engine_Opts(max_ctx=128))
    r = refcpu.RefEngine(path, max_ctx=128, num_threads=NT, kv_f16=True)
    try:
        n = 40
        s = infer.Sampler(0.8, 0.9, rng_seed=4242)
        st0 = s.rng_state
        ids = infer.engine_decode_sample(e, 5, 0, n, s)
        tok, st, near, worst = 5, st0, 0, 0.0
        for i in range(n):
            lg = infer.engine_forward(e2, tok, i).copy()
            worst = max(worst, scaled_err(lg, r.forward(tok, i)))
            coin, st = refcpu.random_f32(st)
            want, margin = exact_pick(lg, 0.8, 0.9, coin)
            if ids[i] != want:
                near += 1
                assert margin <= 1e-6, (i, ids[i], want, margin)
            tok = int(ids[i])
        assert s.rng_state == st
        assert worst <= 1e-3
        assert near <= 2
        print("%s: %d sampled steps, %d boundary cases, logits vs oracle %.3g" % (name, n, near, worst))
    finally:
        infer.engine_destroy(e)
        infer.engine_destroy(e2)
        r.close()


def test_decode_sample_degenerate_settings_equal_greedy(make_model):
    """Temperature 0, and a zero coin with top-p, both reduce to the greedy
    loop: the same ids as oi_engine_decode_greedy."""
    e, ok = infer.engine_load(make_model("tiny-q4_k"), infer.Engine_Opts(max_ctx=128))
    try:
        greedy = infer.engine_decode_greedy(e, 3, 0, 48)
        assert np.array_equal(infer.engine_decode_sample(e, 3, 0, 48, infer.Sampler(0.0, 0.9, rng_seed=9)), greedy)
        assert np.array_equal(infer.engine_decode_sample(e, 3, 0, 48, infer.Sampler(0.6, 0.95, rng_seed=0)), greedy)
        # the logits the sampler saw are the forward path's
        lg = infer.engine_forward(e, 3, 0).copy()
        assert scaled_err(lg, infer.engine_forward(e, 3, 0)) == 0
    finally:
        infer.engine_destroy(e)
