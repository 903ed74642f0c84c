"""The oracle's sampler (oracle/refcpu.c: sampler/sampler.odin:68-199 without
the grammar) pinned bit for bit against an independent float32 numpy
restatement, against float64 arithmetic within the f32 running sums' own
deviation, and by known answers and the reference's degenerate settings
(seed 0, temperature 0).  CPU only."""
import numpy as np
import pytest

import refcpu

F32 = np.float32
M64 = 2 ** 64 - 1


def xorshift(state):
    """random_u32 (sampler.odin:68-73), written from the published
    xorshift64* algorithm: three shifts, then the high word of a multiply."""
    state ^= state >> 12
    state = (state ^ (state << 25)) & M64
    state ^= state >> 27
    return ((state * 0x2545F4914F6CDD1D) & M64) >> 32, state


def coin_of(state):
    u, state = xorshift(state)
    return (u >> 8) / 16777216.0, state


def probs64(logits, t):
    x = np.asarray(logits, np.float64) / t
    e = np.exp(x - x.max())
    return e / e.sum()


def pick64(logits, t, topp, coin):
    """The reference's algorithm in float64 (ties: index order)."""
    p = probs64(logits, t)
    n = p.size
    if topp <= 0 or topp >= 1:
        c = np.cumsum(p)
        i = int(np.searchsorted(c, coin, side="right"))
        return min(i, n - 1), c
    cutoff = (1 - topp) / (n - 1)
    idx = np.nonzero(p >= cutoff)[0]
    order = idx[np.lexsort((idx, -p[idx]))]
    c = np.cumsum(p[order])
    k = int(np.searchsorted(c, topp, side="right"))
    last = min(k, order.size - 1)
    r = coin * c[last]
    j = int(np.searchsorted(c[:last + 1], r, side="right"))
    return int(order[min(j, last)]), c


def test_random_f32_sequences():
    for seed in (1, 42, 0x9E3779B97F4A7C15, 2 ** 63 + 5):
        st, ref = seed, seed
        for _ in range(50):
            v, st = refcpu.random_f32(st)
            c, ref = coin_of(ref)
            assert st == ref and v == F32(c)
    assert refcpu.random_f32(0) == (0.0, 0)  # a zero state stays zero (serve.odin:1544 seeds 0)


def pick32(logits, t, topp, coin):
    """The reference's algorithm restated with numpy in float32: the oracle's
    own softmax for the probabilities (pinned separately), sequential float32
    running sums (np.cumsum accumulates in order), ties in index order."""
    p = refcpu.softmax((np.asarray(logits, F32) / F32(t)).astype(F32))
    n = p.size
    coin = F32(coin)
    if topp <= 0 or topp >= 1:
        c = np.cumsum(p, dtype=F32)
        hit = np.nonzero(coin < c)[0]
        return int(hit[0]) if hit.size else n - 1
    cutoff = F32(F32(1.0) - F32(topp)) / F32(n - 1)
    idx = np.nonzero(p >= cutoff)[0]
    order = idx[np.lexsort((idx, -p[idx]))]
    c = np.cumsum(p[order], dtype=F32)
    over = np.nonzero(c > F32(topp))[0]
    last = int(over[0]) if over.size else order.size - 1
    r = F32(coin * c[last])
    hit = np.nonzero(r < c[:last + 1])[0]
    return int(order[hit[0]]) if hit.size else int(order[last])


CASES = [(t, topp) for t in (0.6, 1.0, 1.7) for topp in (0.0, 0.5, 0.9, 0.95, 1.0)]


@pytest.mark.parametrize("n", [7, 1000, 151936])
def test_sample_matches_float32_restatement(n):
    rng = np.random.default_rng(n)
    logits = (rng.standard_normal(n) * 3).astype(F32)
    for t, topp in CASES:
        st = 1234 + n
        for _ in range(12):
            coin, _ = refcpu.random_f32(st)
            got, st2 = refcpu.sample(logits, t, topp, rng_state=st)
            assert st2 == xorshift(st)[1]
            assert got == pick32(logits, t, topp, coin), (t, topp, st)
            st = st2


@pytest.mark.parametrize("n", [1000, 151936])
def test_float32_sums_against_exact(n):
    """How far the reference's f32 running sums move a pick: where the oracle
    and float64 disagree, the coin (or the top-p target) lies within the f32
    sums' own deviation from the exact sums at that point."""
    rng = np.random.default_rng(n + 1)
    logits = (rng.standard_normal(n) * 3).astype(F32)
    differ = 0
    for t, topp in CASES:
        st = 77 + n
        for _ in range(12):
            coin, _ = refcpu.random_f32(st)
            got, st = refcpu.sample(logits, t, topp, rng_state=st)
            want, c64 = pick64(logits, t, topp, coin)
            if got == want:
                continue
            differ += 1
            p = refcpu.softmax((logits / F32(t)).astype(F32))
            dev = np.max(np.abs(np.cumsum(p, dtype=F32).astype(np.float64) - np.cumsum(p.astype(np.float64))))
            targets = [coin] if topp in (0.0, 1.0) else [topp, coin * c64[min(np.searchsorted(c64, topp, "right"),
                                                                              c64.size - 1)]]
            assert min(np.min(np.abs(c64 - x)) for x in targets) <= 2 * dev + 1e-7
    print("n=%d: %d of %d draws differ from exact arithmetic" % (n, differ, 12 * len(CASES)))
    if n <= 1000:
        assert differ <= 2


def test_temperature_zero_is_first_argmax():
    x = np.array([1.0, 3.0, 3.0, -1.0], F32)
    assert refcpu.sample(x, 0.0, 0.9, rng_state=77) == (1, 77)  # no draw at temperature 0


def test_repeat_penalty_known_answers():
    # positive logits divided, negative multiplied (sampler.odin:154-158)
    assert refcpu.sample(np.array([-1.0, -1.5], F32), 0.0, 0.0, 2.0, [0])[0] == 1  # -2 < -1.5
    # a repeated token is penalised once: 3/2 = 1.5 > 1.4 (twice would give 0.75)
    assert refcpu.sample(np.array([3.0, 0.0, 1.4], F32), 0.0, 0.0, 2.0, [0, 0])[0] == 0
    # out-of-range ids in the window are skipped
    assert refcpu.sample(np.array([3.0, 0.0, 1.4], F32), 0.0, 0.0, 4.0, [-1, 7, 0])[0] == 2
    # penalty 1 is off
    assert refcpu.sample(np.array([3.0, 0.0, 1.4], F32), 0.0, 0.0, 1.0, [0])[0] == 0


def test_zero_coin_picks_the_most_probable():
    """serve.odin:1544 builds the sampler with seed 0: every coin is 0, so top-p
    returns the most probable token and sample_mult the first nonzero one."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(5000).astype(F32)
    assert refcpu.sample(x, 0.6, 0.95, rng_state=0)[0] == int(np.argmax(x))
    assert refcpu.sample(x, 0.6, 0.0, rng_state=0)[0] == 0


def test_equal_probabilities_split_by_coin():
    """Two equal logits: p = (0.5, 0.5) exactly; the coin decides."""
    x = np.array([2.0, 2.0], F32)
    seen = set()
    st = 99
    for _ in range(40):
        coin, _ = refcpu.random_f32(st)
        i, st = refcpu.sample(x, 1.0, 0.0, rng_state=st)
        assert i == (0 if coin < 0.5 else 1)
        seen.add(i)
    assert seen == {0, 1}


def test_record_token_window():
    w = refcpu.record_token([], 5, 1.1)
    assert w == [5]
    w = list(range(64))
    w = refcpu.record_token(w, 99, 1.1)
    assert len(w) == 64 and w[0] == 1 and w[-1] == 99
    assert refcpu.record_token([1, 2], 3, 1.0) == [1, 2]  # off when the penalty is 1
