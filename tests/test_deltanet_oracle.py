"""The oracle's gated DeltaNet step (refcpu.c, restating qwen3_5/ops.odin and
qwen3_5/forward.odin:172-219) pinned by the reference's own known answers
(qwen3_5/tests.odin:13-95, 141-150) and by an independent float64 model of
the whole step; the float64 model with the mistake of the reference's
delta_harness golden (memory read with q, delta_ref.odin:61) must fail the
same bound."""
import numpy as np
import pytest

import npref
import refcpu


def test_delta_first_write():  # tests.odin:13-38
    out, st = refcpu.delta_step(np.zeros((2, 2)), [1, 0], [1, 0], [1, 1], 1.0, 1.0)
    assert np.allclose(out, [1, 1], atol=1e-5) and np.allclose(st, [[1, 1], [0, 0]], atol=1e-5)


def test_delta_partial_beta():  # tests.odin:40-58
    out, _ = refcpu.delta_step(np.zeros((2, 2)), [1, 0], [1, 0], [1, 1], 0.5, 1.0)
    assert np.allclose(out, [0.5, 0.5], atol=1e-5)


def test_delta_decay():  # tests.odin:60-78
    out, st = refcpu.delta_step(np.array([[2.0, 0], [0, 0]]), [1, 0], [1, 0], [1.0, 0.0], 1.0, 0.5)
    assert abs(st[0, 0] - 1.0) <= 1e-5 and abs(out[0] - 1.0) <= 1e-5


def test_conv1d_single_token():  # tests.odin:80-95
    out, st = refcpu.conv1d([0.0], [2.0], [1.0, 1.0], 2)
    assert abs(out[0] - 2.0 / (1.0 + np.exp(-2.0))) <= 1e-5 and st[0] == 0.0


def test_conv1d_window_order():
    # current input last, history oldest first; the state slides by one
    w = np.array([1.0, 10.0, 100.0, 1000.0], np.float32)  # taps: oldest .. current
    out, st = refcpu.conv1d([4.0], [1.0, 2.0, 3.0], w, 4)
    pre = 1.0 * 1 + 10.0 * 2 + 100.0 * 3 + 1000.0 * 4
    assert np.isclose(out[0], pre / (1 + np.exp(-pre)), rtol=1e-6) and np.array_equal(st, [2.0, 3.0, 4.0])


def test_l2norm_unit():  # tests.odin:141-150
    assert np.allclose(refcpu.l2norm([3.0, 4.0]), [0.6, 0.8], atol=1e-5)
    assert np.array_equal(refcpu.l2norm([0.0, 0.0]), [0.0, 0.0])  # the eps floor keeps zero finite


def _case(rng, n_kh, n_vh, hk, hv, kernel, T):
    kd, vd = n_kh * hk, n_vh * hv
    cd = 2 * kd + vd
    return dict(n_kh=n_kh, n_vh=n_vh, hk=hk, hv=hv, kernel=kernel, eps=1e-6,
                qkv=rng.standard_normal((T, cd)), z=rng.standard_normal((T, vd)),
                b=rng.standard_normal((T, n_vh)), a=rng.standard_normal((T, n_vh)),
                conv_w=rng.standard_normal(cd * kernel) * 0.5, a_decay=-np.exp(rng.standard_normal(n_vh) * 0.5),
                dt_bias=rng.standard_normal(n_vh) * 0.5, norm_w=1 + 0.1 * rng.standard_normal(hv),
                conv_state=rng.standard_normal(cd * (kernel - 1)), rec_state=rng.standard_normal(n_vh * hk * hv) * 0.1)


@pytest.mark.parametrize("shape", [(2, 4, 16, 16, 4, 8), (1, 3, 8, 32, 2, 5), (2, 2, 16, 8, 1, 3)])
def test_deltanet_steps_vs_float64(shape):
    c = _case(np.random.default_rng(sum(shape)), *shape)
    args = [c[k] for k in ("n_kh", "n_vh", "hk", "hv", "kernel", "eps", "qkv", "z", "b", "a", "conv_w", "a_decay",
                           "dt_bias", "norm_w", "conv_state", "rec_state")]
    out, cs, rs = refcpu.deltanet_steps(*args)
    ref, rcs, rrs = npref.deltanet_f64(*args)
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err <= 2e-5, err
    assert np.max(np.abs(rs - rrs)) / np.max(np.abs(rrs)) <= 2e-5
    if c["kernel"] > 1:
        assert np.array_equal(cs, rcs.astype(np.float32))  # the window only moves values
    bad, _, _ = npref.deltanet_f64(*args, kv_from_q=True)
    assert np.max(np.abs(out - bad)) / np.max(np.abs(ref)) > 100 * 2e-5


# ----- the chunked form of the delta rule (qwen3_5/metal.odin:416-468) -----

def _chunk_case(rng, C, hk, hv, beta=None, g=None):
    q = rng.standard_normal((C, hk))
    k = rng.standard_normal((C, hk))
    q /= np.linalg.norm(q, axis=1, keepdims=True) * np.sqrt(hk)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.uniform(-1, 1, (C, hv))
    beta = rng.uniform(0.2, 0.8, C) if beta is None else np.broadcast_to(np.float64(beta), (C,))
    g = rng.uniform(0.25, 0.99, C) if g is None else np.broadcast_to(np.float64(g), (C,))
    S = rng.standard_normal((hk, hv)) * 0.1
    f = lambda x: np.asarray(x, np.float32).astype(np.float64)  # the f32 values both sides see
    return f(S), f(q), f(k), f(v), f(beta), f(g)


@pytest.mark.parametrize("C,hk,hv", [(1, 8, 8), (2, 16, 8), (5, 16, 16), (16, 32, 16), (33, 16, 24)])
def test_delta_chunk_f64_equals_tokenwise(C, hk, hv):
    """The chunked form is an exact rewriting of C token steps: in float64 the
    two agree to rounding; each planted mistake in the chunked form departs
    by far more."""
    case = _chunk_case(np.random.default_rng(C * 31 + hk), C, hk, hv)
    o_t, s_t = npref.delta_tokens_f64(*case)
    o_c, s_c = npref.delta_chunk_f64(*case)
    scale = max(np.max(np.abs(o_t)), 1e-30)
    assert np.max(np.abs(o_c - o_t)) / scale <= 1e-12
    assert np.max(np.abs(s_c - s_t)) / np.max(np.abs(s_t)) <= 1e-12
    for m in ("no_ratio", "o_strict", "state_ratio", "l_diag"):
        o_m, s_m = npref.delta_chunk_f64(*case, mistake=m)
        if C == 1 and m in ("no_ratio", "state_ratio"):
            continue  # one token: the ratios are all 1
        err = max(np.max(np.abs(o_m - o_t)) / scale, np.max(np.abs(s_m - s_t)) / np.max(np.abs(s_t)))
        assert err > 1e-3, m


@pytest.mark.parametrize("C", [1, 3, 16, 32, 64])
def test_oracle_delta_chunk_vs_f64(C):
    """refcpu.ref_delta_chunk (f32) against the float64 chunked form at head
    dims 128, decays down to 0.25 (a 64-token chunk's running product reaches
    ~1e-20, still a normal f32)."""
    case = _chunk_case(np.random.default_rng(C), C, 128, 128)
    out, st = refcpu.delta_chunk(*case)
    o64, s64 = npref.delta_chunk_f64(*case)
    assert np.max(np.abs(out - o64)) / np.max(np.abs(o64)) <= 2e-5
    assert np.max(np.abs(st - s64)) / np.max(np.abs(s64)) <= 2e-5
    for m in ("o_strict", "l_diag") + (("no_ratio", "state_ratio") if C > 1 else ()):
        om, sm = npref.delta_chunk_f64(*case, mistake=m)
        assert max(np.max(np.abs(out - om)) / np.max(np.abs(o64)), np.max(np.abs(st - sm)) / np.max(np.abs(s64))) > 1e-3


def _ladder_beta(kind, t):
    return {"real": 0.55, "one": 1.0, "tiny": 0.01, "sin": 0.3 + 0.4 * np.sin(t),
            "saw": 0.2 + 0.6 * ((t * 0.31) % 1.0)}[kind]


def _ladder_g(kind, t):
    return {"real": 0.99, "slow": 0.999, "strong": 0.1, "one": 1.0, "cos": 0.4 + 0.4 * np.cos(t * 0.7),
            "saw": 0.25 + 0.6 * ((t * 0.47) % 1.0)}[kind]


@pytest.mark.parametrize("C,T,bk,gk", [(1, 256, "real", "real"), (2, 256, "real", "real"), (4, 256, "real", "real"),
                                       (8, 256, "real", "real"), (16, 256, "real", "real"),
                                       (16, 1024, "real", "slow"), (16, 1024, "one", "real"),
                                       (16, 256, "sin", "cos"), (16, 256, "saw", "saw"), (16, 256, "tiny", "real"),
                                       (16, 256, "real", "strong"), (16, 256, "real", "one")])
def test_oracle_chunked_ladder(C, T, bk, gk):
    """The reference's chunked-vs-tokenwise ladder (delta_ref.odin:288-399:
    head dims 128, l2-normalized q (times 1/sqrt(128)) and k, v in [-1, 1],
    zero initial state, the listed beta / decay schedules, chunks of C): the
    oracle's chunked form against its token steps, output within the
    reference's 1e-2 absolute bound and, tighter, 1e-4 of the output scale;
    the state too."""
    rng = np.random.default_rng(C * 7 + T)
    t = np.arange(T)
    beta = np.array([_ladder_beta(bk, x) for x in t], np.float32)
    g = np.array([_ladder_g(gk, x) for x in t], np.float32)
    _, q, k, v, _, _ = _chunk_case(rng, T, 128, 128)
    s_tok = np.zeros((128, 128), np.float32)
    out_tok = np.empty((T, 128), np.float32)
    for i in range(T):
        out_tok[i], s_tok = refcpu.delta_step(s_tok, q[i], k[i], v[i], float(beta[i]), float(g[i]))
    s_ch = np.zeros((128, 128), np.float32)
    out_ch = np.empty((T, 128), np.float32)
    for lo in range(0, T, C):
        out_ch[lo:lo + C], s_ch = refcpu.delta_chunk(s_ch, q[lo:lo + C], k[lo:lo + C], v[lo:lo + C],
                                                     beta[lo:lo + C], g[lo:lo + C])
    d = np.max(np.abs(np.float64(out_ch) - out_tok))
    assert d < 1e-2
    assert d <= 1e-4 * np.max(np.abs(out_tok)), d
    assert np.max(np.abs(np.float64(s_ch) - s_tok)) <= 1e-4 * np.max(np.abs(s_tok))


@pytest.mark.parametrize("chunk,T", [(1, 7), (3, 10), (16, 37), (64, 37), (16, 64)])
def test_deltanet_steps_chunked_vs_tokenwise(chunk, T):
    """The whole step with the delta rule in chunks (ragged last chunk) against
    the oracle's token steps and the float64 model; a planted mistake in the
    float64 model still fails the bound."""
    c = _case(np.random.default_rng(chunk * 100 + T), 2, 4, 16, 16, 4, T)
    args = [c[k] for k in ("n_kh", "n_vh", "hk", "hv", "kernel", "eps", "qkv", "z", "b", "a", "conv_w", "a_decay",
                           "dt_bias", "norm_w", "conv_state", "rec_state")]
    out, cs, rs = refcpu.deltanet_steps_chunked(*args[:6], chunk, *args[6:])
    tok, tcs, trs = refcpu.deltanet_steps(*args)
    ref, rcs, rrs = npref.deltanet_f64(*args)
    assert np.array_equal(cs, tcs)
    for got, want in ((out, ref), (rs, rrs)):
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= 2e-5
    assert np.max(np.abs(out - tok)) / np.max(np.abs(tok)) <= 2e-5
    bad, _, _ = npref.deltanet_f64(*args, kv_from_q=True)
    assert np.max(np.abs(out - bad)) / np.max(np.abs(ref)) > 100 * 2e-5
