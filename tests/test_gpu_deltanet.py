"""GPU parity of the gated DeltaNet token step (oi_deltanet_steps,
deltanet.hip) against the oracle (refcpu.ref_deltanet_steps, pinned by the
reference's known answers and a float64 model) at the Qwen3.5 shape of the
measurement plan (16 k heads, 32 v heads, head dims 128, conv kernel 4) over a
trajectory that carries both states.  Bar: outputs and recurrent state within
a scaled error of 1e-5 (f32 sums in another order); the conv window moves
values only, so it must be bit-identical."""
import numpy as np
import pytest

import refcpu
from oi import _native, qwen35

pytestmark = pytest.mark.gpu


def _case(rng, n_kh, n_vh, hk, hv, kernel, T):
    kd, vd = n_kh * hk, n_vh * hv
    cd = 2 * kd + vd
    f = np.float32
    return [n_kh, n_vh, hk, hv, kernel, 1e-6,
            rng.standard_normal((T, cd)).astype(f), rng.standard_normal((T, vd)).astype(f),
            rng.standard_normal((T, n_vh)).astype(f), rng.standard_normal((T, n_vh)).astype(f),
            (rng.standard_normal(cd * kernel) * 0.5).astype(f), (-np.exp(rng.standard_normal(n_vh) * 0.5)).astype(f),
            (rng.standard_normal(n_vh) * 0.5).astype(f), (1 + 0.1 * rng.standard_normal(hv)).astype(f),
            rng.standard_normal(cd * (kernel - 1)).astype(f), (rng.standard_normal(n_vh * hk * hv) * 0.1).astype(f)]


def _err(a, b):
    return float(np.max(np.abs(np.float64(a) - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("n_kh,n_vh,kernel,T", [(16, 32, 4, 12), (2, 6, 4, 5), (4, 4, 1, 3)])
def test_deltanet_trajectory_vs_oracle(n_kh, n_vh, kernel, T):
    args = _case(np.random.default_rng(n_kh * 7 + n_vh + T), n_kh, n_vh, 128, 128, kernel, T)
    out, cs, rs = qwen35.deltanet_steps(*args)
    rout, rcs, rrs = refcpu.deltanet_steps(*args)
    assert _err(out, rout) <= 1e-5, _err(out, rout)
    assert _err(rs, rrs) <= 1e-5, _err(rs, rrs)
    assert np.array_equal(cs, rcs)


def test_deltanet_first_write_closed_form():
    """Zero state, q = k = e0 after the l2norm, beta = sigmoid(30) = 1 in f32,
    decay = exp(0) = 1: the delta rule stores v and reads it back through q
    (scaled by 1/sqrt(128)), so the output is rmsnorm(v / sqrt(128)) * norm_w *
    silu(z) (qwen3_5/tests.odin:13-38 at head dims 128, through the whole
    step)."""
    n_kh, n_vh, hk, hv, kernel = 1, 2, 128, 128, 1
    kd, vd = n_kh * hk, n_vh * hv
    rng = np.random.default_rng(5)
    qkv = np.zeros((1, 2 * kd + vd), np.float32)
    qkv[0, 0] = 2.0       # q of k head 0 along e0
    qkv[0, kd] = 3.0      # k along e0
    v_in = rng.uniform(0.5, 2.0, vd).astype(np.float32)
    qkv[0, 2 * kd:] = v_in
    conv_w = np.ones(2 * kd + vd, np.float32)  # kernel 1: out = silu(x)
    z = rng.standard_normal((1, vd)).astype(np.float32)
    norm_w = (1 + 0.1 * rng.standard_normal(hv)).astype(np.float32)
    out, _, rs = qwen35.deltanet_steps(n_kh, n_vh, hk, hv, kernel, 1e-6, qkv, z, np.full((1, n_vh), 30, np.float32),
                                      np.zeros((1, n_vh), np.float32), conv_w, np.zeros(n_vh, np.float32),
                                      np.zeros(n_vh, np.float32), norm_w, np.zeros(0, np.float32),
                                      np.zeros(n_vh * hk * hv, np.float32))
    v = np.float64(v_in) / (1 + np.exp(-np.float64(v_in)))  # silu
    for vh in range(n_vh):
        vv = v[vh * hv:(vh + 1) * hv]
        zz = np.float64(z[0, vh * hv:(vh + 1) * hv])
        o = vv / np.sqrt(hk)
        ref = o / np.sqrt(np.mean(o * o) + 1e-6) * norm_w * zz / (1 + np.exp(-zz))
        assert _err(out[0, vh * hv:(vh + 1) * hv], ref) <= 1e-5
        st = rs.reshape(n_vh, hk, hv)[vh]
        assert _err(st[0], vv) <= 1e-6 and not np.any(st[1:])


def test_deltanet_rejects_head_dims():
    args = _case(np.random.default_rng(0), 1, 1, 64, 64, 2, 1)
    with pytest.raises(_native.OIError):
        qwen35.deltanet_steps(*args)


def _moderate(args):
    """Decays of 0.2-0.9 per token: a 32-token chunk's running product stays a
    normal f32 (the oracle's chunked form divides running products, which
    turns to 0/0 once one underflows; the kernels work with sums of logs)."""
    rng = np.random.default_rng(len(args[6]))
    T, n_vh = args[8].shape
    args[9] = (rng.standard_normal((T, n_vh)) * 0.5 - 1.0).astype(np.float32)  # a
    args[11] = (-np.exp(rng.standard_normal(n_vh) * 0.25)).astype(np.float32)  # a_decay
    return args


@pytest.mark.parametrize("chunk,T", [(0, 3), (0, 37), (16, 3), (16, 37), (16, 200), (32, 37), (32, 200),
                                     (64, 3), (64, 37), (64, 64), (64, 200), (64, 512)])
def test_deltanet_batched_vs_oracle(chunk, T):
    """oi_deltanet_steps_batched (the prefill kernels: conv over the whole
    trajectory, then the delta rule token by token or in chunks of 16 / 32 /
    64 -- the last on the matrix cores -- with a ragged last chunk) against
    the oracle's same form
    (ref_deltanet_steps / ref_deltanet_steps_chunked) within 1e-5, and against
    the oracle's token steps within 1e-4 (the chunked form sums in another
    order); the conv window moves values only, bit-identical."""
    args = _moderate(_case(np.random.default_rng(T * 3 + chunk), 16, 32, 128, 128, 4, T))
    print("case chunk=%d T=%d" % (chunk, T), flush=True)
    out, cs, rs = qwen35.deltanet_steps_batched(*args[:6], chunk, *args[6:])
    tok, tcs, trs = refcpu.deltanet_steps(*args)
    rout, rcs, rrs = refcpu.deltanet_steps_chunked(*args[:6], chunk, *args[6:]) if chunk else (tok, tcs, trs)
    print("chunk %d T %d: vs oracle %.3g / state %.3g; vs token steps %.3g" %
          (chunk, T, _err(out, rout), _err(rs, rrs), _err(out, tok)))
    assert _err(out, rout) <= 1e-5, _err(out, rout)
    assert _err(rs, rrs) <= 1e-5, _err(rs, rrs)
    assert _err(out, tok) <= 1e-4 and _err(rs, trs) <= 1e-4
    assert np.array_equal(cs, rcs)


def test_deltanet_batched_rejects_bad_chunk():
    args = _case(np.random.default_rng(1), 2, 2, 128, 128, 4, 8)
    for chunk in (8, 48, -1):
        with pytest.raises(RuntimeError, match="chunk"):
            qwen35.deltanet_steps_batched(*args[:6], chunk, *args[6:])
    with pytest.raises(RuntimeError, match="n_tokens"):
        short = _case(np.random.default_rng(1), 2, 2, 128, 128, 4, 2)
        qwen35.deltanet_steps_batched(*short[:6], 16, *short[6:])
