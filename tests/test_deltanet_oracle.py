"""The oracle's gated DeltaNet step (refcpu.c, restating qwen3_5/ops.odin and
forward.odin:172-219) pinned by the reference's own known answers
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
