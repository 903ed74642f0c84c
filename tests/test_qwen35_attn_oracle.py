"""The oracle's Qwen3.5 full-attention step (refcpu.c, restating
qwen3_5/forward.odin:69-127 and qwen3_5/ops.odin:77-89, 163-168) pinned by the
reference's RoPE known answers (qwen3_5/tests.odin:97-125), the inv_freq
closed form, and an independent float64 model of the step; the float64
variants with RoPE over the whole head or without the output gate must fail
the same bound."""
import numpy as np
import pytest

import npref
import refcpu


def test_mrope_zero_pos_is_identity():  # tests.odin:97-112
    inv = refcpu.inv_freq(10000.0, 4)
    assert np.allclose(refcpu.mrope([1.5, -2.0, 3.0, 4.0], 0, inv, 4), [1.5, -2.0, 3.0, 4.0], atol=1e-5)


def test_mrope_partial_passthrough():  # tests.odin:114-125
    inv = refcpu.inv_freq(10000.0, 2)
    v = refcpu.mrope([1.0, 0.0, 5.0, 6.0], 7, inv, 2)
    assert v[2] == 5.0 and v[3] == 6.0
    assert np.allclose(v[:2], [np.cos(7.0), np.sin(7.0)], atol=1e-5)  # pair (0, 1), inv_freq[0] = 1


def test_inv_freq_closed_form():
    inv = refcpu.inv_freq(1e6, 64)
    assert np.allclose(inv, 1e6 ** (-(np.arange(32) / 32.0)), rtol=1e-6)


def _case(rng, n_heads, n_kv, hd, rd, seq_len, pos0, T):
    f = np.float32
    kc = np.zeros((n_kv, seq_len, hd), np.float16)
    vc = np.zeros((n_kv, seq_len, hd), np.float16)
    kc[:, :pos0] = rng.standard_normal((n_kv, pos0, hd))
    vc[:, :pos0] = rng.standard_normal((n_kv, pos0, hd))
    return dict(n_heads=n_heads, n_kv=n_kv, hd=hd, rd=rd, seq_len=seq_len, eps=1e-6, pos0=pos0,
                qproj=rng.standard_normal((T, n_heads * 2 * hd)).astype(f),
                k=rng.standard_normal((T, n_kv * hd)).astype(f), v=rng.standard_normal((T, n_kv * hd)).astype(f),
                q_norm=(1 + 0.1 * rng.standard_normal(hd)).astype(f),
                k_norm=(1 + 0.1 * rng.standard_normal(hd)).astype(f),
                kc=kc.view(np.uint16), vc=vc.view(np.uint16))


@pytest.mark.parametrize("shape", [(4, 2, 32, 8, 64, 0, 6), (2, 1, 16, 16, 40, 20, 4), (4, 4, 8, 0, 16, 3, 3)])
def test_qwen35_attn_vs_float64(shape):
    c = _case(np.random.default_rng(sum(shape)), *shape)
    theta = 1e6
    inv = refcpu.inv_freq(theta, c["rd"]) if c["rd"] else np.zeros(1, np.float32)
    out, kc, vc = refcpu.qwen35_attn_steps(c["n_heads"], c["n_kv"], c["hd"], c["rd"], c["seq_len"], c["eps"],
                                           c["pos0"], c["qproj"], c["k"], c["v"], c["q_norm"], c["k_norm"], inv,
                                           c["kc"], c["vc"])
    args = (c["n_heads"], c["n_kv"], c["hd"], c["rd"], c["seq_len"], c["eps"], c["pos0"], c["qproj"], c["k"],
            c["v"], c["q_norm"], c["k_norm"], theta, c["kc"], c["vc"])
    ref = npref.qwen35_attn_f64(*args)
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err <= 1e-4, err
    for bad in (dict(gate=False), dict(full_rotary=True)):
        if bad.get("full_rotary") and c["rd"] == c["hd"]:
            continue
        alt = npref.qwen35_attn_f64(*args, **bad)
        assert np.max(np.abs(out - alt)) / np.max(np.abs(ref)) > 100 * 1e-4, bad
