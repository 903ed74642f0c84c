"""GPU parity of the Qwen3.5 full-attention step (oi_qwen35_attn_steps,
qwen35_attn.hip) against the oracle (refcpu.ref_qwen35_attn_steps, pinned by
the reference's RoPE known answers and a float64 model), at the Qwen3.5 shape
of the measurement plan (16 q heads of 256 with a gate, 2 kv heads, partial
RoPE over 64 dimensions) and at head_dim 128.  Bar: outputs within a scaled
error of 1e-4 (f32 sums in another order, device sin/cos); the cache entries
written agree to one f16 unit in the last place."""
import numpy as np
import pytest

import refcpu
from oi import _native, qwen35

pytestmark = pytest.mark.gpu


def _case(rng, n_heads, n_kv, hd, seq_len, pos0, T):
    f = np.float32
    kc = np.zeros((n_kv, seq_len, hd), np.float16)
    vc = np.zeros((n_kv, seq_len, hd), np.float16)
    kc[:, :pos0] = rng.standard_normal((n_kv, pos0, hd))
    vc[:, :pos0] = rng.standard_normal((n_kv, pos0, hd))
    return (rng.standard_normal((T, n_heads * 2 * hd)).astype(f), rng.standard_normal((T, n_kv * hd)).astype(f),
            rng.standard_normal((T, n_kv * hd)).astype(f), (1 + 0.1 * rng.standard_normal(hd)).astype(f),
            (1 + 0.1 * rng.standard_normal(hd)).astype(f), kc.view(np.uint16), vc.view(np.uint16))


@pytest.mark.parametrize("kernel", ["lanes", "groups"])
@pytest.mark.parametrize("n_heads,n_kv,hd,rd,seq_len,pos0,T", [
    (16, 2, 256, 64, 1024, 0, 40),     # measurement-plan shape from an empty cache
    (16, 2, 256, 64, 4096, 3000, 4),   # long context: 12 position splits
    (8, 2, 128, 128, 512, 100, 6),     # head_dim 128, full rotary
    (4, 4, 128, 0, 256, 7, 3),         # no rotary dimensions
    (4, 2, 256, 64, 512, 130, 5),      # a group of 2 query heads, head_dim 256
    (12, 2, 128, 64, 256, 70, 3),      # a group of 6 query heads (the dimension-split kernel either way)
])
def test_qwen35_attn_vs_oracle(monkeypatch, kernel, n_heads, n_kv, hd, rd, seq_len, pos0, T):
    """Both kernels: lane per position with one wave per query head (the
    default for groups of 1, 2, 4, 8 query heads) and the dimension-split
    kernel over groups of query heads (OI_Q35_ATTN=groups)."""
    monkeypatch.setenv("OI_Q35_ATTN", kernel)
    qproj, k, v, qn, kn, kc, vc = _case(np.random.default_rng(hd + pos0 + T), n_heads, n_kv, hd, seq_len, pos0, T)
    inv = refcpu.inv_freq(1e7, rd) if rd else np.zeros(1, np.float32)
    args = (n_heads, n_kv, hd, rd, seq_len, 1e-6, pos0, qproj, k, v, qn, kn, inv, kc, vc)
    out, gkc, gvc = qwen35.attn_steps(*args)
    rout, rkc, rvc = refcpu.qwen35_attn_steps(*args)
    err = np.max(np.abs(np.float64(out) - rout)) / np.max(np.abs(rout))
    assert err <= 1e-4, err
    assert np.array_equal(gvc, rvc)  # v is stored as given
    dk = np.abs(gkc.astype(np.int32) - rkc.astype(np.int32))
    assert dk.max() <= 1  # k after norm and RoPE: at most one f16 ulp apart


def test_qwen35_attn_rejects():
    qproj, k, v, qn, kn, kc, vc = _case(np.random.default_rng(1), 4, 2, 96, 64, 0, 1)
    with pytest.raises(_native.OIError):  # head_dim 96 is not built
        qwen35.attn_steps(4, 2, 96, 32, 64, 1e-6, 0, qproj, k, v, qn, kn, np.ones(16, np.float32), kc, vc)
    qproj, k, v, qn, kn, kc, vc = _case(np.random.default_rng(1), 4, 2, 128, 64, 0, 2)
    with pytest.raises(_native.OIError):  # positions past seq_len
        qwen35.attn_steps(4, 2, 128, 32, 64, 1e-6, 63, qproj, k, v, qn, kn, np.ones(16, np.float32), kc, vc)
