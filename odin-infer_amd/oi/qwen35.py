"""Qwen3.5 hybrid-decoder pieces on the device: the gated DeltaNet token step
of a linear-attention layer (qwen3_5/forward.odin:137-225)."""
import ctypes

import numpy as np

from . import _native
from ._native import check


def _f32(x):
    return np.ascontiguousarray(x, np.float32)


def deltanet_steps(n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel, eps, qkv, z, b, a, conv_w, a_decay,
                   dt_bias, norm_w, conv_state, rec_state):
    """Run len(qkv) tokens through oi_deltanet_steps.  Inputs per token:
    qkv [T, conv_dim], z [T, n_v*hv], b, a [T, n_v].  Returns (out [T, n_v*hv],
    conv_state, rec_state) with the states after the last token (copies)."""
    d = _native.DeltaNetDims(n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel, eps)
    qkv, z, b, a = _f32(np.atleast_2d(qkv)), _f32(np.atleast_2d(z)), _f32(np.atleast_2d(b)), _f32(np.atleast_2d(a))
    conv_w, a_decay, dt_bias, norm_w = _f32(conv_w), _f32(a_decay), _f32(dt_bias), _f32(norm_w)
    cs, rs = _f32(conv_state).copy(), _f32(rec_state).copy()
    T = qkv.shape[0]
    out = np.empty((T, n_v_heads * head_v_dim), np.float32)
    p = lambda x: x.ctypes.data
    check(_native.hip().oi_deltanet_steps(ctypes.byref(d), T, p(qkv), p(z), p(b), p(a), p(conv_w), p(a_decay),
                                          p(dt_bias), p(norm_w), p(cs), p(rs), p(out)))
    return out, cs, rs
