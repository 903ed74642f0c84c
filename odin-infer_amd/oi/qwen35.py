"""Qwen3.5 hybrid-decoder pieces on the device: the gated DeltaNet token step
of a linear-attention layer (qwen3_5/forward.odin:137-225) and the attention
of a full-attention layer (qwen3_5/forward.odin:46-135)."""
import ctypes

import numpy as np

from . import _native
from ._native import check


LAYER_FULL_ATTENTION, LAYER_LINEAR_ATTENTION = 0, 1  # qwen3_5/model.odin:18 Layer_Type


def engine_config(e):
    """The qwen3_5 package's engine_config (qwen3_5/engine.odin:104-106 ->
    Config, qwen3_5/model.odin:20-45): a dict of its fields in order,
    layer_types included (0 full attention, 1 gated DeltaNet)."""
    L = _native.hip()
    c = _native.Qwen35Config()
    check(L.oi_engine_config_qwen35(e.handle, ctypes.byref(c)))
    out = {name: getattr(c, name) for name, _ in c._fields_}
    types = np.empty(int(c.n_layers), np.int32)
    check(L.oi_engine_layer_types(e.handle, types.ctypes.data, int(c.n_layers)))
    keys = list(out)
    at = keys.index("full_attn_interval") + 1
    ordered = {k: out[k] for k in keys[:at]}
    ordered["layer_types"] = [int(t) for t in types]
    ordered.update({k: out[k] for k in keys[at:]})
    return ordered


def engine_batch_max():
    """qwen3_5/engine.odin:96-102: tokens per batched chunk (qwen3_5/metal.odin:22)."""
    return int(_native.hip().oi_engine_batch_max())


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


def deltanet_steps_batched(n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel, eps, chunk, qkv, z, b, a,
                           conv_w, a_decay, dt_bias, norm_w, conv_state, rec_state):
    """The same trajectory through oi_deltanet_steps_batched, the batched
    prefill kernels: the delta rule token by token (chunk 0) or in its
    chunked form over chunks of 16 / 32 / 64 tokens.  Returns (out, conv_state,
    rec_state) as deltanet_steps."""
    d = _native.DeltaNetDims(n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel, eps)
    qkv, z, b, a = _f32(np.atleast_2d(qkv)), _f32(np.atleast_2d(z)), _f32(np.atleast_2d(b)), _f32(np.atleast_2d(a))
    conv_w, a_decay, dt_bias, norm_w = _f32(conv_w), _f32(a_decay), _f32(dt_bias), _f32(norm_w)
    cs, rs = _f32(conv_state).copy(), _f32(rec_state).copy()
    T = qkv.shape[0]
    out = np.empty((T, n_v_heads * head_v_dim), np.float32)
    p = lambda x: x.ctypes.data
    check(_native.hip().oi_deltanet_steps_batched(ctypes.byref(d), T, int(chunk), p(qkv), p(z), p(b), p(a),
                                                  p(conv_w), p(a_decay), p(dt_bias), p(norm_w), p(cs), p(rs),
                                                  p(out)))
    return out, cs, rs


def attn_steps(n_heads, n_kv_heads, head_dim, rotary_dim, seq_len, eps, pos0, qproj, k, v, q_norm, k_norm, inv_freq,
               k_cache16, v_cache16):
    """Run len(qproj) tokens from pos0 through oi_qwen35_attn_steps.  qproj
    [T, n_heads*2*head_dim] ([q | gate] per head), k, v [T, n_kv*head_dim];
    caches uint16 f16 bits [n_kv, seq_len, head_dim].  Returns (out [T,
    n_heads*head_dim], k_cache16, v_cache16) (copies)."""
    d = _native.Qwen35AttnDims(n_heads, n_kv_heads, head_dim, rotary_dim, seq_len, eps)
    qproj, k, v = _f32(np.atleast_2d(qproj)), _f32(np.atleast_2d(k)), _f32(np.atleast_2d(v))
    q_norm, k_norm, inv_freq = _f32(q_norm), _f32(k_norm), _f32(inv_freq)
    kc = np.ascontiguousarray(k_cache16, np.uint16).copy()
    vc = np.ascontiguousarray(v_cache16, np.uint16).copy()
    T = qproj.shape[0]
    out = np.empty((T, n_heads * head_dim), np.float32)
    p = lambda x: x.ctypes.data
    check(_native.hip().oi_qwen35_attn_steps(ctypes.byref(d), T, int(pos0), p(qproj), p(k), p(v), p(q_norm),
                                             p(k_norm), p(inv_freq), p(kc), p(vc), p(out)))
    return out, kc, vc
