"""Seeded synthetic GGUF models (liboi_synth.so) and the configurations they
are measured on.

CONFIGS holds the dense-decoder shapes of the measurement plan plus small
shapes for tests.  Weights: 2-D tensors N(0, 0.02) from a generator seeded by
(seed, tensor name, row); F32 norm weights 1 + N(0, 0.02).
"""
import ctypes
import os

import numpy as np

from . import _native
from .ggml import GGML_Type as T


def _spec(dim, hidden, layers, heads, kv_heads, head_dim, vocab, ctx, t_default, t_v, t_down, t_embd, t_out,
          seed=1234, sigma=0.02, norm_sigma=0.02, theta=1e6, eps=1e-6):
    return dict(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv_heads,
                head_dim=head_dim, vocab_size=vocab, context_length=ctx, rope_theta=theta, rms_eps=eps,
                type_default=int(t_default), type_attn_v=int(t_v), type_ffn_down=int(t_down),
                type_embd=int(t_embd), type_output=int(t_out), sigma=sigma, norm_sigma=norm_sigma, seed=seed)


CONFIGS = {
    # Qwen3-0.6B shape, Q8_0 everywhere, tied classifier
    "qwen3-0.6b-q8_0": _spec(1024, 3072, 28, 16, 8, 128, 151936, 40960, T.Q8_0, T.Q8_0, T.Q8_0, T.Q8_0, -1),
    # Qwen3-8B shape, Q4_K_M-style mix: Q6_K attn_v and output
    "qwen3-8b-q4_k_m": _spec(4096, 12288, 36, 32, 8, 128, 151936, 40960, T.Q4_K, T.Q6_K, T.Q4_K, T.Q4_K,
                             T.Q6_K),
    # small shapes for tests
    "tiny-q4_k": _spec(512, 1536, 2, 8, 2, 128, 4096, 1024, T.Q4_K, T.Q6_K, T.Q4_K, T.Q4_K, T.Q6_K, seed=7),
    "tiny-q8_0": _spec(256, 768, 2, 4, 2, 128, 2048, 1024, T.Q8_0, T.Q8_0, T.Q8_0, T.Q8_0, -1, seed=11),
    "tiny-f32": _spec(256, 512, 1, 2, 1, 128, 1024, 512, T.F32, T.F32, T.F32, T.F32, T.F16, seed=3),
    "small-q4_k": _spec(1024, 3072, 4, 16, 4, 128, 8192, 4096, T.Q4_K, T.Q6_K, T.Q4_K, T.Q4_K, T.Q6_K, seed=21),
    # one layer of the Qwen3-8B shape (projection shapes of the batched prefill at full size)
    "8b-1layer-q4_k": _spec(4096, 12288, 1, 32, 8, 128, 4096, 4096, T.Q4_K, T.Q6_K, T.Q4_K, T.Q4_K, T.Q6_K, seed=5),
}


def write_gguf(path, config, n_threads=None, **overrides):
    """Write the synthetic GGUF for `config` (a CONFIGS key or a dict)."""
    spec = dict(CONFIGS[config]) if isinstance(config, str) else dict(config)
    spec.update(overrides)
    s = _native.SynthSpec(**spec, n_threads=n_threads or min(16, os.cpu_count() or 1))
    rc = _native.synth().oi_synth_write_gguf(str(path).encode(), ctypes.byref(s))
    if rc != 0:
        raise RuntimeError("oi_synth_write_gguf failed (%d) for %s" % (rc, path))
    return spec


def quantize_rows(kind, x):
    """float32 [rows, cols] -> GGUF blocks (uint8) of `kind`."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    rows, cols = x.shape
    e, b = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
            12: (256, 144), 14: (256, 210)}[int(kind)]
    out = np.empty(rows * (cols // e) * b, np.uint8)
    rc = _native.synth().oi_quantize_rows(int(kind), x.ctypes.data, rows, cols, out.ctypes.data)
    if rc != 0:
        raise RuntimeError("oi_quantize_rows failed")
    return out


def normal_f16(seed, n, scale=1.0, n_threads=None):
    out = np.empty(n, np.uint16)
    _native.synth().oi_synth_normal_f16(seed, n, scale, out.ctypes.data, n_threads or min(16, os.cpu_count() or 1))
    return out


def normal_f32(seed, n, scale=1.0, n_threads=None):
    out = np.empty(n, np.float32)
    _native.synth().oi_synth_normal_f32(seed, n, scale, out.ctypes.data, n_threads or min(16, os.cpu_count() or 1))
    return out


def tensor_f32(seed, name, rows, cols, sigma=0.02, mean=0.0, n_threads=None):
    out = np.empty((rows, cols), np.float32)
    _native.synth().oi_synth_tensor_f32(seed, name.encode(), rows, cols, sigma, mean, out.ctypes.data,
                                        n_threads or min(16, os.cpu_count() or 1))
    return out


def kv_prefill(seed, n_layers, n_kv_heads, npos, head_dim, n_threads=None):
    """f16 K and V, N(0,1), [n_layers][n_kv_heads][npos][head_dim] (binary16 bits)."""
    n = n_layers * n_kv_heads * npos * head_dim
    k = normal_f16(seed, n, 1.0, n_threads).reshape(n_layers, n_kv_heads, npos, head_dim)
    v = normal_f16(seed + 1, n, 1.0, n_threads).reshape(n_layers, n_kv_heads, npos, head_dim)
    return k, v
