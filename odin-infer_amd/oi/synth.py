"""Seeded synthetic GGUF models (liboi_synth.so) and the configurations they
are measured on.

CONFIGS holds the shapes of the measurement plan (dense Qwen3, Qwen3-MoE and
the Qwen3.5 hybrid) plus small shapes for tests.  Weights: 2-D tensors
N(0, 0.02) from a generator seeded by (seed, tensor name, row); F32 norm
weights 1 + N(0, 0.02); DeltaNet extras: conv1d N(0, 0.25), dt_bias N(0, 0.5),
ssm_a = -exp(N(0, 0.5)).
"""
import ctypes
import os

import numpy as np

from . import _native
from .ggml import GGML_Type as T


def _spec(dim, hidden, layers, heads, kv_heads, head_dim, vocab, ctx, t_default, t_v, t_down, t_embd, t_out,
          seed=1234, sigma=0.02, norm_sigma=0.02, theta=1e6, eps=1e-6, **arch):
    d = dict(dim=dim, hidden_dim=hidden, n_layers=layers, n_heads=heads, n_kv_heads=kv_heads,
             head_dim=head_dim, vocab_size=vocab, context_length=ctx, rope_theta=theta, rms_eps=eps,
             type_default=int(t_default), type_attn_v=int(t_v), type_ffn_down=int(t_down),
             type_embd=int(t_embd), type_output=int(t_out), sigma=sigma, norm_sigma=norm_sigma, seed=seed,
             arch=0, n_experts=0, n_experts_used=0, expert_ffn=0, shared_expert_ffn=0, type_router=int(t_default),
             full_attn_interval=0, rotary_dim=0, lin_n_k_heads=0, lin_n_v_heads=0, lin_head_k_dim=0,
             lin_head_v_dim=0, lin_conv_kernel=0)
    d.update(arch)
    return d


def _moe(dim, layers, heads, kv_heads, vocab, ctx, experts, used, eff, t=T.Q4_K, t_v=T.Q6_K, t_out=T.Q6_K, **kw):
    """Qwen3-MoE (llama.cpp "qwen3moe"): head_dim 128, routed-expert FFN."""
    return _spec(dim, eff, layers, heads, kv_heads, 128, vocab, ctx, t, t_v, t, t, t_out, arch=1, n_experts=experts,
                 n_experts_used=used, expert_ffn=eff, type_router=int(t), **kw)


def _hybrid(dim, hidden, layers, heads, kv_heads, head_dim, vocab, ctx, rotary, lin_k, lin_v, lin_dim, t=T.Q4_K,
            t_out=T.Q6_K, experts=0, used=0, eff=0, shared=0, interval=4, theta=1e7, **kw):
    """Qwen3.5 hybrid ("qwen35"): gated DeltaNet layers, every interval-th layer full
    attention; dense FFN, or routed experts + shared expert when experts > 0."""
    return _spec(dim, hidden if not experts else eff, layers, heads, kv_heads, head_dim, vocab, ctx, t, t, t, t,
                 t_out, theta=theta, arch=2, n_experts=experts, n_experts_used=used, expert_ffn=eff,
                 shared_expert_ffn=shared, type_router=int(t), full_attn_interval=interval, rotary_dim=rotary,
                 lin_n_k_heads=lin_k, lin_n_v_heads=lin_v, lin_head_k_dim=lin_dim, lin_head_v_dim=lin_dim,
                 lin_conv_kernel=4, **kw)


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
    # the older 32-element block types: Q4_0 projections, Q5_1 attn_v, Q5_0 down, Q4_1 embedding
    "tiny-legacy": _spec(256, 768, 2, 4, 2, 128, 2048, 1024, T.Q4_0, T.Q5_1, T.Q5_0, T.Q4_1, T.Q8_0, seed=23),
    # Qwen3-30B-A3B shape: 128 experts top 8, expert inner 768, Q4_K router and experts
    "qwen3-30b-a3b-q4_k": _moe(2048, 48, 32, 4, 151936, 40960, 128, 8, 768),
    # the same per-layer shapes with 4 layers (parity tests)
    "qwen3-30b-a3b-4layer": _moe(2048, 4, 32, 4, 151936, 40960, 128, 8, 768, seed=31),
    "moe-tiny": _moe(256, 2, 4, 2, 2048, 1024, 8, 2, 256, seed=13),
    # Qwen3.5-style hybrid (BASELINE config 5 shapes): 3 DeltaNet layers per full-attention layer,
    # 512 experts top 10 + a shared expert, expert inner 512
    "qwen35-hybrid-moe": _hybrid(2048, 512, 48, 16, 2, 256, 151936, 262144, 64, 16, 32, 128, experts=512,
                                 used=10, eff=512, shared=512),
    "qwen35-hybrid-moe-4layer": _hybrid(2048, 512, 4, 16, 2, 256, 151936, 262144, 64, 16, 32, 128, experts=512,
                                        used=10, eff=512, shared=512, seed=41),
    # two layers of the config 5 shapes (a DeltaNet layer, then a full-attention layer) and of the
    # config 4 shapes: batched prefill parity at full per-layer size
    "qwen35-hybrid-moe-2layer": _hybrid(2048, 512, 2, 16, 2, 256, 151936, 262144, 64, 16, 32, 128, experts=512,
                                        used=10, eff=512, shared=512, interval=2, seed=43),
    "qwen3-30b-a3b-2layer": _moe(2048, 2, 32, 4, 151936, 40960, 128, 8, 768, seed=33),
    # small hybrids for tests: dense FFN (the reference's layout) and routed experts + shared expert
    "qwen35-tiny": _hybrid(256, 512, 4, 4, 2, 128, 2048, 1024, 32, 2, 4, 128, seed=17),
    "qwen35-moe-tiny": _hybrid(256, 256, 4, 4, 2, 256, 2048, 1024, 64, 2, 4, 128, experts=8, used=2, eff=256,
                               shared=256, seed=19),
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
