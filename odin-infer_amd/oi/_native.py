"""Loading of the native libraries built in-tree (odin-infer_amd/build.py)."""
import ctypes
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_HIP = os.path.join(PKG, "liboi_hip.so")
LIB_SYNTH = os.path.join(PKG, "liboi_synth.so")

_hip = None
_synth = None

c_i32, c_i64, c_vp, c_f, c_d = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_double


class OIError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("oi error %d: %s" % (code, msg))
        self.code = code


class DeltaNetDims(ctypes.Structure):
    _fields_ = [("n_k_heads", c_i32), ("n_v_heads", c_i32), ("head_k_dim", c_i32), ("head_v_dim", c_i32),
                ("conv_kernel", c_i32), ("eps", c_f)]


class Qwen35AttnDims(ctypes.Structure):
    _fields_ = [("n_heads", c_i32), ("n_kv_heads", c_i32), ("head_dim", c_i32), ("rotary_dim", c_i32),
                ("seq_len", c_i32), ("eps", c_f)]


class MoeDims(ctypes.Structure):
    _fields_ = [("n_experts", c_i32), ("top_k", c_i32), ("dim", c_i32), ("inter", c_i32), ("norm_topk_prob", c_i32)]


class Opts(ctypes.Structure):
    _fields_ = [("max_ctx", c_i32), ("use_hip", c_i32), ("num_threads", c_i32), ("device", c_i32)]


class Config(ctypes.Structure):
    _fields_ = [("dim", c_i64), ("hidden_dim", c_i64), ("n_layers", c_i64), ("n_heads", c_i64),
                ("n_kv_heads", c_i64), ("vocab_size", c_i64), ("seq_len", c_i64), ("max_seq", c_i64),
                ("head_dim", c_i64), ("rope_freq", c_f), ("rms_eps", c_f)]


class Qwen35Config(ctypes.Structure):
    """oi_qwen35_config: qwen3_5/model.odin:20-45 without layer_types."""
    _fields_ = [("dim", c_i64), ("hidden_dim", c_i64), ("n_layers", c_i64), ("n_heads", c_i64),
                ("n_kv_heads", c_i64), ("head_dim", c_i64), ("vocab_size", c_i64), ("seq_len", c_i64),
                ("max_seq", c_i64), ("rms_eps", c_f), ("rope_theta", c_f), ("partial_rotary", c_f),
                ("rotary_dim", c_i64), ("lin_n_k_heads", c_i64), ("lin_n_v_heads", c_i64),
                ("lin_head_k_dim", c_i64), ("lin_head_v_dim", c_i64), ("lin_conv_kernel", c_i64),
                ("full_attn_interval", c_i64), ("n_full", c_i64), ("n_linear", c_i64)]


class Sampler(ctypes.Structure):
    """oi_sampler (include/oi.h): sampler/sampler.odin:16-29 without the grammar."""
    _fields_ = [("temperature", c_f), ("topp", c_f), ("repeat_penalty", c_f), ("record", c_i32),
                ("rng_state", ctypes.c_uint64), ("n_last", c_i32), ("last", c_i32 * 64)]


# every symbol include/oi.h declares, with (restype, argtypes)
HIP_SYMBOLS = {
    "oi_engine_load": (c_i32, [ctypes.c_char_p, ctypes.POINTER(Opts), ctypes.POINTER(c_vp)]),
    "oi_engine_destroy": (None, [c_vp]),
    "oi_engine_forward": (ctypes.POINTER(c_f), [c_vp, c_i32, c_i32]),
    "oi_engine_prefill": (ctypes.POINTER(c_f), [c_vp, c_vp, c_i32, c_i32]),
    "oi_engine_config": (c_i32, [c_vp, ctypes.POINTER(Config)]),
    "oi_engine_verify_batch": (ctypes.POINTER(c_f), [c_vp, c_vp, c_i32, c_i32]),
    "oi_engine_config_qwen35": (c_i32, [c_vp, ctypes.POINTER(Qwen35Config)]),
    "oi_engine_layer_types": (c_i32, [c_vp, c_vp, c_i32]),
    "oi_engine_batch_max": (c_i32, []),
    "oi_last_error": (ctypes.c_char_p, []),
    "oi_engine_decode_greedy": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp]),
    "oi_engine_kv_fill": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "oi_engine_reset_state": (c_i32, [c_vp]),
    "oi_engine_decode_sample": (c_i32, [c_vp, c_i32, c_i32, c_i32, ctypes.POINTER(Sampler), c_vp]),
    "oi_sample": (c_i32, [c_vp, c_i32, ctypes.POINTER(Sampler), ctypes.POINTER(c_i32)]),
    "oi_engine_save_kv": (c_i32, [c_vp, ctypes.c_char_p, c_i32]),
    "oi_engine_load_kv": (c_i32, [c_vp, ctypes.c_char_p, c_vp]),
    "oi_engine_state_sizes": (c_i32, [c_vp, c_vp]),
    "oi_engine_save_full_state": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp]),
    "oi_engine_restore_full_state": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp]),
    "oi_engine_save_spec_state": (c_i32, [c_vp, c_vp, c_vp]),
    "oi_engine_restore_spec_state": (c_i32, [c_vp, c_vp, c_vp]),
    "oi_engine_logits_device": (c_vp, [c_vp]),
    "oi_engine_stream": (c_vp, [c_vp]),
    "oi_engine_time_kernel": (c_i32, [c_vp, c_i32, c_i32, ctypes.POINTER(c_d), ctypes.POINTER(c_d)]),
    "oi_dequant": (c_i32, [c_i32, c_vp, c_i64, c_vp]),
    "oi_weights_upload": (c_i32, [c_i32, c_vp, c_i64, c_i64, ctypes.POINTER(c_vp)]),
    "oi_weights_free": (None, [c_vp]),
    "oi_weights_bytes": (c_i64, [c_vp]),
    "oi_gemv_launch": (c_i32, [c_vp, c_vp, c_vp, c_vp]),
    "oi_gemv": (c_i32, [c_i32, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "oi_gemm_workspace_bytes": (c_i64, [c_vp, c_i32]),
    "oi_gemm_launch": (c_i32, [c_vp, c_vp, c_i32, c_vp, c_vp, c_i64, c_vp]),
    "oi_gemm": (c_i32, [c_i32, c_vp, c_i64, c_i64, c_vp, c_i32, c_vp]),
    "oi_deltanet_step_launch": (c_i32, [c_vp] * 13 + [c_vp]),
    "oi_deltanet_steps": (c_i32, [c_vp, c_i32] + [c_vp] * 11),
    "oi_deltanet_steps_batched": (c_i32, [c_vp, c_i32, c_i32] + [c_vp] * 11),
    "oi_qwen35_attn_workspace_bytes": (c_i64, [c_vp]),
    "oi_qwen35_attn_step_launch": (c_i32, [c_vp, c_i32] + [c_vp] * 11),
    "oi_qwen35_attn_steps": (c_i32, [c_vp, c_i32, c_i32] + [c_vp] * 9),
    "oi_moe_workspace_bytes": (c_i64, [c_vp]),
    "oi_moe_ffn_launch": (c_i32, [c_vp] * 9),
    "oi_moe_ffn_launch_noalloc": (c_i32, [c_vp] * 8),
    "oi_moe_ffn": (c_i32, [c_vp, c_i32, c_vp, c_i32] + [c_vp] * 7),
}


class SynthSpec(ctypes.Structure):
    _fields_ = [("dim", c_i64), ("hidden_dim", c_i64), ("n_layers", c_i64), ("n_heads", c_i64),
                ("n_kv_heads", c_i64), ("head_dim", c_i64), ("vocab_size", c_i64), ("context_length", c_i64),
                ("rope_theta", c_f), ("rms_eps", c_f), ("type_default", c_i32), ("type_attn_v", c_i32),
                ("type_ffn_down", c_i32), ("type_embd", c_i32), ("type_output", c_i32), ("sigma", c_f),
                ("norm_sigma", c_f), ("seed", ctypes.c_uint64), ("n_threads", c_i32),
                ("arch", c_i32), ("n_experts", c_i32), ("n_experts_used", c_i32), ("expert_ffn", c_i32),
                ("shared_expert_ffn", c_i32), ("type_router", c_i32), ("full_attn_interval", c_i32),
                ("rotary_dim", c_i32), ("lin_n_k_heads", c_i32), ("lin_n_v_heads", c_i32),
                ("lin_head_k_dim", c_i32), ("lin_head_v_dim", c_i32), ("lin_conv_kernel", c_i32)]


SYNTH_SYMBOLS = {
    "oi_synth_write_gguf": (c_i32, [ctypes.c_char_p, ctypes.POINTER(SynthSpec)]),
    "oi_quantize_rows": (c_i32, [c_i32, c_vp, c_i64, c_i64, c_vp]),
    "oi_synth_normal_f32": (None, [ctypes.c_uint64, c_i64, c_f, c_vp, c_i32]),
    "oi_synth_normal_f16": (None, [ctypes.c_uint64, c_i64, c_f, c_vp, c_i32]),
    "oi_synth_tensor_f32": (None, [ctypes.c_uint64, ctypes.c_char_p, c_i64, c_i64, c_f, c_f, c_vp, c_i32]),
}


def _bind(path, symbols):
    if not os.path.exists(path):
        raise OIError(-7, "native library %s is not built (run odin-infer_amd/build.py)" % path)
    L = ctypes.CDLL(path)
    for name, (res, args) in symbols.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def hip():
    global _hip
    if _hip is None:
        _hip = _bind(LIB_HIP, HIP_SYMBOLS)
    return _hip


def synth():
    global _synth
    if _synth is None:
        _synth = _bind(LIB_SYNTH, SYNTH_SYMBOLS)
    return _synth


def check(rc):
    if rc != 0:
        raise OIError(rc, hip().oi_last_error().decode())
    return rc
