"""ctypes wrapper of the CPU oracle (oracle/refcpu.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librefcpu.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        c_i64, c_int, c_vp, c_f = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
        L.ref_last_error.restype = ctypes.c_char_p
        L.ref_row_byte_size.restype = c_i64
        L.ref_row_byte_size.argtypes = [c_int, c_i64]
        L.ref_block_info.argtypes = [c_int, c_vp, c_vp]
        L.ref_is_supported_quant.argtypes = [c_int]
        L.ref_f16_to_f32.restype = c_f
        L.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ref_f32_to_f16.restype = ctypes.c_uint16
        L.ref_f32_to_f16.argtypes = [c_f]
        L.ref_get_scale_min_k4.argtypes = [c_int, c_vp, c_vp, c_vp]
        L.ref_dequant_row.argtypes = [c_int, c_vp, c_i64, c_vp]
        L.ref_dot_f32.restype = c_f
        L.ref_dot_f32.argtypes = [c_vp, c_vp, c_i64]
        L.ref_set_dot_order.argtypes = [c_int]
        L.ref_matmul_t.argtypes = [c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_int]
        L.ref_rmsnorm.argtypes = [c_vp, c_vp, c_vp, c_i64, c_f]
        L.ref_softmax.argtypes = [c_vp, c_i64]
        L.ref_argmax.restype = c_i64
        L.ref_argmax.argtypes = [c_vp, c_i64]
        L.ref_engine_load.restype = c_vp
        L.ref_engine_load.argtypes = [ctypes.c_char_p, c_int, c_int, c_int]
        L.ref_engine_forward.restype = ctypes.POINTER(c_f)
        L.ref_engine_forward.argtypes = [c_vp, c_int, c_int]
        L.ref_engine_prefill.restype = ctypes.POINTER(c_f)
        L.ref_engine_prefill.argtypes = [c_vp, c_vp, c_int, c_int]
        L.ref_engine_verify_batch.restype = ctypes.POINTER(c_f)
        L.ref_engine_route_log.argtypes = [c_vp, c_int]
        L.ref_engine_route_margins.restype = ctypes.POINTER(c_f)
        L.ref_engine_route_margins.argtypes = [c_vp]
        L.ref_engine_verify_batch.argtypes = [c_vp, c_vp, c_int, c_int]
        L.ref_engine_destroy.argtypes = [c_vp]
        L.ref_engine_config.argtypes = [c_vp, c_vp, c_vp]
        L.ref_engine_kv_fill.argtypes = [c_vp, c_int, c_int, c_int, c_vp, c_vp]
        L.ref_engine_hidden.restype = ctypes.POINTER(c_f)
        L.ref_engine_hidden.argtypes = [c_vp]
        L.ref_gemm_f16.argtypes = [c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_vp]
        L.ref_delta_step.argtypes = [c_vp, c_vp, c_vp, c_vp, c_vp, c_f, c_f, c_int, c_int]
        L.ref_conv1d.argtypes = [c_vp, c_vp, c_vp, c_vp, c_i64, c_int]
        L.ref_l2norm_into.argtypes = [c_vp, c_vp, c_i64, c_f]
        L.ref_deltanet_steps.argtypes = [c_int] * 5 + [c_f, c_int] + [c_vp] * 11
        L.ref_delta_chunk.argtypes = [c_vp] * 7 + [c_int] * 3
        L.ref_deltanet_steps_chunked.argtypes = [c_int] * 5 + [c_f, c_int, c_int] + [c_vp] * 11
        L.ref_inv_freq.argtypes = [c_f, c_int, c_vp]
        L.ref_mrope.argtypes = [c_vp, c_int, c_vp, c_int]
        L.ref_qwen35_attn_steps.argtypes = [c_int] * 5 + [c_f, c_int, c_int] + [c_vp] * 9
        L.ref_moe_ffn.argtypes = [c_int] * 6 + [c_vp, c_int] + [c_vp] * 7
        L.ref_engine_reset_state.argtypes = [c_vp]
        L.ref_random_f32.restype = c_f
        L.ref_random_f32.argtypes = [c_vp]
        L.ref_sample.restype = c_i64
        L.ref_sample.argtypes = [c_vp, c_i64, c_f, c_f, c_f, c_vp, c_int, c_vp]
        L.ref_record_token.argtypes = [c_vp, c_vp, ctypes.c_int32, c_f]
        L.ref_engine_save_kv.argtypes = [c_vp, ctypes.c_char_p, c_int]
        L.ref_engine_load_kv.argtypes = [c_vp, ctypes.c_char_p]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data


def row_byte_size(kind, n):
    return lib().ref_row_byte_size(kind, n)


def dequant_row(kind, blocks, n):
    out = np.empty(n, np.float32)
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    lib().ref_dequant_row(kind, _p(src), n, _p(out))
    return out


def dot_f32(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().ref_dot_f32(_p(a), _p(b), len(a))


def set_dot_order(order):
    """0: the reference's summation order in dot_f32; 1: the same 16-element
    steps taken from the end of the row (a second valid f32 evaluation, used
    to measure the oracle's own rounding noise)."""
    lib().ref_set_dot_order(int(order))


def matmul_t(w_blocks, kind, x, d, nthreads=1):
    """xout[d] = W[d, n] . x[n] (infer/matmul.odin:77-109)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_blocks, np.uint8)
    out = np.empty(d, np.float32)
    rc = lib().ref_matmul_t(_p(out), _p(x), kind, _p(w), len(x), d, nthreads)
    if rc:
        raise RuntimeError(lib().ref_last_error().decode())
    return out


def gemm_f16(w_blocks, kind, m, k, x16):
    """C[t][r] = sum_j f16(dequant(W)[r][j]) * x16[t][j] in float64 (x16: uint16 [n][k])."""
    w = np.ascontiguousarray(np.frombuffer(bytes(w_blocks), np.uint8) if not isinstance(w_blocks, np.ndarray)
                             else w_blocks.view(np.uint8))
    x = np.ascontiguousarray(x16, np.uint16)
    n = x.shape[0]
    out = np.zeros((n, m), np.float64)
    if lib().ref_gemm_f16(kind, _p(w), m, k, _p(x), n, _p(out)) != 0:
        raise RuntimeError(lib().ref_last_error().decode())
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    o = np.empty_like(x)
    lib().ref_rmsnorm(_p(o), _p(x), _p(w), len(x), eps)
    return o


def softmax(x):
    x = np.array(x, np.float32)
    lib().ref_softmax(_p(x), len(x))
    return x


def argmax(p):
    p = np.ascontiguousarray(p, np.float32)
    return int(lib().ref_argmax(_p(p), len(p)))


def get_scale_min_k4(j, q12):
    q = np.ascontiguousarray(q12, np.uint8)
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().ref_get_scale_min_k4(j, _p(q), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def random_f32(rng_state):
    """random_f32 (sampler/sampler.odin:75-77): (value, advanced state)."""
    st = ctypes.c_uint64(rng_state)
    v = lib().ref_random_f32(ctypes.byref(st))
    return v, st.value


def sample(logits, temperature, topp, penalty=1.0, last=(), rng_state=0):
    """sampler.sample (sampler/sampler.odin:141-199, no grammar) on a copy of
    logits: (index, advanced rng state)."""
    x = np.array(logits, np.float32, copy=True)
    lt = np.ascontiguousarray(last, np.int32)
    st = ctypes.c_uint64(rng_state)
    i = lib().ref_sample(_p(x), x.size, float(temperature), float(topp), float(penalty), _p(lt) if lt.size else None,
                         int(lt.size), ctypes.byref(st))
    return int(i), st.value


def record_token(last, token, penalty):
    """record_token (sampler.odin:50-56), window 64: the new window."""
    buf = np.zeros(65, np.int32)
    buf[:len(last)] = last
    n = ctypes.c_int(len(last))
    lib().ref_record_token(_p(buf), ctypes.byref(n), int(token), float(penalty))
    return [int(t) for t in buf[:n.value]]


class RefEngine:
    """The reference CPU forward (infer/engine.odin + infer/forward.odin).

    kv_f16=True rounds K/V to binary16 on store, as the reference GPU path's
    f16 cache does (infer/metal.odin:443-454)."""

    def __init__(self, path, max_ctx=4096, num_threads=1, kv_f16=False):
        self.h = lib().ref_engine_load(path.encode(), max_ctx, num_threads, int(kv_f16))
        if not self.h:
            raise RuntimeError("oracle load failed: " + lib().ref_last_error().decode())
        ints = (ctypes.c_int64 * 9)()
        fl = (ctypes.c_float * 2)()
        lib().ref_engine_config(self.h, ints, fl)
        (self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads, self.vocab_size,
         self.seq_len, self.max_seq, self.head_dim) = list(ints)
        self.rope_freq, self.rms_eps = fl[0], fl[1]

    def forward(self, token, pos):
        p = lib().ref_engine_forward(self.h, token, pos)
        if not p:
            raise RuntimeError(lib().ref_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.vocab_size,)).copy()

    def prefill(self, tokens, pos0):
        """engine_forward_batch: the last token's logits (batched chunks with
        f16-staged projections, trailing tokens per token)."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = lib().ref_engine_prefill(self.h, _p(t), int(t.size), int(pos0))
        if not p:
            raise RuntimeError(lib().ref_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(self.vocab_size,)).copy()

    def verify_batch(self, tokens, pos0):
        """engine_verify_batch: the prefill path over `tokens` with every
        position's logits kept, [n][vocab]."""
        t = np.ascontiguousarray(tokens, np.int32)
        p = lib().ref_engine_verify_batch(self.h, _p(t), int(t.size), int(pos0))
        if not p:
            raise RuntimeError(lib().ref_last_error().decode())
        return np.ctypeslib.as_array(p, shape=(int(t.size), self.vocab_size)).copy()

    def route_log(self, on=True):
        """Start (all NaN) or stop recording routing boundary margins."""
        if lib().ref_engine_route_log(self.h, int(bool(on))):
            raise MemoryError("route log")

    def route_margins(self):
        """[seq_len][n_layers]: log(p_k / p_k+1) between the k-th chosen and
        the best unchosen expert of each (position, layer) forwarded while
        recording (NaN elsewhere)."""
        p = lib().ref_engine_route_margins(self.h)
        if not p:
            raise RuntimeError("route log is off")
        return np.ctypeslib.as_array(p, shape=(self.seq_len, self.n_layers)).copy()

    def kv_fill(self, layer, pos0, k16, v16):
        """k16, v16: uint16 [n_kv_heads][npos][head_dim] for one layer."""
        k16 = np.ascontiguousarray(k16, np.uint16)
        v16 = np.ascontiguousarray(v16, np.uint16)
        npos = k16.shape[1]
        rc = lib().ref_engine_kv_fill(self.h, layer, pos0, npos, _p(k16), _p(v16))
        if rc:
            raise RuntimeError(lib().ref_last_error().decode())

    def reset_state(self):
        """engine_reset_state (qwen3_5/engine.odin:112-132)."""
        lib().ref_engine_reset_state(self.h)

    def save_kv(self, path, n_valid_pos):
        """cpu_save_kv (qwen3_5/kv_persist.odin:218-265); raises on failure."""
        if lib().ref_engine_save_kv(self.h, str(path).encode(), int(n_valid_pos)) != 0:
            raise RuntimeError(lib().ref_last_error().decode())

    def load_kv(self, path):
        """cpu_load_kv (kv_persist.odin:267-336): the restored n_valid_pos;
        raises RuntimeError with the reference's message on a refused file."""
        n = lib().ref_engine_load_kv(self.h, str(path).encode())
        if n < 0:
            raise RuntimeError(lib().ref_last_error().decode())
        return n

    def close(self):
        if self.h:
            lib().ref_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def delta_step(state, q, k, v, beta, decay):
    """qwen3_5/ops.odin:120-153 on a copy of state [hk][hv]; returns (out, state)."""
    st = np.ascontiguousarray(state, np.float32).copy()
    hk, hv = st.shape
    q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
    out = np.empty(hv, np.float32)
    lib().ref_delta_step(_p(out), _p(st), _p(q), _p(k), _p(v), float(beta), float(decay), hk, hv)
    return out, st


def conv1d(x, state, w, kernel):
    """qwen3_5/ops.odin:97-117; returns (out, new state)."""
    x = np.ascontiguousarray(x, np.float32)
    st = np.ascontiguousarray(state, np.float32).copy()
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().ref_conv1d(_p(out), _p(x), _p(st), _p(w), x.size, kernel)
    return out, st


def l2norm(x, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    o = np.empty_like(x)
    lib().ref_l2norm_into(_p(o), _p(x), x.size, eps)
    return o


def deltanet_steps(n_kh, n_vh, hk, hv, kernel, eps, qkv, z, b, a, conv_w, a_decay, dt_bias, norm_w, conv_state,
                   rec_state):
    """forward_linear_layer from the projections to the gated RMSNorm over
    len(qkv) tokens; returns (out [T, n_vh*hv], conv_state, rec_state)."""
    f = lambda x: np.ascontiguousarray(x, np.float32)
    qkv, z, b, a = f(np.atleast_2d(qkv)), f(np.atleast_2d(z)), f(np.atleast_2d(b)), f(np.atleast_2d(a))
    conv_w, a_decay, dt_bias, norm_w = f(conv_w), f(a_decay), f(dt_bias), f(norm_w)
    cs, rs = f(conv_state).copy(), f(rec_state).copy()
    T = qkv.shape[0]
    out = np.empty((T, n_vh * hv), np.float32)
    rc = lib().ref_deltanet_steps(n_kh, n_vh, hk, hv, kernel, float(eps), T, _p(qkv), _p(z), _p(b), _p(a),
                                  _p(conv_w), _p(a_decay), _p(dt_bias), _p(norm_w), _p(cs), _p(rs), _p(out))
    if rc:
        raise RuntimeError(lib().ref_last_error().decode())
    return out, cs, rs


def delta_chunk(state, q, k, v, beta, g):
    """ref_delta_chunk: the chunked delta rule (qwen3_5/metal.odin:416-468) for
    one value head over C tokens; returns (out [C, hv], new state [hk, hv])."""
    f = lambda x: np.ascontiguousarray(x, np.float32)
    st = f(state).copy()
    q, k, v, beta, g = f(q), f(k), f(v), f(beta), f(g)
    C, hk = k.shape
    hv = v.shape[1]
    out = np.empty((C, hv), np.float32)
    lib().ref_delta_chunk(_p(out), _p(st), _p(q), _p(k), _p(v), _p(beta), _p(g), C, hk, hv)
    return out, st


def deltanet_steps_chunked(n_kh, n_vh, hk, hv, kernel, eps, chunk, qkv, z, b, a, conv_w, a_decay, dt_bias, norm_w,
                           conv_state, rec_state):
    """deltanet_steps with the delta rule in chunks of `chunk` tokens
    (ref_deltanet_steps_chunked); returns (out, conv_state, rec_state)."""
    f = lambda x: np.ascontiguousarray(x, np.float32)
    qkv, z, b, a = f(np.atleast_2d(qkv)), f(np.atleast_2d(z)), f(np.atleast_2d(b)), f(np.atleast_2d(a))
    conv_w, a_decay, dt_bias, norm_w = f(conv_w), f(a_decay), f(dt_bias), f(norm_w)
    cs, rs = f(conv_state).copy(), f(rec_state).copy()
    T = qkv.shape[0]
    out = np.empty((T, n_vh * hv), np.float32)
    rc = lib().ref_deltanet_steps_chunked(n_kh, n_vh, hk, hv, kernel, float(eps), T, int(chunk), _p(qkv), _p(z),
                                          _p(b), _p(a), _p(conv_w), _p(a_decay), _p(dt_bias), _p(norm_w), _p(cs),
                                          _p(rs), _p(out))
    if rc:
        raise RuntimeError(lib().ref_last_error().decode())
    return out, cs, rs


def inv_freq(theta, rotary_dim):
    out = np.empty(rotary_dim // 2, np.float32)
    lib().ref_inv_freq(float(theta), rotary_dim, _p(out))
    return out


def mrope(v, pos, inv_f, rotary_dim):
    v = np.ascontiguousarray(v, np.float32).copy()
    lib().ref_mrope(_p(v), int(pos), _p(np.ascontiguousarray(inv_f, np.float32)), rotary_dim)
    return v


def qwen35_attn_steps(n_heads, n_kv, hd, rotary_dim, seq_len, eps, pos0, qproj, k, v, q_norm, k_norm, inv_f,
                      kc16, vc16):
    """forward_full_layer's attention over len(qproj) tokens from pos0;
    returns (out [T, n_heads*hd], kc16, vc16)."""
    f = lambda x: np.ascontiguousarray(x, np.float32)
    qproj, k, v = f(np.atleast_2d(qproj)), f(np.atleast_2d(k)), f(np.atleast_2d(v))
    kc = np.ascontiguousarray(kc16, np.uint16).copy()
    vc = np.ascontiguousarray(vc16, np.uint16).copy()
    T = qproj.shape[0]
    out = np.empty((T, n_heads * hd), np.float32)
    rc = lib().ref_qwen35_attn_steps(n_heads, n_kv, hd, rotary_dim, seq_len, float(eps), T, int(pos0), _p(qproj),
                                     _p(k), _p(v), _p(f(q_norm)), _p(f(k_norm)), _p(f(inv_f)), _p(kc), _p(vc),
                                     _p(out))
    if rc:
        raise RuntimeError(lib().ref_last_error().decode())
    return out, kc, vc


def moe_ffn(E, top_k, dim, inter, norm, rtype, router, etype, gate, up, down, x):
    """Routed-expert FFN for one token; returns (y, ids, weights)."""
    b = lambda a: np.ascontiguousarray(a, np.uint8)
    router, gate, up, down = b(router), b(gate), b(up), b(down)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(dim, np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    rc = lib().ref_moe_ffn(E, top_k, dim, inter, int(norm), rtype, _p(router), etype, _p(gate), _p(up), _p(down),
                           _p(x), _p(y), _p(ids), _p(w))
    if rc:
        raise RuntimeError(lib().ref_last_error().decode())
    return y, ids, w
