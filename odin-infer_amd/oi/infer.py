"""Engine API, mirroring the reference's `infer` package (infer/engine.odin:7-60).

    e, ok = engine_load(path, Engine_Opts(max_ctx=4096, use_hip=True))
    logits = engine_forward(e, token, pos)   # numpy view of engine memory
    engine_destroy(e)

Same names, argument meaning and error behaviour as the reference: the
returned logits alias engine-owned memory valid until the next call
(infer/forward.odin:145); an out-of-range token or pos is fatal in the reference
(infer/forward.odin:22-29) and raises OIError(OI_E_RANGE) here.  The reference's
silent CPU fallback when the GPU is missing (infer/engine.odin:23-31) is not
reproduced: engine_load raises instead.
"""
import ctypes
import sys
from dataclasses import dataclass

import numpy as np

from . import _native
from ._native import OIError, check

OI_E_RANGE = -6
KERNELS = {"qkv": 0, "attn": 1, "wo": 2, "gateup": 3, "down": 4, "output": 5, "token": 6, "router": 7,
           "linear_in": 8, "deltanet": 9, "linear_out": 10, "shared": 11}


@dataclass
class Engine_Opts:
    max_ctx: int = 4096
    use_hip: bool = True
    num_threads: int = 1
    device: int = 0


@dataclass
class Config:
    """infer/model.odin:12-24, same fields and order."""
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    seq_len: int
    max_seq: int
    head_dim: int
    rope_freq: float
    rms_eps: float


class Engine:
    def __init__(self, handle, config):
        self._h = handle
        self.config = config
        self.hip_ready = True

    @property
    def handle(self):
        if not self._h:
            raise OIError(-1, "engine destroyed")
        return self._h


def engine_load(path, opts=None):
    """infer/engine.odin:18-34. Returns (Engine, True); raises OIError."""
    opts = opts or Engine_Opts()
    L = _native.hip()
    o = _native.Opts(int(opts.max_ctx), int(bool(opts.use_hip)), int(opts.num_threads), int(opts.device))
    h = ctypes.c_void_p()
    check(L.oi_engine_load(str(path).encode(), ctypes.byref(o), ctypes.byref(h)))
    c = _native.Config()
    check(L.oi_engine_config(h, ctypes.byref(c)))
    cfg = Config(c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.seq_len, c.max_seq,
                 c.head_dim, c.rope_freq, c.rms_eps)
    return Engine(h.value, cfg), True


def engine_destroy(e):
    """infer/engine.odin:36-43."""
    if e._h:
        _native.hip().oi_engine_destroy(e._h)
        e._h = None


def engine_forward(e, token, pos):
    """infer/engine.odin:45-52: logits for `token` at `pos` (predicting pos+1)."""
    p = _native.hip().oi_engine_forward(e.handle, int(token), int(pos))
    if not p:
        L = _native.hip()
        raise OIError(OI_E_RANGE if "out of range" in L.oi_last_error().decode() else -7,
                      L.oi_last_error().decode())
    return np.ctypeslib.as_array(p, shape=(e.config.vocab_size,))


def engine_forward_batch(e, tokens, pos_start):
    """qwen3_5/engine.odin:61-93: consume `tokens` from `pos_start` (batched
    chunks of a multiple of 8, up to 512; the trailing 1-7 one at a time);
    returns the last token's logits (a view of engine memory)."""
    t = np.ascontiguousarray(tokens, np.int32)
    p = _native.hip().oi_engine_prefill(e.handle, t.ctypes.data, int(t.size), int(pos_start))
    if not p:
        L = _native.hip()
        msg = L.oi_last_error().decode()
        raise OIError(OI_E_RANGE if "out of range" in msg else -1 if "no tokens" in msg else -7, msg)
    return np.ctypeslib.as_array(p, shape=(e.config.vocab_size,))


def engine_verify_batch(e, tokens, pos_start):
    """qwen3_5/engine.odin:166-174: consume `tokens` from `pos_start` as
    engine_forward_batch does and return every position's logits, [n][vocab]
    (a view of engine memory, valid until the next call)."""
    t = np.ascontiguousarray(tokens, np.int32)
    p = _native.hip().oi_engine_verify_batch(e.handle, t.ctypes.data, int(t.size), int(pos_start))
    if not p:
        L = _native.hip()
        msg = L.oi_last_error().decode()
        raise OIError(OI_E_RANGE if "out of range" in msg else -1 if "no tokens" in msg else -7, msg)
    return np.ctypeslib.as_array(p, shape=(int(t.size), e.config.vocab_size))


def engine_config(e):
    """infer/engine.odin:54-56."""
    return e.config


def engine_hip_ready(e):
    """counterpart of engine_metal_ready (infer/engine.odin:58-60)."""
    return bool(e._h) and e.hip_ready


def engine_decode_greedy(e, token, pos, n_steps):
    """Device-side greedy token loop; returns the n_steps picked ids."""
    out = np.empty(n_steps, np.int32)
    check(_native.hip().oi_engine_decode_greedy(e.handle, int(token), int(pos), int(n_steps), out.ctypes.data))
    return out


class Sampler:
    """sampler.Sampler (sampler/sampler.odin:16-38) without the grammar:
    build_sampler's temperature, topp and rng seed, enable_repeat_penalty's
    penalty, and the recent-token window that record_token keeps."""

    def __init__(self, temperature, topp, rng_seed=0, repeat_penalty=1.0, record=False, last=()):
        self.temperature, self.topp, self.rng_state = float(temperature), float(topp), int(rng_seed)
        self.repeat_penalty = max(float(repeat_penalty), 1.0)  # enable_repeat_penalty clamps (:42-44)
        self.record = bool(record)
        self.last = [int(t) for t in last][-64:]

    def _c(self):
        c = _native.Sampler(self.temperature, self.topp, self.repeat_penalty, int(self.record), self.rng_state,
                            len(self.last))
        for i, t in enumerate(self.last):
            c.last[i] = t
        return c

    def _take(self, c):
        self.rng_state = c.rng_state
        self.last = [int(c.last[i]) for i in range(c.n_last)]


def sample(s, logits):
    """sampler.sample (sampler.odin:141-199) on the device for host logits;
    the logits are not modified.  Advances s."""
    x = np.ascontiguousarray(logits, np.float32)
    c = s._c()
    out = ctypes.c_int32()
    check(_native.hip().oi_sample(x.ctypes.data, int(x.size), ctypes.byref(c), ctypes.byref(out)))
    s._take(c)
    return out.value


def engine_decode_sample(e, token, pos, n_steps, s):
    """Decode loop with the sampler on the device; returns the n_steps picks
    and advances s."""
    out = np.empty(n_steps, np.int32)
    c = s._c()
    check(_native.hip().oi_engine_decode_sample(e.handle, int(token), int(pos), int(n_steps), ctypes.byref(c),
                                                out.ctypes.data))
    s._take(c)
    return out


def engine_kv_fill(e, layer0, pos0, k16, v16):
    """k16, v16: uint16 [nlayers][n_kv_heads][npos][head_dim] binary16 bits."""
    k16 = np.ascontiguousarray(k16, np.uint16)
    v16 = np.ascontiguousarray(v16, np.uint16)
    nl, _, npos, _ = k16.shape
    check(_native.hip().oi_engine_kv_fill(e.handle, int(layer0), nl, int(pos0), npos, k16.ctypes.data,
                                          v16.ctypes.data))


def engine_time_kernel(e, kernel, iters):
    """(mean us per launch from HIP events, algorithmic bytes per launch)."""
    us = ctypes.c_double()
    b = ctypes.c_double()
    check(_native.hip().oi_engine_time_kernel(e.handle, KERNELS[kernel], int(iters), ctypes.byref(us),
                                              ctypes.byref(b)))
    return us.value, b.value


def engine_stream(e):
    return _native.hip().oi_engine_stream(e.handle)


def engine_reset_state(e):
    """qwen3_5/engine.odin:108-132: zero the KV cache and the DeltaNet states."""
    check(_native.hip().oi_engine_reset_state(e.handle))


def engine_save_kv(e, path, n_valid_pos):
    """engine_save_kv (qwen3_5/kv_persist.odin:365-372): write the .oikv v1
    file of positions [0, n_valid_pos) and the DeltaNet states.  As the
    reference: the message goes to stderr and the result is False on failure."""
    rc = _native.hip().oi_engine_save_kv(e.handle, str(path).encode(), int(n_valid_pos))
    if rc != 0:
        print(_native.hip().oi_last_error().decode(), file=sys.stderr)
    return rc == 0


def engine_load_kv(e, path):
    """engine_load_kv (kv_persist.odin:374-381): (n_valid_pos, True), or
    (0, False) with the reason on stderr when the file is refused."""
    n = ctypes.c_int32()
    rc = _native.hip().oi_engine_load_kv(e.handle, str(path).encode(), ctypes.byref(n))
    if rc != 0:
        print(_native.hip().oi_last_error().decode(), file=sys.stderr)
        return 0, False
    return n.value, True


def engine_state_sizes(e):
    """Byte sizes of (kv_k, kv_v, conv, rec) snapshots."""
    s = (ctypes.c_int64 * 4)()
    check(_native.hip().oi_engine_state_sizes(e.handle, s))
    return tuple(s)


def _buf(n):
    return np.empty(n, np.uint8)


def engine_save_full_state(e):
    """engine_save_full_state (qwen3_5/engine.odin:139-144): host copies
    (kv_k, kv_v, conv, rec) of the device state, in its layout."""
    bufs = [_buf(n) for n in engine_state_sizes(e)]
    check(_native.hip().oi_engine_save_full_state(e.handle, *[b.ctypes.data for b in bufs]))
    return tuple(bufs)


def engine_restore_full_state(e, kv_k, kv_v, conv, rec):
    """engine_restore_full_state (qwen3_5/engine.odin:146-151)."""
    bufs = [np.ascontiguousarray(b, np.uint8) for b in (kv_k, kv_v, conv, rec)]
    for b, n in zip(bufs, engine_state_sizes(e)):
        if b.size != n:
            raise OIError(-1, "snapshot size %d, the engine holds %d" % (b.size, n))
    check(_native.hip().oi_engine_restore_full_state(e.handle, *[b.ctypes.data for b in bufs]))


def engine_save_spec_state(e):
    """engine_save_spec_state (qwen3_5/engine.odin:153-158): (conv, rec)."""
    _, _, nc, nr = engine_state_sizes(e)
    conv, rec = _buf(nc), _buf(nr)
    check(_native.hip().oi_engine_save_spec_state(e.handle, conv.ctypes.data, rec.ctypes.data))
    return conv, rec


def engine_restore_spec_state(e, conv, rec):
    """engine_restore_spec_state (qwen3_5/engine.odin:160-165)."""
    _, _, nc, nr = engine_state_sizes(e)
    conv, rec = np.ascontiguousarray(conv, np.uint8), np.ascontiguousarray(rec, np.uint8)
    if conv.size != nc or rec.size != nr:
        raise OIError(-1, "snapshot sizes differ from the engine's")
    check(_native.hip().oi_engine_restore_spec_state(e.handle, conv.ctypes.data, rec.ctypes.data))


def engine_logits_device(e):
    return _native.hip().oi_engine_logits_device(e.handle)
