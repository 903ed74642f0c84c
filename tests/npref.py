"""Independent numpy restatements used to pin the CPU oracle (oracle/refcpu.c).

They are written from the block formats and the model mathematics, in a
different form from the oracle (vectorised, element-wise, float64 where the
reference is float32), so that a dropped term, a wrong sign or a transposed
index in the oracle fails a comparison:

  * dequant_*_elem: the reference's element-wise decoders k4_dequant_elem
    (qwen3_5/metal.odin:476-486) and k6_dequant_elem (:542-555), vectorised in
    float32 with the same operation order, so they must agree bit-for-bit
    with the row decoders of ggml/quant.odin;
  * scale_min_unpack: 6-bit (scale, min) fields read by bit position;
  * forward_f64: a float64 dense-Qwen3 forward (RMSNorm, per-head q/k norm,
    NEOX RoPE, grouped-query attention, SwiGLU) from the dequantized weights;
  * forward_general_f64: the same for the routed-expert (Qwen3-MoE) and
    hybrid (Qwen3.5: full attention + gated DeltaNet, dense or routed FFN)
    layouts.
"""
import numpy as np

F32 = np.float32


def f16(b2):
    """little-endian byte pairs (..., 2) -> float32"""
    return np.ascontiguousarray(b2).view(np.uint16).astype(np.uint16).view(np.float16).astype(F32)


def scale_min_unpack(q12):
    """(n, 12) uint8 -> sc (n, 8), m (n, 8): bit-field layout of the Q4_K
    scales: entries 0-3 are the low 6 bits of bytes 0-3 (scales) and 4-7
    (mins); entries 4-7 take their low 4 bits from the nibbles of bytes 8-11
    (scale: low nibble, min: high nibble) and their top 2 bits from the top 2
    bits of bytes 0-3 (scales) and 4-7 (mins)."""
    q = q12.astype(np.int64)
    sc = np.zeros((q.shape[0], 8), np.int64)
    m = np.zeros_like(sc)
    for j in range(4):
        sc[:, j] = q[:, j] & 0x3F
        m[:, j] = q[:, 4 + j] & 0x3F
        sc[:, 4 + j] = (q[:, 8 + j] & 0x0F) + 16 * (q[:, j] >> 6)
        m[:, 4 + j] = (q[:, 8 + j] >> 4) + 16 * (q[:, 4 + j] >> 6)
    return sc, m


def dequant_q4k_elem(blocks):
    """(nb*144,) uint8 -> (nb*256,) float32, element-wise form."""
    b = blocks.reshape(-1, 144)
    d, dmin = f16(b[:, 0:2])[:, 0], f16(b[:, 2:4])[:, 0]
    sc, m = scale_min_unpack(b[:, 4:16])
    qs = b[:, 16:].astype(np.int64)
    e = np.arange(256)
    sup, ws = e >> 6, e & 63
    hf, l = ws >> 5, ws & 31
    is_ = sup * 2 + hf
    nib = (qs[:, sup * 32 + l] >> (4 * hf)) & 0xF
    # d * sc * nib - dmin * m, left to right, each op rounded to float32
    t = (d[:, None] * sc[:, is_].astype(F32)).astype(F32)
    t = (t * nib.astype(F32)).astype(F32)
    mm = (dmin[:, None] * m[:, is_].astype(F32)).astype(F32)
    return (t - mm).astype(F32).reshape(-1)


def dequant_q6k_elem(blocks):
    b = blocks.reshape(-1, 210)
    ql, qh = b[:, :128].astype(np.int64), b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(b[:, 208:210])[:, 0]
    e = np.arange(256)
    hf, within = e >> 7, e & 127
    l, sub = within & 31, within >> 5
    is_ = l >> 4
    qloff, qhoff, scoff = hf * 64, hf * 32, hf * 8
    lo_idx = qloff + l + 32 * (sub & 1)
    lo = (ql[:, lo_idx] >> (4 * (sub >> 1))) & 0xF
    hi = (qh[:, qhoff + l] >> (2 * sub)) & 3
    q = (lo | (hi << 4)) - 32
    s = sc[:, scoff + is_ + 2 * sub]
    t = (d[:, None] * s.astype(F32)).astype(F32)
    return (t * q.astype(F32)).astype(F32).reshape(-1)


def dequant_q8_0_elem(blocks):
    b = blocks.reshape(-1, 34)
    d = f16(b[:, 0:2])[:, 0]
    q = b[:, 2:].view(np.int8).astype(F32)
    return (d[:, None] * q).astype(F32).reshape(-1)


def dequant_legacy_elem(kind, blocks):
    """Q4_0 / Q4_1 / Q5_0 / Q5_1 (GGML's 32-element blocks; reader:
    ggml/quant.odin:98-162), element by element: element e of a block takes
    nibble e // 16 of byte e % 16 of qs, and (Q5) bit e of the 32-bit qh as
    its fifth bit.  Q4_0 / Q5_0: (q - 8 | 16) * d; Q4_1 / Q5_1: q * d + m,
    each operation rounded to float32."""
    bb = {2: 18, 3: 20, 6: 22, 7: 24}[kind]
    b = blocks.reshape(-1, bb)
    d = f16(b[:, 0:2])[:, 0]
    has_m = kind in (3, 7)
    m = f16(b[:, 2:4])[:, 0] if has_m else None
    e = np.arange(32)
    if kind in (6, 7):
        o = 4 if has_m else 2
        qh = b[:, o:o + 4].astype(np.int64)
        qh = qh[:, 0] | qh[:, 1] << 8 | qh[:, 2] << 16 | qh[:, 3] << 24
        qs = b[:, o + 4:].astype(np.int64)
        q = ((qs[:, e % 16] >> (4 * (e // 16))) & 0xF) | (((qh[:, None] >> e) & 1) << 4)
        off = 16
    else:
        qs = b[:, 4 if has_m else 2:].astype(np.int64)
        q = (qs[:, e % 16] >> (4 * (e // 16))) & 0xF
        off = 8
    if has_m:
        return ((q.astype(F32) * d[:, None]).astype(F32) + m[:, None]).astype(F32).reshape(-1)
    return ((q - off).astype(F32) * d[:, None]).astype(F32).reshape(-1)


def dequant(kind, blocks, n):
    if kind == 0:
        return np.ascontiguousarray(blocks).view(F32)[:n].copy()
    if kind == 1:
        return f16(np.ascontiguousarray(blocks).reshape(-1, 2))[:, 0][:n]
    if kind in (2, 3, 6, 7):
        return dequant_legacy_elem(kind, blocks)[:n]
    return {8: dequant_q8_0_elem, 12: dequant_q4k_elem, 14: dequant_q6k_elem}[kind](blocks)[:n]


# ------------------------------------------------------------ float64 model --

class GGUFWeights:
    """Minimal GGUF reader for the tests (independent of both parsers under
    test): returns float64 dequantized weights by tensor name."""

    def __init__(self, path):
        import struct
        data = np.fromfile(path, np.uint8)
        self.data = data
        pos = 0

        def rd(fmt):
            nonlocal pos
            v = struct.unpack_from("<" + fmt, data, pos)
            pos += struct.calcsize("<" + fmt)
            return v[0]

        def rstr():
            nonlocal pos
            n = rd("Q")
            s = bytes(data[pos:pos + n]).decode()
            pos += n
            return s

        assert rd("I") == 0x46554747
        rd("I")
        nt, nm = rd("Q"), rd("Q")
        self.meta = {}
        scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}
        for _ in range(nm):
            k = rstr()
            t = rd("I")
            if t == 8:
                self.meta[k] = rstr()
            elif t in scalar:
                self.meta[k] = rd(scalar[t])
            else:
                raise ValueError("array metadata not expected in synthetic files")
        self.tensors = {}
        for _ in range(nt):
            name = rstr()
            nd = rd("I")
            dims = [rd("Q") for _ in range(nd)]
            kind = rd("I")
            off = rd("Q")
            self.tensors[name] = (dims, kind, off)
        align = self.meta.get("general.alignment", 32)
        self.base = (pos + align - 1) // align * align

    def get(self, name):
        dims, kind, off = self.tensors[name]
        n = int(np.prod(dims))
        e, b = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
                12: (256, 144), 14: (256, 210)}[kind]
        dims = [int(d) for d in dims]
        raw = self.data[self.base + off: self.base + off + n // e * b]
        w = dequant(kind, raw, n).astype(np.float64)
        return w.reshape(dims[::-1]) if len(dims) > 1 else w


def forward_f64(W, tokens, f16_kv=True, staged=()):
    """Logits (float64) after each token of `tokens` at positions 0.. .
    Positions in `staged` take the batched prefill path's projections: the
    seven layer matrices and their inputs rounded to f16 before the product
    (qwen3_5/metal.odin:1236-1243, 493-609)."""
    m = W.meta
    D = m["qwen3.embedding_length"]
    L = m["qwen3.block_count"]
    H = m["qwen3.attention.head_count"]
    KVH = m["qwen3.attention.head_count_kv"]
    hd = m["qwen3.attention.key_length"]
    theta = m.get("qwen3.rope.freq_base", 1e6)
    eps = m.get("qwen3.attention.layer_norm_rms_epsilon", 1e-6)
    emb = W.get("token_embd.weight")
    out_w = W.get("output.weight") if "output.weight" in W.tensors else emb

    def rms(x, w):
        return w * x / np.sqrt(np.mean(x * x) + eps)

    def rope(v, pos):  # NEOX pairs (i, i + hd/2)
        i = np.arange(hd // 2)
        ang = pos * theta ** (-(i / (hd // 2)))
        c, s = np.cos(ang), np.sin(ang)
        a, b = v[..., : hd // 2], v[..., hd // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)

    def r16(v):
        return v.astype(np.float16).astype(np.float64) if f16_kv else v

    layers = []
    for l in range(L):
        p = "blk.%d." % l
        layers.append({k: W.get(p + k + ".weight") for k in
                       ["attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm", "attn_q", "attn_k", "attn_v",
                        "attn_output", "ffn_gate", "ffn_down", "ffn_up"]})
    h16 = {}

    def s16(a):
        return a.astype(np.float16).astype(np.float64)

    def mm(name, lw, l, x, st):
        if not st:
            return lw[name] @ x
        if (l, name) not in h16:
            h16[(l, name)] = s16(lw[name])
        return h16[(l, name)] @ s16(x)

    kc = [[] for _ in range(L)]
    vc = [[] for _ in range(L)]
    outs = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        st = pos in staged
        for l, lw in enumerate(layers):
            xb = rms(x, lw["attn_norm"])
            q = mm("attn_q", lw, l, xb, st).reshape(H, hd)
            k = mm("attn_k", lw, l, xb, st).reshape(KVH, hd)
            v = mm("attn_v", lw, l, xb, st).reshape(KVH, hd)
            q = rope(np.stack([rms(qh, lw["attn_q_norm"]) for qh in q]), pos)
            k = rope(np.stack([rms(kh, lw["attn_k_norm"]) for kh in k]), pos)
            kc[l].append(r16(k))
            vc[l].append(r16(v))
            K, V = np.stack(kc[l]), np.stack(vc[l])  # (t, KVH, hd)
            o = np.zeros((H, hd))
            for h in range(H):
                g = h // (H // KVH)
                sc = K[:, g, :] @ q[h] / np.sqrt(hd)
                p_ = np.exp(sc - sc.max())
                p_ /= p_.sum()
                o[h] = p_ @ V[:, g, :]
            x = x + mm("attn_output", lw, l, o.reshape(-1), st)
            xb = rms(x, lw["ffn_norm"])
            gt, up = mm("ffn_gate", lw, l, xb, st), mm("ffn_up", lw, l, xb, st)
            x = x + mm("ffn_down", lw, l, gt / (1 + np.exp(-gt)) * up, st)
        outs.append(out_w @ rms(x, W.get("output_norm.weight")))
    return outs


def deltanet_f64(n_kh, n_vh, hk, hv, kernel, eps, qkv, z, b, a, conv_w, a_decay, dt_bias, norm_w, conv_state,
                 rec_state, kv_from_q=False):
    """Float64 restatement of the gated DeltaNet token step over a trajectory
    (qwen3_5/forward.odin:172-219 with ops.odin's conv1d_step, l2norm,
    delta_recurrent_step).  kv_from_q=True reproduces the golden of
    delta_harness/delta_ref.odin:61, which reads the memory with q instead of
    k (a known mistake there), for tests that must tell the two apart."""
    f = lambda x: np.array(x, np.float64)
    qkv, z, b, a = f(np.atleast_2d(qkv)), f(np.atleast_2d(z)), f(np.atleast_2d(b)), f(np.atleast_2d(a))
    conv_w, a_decay, dt_bias, norm_w = f(conv_w), f(a_decay), f(dt_bias), f(norm_w)
    cs, S = f(conv_state).reshape(-1, kernel - 1) if kernel > 1 else None, f(rec_state).reshape(n_vh, hk, hv)
    kd, vd = n_kh * hk, n_vh * hv
    cw = conv_w.reshape(-1, kernel)
    outs = []
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))
    for t in range(qkv.shape[0]):
        x = qkv[t]
        win = np.concatenate([cs, x[:, None]], axis=1) if kernel > 1 else x[:, None]
        acc = (cw * win).sum(axis=1)
        co = acc * sig(acc)
        if kernel > 1:
            cs = win[:, 1:]
        q = co[:kd].reshape(n_kh, hk)
        k = co[kd:2 * kd].reshape(n_kh, hk)
        v = co[2 * kd:].reshape(n_vh, hv)
        q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-6) / np.sqrt(hk)
        k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), 1e-6)
        o = np.empty((n_vh, hv))
        for vh in range(n_vh):
            kh = vh % n_kh
            beta = sig(b[t, vh])
            sp = a[t, vh] + dt_bias[vh]
            sp = sp if sp > 20 else (0.0 if sp < -20 else np.log1p(np.exp(sp)))
            S[vh] *= np.exp(a_decay[vh] * sp)
            mem = S[vh].T @ (q[kh] if kv_from_q else k[kh])
            delta = (v[vh] - mem) * beta
            S[vh] += np.outer(k[kh], delta)
            o[vh] = S[vh].T @ q[kh]
        o = o / np.sqrt(np.mean(o * o, axis=1, keepdims=True) + eps) * norm_w
        zz = z[t].reshape(n_vh, hv)
        outs.append((o * zz * sig(zz)).reshape(-1))
    return np.array(outs), (cs.reshape(-1) if kernel > 1 else np.zeros(0)), S.reshape(-1)


def delta_tokens_f64(state, q, k, v, beta, g):
    """Float64 gated delta rule token by token (qwen3_5/ops.odin:120-153):
    S *= g_t; d = (v_t - S^T k_t) beta_t; S += k_t d^T; o_t = S^T q_t.
    Returns (out [C, hv], state [hk, hv])."""
    S = np.array(state, np.float64).copy()
    out = []
    for t in range(len(k)):
        S *= g[t]
        d = (np.float64(v[t]) - S.T @ np.float64(k[t])) * beta[t]
        S += np.outer(np.float64(k[t]), d)
        out.append(S.T @ np.float64(q[t]))
    return np.array(out), S


def delta_chunk_f64(state, q, k, v, beta, g, mistake=None):
    """Float64 chunked form of the gated delta rule over C tokens (the math of
    qwen3_5/metal.odin:416-468 chunked_delta), written with matrices: cp the
    running product of the decays, D[t, i] = cp[t] / cp[i],
      (I + tril(beta D (K K^T), -1)) Delta = beta v - beta cp (K S)
      O  = cp (Q S) + tril(D (Q K^T)) Delta
      S' = cp[C-1] S + (K cp[C-1] / cp)^T Delta.
    `mistake` plants one error for tests that must catch it: 'no_ratio' (cp[t]
    for cp[t] / cp[i]), 'o_strict' (O without the i = t term), 'state_ratio'
    (S' without the per-token factors), 'l_diag' (the diagonal kept in the
    substitution).  Returns (out [C, hv], state [hk, hv])."""
    f = lambda x: np.array(x, np.float64)
    S, q, k, v, beta, g = f(state), f(q), f(k), f(v), f(beta), f(g)
    cp = np.cumprod(g)
    D = cp[:, None] / cp[None, :] if mistake != "no_ratio" else np.repeat(cp[:, None], len(cp), 1)
    L = np.tril(beta[:, None] * D * (k @ k.T), 0 if mistake == "l_diag" else -1)
    rhs = beta[:, None] * v - (beta * cp)[:, None] * (k @ S)
    delta = np.linalg.solve(np.eye(len(k)) + L, rhs)
    O = cp[:, None] * (q @ S) + np.tril(D * (q @ k.T), -1 if mistake == "o_strict" else 0) @ delta
    w = cp[-1] / cp if mistake != "state_ratio" else np.ones_like(cp)
    return O, cp[-1] * S + (k * w[:, None]).T @ delta


def qwen35_attn_f64(n_heads, n_kv, hd, rotary_dim, seq_len, eps, pos0, qproj, k, v, q_norm, k_norm, theta,
                    kc16, vc16, full_rotary=False, gate=True):
    """Float64 restatement of forward_full_layer's attention
    (qwen3_5/forward.odin:69-127) over tokens from pos0 with an f16 cache (k/v rounded
    on store).  full_rotary / gate=False give the variants a mistake would
    produce (RoPE over the whole head, no output gate)."""
    f = lambda x: np.array(x, np.float64)
    qproj, k, v = f(np.atleast_2d(qproj)), f(np.atleast_2d(k)), f(np.atleast_2d(v))
    q_norm, k_norm = f(q_norm), f(k_norm)
    K = np.array(kc16, np.uint16).view(np.float16).astype(np.float64).reshape(n_kv, seq_len, hd)
    V = np.array(vc16, np.uint16).view(np.float16).astype(np.float64).reshape(n_kv, seq_len, hd)
    rd = hd if full_rotary else rotary_dim
    half = rd // 2
    inv = theta ** (-(np.arange(half) / (rd / 2.0)))

    def rms(x, w):
        return w * x / np.sqrt(np.mean(x * x) + eps)

    def rope(x, pos):
        x = x.copy()
        a, b = x[:half].copy(), x[half:rd].copy()
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        x[:half], x[half:rd] = a * c - b * s, a * s + b * c
        return x

    outs = []
    for t in range(qproj.shape[0]):
        pos = pos0 + t
        qp = qproj[t].reshape(n_heads, 2, hd)
        q = np.stack([rope(rms(qp[h, 0], q_norm), pos) for h in range(n_heads)])
        kk = np.stack([rope(rms(k[t].reshape(n_kv, hd)[h], k_norm), pos) for h in range(n_kv)])
        K[:, pos] = kk.astype(np.float16).astype(np.float64)
        V[:, pos] = v[t].reshape(n_kv, hd).astype(np.float16).astype(np.float64)
        o = np.empty((n_heads, hd))
        for h in range(n_heads):
            g = h // (n_heads // n_kv)
            sc = K[g, :pos + 1] @ q[h] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            o[h] = (p / p.sum()) @ V[g, :pos + 1]
            if gate:
                o[h] *= 1.0 / (1.0 + np.exp(-qp[h, 1]))
        outs.append(o.reshape(-1))
    return np.array(outs)


def forward_general_f64(W, tokens, moe_renorm=True, shared_gate=True, attn_gate=True, ffn_norm=True, staged=()):
    """Float64 forward of the routed-expert and hybrid layouts: "qwen3moe"
    (Qwen3 attention, routed-expert FFN) and "qwen35" (qwen3_5/forward.odin:
    16-243: every full_attention_interval-th layer full attention with
    [q | gate] heads, partial RoPE and a sigmoid output gate, the others gated
    DeltaNet; the FFN dense or routed experts plus a sigmoid-gated shared
    expert).  Routed experts follow HF Qwen3-MoE / Qwen3-Next: softmax over
    the router logits, the top k (ties to the lower id), weights renormalized,
    y = sum_k w_k down_k(silu(gate_k x) * up_k x) [+ sigmoid(s . x) *
    shared(x)].  The keyword switches give the models a mistake would produce
    (no renormalization, no shared-expert gate, no attention output gate, the
    attention norm's weight used for the FFN norm).
    Logits after each token at positions 0.. (f16-rounded K/V, as the oracle's
    f16 mode).  Positions in `staged` take the batched prefill path's
    projections (forward_gpu_batch, qwen3_5/metal.odin:1510-1634): the
    attention / DeltaNet projections and a dense MLP with weights and inputs
    rounded to f16; the router, routed experts and shared expert exact."""
    m = W.meta
    arch = m["general.architecture"]
    a = arch + "."
    D, L = m[a + "embedding_length"], m[a + "block_count"]
    H, KVH, hd = m[a + "attention.head_count"], m[a + "attention.head_count_kv"], m[a + "attention.key_length"]
    theta = m[a + "rope.freq_base"]
    eps = m[a + "attention.layer_norm_rms_epsilon"]
    E, K = m.get(a + "expert_count", 0), m.get(a + "expert_used_count", 0)
    hybrid = arch == "qwen35"
    if hybrid:
        interval, rd = m[a + "full_attention_interval"], m[a + "rope.dimension_count"]
        nk, nv, hk = m[a + "ssm.group_count"], m[a + "ssm.time_step_rank"], m[a + "ssm.state_size"]
        hv, kern = m[a + "ssm.inner_size"] // nv, m[a + "ssm.conv_kernel"]
    else:
        rd = hd
    emb = W.get("token_embd.weight")
    out_w = W.get("output.weight") if "output.weight" in W.tensors else emb
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))

    def rms(x, w):
        return w * x / np.sqrt(np.mean(x * x) + eps)

    def rope(v, pos):  # pairs (i, i + rd/2) over the first rd dimensions
        half = rd // 2
        inv = theta ** (-(np.arange(half) / (rd / 2.0)))
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        v = v.copy()
        x0, x1 = v[..., :half].copy(), v[..., half:rd].copy()
        v[..., :half], v[..., half:rd] = x0 * c - x1 * s, x0 * s + x1 * c
        return v

    def attention(q, kc, vc, l):
        Kc, Vc = np.stack(kc[l]), np.stack(vc[l])  # (t, KVH, hd)
        o = np.zeros((H, hd))
        for h in range(H):
            g = h // (H // KVH)
            sc = Kc[:, g, :] @ q[h] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            o[h] = (p / p.sum()) @ Vc[:, g, :]
        return o

    r16 = lambda v: v.astype(np.float16).astype(np.float64)
    G = lambda name: W.get(name)
    h16 = {}

    def S(name, st):  # a projection matrix, f16-rounded on a staged position
        if not st:
            return G(name)
        if name not in h16:
            h16[name] = r16(G(name))
        return h16[name]
    kc = [[] for _ in range(L)]
    vc = [[] for _ in range(L)]
    conv = {}
    rec = {}
    outs = []
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        st = pos in staged
        for l in range(L):
            p = "blk.%d." % l
            full = (not hybrid) or (l + 1) % interval == 0
            xb = rms(x, G(p + "attn_norm.weight"))
            xs = r16(xb) if st else xb
            if not hybrid:
                q = (S(p + "attn_q.weight", st) @ xs).reshape(H, hd)
                k = (S(p + "attn_k.weight", st) @ xs).reshape(KVH, hd)
                v = (S(p + "attn_v.weight", st) @ xs).reshape(KVH, hd)
                q = rope(np.stack([rms(qh, G(p + "attn_q_norm.weight")) for qh in q]), pos)
                k = rope(np.stack([rms(kh, G(p + "attn_k_norm.weight")) for kh in k]), pos)
                kc[l].append(r16(k))
                vc[l].append(r16(v))
                o = attention(q, kc, vc, l).reshape(-1)
                x = x + S(p + "attn_output.weight", st) @ (r16(o) if st else o)
            elif full:
                qp = (S(p + "attn_q.weight", st) @ xs).reshape(H, 2, hd)
                k = (S(p + "attn_k.weight", st) @ xs).reshape(KVH, hd)
                v = (S(p + "attn_v.weight", st) @ xs).reshape(KVH, hd)
                q = rope(np.stack([rms(qp[h, 0], G(p + "attn_q_norm.weight")) for h in range(H)]), pos)
                k = rope(np.stack([rms(kh, G(p + "attn_k_norm.weight")) for kh in k]), pos)
                kc[l].append(r16(k))
                vc[l].append(r16(v))
                o = (attention(q, kc, vc, l) * (sig(qp[:, 1, :]) if attn_gate else 1.0)).reshape(-1)
                x = x + S(p + "attn_output.weight", st) @ (r16(o) if st else o)
            else:
                kd, vd = nk * hk, nv * hv
                if l not in conv:
                    conv[l] = np.zeros((2 * kd + vd) * (kern - 1))
                    rec[l] = np.zeros(nv * hk * hv)
                qkv = S(p + "attn_qkv.weight", st) @ xs
                z = S(p + "attn_gate.weight", st) @ xs
                bb = S(p + "ssm_beta.weight", st) @ xs
                aa = S(p + "ssm_alpha.weight", st) @ xs
                o, conv[l], rec[l] = deltanet_f64(nk, nv, hk, hv, kern, eps, qkv, z, bb, aa,
                                                  G(p + "ssm_conv1d.weight").reshape(-1), G(p + "ssm_a"),
                                                  G(p + "ssm_dt.bias"), G(p + "ssm_norm.weight"), conv[l], rec[l])
                x = x + S(p + "ssm_out.weight", st) @ (r16(o[0]) if st else o[0])
            nname = ("post_attention_norm.weight" if hybrid else "ffn_norm.weight") if ffn_norm else "attn_norm.weight"
            xb = rms(x, G(p + nname))
            if E:
                pr = G(p + "ffn_gate_inp.weight") @ xb
                pr = np.exp(pr - pr.max())
                pr /= pr.sum()
                ids = sorted(range(E), key=lambda i: (-pr[i], i))[:K]
                w = pr[ids] / (pr[ids].sum() if moe_renorm else 1.0)
                Ge, Ue, De = G(p + "ffn_gate_exps.weight"), G(p + "ffn_up_exps.weight"), G(p + "ffn_down_exps.weight")
                y = np.zeros(D)
                for wk, ex in zip(w, ids):
                    gt, up = Ge[ex] @ xb, Ue[ex] @ xb
                    y += wk * (De[ex] @ (gt * sig(gt) * up))
                if p + "ffn_gate_inp_shexp.weight" in W.tensors:
                    gs = float((G(p + "ffn_gate_inp_shexp.weight") @ xb).reshape(-1)[0])
                    gt, up = G(p + "ffn_gate_shexp.weight") @ xb, G(p + "ffn_up_shexp.weight") @ xb
                    ys = G(p + "ffn_down_shexp.weight") @ (gt * sig(gt) * up)
                    y += (sig(gs) if shared_gate else 1.0) * ys
                x = x + y
            else:
                xs = r16(xb) if st else xb
                gt, up = S(p + "ffn_gate.weight", st) @ xs, S(p + "ffn_up.weight", st) @ xs
                hh = gt * sig(gt) * up
                x = x + S(p + "ffn_down.weight", st) @ (r16(hh) if st else hh)
        outs.append(out_w @ rms(x, G("output_norm.weight")))
    return outs
