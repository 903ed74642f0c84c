// prefill_hybrid.hip -- the per-token operations of batched prefill for the
// Qwen3.5 hybrid layers, T tokens at once (reference: qwen3_5/metal.odin:
// 1510-1622 forward_gpu_batch; the per-token math is qwen3_5/forward.odin:
// 46-225 and ops.odin).  The projections between them run on the matrix cores
// (gemm.hip); the kernels here read the projections' K-slice partial products
// and sum them in slice order.
//
// Full-attention layer (forward_full_layer):
//   pf_q35_qkv_kernel  [q | gate] split, q / k head RMSNorm, partial RoPE at
//                      pos0 + t, k and v rounded to f16 into the cache; the
//                      causal attention with the sigmoid gate is
//                      prefill.hip's (launch_pf_attn with a gate).
// Linear-attention layer (forward_linear_layer):
//   pf_dn_conv_kernel       causal depthwise conv over the chunk (inputs before
//                           the chunk from the conv state) + silu; the conv
//                           state after the chunk (its last inputs)
//   pf_dn_prep_kernel       per token: l2norm of q (times 1/sqrt(head_k_dim))
//                           and k, beta = sigmoid(b), decay = exp(ssm_a
//                           softplus(a + dt_bias)) and its log
//   pf_dn_delta_kernel      the delta rule over the chunk's tokens in order,
//                           the state held in registers for the whole chunk
//   pf_dn_chunk_kernel      the same in its chunked form (qwen3_5/metal.odin:416-468,
//                           which the reference does not dispatch): 16 or 32
//                           tokens per step, decay ratios from log sums
//   pf_dc_prep_kernel,      the chunked form in chunks of 64 on the matrix
//   pf_dc_state_kernel      cores: the state-free C x C matrices of every
//                           chunk at once, then the state carried through them
//   pf_dc_single_kernel     the same for a prompt of one chunk, in one launch
//   pf_dn_gnorm_kernel      gated RMSNorm, f16 rows for the output projection
//                           (or f32 rows for the host-memory entry point)
//
// Layouts: token-major; partial products [split][T][rows]; the conv state
// [conv_dim][kernel - 1] oldest first and the recurrent state [n_vh][hk][hv]
// are the decode path's, so decode continues from the chunk.

#include "device_common.h"

namespace oi {

// Per token and head (grid (T, ceil(heads / 4)), one wave per head; q, k and
// v heads in that order).  The q projection holds [q | gate] per head
// (qwen3_5/forward.odin:74-82); gate goes out unchanged.  q and k heads: RMSNorm with
// q_norm / k_norm, then RoPE on the first rotary_dim dimensions (pairs i and
// i + rotary_dim / 2, angle pos * inv_freq[i] in f32, qwen3_5/ops.odin:77-89), as
// qwen35_attn.hip does for one token.  Lane l holds dimensions l + 64 e.
template <int HD>
__global__ __launch_bounds__(WG) void pf_q35_qkv_kernel(PfQ35Args a) {
#pragma clang fp contract(off)
    constexpr int DPL = HD / WAVE;
    __shared__ float xs[WG / WAVE][HD];
    const int t = blockIdx.x, lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int hh = (int)blockIdx.y * (WG / WAVE) + wave;
    if (hh >= a.n_heads + 2 * a.n_kv_heads) return;  // whole waves; no workgroup barrier below
    const int pos = a.pos0 + t, QD = a.n_heads * HD, KVD = a.n_kv_heads * HD;
    const bool isq = hh < a.n_heads, isk = !isq && hh < a.n_heads + a.n_kv_heads;
    const int h = isq ? hh : isk ? hh - a.n_heads : hh - a.n_heads - a.n_kv_heads;
    float v[DPL];
    if (isq) {
        const size_t slice = (size_t)a.T * 2 * QD, base = (size_t)t * 2 * QD + (size_t)h * 2 * HD;
        float qg[2 * DPL];  // q, then gate
        parts_gather(qg, a.q, a.qs, slice, [&](int j) { return base + (j / DPL) * HD + lane + WAVE * (j % DPL); });
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            v[e] = qg[e];
            a.gate[(size_t)t * QD + h * HD + lane + WAVE * e] = qg[DPL + e];
        }
    } else {
        const float *src = isk ? a.k : a.v;
        const int split = isk ? a.ks : a.vs;
        const size_t base = (size_t)t * KVD + h * HD + lane;
        parts_gather(v, src, split, (size_t)a.T * KVD, [&](int e) { return base + WAVE * e; });
    }
    if (isq || isk) {
        const float *nw = isq ? a.q_norm : a.k_norm;
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; e++) ss += v[e] * v[e];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
        float *x = xs[wave];
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            v[e] = nw[lane + WAVE * e] * (inv * v[e]);
            x[lane + WAVE * e] = v[e];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        const int half = a.rotary_dim / 2;
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            const int i = lane + WAVE * e;
            if (i < a.rotary_dim) {
                const int pr = i < half ? i : i - half;
                const float ang = (float)pos * a.inv_freq[pr];
                const float c = cosf(ang), sn = sinf(ang);
                v[e] = i < half ? x[i] * c - x[i + half] * sn : x[i - half] * sn + x[i] * c;
            }
        }
    }
    if (isq) {
#pragma unroll
        for (int e = 0; e < DPL; e++) a.qout[(size_t)t * QD + h * HD + lane + WAVE * e] = v[e];
    } else {
        uint16_t *c = (isk ? a.kc : a.vc) + ((size_t)h * a.seq_len + pos) * HD;
#pragma unroll
        for (int e = 0; e < DPL; e++) c[lane + WAVE * e] = f2h(v[e]);
    }
}

// ---------------------------------------------------------------- DeltaNet --

constexpr int DN_TT = 8;  // tokens per thread of the conv

// conv1d_step + silu (qwen3_5/ops.odin:97-116) of channel c for tokens [8 y, 8 y +
// 8): out = silu(w[KS-1] in(t) + sum_k w[k] in(t - (KS-1) + k)), the order
// of the decode step, where in(tau) is the in_qkv projection of token tau of
// the chunk or, before the chunk (tau in [-(KS-1), 0)), the conv state's
// input.  The window and the tokens are gathered together (clamped indices,
// every load unconditional).  The first token block, the only one that reads
// the conv state, also writes the state after the chunk: its last KS-1
// inputs, oldest first (T >= KS-1, so every one comes from the chunk; the
// same thread reads the old state first).  Grid (ceil(conv_dim / 256),
// ceil(T / 8)).
template <int KS>
__global__ __launch_bounds__(WG) void pf_dn_conv_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int KM1 = KS - 1, NX = KM1 + DN_TT;
    static_assert(DN_TT >= KM1, "only the first block's window reaches before the chunk");
    const int CD = 2 * a.n_kh * a.hk + a.n_vh * a.hv;
    const int c = (int)blockIdx.x * WG + threadIdx.x;
    if (c >= CD) return;
    const int t0 = (int)blockIdx.y * DN_TT, t1 = min(a.T, t0 + DN_TT);
    float w[KS], st[KM1 > 0 ? KM1 : 1], xs[NX];  // xs[j] = in(t0 - KM1 + j)
#pragma unroll
    for (int k = 0; k < KS; k++) w[k] = a.conv_w[(size_t)c * KS + k];
#pragma unroll
    for (int k = 0; k < KM1; k++) st[k] = a.conv_state[(size_t)c * KM1 + k];
    parts_gather(xs, a.qkv, a.qkvs, (size_t)a.T * CD,
                 [&](int j) { return (size_t)min(max(t0 - KM1 + j, 0), t1 - 1) * CD + c; });
    if (t0 == 0) {  // t0 is a multiple of DN_TT >= KM1: only the first block reads the state
        float tail[KM1 > 0 ? KM1 : 1];
        if constexpr (KM1 > 0)
            parts_gather(tail, a.qkv, a.qkvs, (size_t)a.T * CD, [&](int k) { return (size_t)(a.T - KM1 + k) * CD + c; });
#pragma unroll
        for (int k = 0; k < KM1; k++) {
            xs[k] = st[k];
            a.conv_state[(size_t)c * KM1 + k] = tail[k];
        }
    }
#pragma unroll
    for (int i = 0; i < DN_TT; i++) {
        if (t0 + i >= t1) break;
        float acc = w[KM1] * xs[KM1 + i];
#pragma unroll
        for (int k = 0; k < KM1; k++) acc += w[k] * xs[i + k];
        a.conv_out[(size_t)(t0 + i) * CD + c] = silu_ref(acc);
    }
}

// Per token (grid T): l2norm of each k head's q and k (qwen3_5/ops.odin:27-37, eps
// 1e-6 a floor on the norm; q also times 1/sqrt(head_k_dim),
// qwen3_5/forward.odin:177-188) into qk [T][2 key_dim] (q heads, then k heads); the
// gates of every value head into gates [T][3 n_vh] (beta, decay, log decay).
template <int HK>
__global__ __launch_bounds__(WG) void pf_dn_prep_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int E = HK / WAVE;
    const int t = blockIdx.x, lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int KD = a.n_kh * HK, CD = 2 * KD + a.n_vh * a.hv;
    for (int kh = wave; kh < a.n_kh; kh += WG / WAVE) {
        const float *q = a.conv_out + (size_t)t * CD + kh * HK, *k = q + KD;
        float qv[E], kv[E], sq = 0.f, sk = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) {
            qv[e] = q[lane + WAVE * e];
            kv[e] = k[lane + WAVE * e];
            sq += qv[e] * qv[e];
            sk += kv[e] * kv[e];
        }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        const float iq = 1.0f / fmaxf(sqrtf(sq), 1e-6f), ik = 1.0f / fmaxf(sqrtf(sk), 1e-6f);
        float *o = a.qk + (size_t)t * 2 * KD + kh * HK;
#pragma unroll
        for (int e = 0; e < E; e++) {
            o[lane + WAVE * e] = qv[e] * iq * (1.0f / sqrtf((float)HK));
            o[KD + lane + WAVE * e] = kv[e] * ik;
        }
    }
    for (int vh = threadIdx.x; vh < a.n_vh; vh += WG) {
        const size_t slice = (size_t)a.T * a.n_vh, i = (size_t)t * a.n_vh + vh;
        const float b = parts_at(a.b, a.bs, slice, i), av = parts_at(a.a, a.as, slice, i);
        const float lg = a.a_decay[vh] * softplus_ref(av + a.dt_bias[vh]);  // log of the decay
        a.gates[(size_t)t * 3 * a.n_vh + vh] = sigmoid_ref(b);
        a.gates[(size_t)t * 3 * a.n_vh + a.n_vh + vh] = expf(lg);
        a.gates[(size_t)t * 3 * a.n_vh + 2 * a.n_vh + vh] = lg;
    }
}

// The delta rule (qwen3_5/forward.odin:193-209) over the chunk's tokens in order:
//   S *= decay;  delta = (v - S^T k) beta;  S += k delta^T;  o = S^T q.
// Grid (n_vh, hv / 16): a workgroup owns 16 state columns of value head vh
// (k head vh % n_kh); each wave 4 columns, lane = 16 column + row group, a
// row group 8 rows, so a lane holds 8 state values for the whole chunk (read
// once, written once).  The column sums over the 16 row groups are DPP sums
// inside the lane's row of 16.  (With 32 columns and 16 rows per lane half
// the SIMDs had no wave and the token recurrence, the kernel's critical path,
// was twice as long per lane.)  Per 32 tokens the workgroup stages the k
// head's q and k, its v columns and the gates in LDS.
constexpr int DN_DB = 32, DN_RG = 16, DN_CW = WG / DN_RG;
template <int HK, int HV>
__global__ __launch_bounds__(WG) void pf_dn_delta_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int RG = DN_RG, RPL = HK / RG, QP = RG * (RPL + 4);  // rows per lane; row group g at (RPL + 4) g
    constexpr int CW = DN_CW;                                       // columns per workgroup (4 per wave)
    static_assert(RPL == 8 && HV % CW == 0 && CW * RG == WG, "head shape");
    __shared__ __attribute__((aligned(16))) float sq[DN_DB][QP];
    __shared__ __attribute__((aligned(16))) float sk[DN_DB][QP];
    __shared__ __attribute__((aligned(16))) float sv[DN_DB][CW];
    __shared__ float sg[DN_DB][2];
    const int vh = blockIdx.x, kh = vh % a.n_kh, c0 = (int)blockIdx.y * CW;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int cl = wave * (WAVE / RG) + lane / RG, rg = lane % RG, j = c0 + cl, i0 = rg * RPL;
    const int KD = a.n_kh * HK, CD = 2 * KD + a.n_vh * HV, VD = a.n_vh * HV;
    float *S = a.state + (size_t)vh * HK * HV;
    float s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) s[r] = S[(size_t)(i0 + r) * HV + j];
    for (int tb = 0; tb < a.T; tb += DN_DB) {
        const int nb = min(DN_DB, a.T - tb);
        // the block's q, k (float4 pieces), v and gates: every load issued
        // before any is used (a loop of load-then-store would wait for each)
        constexpr int QK4 = DN_DB * 2 * HK / 4 / WG, NV4 = DN_DB * CW / 4;  // NV4 <= WG: one float4 of v per thread
        static_assert(QK4 * WG * 4 == DN_DB * 2 * HK && NV4 <= WG, "staging shape");
        float4 qk4[QK4], v4;
        float gv = 0.f;
#pragma unroll
        for (int i = 0; i < QK4; i++) {
            const int idx = threadIdx.x + i * WG, tt = idx / (HK / 2), e4 = idx % (HK / 2);  // HK / 2 float4 per token
            const int side = e4 / (HK / 4), ee = 4 * (e4 % (HK / 4));
            qk4[i] = tt < nb ? *(const float4 *)(a.qk + (size_t)(tb + tt) * 2 * KD + side * KD + kh * HK + ee)
                             : float4{0.f, 0.f, 0.f, 0.f};
        }
        {
            const int tt = threadIdx.x / (CW / 4), c4 = threadIdx.x % (CW / 4);
            v4 = threadIdx.x < NV4 && tt < nb
                     ? *(const float4 *)(a.conv_out + (size_t)(tb + tt) * CD + 2 * KD + vh * HV + c0 + 4 * c4)
                     : float4{0.f, 0.f, 0.f, 0.f};
        }
        if (threadIdx.x < 2 * nb)
            gv = a.gates[(size_t)(tb + threadIdx.x / 2) * 3 * a.n_vh + (threadIdx.x % 2) * a.n_vh + vh];
        __syncthreads();  // the previous block's LDS reads are done
#pragma unroll
        for (int i = 0; i < QK4; i++) {
            const int idx = threadIdx.x + i * WG, tt = idx / (HK / 2), e4 = idx % (HK / 2);
            const int side = e4 / (HK / 4), ee = 4 * (e4 % (HK / 4));
            *(float4 *)&(side ? sk : sq)[tt][ee + (ee / RPL) * 4] = qk4[i];  // 4 | ee, RPL: one row group
        }
        if (threadIdx.x < NV4) *(float4 *)&sv[threadIdx.x / (CW / 4)][4 * (threadIdx.x % (CW / 4))] = v4;
        if (threadIdx.x < 2 * nb) sg[threadIdx.x / 2][threadIdx.x % 2] = gv;
        __syncthreads();
        for (int tt = 0; tt < nb; tt++) {
            const float beta = sg[tt][0], decay = sg[tt][1];
            const float4 *k4 = (const float4 *)&sk[tt][rg * (RPL + 4)], *q4 = (const float4 *)&sq[tt][rg * (RPL + 4)];
            float kn[RPL], qn[RPL];
#pragma unroll
            for (int i = 0; i < RPL / 4; i++) {
                const float4 kk = k4[i], qq = q4[i];
                kn[4 * i] = kk.x; kn[4 * i + 1] = kk.y; kn[4 * i + 2] = kk.z; kn[4 * i + 3] = kk.w;
                qn[4 * i] = qq.x; qn[4 * i + 1] = qq.y; qn[4 * i + 2] = qq.z; qn[4 * i + 3] = qq.w;
            }
            // four partial sums per product (short dependency chains; the
            // token recurrence is the kernel's critical path)
            float kp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < RPL; r++) {
                s[r] = s[r] * decay;
                kp[r & 3] += s[r] * kn[r];
            }
            float kv = (kp[0] + kp[1]) + (kp[2] + kp[3]);
            kv += OI_DPP(kv, 0xB1);  // sum over the lane's row of 16 (the row groups)
            kv += OI_DPP(kv, 0x4E);
            kv += dpp_mirror8(kv);
            kv += OI_DPP(kv, 0x140);
            const float delta = (sv[tt][cl] - kv) * beta;
            float op[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < RPL; r++) {
                s[r] += kn[r] * delta;
                op[r & 3] += s[r] * qn[r];
            }
            float o = (op[0] + op[1]) + (op[2] + op[3]);
            o += OI_DPP(o, 0xB1);
            o += OI_DPP(o, 0x4E);
            o += dpp_mirror8(o);
            o += OI_DPP(o, 0x140);
            if (rg == 0) a.o[(size_t)(tb + tt) * VD + vh * HV + j] = o;
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) S[(size_t)(i0 + r) * HV + j] = s[r];
}

// The chunked form of the delta rule (the math of the reference's
// chunked_delta, qwen3_5/metal.odin:416-468): per chunk of C tokens, with the
// chunk's entry state S fixed, c[t] = sum of the log decays up to t,
//   d_t = beta_t v_t - beta_t e^{c[t]} S^T k_t - sum_{i<t} beta_t e^{c[t]-c[i]} (k_t.k_i) d_i
//   o_t = e^{c[t]} S^T q_t + sum_{i<=t} e^{c[t]-c[i]} (q_t.k_i) d_i
//   S'  = e^{c[C-1]} S + sum_i e^{c[C-1]-c[i]} k_i d_i^T.
// The decay ratios are differences of log sums (the reference divides
// running products, which gives 0/0 once a chunk's product underflows).
// Same grid and lane layout as pf_dn_delta_kernel: S^T k_t and S^T q_t of
// all the chunk's tokens are independent products (DPP sums over the 8 row
// groups), the substitution runs in one lane per column, the state update is
// one rank-C product per lane.
template <int HK, int HV, int C>
__global__ __launch_bounds__(WG) void pf_dn_chunk_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int RG = 8, RPL = HK / RG;
    static_assert(RPL == 16 && HV % 32 == 0, "head shape");
    __shared__ __attribute__((aligned(16))) float sq[C][HK];
    __shared__ __attribute__((aligned(16))) float sk[C][HK];
    __shared__ float sv[C][32];
    __shared__ float sbeta[C], slc[C];
    __shared__ float lm[C][C + 1], om[C][C + 1];  // beta_t e^{c[t]-c[i]} k_t.k_i (i < t); e^{c[t]-c[i]} q_t.k_i (i <= t)
    __shared__ float sik[32][C], siq[32][C], dd[32][C];
    const int vh = blockIdx.x, kh = vh % a.n_kh, c0 = (int)blockIdx.y * 32;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int cl = wave * 8 + (lane >> 3), rg = lane & 7, j = c0 + cl, i0 = rg * RPL;
    const int KD = a.n_kh * HK, CD = 2 * KD + a.n_vh * HV, VD = a.n_vh * HV;
    float *S = a.state + (size_t)vh * HK * HV;
    float s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) s[r] = S[(size_t)(i0 + r) * HV + j];
    for (int tb = 0; tb < a.T; tb += C) {
        const int nb = min(C, a.T - tb);
        __syncthreads();  // the previous chunk's LDS reads are done
        for (int idx = threadIdx.x; idx < nb * 2 * HK; idx += WG) {
            const int tt = idx / (2 * HK), e = idx % (2 * HK), ee = e % HK;
            const float val = a.qk[(size_t)(tb + tt) * 2 * KD + (e < HK ? 0 : KD) + kh * HK + ee];
            (e < HK ? sq : sk)[tt][ee] = val;
        }
        for (int idx = threadIdx.x; idx < nb * 32; idx += WG) {
            const int tt = idx / 32, cc = idx % 32;
            sv[tt][cc] = a.conv_out[(size_t)(tb + tt) * CD + 2 * KD + vh * HV + c0 + cc];
        }
        if (threadIdx.x < nb) {  // beta, and the running sum of the log decays
            const int t = threadIdx.x;
            sbeta[t] = a.gates[(size_t)(tb + t) * 3 * a.n_vh + vh];
            float c = 0.f;
            for (int i = 0; i <= t; i++) c += a.gates[(size_t)(tb + i) * 3 * a.n_vh + 2 * a.n_vh + vh];
            slc[t] = c;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < nb * nb; idx += WG) {  // the chunk's k.k and q.k products
            const int t = idx / nb, i = idx % nb;
            float dk = 0.f, dq = 0.f;
            if (i <= t) {
                const float4 *ki = (const float4 *)sk[i], *kt = (const float4 *)sk[t], *qt = (const float4 *)sq[t];
                for (int c4 = 0; c4 < HK / 4; c4++) {
                    const float4 x = ki[c4], y = kt[c4], z = qt[c4];
                    dk += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
                    dq += x.x * z.x + x.y * z.y + x.z * z.z + x.w * z.w;
                }
            }
            const float ratio = i < t ? expf(slc[t] - slc[i]) : 1.0f;
            lm[t][i] = i < t ? sbeta[t] * ratio * dk : 0.f;
            om[t][i] = i <= t ? ratio * dq : 0.f;
        }
        // S^T k_t and S^T q_t of every token of the chunk (S the entry state)
        for (int t = 0; t < nb; t++) {
            const float4 *k4 = (const float4 *)&sk[t][i0], *q4 = (const float4 *)&sq[t][i0];
            float pk = 0.f, pq = 0.f;
#pragma unroll
            for (int c4 = 0; c4 < RPL / 4; c4++) {
                const float4 kk = k4[c4], qq = q4[c4];
                pk += s[4 * c4] * kk.x + s[4 * c4 + 1] * kk.y + s[4 * c4 + 2] * kk.z + s[4 * c4 + 3] * kk.w;
                pq += s[4 * c4] * qq.x + s[4 * c4 + 1] * qq.y + s[4 * c4 + 2] * qq.z + s[4 * c4 + 3] * qq.w;
            }
            pk += OI_DPP(pk, 0xB1);
            pk += OI_DPP(pk, 0x4E);
            pk += dpp_mirror8(pk);
            pq += OI_DPP(pq, 0xB1);
            pq += OI_DPP(pq, 0x4E);
            pq += dpp_mirror8(pq);
            if (rg == 0) {
                sik[cl][t] = pk;
                siq[cl][t] = pq;
            }
        }
        __syncthreads();
        if (rg == 0) {  // forward substitution and the outputs, one lane per column
            for (int t = 0; t < nb; t++) {
                const float ec = expf(slc[t]);
                float d = sbeta[t] * sv[t][cl] - sbeta[t] * ec * sik[cl][t];
                for (int i = 0; i < t; i++) d -= lm[t][i] * dd[cl][i];
                dd[cl][t] = d;
                float o = ec * siq[cl][t];
                for (int i = 0; i <= t; i++) o += om[t][i] * dd[cl][i];
                a.o[(size_t)(tb + t) * VD + vh * HV + j] = o;
            }
        }
        __syncthreads();
        const float lcC = slc[nb - 1], ecC = expf(lcC);
#pragma unroll
        for (int r = 0; r < RPL; r++) s[r] *= ecC;
        for (int i = 0; i < nb; i++) {
            const float f = expf(lcC - slc[i]), di = dd[cl][i];
            const float4 *k4 = (const float4 *)&sk[i][i0];
#pragma unroll
            for (int c4 = 0; c4 < RPL / 4; c4++) {
                const float4 kk = k4[c4];
                s[4 * c4] += (f * kk.x) * di;
                s[4 * c4 + 1] += (f * kk.y) * di;
                s[4 * c4 + 2] += (f * kk.z) * di;
                s[4 * c4 + 3] += (f * kk.w) * di;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) S[(size_t)(i0 + r) * HV + j] = s[r];
}

// ---- the chunked delta rule on the matrix cores (chunks of 64 tokens) ----
//
// The same math as pf_dn_chunk_kernel in matrix form.  Per value head and
// chunk, with K, Q [64][hk] (q already scaled), V [64][hv], c the running sum
// of the log decays, G_t = e^{c_t}, F_t = e^{c_63 - c_t} (padded tokens past
// the end of the prompt have k = q = v = 0, beta = 0 and log decay 0):
//   L_ti = beta_t e^{c_t - c_i} k_t.k_i (i < t)    M_ti = e^{c_t - c_i} q_t.k_i (i <= t)
//   T = (I + L)^-1,  Tb = T diag(beta)
//   X = V - diag(G) K S,  D = Tb X,  O = diag(G) Q S + M D
//   S' = G_63 S + (diag(F) K)^T D
// (I + L) D = diag(beta) X is the forward substitution of the token form.
// pf_dc_prep_kernel forms Tb, M and c per (value head, chunk) -- they do not
// depend on the state, so every chunk of the call runs at once; the inverse
// is blocked by 16: the diagonal blocks by substitution (a lane per column),
// then T_ba = -T_bb sum_{m=a}^{b-1} L_bm T_ma on the matrix cores.
// pf_dc_state_kernel carries one value head's state through the chunks, a
// workgroup per 32 state columns.  Every product is v_mfma_f32_16x16x4_f32
// (f32 operands, f32 sums): D[16][16] += A[16][4] B[4][16], lane l giving
// A[l % 16][kk] and B[kk][l % 16] for kk = l / 16 and holding
// D[4 (l / 16) + e][l % 16].  Which physical index of the contraction an
// instruction's kk stands for is free as long as A and B agree; it is chosen
// so that a lane's operands over consecutive instructions are consecutive in
// LDS (one 16-byte read per four instructions, all issued before the first).
constexpr int DC = 64;         // tokens per chunk
constexpr int DC_CB = 32;      // state columns per workgroup of pf_dc_state_kernel
constexpr int DC_WG = 512;     // threads of both kernels (two waves per SIMD)
constexpr int DC_WAVES = DC_WG / WAVE;
typedef float dc_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ dc_f32x4 dc_mfma(float a, float b, dc_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// Four instructions over a lane's four consecutive operands, into four
// independent accumulators: a chain of dependent matrix instructions waits
// for each result, four chains keep the matrix core busy.
__device__ __forceinline__ void dc_mfma4(float4 a, float4 b, dc_f32x4 (&c)[4]) {
    c[0] = dc_mfma(a.x, b.x, c[0]);
    c[1] = dc_mfma(a.y, b.y, c[1]);
    c[2] = dc_mfma(a.z, b.z, c[2]);
    c[3] = dc_mfma(a.w, b.w, c[3]);
}
__device__ __forceinline__ dc_f32x4 dc_sum4(const dc_f32x4 (&c)[4]) { return (c[0] + c[1]) + (c[2] + c[3]); }

// x = hi + lo in halves (to ~2^-22 of x) for the products of l2-normalised
// rows, whose elements lie in [-1, 1]: hi.hi + hi.lo + lo.hi on
// v_mfma_f32_16x16x32_f16 (exact half products, f32 sums), lo.lo dropped.
// Lane l gives A[l % 16][8 (l / 16) + e] and B[8 (l / 16) + e][l % 16], e < 8.
typedef _Float16 dc_h8 __attribute__((ext_vector_type(8)));
#define DC_ZERO4 {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}

// [n_vh][n_chunks] of DC_REC floats: Tb [64][64], M [64][64] (lower 16-blocks
// only), c [64] (the running sums of the log decays), the chunk's q | k rows
// [64][2 hk] (written only in the records of value heads vh < n_kh, i.e. of
// k head vh), and the value head's v in column blocks [hv / 16][64][16]: the
// state kernel reads each of its inputs as one contiguous run (q, k and v
// rows in the projection layout are 32 KB apart, so the same few memory
// channels would serve all of a chunk's rows)
constexpr int DC_C = 2 * DC * DC, DC_QKO = DC_C + DC, DC_VO = DC_QKO + DC * 2 * 128;
constexpr int DC_REC = DC_VO + DC * 128;
size_t pf_dc_scratch_floats(int n_vh, int T) { return (size_t)n_vh * ((T + DC - 1) / DC) * DC_REC; }

// inclusive prefix sum over a wave (lane order)
__device__ __forceinline__ float dc_wave_scan(float v) {
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const float o = __shfl_up(v, d, WAVE);
        if (lane >= d) v += o;
    }
    return v;
}

// lower 16-blocks (bi, bj), bj <= bi, in row order
__device__ __forceinline__ void dc_lower_block(int p, int &bi, int &bj) {
    bi = p >= 6 ? 3 : p >= 3 ? 2 : p >= 1 ? 1 : 0;
    bj = p - bi * (bi + 1) / 2;
}

// The chunk's q and k rows of k head kh (zeros past nb) as float4 pieces:
// loaded into registers all at once, then stored to LDS rows of pitch HK + 4
// (a loop that stores each piece as it arrives waits for every load in turn).
// RAW: the conv output's q and k (rows of conv_dim), not yet normalised.
constexpr int DC_QK4 = DC * 128 / 2 / DC_WG;
template <int HK, bool RAW = false>
__device__ __forceinline__ void dc_load_qk(const PfDnArgs &a, dc_f32x4 (&v)[DC_QK4], int tb, int nb, int kh) {
    static_assert(DC * HK / 2 == DC_QK4 * DC_WG, "staging shape");
    const int KD = a.n_kh * HK, pitch = RAW ? 2 * KD + a.n_vh * a.hv : 2 * KD;
    const float *src = RAW ? a.conv_out : a.qk;
#pragma unroll
    for (int i = 0; i < DC_QK4; i++) {
        const int idx = threadIdx.x + i * DC_WG, t = idx / (HK / 2), e4 = idx % (HK / 2);
        const int side = e4 / (HK / 4), ee = 4 * (e4 % (HK / 4));
        v[i] = t < nb ? *(const dc_f32x4 *)(src + (size_t)(tb + t) * pitch + side * KD + kh * HK + ee)
                      : dc_f32x4{0.f, 0.f, 0.f, 0.f};
    }
}
// pf_dn_prep_kernel's l2norm of the loaded raw rows, in registers: thread
// piece i is token tb + idx / (HK / 2) of wave-half side (the 32 lanes of a
// half hold one token's q or k row, four elements each); q also times
// 1/sqrt(HK).  (The row sums run in another order than the prep kernel's.)
template <int HK>
__device__ __forceinline__ void dc_l2norm_qk(dc_f32x4 (&v)[DC_QK4]) {
#pragma clang fp contract(off)
    static_assert(HK / 4 == 32, "a q or k row is half a wave");
    const bool isq = (threadIdx.x & (WAVE - 1)) < 32;
#pragma unroll
    for (int i = 0; i < DC_QK4; i++) {
        float ss = v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, WAVE);
        const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-6f);
#pragma unroll
        for (int e = 0; e < 4; e++) v[i][e] = isq ? v[i][e] * inv * (1.0f / sqrtf((float)HK)) : v[i][e] * inv;
    }
}
template <int HK>
__device__ __forceinline__ void dc_store_qk(const dc_f32x4 (&v)[DC_QK4], float (*sq)[HK + 4], float (*sk)[HK + 4]) {
#pragma unroll
    for (int i = 0; i < DC_QK4; i++) {
        const int idx = threadIdx.x + i * DC_WG, t = idx / (HK / 2), e4 = idx % (HK / 2);
        const int side = e4 / (HK / 4), ee = 4 * (e4 % (HK / 4));
        *(dc_f32x4 *)&(side ? sk : sq)[t][ee] = v[i];
    }
}

// (I + L_bb)^-1 of diagonal block b (one wave; lane < 16 = column) by
// substitution, each row's sum in four fused chains (the critical path)
template <int LP>
__device__ __forceinline__ void dc_invert_diag(const float (*sl)[LP], float (*stt)[LP], int b, int lane) {
    if (lane >= 16) return;
    const int o = 16 * b, j = lane;
    float col[16];
#pragma unroll
    for (int t = 0; t < 16; t++) {
        float p4[4] = {t == j ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < t; i++) p4[i & 3] = fmaf(-sl[o + t][o + i], col[i], p4[i & 3]);
        col[t] = (p4[0] + p4[1]) + (p4[2] + p4[3]);
    }
#pragma unroll
    for (int t = 0; t < 16; t++) stt[o + t][o + j] = col[t];
}

// The blocks below the diagonal, block row by block row (called by every
// thread of the workgroup after the diagonal blocks; ends with a barrier):
// T_ba = -T_bb sum_{m=a}^{b-1} L_bm T_ma, waves a < b one block each.
template <int LP>
__device__ __forceinline__ void dc_invert_below(const float (*sl)[LP], float (*stt)[LP], float (*sz)[16][17], int wave,
                                                int r, int kq) {
    for (int b = 1; b < 4; b++) {
        const int ab = wave;
        if (ab < b) {
            dc_f32x4 zc[4] = DC_ZERO4;
            for (int m = ab; m < b; m++)
#pragma unroll
                for (int k0 = 0; k0 < 16; k0 += 4)
                    zc[k0 / 4] = dc_mfma(sl[16 * b + r][16 * m + k0 + kq], stt[16 * m + k0 + kq][16 * ab + r], zc[k0 / 4]);
            const dc_f32x4 z = dc_sum4(zc);
#pragma unroll
            for (int e = 0; e < 4; e++) sz[wave][4 * kq + e][r] = z[e];
            dc_f32x4 yc[4] = DC_ZERO4;
#pragma unroll
            for (int k0 = 0; k0 < 16; k0 += 4)
                yc[k0 / 4] = dc_mfma(stt[16 * b + r][16 * b + k0 + kq], sz[wave][k0 + kq][r], yc[k0 / 4]);
            const dc_f32x4 y = dc_sum4(yc);
#pragma unroll
            for (int e = 0; e < 4; e++) stt[16 * b + 4 * kq + e][16 * ab + r] = -y[e];
        }
        __syncthreads();
    }
}

template <int HK>
__global__ __launch_bounds__(DC_WG) void pf_dc_prep_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int HP = HK + 8;  // row pitch in halves: 16-byte aligned rows, 4 banks apart
    static_assert(HK % 128 == 0, "k rows in four 32-element lane slices");
    // q and k rows split once into f16 hi and lo parts, as the matrix cores take them
    __shared__ __attribute__((aligned(16))) _Float16 skh[DC][HP], skl[DC][HP], sqh[DC][HP], sql[DC][HP];
    __shared__ float sl[DC][DC + 1], stt[DC][DC + 1], sz[4][16][17];
    __shared__ float slg[DC], slc[DC], sbeta[DC];
    const int vh = blockIdx.x, ch = blockIdx.y, nch = (int)gridDim.y, kh = vh % a.n_kh;
    const int tb = ch * DC, nb = min(DC, a.T - tb);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, r = lane & 15, kq = lane >> 4;
    float *out = a.dc + ((size_t)vh * nch + ch) * DC_REC;
    {  // q and k rows, v rows and the gates: every load issued before any is stored
        static_assert(HK == 128, "record layout");
        constexpr int V4 = DC * 128 / 4 / DC_WG;
        const int CD = 2 * a.n_kh * HK + a.n_vh * 128;
        dc_f32x4 qk4[DC_QK4], v4[V4];
        dc_load_qk<HK>(a, qk4, tb, nb, kh);
#pragma unroll
        for (int i = 0; i < V4; i++) {
            const int idx = threadIdx.x + i * DC_WG, t = idx / 32, c4 = 4 * (idx % 32);
            v4[i] = t < nb ? *(const dc_f32x4 *)(a.conv_out + (size_t)(tb + t) * CD + 2 * a.n_kh * HK + vh * 128 + c4)
                           : dc_f32x4{0.f, 0.f, 0.f, 0.f};
        }
        const int t = threadIdx.x;
        const float b = t < nb ? a.gates[(size_t)(tb + t) * 3 * a.n_vh + vh] : 0.f;
        const float g = t < nb ? a.gates[(size_t)(tb + t) * 3 * a.n_vh + 2 * a.n_vh + vh] : 0.f;
#pragma unroll
        for (int i = 0; i < DC_QK4; i++) {
            const int idx = threadIdx.x + i * DC_WG, tt = idx / (HK / 2), e4 = idx % (HK / 2);
            const int side = e4 / (HK / 4), ee = 4 * (e4 % (HK / 4));
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            h4 hi, lo;
#pragma unroll
            for (int x = 0; x < 4; x++) {
                hi[x] = (_Float16)qk4[i][x];
                lo[x] = (_Float16)(qk4[i][x] - (float)hi[x]);
            }
            *(h4 *)&(side ? skh : sqh)[tt][ee] = hi;
            *(h4 *)&(side ? skl : sql)[tt][ee] = lo;
        }
        if (vh < a.n_kh)  // this record carries k head vh's q | k rows
#pragma unroll
            for (int i = 0; i < DC_QK4; i++) *(dc_f32x4 *)(out + DC_QKO + 4 * (threadIdx.x + i * DC_WG)) = qk4[i];
#pragma unroll
        for (int i = 0; i < V4; i++) {
            const int idx = threadIdx.x + i * DC_WG, tt = idx / 32, c4 = 4 * (idx % 32);
            *(dc_f32x4 *)(out + DC_VO + (c4 / 16) * DC * 16 + tt * 16 + c4 % 16) = v4[i];
        }
        if (t < DC) {
            sbeta[t] = b;
            slg[t] = g;
        }
    }
    __syncthreads();
    if (wave == 0) {  // the running sum of the log decays (kept for the state kernel)
        const float c = dc_wave_scan(slg[lane]);
        slc[lane] = c;
        out[DC_C + lane] = c;
    }
    __syncthreads();
    // k_t.k_i (then q_t.k_i) over the lower 16-blocks, 10 tiles each: lane
    // slice s of a row is its elements 32 s + 8 kq .. + 7
    auto tile = [&](bool isq, int p) {
        int bi, bj;
        dc_lower_block(p, bi, bj);
        const _Float16 *xh = (isq ? sqh : skh)[16 * bi + r] + 8 * kq, *xl = (isq ? sql : skl)[16 * bi + r] + 8 * kq;
        const _Float16 *yh = skh[16 * bj + r] + 8 * kq, *yl = skl[16 * bj + r] + 8 * kq;
        dc_h8 ah[HK / 32], al[HK / 32], bh[HK / 32], bl[HK / 32];
#pragma unroll
        for (int m = 0; m < HK / 32; m++) {
            ah[m] = *(const dc_h8 *)(xh + 32 * m);
            al[m] = *(const dc_h8 *)(xl + 32 * m);
            bh[m] = *(const dc_h8 *)(yh + 32 * m);
            bl[m] = *(const dc_h8 *)(yl + 32 * m);
        }
        float ct[4], bt[4];  // the epilogue's operands, read while the products run
#pragma unroll
        for (int e = 0; e < 4; e++) {
            ct[e] = slc[16 * bi + 4 * kq + e];
            bt[e] = sbeta[16 * bi + 4 * kq + e];
        }
        const float ci = slc[16 * bj + r];
        dc_f32x4 c3[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int m = 0; m < HK / 32; m++) {
            c3[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[m], bh[m], c3[0], 0, 0, 0);
            c3[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[m], bl[m], c3[1], 0, 0, 0);
            c3[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[m], bh[m], c3[2], 0, 0, 0);
        }
        const dc_f32x4 acc = c3[0] + (c3[1] + c3[2]);
        float val[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {  // selects, not branches (exp of a positive difference is discarded)
            const int t = 16 * bi + 4 * kq + e, i = 16 * bj + r;
            const float ratio = expf(ct[e] - ci);
            val[e] = isq ? (i <= t ? ratio * acc[e] : 0.f) : (i < t ? bt[e] * ratio * acc[e] : 0.f);
        }
        if (isq) {
#pragma unroll
            for (int e = 0; e < 4; e++) out[DC * DC + (16 * bi + 4 * kq + e) * DC + 16 * bj + r] = val[e];
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) sl[16 * bi + 4 * kq + e][16 * bj + r] = val[e];
        }
    };
    for (int p = wave; p < 10; p += DC_WAVES) tile(false, p);
    __syncthreads();
    if (wave < 4) {
        dc_invert_diag<DC + 1>(sl, stt, wave, lane);
    } else {  // meanwhile the q.k tiles, which the inverse does not need
        for (int p = wave - 4; p < 10; p += 4) tile(true, p);
    }
    __syncthreads();
    dc_invert_below<DC + 1>(sl, stt, sz, wave, r, kq);
    for (int idx = threadIdx.x; idx < DC * DC; idx += DC_WG) {  // Tb = T diag(beta), lower blocks
        const int t = idx / DC, i = idx % DC;
        if (i / 16 <= t / 16) out[idx] = stt[t][i] * sbeta[i];
    }
}

// The state kernel's inputs of one chunk, held in registers from the load
// (issued while the previous chunk is computed) to the LDS stores: q / k rows,
// Tb and M (whole 64 x 64; only the lower blocks are read), the workgroup's
// v columns and c.
constexpr int DC_TM4 = DC * DC / 4 / DC_WG, DC_V4 = DC * DC_CB / 4 / DC_WG;
static_assert(DC_TM4 * DC_WG * 4 == DC * DC && DC_V4 * DC_WG * 4 == DC * DC_CB, "staging shape");
struct DcStage {
    dc_f32x4 qk4[DC_QK4], tb4[DC_TM4], m4[DC_TM4], v4[DC_V4];
    float lg;
};
__device__ __forceinline__ void dc_stage_load(const PfDnArgs &a, DcStage &g, int vh, int kh, int ch, int nch, int c0) {
    const float *tm = a.dc + ((size_t)vh * nch + ch) * DC_REC;
    const float *qkr = a.dc + ((size_t)kh * nch + ch) * DC_REC + DC_QKO;
#pragma unroll
    for (int i = 0; i < DC_QK4; i++) g.qk4[i] = *(const dc_f32x4 *)(qkr + 4 * (threadIdx.x + i * DC_WG));
#pragma unroll
    for (int i = 0; i < DC_TM4; i++) {
        g.tb4[i] = *(const dc_f32x4 *)(tm + 4 * (threadIdx.x + i * DC_WG));
        g.m4[i] = *(const dc_f32x4 *)(tm + DC * DC + 4 * (threadIdx.x + i * DC_WG));
    }
#pragma unroll
    for (int i = 0; i < DC_V4; i++) {  // the record's 16-column blocks c0 / 16 and c0 / 16 + 1, [64][16] each
        const int idx = threadIdx.x + i * DC_WG, blk = idx / (DC * 4), w4 = idx % (DC * 4);
        g.v4[i] = *(const dc_f32x4 *)(tm + DC_VO + (c0 / 16 + blk) * DC * 16 + 4 * w4);
    }
    g.lg = threadIdx.x < DC ? tm[DC_C + threadIdx.x] : 0.f;
}

// A workgroup carries 32 state columns (two 16-column tiles).  Waves 0-3
// form K S for token rows 16 w (then X), waves 4-7 Q S for token rows
// 16 (w - 4) (then O); wave w forms D for token rows 16 (w / 2), column tile
// w % 2; every wave owns state rows 16 w .. 16 w + 15 of both column tiles
// (8 values per lane for the whole prompt).  X, D and the state are kept
// transposed in LDS ([column][row]) so that a lane reads its B operands 16
// bytes at a time.
template <int HK, int HV>
__global__ __launch_bounds__(DC_WG) void pf_dc_state_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int KP = HK + 4, TP = DC + 4;
    static_assert(HK == 16 * DC_WAVES && HV % DC_CB == 0 && DC_CB == 32, "a state row tile per wave");
    __shared__ __attribute__((aligned(16))) float sk[DC][KP];
    __shared__ __attribute__((aligned(16))) float sq[DC][KP];
    __shared__ __attribute__((aligned(16))) float stb[DC][TP];
    __shared__ __attribute__((aligned(16))) float sm[DC][TP];
    __shared__ __attribute__((aligned(16))) float sst[DC_CB][KP];  // S^T
    __shared__ __attribute__((aligned(16))) float sxt[DC_CB][TP];  // X^T
    __shared__ __attribute__((aligned(16))) float sdt[DC_CB][TP];  // D^T
    __shared__ __attribute__((aligned(16))) float sv[DC][DC_CB];
    __shared__ float slg[DC];  // c
    const int vh = blockIdx.x, kh = vh % a.n_kh, c0 = (int)blockIdx.y * DC_CB, nch = (a.T + DC - 1) / DC;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, r = lane & 15, kq = lane >> 4;
    const int VD = a.n_vh * HV;
    float *S = a.state + (size_t)vh * HK * HV;
    dc_f32x4 st[2];  // state rows 16 wave + 4 kq + e, columns c0 + 16 ct + r
#pragma unroll
    for (int ct = 0; ct < 2; ct++)
#pragma unroll
        for (int e = 0; e < 4; e++) st[ct][e] = S[(size_t)(16 * wave + 4 * kq + e) * HV + c0 + 16 * ct + r];
    // the inputs of chunk ch + 1 are loaded into registers at the start of
    // chunk ch and stored to LDS after its last LDS read (so no register array
    // lives across iterations)
    auto put = [&](const DcStage &g) __attribute__((always_inline)) {
        dc_store_qk<HK>(g.qk4, sq, sk);
#pragma unroll
        for (int i = 0; i < DC_TM4; i++) {
            const int idx = 4 * (threadIdx.x + i * DC_WG);
            *(dc_f32x4 *)&stb[idx / DC][idx % DC] = g.tb4[i];
            *(dc_f32x4 *)&sm[idx / DC][idx % DC] = g.m4[i];
        }
#pragma unroll
        for (int i = 0; i < DC_V4; i++) {
            const int idx = threadIdx.x + i * DC_WG, blk = idx / (DC * 4), w4 = idx % (DC * 4);
            *(dc_f32x4 *)&sv[w4 / 4][16 * blk + 4 * (w4 % 4)] = g.v4[i];
        }
        if (threadIdx.x < DC) slg[threadIdx.x] = g.lg;
#pragma unroll
        for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int e = 0; e < 4; e++) sst[16 * ct + r][16 * wave + 4 * kq + e] = st[ct][e];
    };
    {
        DcStage g;
        dc_stage_load(a, g, vh, kh, 0, nch, c0);
        put(g);
    }
    for (int ch = 0; ch < nch; ch++) {
        const int tb = ch * DC, nb = min(DC, a.T - tb);
        DcStage g;  // chunk ch + 1
        if (ch + 1 < nch) dc_stage_load(a, g, vh, kh, ch + 1, nch, c0);
        __syncthreads();
        // K S (waves 0-3) or Q S (waves 4-7) for token rows 16 rt, both
        // column tiles; instruction 4 m + x of a lane sums state row 32 kq + 4 m + x
        const int rt = wave & 3;
        dc_f32x4 u[2];
        {
            const float *xr = (wave < 4 ? sk : sq)[16 * rt + r] + 32 * kq;
            float4 xa[8];
#pragma unroll
            for (int m = 0; m < 8; m++) xa[m] = *(const float4 *)(xr + 4 * m);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                const float *yr = sst[16 * ct + r] + 32 * kq;
                float4 yb[8];
#pragma unroll
                for (int m = 0; m < 8; m++) yb[m] = *(const float4 *)(yr + 4 * m);
                dc_f32x4 uc[4] = DC_ZERO4;
#pragma unroll
                for (int m = 0; m < 8; m++) dc_mfma4(xa[m], yb[m], uc);
                u[ct] = dc_sum4(uc);
            }
        }
        if (wave < 4)  // X = V - G (K S), transposed
#pragma unroll
            for (int ct = 0; ct < 2; ct++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 16 * rt + 4 * kq + e;
                    sxt[16 * ct + r][t] = sv[t][16 * ct + r] - expf(slg[t]) * u[ct][e];
                }
        __syncthreads();
        {  // D = Tb X for token rows 16 (wave / 2), column tile wave % 2:
           // instruction 4 bj + x sums token 16 bj + 4 kq + x
            const int dr = wave >> 1, dcol = 16 * (wave & 1) + r;
            dc_f32x4 dc[4] = DC_ZERO4;
            for (int bj = 0; bj <= dr; bj++)
                dc_mfma4(*(const float4 *)&stb[16 * dr + r][16 * bj + 4 * kq],
                         *(const float4 *)&sxt[dcol][16 * bj + 4 * kq], dc);
            const dc_f32x4 d = dc_sum4(dc);
#pragma unroll
            for (int e = 0; e < 4; e++) sdt[dcol][16 * dr + 4 * kq + e] = d[e];
        }
        __syncthreads();
        if (wave >= 4) {  // O = G (Q S) + M D for token rows 16 rt, both column tiles
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                dc_f32x4 oc[4] = DC_ZERO4;
                for (int bj = 0; bj <= rt; bj++)
                    dc_mfma4(*(const float4 *)&sm[16 * rt + r][16 * bj + 4 * kq],
                             *(const float4 *)&sdt[16 * ct + r][16 * bj + 4 * kq], oc);
                const dc_f32x4 o = dc_sum4(oc);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 16 * rt + 4 * kq + e;
                    if (t < nb) a.o[(size_t)(tb + t) * VD + vh * HV + c0 + 16 * ct + r] = expf(slg[t]) * u[ct][e] + o[e];
                }
            }
        }
        {  // S' = G_63 S + (diag(F) K)^T D for state rows 16 wave: instruction
           // 4 m + x sums token 16 m + 4 kq + x
            const float c63 = slg[DC - 1];
            float4 ka[4];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int k0 = 16 * m + 4 * kq;
                ka[m].x = expf(c63 - slg[k0]) * sk[k0][16 * wave + r];
                ka[m].y = expf(c63 - slg[k0 + 1]) * sk[k0 + 1][16 * wave + r];
                ka[m].z = expf(c63 - slg[k0 + 2]) * sk[k0 + 2][16 * wave + r];
                ka[m].w = expf(c63 - slg[k0 + 3]) * sk[k0 + 3][16 * wave + r];
            }
            const float g63 = expf(c63);
#pragma unroll
            for (int ct = 0; ct < 2; ct++) {
                dc_f32x4 sc[4] = DC_ZERO4;
                sc[0] = st[ct] * g63;
#pragma unroll
                for (int m = 0; m < 4; m++) dc_mfma4(ka[m], *(const float4 *)&sdt[16 * ct + r][16 * m + 4 * kq], sc);
                st[ct] = dc_sum4(sc);
            }
        }
        __syncthreads();  // every read of this chunk's LDS inputs is done
        if (ch + 1 < nch) put(g);
    }
#pragma unroll
    for (int ct = 0; ct < 2; ct++)
#pragma unroll
        for (int e = 0; e < 4; e++) S[(size_t)(16 * wave + 4 * kq + e) * HV + c0 + 16 * ct + r] = st[ct][e];
}

// A prompt of at most 64 tokens is one chunk: pf_dc_single_kernel does the
// prep kernel's work and the state kernel's in one launch, per (value head,
// 32 state columns), with every intermediate in LDS (the four workgroups of
// a value head each form its L, M and inverse).  The state-free products
// k.k and q.k run in f32 here; K S and Q S, which do not depend on the
// inverse, run while waves 0-3 invert the diagonal blocks.
template <int HK, int HV>
__global__ __launch_bounds__(DC_WG) void pf_dc_single_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int KP = HK + 4, TP = DC + 4;
    static_assert(HK == 16 * DC_WAVES && HV % DC_CB == 0 && DC_CB == 32, "a state row tile per wave");
    __shared__ __attribute__((aligned(16))) float sk[DC][KP];
    __shared__ __attribute__((aligned(16))) float sq[DC][KP];
    __shared__ __attribute__((aligned(16))) float sl[DC][TP];   // L; then X^T and D^T
    __shared__ __attribute__((aligned(16))) float stt[DC][TP];  // T
    __shared__ __attribute__((aligned(16))) float sm[DC][TP];   // M
    __shared__ __attribute__((aligned(16))) float sst[DC_CB][KP];  // S^T
    __shared__ __attribute__((aligned(16))) float sv[DC][DC_CB];
    __shared__ float sz[4][16][17], slg[DC], slc[DC];
    __shared__ __attribute__((aligned(16))) float sbeta[DC];  // read 16 bytes at a time
    static_assert(2 * DC_CB <= DC, "X^T and D^T fit where L was");
    float(*sxt)[TP] = sl;
    float(*sdt)[TP] = sl + DC_CB;
    const int vh = blockIdx.x, kh = vh % a.n_kh, c0 = (int)blockIdx.y * DC_CB, nb = a.T;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, r = lane & 15, kq = lane >> 4;
    const int KD = a.n_kh * HK, CD = 2 * KD + a.n_vh * HV, VD = a.n_vh * HV;
    float *S = a.state + (size_t)vh * HK * HV;
    dc_f32x4 st[2];  // state rows 16 wave + 4 kq + e, columns c0 + 16 ct + r
    {  // every load issued before any is stored
        constexpr int V4 = DC * DC_CB / 4 / DC_WG;
        static_assert(V4 == 1, "one v piece per thread");
        // (this kernel also does pf_dn_prep_kernel's work for its heads: the
        // conv output's q / k rows l2-normalised here, the gates from the b
        // and a projections)
        dc_f32x4 qk4[DC_QK4];
        dc_load_qk<HK, true>(a, qk4, 0, nb, kh);
        const int vt = threadIdx.x / (DC_CB / 4), vc = 4 * (threadIdx.x % (DC_CB / 4));
        const dc_f32x4 v4 = vt < nb ? *(const dc_f32x4 *)(a.conv_out + (size_t)vt * CD + 2 * KD + vh * HV + c0 + vc)
                                    : dc_f32x4{0.f, 0.f, 0.f, 0.f};
        const int t = threadIdx.x;
        float b = 0.f, g = 0.f;
        if (t < nb) {
            const size_t slice = (size_t)a.T * a.n_vh, i = (size_t)t * a.n_vh + vh;
            const float bb = parts_at(a.b, a.bs, slice, i), av = parts_at(a.a, a.as, slice, i);
            g = a.a_decay[vh] * softplus_ref(av + a.dt_bias[vh]);  // log of the decay
            b = sigmoid_ref(bb);
        }
        dc_l2norm_qk<HK>(qk4);
#pragma unroll
        for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int e = 0; e < 4; e++) st[ct][e] = S[(size_t)(16 * wave + 4 * kq + e) * HV + c0 + 16 * ct + r];
        dc_store_qk<HK>(qk4, sq, sk);
        *(dc_f32x4 *)&sv[vt][vc] = v4;
        if (t < DC) {
            sbeta[t] = b;
            slg[t] = g;
        }
#pragma unroll
        for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int e = 0; e < 4; e++) sst[16 * ct + r][16 * wave + 4 * kq + e] = st[ct][e];
    }
    __syncthreads();
    if (wave == 0) slc[lane] = dc_wave_scan(slg[lane]);
    __syncthreads();
    // k_t.k_i (into L) or q_t.k_i (into M) of lower 16-block p; instruction
    // 4 m + x of a lane sums element 32 kq + 4 m + x of the rows
    auto tile = [&](bool isq, int p) __attribute__((always_inline)) {
        int bi, bj;
        dc_lower_block(p, bi, bj);
        const float *xr = (isq ? sq : sk)[16 * bi + r] + 32 * kq, *yr = sk[16 * bj + r] + 32 * kq;
        float4 xa[8], yb[8];
#pragma unroll
        for (int m = 0; m < 8; m++) {
            xa[m] = *(const float4 *)(xr + 4 * m);
            yb[m] = *(const float4 *)(yr + 4 * m);
        }
        float ct4[4], bt4[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            ct4[e] = slc[16 * bi + 4 * kq + e];
            bt4[e] = sbeta[16 * bi + 4 * kq + e];
        }
        const float ci = slc[16 * bj + r];
        dc_f32x4 c4[4] = DC_ZERO4;
#pragma unroll
        for (int m = 0; m < 8; m++) dc_mfma4(xa[m], yb[m], c4);
        const dc_f32x4 acc = dc_sum4(c4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = 16 * bi + 4 * kq + e, i = 16 * bj + r;
            const float ratio = expf(ct4[e] - ci);
            if (isq) sm[t][i] = i <= t ? ratio * acc[e] : 0.f;
            else sl[t][i] = i < t ? bt4[e] * ratio * acc[e] : 0.f;
        }
    };
    for (int p = wave; p < 10; p += DC_WAVES) tile(false, p);
    __syncthreads();
    if (wave < 4) dc_invert_diag<TP>(sl, stt, wave, lane);
    else
        for (int p = wave - 4; p < 10; p += 4) tile(true, p);
    // K S (waves 0-3) or Q S (waves 4-7) for token rows 16 rt, both column
    // tiles; instruction 4 m + x of a lane sums state row 32 kq + 4 m + x
    const int rt = wave & 3;
    dc_f32x4 u[2];
    {
        const float *xr = (wave < 4 ? sk : sq)[16 * rt + r] + 32 * kq;
        float4 xa[8];
#pragma unroll
        for (int m = 0; m < 8; m++) xa[m] = *(const float4 *)(xr + 4 * m);
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            const float *yr = sst[16 * ct + r] + 32 * kq;
            float4 yb[8];
#pragma unroll
            for (int m = 0; m < 8; m++) yb[m] = *(const float4 *)(yr + 4 * m);
            dc_f32x4 uc[4] = DC_ZERO4;
#pragma unroll
            for (int m = 0; m < 8; m++) dc_mfma4(xa[m], yb[m], uc);
            u[ct] = dc_sum4(uc);
        }
    }
    __syncthreads();
    dc_invert_below<TP>(sl, stt, sz, wave, r, kq);  // ends with a barrier: L is free
    if (wave < 4)  // X = V - G (K S), transposed
#pragma unroll
        for (int ct = 0; ct < 2; ct++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 16 * rt + 4 * kq + e;
                sxt[16 * ct + r][t] = sv[t][16 * ct + r] - expf(slc[t]) * u[ct][e];
            }
    __syncthreads();
    {  // D = T diag(beta) X for token rows 16 (wave / 2), column tile wave % 2
        const int dr = wave >> 1, dcol = 16 * (wave & 1) + r;
        dc_f32x4 dc[4] = DC_ZERO4;
        for (int bj = 0; bj <= dr; bj++) {
            const float4 tr = *(const float4 *)&stt[16 * dr + r][16 * bj + 4 * kq];
            const float4 bb = *(const float4 *)&sbeta[16 * bj + 4 * kq];
            dc_mfma4(float4{tr.x * bb.x, tr.y * bb.y, tr.z * bb.z, tr.w * bb.w},
                     *(const float4 *)&sxt[dcol][16 * bj + 4 * kq], dc);
        }
        const dc_f32x4 d = dc_sum4(dc);
#pragma unroll
        for (int e = 0; e < 4; e++) sdt[dcol][16 * dr + 4 * kq + e] = d[e];
    }
    __syncthreads();
    if (wave >= 4) {  // O = G (Q S) + M D for token rows 16 rt, both column tiles
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            dc_f32x4 oc[4] = DC_ZERO4;
            for (int bj = 0; bj <= rt; bj++)
                dc_mfma4(*(const float4 *)&sm[16 * rt + r][16 * bj + 4 * kq],
                         *(const float4 *)&sdt[16 * ct + r][16 * bj + 4 * kq], oc);
            const dc_f32x4 o = dc_sum4(oc);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 16 * rt + 4 * kq + e;
                if (t < nb) a.o[(size_t)t * VD + vh * HV + c0 + 16 * ct + r] = expf(slc[t]) * u[ct][e] + o[e];
            }
        }
    }
    {  // S' = G_63 S + (diag(F) K)^T D for state rows 16 wave
        const float c63 = slc[DC - 1];
        float4 ka[4];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int k0 = 16 * m + 4 * kq;
            ka[m].x = expf(c63 - slc[k0]) * sk[k0][16 * wave + r];
            ka[m].y = expf(c63 - slc[k0 + 1]) * sk[k0 + 1][16 * wave + r];
            ka[m].z = expf(c63 - slc[k0 + 2]) * sk[k0 + 2][16 * wave + r];
            ka[m].w = expf(c63 - slc[k0 + 3]) * sk[k0 + 3][16 * wave + r];
        }
        const float g63 = expf(c63);
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            dc_f32x4 sc[4] = DC_ZERO4;
            sc[0] = st[ct] * g63;
#pragma unroll
            for (int m = 0; m < 4; m++) dc_mfma4(ka[m], *(const float4 *)&sdt[16 * ct + r][16 * m + 4 * kq], sc);
            st[ct] = dc_sum4(sc);
#pragma unroll
            for (int e = 0; e < 4; e++) S[(size_t)(16 * wave + 4 * kq + e) * HV + c0 + 16 * ct + r] = st[ct][e];
        }
    }
}

// gated RMSNorm (qwen3_5/forward.odin:211-218): per token and value head, out =
// f16(norm_w[j] (inv o[j]) silu(z[j])), inv = 1 / sqrt(sum o^2 / hv + eps); z
// from the in_z projection's partial products.  Grid (T, ceil(n_vh / (4
// GN_NH))): each wave takes GN_NH heads, their o and z requested together.
constexpr int GN_NH = 2;
template <int HV>
__global__ __launch_bounds__(WG) void pf_dn_gnorm_kernel(PfDnArgs a) {
#pragma clang fp contract(off)
    constexpr int E = HV / WAVE, NH = GN_NH, NV = NH * E;  // dimensions per lane; heads per wave
    const int t = blockIdx.x, lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int vh0 = ((int)blockIdx.y * (WG / WAVE) + wave) * NH;
    if (vh0 >= a.n_vh) return;  // whole waves; no workgroup barrier below
    const int VD = a.n_vh * HV;
    // value v of the wave: head vh0 + v / E (clamped), dimension lane + 64 (v % E)
    auto at = [&](int v) { return (size_t)t * VD + min(vh0 + v / E, a.n_vh - 1) * HV + lane + WAVE * (v % E); };
    float o[NV], z[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) o[v] = a.o[at(v)];
    parts_gather(z, a.z, a.zs, (size_t)a.T * VD, at);
#pragma unroll
    for (int h = 0; h < NH; h++) {
        if (vh0 + h >= a.n_vh) break;  // uniform
        const int vh = vh0 + h;
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) ss += o[h * E + e] * o[h * E + e];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HV + a.eps);
#pragma unroll
        for (int e = 0; e < E; e++) {
            const int j = lane + WAVE * e;
            const float v = a.norm_w[j] * (inv * o[h * E + e]) * silu_ref(z[h * E + e]);
            if (a.out32) a.out32[(size_t)t * VD + vh * HV + j] = v;
            else a.out16[(size_t)t * VD + vh * HV + j] = f2h(v);
        }
    }
}

static unsigned nblk(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_pf_q35_qkv(const PfQ35Args &a, int head_dim, hipStream_t st) {
    if (a.rotary_dim < 0 || a.rotary_dim > head_dim || a.rotary_dim % 2) return hipErrorInvalidValue;
    const dim3 grid((unsigned)a.T, nblk(a.n_heads + 2 * a.n_kv_heads, WG / WAVE));
    if (head_dim == 128) hipLaunchKernelGGL(pf_q35_qkv_kernel<128>, grid, dim3(WG), 0, st, a);
    else if (head_dim == 256) hipLaunchKernelGGL(pf_q35_qkv_kernel<256>, grid, dim3(WG), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

bool pf_dn_supported(int hk, int hv, int kernel) { return hk == 128 && hv == 128 && kernel == 4; }

hipError_t launch_pf_deltanet(const PfDnArgs &a, hipStream_t st) {
    if (!pf_dn_supported(a.hk, a.hv, a.kernel) || a.T < a.kernel - 1 || a.n_kh <= 0 || a.n_vh % a.n_kh ||
        (a.chunk != 0 && a.chunk != 16 && a.chunk != 32 && a.chunk != 64) || (a.chunk == 64 && !a.dc))
        return hipErrorInvalidValue;
    const int CD = 2 * a.n_kh * a.hk + a.n_vh * a.hv;
    hipLaunchKernelGGL(pf_dn_conv_kernel<4>, dim3(nblk(CD, WG), nblk(a.T, DN_TT)), dim3(WG), 0, st, a);
    const dim3 dgrid((unsigned)a.n_vh, 128 / 32);
    // the one-launch chunk normalises q / k and forms the gates itself
    if (!(a.chunk == 64 && a.T <= DC)) hipLaunchKernelGGL(pf_dn_prep_kernel<128>, dim3((unsigned)a.T), dim3(WG), 0, st, a);
    if (a.chunk == 64 && a.T <= DC) {
        hipLaunchKernelGGL((pf_dc_single_kernel<128, 128>), dim3((unsigned)a.n_vh, 128 / DC_CB), dim3(DC_WG), 0, st,
                           a);
    } else if (a.chunk == 64) {
        hipLaunchKernelGGL(pf_dc_prep_kernel<128>, dim3((unsigned)a.n_vh, nblk(a.T, DC)), dim3(DC_WG), 0, st, a);
        hipLaunchKernelGGL((pf_dc_state_kernel<128, 128>), dim3((unsigned)a.n_vh, 128 / DC_CB), dim3(DC_WG), 0, st,
                           a);
    } else if (a.chunk == 16) hipLaunchKernelGGL((pf_dn_chunk_kernel<128, 128, 16>), dgrid, dim3(WG), 0, st, a);
    else if (a.chunk == 32) hipLaunchKernelGGL((pf_dn_chunk_kernel<128, 128, 32>), dgrid, dim3(WG), 0, st, a);
    else hipLaunchKernelGGL((pf_dn_delta_kernel<128, 128>), dim3((unsigned)a.n_vh, 128 / DN_CW), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(pf_dn_gnorm_kernel<128>, dim3((unsigned)a.T, nblk(a.n_vh, (WG / WAVE) * GN_NH)), dim3(WG), 0, st,
                       a);
    return hipGetLastError();
}

}  // namespace oi
