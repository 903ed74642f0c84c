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
//                           the chunk from the conv state) + silu
//   pf_dn_conv_state_kernel the conv state after the chunk (its last inputs)
//   pf_dn_prep_kernel       per token: l2norm of q (times 1/sqrt(head_k_dim))
//                           and k, beta = sigmoid(b), decay = exp(ssm_a
//                           softplus(a + dt_bias)) and its log
//   pf_dn_delta_kernel      the delta rule over the chunk's tokens in order,
//                           the state held in registers for the whole chunk
//   pf_dn_chunk_kernel      the same in its chunked form (qwen3_5/metal.odin:416-468,
//                           which the reference does not dispatch): 16 or 32
//                           tokens per step, decay ratios from log sums
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
// every load unconditional).  Grid (ceil(conv_dim / 256), ceil(T / 8)).
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
#pragma unroll
        for (int k = 0; k < KM1; k++) xs[k] = st[k];
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

// the conv state after the chunk: its last KS-1 inputs, oldest first (runs
// after pf_dn_conv_kernel, which reads the state from before the chunk;
// T >= KS-1, so every one comes from the chunk)
template <int KS>
__global__ __launch_bounds__(WG) void pf_dn_conv_state_kernel(PfDnArgs a) {
    constexpr int KM1 = KS > 1 ? KS - 1 : 1;
    const int CD = 2 * a.n_kh * a.hk + a.n_vh * a.hv;
    const int c = (int)blockIdx.x * WG + threadIdx.x;
    if (c >= CD || KS < 2) return;
    float x[KM1];
    parts_gather(x, a.qkv, a.qkvs, (size_t)a.T * CD, [&](int k) { return (size_t)(a.T - KM1 + k) * CD + c; });
#pragma unroll
    for (int k = 0; k < KM1; k++) a.conv_state[(size_t)c * KM1 + k] = x[k];
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
        (a.chunk != 0 && a.chunk != 16 && a.chunk != 32))
        return hipErrorInvalidValue;
    const int CD = 2 * a.n_kh * a.hk + a.n_vh * a.hv;
    hipLaunchKernelGGL(pf_dn_conv_kernel<4>, dim3(nblk(CD, WG), nblk(a.T, DN_TT)), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(pf_dn_conv_state_kernel<4>, dim3(nblk(CD, WG)), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(pf_dn_prep_kernel<128>, dim3((unsigned)a.T), dim3(WG), 0, st, a);
    const dim3 dgrid((unsigned)a.n_vh, 128 / 32);
    if (a.chunk == 16) hipLaunchKernelGGL((pf_dn_chunk_kernel<128, 128, 16>), dgrid, dim3(WG), 0, st, a);
    else if (a.chunk == 32) hipLaunchKernelGGL((pf_dn_chunk_kernel<128, 128, 32>), dgrid, dim3(WG), 0, st, a);
    else hipLaunchKernelGGL((pf_dn_delta_kernel<128, 128>), dim3((unsigned)a.n_vh, 128 / DN_CW), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(pf_dn_gnorm_kernel<128>, dim3((unsigned)a.T, nblk(a.n_vh, (WG / WAVE) * GN_NH)), dim3(WG), 0, st,
                       a);
    return hipGetLastError();
}

}  // namespace oi
