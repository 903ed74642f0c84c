// deltanet.hip -- the gated DeltaNet (linear attention) token step of the
// Qwen3.5 hybrid decoder, between its input projections (in_qkv, in_z, in_b,
// in_a) and its output projection (reference: qwen3_5/forward.odin:137-225
// forward_linear_layer; qwen3_5/ops.odin:7-37 sigmoid / silu / softplus / l2norm,
// qwen3_5/ops.odin:97-161 conv1d_step and delta_recurrent_step).
//
// dn_conv_kernel: depthwise causal conv over the kernel window (current input
//   last, history oldest first), silu, history slide; one thread per channel.
// dn_delta_kernel: one workgroup per value head vh (k head vh % n_kh,
//   qwen3_5/forward.odin:193): l2-normalize q and k of the k head (q also scaled by
//   1/sqrt(head_k_dim)), beta = sigmoid(b), decay = exp(ssm_a * softplus(a +
//   dt_bias)) (ssm_a already holds -exp(A_log)), then the delta rule on the
//   head's state S [head_k_dim][head_v_dim] (k outer, v inner):
//     S *= decay;  delta = (v - S^T k) beta;  S += k delta^T;  o = S^T q
//   and the gated RMSNorm o = rmsnorm(o) * norm_w * silu(z).
//   Thread t owns column j = t % head_v_dim over rows rg*R .. rg*R+R-1
//   (rg = t / head_v_dim), so S is read once and written once per token
//   (coalesced: consecutive threads, consecutive columns); the two column
//   sums S^T k and S^T q are reduced over the row groups through LDS.
// The state is HBM-bound: 4 * head_k_dim * head_v_dim bytes read and written
// per value head and token.  dn_step_kernel does both in one launch when the
// value heads are one or two per k head (below).  The engine's token loop
// uses dn_cols_kernel instead: the conv in the in_qkv GEMV's epilogue, the
// delta rule over many more workgroups, the gated norm in the output GEMV's
// prologue.

#include "device_common.h"

namespace oi {

__global__ __launch_bounds__(WG) void dn_conv_kernel(DnArgs a) {
#pragma clang fp contract(off)
    const int c = (int)blockIdx.x * WG + threadIdx.x;
    const int conv_dim = 2 * a.n_kh * a.hk + a.n_vh * a.hv, km1 = a.kernel - 1;
    if (c >= conv_dim) return;
    const float *w = a.conv_w + (size_t)c * a.kernel;
    float *st = a.conv_state + (size_t)c * km1;
    const float x = a.qkv[c];
    float acc = w[km1] * x;
    for (int k = 0; k < km1; k++) acc += w[k] * st[k];
    a.conv_out[c] = silu_ref(acc);
    for (int k = 0; k < km1 - 1; k++) st[k] = st[k + 1];
    if (km1 > 0) st[km1 - 1] = x;
}

template <int HK, int HV>
__global__ __launch_bounds__(1024) void dn_delta_kernel(DnArgs a) {
#pragma clang fp contract(off)
    constexpr int NT = 1024, RG = NT / HV, R = HK / RG;  // row groups, rows per thread
    static_assert(HK % RG == 0 && NT % HV == 0, "head shape");
    __shared__ float qn[HK], kn[HK];
    __shared__ float part[2][RG][HV];
    __shared__ float red[NT / WAVE];
    __shared__ float sc[4];
    const int vh = blockIdx.x, kh = vh % a.n_kh, t = threadIdx.x;
    const int lane = t & (WAVE - 1), wave = t / WAVE;
    const int key_dim = a.n_kh * HK;
    // l2norm of q and k of the k head (qwen3_5/ops.odin:27-37), eps 1e-6 a floor on the norm
    const float *qr = a.conv_out + kh * HK, *kr = a.conv_out + key_dim + kh * HK;
    float sq = 0.f, sk = 0.f;
    if (t < HK) {
        sq = qr[t] * qr[t];
        sk = kr[t] * kr[t];
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (t == 0) {
        float s = 0.f;
        for (int w = 0; w < (HK + WAVE - 1) / WAVE; w++) s += red[w];
        sc[0] = s;
    }
    __syncthreads();
    if (lane == 0) red[wave] = sk;
    __syncthreads();
    if (t == 0) {
        float s = 0.f;
        for (int w = 0; w < (HK + WAVE - 1) / WAVE; w++) s += red[w];
        sc[1] = s;
        const float b = a.b[vh];
        sc[2] = sigmoid_ref(b);
        sc[3] = expf(a.a_decay[vh] * softplus_ref(a.a[vh] + a.dt_bias[vh]));
    }
    __syncthreads();
    if (t < HK) {
        const float iq = 1.0f / fmaxf(sqrtf(sc[0]), 1e-6f), ik = 1.0f / fmaxf(sqrtf(sc[1]), 1e-6f);
        qn[t] = qr[t] * iq * (1.0f / sqrtf((float)HK));
        kn[t] = kr[t] * ik;
    }
    __syncthreads();
    const float beta = sc[2], decay = sc[3];
    const int j = t % HV, rg = t / HV, i0 = rg * R;
    float *S = a.state + (size_t)vh * HK * HV;
    float s[R];
    float kv = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        s[r] = S[(size_t)(i0 + r) * HV + j] * decay;
        kv += s[r] * kn[i0 + r];
    }
    part[0][rg][j] = kv;
    __syncthreads();
    float kvmem = 0.f;
#pragma unroll
    for (int g = 0; g < RG; g++) kvmem += part[0][g][j];
    const float v = a.conv_out[2 * key_dim + vh * HV + j];
    const float delta = (v - kvmem) * beta;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        s[r] += kn[i0 + r] * delta;
        S[(size_t)(i0 + r) * HV + j] = s[r];
        o += s[r] * qn[i0 + r];
    }
    part[1][rg][j] = o;
    __syncthreads();
    // gated RMSNorm over the head's outputs (qwen3_5/forward.odin:211-218)
    float oj = 0.f;
    if (rg == 0) {
#pragma unroll
        for (int g = 0; g < RG; g++) oj += part[1][g][j];
    }
    float ss = rg == 0 ? oj * oj : 0.f;
    ss = wave_sum(ss);
    __syncthreads();
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (rg == 0) {
        float tot = 0.f;
        for (int w = 0; w < (HV + WAVE - 1) / WAVE; w++) tot += red[w];
        const float inv = 1.0f / sqrtf(tot / (float)HV + a.eps);
        const float z = a.z[vh * HV + j];
        a.out[vh * HV + j] = a.norm_w[j] * (inv * oj) * silu_ref(z);
    }
}

// The whole step in one launch: one workgroup per k head kh and its G value
// heads vh = kh + g n_kh (vh % n_kh == kh), so that the workgroup owns the
// conv windows of every channel it reads (its q and k channels and its value
// heads' v channels) and can slide them without racing another workgroup.
// The conv and the gates are computed as in dn_conv_kernel / dn_delta_kernel;
// then the G heads' states are updated side by side, 1024 / G threads each
// (thread owns column j over R = HK G / 8 rows).
template <int HK, int HV, int G>
__global__ __launch_bounds__(1024) void dn_step_kernel(DnArgs a) {
#pragma clang fp contract(off)
    constexpr int NT = 1024, TPH = NT / G, RG = TPH / HV, R = HK / RG;
    static_assert(TPH % HV == 0 && HK % RG == 0 && 2 * HK + G * HV <= NT, "head shape");
    __shared__ float qn[HK], kn[HK], vv[G][HV];
    __shared__ float part[2][G][RG][HV];
    __shared__ float red[NT / WAVE];
    __shared__ float sc[2 + 2 * G];
    const int kh = blockIdx.x, t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE;
    const int key_dim = a.n_kh * HK, km1 = a.kernel - 1;
    // this thread's part of its head's state, requested first: the loads
    // overlap the conv and the gates, which do not depend on them
    const int g = t / TPH, tt = t % TPH, j = tt % HV, rg = tt / HV, i0 = rg * R;
    const int vh = kh + g * a.n_kh;
    float *S = a.state + (size_t)vh * HK * HV;
    float s[R];
#pragma unroll
    for (int r = 0; r < R; r++) s[r] = S[(size_t)(i0 + r) * HV + j];
    // conv1d_step + silu of the workgroup's channels (qwen3_5/ops.odin:97-116)
    if (t < 2 * HK + G * HV) {
        int c;
        if (t < HK) c = kh * HK + t;
        else if (t < 2 * HK) c = key_dim + kh * HK + (t - HK);
        else c = 2 * key_dim + (kh + ((t - 2 * HK) / HV) * a.n_kh) * HV + (t - 2 * HK) % HV;
        const float *w = a.conv_w + (size_t)c * a.kernel;
        float *st = a.conv_state + (size_t)c * km1;
        const float x = a.qkv[c];
        float acc = w[km1] * x;
        for (int k = 0; k < km1; k++) acc += w[k] * st[k];
        const float o = silu_ref(acc);
        for (int k = 0; k < km1 - 1; k++) st[k] = st[k + 1];
        if (km1 > 0) st[km1 - 1] = x;
        if (t < HK) qn[t] = o;
        else if (t < 2 * HK) kn[t - HK] = o;
        else vv[(t - 2 * HK) / HV][(t - 2 * HK) % HV] = o;
    }
    __syncthreads();
    // l2norm of q and k (qwen3_5/ops.odin:27-37), the gates of the G heads
    float sq = 0.f, sk = 0.f;
    if (t < HK) {
        sq = qn[t] * qn[t];
        sk = kn[t] * kn[t];
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (t == 0) {
        float s = 0.f;
        for (int w = 0; w < (HK + WAVE - 1) / WAVE; w++) s += red[w];
        sc[0] = s;
    }
    __syncthreads();
    if (lane == 0) red[wave] = sk;
    __syncthreads();
    if (t == 0) {
        float s = 0.f;
        for (int w = 0; w < (HK + WAVE - 1) / WAVE; w++) s += red[w];
        sc[1] = s;
    }
    if (t < G) {
        const int vh = kh + t * a.n_kh;
        sc[2 + t] = sigmoid_ref(a.b[vh]);
        sc[2 + G + t] = expf(a.a_decay[vh] * softplus_ref(a.a[vh] + a.dt_bias[vh]));
    }
    __syncthreads();
    if (t < HK) {
        const float iq = 1.0f / fmaxf(sqrtf(sc[0]), 1e-6f), ik = 1.0f / fmaxf(sqrtf(sc[1]), 1e-6f);
        qn[t] = qn[t] * iq * (1.0f / sqrtf((float)HK));
        kn[t] = kn[t] * ik;
    }
    __syncthreads();
    // delta rule of head g on its state (qwen3_5/forward.odin:193-209)
    const float beta = sc[2 + g], decay = sc[2 + G + g];
    float kv = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        s[r] = s[r] * decay;
        kv += s[r] * kn[i0 + r];
    }
    part[0][g][rg][j] = kv;
    __syncthreads();
    float kvmem = 0.f;
#pragma unroll
    for (int q = 0; q < RG; q++) kvmem += part[0][g][q][j];
    const float delta = (vv[g][j] - kvmem) * beta;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        s[r] += kn[i0 + r] * delta;
        S[(size_t)(i0 + r) * HV + j] = s[r];
        o += s[r] * qn[i0 + r];
    }
    part[1][g][rg][j] = o;
    __syncthreads();
    // gated RMSNorm over each head's outputs (qwen3_5/forward.odin:211-218)
    float oj = 0.f;
    if (rg == 0) {
#pragma unroll
        for (int q = 0; q < RG; q++) oj += part[1][g][q][j];
    }
    float ss = rg == 0 ? oj * oj : 0.f;
    ss = wave_sum(ss);
    __syncthreads();
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (rg == 0) {
        float tot = 0.f;
        const int w0 = g * TPH / WAVE;
        for (int w = 0; w < (HV + WAVE - 1) / WAVE; w++) tot += red[w0 + w];
        const float inv = 1.0f / sqrtf(tot / (float)HV + a.eps);
        const float z = a.z[vh * HV + j];
        a.out[vh * HV + j] = a.norm_w[j] * (inv * oj) * silu_ref(z);
    }
}

// The delta rule alone (the token loop's form: the in_qkv GEMV has applied
// the conv, the output GEMV's prologue finishes the gated norm from the
// outputs times silu(z) and the per-workgroup sums of squares written here).  Grid (n_vh,
// hv / 32): a workgroup owns 32 state columns of value head vh, so the state
// is spread over n_vh * hv / 32 workgroups (128 at 32 value heads) and every
// row segment a workgroup reads is one 128-byte line.  Lane = 8 column +
// row group, a row group 16 rows: a lane holds 16 state values; the column
// sums over the 8 row groups are DPP sums inside the lane's group of 8.  Each
// lane normalizes its 16 rows of q and k itself (the sums of squares over the
// same groups of 8).
template <int HK, int HV>
__global__ __launch_bounds__(WG) void dn_cols_kernel(DnArgs a) {
#pragma clang fp contract(off)
    constexpr int RPL = HK / 8;
    static_assert(RPL == 16 && HV % 32 == 0, "head shape");
    const int vh = blockIdx.x, kh = vh % a.n_kh, c0 = (int)blockIdx.y * 32;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int cl = wave * 8 + (lane >> 3), rg = lane & 7, j = c0 + cl, i0 = rg * RPL;
    const int KD = a.n_kh * HK;
    float *S = a.state + (size_t)vh * HK * HV;
    float s[RPL];
#pragma unroll
    for (int r = 0; r < RPL; r++) s[r] = S[(size_t)(i0 + r) * HV + j];
    const float4 *q4 = (const float4 *)(a.conv_out + kh * HK + i0);
    const float4 *k4 = (const float4 *)(a.conv_out + KD + kh * HK + i0);
    float qn[RPL], kn[RPL];
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) {
        const float4 qq = q4[i], kk = k4[i];
        qn[4 * i] = qq.x; qn[4 * i + 1] = qq.y; qn[4 * i + 2] = qq.z; qn[4 * i + 3] = qq.w;
        kn[4 * i] = kk.x; kn[4 * i + 1] = kk.y; kn[4 * i + 2] = kk.z; kn[4 * i + 3] = kk.w;
    }
    const float v = a.conv_out[2 * KD + vh * HV + j];
    const float beta = sigmoid_ref(a.b[vh]);
    const float decay = expf(a.a_decay[vh] * softplus_ref(a.a[vh] + a.dt_bias[vh]));
    // l2norm of q and k (qwen3_5/ops.odin:27-37), eps 1e-6 a floor on the norm
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        sq += qn[r] * qn[r];
        sk += kn[r] * kn[r];
    }
    sq += OI_DPP(sq, 0xB1);
    sq += OI_DPP(sq, 0x4E);
    sq += dpp_mirror8(sq);
    sk += OI_DPP(sk, 0xB1);
    sk += OI_DPP(sk, 0x4E);
    sk += dpp_mirror8(sk);
    const float iq = 1.0f / fmaxf(sqrtf(sq), 1e-6f), ik = 1.0f / fmaxf(sqrtf(sk), 1e-6f);
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        qn[r] = qn[r] * iq * (1.0f / sqrtf((float)HK));
        kn[r] = kn[r] * ik;
    }
    // delta rule (qwen3_5/forward.odin:193-209)
    float kv = 0.f;
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        s[r] = s[r] * decay;
        kv += s[r] * kn[r];
    }
    kv += OI_DPP(kv, 0xB1);
    kv += OI_DPP(kv, 0x4E);
    kv += dpp_mirror8(kv);
    const float delta = (v - kv) * beta;
    float o = 0.f;
#pragma unroll
    for (int r = 0; r < RPL; r++) {
        s[r] += kn[r] * delta;
        S[(size_t)(i0 + r) * HV + j] = s[r];
        o += s[r] * qn[r];
    }
    o += OI_DPP(o, 0xB1);
    o += OI_DPP(o, 0x4E);
    o += dpp_mirror8(o);
    // for the gated norm (qwen3_5/forward.odin:211-218) in the output GEMV's prologue:
    // o silu(z) per column, and this workgroup's part of the head's sum of o^2
    __shared__ float wss[WG / WAVE];
    const float ss = wave_sum(rg == 0 ? o * o : 0.f);
    if (lane == 0) wss[wave] = ss;
    if (rg == 0) a.out[vh * HV + j] = o * silu_ref(a.z[vh * HV + j]);
    __syncthreads();
    if (threadIdx.x == 0) a.ssq[vh * (HV / 32) + blockIdx.y] = (wss[0] + wss[1]) + (wss[2] + wss[3]);
}

hipError_t launch_deltanet(const DnArgs &a, hipStream_t st) {
    if (a.hk != 128 || a.hv != 128 || a.kernel < 1 || a.n_kh <= 0 || a.n_vh <= 0) return hipErrorInvalidValue;
    if (a.cols) {
        hipLaunchKernelGGL((dn_cols_kernel<128, 128>), dim3((unsigned)a.n_vh, 128 / 32), dim3(WG), 0, st, a);
        return hipGetLastError();
    }
    if (a.n_vh == a.n_kh) {
        hipLaunchKernelGGL((dn_step_kernel<128, 128, 1>), dim3((unsigned)a.n_kh), dim3(1024), 0, st, a);
        return hipGetLastError();
    }
    if (a.n_vh == 2 * a.n_kh) {
        hipLaunchKernelGGL((dn_step_kernel<128, 128, 2>), dim3((unsigned)a.n_kh), dim3(1024), 0, st, a);
        return hipGetLastError();
    }
    // other head ratios: the conv pass, then one workgroup per value head
    const int conv_dim = 2 * a.n_kh * a.hk + a.n_vh * a.hv;
    hipLaunchKernelGGL(dn_conv_kernel, dim3((unsigned)((conv_dim + WG - 1) / WG)), dim3(WG), 0, st, a);
    hipLaunchKernelGGL((dn_delta_kernel<128, 128>), dim3((unsigned)a.n_vh), dim3(1024), 0, st, a);
    return hipGetLastError();
}

}  // namespace oi
