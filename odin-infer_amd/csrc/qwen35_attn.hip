// qwen35_attn.hip -- the attention of a Qwen3.5 full-attention layer for one
// token, between its projections and its output projection (reference:
// qwen3_5/forward.odin:46-135 forward_full_layer; ops.odin:77-89
// apply_mrope_text_head, ops.odin:163-168 inv_freq_default).  What differs from
// the Qwen3 decoder: the q projection holds [q | gate] per head, RoPE rotates
// only the first rotary_dim dimensions (pairs i and i + rotary_dim/2, angles
// pos * inv_freq[i] computed in f32), scores are dot * (1/sqrt(head_dim)), and
// the attention output is multiplied by sigmoid(gate).
//
// q35_prep_kernel (grid n_heads + n_kv_heads): RMSNorm + partial RoPE of one
//   q head (to qbuf) or one k head (to the f16 cache at pos, with v).
// q35_attn_kernel (grid (n_kv_heads, splits)): positions [s CH, (s+1) CH) of
//   one kv head for all its query heads, one partial (m, l, o[head_dim]) per
//   query head and split.
// q35_combine_kernel (grid n_heads): merge of the splits, o / l, times
//   sigmoid(gate).  Kernel boundaries order the cache store and the partials.

#include "device_common.h"

namespace oi {

constexpr int Q35_CH = 64;   // positions per attention workgroup
constexpr int Q35_GMAX = 8;  // query heads per kv head
constexpr int Q35_MAXS = 2048;  // position splits (contexts up to 131072)

static __device__ __forceinline__ float q35_sigmoid(float x) {
#pragma clang fp contract(off)
    if (x >= 0.0f) {
        const float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = expf(x);
    return z / (1.0f + z);
}

template <int HD>
__global__ __launch_bounds__(WG) void q35_prep_kernel(Q35Args a) {
#pragma clang fp contract(off)
    __shared__ float red[WG / WAVE];
    __shared__ float xs[HD];
    const int hh = blockIdx.x, t = threadIdx.x;
    const bool isq = hh < a.n_heads;
    const int h = isq ? hh : hh - a.n_heads;
    const float *src = isq ? a.qproj + (size_t)h * 2 * HD : a.k + (size_t)h * HD;
    const float *nw = isq ? a.q_norm : a.k_norm;
    float ss = 0.f;
    for (int i = t; i < HD; i += WG) ss += src[i] * src[i];
    ss = wave_sum(ss);
    if ((t & (WAVE - 1)) == 0) red[t / WAVE] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < WG / WAVE; w++) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / (float)HD + a.eps);
    for (int i = t; i < HD; i += WG) xs[i] = nw[i] * (inv * src[i]);
    __syncthreads();
    const int half = a.rotary_dim / 2;
    float vout[(HD + WG - 1) / WG];
#pragma unroll
    for (int r = 0; r < (HD + WG - 1) / WG; r++) {
        const int i = t + WG * r;
        if (i >= HD) continue;
        float v = xs[i];
        if (i < a.rotary_dim) {  // ops.odin:77-89
            const int p = i < half ? i : i - half;
            const float ang = (float)a.pos * a.inv_freq[p];
            const float c = cosf(ang), s = sinf(ang);
            v = i < half ? xs[i] * c - xs[i + half] * s : xs[i - half] * s + xs[i] * c;
        }
        vout[r] = v;
    }
#pragma unroll
    for (int r = 0; r < (HD + WG - 1) / WG; r++) {
        const int i = t + WG * r;
        if (i >= HD) continue;
        if (isq) a.qbuf[(size_t)h * HD + i] = vout[r];
        else {
            const size_t off = ((size_t)h * a.seq_len + a.pos) * HD + i;
            a.kc[off] = f2h(vout[r]);
            a.vc[off] = f2h(a.v[(size_t)h * HD + i]);
        }
    }
}

// One workgroup per (kv head, split of Q35_CH positions): the split's K and V
// rows are staged in LDS once and serve all G = n_heads / n_kv_heads query
// heads of the group (the cache is read once per token, not G times).  Wave w
// takes query heads w, w + 4, ...; lane = position for the scores, then
// o[d] += p_j v_j[d] with lane l holding dimensions DPL l .. DPL l + DPL-1.
template <int HD>
__global__ __launch_bounds__(WG) void q35_attn_kernel(Q35Args a) {
    constexpr int DPL = HD / WAVE, NW = WG / WAVE, KP = HD + 8;  // K rows padded against bank conflicts
    __shared__ __attribute__((aligned(16))) uint16_t ks[Q35_CH * KP];
    __shared__ __attribute__((aligned(16))) uint16_t vs[Q35_CH * HD];
    __shared__ float qs[Q35_GMAX][HD];
    const int kvh = blockIdx.x, sp = blockIdx.y, G = a.n_heads / a.n_kv_heads;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int L = a.pos + 1, t0 = sp * Q35_CH, n = min(Q35_CH, L - t0);
    const uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD, *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    for (int i = threadIdx.x; i < Q35_CH * HD / 8; i += WG) {
        const int r = i / (HD / 8), c = i % (HD / 8), row = t0 + min(r, n - 1);
        *(u32x4 *)(ks + r * KP + 8 * c) = *(const u32x4 *)(kc + (size_t)row * HD + 8 * c);
        *(u32x4 *)(vs + r * HD + 8 * c) = *(const u32x4 *)(vc + (size_t)row * HD + 8 * c);
    }
    for (int i = threadIdx.x; i < G * HD; i += WG) qs[i / HD][i % HD] = a.qbuf[(size_t)kvh * G * HD + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    for (int g = wave; g < G; g += NW) {
        const int h = kvh * G + g;
        float m = -INFINITY, l = 0.f, o[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) o[e] = 0.f;
        for (int base = 0; base < n; base += WAVE) {
            const int r = base + lane;
            float s = -INFINITY;
            if (r < n) {
                const uint16_t *kr = ks + r * KP;
                float acc = 0.f;
                for (int c = 0; c < HD / 8; c++) {
                    const u32x4 w = *(const u32x4 *)(kr + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; e++) acc += qs[g][8 * c + e] * h2f((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
                }
                s = acc * scale;
            }
            float bm = s;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, WAVE));
            const float mn = fmaxf(m, bm), alpha = expf(m - mn);
            const float pj = r < n ? expf(s - mn) : 0.f;
            l = l * alpha + wave_sum(pj);
#pragma unroll
            for (int e = 0; e < DPL; e++) o[e] *= alpha;
            const int nj = min(WAVE, n - base);
            for (int j = 0; j < nj; j++) {
                const float pb = __shfl(pj, j, WAVE);
                const uint16_t *vr = vs + (base + j) * HD + DPL * lane;
#pragma unroll
                for (int e = 0; e < DPL; e += 2) {
                    const uint32_t w = *(const uint32_t *)(vr + e);
                    o[e] += pb * h2f(w & 0xFFFFu);
                    o[e + 1] += pb * h2f(w >> 16);
                }
            }
            m = mn;
        }
        float *pt = a.part + ((size_t)h * a.max_splits + sp) * (HD + 2);
#pragma unroll
        for (int e = 0; e < DPL; e++) pt[DPL * lane + e] = o[e];
        if (lane == 0) {
            pt[HD] = m;
            pt[HD + 1] = l;
        }
    }
}

// Merge of a head's splits: the split weights exp(m_s - M) are formed once
// (in LDS), then every thread sums its dimensions over the splits with the
// loads independent of each other.
template <int HD>
__global__ __launch_bounds__(WG) void q35_combine_kernel(Q35Args a) {
#pragma clang fp contract(off)
    __shared__ float wsp[Q35_MAXS];
    __shared__ float red[WG / WAVE];
    const int h = blockIdx.x, ns = (a.pos + Q35_CH) / Q35_CH, t = threadIdx.x;
    const int lane = t & (WAVE - 1), wave = t / WAVE;
    const float *pb = a.part + (size_t)h * a.max_splits * (HD + 2);
    float mx = -INFINITY;
    for (int s = t; s < ns; s += WG) mx = fmaxf(mx, pb[(size_t)s * (HD + 2) + HD]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < WG / WAVE; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float lp = 0.f;
    for (int s = t; s < ns; s += WG) {
        const float ms = pb[(size_t)s * (HD + 2) + HD];
        const float w = ms == -INFINITY ? 0.f : expf(ms - M);
        wsp[s] = w;
        lp += pb[(size_t)s * (HD + 2) + HD + 1] * w;
    }
    lp = wave_sum(lp);
    if (lane == 0) red[wave] = lp;
    __syncthreads();
    float lt = 0.f;
#pragma unroll
    for (int w = 0; w < WG / WAVE; w++) lt += red[w];
    for (int i = t; i < HD; i += WG) {
        float acc = 0.f;
#pragma unroll 8
        for (int s = 0; s < ns; s++) acc += pb[(size_t)s * (HD + 2) + i] * wsp[s];
        const float gate = a.qproj[(size_t)h * 2 * HD + HD + i];
        a.out[(size_t)h * HD + i] = (acc / lt) * q35_sigmoid(gate);
    }
}

int q35_max_splits(int seq_len) { return (seq_len + Q35_CH - 1) / Q35_CH; }

hipError_t launch_q35_attn(const Q35Args &a, int head_dim, hipStream_t st) {
    const int ns = (a.pos + Q35_CH) / Q35_CH;
    if (ns > a.max_splits || a.rotary_dim < 0 || a.rotary_dim > head_dim || a.rotary_dim % 2 ||
        a.n_heads / a.n_kv_heads > Q35_GMAX || ns > Q35_MAXS)
        return hipErrorInvalidValue;
    const dim3 g1((unsigned)(a.n_heads + a.n_kv_heads)), g2((unsigned)a.n_kv_heads, (unsigned)ns), g3((unsigned)a.n_heads);
    if (head_dim == 256) {
        hipLaunchKernelGGL(q35_prep_kernel<256>, g1, dim3(WG), 0, st, a);
        hipLaunchKernelGGL(q35_attn_kernel<256>, g2, dim3(WG), 0, st, a);
        hipLaunchKernelGGL(q35_combine_kernel<256>, g3, dim3(WG), 0, st, a);
    } else if (head_dim == 128) {
        hipLaunchKernelGGL(q35_prep_kernel<128>, g1, dim3(WG), 0, st, a);
        hipLaunchKernelGGL(q35_attn_kernel<128>, g2, dim3(WG), 0, st, a);
        hipLaunchKernelGGL(q35_combine_kernel<128>, g3, dim3(WG), 0, st, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace oi
