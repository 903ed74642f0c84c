// qwen35_attn.hip -- the attention of a Qwen3.5 full-attention layer for one
// token, between its projections and its output projection (reference:
// qwen3_5/forward.odin:46-135 forward_full_layer; qwen3_5/ops.odin:77-89
// apply_mrope_text_head, qwen3_5/ops.odin:163-168 inv_freq_default).  What differs from
// the Qwen3 decoder: the q projection holds [q | gate] per head, RoPE rotates
// only the first rotary_dim dimensions (pairs i and i + rotary_dim/2, angles
// pos * inv_freq[i] computed in f32), scores are dot * (1/sqrt(head_dim)), and
// the attention output is multiplied by sigmoid(gate).
//
// q35_attn_kernel (grid (kv head x group of its query heads, splits)):
//   RMSNorm + partial RoPE of the group's q heads (and, in the split holding
//   pos, of the new k, stored with v to the f16 cache), then positions
//   [s CH, (s+1) CH) of the kv head for the group: one partial
//   (m, l, o[head_dim]) per query head and split.
// q35_combine_kernel (grid (n_heads, head_dim / 64)): merge of the splits,
//   o / l, times sigmoid(gate).  Kernel boundaries order the cache store and
//   the partials.

#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "device_common.h"

namespace oi {

constexpr int Q35_CH = 64;   // positions per attention workgroup
constexpr int Q35_GMAX = 8;  // query heads per kv head
constexpr int Q35_MAXS = 2048;  // position splits (contexts up to 131072)

// One workgroup per (kv head, group of GW (4, 2 or 1) of its query heads, split of
// Q35_CH positions).  The split's K (rows padded against bank conflicts) and
// V rows and the group's rotated q are staged in LDS; then
//   scores: lane = position, wave = quarter of the dimensions, each K value
//           read once for all the group's heads, partial sums through LDS;
//   softmax of the split, one wave per head;
//   o = sum_t p_t v_t: lane holds DPL dimensions, wave takes positions
//           w, w + 4, ..., each V value read once for all heads;
// and one partial (m, l, o[head_dim]) per query head and split.
template <int HD, int GW>
__global__ __launch_bounds__(WG) void q35_attn_kernel(Q35Args a) {
    constexpr int NW = WG / WAVE, DPW = HD / NW, DPL = HD / WAVE, KP = HD + 8;
    __shared__ __attribute__((aligned(16))) uint16_t ks[Q35_CH * KP];  // later: o partials [NW][GW][HD] f32
    __shared__ __attribute__((aligned(16))) uint16_t vs[Q35_CH * HD];
    __shared__ __attribute__((aligned(16))) float qs[GW][HD];
    __shared__ float sp[NW][GW][Q35_CH];
    __shared__ float mx[GW], sm[GW];
    static_assert(NW * GW * HD * 4 <= Q35_CH * KP * 2, "o partials fit in the K tile");
    const int G = a.n_heads / a.n_kv_heads, ngrp = G / GW;
    const int kvh = blockIdx.x / ngrp, h0 = kvh * G + (blockIdx.x % ngrp) * GW, sp_i = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state ? a.state[ST_POS] : a.pos;  // the token loop keeps pos on the device
    const int L = pos + 1, t0 = sp_i * Q35_CH, n = min(Q35_CH, L - t0);
    if (t0 > pos) return;  // a split past pos (graph launches size the grid for seq_len)
    const uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD, *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    // every tile load is issued before the first LDS store, so the loads
    // stream instead of waiting one by one
    constexpr int NLD = Q35_CH * HD / 8 / WG;
    u32x4 kr[NLD], vr[NLD];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int i = tid + j * WG, r = i / (HD / 8), c = i % (HD / 8), row = t0 + min(r, n - 1);
        kr[j] = ldg_nt((const u32x4 *)(kc + (size_t)row * HD + 8 * c));
        vr[j] = ldg_nt((const u32x4 *)(vc + (size_t)row * HD + 8 * c));
    }
    // this workgroup's q heads, and in the split that holds pos the new k and
    // v: RMSNorm (ops.odin rmsnorm) and partial RoPE (qwen3_5/ops.odin:77-89); the
    // new k / v go to the cache and to the LDS tile row pos - t0
    const bool has_pos = pos < t0 + Q35_CH;
    for (int i = tid; i < GW * HD; i += WG) qs[i / HD][i % HD] = a.qproj[(size_t)(h0 + i / HD) * 2 * HD + i % HD];
    __shared__ float kn[HD], vn[HD];
    if (has_pos)
        for (int i = tid; i < HD; i += WG) {
            kn[i] = a.k[(size_t)kvh * HD + i];
            vn[i] = a.v[(size_t)kvh * HD + i];
        }
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int i = tid + j * WG, r = i / (HD / 8), c = i % (HD / 8);
        *(u32x4 *)(ks + r * KP + 8 * c) = kr[j];
        *(u32x4 *)(vs + r * HD + 8 * c) = vr[j];
    }
    __syncthreads();
    for (int g = wave; g < GW + (has_pos ? 1 : 0); g += NW) {
#pragma clang fp contract(off)
        float *x = g < GW ? qs[g] : kn;
        const float *w = g < GW ? a.q_norm : a.k_norm;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += x[i] * x[i];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
        float xv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) xv[e] = w[lane + WAVE * e] * (inv * x[lane + WAVE * e]);
#pragma unroll
        for (int e = 0; e < DPL; e++) x[lane + WAVE * e] = xv[e];
        const int half = a.rotary_dim / 2;
        float yv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            const int i = lane + WAVE * e;
            float v = xv[e];
            if (i < a.rotary_dim) {
                const int pr = i < half ? i : i - half;
                const float ang = (float)pos * a.inv_freq[pr];
                const float c = cosf(ang), sn = sinf(ang);
                v = i < half ? x[i] * c - x[i + half] * sn : x[i - half] * sn + x[i] * c;
            }
            yv[e] = v;
        }
#pragma unroll
        for (int e = 0; e < DPL; e++) x[lane + WAVE * e] = yv[e];
    }
    __syncthreads();
    if (has_pos) {
        const int tl = pos - t0;
        for (int i = tid; i < HD; i += WG) {
            const uint16_t kb = f2h(kn[i]), vb = f2h(vn[i]);
            ks[tl * KP + i] = kb;
            vs[tl * HD + i] = vb;
            if (blockIdx.x % ngrp == 0) {
                a.kc[((size_t)kvh * a.seq_len + pos) * HD + i] = kb;
                a.vc[((size_t)kvh * a.seq_len + pos) * HD + i] = vb;
            }
        }
    }
    __syncthreads();
    {
        float acc[GW];
#pragma unroll
        for (int g = 0; g < GW; g++) acc[g] = 0.f;
        const uint16_t *kr = ks + lane * KP + wave * DPW;
#pragma unroll 4
        for (int c = 0; c < DPW / 8; c++) {
            const u32x4 w = *(const u32x4 *)(kr + 8 * c);
            float kv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) kv[e] = h2f((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
#pragma unroll
            for (int g = 0; g < GW; g++) {
                const float4 q0 = *(const float4 *)&qs[g][wave * DPW + 8 * c];
                const float4 q1 = *(const float4 *)&qs[g][wave * DPW + 8 * c + 4];
                acc[g] += q0.x * kv[0] + q0.y * kv[1] + q0.z * kv[2] + q0.w * kv[3] + q1.x * kv[4] + q1.y * kv[5] +
                          q1.z * kv[6] + q1.w * kv[7];
            }
        }
#pragma unroll
        for (int g = 0; g < GW; g++) sp[wave][g][lane] = acc[g];
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    for (int g = wave; g < GW; g += NW) {
        const float s = lane < n ? ((sp[0][g][lane] + sp[1][g][lane]) + (sp[2][g][lane] + sp[3][g][lane])) * scale
                                 : -INFINITY;
        float m = s;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, WAVE));
        const float e = lane < n ? expf(s - m) : 0.f;
        sp[0][g][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            mx[g] = m;
            sm[g] = l;
        }
    }
    __syncthreads();
    float *ob = (float *)ks;  // [NW][GW][HD]; the K tile is no longer read
    {
        float acc[GW][DPL];
#pragma unroll
        for (int g = 0; g < GW; g++)
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[g][e] = 0.f;
        for (int t = wave; t < n; t += NW) {
            float vv[DPL];
            const uint16_t *vr = vs + t * HD + DPL * lane;
#pragma unroll
            for (int e = 0; e < DPL; e += 2) {
                const uint32_t w = *(const uint32_t *)(vr + e);
                vv[e] = h2f(w & 0xFFFFu);
                vv[e + 1] = h2f(w >> 16);
            }
#pragma unroll
            for (int g = 0; g < GW; g++) {
                const float p = sp[0][g][t];
#pragma unroll
                for (int e = 0; e < DPL; e++) acc[g][e] += p * vv[e];
            }
        }
#pragma unroll
        for (int g = 0; g < GW; g++)
#pragma unroll
            for (int e = 0; e < DPL; e++) ob[(wave * GW + g) * HD + DPL * lane + e] = acc[g][e];
    }
    __syncthreads();
    for (int i = tid; i < GW * HD; i += WG) {
        const int g = i / HD, d = i % HD;
        float *pt = a.part + ((size_t)(h0 + g) * a.max_splits + sp_i) * (HD + 2);
        pt[d] = (ob[(0 * GW + g) * HD + d] + ob[(1 * GW + g) * HD + d]) +
                (ob[(2 * GW + g) * HD + d] + ob[(3 * GW + g) * HD + d]);
        if (d == 0) {
            pt[HD] = mx[g];
            pt[HD + 1] = sm[g];
        }
    }
}

// q35_lane_kernel, grid (splits, n_kv_heads): one workgroup per (split of
// Q35_CH positions, kv head) serves every query head of the kv head's group,
// so each K / V row is read once, with one wave per query head (at least 4
// waves) and no workgroup barrier after the staging:
//   1. requests this token's q halves of the group's [q | gate] slices, k, v
//      and the norm weights, then its K and V tiles (16 B per lane);
//   2. RMSNorm and partial RoPE of the group's q heads (and, in the split that
//      holds pos, of the new k, which goes with v to the f16 cache and to the
//      LDS tile row pos - t0), as q35_attn_kernel;
//   3. one wave per query head: scores with lane = position (the whole dot
//      product of its K row, four chains) times 1/sqrt(head_dim), the split's
//      max and exp-sum by wave reductions, p through the wave's LDS row, then
//      o = sum_t p_t v_t with HD / 64 dimensions per lane, and the partial
//      (o, m, l) that q35_combine_kernel merges.
static constexpr int q35_lane_threads(int G) { return G > 4 ? G * WAVE : WG; }
template <int HD, int G>
__global__ __launch_bounds__(q35_lane_threads(G)) void q35_lane_kernel(Q35Args a) {
    constexpr int NT = q35_lane_threads(G), CH = Q35_CH, KP = HD + 8, CPR = HD / 8, NLD = CH * CPR / NT;
    constexpr int DPL = HD / WAVE, QPT = (G * HD + NT - 1) / NT;
    static_assert(CH == WAVE && NLD * NT == CH * CPR, "one position per lane, whole tile loads");
    __shared__ __attribute__((aligned(16))) uint16_t ks[CH * KP];
    __shared__ __attribute__((aligned(16))) uint16_t vs[CH * HD];
    __shared__ __attribute__((aligned(16))) float qs[G][HD];
    __shared__ float kn[HD], vn[HD], qw[HD], kw[HD];
    __shared__ __attribute__((aligned(16))) float sp[G][CH];
    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state ? a.state[ST_POS] : a.pos;  // the token loop keeps pos on the device
    const int t0 = split * CH;
    if (t0 > pos) return;  // a split past pos (graph launches size the grid for seq_len)
    const int n = min(CH, pos + 1 - t0);
    const bool has_pos = pos < t0 + CH;
    uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD, *vc = a.vc + (size_t)kvh * a.seq_len * HD;

    // 1. the small loads first (vector loads return in order), then the tiles
    float qreg[QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = min(tid + i * NT, G * HD - 1);
        qreg[i] = a.qproj[(size_t)(kvh * G + idx / HD) * 2 * HD + idx % HD];
    }
    const int hi = min(tid, HD - 1);
    const float kraw = a.k[(size_t)kvh * HD + hi], vraw = a.v[(size_t)kvh * HD + hi];
    const float qnr = a.q_norm[hi], knr = a.k_norm[hi];
    u32x4 kr[NLD], vr[NLD];
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int c = tid + j * NT, tl = min(c / CPR, n - 1), ch = c % CPR;
        kr[j] = ldg_nt((const u32x4 *)(kc + (size_t)(t0 + tl) * HD) + ch);
        vr[j] = ldg_nt((const u32x4 *)(vc + (size_t)(t0 + tl) * HD) + ch);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. RMSNorm (ops.odin rmsnorm) and partial RoPE (qwen3_5/ops.odin:77-89)
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * NT;
        if (idx < G * HD) qs[idx / HD][idx % HD] = qreg[i];
    }
    if (tid < HD) {
        kn[tid] = kraw;
        vn[tid] = vraw;
        qw[tid] = qnr;
        kw[tid] = knr;
    }
    __syncthreads();
    for (int g = wave; g < G + (has_pos ? 1 : 0); g += NT / WAVE) {
#pragma clang fp contract(off)
        float *x = g < G ? qs[g] : kn;
        const float *w = g < G ? qw : kw;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += x[i] * x[i];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + a.eps);
        float xv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) xv[e] = w[lane + WAVE * e] * (inv * x[lane + WAVE * e]);
#pragma unroll
        for (int e = 0; e < DPL; e++) x[lane + WAVE * e] = xv[e];
        const int half = a.rotary_dim / 2;
        float yv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            const int i = lane + WAVE * e;
            float v = xv[e];
            if (i < a.rotary_dim) {
                const int pr = i < half ? i : i - half;
                const float ang = (float)pos * a.inv_freq[pr];
                const float c = cosf(ang), sn = sinf(ang);
                v = i < half ? x[i] * c - x[i + half] * sn : x[i - half] * sn + x[i] * c;
            }
            yv[e] = v;
        }
#pragma unroll
        for (int e = 0; e < DPL; e++) x[lane + WAVE * e] = yv[e];
    }

    // 3. the tiles in LDS (rows at or past n are zero; row pos - t0 is set below)
#pragma unroll
    for (int j = 0; j < NLD; j++) {
        const int c = tid + j * NT, tl = c / CPR, ch = c % CPR;
        const bool ok = tl < n && t0 + tl != pos;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4 *)(ks + tl * KP + ch * 8) = ok ? kr[j] : z;
        *(u32x4 *)(vs + tl * HD + ch * 8) = ok ? vr[j] : z;
    }
    __syncthreads();
    if (has_pos) {
        const int tl = pos - t0;
        for (int i = tid; i < HD; i += NT) {
            const uint16_t kb = f2h(kn[i]), vb = f2h(vn[i]);
            kc[(size_t)pos * HD + i] = kb;
            vc[(size_t)pos * HD + i] = vb;
            ks[tl * KP + i] = kb;
            vs[tl * HD + i] = vb;
        }
        __syncthreads();
    }

    // 4. one wave per query head
    const float scale = 1.0f / sqrtf((float)HD);
    for (int g = wave; g < G; g += NT / WAVE) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            const u32x4 w = *(const u32x4 *)(ks + lane * KP + 8 * c);
            const float4 q0 = *(const float4 *)&qs[g][8 * c];
            const float4 q1 = *(const float4 *)&qs[g][8 * c + 4];
            acc[c & 3] += q0.x * h2f(w.x & 0xFFFFu) + q0.y * h2f(w.x >> 16) + q0.z * h2f(w.y & 0xFFFFu) +
                          q0.w * h2f(w.y >> 16) + q1.x * h2f(w.z & 0xFFFFu) + q1.y * h2f(w.z >> 16) +
                          q1.z * h2f(w.w & 0xFFFFu) + q1.w * h2f(w.w >> 16);
        }
        const float s = lane < n ? ((acc[0] + acc[1]) + (acc[2] + acc[3])) * scale : -INFINITY;
        const float m = wave_max_all(s);
        const float e = lane < n ? expf(s - m) : 0.f;
        sp[g][lane] = e;  // this wave's row only: DS operations of one wave complete in order
        const float l = wave_sum(e);
        __builtin_amdgcn_wave_barrier();
        float o[4][DPL];
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int d = 0; d < DPL; d++) o[j][d] = 0.f;
#pragma unroll 4
        for (int t4 = 0; t4 < CH; t4 += 4) {
            const float4 p4 = *(const float4 *)&sp[g][t4];  // rows past n hold p = 0 and zero V
            const float pw[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint16_t *vrow = vs + (t4 + j) * HD + DPL * lane;
                float vv[DPL];
#pragma unroll
                for (int d = 0; d < DPL; d += 2) {
                    const uint32_t w2 = *(const uint32_t *)(vrow + d);
                    vv[d] = h2f(w2 & 0xFFFFu);
                    vv[d + 1] = h2f(w2 >> 16);
                }
#pragma unroll
                for (int d = 0; d < DPL; d++) o[j][d] += pw[j] * vv[d];
            }
        }
        float *pt = a.part + ((size_t)(kvh * G + g) * a.max_splits + split) * (HD + 2);
#pragma unroll
        for (int d = 0; d < DPL; d++) pt[DPL * lane + d] = (o[0][d] + o[1][d]) + (o[2][d] + o[3][d]);
        if (lane == 0) {
            pt[HD] = m;
            pt[HD + 1] = l;
        }
    }
}

// Merge of a head's splits: one query head and 64 of its dimensions per
// workgroup (grid (n_heads, HD / 64)), the 4 waves taking every 4th split,
// the first Q35_PF splits' values requested together with the (m, l) pairs
// (one memory round trip); the split weights exp(m_s - M) are formed once in
// LDS by one wave.  out = (o / l) sigmoid(gate).
constexpr int Q35_PF = 20;
template <int HD>
__global__ __launch_bounds__(WG) void q35_combine_kernel(Q35Args a) {
#pragma clang fp contract(off)
    __shared__ float wm[Q35_MAXS], wl[Q35_MAXS];
    __shared__ float ored[WG / WAVE][WAVE];
    __shared__ float Ls;
    const int pos = a.state ? a.state[ST_POS] : a.pos;
    const int h = blockIdx.x, ns = (pos + Q35_CH) / Q35_CH, t = threadIdx.x;
    const int lane = t & (WAVE - 1), wave = t / WAVE, i = blockIdx.y * WAVE + lane;
    const float *pb = a.part + (size_t)h * a.max_splits * (HD + 2);
    float ov[Q35_PF];
#pragma unroll
    for (int k = 0; k < Q35_PF; k++) {
        const int s = wave + (WG / WAVE) * k;
        ov[k] = s < ns ? pb[(size_t)s * (HD + 2) + i] : 0.f;
    }
    const float gate = a.qproj[(size_t)h * 2 * HD + HD + i];
    for (int s = t; s < ns; s += WG) {
        wm[s] = pb[(size_t)s * (HD + 2) + HD];
        wl[s] = pb[(size_t)s * (HD + 2) + HD + 1];
    }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
        for (int s = lane; s < ns; s += WAVE) M = fmaxf(M, wm[s]);
        M = wave_max_all(M);
        float L = 0.f;
        for (int s = lane; s < ns; s += WAVE) {
            const float ms = wm[s];
            const float w = ms == -INFINITY ? 0.f : expf(ms - M);
            wm[s] = w;
            L += wl[s] * w;
        }
        L = wave_sum(L);
        if (lane == 0) Ls = L;
    }
    __syncthreads();
    float O = 0.f;
#pragma unroll
    for (int k = 0; k < Q35_PF; k++) {
        const int s = wave + (WG / WAVE) * k;
        if (s < ns) O += ov[k] * wm[s];
    }
    for (int s = wave + (WG / WAVE) * Q35_PF; s < ns; s += WG / WAVE) O += pb[(size_t)s * (HD + 2) + i] * wm[s];
    ored[wave][lane] = O;
    __syncthreads();
    if (wave == 0)
        a.out[(size_t)h * HD + i] = (((ored[0][lane] + ored[1][lane]) + (ored[2][lane] + ored[3][lane])) / Ls) *
                                   sigmoid_ref(gate);
}

int q35_max_splits(int seq_len) { return (seq_len + Q35_CH - 1) / Q35_CH; }

hipError_t launch_q35_attn(const Q35Args &a, int head_dim, hipStream_t st) {
    // with a device-side pos the grid covers every split of the cache
    const int ns = a.state ? a.max_splits : (a.pos + Q35_CH) / Q35_CH;
    if (ns > a.max_splits || a.rotary_dim < 0 || a.rotary_dim > head_dim || a.rotary_dim % 2 ||
        a.n_heads / a.n_kv_heads > Q35_GMAX || ns > Q35_MAXS)
        return hipErrorInvalidValue;
    const int G = a.n_heads / a.n_kv_heads, gw = G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
    const dim3 g2((unsigned)(a.n_kv_heads * (G / gw)), (unsigned)ns), g3((unsigned)a.n_heads, (unsigned)(head_dim / WAVE));
    // the lane-per-position kernel (default; groups of 1, 2, 4 or 8 query
    // heads), or the dimension-split kernel over groups of gw query heads
    // (other groups, and OI_Q35_ATTN=groups)
    const char *qa = std::getenv("OI_Q35_ATTN");
    const bool lanes = !(qa && std::strcmp(qa, "groups") == 0) && (G == 1 || G == 2 || G == 4 || G == 8);
    const dim3 gl((unsigned)ns, (unsigned)a.n_kv_heads);
    auto attn = [&](auto hd_tag) {
        constexpr int HD = decltype(hd_tag)::value;
        if (lanes) {
            switch (G) {
            case 1: hipLaunchKernelGGL((q35_lane_kernel<HD, 1>), gl, dim3(q35_lane_threads(1)), 0, st, a); break;
            case 2: hipLaunchKernelGGL((q35_lane_kernel<HD, 2>), gl, dim3(q35_lane_threads(2)), 0, st, a); break;
            case 4: hipLaunchKernelGGL((q35_lane_kernel<HD, 4>), gl, dim3(q35_lane_threads(4)), 0, st, a); break;
            default: hipLaunchKernelGGL((q35_lane_kernel<HD, 8>), gl, dim3(q35_lane_threads(8)), 0, st, a); break;
            }
            hipLaunchKernelGGL(q35_combine_kernel<HD>, g3, dim3(WG), 0, st, a);
            return;
        }
        if (gw == 4) hipLaunchKernelGGL((q35_attn_kernel<HD, 4>), g2, dim3(WG), 0, st, a);
        else if (gw == 2) hipLaunchKernelGGL((q35_attn_kernel<HD, 2>), g2, dim3(WG), 0, st, a);
        else hipLaunchKernelGGL((q35_attn_kernel<HD, 1>), g2, dim3(WG), 0, st, a);
        hipLaunchKernelGGL(q35_combine_kernel<HD>, g3, dim3(WG), 0, st, a);
    };
    if (head_dim == 256) attn(std::integral_constant<int, 256>{});
    else if (head_dim == 128) attn(std::integral_constant<int, 128>{});
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace oi
