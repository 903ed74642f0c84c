// attn.hip -- split-L grouped-query decode attention over the f16 KV cache
// (reference: infer/forward.odin:117-175; f16 cache as infer/metal.odin:443-474).
//
// attn_kernel, grid (splits, n_kv_heads): a workgroup takes CH consecutive
// positions of one KV head and serves all G = n_heads / n_kv_heads query
// heads of the group, so each K/V row is read from HBM once per token (the
// reference re-reads it for every query head).  Per workgroup:
//   1. request this token's q (G heads), k, v, cos/sin and norm weights,
//      then its K and V tiles (16 B per lane, coalesced); every load is
//      unconditional (rows past the range re-read a valid row and are zeroed
//      later), so the compiler waits for the small loads alone while the
//      tiles stream,
//   2. RMSNorm + RoPE the G query heads (and, in the split that holds `pos`,
//      the new key; K/V[pos] are rounded to f16 and stored),
//   3. stage K (rows padded against bank conflicts) and V in LDS,
//   4. scores: lane l takes positions l, l+64, ... over a quarter of the
//      dimensions (one quarter per wave); divided by sqrt(hd) (forward.odin:158),
//   5. split max / exp-sum per head, o = sum_t p v_t (2 dims per lane),
//   6. write (o, m, l) to the partial buffer.
// attn_combine_kernel merges the splits of each query head with
// exp(m_s - M) weights; the kernel boundary orders the partial writes before
// the reads, so no fences or atomics are needed.  (Merging in the last
// arriving split instead costs a store-completion wait, an atomic and the
// partial reads in series, which measured slower than the kernel boundary.)
// The current position is used from LDS, so no workgroup reads a cache
// entry written in this launch.

#include "device_common.h"

namespace oi {

template <int HD>
struct AttnShape {
    static constexpr int CH = 64;                     // positions per workgroup (one per lane)
    static constexpr int KPAD = HD + 8;               // LDS row stride of K, in halves
    static constexpr int CPR = HD / 8;                // 16-byte chunks per row
    static constexpr int NLD = CH * CPR / WG;         // loads per thread per tensor
    static constexpr int DPW = HD / 4;                // score dimensions per wave
    static constexpr int DPL = HD / WAVE;             // o dimensions per lane
    static constexpr int PPL = CH / WAVE;             // score positions per lane
};
constexpr int ATTN_MAX_SPLITS = 1024;

static __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

template <int HD, int G>
__global__ __launch_bounds__(WG) void attn_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
    __shared__ __attribute__((aligned(16))) uint16_t ks[S::CH * S::KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t vs[S::CH * HD];
    __shared__ __attribute__((aligned(16))) float qr[G][HD];
    __shared__ float kp[HD], vp[HD], qn[HD], kn[HD];
    __shared__ float sp[4][G][S::CH];  // per-wave partial scores, then p in sp[0]
    __shared__ float ob[4][G][HD];
    __shared__ float mx[G], sm[G], nrm[G + 1];
    __shared__ float2 csl[HD / 2];

    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state[ST_POS];
    const int t0 = split * S::CH;
    if (t0 > pos) return;
    const int t1 = min(t0 + S::CH, pos + 1), n = t1 - t0;
    uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD;
    uint16_t *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    const bool has_pos = pos < t1;

    // 1. small loads first (vector loads return in order), then the tiles
    constexpr int QPT = (G * HD + WG - 1) / WG;
    float qreg[QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++) qreg[i] = a.q[(size_t)kvh * G * HD + min(tid + i * WG, G * HD - 1)];
    const int hi = min(tid, HD - 1);
    const float kraw = a.k[(size_t)kvh * HD + hi], vraw = a.v[(size_t)kvh * HD + hi];
    const float2 csr = a.rope_cs[(size_t)pos * (HD / 2) + min(tid, HD / 2 - 1)];
    const float qnr = a.q_norm[hi], knr = a.k_norm[hi];
    u32x4 kr[S::NLD], vr[S::NLD];
#pragma unroll
    for (int j = 0; j < S::NLD; j++) {
        const int c = tid + j * WG, tl = min(c / S::CPR, n - 1), ch = c % S::CPR;
        kr[j] = ldg_nt((const u32x4 *)(kc + (size_t)(t0 + tl) * HD) + ch);
        vr[j] = ldg_nt((const u32x4 *)(vc + (size_t)(t0 + tl) * HD) + ch);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. RMSNorm + RoPE of the G query heads (and of k at pos): ops.odin:7-19,
    //    forward.odin:117-145; cos/sin come from the host-built table
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const int idx = tid + i * WG;
        if (idx < G * HD) qr[idx / HD][idx % HD] = qreg[i];
    }
    if (tid < HD) {
        kp[tid] = kraw;
        vp[tid] = vraw;
        qn[tid] = qnr;
        kn[tid] = knr;
    }
    if (tid < HD / 2) csl[tid] = csr;
    __syncthreads();
    const int nvec = G + (has_pos ? 1 : 0);
    for (int g = wave; g < nvec; g += WG / WAVE) {
        const float *src = g < G ? qr[g] : kp;
        float ss = 0.f;
        for (int i = lane; i < HD; i += WAVE) ss += src[i] * src[i];
        ss = wave_sum(ss);
        if (lane == 0) nrm[g] = 1.0f / sqrtf(ss / (float)HD + a.eps);
    }
    __syncthreads();
    for (int idx = tid; idx < nvec * (HD / 2); idx += WG) {
#pragma clang fp contract(off)
        const int g = idx / (HD / 2), i = idx % (HD / 2);
        float *v = g < G ? qr[g] : kp;
        const float *w = g < G ? qn : kn;
        const float s = nrm[g];
        const float x = w[i] * (s * v[i]);
        const float y = w[i + HD / 2] * (s * v[i + HD / 2]);
        const float c = csl[i].x, sn = csl[i].y;
        v[i] = x * c - y * sn;
        v[i + HD / 2] = x * sn + y * c;
    }

    // 3. stage the tiles in LDS (rows at or past n are zero; row pos-t0 is set below)
#pragma unroll
    for (int j = 0; j < S::NLD; j++) {
        const int c = tid + j * WG, tl = c / S::CPR, ch = c % S::CPR;
        const bool ok = tl < n && t0 + tl != pos;
        const u32x4 z = {0u, 0u, 0u, 0u};
        *(u32x4 *)(ks + tl * S::KPAD + ch * 8) = ok ? kr[j] : z;
        *(u32x4 *)(vs + tl * HD + ch * 8) = ok ? vr[j] : z;
    }
    __syncthreads();
    if (has_pos) {
        const int tl = pos - t0;
        for (int i = tid; i < HD; i += WG) {
            const uint16_t kb = f2h(kp[i]), vb = f2h(vp[i]);
            kc[(size_t)pos * HD + i] = kb;
            vc[(size_t)pos * HD + i] = vb;
            ks[tl * S::KPAD + i] = kb;
            vs[tl * HD + i] = vb;
        }
        __syncthreads();
    }

    // 4. partial scores: lane = positions lane + 64 p, wave = quarter of the dimensions
    {
        float acc[G][S::PPL];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int p = 0; p < S::PPL; p++) acc[g][p] = 0.f;
#pragma unroll
        for (int c = 0; c < S::DPW / 8; c++) {
#pragma unroll
            for (int p = 0; p < S::PPL; p++) {
                const u32x4 w = *(const u32x4 *)(ks + (lane + WAVE * p) * S::KPAD + wave * S::DPW + 8 * c);
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
                float kv[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    kv[2 * e] = h2f(ws[e] & 0xFFFFu);
                    kv[2 * e + 1] = h2f(ws[e] >> 16);
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float4 q0 = *(const float4 *)&qr[g][wave * S::DPW + 8 * c];
                    const float4 q1 = *(const float4 *)&qr[g][wave * S::DPW + 8 * c + 4];
                    acc[g][p] += q0.x * kv[0] + q0.y * kv[1] + q0.z * kv[2] + q0.w * kv[3] + q1.x * kv[4] +
                                 q1.y * kv[5] + q1.z * kv[6] + q1.w * kv[7];
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int p = 0; p < S::PPL; p++) sp[wave][g][lane + WAVE * p] = acc[g][p];
    }
    __syncthreads();

    // 5. scores, split-local max and exp-sum (ops.odin:21-37), one wave per head
    const float div = sqrtf((float)HD);
    for (int g = wave; g < G; g += WG / WAVE) {
        float sc[S::PPL], m = -INFINITY;
#pragma unroll
        for (int p = 0; p < S::PPL; p++) {
            const int t = lane + WAVE * p;
            sc[p] = t < n ? ((sp[0][g][t] + sp[1][g][t]) + (sp[2][g][t] + sp[3][g][t])) / div : -INFINITY;
            m = fmaxf(m, sc[p]);
        }
        m = wave_max(m);
        float l = 0.f;
#pragma unroll
        for (int p = 0; p < S::PPL; p++) {
            const int t = lane + WAVE * p;
            const float e = t < n ? expf(sc[p] - m) : 0.f;
            sp[0][g][t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            mx[g] = m;
            sm[g] = l;
        }
    }
    __syncthreads();

    // o_g = sum_t p_g(t) v(t): lane holds DPL dims, wave w takes t = w, w+4, ...
    {
        float acc[G][S::DPL];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < S::DPL; e++) acc[g][e] = 0.f;
        for (int tl = wave; tl < n; tl += WG / WAVE) {
            float vv[S::DPL];
            if (S::DPL == 2) {
                const uint32_t w = *(const uint32_t *)(vs + tl * HD + 2 * lane);
                vv[0] = h2f(w & 0xFFFFu);
                vv[S::DPL - 1] = h2f(w >> 16);
            } else {
                const u32x2 w = *(const u32x2 *)(vs + tl * HD + S::DPL * lane);
                const uint32_t ws[2] = {w.x, w.y};
#pragma unroll
                for (int e = 0; e < S::DPL; e++) vv[e] = h2f((ws[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sp[0][g][tl];
#pragma unroll
                for (int e = 0; e < S::DPL; e++) acc[g][e] += p * vv[e];
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < S::DPL; e++) ob[wave][g][S::DPL * lane + e] = acc[g][e];
    }
    __syncthreads();

    // 6. partial (o, m, l) of this split
    const int stride = HD + 2;
    for (int idx = tid; idx < G * HD; idx += WG) {
        const int g = idx / HD, i = idx % HD;
        const float o = (ob[0][g][i] + ob[1][g][i]) + (ob[2][g][i] + ob[3][g][i]);
        float *pp = a.part + ((size_t)(kvh * G + g) * a.max_splits + split) * stride;
        pp[i] = o;
        if (i == 0) {
            pp[HD] = mx[g];
            pp[HD + 1] = sm[g];
        }
    }
}

// O_h = sum_s exp(m_s - M) o_s / sum_s exp(m_s - M) l_s  for one query head and
// 64 of its dimensions; the 4 waves take every 4th split.
template <int HD>
__global__ __launch_bounds__(WG) void attn_combine_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
    __shared__ float wm[ATTN_MAX_SPLITS], wl[ATTN_MAX_SPLITS];
    __shared__ float ored[WG / WAVE][WAVE];
    __shared__ float Ls;
    const int h = blockIdx.x, i = blockIdx.y * WAVE + (threadIdx.x & (WAVE - 1));
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state[ST_POS];
    const int nsplit = pos / S::CH + 1;
    const int stride = HD + 2;
    const float *pb = a.part + (size_t)h * a.max_splits * stride;
    for (int s = tid; s < nsplit; s += WG) {
        wm[s] = pb[(size_t)s * stride + HD];
        wl[s] = pb[(size_t)s * stride + HD + 1];
    }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
        for (int s = lane; s < nsplit; s += WAVE) M = fmaxf(M, wm[s]);
        M = wave_max(M);
        float L = 0.f;
        for (int s = lane; s < nsplit; s += WAVE) {
            const float f = expf(wm[s] - M);
            wm[s] = f;
            L += f * wl[s];
        }
        L = wave_sum(L);
        if (lane == 0) Ls = L;
    }
    __syncthreads();
    float O = 0.f;
#pragma unroll 8
    for (int s = wave; s < nsplit; s += WG / WAVE) O += wm[s] * pb[(size_t)s * stride + i];
    ored[wave][lane] = O;
    __syncthreads();
    if (wave == 0) a.out[(size_t)h * HD + i] = ((ored[0][lane] + ored[1][lane]) + (ored[2][lane] + ored[3][lane])) / Ls;
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs &a, int G, hipStream_t st) {
    dim3 grid(a.max_splits, a.n_kv_heads), block(WG);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.n_heads, HD / WAVE), dim3(WG), 0, st, a);
    return hipGetLastError();
}

int attn_chunk(int head_dim) { return head_dim == 256 ? AttnShape<256>::CH : AttnShape<128>::CH; }
int attn_max_splits() { return ATTN_MAX_SPLITS; }

hipError_t launch_attn(const AttnArgs &a, int head_dim, hipStream_t st) {
    const int G = a.n_heads / a.n_kv_heads;
    if (a.max_splits > ATTN_MAX_SPLITS || a.chunk != attn_chunk(head_dim)) return hipErrorInvalidValue;
    if (head_dim == 128) return launch_attn_hd<128>(a, G, st);
    if (head_dim == 256) return launch_attn_hd<256>(a, G, st);
    return hipErrorInvalidValue;
}

}  // namespace oi
