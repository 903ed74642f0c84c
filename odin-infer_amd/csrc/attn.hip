// attn.hip -- split-L grouped-query decode attention over the f16 KV cache
// (reference: infer/forward.odin:117-175; f16 cache as infer/metal.odin:443-474).
//
// Grid: (splits, n_kv_heads).  A workgroup takes CH consecutive positions of
// one KV head and serves all G = n_heads / n_kv_heads query heads of that
// group, so each K/V row is read from HBM once per token (the reference
// re-reads it for every query head).  Per workgroup:
//   1. issue every K and V load of its positions (16 B per lane) up front,
//   2. meanwhile RMSNorm + RoPE the G query heads (and, in the split that
//      holds `pos`, the new key; K/V[pos] are rounded to f16 and stored),
//   3. scores q.k / sqrt(hd), split max and exp-sum, o = sum p v,
//   4. write (o, m, l) to a partial buffer.
// attn_combine_kernel then merges the splits of every query head with
// exp(m_s - M) weights (a separate launch: the kernel boundary orders the
// partial writes before the reads, with no fences or atomics).
// The current position is used from LDS, so no workgroup reads a cache entry
// written in the same launch.

#include "device_common.h"

namespace oi {

template <int HD>
struct AttnShape {
    static constexpr int LPP = HD / 8;     // lanes per position (8 halves = 16 B each)
    static constexpr int PPR = WG / LPP;   // positions per load round
    static constexpr int CH = 16384 / HD;  // positions per workgroup
    static constexpr int NR = CH / PPR;    // load rounds per thread
};
constexpr int ATTN_MAX_SPLITS = 512;

static __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

static __device__ __forceinline__ void unpack8(const u32x4 &w, float *out) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        out[2 * e] = h2f(ws[e] & 0xFFFFu);
        out[2 * e + 1] = h2f(ws[e] >> 16);
    }
}

template <int HD, int G>
__global__ __launch_bounds__(WG) void attn_kernel(AttnArgs a) {
    using S = AttnShape<HD>;
    constexpr int OSZ = 4 * G * HD;
    __shared__ float qr[G][HD];
    __shared__ float kp[HD], vp[HD];
    __shared__ float sc[G][S::CH];
    __shared__ float mx[G], sm[G], nrm[G + 1];
    __shared__ float obuf[OSZ];  // o reduction

    const int split = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pos = a.state[1];
    const int t0 = split * S::CH;
    if (t0 > pos) return;
    const int t1 = min(t0 + S::CH, pos + 1), n = t1 - t0;
    uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD;
    uint16_t *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    const int sub = tid % S::LPP, pslot = tid / S::LPP;

    // 1. all K and V loads of this split in flight
    u32x4 kreg[S::NR], vreg[S::NR];
#pragma unroll
    for (int j = 0; j < S::NR; j++) {
        const int tl = pslot + S::PPR * j, t = t0 + tl;
        if (tl < n && t != pos) {
            kreg[j] = ldg_nt((const u32x4 *)(kc + (size_t)t * HD) + sub);
            vreg[j] = ldg_nt((const u32x4 *)(vc + (size_t)t * HD) + sub);
        } else {
            kreg[j] = u32x4{0u, 0u, 0u, 0u};
            vreg[j] = u32x4{0u, 0u, 0u, 0u};
        }
    }

    // 2. RMSNorm + RoPE of the G query heads (and of k at pos), ops.odin:7-19
    //    and forward.odin:117-145; cos/sin come from the host-built table
    const bool has_pos = pos >= t0 && pos < t1;
    const float2 *cs = a.rope_cs + (size_t)pos * (HD / 2);
    for (int i = tid; i < G * HD; i += WG) qr[i / HD][i % HD] = a.q[(size_t)kvh * G * HD + i];
    if (has_pos)
        for (int i = tid; i < HD; i += WG) {
            kp[i] = a.k[(size_t)kvh * HD + i];
            vp[i] = a.v[(size_t)kvh * HD + i];
        }
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
        const float *w = g < G ? a.q_norm : a.k_norm;
        const float s = nrm[g];
        const float x = w[i] * (s * v[i]);
        const float y = w[i + HD / 2] * (s * v[i + HD / 2]);
        const float c = cs[i].x, sn = cs[i].y;
        v[i] = x * c - y * sn;
        v[i + HD / 2] = x * sn + y * c;
    }
    __syncthreads();
    if (has_pos) {
        for (int i = tid; i < HD; i += WG) {
            const uint16_t kb = f2h(kp[i]), vb = f2h(vp[i]);
            kc[(size_t)pos * HD + i] = kb;
            vc[(size_t)pos * HD + i] = vb;
            kp[i] = h2f(kb);
            vp[i] = h2f(vb);
        }
        __syncthreads();
    }

    // 3. scores (forward.odin:152-159: the dot is divided by sqrt(head_dim))
    const float div = sqrtf((float)HD);
#pragma unroll
    for (int j = 0; j < S::NR; j++) {
        const int tl = pslot + S::PPR * j, t = t0 + tl;
        float kv[8];
        if (t == pos) {
#pragma unroll
            for (int e = 0; e < 8; e++) kv[e] = kp[8 * sub + e];
        } else {
            unpack8(kreg[j], kv);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) d += qr[g][8 * sub + e] * kv[e];
#pragma unroll
            for (int o = S::LPP / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, S::LPP);
            if (sub == 0 && tl < n) sc[g][tl] = d / div;
        }
    }
    __syncthreads();

    // split-local softmax statistics (ops.odin:21-37 over this split)
    for (int g = wave; g < G; g += WG / WAVE) {
        float m = -INFINITY;
        for (int i = lane; i < n; i += WAVE) m = fmaxf(m, sc[g][i]);
        m = wave_max(m);
        float l = 0.f;
        for (int i = lane; i < n; i += WAVE) {
            const float e = expf(sc[g][i] - m);
            sc[g][i] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            mx[g] = m;
            sm[g] = l;
        }
    }
    __syncthreads();

    // o_g = sum_t p_g(t) v(t) over this split
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
#pragma unroll
    for (int j = 0; j < S::NR; j++) {
        const int tl = pslot + S::PPR * j, t = t0 + tl;
        if (tl < n) {
            float vv[8];
            if (t == pos) {
#pragma unroll
                for (int e = 0; e < 8; e++) vv[e] = vp[8 * sub + e];
            } else {
                unpack8(vreg[j], vv);
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sc[g][tl];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] += p * vv[e];
            }
        }
    }
#pragma unroll
    for (int o = S::LPP; o < WAVE; o <<= 1)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] += __shfl_xor(acc[g][e], o, WAVE);
    float(*ored)[G][HD] = (float(*)[G][HD])obuf;
    if (lane < S::LPP)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) ored[wave][g][8 * sub + e] = acc[g][e];
    __syncthreads();

    // 4. partial (o, m, l) of this split
    const int stride = HD + 2;
    for (int idx = tid; idx < G * HD; idx += WG) {
        const int g = idx / HD, i = idx % HD;
        const float o = (ored[0][g][i] + ored[1][g][i]) + (ored[2][g][i] + ored[3][g][i]);
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
    const int pos = a.state[1];
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
