// prefill.hip -- the per-token operations of batched prefill for T tokens at
// once (reference: qwen3_5/metal.odin:1472-1654 forward_gpu_batch; the per-token
// math is infer/forward.odin:17-146).  The projections between them run on the
// matrix cores (gemm.hip) with f16-staged operands, as the reference's MMQ; the
// kernels here take the projections' K-slice partial products directly and sum
// them in slice order, so no separate reduction runs.
//
// Layouts: activations token-major, x [T][dim] f32; the inputs of the
// projections f16 [T][K]; the KV cache f16 [n_kv_heads][seq_len][head_dim] per
// layer, shared with the decode path.  Token t sits at position pos0 + t.

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "device_common.h"

namespace oi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int BS = WG>
static __device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    __syncthreads();  // red reusable
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < BS / WAVE; w++) s += red[w];
    return s;
}

// x[t] += (sum of the K-slice partial products) when part is set, then
// out[t] = f16 of x[t]'s RMSNorm with w: w[i] * (s * x[i]), s = 1 / sqrt(sum
// x^2 / dim + eps) (ops.odin rmsnorm; the reference converts the f32 result
// to half for the projection, qwen3_5/metal.odin:1236-1242).  The residual add of one
// sublayer fused with the next sublayer's norm; x read once, kept in
// registers (NV float4 per thread).  The row, the norm weights and the first
// 16 / NV slices are requested together, the slices summed in order (one
// memory round trip per slice took ~9 us at 64 tokens and 8 slices).  With
// myd set, the addend is instead a routed-expert FFN's output, the weighted
// sum of the token's kp pair rows in slot order, sum_s mw[t kp + s] myd[t kp
// + s] (the sum of pf_moe_combine_kernel, which this replaces ahead of a norm).
// Grid: T, BS threads (512 where dim allows one float4 per thread: twice the
// loads in flight per token, 6.6 -> 5.6 us at config 5's 64-token chunk);
// dim <= BS * 4 * NV.  With xq set (and out32), the f32 norm output is also
// quantized for the int8 expert and router kernels: qi_quant_row's planes,
// group sums and scale of the row (MtGemvArgs::xq), the same values as
// launch_qi_rows computes from out32.
constexpr int PF_NPT = 64;
template <int NV, int BS = WG>
__global__ __launch_bounds__(BS) void pf_addnorm16_kernel(float *x, const float *part, int split, const float *w,
                                                          float eps, int dim, int T, uint16_t *out, float *out32,
                                                          const float *mw, const float *myd, int kp, u32x4 *xq,
                                                          float *xq_sum, float *xq_scale) {
#pragma clang fp contract(off)
    constexpr int PB = NV >= 16 ? 1 : 16 / NV;  // slices per round trip
    __shared__ float red[BS / WAVE];
    const size_t t = blockIdx.x;
    const int d4 = dim / 4;
    float4 *xt = (float4 *)(x + t * dim);
    const float4 *w4 = (const float4 *)w;
    float4 v[NV], wv[NV];
#pragma unroll
    for (int r = 0; r < NV; r++) {  // every load of the row issued before any use
        const int i = threadIdx.x + BS * r;
        if (i < d4) {
            v[r] = xt[i];
            wv[r] = w4[i];
        }
    }
    if (part) {
        const float4 *p4 = (const float4 *)part + t * d4;
        const size_t slice = (size_t)T * d4;
        for (int z0 = 0; z0 < split; z0 += PB) {
            float4 pz[PB][NV];
#pragma unroll
            for (int k = 0; k < PB; k++)
                if (z0 + k < split) {
#pragma unroll
                    for (int r = 0; r < NV; r++) {
                        const int i = threadIdx.x + BS * r;
                        if (i < d4) pz[k][r] = p4[(z0 + k) * slice + i];
                    }
                }
#pragma unroll
            for (int k = 0; k < PB; k++)
                if (z0 + k < split) {
#pragma unroll
                    for (int r = 0; r < NV; r++) {
                        const int i = threadIdx.x + BS * r;
                        if (i < d4) {
                            v[r].x += pz[k][r].x; v[r].y += pz[k][r].y; v[r].z += pz[k][r].z; v[r].w += pz[k][r].w;
                        }
                    }
                }
        }
    }
    if (myd) {
        float4 acc[NV];
#pragma unroll
        for (int r = 0; r < NV; r++) acc[r] = float4{0.f, 0.f, 0.f, 0.f};
        const float4 *y4 = (const float4 *)myd + t * kp * d4;
        for (int s0 = 0; s0 < kp; s0 += PB) {
            float4 yz[PB][NV];
            float wz[PB];
#pragma unroll
            for (int k = 0; k < PB; k++)
                if (s0 + k < kp) {
                    wz[k] = mw[t * kp + s0 + k];
#pragma unroll
                    for (int r = 0; r < NV; r++) {
                        const int i = threadIdx.x + BS * r;
                        if (i < d4) yz[k][r] = y4[(s0 + k) * d4 + i];
                    }
                }
#pragma unroll
            for (int k = 0; k < PB; k++)
                if (s0 + k < kp) {
#pragma unroll
                    for (int r = 0; r < NV; r++) {
                        acc[r].x += wz[k] * yz[k][r].x; acc[r].y += wz[k] * yz[k][r].y;
                        acc[r].z += wz[k] * yz[k][r].z; acc[r].w += wz[k] * yz[k][r].w;
                    }
                }
        }
#pragma unroll
        for (int r = 0; r < NV; r++) {
            v[r].x += acc[r].x; v[r].y += acc[r].y; v[r].z += acc[r].z; v[r].w += acc[r].w;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = threadIdx.x + BS * r;
        if (i < d4) ss += v[r].x * v[r].x + v[r].y * v[r].y + v[r].z * v[r].z + v[r].w * v[r].w;
    }
    ss = block_sum<BS>(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)dim + eps);
    uint2 *o4 = (uint2 *)(out + t * dim);
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = threadIdx.x + BS * r;
        if (i < d4) {
            if (part || myd) xt[i] = v[r];
            const float4 n{wv[r].x * (s * v[r].x), wv[r].y * (s * v[r].y), wv[r].z * (s * v[r].z),
                           wv[r].w * (s * v[r].w)};
            o4[i] = uint2{(uint32_t)f2h(n.x) | ((uint32_t)f2h(n.y) << 16), (uint32_t)f2h(n.z) | ((uint32_t)f2h(n.w) << 16)};
            if (out32) ((float4 *)(out32 + t * dim))[i] = n;
            v[r] = n;
        }
    }
    if (xq) qi_quant_row<NV, BS>(v, dim, t, red, xq, xq_sum, xq_scale);
}

// Per token and head (grid (T, ceil(heads / 4)), one wave per head; q, k
// and v heads in that order): q and k heads RMSNorm'd with
// q_norm / k_norm and rotated at pos0 + t (infer/forward.odin:57-85, pairs i and
// i + hd/2); k and v rounded to f16 into the cache at pos0 + t; q kept in f32.
// Lane l holds dimensions l + 64 e, so the RoPE pair of e is e + DPL/2.
template <int HD>
__global__ __launch_bounds__(WG) void pf_qkv_kernel(PfQkvArgs a) {
#pragma clang fp contract(off)
    constexpr int DPL = HD / WAVE;
    const int t = blockIdx.x, lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int pos = a.pos0 + t, QD = a.n_heads * HD, KVD = a.n_kv_heads * HD;
    {
        const int hh = (int)blockIdx.y * (WG / WAVE) + wave;
        if (hh >= a.n_heads + 2 * a.n_kv_heads) return;
        const bool isq = hh < a.n_heads, isk = !isq && hh < a.n_heads + a.n_kv_heads;
        const int h = isq ? hh : isk ? hh - a.n_heads : hh - a.n_heads - a.n_kv_heads;
        const float *src = isq ? a.q : isk ? a.k : a.v;
        const int split = isq ? a.qs : isk ? a.ks : a.vs;
        const int rows = isq ? QD : KVD;
        float v[DPL];
        const size_t base = (size_t)t * rows + h * HD + lane;
        parts_gather(v, src, split, (size_t)a.T * rows, [&](int e) { return base + WAVE * e; });
        if (isq || isk) {
            const float *nw = isq ? a.q_norm : a.k_norm;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; e++) ss += v[e] * v[e];
            ss = wave_sum(ss);
            const float s = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
            for (int e = 0; e < DPL; e++) v[e] = nw[lane + WAVE * e] * (s * v[e]);
#pragma unroll
            for (int e = 0; e < DPL / 2; e++) {
                const float2 cs = a.rope_cs[(size_t)pos * (HD / 2) + lane + WAVE * e];
                const float x = v[e], y = v[e + DPL / 2];
                v[e] = x * cs.x - y * cs.y;
                v[e + DPL / 2] = x * cs.y + y * cs.x;
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
}

struct PfAttnArgs {
    const float *q;             // [T][n_heads * head_dim]
    const uint16_t *kc, *vc;    // this layer's cache
    uint16_t *out;              // [T][n_heads * head_dim] f16 (the wo projection's input)
    int32_t pos0, seq_len, n_heads, n_kv_heads;
    const float *gate;          // null, or [T][n_heads * head_dim]: out *= sigmoid(gate) (Qwen3.5)
};

// the attention output of one element, gated when the layer has a gate
static __device__ __forceinline__ float pf_gated(const PfAttnArgs &a, float o, size_t i) {
#pragma clang fp contract(off)
    return a.gate ? o * sigmoid_ref(a.gate[i]) : o;
}

// Causal attention of token t (query head h, grid (n_heads, T)) over positions
// 0 .. pos0 + t of the f16 cache (infer/forward.odin:87-115: scores q.k / sqrt(hd),
// softmax, weighted sum of v).  Each wave takes blocks of 64 positions (lane =
// position) with a running max and sum; the four waves' (m, l, o) are merged
// at the end.  Lane l accumulates dimensions DPL l .. DPL l + DPL-1.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_kernel(PfAttnArgs a) {
    constexpr int DPL = HD / WAVE, NW = WG / WAVE;
    __shared__ float qs[HD];
    __shared__ float mw[NW], lw[NW];
    __shared__ float ow[NW][HD];
    const int h = blockIdx.x, t = blockIdx.y;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int QD = a.n_heads * HD, kvh = h / (a.n_heads / a.n_kv_heads), L = a.pos0 + t + 1;
    for (int i = threadIdx.x; i < HD; i += WG) qs[i] = a.q[(size_t)t * QD + h * HD + i];
    __syncthreads();
    const uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD, *vc = a.vc + (size_t)kvh * a.seq_len * HD;
    const float rs = sqrtf((float)HD);
    float m = -INFINITY, l = 0.f, o[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) o[e] = 0.f;
    for (int base = WAVE * wave; base < L; base += WG) {
        const int p = base + lane;
        float s = -INFINITY;
        if (p < L) {
            const u32x4 *kr = (const u32x4 *)(kc + (size_t)p * HD);
            float acc = 0.f;
            for (int c = 0; c < HD / 8; c++) {
                const u32x4 w = kr[c];
#pragma unroll
                for (int e = 0; e < 8; e++) acc += qs[8 * c + e] * h2f((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            }
            s = acc / rs;
        }
        float bm = s;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, WAVE));
        const float mn = fmaxf(m, bm), alpha = expf(m - mn);
        const float pj = p < L ? expf(s - mn) : 0.f;
        l = l * alpha + wave_sum(pj);
#pragma unroll
        for (int e = 0; e < DPL; e++) o[e] *= alpha;
        const int nj = min(WAVE, L - base);
        for (int j = 0; j < nj; j++) {
            const float pb = __shfl(pj, j, WAVE);
            const uint16_t *vr = vc + (size_t)(base + j) * HD + DPL * lane;
            if constexpr (DPL == 2) {
                const uint32_t w = *(const uint32_t *)vr;
                o[0] += pb * h2f(w & 0xFFFFu);
                o[1] += pb * h2f(w >> 16);
            } else {
                const u32x2 w = *(const u32x2 *)vr;
#pragma unroll
                for (int e = 0; e < DPL; e++) o[e] += pb * h2f((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
            }
        }
        m = mn;
    }
    if (lane == 0) {
        mw[wave] = m;
        lw[wave] = l;
    }
#pragma unroll
    for (int e = 0; e < DPL; e++) ow[wave][DPL * lane + e] = o[e];
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, mw[w]);
    float lt = 0.f, sc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) {
        sc[w] = mw[w] == -INFINITY ? 0.f : expf(mw[w] - M);  // a wave with no positions adds nothing
        lt += lw[w] * sc[w];
    }
    for (int i = threadIdx.x; i < HD; i += WG) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) acc += ow[w][i] * sc[w];
        a.out[(size_t)t * QD + h * HD + i] = f2h(pf_gated(a, acc / lt, (size_t)t * QD + h * HD + i));
    }
}

// Causal attention on the matrix cores for head_dim 128 or 256, grid (n_heads,
// ceil(T / 64)): a workgroup takes 64 queries of one head (wave w: queries
// 16w .. 16w+15) and walks the keys in blocks of 64 up to its last query's
// position.  Per block, K (rows padded to HD + 8 halves) and V transposed (V^T,
// rows of 68 halves) are staged in LDS; then per wave
//   S^T[key][query] = K Q^T  (v_mfma_f32_16x16x32_f16; A = K rows, B = Q),
//   online softmax per query (running max, exp, running sum),
//   O^T[d][query] += V^T P^T (A = V^T rows, B = P).
// In the S^T result lane (q, g) holds keys 4g+e of each 16-key tile for query
// q, which is, without any lane exchange, the B operand of the second product
// when its K index k = 8g + e stands for key 4g + e (e < 4) or 16 + 4g + e - 4
// of a 32-key chunk; V^T is read with the same map.  Precision: q and p are
// split into f16 hi + lo halves (two products each), K and V are exact f16,
// accumulation is f32, so scores and weights keep about 22 bits, close to the
// reference's f32 arithmetic (infer/forward.odin:87-115).
constexpr int FA_VP = 68;  // LDS row stride (halves) of V^T; K rows: HD + 8

static __device__ __forceinline__ void split16(const float (&v)[8], h8 &hi, h8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        hi[e] = (_Float16)v[e];
        lo[e] = (_Float16)(v[e] - (float)hi[e]);
    }
}

// SPLIT: the key blocks are divided over gridDim.z workgroups (a short chunk
// has too few query tiles to fill the GPU); each writes its queries'
// unnormalized (o, m, l) to ws [split][T][n_heads][HD + 2] and
// pf_fattn_merge_kernel combines them.
template <int HD, bool SPLIT = false>
__global__ __launch_bounds__(WG) void pf_fattn_kernel(PfAttnArgs a, int T, float *ws = nullptr) {
    constexpr int FA_KP = HD + 8, NC = HD / 32, NDT = HD / 16;  // K row stride; 32-wide K chunks; 16-wide d tiles
    __shared__ __attribute__((aligned(16))) uint16_t ks[64 * FA_KP];
    __shared__ __attribute__((aligned(16))) uint16_t vt[HD * FA_VP];
    const int h = blockIdx.x, t0 = 64 * (int)blockIdx.y;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int q = lane & 15, g = lane >> 4;
    const int QD = a.n_heads * HD, kvh = h / (a.n_heads / a.n_kv_heads);
    const int tq = t0 + 16 * wave + q;                    // this lane's query (token)
    const int qpos = a.pos0 + min(tq, T - 1);             // its position
    const int last = a.pos0 + min(t0 + 63, T - 1);        // the workgroup's last query position
    const int lmax = a.pos0 + T;                          // cache rows written so far
    const uint16_t *kc = a.kc + (size_t)kvh * a.seq_len * HD, *vc = a.vc + (size_t)kvh * a.seq_len * HD;

    // B operand of S^T: Q[query q][d = 32c + 8g + e], hi and lo halves
    h8 qh[NC], ql[NC];
    {
        const float *qr = a.q + (size_t)min(tq, T - 1) * QD + h * HD;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float v[8];
            const float4 v0 = *(const float4 *)(qr + 32 * c + 8 * g), v1 = *(const float4 *)(qr + 32 * c + 8 * g + 4);
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
            split16(v, qh[c], ql[c]);
        }
    }
    const float rs = sqrtf((float)HD);
    float m = -INFINITY, lsum = 0.f;
    f32x4v o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = f32x4v{0.f, 0.f, 0.f, 0.f};

    int kb0 = 0, kb1 = last / 64 + 1;  // this workgroup's key blocks
    if (SPLIT) {
        const int nb = kb1, ns = (int)gridDim.z, z = (int)blockIdx.z;
        kb0 = (int)((long)nb * z / ns);
        kb1 = (int)((long)nb * (z + 1) / ns);
    }
    for (int kb = kb0; kb < kb1; kb++) {
        // stage K and V^T of keys 64 kb .. +63 (rows past the written range
        // re-read the last written row; their scores are masked)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 64 * (HD / 8) / WG; i++) {
            const int piece = threadIdx.x + WG * i, r = piece / (HD / 8), c8 = piece % (HD / 8);  // row r, 8 halves at 8 c8
            const int p = min(64 * kb + r, lmax - 1);
            const u32x4 kv = *(const u32x4 *)(kc + (size_t)p * HD + 8 * c8);
            *(u32x4 *)(ks + r * FA_KP + 8 * c8) = kv;
            const u32x4 vv = *(const u32x4 *)(vc + (size_t)p * HD + 8 * c8);
#pragma unroll
            for (int e = 0; e < 8; e++) vt[(8 * c8 + e) * FA_VP + r] = (uint16_t)((vv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
        }
        __syncthreads();
        // S^T tiles kt (keys 16 kt + 4g + e for query q)
        float s[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f32x4v acc = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const h8 kA = __builtin_bit_cast(h8, *(const u32x4 *)(ks + (16 * kt + q) * FA_KP + 32 * c + 8 * g));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kA, qh[c], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kA, ql[c], acc, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int p = 64 * kb + 16 * kt + 4 * g + e;
                s[kt][e] = p <= qpos ? acc[e] / rs : -INFINITY;
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) bm = fmaxf(bm, s[kt][e]);
        bm = fmaxf(bm, __shfl_xor(bm, 16, WAVE));
        bm = fmaxf(bm, __shfl_xor(bm, 32, WAVE));
        // (a key-split block may have no key visible to this query yet: m and
        // mn stay -inf and nothing is added)
        const float mn = fmaxf(m, bm), alpha = mn == -INFINITY ? 1.f : expf(m - mn);
        m = mn;
        float ps = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s[kt][e] = mn == -INFINITY ? 0.f : expf(s[kt][e] - mn);
                ps += s[kt][e];
            }
        lsum = lsum * alpha + ps;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[dt] *= alpha;
        // O^T += V^T P^T over the two 32-key chunks
#pragma unroll
        for (int kc2 = 0; kc2 < 2; kc2++) {
            float pv[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pv[e] = s[2 * kc2][e];
                pv[4 + e] = s[2 * kc2 + 1][e];
            }
            h8 ph, pl;
            split16(pv, ph, pl);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const uint16_t *vr = vt + (16 * dt + q) * FA_VP + 32 * kc2 + 4 * g;
                const u32x2 v0 = *(const u32x2 *)vr, v1 = *(const u32x2 *)(vr + 16);
                const h8 vA = __builtin_bit_cast(h8, u32x4{v0.x, v0.y, v1.x, v1.y});
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vA, ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vA, pl, o[dt], 0, 0, 0);
            }
        }
    }
    lsum += __shfl_xor(lsum, 16, WAVE);
    lsum += __shfl_xor(lsum, 32, WAVE);
    if (SPLIT) {  // this split's (o, m, l) of the lane's query
        if (tq < T) {
            float *pp = ws + (((size_t)blockIdx.z * T + tq) * a.n_heads + h) * (HD + 2);
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) *(float4 *)(pp + 16 * dt + 4 * g) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
            if (g == 0) {
                pp[HD] = m;
                pp[HD + 1] = lsum;
            }
        }
        return;
    }
    if (tq < T) {
        const size_t d0 = (size_t)tq * QD + h * HD + 4 * g;
        uint16_t *dst = a.out + d0;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            float r[4];
#pragma unroll
            for (int e = 0; e < 4; e++) r[e] = pf_gated(a, o[dt][e] / lsum, d0 + 16 * dt + e);
            const uint32_t w0 = (uint32_t)f2h(r[0]) | ((uint32_t)f2h(r[1]) << 16);
            const uint32_t w1 = (uint32_t)f2h(r[2]) | ((uint32_t)f2h(r[3]) << 16);
            *(u32x2 *)(dst + 16 * dt) = u32x2{w0, w1};
        }
    }
}

// The splits of pf_fattn_kernel<HD, true> for token t and head h (grid (T,
// n_heads), thread d): O = sum_s e^{m_s - M} o_s / sum_s e^{m_s - M} l_s.
template <int HD>
__global__ __launch_bounds__(HD) void pf_fattn_merge_kernel(PfAttnArgs a, int T, const float *ws, int ns) {
#pragma clang fp contract(off)
    const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x, QD = a.n_heads * HD;
    const size_t stride = (size_t)T * a.n_heads * (HD + 2), base = ((size_t)t * a.n_heads + h) * (HD + 2);
    float M = -INFINITY;
    for (int z = 0; z < ns; z++) M = fmaxf(M, ws[z * stride + base + HD]);
    float L = 0.f, O = 0.f;
    for (int z = 0; z < ns; z++) {
        const float mz = ws[z * stride + base + HD];
        const float f = mz == -INFINITY ? 0.f : expf(mz - M);  // a split with no visible key adds nothing
        L += f * ws[z * stride + base + HD + 1];
        O += f * ws[z * stride + base + d];
    }
    const size_t i = (size_t)t * QD + h * HD + d;
    a.out[i] = f2h(pf_gated(a, O / L, i));
}

// x[i] += sum of the partial products of element i (the residual adds,
// infer/forward.odin:119-121, 137-139)
__global__ __launch_bounds__(WG) void pf_add_kernel(float *x, const float *part, int split, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i < total) x[i] += parts_at(part, split, (size_t)total, (size_t)i);
}

// out[i] = f16(silu(g[i]) * u[i]) from the gate and up projections' partial
// products (infer/forward.odin:128-132, separately rounded as the reference)
__global__ __launch_bounds__(WG) void pf_swiglu16_kernel(const float *g, int gs, const float *u, int us, int64_t total,
                                                         uint16_t *out) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i >= total) return;
    float val = parts_at(g, gs, (size_t)total, (size_t)i);
    val *= 1.0f / (1.0f + expf(-val));
    val *= parts_at(u, us, (size_t)total, (size_t)i);
    out[i] = f2h(val);
}

static unsigned blocks(int64_t n) { return (unsigned)((n + WG - 1) / WG); }

// OI_PREFILL_ATTN=lanes: head_dim 256 always on the lane-per-position kernel (tests)
static bool pf_attn_lanes() {
    const char *e = std::getenv("OI_PREFILL_ATTN");
    return e && std::strcmp(e, "lanes") == 0;
}

hipError_t launch_pf_qkv(const PfQkvArgs &a, int head_dim, hipStream_t st) {
    const dim3 grid((unsigned)a.T, (unsigned)((a.n_heads + 2 * a.n_kv_heads + WG / WAVE - 1) / (WG / WAVE)));
    if (head_dim == 128) hipLaunchKernelGGL(pf_qkv_kernel<128>, grid, dim3(WG), 0, st, a);
    else if (head_dim == 256) hipLaunchKernelGGL(pf_qkv_kernel<256>, grid, dim3(WG), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_attn(const float *q, const uint16_t *kc, const uint16_t *vc, uint16_t *out, int T, int pos0,
                          int seq_len, int n_heads, int n_kv_heads, int head_dim, hipStream_t st, const float *gate,
                          float *ws, size_t ws_bytes) {
    PfAttnArgs a{q, kc, vc, out, pos0, seq_len, n_heads, n_kv_heads, gate};
    const dim3 grid((unsigned)n_heads, (unsigned)T);
    const dim3 fgrid((unsigned)n_heads, (unsigned)((T + 63) / 64));
    // a short chunk at head_dim 256: the key blocks split over workgroups (up
    // to 16 per query tile, at least 2 blocks each) when the workspace holds
    // the partials
    const int nkb = (pos0 + T + 63) / 64, qt = (T + 63) / 64;
    const size_t per = (size_t)T * n_heads * (head_dim + 2) * 4;
    int ns = std::min(16, nkb / 2);
    if (ws && per > 0) ns = std::min<int>(ns, (int)(ws_bytes / per));
    if (head_dim == 256 && T < 128 && !pf_attn_lanes() && ws && ns >= 2 && qt * n_heads < 256) {
        hipLaunchKernelGGL((pf_fattn_kernel<256, true>), dim3((unsigned)n_heads, (unsigned)qt, (unsigned)ns), dim3(WG),
                           0, st, a, T, ws);
        hipLaunchKernelGGL(pf_fattn_merge_kernel<256>, dim3((unsigned)T, (unsigned)n_heads), dim3(256), 0, st, a, T,
                           (const float *)ws, ns);
        return hipGetLastError();
    }
    if (head_dim == 128) hipLaunchKernelGGL((pf_fattn_kernel<128>), fgrid, dim3(WG), 0, st, a, T, nullptr);
    // head_dim 256: the matrix cores from 128 tokens on; a shorter chunk gives
    // them one workgroup per head only (16 at config 5), where one workgroup per
    // (head, token) on the lane-per-position kernel is faster
    else if (head_dim == 256 && T >= 128 && !pf_attn_lanes())
        hipLaunchKernelGGL((pf_fattn_kernel<256>), fgrid, dim3(WG), 0, st, a, T, nullptr);
    else if (head_dim == 256) hipLaunchKernelGGL(pf_attn_kernel<256>, grid, dim3(WG), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_addnorm16(float *x, const float *part, int split, const float *w, float eps, int dim, int T,
                               uint16_t *out, hipStream_t st, float *out32, const float *mw, const float *myd, int kp,
                               void *xq, float *xq_sum, float *xq_scale) {
    if (dim > WG * PF_NPT || (myd && (part || !mw || kp < 1))) return hipErrorInvalidValue;
    if (xq && (!out32 || !xq_sum || !xq_scale || dim % 256 || dim > 4096)) return hipErrorInvalidValue;
    u32x4 *q = (u32x4 *)xq;
    const int nv = (dim / 4 + WG - 1) / WG;
#define PF_AN(NV)                                                                                              \
    hipLaunchKernelGGL(pf_addnorm16_kernel<NV>, dim3(T), dim3(WG), 0, st, x, part, split, w, eps, dim, T, out, out32, \
                       mw, myd, kp, q, xq_sum, xq_scale)
    if (dim / 4 <= 2 * WG && dim / 4 > WG)
        hipLaunchKernelGGL((pf_addnorm16_kernel<1, 2 * WG>), dim3(T), dim3(2 * WG), 0, st, x, part, split, w, eps, dim, T,
                           out, out32, mw, myd, kp, q, xq_sum, xq_scale);
    else if (nv <= 1) PF_AN(1);
    else if (nv <= 2) PF_AN(2);
    else if (nv <= 4) PF_AN(4);
    else if (nv <= 8) PF_AN(8);
    else PF_AN(16);
#undef PF_AN
    return hipGetLastError();
}

hipError_t launch_pf_add(float *x, const float *part, int split, int64_t total, hipStream_t st) {
    hipLaunchKernelGGL(pf_add_kernel, dim3(blocks(total)), dim3(WG), 0, st, x, part, split, total);
    return hipGetLastError();
}

hipError_t launch_pf_swiglu16(const float *g, int gs, const float *u, int us, int64_t total, uint16_t *out,
                              hipStream_t st) {
    hipLaunchKernelGGL(pf_swiglu16_kernel, dim3(blocks(total)), dim3(WG), 0, st, g, gs, u, us, total, out);
    return hipGetLastError();
}

}  // namespace oi
