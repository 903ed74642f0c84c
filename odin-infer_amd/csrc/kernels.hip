// kernels.hip -- gfx950 kernels of the decode token loop.
//
//   gemv_kernel    GEMV for any device type (F32, F16, Q8_0, Q4_0, Q4_1, Q5_0,
//                  Q5_1, Q4_K, Q6_K) in
//                  float arithmetic, with the same fused prologue/epilogues as
//                  gemv_q_kernel (gemv.hip), used where that one does not apply
//                  (reference: infer/matmul.odin:77-109, ggml/quant.odin:76-282)
//   embed_kernel   token embedding row (infer/forward.odin:12-15, 43), preceded by the
//                  reduction of the previous step's argmax partials
//                  (sampler/sampler.odin:79-89)
//   dequant_kernel bit-exact dequant of a matrix (test hook)
//   moe_*          routed-expert FFN for shapes the quantized GEMV does not take
//   kv_export/import_kernel  f16 head-major cache <-> f32 position-major rows
//                  (the .oikv state file's layout)
//
// Wave64 throughout; workgroups of 256 threads (4 waves).

#include <algorithm>

#include "device_common.h"

namespace oi {

// --------------------------------------------------------------------------
// Bit-exact unit decoders (64 weights each).  Contraction is off so every
// product and difference is rounded separately, as in the reference.
// --------------------------------------------------------------------------

// Q4_K unit u of a row: ggml/quant.odin:178-209
__device__ void decode_unit_q4k(const DMat &m, int row, int u, float *out) {
#pragma clang fp contract(off)
    const int U = m.cols >> 6, p = u & 3;
    const size_t ui = (size_t)row * U + u;
    const u32x4 hdr = *(const u32x4 *)(m.s + ((size_t)row * (m.cols >> 8) + (u >> 2)) * 16);
    const u32x4 q0 = *(const u32x4 *)(m.q + ui * 16);
    const u32x4 q1 = *(const u32x4 *)(m.q + m.plane + ui * 16);
    const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    uint32_t sc0, m0, sc1, m1;
    q4k_scales(p, hdr.y, hdr.z, hdr.w, sc0, m0, sc1, m1);
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int l = 0; l < 32; l++) {
        const uint32_t b = (qw[l >> 2] >> ((l & 3) * 8)) & 0xFFu;
        out[l] = d1 * (float)(b & 0xFu) - mm1;
        out[32 + l] = d2 * (float)(b >> 4) - mm2;
    }
}

// Q6_K unit u: ggml/quant.odin:212-247.  out[16k + i] is element
// 128h + 32k + l0 + i of the super-block.
__device__ void decode_unit_q6k(const DMat &m, int row, int u, float *out) {
#pragma clang fp contract(off)
    const int U = m.cols >> 6, nsb = m.cols >> 8;
    const int sb = u >> 2, h = (u >> 1) & 1, l0 = (u & 1) * 16;
    const size_t ui = (size_t)row * U + u, sbi = (size_t)row * nsb + sb;
    const uint8_t *qlA = m.q + ui * 16;                // ql[64h + l0 + i]
    const uint8_t *qlB = m.q + m.plane + ui * 16;      // ql[64h + 32 + l0 + i]
    const uint8_t *qh = m.q + 2 * m.plane + ui * 16;   // qh[32h + l0 + i]
    const int8_t *sc = (const int8_t *)(m.s + sbi * 16) + 8 * h;
    const float d = h2f(m.d[sbi]);
    const int is = l0 / 16;
    for (int i = 0; i < 16; i++) {
        const int q1 = (int)((qlA[i] & 0xF) | (((qh[i] >> 0) & 3) << 4)) - 32;
        const int q2 = (int)((qlB[i] & 0xF) | (((qh[i] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((qlA[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((qlB[i] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32;
        out[i] = d * (float)sc[is + 0] * (float)q1;
        out[16 + i] = d * (float)sc[is + 2] * (float)q2;
        out[32 + i] = d * (float)sc[is + 4] * (float)q3;
        out[48 + i] = d * (float)sc[is + 6] * (float)q4;
    }
}

// The 32-element block types kept in their GGUF layout (rows of cols/32
// blocks of bb bytes): unit u is blocks 2u and 2u+1 of the row,
// ggml/quant.odin:98-162 (separately rounded mul then add; element j and
// j + 16 from the low and high nibble of byte j).
__device__ void decode_unit_legacy(const DMat &m, int row, int u, float *out) {
#pragma clang fp contract(off)
    const int bb = m.type == T_Q4_0 ? 18 : m.type == T_Q4_1 ? 20 : m.type == T_Q5_0 ? 22 : 24;
    const uint8_t *rowp = m.q + (size_t)row * (m.cols >> 5) * bb;
    for (int h = 0; h < 2; h++) {
        const uint8_t *b = rowp + (size_t)(2 * u + h) * bb;
        const float d = h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        float *o = out + 32 * h;
        if (m.type == T_Q4_0) {
            for (int j = 0; j < 16; j++) {
                o[j] = (float)((int)(b[2 + j] & 0xF) - 8) * d;
                o[j + 16] = (float)((int)(b[2 + j] >> 4) - 8) * d;
            }
        } else if (m.type == T_Q4_1) {
            const float mn = h2f((uint32_t)b[2] | ((uint32_t)b[3] << 8));
            for (int j = 0; j < 16; j++) {
                o[j] = (float)(b[4 + j] & 0xF) * d + mn;
                o[j + 16] = (float)(b[4 + j] >> 4) * d + mn;
            }
        } else {
            const bool q51 = m.type == T_Q5_1;
            const float mn = q51 ? h2f((uint32_t)b[2] | ((uint32_t)b[3] << 8)) : 0.f;
            const uint8_t *qhp = b + (q51 ? 4 : 2), *qs = b + (q51 ? 8 : 6);
            const uint32_t qh = (uint32_t)qhp[0] | (uint32_t)qhp[1] << 8 | (uint32_t)qhp[2] << 16 | (uint32_t)qhp[3] << 24;
            for (int j = 0; j < 16; j++) {
                const uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
                const int x0 = (int)((qs[j] & 0xFu) | xh0), x1 = (int)((qs[j] >> 4) | xh1);
                if (q51) {
                    o[j] = (float)x0 * d + mn;
                    o[j + 16] = (float)x1 * d + mn;
                } else {
                    o[j] = (float)(x0 - 16) * d;
                    o[j + 16] = (float)(x1 - 16) * d;
                }
            }
        }
    }
}

// Any type: decode unit u of `row` into out[64] (order: see unit_elem).
__device__ void decode_unit(const DMat &m, int row, int u, float *out) {
#pragma clang fp contract(off)
    switch (m.type) {
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: decode_unit_legacy(m, row, u, out); break;
    case T_Q4_K: decode_unit_q4k(m, row, u, out); break;
    case T_Q6_K: decode_unit_q6k(m, row, u, out); break;
    case T_Q8_0: {  // ggml/quant.odin:87-96
        const size_t ui = (size_t)row * (m.cols >> 6) + u;
        const size_t b0 = (size_t)row * (m.cols >> 5) + 2 * u;
        for (int c = 0; c < 4; c++) {
            const float d = h2f(m.d[b0 + (c >> 1)]);
            const int8_t *qs = (const int8_t *)(m.q + c * m.plane + ui * 16);
            for (int j = 0; j < 16; j++) out[16 * c + j] = d * (float)qs[j];
        }
        break;
    }
    case T_F16: {
        const uint16_t *p = (const uint16_t *)m.q + (size_t)row * m.cols + 64 * u;
        for (int j = 0; j < 64; j++) out[j] = h2f(p[j]);
        break;
    }
    default: {  // F32
        const float *p = (const float *)m.q + (size_t)row * m.cols + 64 * u;
        for (int j = 0; j < 64; j++) out[j] = p[j];
        break;
    }
    }
}

// Element index (within the row) of the j-th value that decode_unit writes.
__device__ __forceinline__ int unit_elem(int type, int u, int j) {
    if (type == T_Q6_K) {
        const int sb = u >> 2, h = (u >> 1) & 1, l0 = (u & 1) * 16;
        return 256 * sb + 128 * h + 32 * (j >> 4) + l0 + (j & 15);
    }
    return 64 * u + j;
}

// --------------------------------------------------------------- dequant --
__global__ __launch_bounds__(WG) void dequant_kernel(DMat m, float *out) {
    const int units = m.cols / 64;
    const long gid = (long)blockIdx.x * WG + threadIdx.x;
    if (gid >= (long)m.rows * units) return;
    const int row = (int)(gid / units), u = (int)(gid % units);
    float v[64];
    decode_unit(m, row, u, v);
    float *o = out + (size_t)row * m.cols;
    for (int j = 0; j < 64; j++) o[unit_elem(m.type, u, j)] = v[j];
}

// ------------------------------------------------------------- embedding --
// x[t] = dequant(token_embd[tokens[t]]) for the tokens of a prefill batch
// (forward_gpu_batch's get_embedding_row per token, qwen3_5/metal.odin:1499-1501).
// Grid (ceil(units / WG), n): one unit of 64 weights per thread.
__global__ __launch_bounds__(WG) void embed_rows_kernel(DMat emb, const int32_t *tokens, float *x) {
    const int units = emb.cols / 64, u = (int)blockIdx.x * WG + threadIdx.x, t = blockIdx.y;
    if (u >= units) return;
    float v[64];
    decode_unit(emb, tokens[t], u, v);
    float *o = x + (size_t)t * emb.cols;
    for (int j = 0; j < 64; j++) o[unit_elem(emb.type, u, j)] = v[j];
}

static // x = dequant(token_embd[token]) (infer/forward.odin:72-75, 103)
__global__ __launch_bounds__(WG) void embed_kernel(DMat emb, int32_t *state, float *x, int32_t vocab,
                                                   const float *am_val, const int32_t *am_idx, int32_t *tokens_out,
                                                   int finalize_only) {
    __shared__ float rv[WG / WAVE];
    __shared__ int ri[WG / WAVE];
    __shared__ int tok_s;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int pending = state[ST_PENDING];
    if (pending) {  // first maximum of the previous logits wins
        const int npart = state[ST_NPART];
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int i = tid; i < npart; i += WG)
            if (better(am_val[i], am_idx[i], bv, bi)) {
                bv = am_val[i];
                bi = am_idx[i];
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, WAVE);
            const int oi = __shfl_xor(bi, o, WAVE);
            if (better(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            rv[wave] = bv;
            ri[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < WG / WAVE; w++)
                if (better(rv[w], ri[w], bv, bi)) {
                    bv = rv[w];
                    bi = ri[w];
                }
            if (bi == 0x7FFFFFFF) bi = 0;  // all NaN: index 0, as the reference's scan
            const int step = state[ST_STEP];
            if (tokens_out && step >= 0 && step < state[ST_CAP]) tokens_out[step] = bi;
            state[ST_STEP] = step + 1;
            state[ST_TOKEN] = bi;
            state[ST_POS] = state[ST_POS] + 1;
            state[ST_PENDING] = 0;
            tok_s = bi;
        }
    } else if (tid == 0) {
        tok_s = state[ST_TOKEN];
    }
    __syncthreads();
    if (finalize_only) return;
    int tok = tok_s;
    if (tok < 0 || tok >= vocab) tok = 0;  // the host checks the range first
    const int units = emb.cols / 64;
    for (int u = tid; u < units; u += WG) {
        float v[64];
        decode_unit(emb, tok, u, v);
        for (int j = 0; j < 64; j++) x[unit_elem(emb.type, u, j)] = v[j];
    }
}

// ------------------------------------------------------------------ GEMV --


// x in LDS: float4 chunk c (elements 4c..4c+3) lives at a swizzled slot so
// that the 64 lanes of a wave, each reading chunk k of its own 64-element
// unit, hit distinct banks.
__device__ __forceinline__ int xswz(int c) { return (c & ~15) | ((c & 15) ^ ((c >> 4) & 15)); }

struct XView {
    const float4 *x4;  // LDS, swizzled
    const float *s16;  // LDS, sums of 16 consecutive elements
    __device__ __forceinline__ float4 chunk(int c) const { return x4[xswz(c)]; }
};

__device__ __forceinline__ float dot4_nib(uint32_t w, float4 x) {
    // four bytes of w, each 0..255, times x
    return (float)(w & 0xFFu) * x.x + (float)((w >> 8) & 0xFFu) * x.y + (float)((w >> 16) & 0xFFu) * x.z +
           (float)(w >> 24) * x.w;
}

// dot of one unit of the row with x (from LDS), via the exact decode
__device__ __forceinline__ float dot_unit(const DMat &m, int row, int u, const XView &xv) {
    if (m.type == T_F32) {
        const float4 *p = (const float4 *)((const float *)m.q + (size_t)row * m.cols + 64 * u);
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 w = p[i];
            const float4 x = xv.chunk(u * 16 + i);
            a += w.x * x.x + w.y * x.y + w.z * x.z + w.w * x.w;
        }
        return a;
    }
    float w[64];
    decode_unit(m, row, u, w);
    float a = 0.f;
    for (int j = 0; j < 64; j++) {
        const int g = unit_elem(m.type, u, j);  // element of the row
        a += w[j] * ((const float *)&xv.x4[xswz(g >> 2)])[g & 3];
    }
    return a;
}

// acc[r] += sum over lane units of row rows[r] (r < R); rows >= m.rows skipped
template <int R>
__device__ __forceinline__ void gemv_rows(const DMat &m, const int *rows, int j, int lpr, const XView &xv,
                                          float *acc) {
    const int U = m.cols >> 6;
    for (int u = j; u < U; u += lpr)
#pragma unroll
        for (int r = 0; r < R; r++)
            if (rows[r] < m.rows) acc[r] += dot_unit(m, rows[r], u, xv);
}

// Workgroup tile: 4 waves; each wave holds 64/lpr lane groups; each group
// owns R consecutive rows and lpr lanes that split the row's units.
template <int R>
__global__ __launch_bounds__(WG) void gemv_kernel(GemvArgs a) {
    extern __shared__ float4 smem[];
    __shared__ float red[WG / WAVE];
    __shared__ int redi[WG / WAVE];
    const int K = a.K, tid = threadIdx.x;
    float4 *x4 = smem;
    float *s16 = (float *)(smem + K / 4);

    // ---- prologue: x (optionally RMS-normalised, infer/ops.odin:7-19) into LDS
    const float4 *gx = (const float4 *)a.x;
    float s = 1.f;
    if (a.norm_w) {
        float ss = 0.f;
        for (int c = tid; c < K / 4; c += WG) {
            const float4 v = gx[c];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if ((tid & (WAVE - 1)) == 0) red[tid / WAVE] = ss;
        __syncthreads();
        ss = red[0] + red[1] + red[2] + red[3];
        s = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    {
#pragma clang fp contract(off)
        const float4 *nw = (const float4 *)a.norm_w;
        for (int c = tid; c < K / 4; c += WG) {
            float4 v = gx[c];
            if (nw) {
                const float4 w = nw[c];
                v.x = w.x * (s * v.x);
                v.y = w.y * (s * v.y);
                v.z = w.z * (s * v.z);
                v.w = w.w * (s * v.w);
            }
            x4[xswz(c)] = v;
        }
    }
    __syncthreads();
    for (int g = tid; g < K / 16; g += WG) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = x4[xswz(4 * g + i)];
            t += (v.x + v.y) + (v.z + v.w);
        }
        s16[g] = t;
    }
    __syncthreads();
    const XView xv{x4, s16};

    // ---- segment and rows of this workgroup
    const int wg = blockIdx.x;
    int seg = 0;
    if (a.nseg > 1 && a.mode != GEMV_SWIGLU && wg >= a.seg[1].wg_begin) seg = 1;
    for (int i = 2; i < a.nseg; i++)
        if (wg >= a.seg[i].wg_begin) seg = i;
    const GemvSeg &S = a.seg[seg];
    const int lane = tid & (WAVE - 1), wave = tid / WAVE;
    const int lpr = a.lpr, gpw = WAVE / lpr;
    const int grp = lane / lpr, j = lane & (lpr - 1);
    const int row0 = (wg - S.wg_begin) * a.rows_per_wg + (wave * gpw + grp) * R;
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = row0 + r;

    float acc[R], acc2[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = acc2[r] = 0.f;
    gemv_rows<R>(S.m, rows, j, lpr, xv, acc);
    if (a.mode == GEMV_SWIGLU) gemv_rows<R>(a.seg[1].m, rows, j, lpr, xv, acc2);

    // reduce over the lpr lanes of the group
    for (int o = lpr >> 1; o > 0; o >>= 1) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] += __shfl_xor(acc[r], o, WAVE);
            if (a.mode == GEMV_SWIGLU) acc2[r] += __shfl_xor(acc2[r], o, WAVE);
        }
    }

    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    if (j == 0) {
#pragma clang fp contract(off)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = rows[r];
            if (row >= S.m.rows) continue;
            if (a.mode == GEMV_ADD) {
                S.y[row] += a.ygate ? acc[r] * (1.0f / (1.0f + expf(-a.ygate[0]))) : acc[r];
            } else if (a.mode == GEMV_SWIGLU) {  // infer/forward.odin:128-132
                float val = acc[r];
                val *= 1.0f / (1.0f + expf(-val));
                val *= acc2[r];
                S.y[row] = val;
            } else {
                S.y[row] = acc[r];
                if (better(acc[r], row, bv, bi)) { bv = acc[r]; bi = row; }
            }
        }
    }
    if (a.mode != GEMV_ARGMAX) return;

    // ---- greedy argmax partial of this workgroup (first maximum wins)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, WAVE);
        const int oi = __shfl_xor(bi, o, WAVE);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { red[wave] = bv; redi[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < WG / WAVE; w++)
            if (better(red[w], redi[w], bv, bi)) { bv = red[w]; bi = redi[w]; }
        a.am_val[wg] = bv;
        a.am_idx[wg] = bi;
        if (wg == 0) a.state[ST_PENDING] = 1;
    }
}

bool plan_gemv(GemvArgs &a) {
    if (a.K <= 0 || a.K % 64 || a.nseg < 1 || a.nseg > GEMV_MAX_SEG) return false;
    if (gemv_q_supported(a)) {
        plan_gemv_q(a);
        return true;
    }
    if (a.gss || a.conv_w) return false;  // prologue / epilogue of gemv_q_kernel only
    a.kernel = 0;
    const int U = a.K / 64;
    int lpr = 1;
    while (lpr < 64 && U % (lpr * 2) == 0) lpr *= 2;
    a.lpr = lpr;
    const int gpw = 64 / lpr;
    long rows = 0;
    for (int i = 0; i < (a.mode == GEMV_SWIGLU ? 1 : a.nseg); i++) rows += a.seg[i].m.rows;
    // rows per lane group: the largest R in {4,2,1} that still gives >= 512 workgroups
    int R = 4;
    while (R > 1 && rows / (4L * gpw * R) < 512) R >>= 1;
    if (a.mode == GEMV_SWIGLU && R > 2) R = 2;
    a.rows_per_wg = 4 * gpw * R;
    int wg = 0;
    for (int i = 0; i < a.nseg; i++) {
        a.seg[i].wg_begin = wg;
        if (a.mode == GEMV_SWIGLU && i == 1) {
            a.seg[1].wg_begin = 0;
            break;
        }
        wg += (a.seg[i].m.rows + a.rows_per_wg - 1) / a.rows_per_wg;
    }
    a.total_wgs = wg;
    return true;
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t st) {
    if (a.kernel == 1) return launch_gemv_q(a, st);
    const size_t lds = (size_t)a.K * 4 + (size_t)(a.K / 16) * 4;
    const int R = a.rows_per_wg / (4 * (64 / a.lpr));
    dim3 grid(a.total_wgs), block(WG);
    switch (R) {
    case 4: hipLaunchKernelGGL(gemv_kernel<4>, grid, block, lds, st, a); break;
    case 2: hipLaunchKernelGGL(gemv_kernel<2>, grid, block, lds, st, a); break;
    default: hipLaunchKernelGGL(gemv_kernel<1>, grid, block, lds, st, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_embed(const DMat &emb, int32_t *state, float *x, int32_t vocab, const float *am_val,
                        const int32_t *am_idx, int32_t *tokens_out, int finalize_only, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(WG), 0, st, emb, state, x, vocab, am_val, am_idx, tokens_out,
                       finalize_only);
    return hipGetLastError();
}

// ------------------------------------------------------------------- MoE --
// Router top-k and the selected experts' SwiGLU FFN for one token, with the
// expert ids chosen on the device.  The reference has no MoE code
// (qwen3_5/model.odin:80-82 and qwen3_5/forward.odin:227-243 are dense); the
// convention is HF Qwen3-MoE's: softmax over all router logits, the top k
// (ties to the lower id), optionally renormalized to sum 1; expert e:
// down_e(silu(gate_e x) * up_e x); output sum_k w_k y_k.  Expert matrices are
// stacked: gate and up [n_experts * inter][dim], down [n_experts * dim][inter].


// one workgroup: softmax of the n router logits, then every expert's rank
// (the number of experts with a larger p, or an equal p and a lower id:
// the order of k rounds of first-maximum argmax) computed in parallel; the
// experts of rank < k write their id and weight (p or p / sum of the chosen)
__global__ __launch_bounds__(WG) void moe_topk_kernel(MoeArgs a) {
#pragma clang fp contract(off)
    __shared__ float p[MOE_MAX_EXPERTS];
    __shared__ float red[WG / WAVE];
    __shared__ float sel[MOE_MAX_K];
    const int n = a.n_experts, t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE;
    float mx = -INFINITY;
    for (int i = t; i < n; i += WG) mx = fmaxf(mx, a.logits[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < WG / WAVE; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float sum = 0.f;
    for (int i = t; i < n; i += WG) {
        const float e = expf(a.logits[i] - M);
        p[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < WG / WAVE; w++) tot += red[w];
    for (int i = t; i < n; i += WG) p[i] = p[i] / tot;
    if (t < a.top_k) {  // defined ids and weights even if NaN logits leave a rank unfilled
        sel[t] = 0.f;
        a.ids[t] = 0;
    }
    __syncthreads();
    for (int i = t; i < n; i += WG) {
        const float pi = p[i];
        int rank = 0;
        for (int j = 0; j < n; j++) rank += better(p[j], j, pi, i) ? 1 : 0;
        if (rank < a.top_k) {
            a.ids[rank] = i;
            sel[rank] = pi;
        }
    }
    __syncthreads();
    if (t < a.top_k) {
        float s = 0.f;
        for (int k = 0; k < a.top_k; k++) s += sel[k];  // in rank order, as the sequential selection
        a.w[t] = a.norm_topk ? sel[t] / s : sel[t];
    }
}

// x (n floats) into LDS in the swizzled layout of XView
__device__ __forceinline__ void moe_stage_x(const float *x, int n, float4 *x4) {
    for (int c = threadIdx.x; c < n / 4; c += WG) x4[xswz(c)] = ((const float4 *)x)[c];
}

// h[k][r] = silu(gate_e x)[r] * (up_e x)[r], e = ids[k]; grid (top_k,
// ceil(inter / 4)), one row per wave: the lanes take the (matrix, unit) pairs
// of the row's gate and up dot products, so all of the row's loads are in
// flight at once
__global__ __launch_bounds__(WG) void moe_gateup_kernel(MoeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ float4 smem[];
    const int k = blockIdx.x, e = min(max(a.ids[k], 0), a.n_experts - 1);  // ids come from the device
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    moe_stage_x(a.x, a.dim, smem);
    __syncthreads();
    const int r = (int)blockIdx.y * 4 + wave;
    if (r >= a.inter) return;
    const XView xv{smem, nullptr};
    const DMat g = sub_rows(a.gate, e * a.inter, a.inter), u = sub_rows(a.up, e * a.inter, a.inter);
    const int U = a.dim >> 6;
    float sg = 0.f, su = 0.f;
    for (int j = lane; j < 2 * U; j += WAVE) {
        if (j < U) sg += dot_unit(g, r, j, xv);
        else su += dot_unit(u, r, j - U, xv);
    }
    sg = wave_sum(sg);
    su = wave_sum(su);
    if (lane == 0) {
        const float sig = sg >= 0.f ? 1.0f / (1.0f + expf(-sg)) : expf(sg) / (1.0f + expf(sg));
        a.h[(size_t)k * a.inter + r] = sg * sig * su;
    }
}

// y[r] = sum_k w_k (down_{ids[k]} h_k)[r]; grid ceil(dim / 4), one row per
// wave, the lanes taking the (expert, unit) pairs so that all of the row's
// loads are in flight at once; the pair products go through LDS and are
// summed per expert, then weighted, in expert order
__global__ __launch_bounds__(WG) void moe_down_kernel(MoeArgs a) {
    extern __shared__ float4 smem[];
    __shared__ float part[WG / WAVE][MOE_MAX_K * 4];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int X4 = a.inter / 4;  // float4 slots per expert vector
    for (int k = 0; k < a.top_k; k++) moe_stage_x(a.h + (size_t)k * a.inter, a.inter, smem + (size_t)k * X4);
    __syncthreads();
    const int r = (int)blockIdx.x * 4 + wave;
    if (r >= a.dim) return;
    const int U = a.inter >> 6, P = a.top_k * U, NB = (MOE_MAX_K * 4 / U) * U;  // batches end on experts
    float y = 0.f;
    for (int p0 = 0; p0 < P; p0 += NB) {
        const int np = min(P - p0, NB);
        for (int j = lane; j < np; j += WAVE) {
            const int pr = p0 + j, k = pr / U, u = pr % U;
            const DMat d = sub_rows(a.down, min(max(a.ids[k], 0), a.n_experts - 1) * a.dim, a.dim);
            part[wave][j] = dot_unit(d, r, u, XView{smem + (size_t)k * X4, nullptr});
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            float s = 0.f;
            for (int j = 0; j < np; j++) {
                s += part[wave][j];
                if ((j + 1) % U == 0) {
                    y += a.w[(p0 + j) / U] * s;
                    s = 0.f;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) a.y[r] = y;
}

hipError_t launch_moe(const MoeArgs &a, const GemvArgs &router, const GemvArgs *gu, const GemvArgs *dn,
                      hipStream_t st) {
    if (a.n_experts > MOE_MAX_EXPERTS || a.top_k > MOE_MAX_K || a.top_k < 1 || a.top_k > a.n_experts ||
        a.dim % 64 || a.inter % 64 || a.inter > 64 * MOE_MAX_K * 4)
        return hipErrorInvalidValue;
    hipError_t r = launch_gemv(router, st);
    if (r != hipSuccess) return r;
    if (!gu || !gu->moe_logits) hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(WG), 0, st, a);
    if (gu) {
        r = launch_gemv_q_moe(*gu, MOE_ROWS, st);
        if (r != hipSuccess) return r;
    } else {
        hipLaunchKernelGGL(moe_gateup_kernel, dim3((unsigned)a.top_k, (unsigned)((a.inter + 3) / 4)), dim3(WG),
                           (size_t)a.dim * 4, st, a);
    }
    if (dn) {
        r = launch_gemv_q_moe(*dn, MOE_COLS, st);
        if (r != hipSuccess) return r;
    } else {
        hipLaunchKernelGGL(moe_down_kernel, dim3((unsigned)((a.dim + 3) / 4)), dim3(WG),
                           (size_t)a.top_k * a.inter * 4, st, a);
    }
    return hipGetLastError();
}

// --------------------------------------------- routed experts, prefill --
// The routed-expert FFN of a prefill chunk in f32, the arithmetic of the
// per-token path (router, softmax, top-k, renormalized weights, the chosen
// experts' SwiGLU and down projections; the reference has no MoE, so nothing
// here is staged in f16).  Pairs p = t kp + s (token t, its s-th chosen
// expert) are grouped by expert, and a multi-token GEMV reads the rows of
// each chosen expert once for all of its pairs.

constexpr int MT_CMAX = 8;  // pairs per pass of the multi-token GEMV

// the 64 decoded weights w of unit u dotted with x (LDS, XView's swizzle):
// they are four runs of 16 consecutive row elements (unit_elem)
__device__ __forceinline__ float dot_unit_x(const float *w, int type, int u, const float4 *x4) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int c0 = unit_elem(type, u, 16 * k) >> 2;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 x = x4[xswz(c0 + i)];
            const float *wk = w + 16 * k + 4 * i;
            a += wk[0] * x.x + wk[1] * x.y + wk[2] * x.z + wk[3] * x.w;
        }
    }
    return a;
}

// Work item (expert e, pair slice, row tile): rows [tile * tile_rows,
// +tile_rows) of expert e against pairs [slice * pair_slice, +pair_slice) of
// e's list, cmax pairs per pass with their x rows in LDS.  Lane groups of lpr lanes (the smallest power of two >= the row's
// units, at most 64) take one row each and split its units; each unit is
// decoded once (decode_unit, exact) for all the pass's pairs.
// y[p][r] = row r . x  or, for a SwiGLU pair of matrices,
// silu(gate_r . x) * (up_r . x) (infer/forward.odin:128-132).
__global__ __launch_bounds__(WG) void mt_gemv_kernel(MtGemvArgs a, int cmax) {
#pragma clang fp contract(off)
    extern __shared__ float4 smem[];
    const int it = blockIdx.x;
    int e = 0, tile, slice, n, base;
    if (a.dense_n > 0) {
        tile = it % a.tiles;
        slice = it / a.tiles;
        n = a.dense_n;
        base = 0;
    } else {
        if (it >= *a.nitems) return;
        e = a.items[2 * it];
        tile = a.items[2 * it + 1] & 0xFFFF;
        slice = a.items[2 * it + 1] >> 16;
        n = a.cnt[e];
        base = a.off[e];
    }
    base += slice * a.pair_slice;
    n = min(a.pair_slice, n - slice * a.pair_slice);
    const int r0 = tile * a.tile_rows, r1 = min(a.rows, r0 + a.tile_rows);
    if (r0 >= r1) return;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int U = a.K >> 6, K4 = a.K >> 2;
    int lpr = 1;
    while (lpr < U && lpr < WAVE) lpr <<= 1;
    const int gpw = WAVE / lpr, grp = lane / lpr, gl = lane % lpr;
    const DMat g = sub_rows(a.m, e * a.rows, a.rows);
    const DMat up = a.swiglu ? sub_rows(a.m2, e * a.rows, a.rows) : g;
    for (int c0 = 0; c0 < n; c0 += cmax) {
        const int nc = min(cmax, n - c0);
        __syncthreads();  // the previous pass's x reads are done
        for (int idx = threadIdx.x; idx < nc * K4; idx += WG) {
            const int j = idx / K4, c = idx % K4;
            const int p = a.dense_n > 0 ? base + c0 + j : a.list[base + c0 + j];
            smem[j * K4 + xswz(c)] = ((const float4 *)(a.x + (size_t)(p / a.xdiv) * a.K))[c];
        }
        __syncthreads();
        for (int r = r0 + wave * gpw + grp; r < r1; r += (WG / WAVE) * gpw) {
            float ag[MT_CMAX], au[MT_CMAX];
#pragma unroll
            for (int j = 0; j < MT_CMAX; j++) ag[j] = au[j] = 0.f;
            for (int u = gl; u < U; u += lpr) {
                float w[64];
                decode_unit(g, r, u, w);
#pragma unroll
                for (int j = 0; j < MT_CMAX; j++)
                    if (j < nc) ag[j] += dot_unit_x(w, g.type, u, smem + j * K4);
                if (a.swiglu) {
                    decode_unit(up, r, u, w);
#pragma unroll
                    for (int j = 0; j < MT_CMAX; j++)
                        if (j < nc) au[j] += dot_unit_x(w, up.type, u, smem + j * K4);
                }
            }
#pragma unroll
            for (int j = 0; j < MT_CMAX; j++) {
                if (j < nc) {
                    ag[j] = lane_group_sum(ag[j], lpr);
                    if (a.swiglu) au[j] = lane_group_sum(au[j], lpr);
                }
            }
            if (gl == 0) {
#pragma unroll
                for (int j = 0; j < MT_CMAX; j++) {
                    if (j < nc) {
                        const int p = a.dense_n > 0 ? base + c0 + j : a.list[base + c0 + j];
                        float v = ag[j];
                        if (a.swiglu) {
                            v *= 1.0f / (1.0f + expf(-v));
                            v *= au[j];
                        }
                        a.y[(size_t)p * a.rows + r] = v;
                    }
                }
            }
        }
    }
}

static int mt_lpr(int32_t K) {
    int lpr = 1;
    while (lpr < K / 64 && lpr < WAVE) lpr <<= 1;
    return lpr;
}
bool mt_gemv_supported(const DMat &m, int32_t K) {
    return K > 0 && K % 64 == 0 && K <= 16384 && m.cols == K &&
           (m.type == T_Q4_K || m.type == T_Q6_K || m.type == T_Q8_0 || m.type == T_F32 || m.type == T_F16 ||
            m.type == T_Q4_0 || m.type == T_Q4_1 || m.type == T_Q5_0 || m.type == T_Q5_1);
}
// eight passes of the workgroup's lane groups
int mt_gemv_tile_rows(int32_t K, int32_t rows) { return std::min<int32_t>(rows, 8 * (WG / WAVE) * (WAVE / mt_lpr(K))); }

hipError_t launch_mt_gemv(const MtGemvArgs &a, int max_items, hipStream_t st) {
    if (!mt_gemv_supported(a.m, a.K) || (a.swiglu && !mt_gemv_supported(a.m2, a.K)) || a.tile_rows <= 0 ||
        a.rows <= 0 || a.xdiv <= 0 || max_items <= 0 || a.pair_slice <= 0 ||
        (a.dense_n > 0 && (a.tiles != (a.rows + a.tile_rows - 1) / a.tile_rows ||
                           max_items != a.tiles * ((a.dense_n + a.pair_slice - 1) / a.pair_slice))))
        return hipErrorInvalidValue;
    const int cmax = std::max(1, std::min(MT_CMAX, 16384 / a.K));  // <= 64 KB of x in LDS
    hipLaunchKernelGGL(mt_gemv_kernel, dim3((unsigned)max_items), dim3(WG), (size_t)cmax * a.K * 4, st, a, cmax);
    return hipGetLastError();
}

// ---- the same on the matrix cores (f32 MFMA): Q4_K / Q6_K / Q8_0 experts
//
// v_mfma_f32_16x16x4_f32: D[16][16] += A[16][4] B[4][16]; lane l gives
// A[i][k] with i = l % 16, k = l / 16, and B[k][j] with j = l % 16, k = l / 16,
// and holds D[i][j] for j = l % 16, i = 4 (l / 16) + e (e < 4).  Lane l takes
// row i of its wave's 16 and pair j = i of the item's 16; for each 64-weight
// unit it decodes the quarter g = l / 16 (16 weights, exact), reads the same
// 16 K positions of its pair's x, and 16 products sum the unit over the four
// quarters.  f32 operands and accumulation: the arithmetic of mt_gemv_kernel
// up to the order of the sums.
constexpr int MM_PAIRS = 16, MM_ROWS = 16 * (WG / WAVE), MM_KC = 256;
static_assert(MM_PAIRS == MT_MFMA_PAIRS && MM_ROWS == MT_MFMA_ROWS, "item shape");

// Quarter g of unit u of `row`: the weights at row elements
// unit_elem(type, u, 16 g) + s, s < 16 (decode_unit's values).  load_quarter
// issues the loads (raw bytes), decode_quarter does the arithmetic, so the
// loads of later units can be in flight while earlier ones are used.
struct QRaw {
    u32x4 a, b;  // Q4_K: quants (plane g & 1), header; Q6_K: ql (plane g & 1), qh; Q8_0: quants (plane g)
    uint32_t x;  // Q6_K: d | scale << 16; Q8_0: d
};
__device__ __forceinline__ QRaw load_quarter(const DMat &m, int row, int u, int g) {
    const size_t ui = (size_t)row * (m.cols >> 6) + u;
    QRaw r;
    if (m.type == T_Q4_K) {
        r.a = *(const u32x4 *)(m.q + (g & 1) * m.plane + ui * 16);
        r.b = *(const u32x4 *)(m.s + ((size_t)row * (m.cols >> 8) + (u >> 2)) * 16);
        r.x = 0;
    } else if (m.type == T_Q6_K) {
        const size_t sbi = (size_t)row * (m.cols >> 8) + (u >> 2);
        r.a = *(const u32x4 *)(m.q + (g & 1) * m.plane + ui * 16);
        r.b = *(const u32x4 *)(m.q + 2 * m.plane + ui * 16);
        const uint8_t sc = m.s[sbi * 16 + 8 * ((u >> 1) & 1) + (u & 1) + 2 * g];
        r.x = (uint32_t)m.d[sbi] | ((uint32_t)sc << 16);
    } else {
        r.a = *(const u32x4 *)(m.q + g * m.plane + ui * 16);
        r.b = u32x4{0u, 0u, 0u, 0u};
        r.x = m.d[(size_t)row * (m.cols >> 5) + 2 * u + (g >> 1)];
    }
    return r;
}
__device__ __forceinline__ void decode_quarter(int type, const QRaw &r, int u, int g, float *w) {
#pragma clang fp contract(off)
    const uint32_t qw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    if (type == T_Q4_K) {  // ggml/quant.odin:178-209
        const float d = h2f(r.b.x & 0xFFFFu), dmin = h2f(r.b.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        q4k_scales(u & 3, r.b.y, r.b.z, r.b.w, sc0, m0, sc1, m1);
        const bool hi = g >= 2;
        const float dd = d * (float)(hi ? sc1 : sc0), mm = dmin * (float)(hi ? m1 : m0);
#pragma unroll
        for (int l = 0; l < 16; l++) {
            const uint32_t b = (qw[l >> 2] >> ((l & 3) * 8)) & 0xFFu;
            w[l] = dd * (float)(hi ? b >> 4 : b & 0xFu) - mm;
        }
    } else if (type == T_Q6_K) {  // ggml/quant.odin:212-247
        const float dsc = h2f(r.x & 0xFFFFu) * (float)(int8_t)(r.x >> 16);
        const uint32_t hw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t ql = (qw[i >> 2] >> ((i & 3) * 8)) & 0xFFu, qh = (hw[i >> 2] >> ((i & 3) * 8)) & 0xFFu;
            const int q = (int)((g < 2 ? (ql & 0xFu) : (ql >> 4)) | (((qh >> (2 * g)) & 3u) << 4)) - 32;
            w[i] = dsc * (float)q;
        }
    } else {  // Q8_0, ggml/quant.odin:87-96
        const float d = h2f(r.x & 0xFFFFu);
#pragma unroll
        for (int j = 0; j < 16; j++) w[j] = d * (float)(int8_t)((qw[j >> 2] >> ((j & 3) * 8)) & 0xFFu);
    }
}

typedef float mm_f32x4 __attribute__((ext_vector_type(4)));

// Work item (expert e, slice of 16 pairs, tile of 64 rows); the x rows of the
// slice's pairs staged in LDS, whole when they fit (few pairs), else KC K
// positions (KC / 256 super-blocks) at a time; rows padded by 4 floats; lanes
// of pairs past the slice's count give B = 0.  Each lane keeps the raw loads of the next super-block's 4 units in
// flight while it decodes and multiplies the current one's.
template <int KC>
__global__ __launch_bounds__(WG) void mt_mfma_kernel(MtGemvArgs a) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float xs[MM_PAIRS][KC + 4];
    const int it = blockIdx.x;
    if (it >= *a.nitems) return;
    const int e = a.items[2 * it], tile = a.items[2 * it + 1] & 0xFFFF, slice = a.items[2 * it + 1] >> 16;
    const int base = a.off[e] + slice * MM_PAIRS, n = min(MM_PAIRS, a.cnt[e] - slice * MM_PAIRS);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, i16 = lane & 15, g = lane >> 4;
    const int row0 = tile * MM_ROWS + 16 * wave;
    const bool active = row0 < a.rows;  // rows % 16 == 0
    const int row = min(row0 + i16, a.rows - 1);
    const DMat gm = sub_rows(a.m, e * a.rows, a.rows);
    const DMat um = a.swiglu ? sub_rows(a.m2, e * a.rows, a.rows) : gm;
    const int nsb = a.K / MM_KC;  // super-blocks
    const bool whole = n * (a.K + 4) <= MM_PAIRS * (KC + 4);  // every x row in LDS at once
    const int xstride = whole ? a.K + 4 : KC + 4;
    float *xsf = &xs[0][0];
    mm_f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    QRaw rg[4], ru[4];
    if (active) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            rg[s] = load_quarter(gm, row, s, g);
            if (a.swiglu) ru[s] = load_quarter(um, row, s, g);
        }
    }
    for (int c = 0; c < nsb; c++) {
        const int k0 = whole ? 0 : (c / (KC / MM_KC)) * KC, kw = whole ? a.K : KC;
        if (whole ? c == 0 : c % (KC / MM_KC) == 0) {
            __syncthreads();  // the previous chunk's reads are done
            for (int idx = threadIdx.x; idx < n * kw / 4; idx += WG) {
                const int j = idx / (kw / 4), q = idx % (kw / 4);
                *(float4 *)(xsf + j * xstride + 4 * q) =
                    ((const float4 *)(a.x + (size_t)(a.list[base + j] / a.xdiv) * a.K + k0))[q];
            }
            __syncthreads();
        }
        if (!active) continue;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int u = 4 * c + s;
            float w[16], wu[16], xv[16];
            decode_quarter(gm.type, rg[s], u, g, w);
            if (a.swiglu) decode_quarter(um.type, ru[s], u, g, wu);
            if (c + 1 < nsb) {  // the next super-block's unit s
                rg[s] = load_quarter(gm, row, u + 4, g);
                if (a.swiglu) ru[s] = load_quarter(um, row, u + 4, g);
            }
            const float4 *xr = (const float4 *)(xsf + i16 * xstride + unit_elem(gm.type, u, 16 * g) - k0);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
                if (i16 < n) t = xr[q];  // rows past n are not staged
                xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
            }
#pragma unroll
            for (int s2 = 0; s2 < 16; s2++) accg = __builtin_amdgcn_mfma_f32_16x16x4f32(w[s2], xv[s2], accg, 0, 0, 0);
            if (a.swiglu) {
#pragma unroll
                for (int s2 = 0; s2 < 16; s2++)
                    accu = __builtin_amdgcn_mfma_f32_16x16x4f32(wu[s2], xv[s2], accu, 0, 0, 0);
            }
        }
    }
    if (!active || i16 >= n) return;
    const int p = a.list[base + i16];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float v = accg[r];
        if (a.swiglu) {
            v *= 1.0f / (1.0f + expf(-v));
            v *= accu[r];
        }
        a.y[(size_t)p * a.rows + row0 + 4 * g + r] = v;
    }
}

// ---- Q4_K experts on f16 MFMA with the weights exact --------------------
//
// A Q4_K weight is d1 q - m1 with q in 0..15 and (d1, m1) per 32 weights
// (one sub-block) and row, so a sub-block's dot product with x is
//   d1 sum(q x) - m1 sum(x),
// and sum(q x) runs on v_mfma_f32_16x16x32_f16: q is an exact half, x is
// split into hi = f16(x) and lo = f16(x - hi) (x to ~2^-22), two products per
// sub-block with f32 accumulation; sum(x) is the f32 sum of x.  The weights
// are never rounded (the staged path rounds d1 q - m1 to f16), so this is the
// f32 arithmetic of mt_gemv_kernel up to the order of the sums and the x split.
// Operand layout (per lane l, 8 halves): A[i][k], i = l % 16, k = 8 (l / 16) + e;
// B[k][j], j = l % 16; D[i][j]: j = l % 16, i = 4 (l / 16) + e.  Lane (i, g =
// l / 16) loads bytes 8g .. 8g+7 of row i's 32 quant bytes of a unit (low
// nibbles: sub-block 0's K positions 8g + e, high nibbles sub-block 1's), and
// the x halves of pair i at the same K positions.
typedef _Float16 mq_h8 __attribute__((ext_vector_type(8)));

// the 8 nibbles (low when hi == false) of 8 bytes as exact halves
__device__ __forceinline__ mq_h8 nibbles_h8(uint32_t w0, uint32_t w1, bool hi) {
    const uint32_t n0 = (hi ? w0 >> 4 : w0) & 0x0F0F0F0Fu, n1 = (hi ? w1 >> 4 : w1) & 0x0F0F0F0Fu;
    // bytes [n, 0x64] form the half 1024 + n; subtract 1024 (exact)
    u32x4 v;
    v.x = __builtin_amdgcn_perm(0x64646464u, n0, 0x07010600u);
    v.y = __builtin_amdgcn_perm(0x64646464u, n0, 0x07030602u);
    v.z = __builtin_amdgcn_perm(0x64646464u, n1, 0x07010600u);
    v.w = __builtin_amdgcn_perm(0x64646464u, n1, 0x07030602u);
    mq_h8 h = __builtin_bit_cast(mq_h8, v);
    const mq_h8 bias = {1024.f16, 1024.f16, 1024.f16, 1024.f16, 1024.f16, 1024.f16, 1024.f16, 1024.f16};
    return h - bias;
}

// Per KC-wide chunk of K: the chunk's weight loads (8 bytes per unit and
// lane, the row headers) are issued first, then the x rows of the item's
// pairs are staged (hi / lo halves, f32 sums per 32) while they travel; the
// header lanes write (d1, m1) of every sub-block of their row to LDS once per
// chunk.
template <int KC>
__global__ __launch_bounds__(WG) void mt_q4mfma_kernel(MtGemvArgs a) {
#pragma clang fp contract(off)
    constexpr int XP = KC + 8, NU = KC / 64, NS = KC / 256, NB = KC / 32;  // LDS row stride; units, super-blocks, sub-blocks
    __shared__ __attribute__((aligned(16))) uint16_t xh[MM_PAIRS][XP];
    __shared__ __attribute__((aligned(16))) uint16_t xl[MM_PAIRS][XP];
    __shared__ float sx[MM_PAIRS][NB];
    __shared__ __attribute__((aligned(16))) float scl[2][WG / WAVE][16][2 * NB];  // (d, m) per sub-block of a row
    const int it = blockIdx.x;
    if (it >= *a.nitems) return;
    const int e = a.items[2 * it], tile = a.items[2 * it + 1] & 0xFFFF, slice = a.items[2 * it + 1] >> 16;
    const int base = a.off[e] + slice * MM_PAIRS, n = min(MM_PAIRS, a.cnt[e] - slice * MM_PAIRS);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, i16 = lane & 15, g = lane >> 4;
    const int row0 = tile * MM_ROWS + 16 * wave;
    const bool active = row0 < a.rows;  // rows % 16 == 0
    const int row = min(row0 + i16, a.rows - 1);
    const DMat gm = sub_rows(a.m, e * a.rows, a.rows);
    const DMat um = a.swiglu ? sub_rows(a.m2, e * a.rows, a.rows) : gm;
    // a runtime count: with a constant 2 the compiler keeps twice the
    // registers (300 VGPRs, one wave per SIMD)
    const int nmat = a.swiglu ? 2 : 1;
    const int U = a.K >> 6;
    mm_f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < a.K; c0 += KC) {
        uint32_t qw[2][NU][2];
        u32x4 hd[2][NS];
        if (active) {
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                if (mi >= nmat) break;
                const DMat &m = mi ? um : gm;
#pragma unroll
                for (int k = 0; k < NU; k++) {
                    const size_t ui = (size_t)row * U + c0 / 64 + k;
                    const u32x2 q = *(const u32x2 *)(m.q + (g >> 1) * m.plane + ui * 16 + 8 * (g & 1));
                    qw[mi][k][0] = q.x;
                    qw[mi][k][1] = q.y;
                }
                if (g == 0) {
#pragma unroll
                    for (int k = 0; k < NS; k++)
                        hd[mi][k] = *(const u32x4 *)(m.s + ((size_t)row * (m.cols >> 8) + c0 / 256 + k) * 16);
                }
            }
        }
        __syncthreads();  // the previous chunk's LDS reads are done
        // x rows of the item's pairs, 8 elements per step: hi / lo halves and
        // the f32 sum of each 32 (four consecutive threads, DPP)
        for (int idx0 = 0; idx0 < n * (KC / 8); idx0 += WG) {
            const int idx = idx0 + threadIdx.x, j = idx / (KC / 8), c8 = idx % (KC / 8);
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (j < n) {
                const float4 *xr = (const float4 *)(a.x + (size_t)(a.list[base + j] / a.xdiv) * a.K + c0 + 8 * c8);
                const float4 p0 = xr[0], p1 = xr[1];
                v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
                v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
            }
            uint32_t hw[4], lw[4];
            float s8 = 0.f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint16_t h0 = f2h(v[2 * q]), h1 = f2h(v[2 * q + 1]);
                const uint16_t l0 = f2h(v[2 * q] - h2f(h0)), l1 = f2h(v[2 * q + 1] - h2f(h1));
                hw[q] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                lw[q] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                s8 += v[2 * q] + v[2 * q + 1];
            }
            s8 = dpp_sum4(s8);  // the 32 elements of one sub-block (c8 = 4 b .. 4 b + 3)
            if (j < n) {
                *(u32x4 *)&xh[j][8 * c8] = u32x4{hw[0], hw[1], hw[2], hw[3]};
                *(u32x4 *)&xl[j][8 * c8] = u32x4{lw[0], lw[1], lw[2], lw[3]};
                if ((c8 & 3) == 0) sx[j][c8 / 4] = s8;
            }
        }
        if (active && g == 0) {  // (d1, m1) of every sub-block of this row in the chunk
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                if (mi >= nmat) break;
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    const float d = h2f(hd[mi][k].x & 0xFFFFu), dmin = h2f(hd[mi][k].x >> 16);
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        uint32_t sc0, m0, sc1, m1;
                        q4k_scales(p, hd[mi][k].y, hd[mi][k].z, hd[mi][k].w, sc0, m0, sc1, m1);
                        *(float4 *)&scl[mi][wave][i16][2 * (8 * k + 2 * p)] =
                            make_float4(d * (float)sc0, dmin * (float)m0, d * (float)sc1, dmin * (float)m1);
                    }
                }
            }
        }
        __syncthreads();
        if (!active) continue;
#pragma unroll
        for (int k = 0; k < NU; k++) {
#pragma unroll
            for (int sb = 0; sb < 2; sb++) {
                const int b = 2 * k + sb, kx = 32 * b + 8 * g;  // sub-block in the chunk; this lane's K positions
                u32x4 bh = {0u, 0u, 0u, 0u}, bl = {0u, 0u, 0u, 0u};
                float sxv = 0.f;
                if (i16 < n) {
                    bh = *(const u32x4 *)&xh[i16][kx];
                    bl = *(const u32x4 *)&xl[i16][kx];
                    sxv = sx[i16][b];
                }
                const mq_h8 Bh = __builtin_bit_cast(mq_h8, bh), Bl = __builtin_bit_cast(mq_h8, bl);
#pragma unroll
                for (int mi = 0; mi < 2; mi++) {
                    if (mi >= nmat) break;
                    const mq_h8 A = nibbles_h8(qw[mi][k][0], qw[mi][k][1], sb == 1);
                    mm_f32x4 t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bh, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bl, t, 0, 0, 0);
                    mm_f32x4 &acc = mi ? accu : accg;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float2 dm = *(const float2 *)&scl[mi][wave][4 * g + r][2 * b];
                        acc[r] += dm.x * t[r] - dm.y * sxv;
                    }
                }
            }
        }
    }
    if (!active || i16 >= n) return;
    const int p = a.list[base + i16];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float v = accg[r];
        if (a.swiglu) {
            v *= 1.0f / (1.0f + expf(-v));
            v *= accu[r];
        }
        a.y[(size_t)p * a.rows + row0 + 4 * g + r] = v;
    }
}

// mt_q4mfma_kernel for items of at most MF_PAIRS pairs (a short chunk
// spreads its pairs over many experts: ~1.4 per expert at 64 tokens of top 10
// of 512).  An item is (expert, pair slice) and one matrix: the workgroup
// streams ALL row tiles of that matrix for its pairs (the item's descriptor,
// pair lists and x rows are read once, then the weights stream without a
// break: a step is one 256-wide chunk of K of one 64-row tile, and the next
// step's weights are in flight while the current one is computed, across tile
// boundaries).  The x rows of the item's pairs are staged in LDS once for the
// whole K (hi / lo halves and the f32 sums per 32); with x2 set they are
// silu(x) * x2 (the SwiGLU of separately computed gate and up rows, the
// reference's order).  A SwiGLU pair runs as two halves of the grid (blocks
// past mat_items take m2 into y2), so one matrix's registers fit three waves
// per SIMD.  The sub-block scales of a step go through the wave's own LDS
// rows (written by the header lanes, read after a wave barrier: a wave's DS
// operations complete in order).
constexpr int MF_PAIRS = MT_MFMA_FEW;
template <int KC>
__global__ __launch_bounds__(WG) void mt_q4mfma_few_kernel(MtGemvArgs a) {
#pragma clang fp contract(off)
    constexpr int NU = KC / 64, NS = KC / 256, NB = KC / 32;
    extern __shared__ __attribute__((aligned(16))) uint16_t mf_smem[];
    __shared__ __attribute__((aligned(16))) float scl[WG / WAVE][16][2 * NB];  // (d, m) per sub-block of a row
    const bool second = a.mat_items > 0 && (int)blockIdx.x >= a.mat_items;
    const int it = second ? (int)blockIdx.x - a.mat_items : (int)blockIdx.x;
    if (it >= *a.nitems) return;
    const int XP = a.K + 8;
    uint16_t *xh = mf_smem, *xl = mf_smem + MF_PAIRS * XP;
    float *sx = (float *)(mf_smem + 2 * MF_PAIRS * XP);  // [MF_PAIRS][K / 32]
    const int e = a.items[2 * it], slice = a.items[2 * it + 1] >> 16;
    const int base = a.off[e] + slice * MF_PAIRS, n = min(MF_PAIRS, a.cnt[e] - slice * MF_PAIRS);
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, i16 = lane & 15, g = lane >> 4;
    const DMat m = sub_rows(second ? a.m2 : a.m, e * a.rows, a.rows);
    float *y = second ? a.y2 : a.y;
    const int U = a.K >> 6, nch = a.K / KC, K32 = a.K / 32;
    const int ntile = a.rows / MM_ROWS, nstep = ntile * nch;  // rows % 64 == 0
    constexpr int NSTG = 4;  // ring stages: three steps in flight while one is computed
    uint32_t qw[NSTG][NU][2];  // [stage][unit][word]
    u32x4 hd[NSTG][NS];
    // the same loads in every call (a step past the end re-reads the last one),
    // so that the compiler waits for exactly the stage it consumes
    auto issue = [&](int st, int stg) {
        const int ss = min(st, nstep - 1), c = ss % nch, r = (ss / nch) * MM_ROWS + 16 * wave + i16;
#pragma unroll
        for (int k = 0; k < NU; k++) {
            const size_t ui = (size_t)r * U + c * (KC / 64) + k;
            const u32x2 q = *(const u32x2 *)(m.q + (g >> 1) * m.plane + ui * 16 + 8 * (g & 1));
            qw[stg][k][0] = q.x;
            qw[stg][k][1] = q.y;
        }
#pragma unroll
        for (int k = 0; k < NS; k++) hd[stg][k] = *(const u32x4 *)(m.s + ((size_t)r * (m.cols >> 8) + c * NS + k) * 16);
    };
#pragma unroll
    for (int i = 0; i < NSTG - 1; i++) issue(i, i);
    // x rows of the item's pairs for the whole K, 8 elements per step
    for (int idx = threadIdx.x; idx < n * (a.K / 8); idx += WG) {
        const int j = idx / (a.K / 8), c8 = idx % (a.K / 8);
        const size_t xo = (size_t)(a.list[base + j] / a.xdiv) * a.K + 8 * c8;
        const float4 *xr = (const float4 *)(a.x + xo);
        const float4 p0 = xr[0], p1 = xr[1];
        float v[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        if (a.x2) {  // SwiGLU: v = silu(gate) * up (infer/forward.odin:128-132)
            const float4 *ur = (const float4 *)(a.x2 + xo);
            const float4 u0 = ur[0], u1 = ur[1];
            const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int q = 0; q < 8; q++) {
                v[q] *= 1.0f / (1.0f + expf(-v[q]));
                v[q] *= u[q];
            }
        }
        uint32_t hw[4], lw[4];
        float s8 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint16_t h0 = f2h(v[2 * q]), h1 = f2h(v[2 * q + 1]);
            const uint16_t l0 = f2h(v[2 * q] - h2f(h0)), l1 = f2h(v[2 * q + 1] - h2f(h1));
            hw[q] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            lw[q] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            s8 += v[2 * q] + v[2 * q + 1];
        }
        // the 32 elements of one sub-block: four consecutive c8 of one pair
        // (n * K / 8 is a multiple of 4, so whole groups of 4 threads run here)
        s8 = dpp_sum4(s8);
        *(u32x4 *)&xh[j * XP + 8 * c8] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        *(u32x4 *)&xl[j * XP + 8 * c8] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        if ((c8 & 3) == 0) sx[j * K32 + c8 / 4] = s8;
    }
    __syncthreads();
    const int p = i16 < n ? a.list[base + i16] : 0;
    mm_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int st, int stg) {
        const int c = st % nch;
        if (g == 0) {  // (d1, m1) of every sub-block of this row in the chunk
#pragma unroll
            for (int k = 0; k < NS; k++) {
                const float d = h2f(hd[stg][k].x & 0xFFFFu), dmin = h2f(hd[stg][k].x >> 16);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    uint32_t sc0, m0, sc1, m1;
                    q4k_scales(q, hd[stg][k].y, hd[stg][k].z, hd[stg][k].w, sc0, m0, sc1, m1);
                    *(float4 *)&scl[wave][i16][2 * (8 * k + 2 * q)] =
                        make_float4(d * (float)sc0, dmin * (float)m0, d * (float)sc1, dmin * (float)m1);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < NU; k++) {
#pragma unroll
            for (int sb = 0; sb < 2; sb++) {
                const int b = 2 * k + sb, kx = c * KC + 32 * b + 8 * g;  // this lane's K positions
                u32x4 bh = {0u, 0u, 0u, 0u}, bl = {0u, 0u, 0u, 0u};
                float sxv = 0.f;
                if (i16 < n) {
                    bh = *(const u32x4 *)&xh[i16 * XP + kx];
                    bl = *(const u32x4 *)&xl[i16 * XP + kx];
                    sxv = sx[i16 * K32 + c * NB + b];
                }
                const mq_h8 A = nibbles_h8(qw[stg][k][0], qw[stg][k][1], sb == 1);
                mm_f32x4 t = {0.f, 0.f, 0.f, 0.f};
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(mq_h8, bh), t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(mq_h8, bl), t, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float2 dm = *(const float2 *)&scl[wave][4 * g + r][2 * b];
                    acc[r] += dm.x * t[r] - dm.y * sxv;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the scale reads are done before the next step writes them
        if (c == nch - 1) {  // the tile's rows are complete
            if (i16 < n) {
                const int row0 = (st / nch) * MM_ROWS + 16 * wave + 4 * g;
#pragma unroll
                for (int r = 0; r < 4; r++) y[(size_t)p * a.rows + row0 + r] = acc[r];
            }
            acc = mm_f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // NSTG steps per pass, so each stage index is static; every pass issues
    // the same loads (clamped to the last step), only the computation stops
    // at the end
    for (int st = 0; st < nstep; st += NSTG) {
#pragma unroll
        for (int j = 0; j < NSTG; j++) {
            issue(st + j + NSTG - 1, (j + NSTG - 1) % NSTG);
            if (st + j < nstep) compute(st + j, j);
        }
    }
}

bool mt_mfma_supported(const DMat &m, int32_t K, int32_t rows) {
    return (m.type == T_Q4_K || m.type == T_Q6_K || m.type == T_Q8_0) && m.cols == K && K % MM_KC == 0 &&
           rows % 16 == 0;
}

hipError_t launch_mt_mfma(const MtGemvArgs &a, int max_items, hipStream_t st, bool f32_only) {
    if (!mt_mfma_supported(a.m, a.K, a.rows) || (a.swiglu && (!mt_mfma_supported(a.m2, a.K, a.rows) ||
                                                              a.m2.type != a.m.type)) ||
        a.tile_rows != MM_ROWS || (a.pair_slice != MM_PAIRS && a.pair_slice != MF_PAIRS) || a.xdiv <= 0 ||
        max_items <= 0 || a.dense_n > 0)
        return hipErrorInvalidValue;
    if (a.pair_slice == MF_PAIRS) {  // few pairs per item: Q4_K, x staged whole, every row tile per item
        const size_t lds = (size_t)MF_PAIRS * (a.K + 8) * 4 + (size_t)MF_PAIRS * (a.K / 32) * 4;
        if (a.m.type != T_Q4_K || f32_only || lds > 96 * 1024 || a.rows % MM_ROWS || a.tiles != 1 ||
            (a.swiglu && !a.y2))
            return hipErrorInvalidValue;
        MtGemvArgs b = a;
        b.mat_items = a.swiglu ? max_items : 0;  // gate into y, up into y2 (the SwiGLU is the consumer's)
        const dim3 grid((unsigned)(a.swiglu ? 2 * max_items : max_items));
        hipLaunchKernelGGL(mt_q4mfma_few_kernel<MM_KC>, grid, dim3(WG), lds, st, b);
        return hipGetLastError();
    }
    if (a.m.type == T_Q4_K && !f32_only) {
        const dim3 grid((unsigned)max_items);
        hipLaunchKernelGGL(mt_q4mfma_kernel<MM_KC>, grid, dim3(WG), 0, st, a);  // 512: 256 VGPRs, slower
    } else if (a.K % 512 == 0) {
        hipLaunchKernelGGL(mt_mfma_kernel<512>, dim3((unsigned)max_items), dim3(WG), 0, st, a);
    } else {
        hipLaunchKernelGGL(mt_mfma_kernel<MM_KC>, dim3((unsigned)max_items), dim3(WG), 0, st, a);
    }
    return hipGetLastError();
}

// Router softmax and top-k of every token of the chunk (grid T): the
// selection of moe_topk_kernel (rank = the number of experts with a larger p,
// or an equal p and a lower id), then the merged shared expert (id
// n_experts, weight sigmoid of its gate logit, the dot product of its gate
// row with the token's normed x, computed here) in slot top_k.
__global__ __launch_bounds__(WG) void pf_moe_topk_kernel(PfMoeArgs a) {
#pragma clang fp contract(off)
    __shared__ float p[MOE_MAX_EXPERTS];
    __shared__ float red[WG / WAVE];
    __shared__ float sel[MOE_MAX_K];
    __shared__ int sid[MOE_MAX_K];
    __shared__ float sgl;
    const int n = a.n_experts, t = threadIdx.x, lane = t & (WAVE - 1), wave = t / WAVE, tok = blockIdx.x;
    if (a.kp > a.top_k) {  // the shared expert's gate logit: one unit per thread, then a block sum
        const int U = a.sh_inp.cols >> 6;
        float acc = 0.f;
        for (int u = t; u < U; u += WG) {
            float w[64];
            decode_unit(a.sh_inp, 0, u, w);
            const float *x = a.xn + (size_t)tok * a.sh_inp.cols;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 *xr = (const float4 *)(x + unit_elem(a.sh_inp.type, u, 16 * k));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 xv = xr[i];
                    const float *wk = w + 16 * k + 4 * i;
                    acc += wk[0] * xv.x + wk[1] * xv.y + wk[2] * xv.z + wk[3] * xv.w;
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) red[wave] = acc;
        __syncthreads();
        if (t == 0) sgl = red[0] + red[1] + red[2] + red[3];
        __syncthreads();
    }
    const float *lg = a.logits + (size_t)tok * n;
    float mx = -INFINITY;
    for (int i = t; i < n; i += WG) mx = fmaxf(mx, lg[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < WG / WAVE; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float sum = 0.f;
    for (int i = t; i < n; i += WG) {
        const float e = expf(lg[i] - M);
        p[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < WG / WAVE; w++) tot += red[w];
    for (int i = t; i < n; i += WG) p[i] = p[i] / tot;
    if (t < a.top_k) {  // defined ids and weights even if NaN logits leave a rank unfilled
        sel[t] = 0.f;
        sid[t] = 0;
    }
    __syncthreads();
    // The k best in the order (p descending, id ascending), i.e. k rounds of
    // first-maximum selection.  Keys: bit 41 set for a defined p (>= +0, so its
    // bits order as unsigned integers), p's bits at 40..10, 1023 - id at 9..0.
    // Each wave keeps its k best keys as candidates (an expert among the k best
    // has fewer than k better experts in its wave), then a candidate's rank
    // among the candidates is its rank among all experts when it is below k
    // (every expert better than one of the k best is itself a candidate).
    __shared__ unsigned long long cand[(WG / WAVE) * MOE_MAX_K];
    {
        constexpr int NV = MOE_MAX_EXPERTS / WG;
        const int k = a.top_k;
        unsigned long long v[NV];
        int nvalid = 0;
#pragma unroll
        for (int q = 0; q < NV; q++) {
            const int i = t + q * WG;
            const float pi = i < n ? p[i] : __builtin_nanf("");
            v[q] = pi >= 0.f ? (1ull << 41) | ((unsigned long long)__float_as_uint(pi) << 10) | (unsigned)(1023 - i)
                             : 0ull;
            nvalid += __popcll(__ballot(v[q] != 0ull));
        }
        const unsigned long long T = nvalid > k ? wave_kth_key(v, k) : 1ull;
        int slot = 0;
#pragma unroll
        for (int q = 0; q < NV; q++) {
            const unsigned long long m = __ballot(v[q] >= T);
            const int at = slot + __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
            if (v[q] >= T && at < k) cand[wave * k + at] = v[q];
            slot += __popcll(m);
        }
        for (int q = slot + lane; q < k; q += WAVE) cand[wave * k + q] = 0ull;
        __syncthreads();
        if (t < (WG / WAVE) * k) {
            const unsigned long long c = cand[t];
            if (c != 0ull) {
                int rank = 0;
                for (int j = 0; j < (WG / WAVE) * k; j++) rank += cand[j] > c ? 1 : 0;
                if (rank < k) {
                    const int id = 1023 - (int)(c & 1023ull);
                    sid[rank] = id;
                    sel[rank] = p[id];
                }
            }
        }
    }
    __syncthreads();
    if (t < a.kp) {
        int id;
        float w;
        if (t < a.top_k) {
            float s = 0.f;
            for (int k = 0; k < a.top_k; k++) s += sel[k];  // in rank order, as the sequential selection
            id = sid[t];
            w = a.norm_topk ? sel[t] / s : sel[t];
        } else {  // the shared expert
            id = n;
            w = 1.0f / (1.0f + expf(-sgl));
        }
        a.ids[(size_t)tok * a.kp + t] = id;
        a.w[(size_t)tok * a.kp + t] = w;
    }
}

// exclusive prefix sum of v over threads (one value per thread of the
// 1024-thread workgroup); *total receives the sum
__device__ __forceinline__ int block_excl_scan(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
    int x = v;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const int y = __shfl_up(x, o, WAVE);
        if (lane >= o) x += y;
    }
    __syncthreads();  // wsum reusable
    if (lane == WAVE - 1) wsum[wave] = x;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < nw; w++) {
        const int s = wsum[w];
        if (w < wave) before += s;
        all += s;
    }
    *total = all;
    return before + x - v;
}

// Pairs grouped by expert (one workgroup of 1024 threads, one expert per
// thread): counts, offsets, the pair lists (any order within an expert: each
// pair's result is its own), and the work items (expert; pair slice << 16 |
// row tile) of the gate/up and down multi-token GEMVs: tiles_gu / tiles_dn
// row tiles per slice of pair_slice pairs of each chosen expert.
__global__ __launch_bounds__(1024) void pf_moe_group_kernel(PfMoeArgs a) {
    __shared__ int cnt[1024], fill[1024], wsum[16];
    const int ne = a.n_experts + (a.kp > a.top_k ? 1 : 0), P = a.T * a.kp, e = threadIdx.x;
    if (e < ne) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) atomicAdd(&cnt[min(max(a.ids[p], 0), ne - 1)], 1);
    __syncthreads();
    const int c = e < ne ? cnt[e] : 0, ns = (c + a.pair_slice - 1) / a.pair_slice;
    int tp, tg, td;
    const int off = block_excl_scan(c, wsum, &tp);
    const int og = block_excl_scan(ns * a.tiles_gu, wsum, &tg);
    const int od = block_excl_scan(ns * a.tiles_dn, wsum, &td);
    if (e < ne) {
        a.off[e] = off;
        a.cnt[e] = c;
        for (int i = 0; i < ns * a.tiles_gu; i++) {
            a.items_gu[2 * (og + i)] = e;
            a.items_gu[2 * (og + i) + 1] = ((i / a.tiles_gu) << 16) | (i % a.tiles_gu);
        }
        for (int i = 0; i < ns * a.tiles_dn; i++) {
            a.items_dn[2 * (od + i)] = e;
            a.items_dn[2 * (od + i) + 1] = ((i / a.tiles_dn) << 16) | (i % a.tiles_dn);
        }
        fill[e] = off;  // the next free slot of e
    }
    if (threadIdx.x == 0) {
        a.nitems[0] = tg;
        a.nitems[1] = td;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int x = min(max(a.ids[p], 0), ne - 1);
        a.list[atomicAdd(&fill[x], 1)] = p;
    }
}

// out[t][r] = sum over the token's slots s (rank order, the shared expert
// last) of w[t][s] yd[t kp + s][r]
__global__ __launch_bounds__(WG) void pf_moe_combine_kernel(PfMoeArgs a) {
#pragma clang fp contract(off)
    const int t = blockIdx.y, r = (int)blockIdx.x * WG + threadIdx.x;
    if (r >= a.dim) return;
    float acc = 0.f;
    for (int s0 = 0; s0 < a.kp; s0 += 8) {  // 8 slots' rows requested together, summed in slot order
        float y[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (s0 + k < a.kp) y[k] = a.yd[((size_t)t * a.kp + s0 + k) * a.dim + r];
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (s0 + k < a.kp) acc += a.w[(size_t)t * a.kp + s0 + k] * y[k];
    }
    a.out[(size_t)t * a.dim + r] = acc;
}

hipError_t launch_pf_moe_route(const PfMoeArgs &a, hipStream_t st) {
    const int ne = a.n_experts + (a.kp > a.top_k ? 1 : 0);
    if (a.T <= 0 || a.n_experts <= 0 || ne > 1024 || a.top_k < 1 || a.top_k > MOE_MAX_K || a.top_k > a.n_experts ||
        a.kp < a.top_k || a.kp > a.top_k + 1 || (a.kp > a.top_k && (!a.xn || a.sh_inp.rows < 1 ||
                                                                  a.sh_inp.cols % 64 || a.sh_inp.cols > 16384)) ||
        a.tiles_gu > 0xFFFF ||
        a.tiles_dn > 0xFFFF || a.pair_slice <= 0 || (int64_t)a.T * a.kp / a.pair_slice >= 0x7FFF)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_moe_topk_kernel, dim3((unsigned)a.T), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(pf_moe_group_kernel, dim3(1), dim3(1024), 0, st, a);
    return hipGetLastError();
}

// The router as one "expert" whose pairs are the chunk's tokens in order
// (list[t] = t), in slices of MT_MFMA_FEW tokens and `tiles` row tiles: the
// work items of mt_q4i8_kernel (off, cnt and the item count in the same
// buffer's tail).  One workgroup.
__global__ __launch_bounds__(WG) void pf_router_items_kernel(int T, int tiles, int32_t *list, int32_t *items,
                                                              int32_t *hdr) {
    const int ns = (T + MT_MFMA_FEW - 1) / MT_MFMA_FEW;
    for (int t = threadIdx.x; t < T; t += WG) list[t] = t;
    for (int i = threadIdx.x; i < ns * tiles; i += WG) {
        items[2 * i] = 0;
        items[2 * i + 1] = ((i / tiles) << 16) | (i % tiles);
    }
    if (threadIdx.x == 0) {
        hdr[0] = 0;           // off
        hdr[1] = T;           // cnt
        hdr[2] = ns * tiles;  // items
    }
}

hipError_t launch_pf_router_items(int T, int tiles, int32_t *list, int32_t *items, int32_t *hdr, hipStream_t st) {
    if (T <= 0 || tiles <= 0 || tiles > 0xFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_router_items_kernel, dim3(1), dim3(WG), 0, st, T, tiles, list, items, hdr);
    return hipGetLastError();
}

hipError_t launch_pf_moe_combine(const PfMoeArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(pf_moe_combine_kernel, dim3((unsigned)((a.dim + WG - 1) / WG), (unsigned)a.T), dim3(WG), 0, st,
                       a);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const DMat &emb, const int32_t *tokens, int n, float *x, hipStream_t st) {
    const int units = emb.cols / 64;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)((units + WG - 1) / WG), (unsigned)n), dim3(WG), 0, st, emb,
                       tokens, x);
    return hipGetLastError();
}

// ------------------------------------------------------- KV conversion --
// The .oikv state file holds K and V as f32 rows [pos][n_kv * hd]
// (qwen3_5/kv_persist.odin:210-260); the device cache is f16 head-major
// [n_kv][seq_len][hd] (infer/metal.odin:443-454).  One thread per element of
// positions [0, n); consecutive threads take consecutive dimensions of one
// head, so the f16 side is read or written 128 contiguous bytes per 64 lanes.
__global__ __launch_bounds__(WG) void kv_export_kernel(const uint16_t *c, float *out, int n, int n_kv, int seq_len,
                                                       int hd) {
    const long i = (long)blockIdx.x * WG + threadIdx.x;  // over [n_kv][n][hd]
    if (i >= (long)n_kv * n * hd) return;
    const int d = (int)(i % hd), t = (int)((i / hd) % n), h = (int)(i / ((long)hd * n));
    out[((size_t)t * n_kv + h) * hd + d] = h2f(c[((size_t)h * seq_len + t) * hd + d]);
}

// f32 -> f16 round to nearest even (the reference's f16(x) cast,
// qwen3_5/metal.odin:912-940)
__global__ __launch_bounds__(WG) void kv_import_kernel(const float *in, uint16_t *c, int n, int n_kv, int seq_len,
                                                       int hd) {
    const long i = (long)blockIdx.x * WG + threadIdx.x;
    if (i >= (long)n_kv * n * hd) return;
    const int d = (int)(i % hd), t = (int)((i / hd) % n), h = (int)(i / ((long)hd * n));
    c[((size_t)h * seq_len + t) * hd + d] = f2h(in[((size_t)t * n_kv + h) * hd + d]);
}

hipError_t launch_kv_convert(bool to_f32, uint16_t *cache, float *rows, int n, int n_kv, int seq_len, int hd,
                             hipStream_t st) {
    const long total = (long)n_kv * n * hd;
    if (total <= 0) return hipSuccess;
    const dim3 grid((unsigned)((total + WG - 1) / WG));
    if (to_f32)
        hipLaunchKernelGGL(kv_export_kernel, grid, dim3(WG), 0, st, cache, rows, n, n_kv, seq_len, hd);
    else
        hipLaunchKernelGGL(kv_import_kernel, grid, dim3(WG), 0, st, rows, cache, n, n_kv, seq_len, hd);
    return hipGetLastError();
}

hipError_t launch_dequant(const DMat &m, float *out, hipStream_t st) {
    const long units = (long)m.rows * (m.cols / 64);
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((units + WG - 1) / WG)), dim3(WG), 0, st, m, out);
    return hipGetLastError();
}

}  // namespace oi
