// device_common.h -- device helpers shared by the gfx950 kernels.
#pragma once
#include "oi_kernels.h"

namespace oi {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr int WG = 256;

static __device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// f32 -> f16, round to nearest even, of the f32 value f.  The empty asm keeps
// the compiler from folding the conversion into the instruction that computed
// f: v_fma_mixlo/mixhi_f16 round the exact product or sum to f16 once, which
// differs from rounding it to f32 first in about 1 of 10^4 cases on gfx950.
static __device__ __forceinline__ uint16_t f2h(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <class T>
static __device__ __forceinline__ T ldg_nt(const T *p) {
    return __builtin_nontemporal_load(p);
}

// (sc, m) of groups 2p and 2p+1 of a Q4_K super-block from the device header
// words hw1..hw3 (bits 24p..24p+23 of the 96-bit tail, see DMat)
static __device__ __forceinline__ void q4k_scales(int p, uint32_t hw1, uint32_t hw2, uint32_t hw3, uint32_t &sc0,
                                                  uint32_t &m0, uint32_t &sc1, uint32_t &m1) {
    const uint32_t lo = p == 0 || p == 1 ? hw1 : (p == 2 ? hw2 : hw3), hi = p < 2 ? hw2 : hw3;
    const uint32_t f = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)((24 * p) & 31));
    sc0 = f & 63u;
    m0 = (f >> 6) & 63u;
    sc1 = (f >> 12) & 63u;
    m1 = (f >> 18) & 63u;
}

// Cross-lane moves within rows of 16 lanes (DPP), cheaper than LDS-routed
// shuffles: quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror (lane i of
// each 8 <-> 7-i) and row_mirror (lane i of each 16 <-> 15-i).
#define OI_DPP(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
static __device__ __forceinline__ float dpp_sum4(float v) {  // sum over aligned groups of 4 lanes
    v += OI_DPP(v, 0xB1);
    return v + OI_DPP(v, 0x4E);
}
static __device__ __forceinline__ float dpp_mirror8(float v) { return OI_DPP(v, 0x141); }
static __device__ __forceinline__ float dpp_max8(float v) {  // max over aligned groups of 8 lanes
    v = fmaxf(v, OI_DPP(v, 0xB1));
    v = fmaxf(v, OI_DPP(v, 0x4E));
    return fmaxf(v, OI_DPP(v, 0x141));
}
// lane j's value (j uniform), read into a scalar register
static __device__ __forceinline__ float lane_value(float v, int j) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}
// sum over aligned groups of n lanes (n a power of two <= 64); every lane of
// a group ends with the group's sum.  Rows of 16 by DPP, then the rows' sums
// read out of lanes 0, 16, 32, 48 and added as (r0 + r1) + (r2 + r3) (the
// order of the two xor-16 / xor-32 butterfly steps, without their two LDS
// round trips).  The whole wave must be active.
static __device__ __forceinline__ float lane_group_sum(float v, int n) {
    if (n >= 2) v += OI_DPP(v, 0xB1);
    if (n >= 4) v += OI_DPP(v, 0x4E);
    if (n >= 8) v += OI_DPP(v, 0x141);
    if (n >= 16) v += OI_DPP(v, 0x140);
    if (n >= 32) {
        const float lo = lane_value(v, 0) + lane_value(v, 16), hi = lane_value(v, 32) + lane_value(v, 48);
        v = n >= 64 ? lo + hi : (__lane_id() < 32 ? lo : hi);
    }
    return v;
}
static __device__ __forceinline__ float wave_sum(float v) { return lane_group_sum(v, WAVE); }
// maximum over the wave (whole wave active)
static __device__ __forceinline__ float wave_max_all(float v) {
    v = fmaxf(v, OI_DPP(v, 0xB1));
    v = fmaxf(v, OI_DPP(v, 0x4E));
    v = fmaxf(v, OI_DPP(v, 0x141));
    v = fmaxf(v, OI_DPP(v, 0x140));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Qwen3.5 activations (qwen3_5/ops.odin:7-15 sigmoid: the branch keeps exp's
// argument <= 0; silu = x sigmoid(x))
static __device__ __forceinline__ float sigmoid_ref(float x) {
#pragma clang fp contract(off)
    if (x >= 0.0f) {
        const float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = expf(x);
    return z / (1.0f + z);
}
static __device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }
// qwen3_5/ops.odin:20-24 (the logarithm in double precision, as the reference)
static __device__ __forceinline__ float softplus_ref(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return 0.0f;
    return (float)log((double)(1.0f + expf(x)));
}

// sum of the K-slice partial products of element i (a split projection's
// slices, each `slice` floats, summed in slice order)
static __device__ __forceinline__ float parts_at(const float *p, int split, size_t slice, size_t i) {
    // slices requested 8 at a time (a runtime trip count would make every
    // load wait for the sum before it), summed in slice order
    float s = p[i];
    for (int z0 = 1; z0 < split; z0 += 8) {
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (z0 + k < split) t[k] = p[(size_t)(z0 + k) * slice + i];
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (z0 + k < split) s += t[k];
    }
    return s;
}

// v[j] = parts_at(p, split, slice, idx(j)) for j < N, with the same sums in
// the same order, but the loads of max(1, 16 / N) slices are requested
// together: ceil(split / that) memory round trips instead of one per element
// and slice (a runtime trip count inside the element loop makes every load
// wait for the one before)
template <int N, class F>
static __device__ __forceinline__ void parts_gather(float (&v)[N], const float *p, int split, size_t slice, F idx) {
    constexpr int B = N >= 16 ? 1 : 16 / N;
#pragma unroll
    for (int j = 0; j < N; j++) v[j] = p[idx(j)];
    for (int z0 = 1; z0 < split; z0 += B) {
        float t[B][N];
#pragma unroll
        for (int k = 0; k < B; k++) {
            const float *q = p + (size_t)(z0 + k) * slice;
            if (z0 + k < split) {
#pragma unroll
                for (int j = 0; j < N; j++) t[k][j] = q[idx(j)];
            }
        }
#pragma unroll
        for (int k = 0; k < B; k++)
            if (z0 + k < split) {
#pragma unroll
                for (int j = 0; j < N; j++) v[j] += t[k][j];
            }
    }
}

// (value, index) order of a greedy argmax that keeps the first maximum
// (sampler/sampler.odin:79-89 scans with a strict '>')
static __device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// rows [r0, r0 + n) of m as a matrix of its own (same planes)
static __device__ __forceinline__ DMat sub_rows(const DMat &m, int r0, int n) {
    DMat s = m;
    s.rows = n;
    const size_t r = (size_t)r0;
    switch (m.type) {
    case T_Q4_K: s.q += r * (m.cols >> 6) * 16; s.s += r * (m.cols >> 8) * 16; break;
    case T_Q6_K: s.q += r * (m.cols >> 6) * 16; s.s += r * (m.cols >> 8) * 16; s.d += r * (m.cols >> 8); break;
    case T_Q8_0: s.q += r * (m.cols >> 6) * 16; s.d += r * (m.cols >> 5); break;
    case T_F16: s.q += r * m.cols * 2; break;
    case T_Q4_0: s.q += r * (m.cols >> 5) * 18; break;
    case T_Q4_1: s.q += r * (m.cols >> 5) * 20; break;
    case T_Q5_0: s.q += r * (m.cols >> 5) * 22; break;
    case T_Q5_1: s.q += r * (m.cols >> 5) * 24; break;
    default: s.q += r * m.cols * 4; break;
    }
    return s;
}

// The k-th largest of the wave's keys v[0..NV) (the caller has checked that
// more than k are nonzero; nonzero keys are distinct), one bit at a time from
// the top: the largest T with at least k keys >= T, ending early once exactly
// k keys are >= T.  Counts are ballots, so every lane of the wave takes part.
template <int NV>
static __device__ __forceinline__ unsigned long long wave_kth_key(const unsigned long long (&v)[NV], int k) {
    unsigned long long T = 0ull;
#pragma unroll
    for (int b = 41; b >= 0; b--) {
        const unsigned long long tr = T | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NV; i++) cnt += __popcll(__ballot(v[i] >= tr));
        if (cnt >= k) {
            T = tr;
            if (cnt == k) break;
        }
    }
    return T;
}

// Rows for the int8 expert and router kernels (mt_q4i8_kernel's A operand):
// a row scaled by one factor, s = max|x| / QI_MAX, to integers below 2^28,
// split into four 7-bit planes (the top one signed).
constexpr float QI_MAX = 268434432.f;  // 2^28 - 2^10: the rounded product stays below 2^28
// Row r held as NV float4 per thread of a BS-thread workgroup (float4 c =
// thread + BS i, K / 4 a multiple of 64): its planes stored slot by slot in
// the kernel's operand order (unit u, lane group G, plane pl: 16 bytes at
// ((r U + u) 16 + 4 G + pl)), its 32-element group sums and its scale, with
// that kernel's own prologue arithmetic (the same maximum, rounding, and sum
// order over the same lanes).  red: BS / 64 floats of LDS, free on entry
// after a barrier.
template <int NV, int BS>
static __device__ __forceinline__ void qi_quant_row(const float4 (&v)[NV], int K, size_t r, float *red, u32x4 *q,
                                                    float *gsum, float *scale) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid / WAVE, U = K >> 6;
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = tid + i * BS;
        if (c < K / 4) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    amax = wave_max_all(amax);
    __syncthreads();  // the previous use of red is complete
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float mx = 0.f;
#pragma unroll
    for (int w = 0; w < BS / WAVE; w++) mx = fmaxf(mx, red[w]);
    const float inv = mx > 0.f ? QI_MAX / mx : 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = tid + i * BS;
        if (c >= K / 4) break;  // whole waves
        const float4 t = v[i];
        const float sum = (t.x + t.y) + (t.z + t.w);
        const float sum16 = dpp_sum4(sum);
        const float sum32 = sum16 + dpp_mirror8(sum16);
        if ((c & 7) == 0) gsum[r * (K / 32) + (c >> 3)] = sum32;
        const int qi[4] = {(int)rintf(t.x * inv), (int)rintf(t.y * inv), (int)rintf(t.z * inv), (int)rintf(t.w * inv)};
        const int u = c >> 4, i4 = c & 15;
        uint32_t *dst = (uint32_t *)(q + (r * U + u) * 16 + ((i4 >> 1) & 3) * 4) + ((i4 >> 3) & 1) * 2 + (i4 & 1);
#pragma unroll
        for (int pl = 0; pl < 4; pl++) {
            const int sh = 21 - 7 * pl;
            uint32_t b = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) b |= ((uint32_t)(qi[k] >> sh) & (pl == 0 ? 0xFFu : 0x7Fu)) << (8 * k);
            dst[pl * 4] = b;
        }
    }
    if (tid == 0) scale[r] = mx / QI_MAX;
}

}  // namespace oi
