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
static __device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <class T>
static __device__ __forceinline__ T ldg_nt(const T *p) {
    return __builtin_nontemporal_load(p);
}

// byte i (0..11) of the packed Q4_K scales held in three words
static __device__ __forceinline__ uint32_t sbyte(const uint32_t sw[3], int i) {
    uint32_t w = i < 4 ? sw[0] : (i < 8 ? sw[1] : sw[2]);
    return (w >> ((i & 3) * 8)) & 0xFFu;
}

// get_scale_min_k4 (ggml/quant.odin:64-73)
static __device__ __forceinline__ void scale_min_k4(int j, const uint32_t sw[3], uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = sbyte(sw, j) & 63u;
        m = sbyte(sw, j + 4) & 63u;
    } else {
        sc = (sbyte(sw, j + 4) & 0xFu) | ((sbyte(sw, j - 4) >> 6) << 4);
        m = (sbyte(sw, j + 4) >> 4) | ((sbyte(sw, j) >> 6) << 4);
    }
}


static __device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// (value, index) order of a greedy argmax that keeps the first maximum
// (sampler/sampler.odin:79-89 scans with a strict '>')
static __device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

}  // namespace oi
