// synth.cpp -- seeded synthetic GGUF writer (dense Qwen3, Qwen3-MoE, Qwen3.5
// hybrid) and block quantizers.
//
// New code: the reference only reads GGUF (ggml/gguf.odin:167-229) and only
// dequantizes (ggml/quant.odin:76-282).  Block layouts written here are the
// ones those readers decode; each quantizer states the layout it fills.

#include "oi_synth.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

// ggml type ids (ggml/gguf.odin:27-42)
enum { OI_T_F32 = 0, OI_T_F16 = 1, OI_T_Q4_0 = 2, OI_T_Q4_1 = 3, OI_T_Q5_0 = 6, OI_T_Q5_1 = 7,
       OI_T_Q8_0 = 8, OI_T_Q4_K = 12, OI_T_Q6_K = 14 };

// ------------------------------------------------------------------ random --

inline uint64_t splitmix64(uint64_t &s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Xoshiro {  // xoshiro256**
    uint64_t s[4];
    explicit Xoshiro(uint64_t seed) {
        uint64_t t = seed;
        for (auto &v : s) v = splitmix64(t);
    }
    static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    inline uint64_t next() {
        uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
        s[2] ^= t; s[3] = rotl(s[3], 45);
        return r;
    }
    // uniform in (0, 1], 53-bit
    inline double uniform() { return ((next() >> 11) + 1) * (1.0 / 9007199254740992.0); }
};

// Box-Muller, pairs of N(0,1) in double, returned as float.
inline void fill_normal(Xoshiro &g, float *out, int64_t n, float scale, float mean) {
    int64_t i = 0;
    for (; i + 1 < n; i += 2) {
        double u1 = g.uniform(), u2 = g.uniform();
        double r = std::sqrt(-2.0 * std::log(u1)), a = 6.283185307179586 * u2;
        out[i] = (float)(mean + scale * r * std::cos(a));
        out[i + 1] = (float)(mean + scale * r * std::sin(a));
    }
    if (i < n) {
        double u1 = g.uniform(), u2 = g.uniform();
        out[i] = (float)(mean + scale * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
}

uint64_t fnv1a(const char *s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; ++s) h = (h ^ (uint8_t)*s) * 0x100000001b3ull;
    return h;
}

uint64_t row_seed(uint64_t seed, uint64_t name_hash, int64_t row) {
    uint64_t t = seed ^ (name_hash * 0x9E3779B97F4A7C15ull) ^ ((uint64_t)row * 0xD1B54A32D192ED03ull);
    splitmix64(t);
    return splitmix64(t);
}

template <class F>
void parallel_for(int64_t n, int nthreads, F f) {
    if (nthreads <= 1 || n < 2) {
        f(0, n);
        return;
    }
    int nt = (int)std::min<int64_t>(nthreads, n);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++) {
        int64_t a = n * t / nt, b = n * (t + 1) / nt;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto &x : th) x.join();
}

// ------------------------------------------------------------------- f16 ---

// binary32 -> binary16 bits, round to nearest even (via the float rounding of
// a scaled value; handles subnormals, overflow, inf and nan).
uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    float a;
    std::memcpy(&a, &ax, 4);
    if (ax < 0x38800000u) {
        // subnormal range: the f16 value is an integer multiple of 2^-24;
        // adding 0.5 (2^-1) shifts the ulp of a float to 2^-24, so the float
        // add rounds (RNE) at exactly the f16 subnormal grid.
        float t = a + 0.5f;
        uint32_t tb;
        std::memcpy(&tb, &t, 4);
        return (uint16_t)(sign | (tb - 0x3F000000u));
    }
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t e = (ax >> 23) - 112;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    q += (rem > 0x1000u) || (rem == 0x1000u && (q & 1u));
    return (uint16_t)(sign | q);
}

float f16_bits_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 1024), (int)e - 25);
    return s ? -v : v;
}

inline void put_f16(uint8_t *p, float f) {
    uint16_t h = f32_to_f16_bits(f);
    p[0] = (uint8_t)h;
    p[1] = (uint8_t)(h >> 8);
}

inline int nearest_int(float v) { return (int)std::nearbyint(v); }

// -------------------------------------------------------------- quantizers --

// Q8_0: block of 32 = f16 d + 32 x int8 (ggml/quant.odin:87-96 decodes it).
void quant_q8_0(const float *x, int64_t n, uint8_t *y) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, y += 34) {
        float amax = 0;
        for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
        float d = amax / 127.0f;
        put_f16(y, d);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d));
        float id = dq != 0 ? 1.0f / dq : 0.0f;
        for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)std::clamp(nearest_int(x[j] * id), -127, 127);
    }
}

// Q4_0: f16 d + 16 bytes; element j in low nibble of byte j, j+16 in high;
// value (q-8)*d (ggml/quant.odin:98-111).
void quant_q4_0(const float *x, int64_t n, uint8_t *y) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, y += 18) {
        float amax = 0, vmax = 0;
        for (int j = 0; j < 32; j++)
            if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); vmax = x[j]; }
        float d = vmax / -8.0f;
        put_f16(y, d);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d));
        float id = dq != 0 ? 1.0f / dq : 0.0f;
        for (int j = 0; j < 16; j++) {
            int a = std::clamp(nearest_int(x[j] * id) + 8, 0, 15);
            int c = std::clamp(nearest_int(x[j + 16] * id) + 8, 0, 15);
            y[2 + j] = (uint8_t)(a | (c << 4));
        }
    }
}

// Q4_1: f16 d, f16 m + 16 bytes; value q*d + m (ggml/quant.odin:113-125).
void quant_q4_1(const float *x, int64_t n, uint8_t *y) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, y += 20) {
        float mn = x[0], mx = x[0];
        for (int j = 1; j < 32; j++) { mn = std::min(mn, x[j]); mx = std::max(mx, x[j]); }
        float d = (mx - mn) / 15.0f;
        put_f16(y, d);
        put_f16(y + 2, mn);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d)), mq = f16_bits_to_f32(f32_to_f16_bits(mn));
        float id = dq != 0 ? 1.0f / dq : 0.0f;
        for (int j = 0; j < 16; j++) {
            int a = std::clamp(nearest_int((x[j] - mq) * id), 0, 15);
            int c = std::clamp(nearest_int((x[j + 16] - mq) * id), 0, 15);
            y[4 + j] = (uint8_t)(a | (c << 4));
        }
    }
}

// Q5_0: f16 d, u32 qh (bit j = 5th bit of element j), 16 bytes of nibbles;
// value (q-16)*d (ggml/quant.odin:127-143).
void quant_q5_0(const float *x, int64_t n, uint8_t *y) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, y += 22) {
        float amax = 0, vmax = 0;
        for (int j = 0; j < 32; j++)
            if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); vmax = x[j]; }
        float d = vmax / -16.0f;
        put_f16(y, d);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d));
        float id = dq != 0 ? 1.0f / dq : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            int a = std::clamp(nearest_int(x[j] * id) + 16, 0, 31);
            int c = std::clamp(nearest_int(x[j + 16] * id) + 16, 0, 31);
            y[6 + j] = (uint8_t)((a & 15) | ((c & 15) << 4));
            qh |= (uint32_t)((a >> 4) & 1) << j;
            qh |= (uint32_t)((c >> 4) & 1) << (j + 16);
        }
        std::memcpy(y + 2, &qh, 4);
    }
}

// Q5_1: f16 d, f16 m, u32 qh, 16 bytes; value q*d + m (ggml/quant.odin:145-162).
void quant_q5_1(const float *x, int64_t n, uint8_t *y) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, y += 24) {
        float mn = x[0], mx = x[0];
        for (int j = 1; j < 32; j++) { mn = std::min(mn, x[j]); mx = std::max(mx, x[j]); }
        float d = (mx - mn) / 31.0f;
        put_f16(y, d);
        put_f16(y + 2, mn);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d)), mq = f16_bits_to_f32(f32_to_f16_bits(mn));
        float id = dq != 0 ? 1.0f / dq : 0.0f;
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            int a = std::clamp(nearest_int((x[j] - mq) * id), 0, 31);
            int c = std::clamp(nearest_int((x[j + 16] - mq) * id), 0, 31);
            y[8 + j] = (uint8_t)((a & 15) | ((c & 15) << 4));
            qh |= (uint32_t)((a >> 4) & 1) << j;
            qh |= (uint32_t)((c >> 4) & 1) << (j + 16);
        }
        std::memcpy(y + 4, &qh, 4);
    }
}

// Q4_K: super-block of 256 = f16 d, f16 dmin, 12 bytes of packed 6-bit
// (scale, min) for 8 groups of 32, 128 bytes of nibbles.  Group 2p holds the
// low nibbles of qs[32p..32p+31], group 2p+1 the high nibbles; element value
// d*sc*q - dmin*m (ggml/quant.odin:178-209; unpacking at :64-73).
void quant_q4_k(const float *x, int64_t n, uint8_t *y) {
    for (int64_t sb = 0; sb < n / 256; sb++, x += 256, y += 144) {
        float scale[8], mins[8];
        for (int g = 0; g < 8; g++) {
            const float *v = x + 32 * g;
            float mn = v[0], mx = v[0];
            for (int j = 1; j < 32; j++) { mn = std::min(mn, v[j]); mx = std::max(mx, v[j]); }
            if (mn > 0) mn = 0;
            scale[g] = (mx - mn) / 15.0f;
            mins[g] = -mn;
        }
        float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(mins, mins + 8);
        float d = ms / 63.0f, dmin = mm / 63.0f;
        put_f16(y, d);
        put_f16(y + 2, dmin);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d)), dmq = f16_bits_to_f32(f32_to_f16_bits(dmin));
        uint8_t sc[8], m[8];
        for (int g = 0; g < 8; g++) {
            sc[g] = (uint8_t)(dq > 0 ? std::clamp(nearest_int(scale[g] / dq), 0, 63) : 0);
            m[g] = (uint8_t)(dmq > 0 ? std::clamp(nearest_int(mins[g] / dmq), 0, 63) : 0);
        }
        uint8_t *s = y + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t q[256];
        for (int g = 0; g < 8; g++) {
            float step = dq * (float)sc[g], off = dmq * (float)m[g];
            for (int j = 0; j < 32; j++)
                q[32 * g + j] = (uint8_t)(step > 0 ? std::clamp(nearest_int((x[32 * g + j] + off) / step), 0, 15) : 0);
        }
        uint8_t *qs = y + 16;
        for (int p = 0; p < 4; p++)
            for (int l = 0; l < 32; l++) qs[32 * p + l] = (uint8_t)(q[64 * p + l] | (q[64 * p + 32 + l] << 4));
    }
}

// Q6_K: super-block of 256 = ql[128], qh[64], int8 scales[16] (one per 16
// elements), f16 d.  Element e = 128h + 32k + l (h<2, k<4, l<32) has its low
// 4 bits in ql[64h + l + 32(k&1)] (nibble k>>1) and its high 2 bits in
// qh[32h + l] bits 2k..2k+1; value d*sc[e/16]*(q-32) (ggml/quant.odin:212-247).
void quant_q6_k(const float *x, int64_t n, uint8_t *y) {
    for (int64_t sb = 0; sb < n / 256; sb++, x += 256, y += 210) {
        float scale[16];
        for (int i = 0; i < 16; i++) {
            float amax = 0;
            for (int j = 0; j < 16; j++) amax = std::max(amax, std::fabs(x[16 * i + j]));
            scale[i] = amax / 31.0f;
        }
        float ms = *std::max_element(scale, scale + 16);
        float d = ms / 127.0f;
        put_f16(y + 208, d);
        float dq = f16_bits_to_f32(f32_to_f16_bits(d));
        int8_t *sc = (int8_t *)(y + 192);
        uint8_t q[256];
        for (int i = 0; i < 16; i++) {
            int s = dq > 0 ? std::clamp(nearest_int(scale[i] / dq), -128, 127) : 0;
            sc[i] = (int8_t)s;
            float step = dq * (float)s;
            for (int j = 0; j < 16; j++)
                q[16 * i + j] = (uint8_t)(step != 0 ? std::clamp(nearest_int(x[16 * i + j] / step), -32, 31) + 32 : 32);
        }
        uint8_t *ql = y, *qh = y + 128;
        std::memset(ql, 0, 128);
        std::memset(qh, 0, 64);
        for (int h = 0; h < 2; h++)
            for (int k = 0; k < 4; k++)
                for (int l = 0; l < 32; l++) {
                    int e = 128 * h + 32 * k + l;
                    ql[64 * h + l + 32 * (k & 1)] |= (uint8_t)((q[e] & 15) << (4 * (k >> 1)));
                    qh[32 * h + l] |= (uint8_t)((q[e] >> 4) << (2 * k));
                }
    }
}

int block_info(int t, int *elems, int *bytes) {
    switch (t) {
    case OI_T_F32: *elems = 1; *bytes = 4; return 0;
    case OI_T_F16: *elems = 1; *bytes = 2; return 0;
    case OI_T_Q4_0: *elems = 32; *bytes = 18; return 0;
    case OI_T_Q4_1: *elems = 32; *bytes = 20; return 0;
    case OI_T_Q5_0: *elems = 32; *bytes = 22; return 0;
    case OI_T_Q5_1: *elems = 32; *bytes = 24; return 0;
    case OI_T_Q8_0: *elems = 32; *bytes = 34; return 0;
    case OI_T_Q4_K: *elems = 256; *bytes = 144; return 0;
    case OI_T_Q6_K: *elems = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

int quantize_row(int t, const float *x, int64_t n, uint8_t *y) {
    int e, b;
    if (block_info(t, &e, &b) || n % e) return -1;
    switch (t) {
    case OI_T_F32: std::memcpy(y, x, (size_t)n * 4); return 0;
    case OI_T_F16:
        for (int64_t i = 0; i < n; i++) put_f16(y + 2 * i, x[i]);
        return 0;
    case OI_T_Q4_0: quant_q4_0(x, n, y); return 0;
    case OI_T_Q4_1: quant_q4_1(x, n, y); return 0;
    case OI_T_Q5_0: quant_q5_0(x, n, y); return 0;
    case OI_T_Q5_1: quant_q5_1(x, n, y); return 0;
    case OI_T_Q8_0: quant_q8_0(x, n, y); return 0;
    case OI_T_Q4_K: quant_q4_k(x, n, y); return 0;
    case OI_T_Q6_K: quant_q6_k(x, n, y); return 0;
    default: return -1;
    }
}

// --------------------------------------------------------------- writer -----

struct Writer {
    FILE *f = nullptr;
    bool ok = true;
    void raw(const void *p, size_t n) {
        if (ok && n && std::fwrite(p, 1, n, f) != n) ok = false;
    }
    void u32(uint32_t v) { raw(&v, 4); }
    void u64(uint64_t v) { raw(&v, 8); }
    void str(const std::string &s) { u64(s.size()); raw(s.data(), s.size()); }
};

struct TensorPlan {
    std::string name;
    int type;
    std::vector<uint64_t> dims;  // GGUF order: dims[0] is the row length
    int64_t rows, cols;          // generated as rows x cols (rows = product of dims[1..])
    float sigma, mean;
    int transform;               // 0: as drawn; 1: -exp(v) (ssm_a = -exp(A_log))
    uint64_t offset, bytes;
};

}  // namespace

extern "C" {

int oi_quantize_rows(int32_t type, const float *src, int64_t nrows, int64_t ncols, uint8_t *dst) {
    int e, b;
    if (!src || !dst || nrows < 0 || ncols <= 0 || block_info(type, &e, &b) || ncols % e) return -1;
    const int64_t rb = ncols / e * b;
    const int nt = (int)std::min<int64_t>(16, std::max<unsigned>(1u, std::thread::hardware_concurrency()));
    parallel_for(nrows, nrows * ncols >= (1 << 20) ? nt : 1, [&](int64_t a, int64_t z) {
        for (int64_t r = a; r < z; r++) quantize_row(type, src + r * ncols, ncols, dst + r * rb);
    });
    return 0;
}

void oi_synth_normal_f32(uint64_t seed, int64_t n, float scale, float *out, int32_t n_threads) {
    const int64_t chunk = 1 << 16;
    int64_t nchunks = (n + chunk - 1) / chunk;
    parallel_for(nchunks, n_threads, [&](int64_t a, int64_t b) {
        for (int64_t c = a; c < b; c++) {
            Xoshiro g(row_seed(seed, 0x6b76u, c));
            fill_normal(g, out + c * chunk, std::min(chunk, n - c * chunk), scale, 0.0f);
        }
    });
}

void oi_synth_normal_f16(uint64_t seed, int64_t n, float scale, uint16_t *out, int32_t n_threads) {
    const int64_t chunk = 1 << 16;
    int64_t nchunks = (n + chunk - 1) / chunk;
    parallel_for(nchunks, n_threads, [&](int64_t a, int64_t b) {
        std::vector<float> tmp(chunk);
        for (int64_t c = a; c < b; c++) {
            Xoshiro g(row_seed(seed, 0x6b76u, c));
            int64_t m = std::min(chunk, n - c * chunk);
            fill_normal(g, tmp.data(), m, scale, 0.0f);
            for (int64_t i = 0; i < m; i++) out[c * chunk + i] = f32_to_f16_bits(tmp[i]);
        }
    });
}

void oi_synth_tensor_f32(uint64_t seed, const char *name, int64_t rows, int64_t cols, float sigma,
                         float mean, float *out, int32_t n_threads) {
    uint64_t h = fnv1a(name);
    parallel_for(rows, n_threads, [&](int64_t a, int64_t b) {
        for (int64_t r = a; r < b; r++) {
            Xoshiro g(row_seed(seed, h, r));
            fill_normal(g, out + r * cols, cols, sigma, mean);
        }
    });
}

int oi_synth_write_gguf(const char *path, const oi_synth_spec *s) {
    if (!path || !s || s->dim <= 0 || s->n_layers <= 0 || s->n_heads <= 0 || s->n_kv_heads <= 0 ||
        s->head_dim <= 0 || s->vocab_size <= 0 || s->hidden_dim <= 0 || s->arch < 0 || s->arch > 2)
        return -1;
    const bool moe = s->arch == 1 || (s->arch == 2 && s->n_experts > 0);
    if (moe && (s->n_experts <= 0 || s->n_experts_used <= 0 || s->n_experts_used > s->n_experts ||
                s->expert_ffn <= 0))
        return -1;
    if (s->arch == 2 && (s->full_attn_interval <= 0 || s->rotary_dim <= 0 || s->lin_n_k_heads <= 0 ||
                         s->lin_n_v_heads <= 0 || s->lin_head_k_dim <= 0 || s->lin_head_v_dim <= 0 ||
                         s->lin_conv_kernel <= 0))
        return -1;
    const int nt = s->n_threads > 0 ? s->n_threads : 1;
    std::vector<TensorPlan> plan;
    auto add2 = [&](const std::string &nm, int type, int64_t rows, int64_t cols) {
        plan.push_back({nm, type, {(uint64_t)cols, (uint64_t)rows}, rows, cols, s->sigma, 0.0f, 0, 0, 0});
    };
    auto add3 = [&](const std::string &nm, int type, int64_t n_exp, int64_t rows, int64_t cols) {
        plan.push_back({nm, type, {(uint64_t)cols, (uint64_t)rows, (uint64_t)n_exp}, n_exp * rows, cols, s->sigma,
                        0.0f, 0, 0, 0});
    };
    auto add1 = [&](const std::string &nm, int64_t n) {  // F32 norm weight, 1 + N(0, norm_sigma)
        plan.push_back({nm, OI_T_F32, {(uint64_t)n}, 1, n, s->norm_sigma, 1.0f, 0, 0, 0});
    };
    auto add1v = [&](const std::string &nm, int64_t n, float sigma, float mean, int transform) {
        plan.push_back({nm, OI_T_F32, {(uint64_t)n}, 1, n, sigma, mean, transform, 0, 0});
    };
    const int64_t D = s->dim, H = s->hidden_dim, Q = s->n_heads * s->head_dim, KV = s->n_kv_heads * s->head_dim;
    const int64_t E = s->n_experts, EF = s->expert_ffn, SF = s->shared_expert_ffn;
    const int64_t KD = (int64_t)s->lin_n_k_heads * s->lin_head_k_dim, VD = (int64_t)s->lin_n_v_heads * s->lin_head_v_dim;
    const int64_t CD = 2 * KD + VD;
    add2("token_embd.weight", s->type_embd, s->vocab_size, D);
    add1("output_norm.weight", D);
    if (s->type_output >= 0) add2("output.weight", s->type_output, s->vocab_size, D);
    for (int64_t l = 0; l < s->n_layers; l++) {
        std::string p = "blk." + std::to_string(l) + ".";
        add1(p + "attn_norm.weight", D);
        // the Qwen3.5 loader calls the FFN norm post_attention_norm (qwen3_5/model.odin:325)
        add1(p + (s->arch == 2 ? "post_attention_norm.weight" : "ffn_norm.weight"), D);
        const bool full = s->arch != 2 || (l + 1) % s->full_attn_interval == 0;  // qwen3_5/model.odin:289-300
        if (full) {
            add1(p + "attn_q_norm.weight", s->head_dim);
            add1(p + "attn_k_norm.weight", s->head_dim);
            add2(p + "attn_q.weight", s->type_default, s->arch == 2 ? 2 * Q : Q, D);  // [q | gate] per head
            add2(p + "attn_k.weight", s->type_default, KV, D);
            add2(p + "attn_v.weight", s->type_attn_v, KV, D);
            add2(p + "attn_output.weight", s->type_default, D, Q);
        } else {  // gated DeltaNet (qwen3_5/model.odin:346-360)
            add2(p + "attn_qkv.weight", s->type_default, CD, D);
            add2(p + "attn_gate.weight", s->type_default, VD, D);
            add2(p + "ssm_beta.weight", s->type_default, s->lin_n_v_heads, D);
            add2(p + "ssm_alpha.weight", s->type_default, s->lin_n_v_heads, D);
            plan.push_back({p + "ssm_conv1d.weight", OI_T_F32,
                            {(uint64_t)s->lin_conv_kernel, (uint64_t)CD}, CD, s->lin_conv_kernel, 0.25f, 0.0f, 0, 0, 0});
            add1v(p + "ssm_dt.bias", s->lin_n_v_heads, 0.5f, 0.0f, 0);
            add1v(p + "ssm_a", s->lin_n_v_heads, 0.5f, 0.0f, 1);
            add1(p + "ssm_norm.weight", s->lin_head_v_dim);
            add2(p + "ssm_out.weight", s->type_default, D, VD);
        }
        if (!moe) {
            add2(p + "ffn_gate.weight", s->type_default, H, D);
            add2(p + "ffn_down.weight", s->type_ffn_down, D, H);
            add2(p + "ffn_up.weight", s->type_default, H, D);
        } else {
            add2(p + "ffn_gate_inp.weight", s->type_router, E, D);
            add3(p + "ffn_gate_exps.weight", s->type_default, E, EF, D);
            add3(p + "ffn_up_exps.weight", s->type_default, E, EF, D);
            add3(p + "ffn_down_exps.weight", s->type_ffn_down, E, D, EF);
            if (s->arch == 2 && SF > 0) {
                add2(p + "ffn_gate_inp_shexp.weight", s->type_router, 1, D);
                add2(p + "ffn_gate_shexp.weight", s->type_default, SF, D);
                add2(p + "ffn_up_shexp.weight", s->type_default, SF, D);
                add2(p + "ffn_down_shexp.weight", s->type_ffn_down, D, SF);
            }
        }
    }
    const uint64_t align = 32;
    uint64_t off = 0;
    for (auto &t : plan) {
        int e, b;
        if (block_info(t.type, &e, &b) || t.cols % e) return -2;
        t.bytes = (uint64_t)(t.rows * (t.cols / e) * b);
        t.offset = off;
        off = (off + t.bytes + align - 1) & ~(align - 1);
    }
    Writer w;
    w.f = std::fopen(path, "wb");
    if (!w.f) return -3;
    const char *arch = s->arch == 0 ? "qwen3" : s->arch == 1 ? "qwen3moe" : "qwen35";
    const std::string a = std::string(arch) + ".";
    // metadata: the keys the loaders read (infer/model.odin:103-134;
    // qwen3_5/model.odin:245-282), plus the expert counts of routed-expert models
    struct MetaKV {
        std::string k;
        int kind;  // 4 u32, 6 f32, 8 string
        uint32_t u;
        float f;
        std::string str;
    };
    std::vector<MetaKV> meta;
    auto kv_u32 = [&](const std::string &k, int64_t v) { meta.push_back({k, 4, (uint32_t)v, 0.f, ""}); };
    auto kv_f32 = [&](const std::string &k, float v) { meta.push_back({k, 6, 0, v, ""}); };
    meta.push_back({"general.architecture", 8, 0, 0.f, arch});
    meta.push_back({"general.name", 8, 0, 0.f, "odin-infer-amd synthetic"});
    kv_u32("general.alignment", (int64_t)align);
    kv_u32(a + "embedding_length", D);
    kv_u32(a + "feed_forward_length", moe ? EF : H);
    kv_u32(a + "block_count", s->n_layers);
    kv_u32(a + "attention.head_count", s->n_heads);
    kv_u32(a + "attention.head_count_kv", s->n_kv_heads);
    kv_u32(a + "context_length", s->context_length);
    kv_u32(a + "attention.key_length", s->head_dim);
    kv_u32(a + "attention.value_length", s->head_dim);
    kv_f32(a + "rope.freq_base", s->rope_theta);
    kv_f32(a + "attention.layer_norm_rms_epsilon", s->rms_eps);
    if (moe) {
        kv_u32(a + "expert_count", E);
        kv_u32(a + "expert_used_count", s->n_experts_used);
        kv_u32(a + "expert_feed_forward_length", EF);
        if (s->arch == 2 && SF > 0) kv_u32(a + "expert_shared_feed_forward_length", SF);
    }
    if (s->arch == 2) {
        kv_u32(a + "ssm.group_count", s->lin_n_k_heads);
        kv_u32(a + "ssm.time_step_rank", s->lin_n_v_heads);
        kv_u32(a + "ssm.state_size", s->lin_head_k_dim);
        kv_u32(a + "ssm.inner_size", VD);
        kv_u32(a + "ssm.conv_kernel", s->lin_conv_kernel);
        kv_u32(a + "full_attention_interval", s->full_attn_interval);
        kv_u32(a + "rope.dimension_count", s->rotary_dim);
    }
    // header (ggml/gguf.odin:177-189)
    w.u32(0x46554747u);
    w.u32(3);
    w.u64(plan.size());
    w.u64(meta.size());
    for (auto &m : meta) {
        w.str(m.k);
        w.u32((uint32_t)m.kind);
        if (m.kind == 4) w.u32(m.u);
        else if (m.kind == 6) w.raw(&m.f, 4);
        else w.str(m.str);
    }
    // tensor infos (ggml/gguf.odin:198-212): dims[0] is the row length
    for (auto &t : plan) {
        w.str(t.name);
        w.u32((uint32_t)t.dims.size());
        for (uint64_t d : t.dims) w.u64(d);
        w.u32((uint32_t)t.type);
        w.u64(t.offset);
    }
    long pos = std::ftell(w.f);
    std::vector<uint8_t> pad(align, 0);
    w.raw(pad.data(), (size_t)(((uint64_t)pos + align - 1) / align * align - (uint64_t)pos));
    uint64_t written = 0;
    std::vector<uint8_t> buf;
    for (auto &t : plan) {
        if (t.offset > written) w.raw(pad.data(), (size_t)(t.offset - written));
        written = t.offset;
        buf.assign(t.bytes, 0);
        int e = 1, b = 4;
        block_info(t.type, &e, &b);
        const int64_t rb = t.cols / e * b;
        const uint64_t h = fnv1a(t.name.c_str());
        bool bad = false;
        parallel_for(t.rows, nt, [&](int64_t a0, int64_t z) {
            std::vector<float> row((size_t)t.cols);
            for (int64_t r = a0; r < z; r++) {
                Xoshiro g(row_seed(s->seed, h, r));
                fill_normal(g, row.data(), t.cols, t.sigma, t.mean);
                if (t.transform == 1)
                    for (auto &v : row) v = -std::exp(v);
                if (quantize_row(t.type, row.data(), t.cols, buf.data() + r * rb)) bad = true;
            }
        });
        if (bad) { std::fclose(w.f); return -4; }
        w.raw(buf.data(), buf.size());
        written += t.bytes;
    }
    bool ok = w.ok;
    if (std::fclose(w.f) != 0) ok = false;
    return ok ? 0 : -5;
}

}  // extern "C"
