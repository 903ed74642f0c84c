// oi_kernels.h -- descriptors shared by the host code and the gfx950 kernels,
// and the host-side launchers of every kernel in kernels.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oi {

// ggml type ids (reference ggml/gguf.odin:27-42)
enum : int32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

// A weight matrix resident in HBM, in the GEMV layout.  Every matrix is cut
// into "units" of 64 consecutive weights of one row; a unit is the work of
// one lane.  Per type:
//   Q4_K  q: the GGUF super-blocks unchanged (144 B = 16 B header + 128 B of
//         nibbles; 144 is a multiple of 16, so every 16 B piece is aligned).
//         Unit u of a row = super-block u/4, group pair u%4.
//   Q6_K  q: per super-block the 128 B of ql then the 64 B of qh (192 B);
//         s: the 16 int8 scales per super-block; d: f16 d per super-block.
//         (The GGUF 210 B block is only 2 B aligned; this split keeps the
//         byte count and makes every load a naturally aligned 16 B piece.)
//         Unit u = super-block u/4, half h=(u%4)/2, columns l0=16*(u%2).
//   Q8_0  q: 32 B of int8 per block; d: f16 d per block.  Unit = 2 blocks.
//   F32/F16  q: the values.
struct DMat {
    int32_t type;
    int32_t rows;
    int32_t cols;
    int32_t pad;
    const uint8_t *q;
    const uint8_t *s;
    const uint16_t *d;
};

enum GemvMode : int32_t {
    GEMV_STORE = 0,   // y[r] = W x
    GEMV_ADD = 1,     // y[r] += W x            (residual epilogue)
    GEMV_SWIGLU = 2,  // y[r] = silu(Wg x) * (Wu x); seg[0]=gate, seg[1]=up
    GEMV_ARGMAX = 3   // y[r] = W x, then greedy argmax over all rows
};

struct GemvSeg {
    DMat m;
    float *y;
    int32_t wg_begin;  // first workgroup of this segment
    int32_t pad;
};

struct GemvArgs {
    GemvSeg seg[3];
    int32_t nseg;
    int32_t mode;
    int32_t K;             // row length (all segments)
    int32_t lpr;           // lanes per row (power of two, <= 64)
    int32_t rows_per_wg;
    int32_t total_wgs;
    const float *x;        // input vector, K floats
    const float *norm_w;   // if set: x is replaced by rmsnorm(x) * norm_w
    float eps;
    int32_t pad;
    // GEMV_ARGMAX
    float *am_val;         // [total_wgs]
    int32_t *am_idx;       // [total_wgs]
    int32_t *am_counter;   // 1 int, zero between launches
    int32_t *state;        // [token, pos, step, err]
    int32_t *tokens_out;   // greedy ids by step
};

struct AttnArgs {
    const float *q, *k, *v;    // this token's raw projections
    const float *q_norm, *k_norm;
    float eps;
    int32_t seq_len;
    const float2 *rope_cs;     // [seq_len][head_dim/2] (cos, sin)
    uint16_t *kc, *vc;         // this layer: [n_kv_heads][seq_len][head_dim] f16 bits
    const int32_t *state;      // pos = state[1]
    int32_t chunk;             // positions per split
    int32_t max_splits;
    float *part;               // [n_heads][max_splits][head_dim + 2]
    int32_t *counters;         // [n_kv_heads], zero between launches
    float *out;                // [n_heads * head_dim]
    int32_t n_heads, n_kv_heads;
};

// Host launchers (kernels.hip).  All return hipSuccess or the launch error.
hipError_t launch_gemv(const GemvArgs &a, hipStream_t st);
hipError_t launch_attn(const AttnArgs &a, int head_dim, hipStream_t st);
hipError_t launch_embed(const DMat &emb, const int32_t *state, float *x, int32_t vocab, hipStream_t st);
hipError_t launch_dequant(const DMat &m, float *out, hipStream_t st);

// Plan a GEMV over segments sharing one K: fills lpr, rows_per_wg, wg_begin,
// total_wgs.  Returns false if K is not a multiple of 64.
bool plan_gemv(GemvArgs &a);

}  // namespace oi
