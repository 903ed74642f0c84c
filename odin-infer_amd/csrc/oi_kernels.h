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
    int32_t ntiles;    // row tiles of this segment (gemv_q_kernel)
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
    int32_t kernel;        // 0: gemv_kernel (any type), 1: gemv_q_kernel (Q4_K/Q6_K/Q8_0)
    // GEMV_ARGMAX: per-workgroup (max, lowest index); reduced by the next
    // embedding step, which state[4] = 1 asks for
    float *am_val;         // [total_wgs]
    int32_t *am_idx;       // [total_wgs]
    int32_t *state;
};

// Device state of the token loop (int32 x 8):
//   [0] token  [1] pos  [2] step  [3] capacity of tokens_out
//   [4] argmax pending  [5] number of argmax partials
enum { ST_TOKEN = 0, ST_POS = 1, ST_STEP = 2, ST_CAP = 3, ST_PENDING = 4, ST_NPART = 5, ST_WORDS = 8 };

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
    float *out;                // [n_heads * head_dim]
    int32_t n_heads, n_kv_heads;
};

// Host launchers (kernels.hip).  All return hipSuccess or the launch error.
hipError_t launch_gemv(const GemvArgs &a, hipStream_t st);
hipError_t launch_attn(const AttnArgs &a, int head_dim, hipStream_t st);
// Embedding of state[token] into x.  If state[4] is set, first reduces the
// pending argmax partials of the previous step: token = argmax, pos += 1,
// tokens_out[step++] = token.  finalize_only: do the reduction and stop.
hipError_t launch_embed(const DMat &emb, int32_t *state, float *x, int32_t vocab, const float *am_val,
                        const int32_t *am_idx, int32_t *tokens_out, int finalize_only, hipStream_t st);
int attn_chunk(int head_dim);
int attn_max_splits();
hipError_t launch_dequant(const DMat &m, float *out, hipStream_t st);

// Plan a GEMV over segments sharing one K: picks the kernel and fills lpr,
// rows_per_wg, wg_begin, ntiles, total_wgs.  False if K is not a multiple of 64.
bool plan_gemv(GemvArgs &a);
bool gemv_q_supported(const GemvArgs &a);
void plan_gemv_q(GemvArgs &a);
hipError_t launch_gemv_q(const GemvArgs &a, hipStream_t st);

}  // namespace oi
