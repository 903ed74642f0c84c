// oi_kernels.h -- descriptors shared by the host code and the gfx950 kernels,
// and the host-side launchers of every kernel in kernels.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oi {

// ggml type ids (reference ggml/gguf.odin:27-42)
enum : int32_t { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q4_K = 12,
                 T_Q6_K = 14 };

// A weight matrix resident in HBM, in the GEMV layout.  Every row is cut into
// U = cols/64 "units" of 64 consecutive weights; a unit is the work of one
// lane.  The bytes of a unit are split into 16-byte pieces, and piece k of
// every (row, unit) is stored in plane k in (row, unit) order, so the 64
// lanes of a wave reading piece k of 64 consecutive units read one
// contiguous 1 KB.  The byte count equals the GGUF one.  Per type:
//   Q4_K  plane 0: qs[32p .. 32p+15] and plane 1: qs[32p+16 .. 32p+31] of
//         super-block u/4, group pair p = u%4;  s: a 16-byte header per
//         (row, sb): f16 d, f16 dmin, then the eight 6-bit scales and mins
//         regrouped as four 24-bit fields, field p = sc(2p) | m(2p) << 6 |
//         sc(2p+1) << 12 | m(2p+1) << 18 at bits 24p.. of the 96-bit tail
//         (the GGUF packing, ggml/quant.odin:64-73, spread one group pair's
//         values over three bytes; the values are unchanged).
//   Q6_K  unit u = super-block u/4, half h = (u/2)%2, columns l0 = 16(u%2):
//         plane 0: ql[64h+l0 ..+15], plane 1: ql[64h+32+l0 ..+15],
//         plane 2: qh[32h+l0 ..+15];  s: 16 int8 scales per (row, sb);
//         d: f16 d per (row, sb).
//   Q8_0  unit u = blocks 2u, 2u+1: plane c = int8 values 16c .. 16c+15 of
//         the unit;  d: f16 d per (row, block).
//   F32/F16  q: the values, row-major.
//   Q4_0/Q4_1/Q5_0/Q5_1  q: the GGUF blocks, row-major (decoded by the generic
//         GEMV; the reference's CPU path reads them, ggml/quant.odin:98-162).
struct DMat {
    int32_t type;
    int32_t rows;
    int32_t cols;
    int32_t pad;
    const uint8_t *q;   // plane 0
    int64_t plane;      // bytes from one plane to the next (rows * U * 16)
    const uint8_t *s;
    const uint16_t *d;
};

enum GemvMode : int32_t {
    GEMV_STORE = 0,   // y[r] = W x
    GEMV_ADD = 1,     // y[r] += W x            (residual epilogue; y[r] += sigmoid(ygate[0]) W x with ygate)
    GEMV_SWIGLU = 2,  // y[r] = silu(Wg x) * (Wu x); seg[0]=gate, seg[1]=up
    GEMV_ARGMAX = 3   // y[r] = W x, then greedy argmax over all rows
};

struct GemvSeg {
    DMat m;
    float *y;
    int32_t wg_begin;  // first workgroup of this segment
    int32_t ntiles;    // row tiles of this segment (gemv_q_kernel)
};

constexpr int GEMV_MAX_SEG = 4;

struct GemvArgs {
    GemvSeg seg[GEMV_MAX_SEG];
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
    int32_t wg_base;       // gemv_q_kernel: workgroup index of blockIdx.x 0 (one launch per weight type)
    int32_t tiles_per_wg;  // gemv_q_kernel: most tiles any workgroup takes (sizes its output buffer)
    // routed experts (launch_gemv_q_moe): moe_ids[moe_k] are the experts chosen on
    // the device (of moe_n).  Rows mode: virtual row v is row v % moe_blk of expert
    // ids[v / moe_blk] (seg m.rows = moe_k * moe_blk).  Columns mode: the row is the
    // concatenation over k of row r of expert ids[k] (moe_blk units each, K =
    // moe_k * 64 * moe_blk), each expert's part weighted by moe_w[k].
    const int32_t *moe_ids;
    const float *moe_w;
    int32_t moe_k, moe_n, moe_blk;
    // rows mode with moe_logits set: every workgroup routes itself from the
    // router logits (softmax, top moe_k, weights renormalized if moe_norm) and
    // workgroup 0 writes the ids and weights to moe_ids_out / moe_w_out
    const float *moe_logits;
    int32_t *moe_ids_out;
    float *moe_w_out;
    int32_t moe_norm;
    // a shared expert stored as expert moe_n of the stacked matrices (moe_nblk =
    // moe_n + 1 blocks): routing picks moe_sel (< moe_k) experts and adds
    // expert moe_n as part moe_sel with weight sigmoid(moe_sgate[0]); 0 / null:
    // no shared expert (moe_sel = moe_k, moe_nblk = moe_n)
    int32_t moe_sel, moe_nblk;
    const float *moe_sgate;
    // rows mode, router fused (MOE_ROWS_R): the router matrix (moe_n rows of K,
    // the experts' weight type); every workgroup computes the router logits
    // from its RMSNormed x before routing (no router launch, no moe_logits)
    DMat moe_router;
    // GEMV_ADD: if set, the product is scaled by sigmoid(ygate[0]) before the add
    // (the shared expert's gate of a Qwen3-Next-style MoE layer)
    const float *ygate;
    // gemv_q_kernel only.  gss set: the prologue finishes the gated RMSNorm of
    // a DeltaNet layer's output per head of 128: x holds o silu(z), gss
    // [heads][4] partial sums of o^2, x = norm_w[j] (inv_h x) with inv_h =
    // 1 / sqrt(sum / 128 + eps) (norm_w [128]).  conv_w set (GEMV_STORE):
    // segment 0's rows are the channels of the DeltaNet conv, stored as
    // silu(conv) with conv_state [rows][conv_kernel - 1] slid (the in_qkv
    // projection of the token step).
    const float *gss;
    const float *conv_w;
    float *conv_state;
    int32_t conv_kernel;
};

// Device state of the token loop (int32 x 8):
//   [0] token  [1] pos  [2] step  [3] capacity of tokens_out
//   [4] argmax pending  [5] number of argmax partials
enum { ST_TOKEN = 0, ST_POS = 1, ST_STEP = 2, ST_CAP = 3, ST_PENDING = 4, ST_NPART = 5, ST_WORDS = 8 };

// Sampler state in device memory (sampler/sampler.odin:16-29 without the
// grammar): updated by every draw (rng) and, with `record`, by every pick
// (record_token, window SAMPLE_WINDOW).
constexpr int SAMPLE_WINDOW = 64;
struct SampleState {
    float temperature, topp, penalty;
    int32_t record;
    uint64_t rng;
    int32_t n_last;
    int32_t last[SAMPLE_WINDOW];  // oldest first
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
    float *part;               // [n_kv_heads][max_splits][group][head_dim + 2]
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
// Splits of the decode attention at this shape (the grid's first dimension,
// the partial buffer's split count); *chunk: positions per split, 0 when the
// kernel sizes its splits from pos at run time.  fixed: splits of 64 on the
// lane-per-position kernel at every head_dim; otherwise head_dim 128 takes
// the matrix-core kernel.
int attn_plan(int head_dim, int n_kv_heads, int seq_len, int *chunk, bool fixed);
hipError_t launch_dequant(const DMat &m, float *out, hipStream_t st);
// One draw of the sampler (sample.hip) from logits[0, n); p: n floats of
// scratch, work: sample_work_bytes() of scratch.  mode: sample_mode() of the
// state's temperature and topp (the launch sequence depends on it).  With
// `state` set the pick advances the token loop (token, pos, step, pending as
// the greedy reduction does) and is stored at tokens_out[step]; `pick`, if
// set, receives it too.
enum { SAMPLE_GREEDY = 0, SAMPLE_MULT = 1, SAMPLE_TOPP = 2 };
int sample_mode(float temperature, float topp, int n);
size_t sample_work_bytes();
hipError_t launch_sample(const float *logits, float *p, int n, SampleState *ss, int mode, void *work, int32_t *state,
                         int32_t *tokens_out, int32_t *pick, hipStream_t st);
int sample_max_vocab();  // largest n launch_sample takes
// f16 head-major cache [n_kv][seq_len][hd], positions [0, n) <-> f32 rows
// [n][n_kv * hd]; to_f32: cache -> rows, else rows -> cache (RNE)
hipError_t launch_kv_convert(bool to_f32, uint16_t *cache, float *rows, int n, int n_kv, int seq_len, int hd,
                             hipStream_t st);

// Plan a GEMV over segments sharing one K: picks the kernel and fills lpr,
// rows_per_wg, wg_begin, ntiles, total_wgs.  False if K is not a multiple of 64.
bool plan_gemv(GemvArgs &a);
bool gemv_q_supported(const GemvArgs &a);
void plan_gemv_q(GemvArgs &a);
hipError_t launch_gemv_q(const GemvArgs &a, hipStream_t st);
// routed-expert GEMV (moe = MOE_ROWS: SwiGLU over the chosen experts' gate/up
// rows; MOE_ROWS_R: the same with the router fused into the launch, from
// GemvArgs::moe_router; MOE_COLS: down over the chosen experts' rows,
// weighted); a planned by plan_gemv_q; false from gemv_q_moe_supported means
// the generic kernels
enum { MOE_ROWS = 1, MOE_COLS = 2, MOE_ROWS_R = 3 };
bool gemv_q_moe_supported(const GemvArgs &a, int moe);
hipError_t launch_gemv_q_moe(const GemvArgs &a, int moe, hipStream_t st);

// gemm.hip: batched projection c[t][r] = sum_k f16(deq(W))[r][k] x[t][k]
bool gemm_supported(const DMat &m);
// K slices for n tokens when part_bytes of partial products fit (1 = none)
int gemm_split(const DMat &m, int32_t n, size_t part_bytes);
// part: room for the K slices' partial products (split * n * rows floats);
// null or small: fewer slices
hipError_t launch_gemm(const DMat &m, const uint16_t *x, int32_t n, float *c, float *part, size_t part_bytes,
                       hipStream_t st);

// gemm.hip, for consumers that sum the K slices themselves: the partial
// products go to part ([split][n][rows]; with split 1 the product itself)
// gemm.hip: gate and up in one pass with the SwiGLU epilogue, h [n][rows] f16
bool gemm_swiglu_supported(const DMat &gate, const DMat &up, int32_t n);
hipError_t launch_gemm_swiglu(const DMat &gate, const DMat &up, const uint16_t *x, int32_t n, uint16_t *h,
                              hipStream_t st);
hipError_t launch_gemm_parts(const DMat &m, const uint16_t *x, int32_t n, float *part, size_t part_bytes, int *split,
                             hipStream_t st);
// launch_gemm_parts of up to 4 projections of the same x (same type and K) in
// one launch: matrix i's partial products to part[i], its slice count to split[i]
hipError_t launch_gemm_parts_multi(const DMat *const *m, float *const *part, const size_t *part_bytes, int nseg,
                                   const uint16_t *x, int32_t n, int *split, hipStream_t st);

// prefill.hip: the per-token operations of batched prefill
struct PfQkvArgs {
    const float *q, *k, *v;     // projections' partial products [split][T][rows]
    int32_t qs, ks, vs;         // their K slices
    const float *q_norm, *k_norm;
    float eps;
    const float2 *rope_cs;      // [seq_len][head_dim / 2]
    uint16_t *kc, *vc;          // this layer's cache
    float *qout;                // [T][n_heads * head_dim]
    int32_t T, pos0, seq_len, n_heads, n_kv_heads;
};
hipError_t launch_pf_qkv(const PfQkvArgs &a, int head_dim, hipStream_t st);
// gate: null, or [T][n_heads * head_dim] f32, the output multiplied by its
// sigmoid before rounding (the Qwen3.5 attention's output gate)
// ws: optional scratch for the key-split form of short chunks (head_dim 256:
// [splits][T][n_heads][head_dim + 2] floats, splits <= 16); unused if too small
hipError_t launch_pf_attn(const float *q, const uint16_t *kc, const uint16_t *vc, uint16_t *out, int T, int pos0,
                          int seq_len, int n_heads, int n_kv_heads, int head_dim, hipStream_t st,
                          const float *gate = nullptr, float *ws = nullptr, size_t ws_bytes = 0);
hipError_t launch_pf_add(float *x, const float *part, int split, int64_t total, hipStream_t st);
// x += partial-product sums (part may be null), then out = f16(rmsnorm(x) * w); dim <= 16384
// out32: null, or [T][dim] f32 that receives the norm's f32 result as well
// myd (with part null): x += sum_s mw[t kp + s] myd[(t kp + s) dim ..], a routed FFN's pair rows
hipError_t launch_pf_addnorm16(float *x, const float *part, int split, const float *w, float eps, int dim, int T,
                               uint16_t *out, hipStream_t st, float *out32 = nullptr, const float *mw = nullptr,
                               const float *myd = nullptr, int kp = 0, void *xq = nullptr, float *xq_sum = nullptr,
                               float *xq_scale = nullptr);
hipError_t launch_pf_swiglu16(const float *g, int gs, const float *u, int us, int64_t total, uint16_t *out,
                              hipStream_t st);
// prefill_hybrid.hip: batched prefill of the Qwen3.5 hybrid layers
struct PfQ35Args {
    const float *q, *k, *v;        // projections' partial products [split][T][rows]; q rows [n_heads][q | gate]
    int32_t qs, ks, vs;            // their K slices
    const float *q_norm, *k_norm;  // [head_dim]
    const float *inv_freq;         // [rotary_dim / 2]
    float eps;
    int32_t rotary_dim;
    uint16_t *kc, *vc;             // this layer's cache
    float *qout, *gate;            // [T][n_heads * head_dim]: rotated q, gate
    int32_t T, pos0, seq_len, n_heads, n_kv_heads;
};
hipError_t launch_pf_q35_qkv(const PfQ35Args &a, int head_dim, hipStream_t st);
struct PfDnArgs {
    const float *qkv, *z, *b, *a;  // in_qkv / in_z / in_b / in_a partial products [split][T][rows]
    int32_t qkvs, zs, bs, as;      // their K slices
    const float *conv_w;           // [conv_dim][kernel]
    const float *a_decay, *dt_bias;  // [n_vh]
    const float *norm_w;           // [hv]
    float eps;
    float *conv_state;             // [conv_dim][kernel - 1], oldest first
    float *state;                  // [n_vh][hk][hv]
    float *conv_out;               // scratch [T][conv_dim]
    float *qk;                     // scratch [T][2 n_kh hk]: normalized q (scaled), k
    float *gates;                  // scratch [T][3 n_vh]: beta, decay, log decay
    float *o;                      // scratch [T][n_vh hv]: delta-rule outputs
    uint16_t *out16;               // [T][n_vh hv]: gated-normed, f16 (the output projection's input)
    float *out32;                  // or, when set, the same in f32
    int32_t T, n_kh, n_vh, hk, hv, kernel;
    int32_t chunk;                 // 0: the delta rule token by token; 16 / 32 / 64: its chunked form
    float *dc;                     // chunk 64: scratch of pf_dc_scratch_floats(n_vh, T) floats
};
bool pf_dn_supported(int hk, int hv, int kernel);
size_t pf_dc_scratch_floats(int n_vh, int T);
hipError_t launch_pf_deltanet(const PfDnArgs &a, hipStream_t st);
// kernels.hip: the routed-expert FFN of a prefill chunk.  Pairs p = t * kp + s
// (token t, slot s of its kp chosen experts) are grouped by expert; a
// multi-token GEMV reads each chosen expert's rows once for all of its pairs.
struct MtGemvArgs {
    DMat m, m2;                    // stacked matrices [n_exp * rows][K] (m2: up of a SwiGLU pair)
    int32_t swiglu, K, rows, xdiv, tile_rows, dense_n, pair_slice, tiles;
    const float *x;                // activation rows [*][K]: pair p reads row p / xdiv
    float *y;                      // output rows [pairs][rows]
    const int32_t *list, *off, *cnt;  // pairs by expert: list[off[e] .. off[e] + cnt[e])
    const int32_t *items, *nitems; // work items [2]: expert, pair slice << 16 | row tile; their count
    // items of MT_MFMA_FEW pairs only: a SwiGLU pair writes gate rows to y and
    // up rows to y2 (set by the launcher: blocks from mat_items on take m2);
    // x2 set: the x rows are silu(x) * x2 (the SwiGLU of such gate and up rows)
    float *y2;
    const float *x2;
    int32_t mat_items;
    // set (with x2 unset): the x rows already quantized (launch_pf_addnorm16's
    // xq) -- planes in the int8 kernel's operand order, group sums, scales per row
    const void *xq;
    const float *xq_sum, *xq_scale;
};
// dense_n > 0: one "expert" (e = 0) holding pairs 0 .. dense_n-1, no lists (a
// plain multi-token GEMV); item it = slice * tiles + row tile, max_items =
// tiles * ceil(dense_n / pair_slice)
constexpr int MT_PAIR_SLICE = 32;  // pairs per work item of the routed-expert prefill
bool mt_gemv_supported(const DMat &m, int32_t K);
int mt_gemv_tile_rows(int32_t K, int32_t rows);
hipError_t launch_mt_gemv(const MtGemvArgs &a, int max_items, hipStream_t st);
// the same on the matrix cores for Q4_K / Q6_K / Q8_0 matrices with K % 256 ==
// 0 and rows % 16 == 0: items of 16 pairs x 64 rows; Q4_K on f16 MFMA with the
// weights exact (raw quants, scales per 32 in f32, x split hi + lo) unless
// f32_only, the others (and f32_only) on f32 MFMA of the decoded weights
constexpr int MT_MFMA_PAIRS = 16, MT_MFMA_ROWS = 64;
// items of at most MT_MFMA_FEW pairs (pair_slice == MT_MFMA_FEW, tiles == 1: an
// item covers every row tile): Q4_K only, the x rows staged once for the whole
// K (K <= ~5600), the weights streaming through all row tiles with the next
// step in flight; for chunks whose pairs spread thinly over the experts.  A
// SwiGLU pair leaves gate in y and up in y2; the down launch applies the
// SwiGLU to its x rows (x2 = up)
constexpr int MT_MFMA_FEW = 4;
// the same items (<= MT_MFMA_FEW pairs, every row tile) on the decode GEMV's
// int8 dot4 arithmetic (gemv.hip): Q4_K with K / 64 in {8, 16, 32, 64}
bool mt_dot4_supported(const DMat &m, int32_t K, int32_t rows);
hipError_t launch_mt_dot4(const MtGemvArgs &a, int max_items, hipStream_t st);
bool mt_q4i8_supported(const DMat &m, int32_t K, int32_t rows);
hipError_t launch_mt_q4i8(const MtGemvArgs &a, int max_items, hipStream_t st);
bool mt_mfma_supported(const DMat &m, int32_t K, int32_t rows);
hipError_t launch_mt_mfma(const MtGemvArgs &a, int max_items, hipStream_t st, bool f32_only = false);
struct PfMoeArgs {
    const float *logits;           // [T][n_experts]
    DMat sh_inp;                   // the shared expert's gate row (when kp > top_k)
    const float *xn;               // [T][dim] the normed x (f32)
    int32_t *ids;                  // [T][kp] expert (n_experts = the merged shared expert)
    float *w;                      // [T][kp]
    int32_t *list, *off, *cnt, *fill;  // [T kp], [n_exp] x 3
    int32_t *items_gu, *items_dn, *nitems;  // [2 * tiles * (n_exp + T kp / pair_slice)], [2]
    const float *yd;               // [T kp][dim] down outputs per pair
    float *out;                    // [T][dim] the weighted sums
    int32_t T, n_experts, top_k, kp, norm_topk, tiles_gu, tiles_dn, dim, pair_slice;
};
hipError_t launch_pf_moe_route(const PfMoeArgs &a, hipStream_t st);
hipError_t launch_pf_moe_combine(const PfMoeArgs &a, hipStream_t st);
hipError_t launch_pf_router_items(int T, int tiles, int32_t *list, int32_t *items, int32_t *hdr, hipStream_t st);
// deltanet.hip: the gated DeltaNet token step (between the input and output
// projections of a Qwen3.5 linear-attention layer)
struct DnArgs {
    const float *qkv;              // in_qkv projection [conv_dim], conv_dim = 2 n_kh hk + n_vh hv
    const float *z, *b, *a;        // in_z [n_vh hv], in_b [n_vh], in_a [n_vh]
    const float *conv_w;           // [conv_dim][kernel]
    const float *a_decay, *dt_bias;  // [n_vh] (a_decay = ssm_a = -exp(A_log))
    const float *norm_w;           // [hv]
    float eps;
    float *conv_state;             // [conv_dim][kernel - 1], oldest first
    float *state;                  // [n_vh][hk][hv]
    float *conv_out;               // scratch [conv_dim]
    float *out;                    // [n_vh hv]
    int32_t n_kh, n_vh, hk, hv, kernel;
    // 1: the delta rule alone over (value head, 32 columns) workgroups, conv_out
    // already holding the conv (the in_qkv GEMV's epilogue); out gets
    // o silu(z) and ssq [n_vh][hv / 32] the sums of o^2 per workgroup (the
    // output GEMV's prologue finishes the gated norm)
    int32_t cols;
    float *ssq;
};
hipError_t launch_deltanet(const DnArgs &a, hipStream_t st);

// qwen35_attn.hip: attention of a Qwen3.5 full-attention layer for one token
struct Q35Args {
    const float *qproj;            // [n_heads][2][head_dim]: q then gate per head
    const float *k, *v;            // [n_kv_heads * head_dim]
    const float *q_norm, *k_norm;  // [head_dim]
    const float *inv_freq;         // [rotary_dim / 2]
    float eps;
    int32_t rotary_dim, pos, seq_len, n_heads, n_kv_heads, max_splits;
    uint16_t *kc, *vc;             // [n_kv_heads][seq_len][head_dim] f16
    float *qbuf;                   // scratch [n_heads * head_dim]
    float *part;                   // scratch [n_heads][max_splits][head_dim + 2]
    float *out;                    // [n_heads * head_dim]
    const int32_t *state;          // if set, pos = state[ST_POS] (the token loop's device state) instead of pos
};
int q35_max_splits(int seq_len);
hipError_t launch_q35_attn(const Q35Args &a, int head_dim, hipStream_t st);

// kernels.hip: router top-k and selected-expert SwiGLU FFN for one token
constexpr int MOE_MAX_EXPERTS = 1024, MOE_MAX_K = 32;
struct MoeArgs {
    DMat gate, up, down;       // stacked expert matrices
    const float *x;            // [dim]
    const float *logits;       // router output [n_experts]
    int32_t *ids;              // [top_k]
    float *w;                  // [top_k]
    float *h;                  // [top_k][inter]
    float *y;                  // [dim]
    int32_t n_experts, top_k, dim, inter, norm_topk;
};
// router: a planned GEMV writing `logits`; gu / dn: planned routed-expert
// GEMVs (launch_gemv_q_moe) for gate/up and down, or null for the generic kernels
hipError_t launch_moe(const MoeArgs &a, const GemvArgs &router, const GemvArgs *gu, const GemvArgs *dn,
                      hipStream_t st);

// engine.cpp: records a failure for oi_last_error(); returns code
int set_error(int code, const char *msg);

// kernels.hip: x[t] = dequant(emb[tokens[t]]) for n tokens
hipError_t launch_embed_rows(const DMat &emb, const int32_t *tokens, int n, float *x, hipStream_t st);

}  // namespace oi
