/*
 * oi.h -- C ABI of the MI355X (gfx950) HIP library that replaces the
 * arithmetic of odin-infer's token loop.
 *
 * The Odin host keeps the reference's Engine API (infer/engine.odin:7-60) and
 * binds these entry points with `foreign import` (odin-infer_amd/odin/
 * engine.odin).  Plain C types only: no torch, no HIP types in signatures.
 * Streams are passed as `void*` (a hipStream_t, NULL = the library's stream).
 *
 * Errors: functions returning int return 0 on success and a negative code on
 * failure; functions returning a pointer return NULL.  Either way the message
 * is available from oi_last_error() (thread-local).
 */
#ifndef OI_H
#define OI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor type ids (reference: ggml/gguf.odin:27-42). */
enum {
    OI_TYPE_F32 = 0, OI_TYPE_F16 = 1, OI_TYPE_Q4_0 = 2, OI_TYPE_Q4_1 = 3,
    OI_TYPE_Q5_0 = 6, OI_TYPE_Q5_1 = 7, OI_TYPE_Q8_0 = 8, OI_TYPE_Q8_1 = 9,
    OI_TYPE_Q2_K = 10, OI_TYPE_Q3_K = 11, OI_TYPE_Q4_K = 12, OI_TYPE_Q5_K = 13,
    OI_TYPE_Q6_K = 14, OI_TYPE_Q8_K = 15
};

/* Error codes. */
enum {
    OI_OK = 0,
    OI_E_ARG = -1,        /* bad argument (null pointer, bad size, bad type) */
    OI_E_IO = -2,         /* file could not be opened or mapped */
    OI_E_FORMAT = -3,     /* not a GGUF v2/v3 file, truncated or corrupt */
    OI_E_MODEL = -4,      /* missing metadata key / tensor, wrong tensor type */
    OI_E_UNSUPPORTED = -5,/* quant type not supported on this path */
    OI_E_RANGE = -6,      /* token or pos out of range */
    OI_E_DEVICE = -7,     /* no usable gfx950 device, or a HIP call failed */
    OI_E_NOMEM = -8       /* device or pinned host allocation failed */
};

/* Engine_Opts (reference: infer/engine.odin:7-11).  `use_hip` replaces
 * `use_metal`; there is no CPU fallback in this library. */
typedef struct oi_opts {
    int32_t max_ctx;     /* KV capacity cap; seq_len = min(context_length, max_ctx) */
    int32_t use_hip;     /* must be 1 */
    int32_t num_threads; /* accepted for source compatibility; unused on the GPU */
    int32_t device;      /* HIP device ordinal */
} oi_opts;

/* Config (reference: infer/model.odin:12-24), same field order. */
typedef struct oi_config {
    int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size;
    int64_t seq_len, max_seq, head_dim;
    float rope_freq, rms_eps;
} oi_config;

typedef struct oi_engine oi_engine;
typedef struct oi_weights oi_weights;

/* ------------------------------------------------------------ engine API --- */

/* engine_load (infer/engine.odin:18-34 -> infer/model.odin:216-242):
 * parse the GGUF at `path`, check the tensors the loader of its architecture
 * requires, upload weights to HBM and allocate the f16 KV cache
 * [layer][kv_head][seq_len][head_dim].  Architectures (general.architecture):
 * "qwen3" (the dense loader, infer/model.odin:99-179), "qwen35" (the hybrid
 * loader, qwen3_5/model.odin:225-364: full-attention layers with a KV cache,
 * gated DeltaNet layers with conv and recurrent states) and, with no reference
 * loader, routed-expert FFNs ("qwen3moe", and "qwen35" files with
 * expert_count): ffn_gate_inp + ffn_{gate,up,down}_exps, optionally a shared
 * expert (ffn_*_shexp).  Config: for routed experts hidden_dim is the expert
 * inner size; for "qwen35" n_heads / n_kv_heads / head_dim are the
 * full-attention layers'.  Returns 0 and *out on success. */
int oi_engine_load(const char *path, const oi_opts *opts, oi_engine **out);

/* engine_destroy (infer/engine.odin:36-43). NULL is allowed. */
void oi_engine_destroy(oi_engine *e);

/* engine_forward (infer/engine.odin:45-52 -> infer/forward.odin:17-146):
 * consume `token` at `pos`, write K/V[pos], return vocab_size logits that
 * predict pos+1.  The pointer is engine-owned pinned host memory, valid until
 * the next call on this engine.  NULL on error (token/pos out of range:
 * the reference prints and exits, infer/forward.odin:22-29; the Odin binding does
 * the same). */
const float *oi_engine_forward(oi_engine *e, int32_t token, int32_t pos);

/* engine_forward_batch (qwen3_5/engine.odin:61-93 -> qwen3_5/metal.odin:1472-1654
 * forward_gpu_batch): consume tokens[0..n) at positions pos0 .. pos0+n-1 and
 * return the logits of the last one (engine-owned pinned host memory, as
 * oi_engine_forward).  Chunks of up to 512 tokens, cut to a multiple of 8, run
 * batched: the seven projections of each layer on the matrix cores with f16
 * operands and f32 accumulation (the reference's MMQ), the per-token operations
 * (norms, RoPE, cache store, causal attention, SwiGLU, residuals) in f32; the
 * trailing 1-7 tokens go through oi_engine_forward's path.  A model whose
 * projections the batched kernels cannot take (type other than Q4_K / Q6_K /
 * Q8_0, or a row length not a multiple of 256) runs every token through that
 * path, as the reference's non-Metal fallback (qwen3_5/engine.odin:86-91).  NULL on
 * error: n <= 0, positions past seq_len, or a token out of range. */
const float *oi_engine_prefill(oi_engine *e, const int32_t *tokens, int32_t n, int32_t pos0);

/* engine_verify_batch (qwen3_5/engine.odin:166-174: forward_gpu_batch, then
 * metal_verify_batch_logits, qwen3_5/metal.odin:1707-1747): consume
 * tokens[0..n) at positions pos0 .. pos0+n-1 exactly as oi_engine_prefill
 * does (same chunking, same state afterwards) and return the logits of every
 * position: n rows of vocab_size floats, row i predicting position pos0+i+1
 * (engine-owned pinned host memory, valid until the next call of this
 * procedure).  Each row is the final RMSNorm and classifier of that token's
 * hidden state in f32 (the decode path's GEMV, as the reference's per-row
 * enc_gemv).  NULL on the errors of oi_engine_prefill, or OI_E_NOMEM when the
 * n x vocab buffer cannot be allocated. */
const float *oi_engine_verify_batch(oi_engine *e, const int32_t *tokens, int32_t n, int32_t pos0);

/* engine_batch_max (qwen3_5/engine.odin:96-102): the most tokens one batched
 * chunk of oi_engine_prefill / oi_engine_verify_batch takes (qwen3_5/metal.odin:22
 * MAX_BATCH_T). */
int32_t oi_engine_batch_max(void);

/* engine_config (infer/engine.odin:54-56). */
int oi_engine_config(const oi_engine *e, oi_config *out);

/* Config of the qwen3_5 package (qwen3_5/model.odin:20-45), its fields in that
 * order without the layer_types slice (oi_engine_layer_types gives it).  For
 * a hybrid ("qwen35") file: the partial RoPE width and fraction, the DeltaNet
 * dimensions and the full-attention interval of the file; for the other
 * layouts every layer is full attention over the whole head (rotary_dim =
 * head_dim, partial_rotary = 1, lin_* = 0, full_attn_interval = 1).  n_full and
 * n_linear count the layers of each kind. */
typedef struct oi_qwen35_config {
    int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size, seq_len, max_seq;
    float rms_eps, rope_theta, partial_rotary;
    int64_t rotary_dim, lin_n_k_heads, lin_n_v_heads, lin_head_k_dim, lin_head_v_dim, lin_conv_kernel;
    int64_t full_attn_interval, n_full, n_linear;
} oi_qwen35_config;
int oi_engine_config_qwen35(const oi_engine *e, oi_qwen35_config *out);

/* Config.layer_types (qwen3_5/model.odin:288-300): out[l] = 0 for a
 * full-attention layer, 1 for a gated-DeltaNet layer (the order of the
 * reference's Layer_Type enum); n must equal n_layers (OI_E_ARG otherwise). */
int oi_engine_layer_types(const oi_engine *e, int32_t *out, int32_t n);

/* Message of the last failure on this thread. */
const char *oi_last_error(void);

/* ------------------------------------------------- token loop (device side) --- */

/* Greedy decode of `n_steps` tokens with the whole loop on the device: step i
 * consumes the current token at pos+i and picks the next one by argmax with
 * ties to the lowest id (sampler/sampler.odin:79-89), as the caller loop
 * serve_harness/serve.odin:514-525 does with greedy sampling.  Writes the
 * n_steps picked ids to out_tokens (host memory).  No logits cross PCIe. */
int oi_engine_decode_greedy(oi_engine *e, int32_t token, int32_t pos, int32_t n_steps,
                            int32_t *out_tokens);

/* Sampler (sampler/sampler.odin:16-29 build_sampler / enable_repeat_penalty,
 * without the JSON grammar mask).  The state is the caller's and is written
 * back after each call: rng_state advanced once per draw (xorshift64*,
 * random_u32 :68-73), and, with record set and repeat_penalty != 1, last[]
 * extended by each pick and trimmed to the newest 64 (record_token :50-56). */
typedef struct oi_sampler {
    float temperature;    /* 0: first maximum (sample_argmax :79-89) */
    float topp;           /* in (0, 1): sample_topp (:106-139); otherwise sample_mult (:91-100) */
    float repeat_penalty; /* 1: off; logits of distinct recent tokens divided (> 0) or multiplied */
    int32_t record;       /* 1: append each pick to last[] as record_token does */
    uint64_t rng_state;
    int32_t n_last;       /* tokens in last[], oldest first (<= 64) */
    int32_t last[64];
} oi_sampler;

/* Decode loop with sampling on the device (the caller loop of
 * serve_harness/serve.odin:514-525 with sampler.sample): step i consumes the
 * current token at pos+i and draws the next as sample() does -- penalty,
 * temperature, softmax, one coin, multinomial or top-p -- on the device.
 * Running probabilities are summed exactly (64-bit fixed point, 2^-40), so a
 * pick differs from the reference's sequential f32 sums only where the coin
 * lies within their rounding of a boundary.  Writes the n_steps picks to
 * out_tokens and the advanced sampler state to *s. */
int oi_engine_decode_sample(oi_engine *e, int32_t token, int32_t pos, int32_t n_steps, oi_sampler *s,
                            int32_t *out_tokens);

/* One draw of the same sampler on n host logits (synchronous; the logits are
 * not modified).  *s is advanced as above. */
int oi_sample(const float *logits, int32_t n, oi_sampler *s, int32_t *out_token);

/* Overwrite positions [pos0, pos0+npos) of layers [layer0, layer0+nlayers) of
 * the f16 KV cache with host data laid out [layer][kv_head][npos][head_dim]
 * (binary16 bits).  Used to pre-fill long contexts for measurement. */
int oi_engine_kv_fill(oi_engine *e, int32_t layer0, int32_t nlayers, int32_t pos0, int32_t npos,
                      const uint16_t *k_f16, const uint16_t *v_f16);

/* engine_reset_state (qwen3_5/engine.odin:108-132): zero every
 * position-evolving state -- the KV cache of the attention layers, the conv
 * and recurrent states of the DeltaNet layers -- so a new prompt can start at
 * position 0 (the DeltaNet recurrence cannot be rewound). */
int oi_engine_reset_state(oi_engine *e);

/* ------------------------------------------------- state persistence ---
 * The position-evolving state: the K/V cache of the attention layers and the
 * conv / recurrent states of the DeltaNet layers, in layer order. */

/* engine_save_kv (qwen3_5/kv_persist.odin:365-372, metal_save_kv
 * qwen3_5/metal.odin:780-862): write the .oikv v1 file -- a 60-byte
 * little-endian header (magic 0x4F494B56, version 1, arch, FNV-1a 64
 * fingerprint of dim, n_layers, n_heads, n_kv_heads, head_dim, the four
 * DeltaNet head counts / dims, conv kernel and vocab_size; n_valid_pos,
 * seq_len, n_full, n_linear, kv_dim, conv_dim, conv kernel, n_v_heads,
 * head_k_dim, head_v_dim), then per attention layer K and V as f32
 * [n_valid_pos][kv_dim], then every conv state and every recurrent state
 * (f32), then the IEEE CRC-32 of all of it.  arch is 2 for the qwen35 layout
 * (the reference's value); the qwen3 and qwen3moe layouts, which the
 * reference does not persist, write 1 and 3.  OI_E_RANGE if n_valid_pos is
 * outside [0, seq_len]; OI_E_IO on a file error. */
int oi_engine_save_kv(oi_engine *e, const char *path, int32_t n_valid_pos);

/* engine_load_kv (qwen3_5/kv_persist.odin:374-381, metal_load_kv
 * qwen3_5/metal.odin:864-962): check magic, version, arch, fingerprint, seq_len,
 * n_valid_pos <= seq_len, the layer dims, the file size and the CRC -- all
 * before any state changes -- then zero the K/V cache, read the file's
 * positions (f32 -> f16, round to nearest even) and the DeltaNet states.
 * *n_valid_pos receives the restored length (the next position to fill).
 * OI_E_IO (cannot open) or OI_E_FORMAT with the reference's message. */
int oi_engine_load_kv(oi_engine *e, const char *path, int32_t *n_valid_pos);

/* engine_save_full_state / engine_restore_full_state (qwen3_5/engine.odin:
 * 139-151, qwen3_5/metal.odin:1655-1676): byte copies of the device state in its own
 * layout -- kv_k and kv_v f16 [n_attention_layers][n_kv_heads][seq_len]
 * [head_dim], conv f32 [n_linear][conv_dim][kernel-1], rec f32 [n_linear]
 * [n_v_heads][head_k_dim][head_v_dim].  The buffers are the caller's, in host
 * or device memory (a prefix snapshot can stay in HBM); sizes in bytes from
 * oi_engine_state_sizes (a zero size takes a null pointer). */
int oi_engine_state_sizes(oi_engine *e, int64_t sizes[4]);
int oi_engine_save_full_state(oi_engine *e, void *kv_k, void *kv_v, void *conv, void *rec);
int oi_engine_restore_full_state(oi_engine *e, const void *kv_k, const void *kv_v, const void *conv,
                                 const void *rec);

/* engine_save_spec_state / engine_restore_spec_state (qwen3_5/engine.odin:
 * 153-165, qwen3_5/metal.odin:1678-1700): the conv and recurrent states alone, for a
 * speculative-decoding rollback. */
int oi_engine_save_spec_state(oi_engine *e, void *conv, void *rec);
int oi_engine_restore_spec_state(oi_engine *e, const void *conv, const void *rec);

/* Device pointer to the engine's last logits (vocab_size floats). */
const float *oi_engine_logits_device(oi_engine *e);

/* Stream the engine enqueues on (a hipStream_t). */
void *oi_engine_stream(oi_engine *e);

/* Kernels of the token loop, for oi_engine_time_kernel. */
enum {
    OI_KERNEL_QKV = 0,     /* RMSNorm + fused Q/K/V GEMV */
    OI_KERNEL_ATTN = 1,    /* q/k norm + RoPE + KV store + split-L attention */
    OI_KERNEL_WO = 2,      /* attention output GEMV + residual */
    OI_KERNEL_GATEUP = 3,  /* RMSNorm + gate/up GEMV + SwiGLU */
    OI_KERNEL_DOWN = 4,    /* down GEMV + residual */
    OI_KERNEL_OUTPUT = 5,  /* final RMSNorm + vocab GEMV + greedy argmax */
    OI_KERNEL_TOKEN = 6,   /* one whole token step (the captured graph) */
    OI_KERNEL_ROUTER = 7,  /* MoE router GEMV (+ the shared expert's gate row) */
    OI_KERNEL_LINEAR_IN = 8,   /* Qwen3.5 DeltaNet input projections (qkv, z, b, a) */
    OI_KERNEL_DELTANET = 9,    /* Qwen3.5 gated DeltaNet token step */
    OI_KERNEL_LINEAR_OUT = 10, /* Qwen3.5 DeltaNet output projection + residual */
    OI_KERNEL_SHARED = 11      /* MoE shared expert: gate/up, then down + gated residual */
};

/* Launch one kernel of the token loop `iters` times on the engine's stream,
 * outside the graph, cycling through the layers' weights; report the mean
 * duration per launch measured with HIP events on that stream (*avg_us) and
 * the algorithmic HBM bytes of one launch (*bytes).  The attention kernel is
 * timed at the position of the last forward/decode call.  Leaves the
 * activations and the KV entry at that position modified.
 * OI_KERNEL_TOKEN times `iters` consecutive greedy token steps from the last
 * forward/decode position (moved back so they fit the context); *bytes is
 * then the whole step's algorithmic bytes at the mean position. */
int oi_engine_time_kernel(oi_engine *e, int32_t kernel, int32_t iters, double *avg_us, double *bytes);

/* --------------------------------------------------- kernels (test, bench) --- */

/* dequant_row (ggml/quant.odin:76-175) on the device for `n` elements of
 * `type` stored in `blocks` (host memory, GGUF block layout).  The blocks go
 * through the same device repack and unpack code as the GEMV, and the result
 * is bit-exact with the reference.  Types: F32, F16, Q8_0, Q4_K, Q6_K. */
int oi_dequant(int32_t type, const void *blocks, int64_t n, float *out);

/* Upload a rows x cols matrix of `type` (GGUF layout, host memory) into HBM
 * in the GEMV kernels' layout. */
int oi_weights_upload(int32_t type, const void *host_blocks, int64_t rows, int64_t cols,
                      oi_weights **out);
void oi_weights_free(oi_weights *w);
int64_t oi_weights_bytes(const oi_weights *w); /* GGUF bytes of the matrix */

/* matmul_t (infer/matmul.odin:77-109): y[rows] = W[rows,cols] . x[cols] with
 * x and y in device memory (f32), enqueued on `stream`. */
int oi_gemv_launch(const oi_weights *w, const float *x_dev, float *y_dev, void *stream);

/* Host-memory convenience form of oi_gemv_launch (synchronous). */
int oi_gemv(int32_t type, const void *host_blocks, int64_t rows, int64_t cols, const float *x,
            float *y);

/* Batched projection for prefill: the reference's MMQ kernels
 * (qwen3_5/metal.odin:493-609 gemm_q4k_f32 / gemm_q6k_f32; gemm_harness/
 * gemm_test.odin:97-135, 297-337): c[t][r] = sum_k f16(dequant(W)[r][k]) * x[t][k]
 * for n tokens, f32 accumulation, on the matrix cores.  x_dev: n x cols f16
 * (token-major), c_dev: n x rows f32 (token-major) -- the transposes of the
 * harness's B[K][N] and C[M][N].  Types Q4_K, Q6_K and Q8_0 with cols % 256 == 0
 * (the reference's K % 256 condition, BATCHED_PREFILL.md:205-207).  Enqueued on
 * `stream`.  `workspace` (device memory, may be NULL) holds the partial
 * products when K is split over workgroups; with less than
 * oi_gemm_workspace_bytes(w, n) bytes the split is reduced to what fits (none
 * needs no workspace).  Calls that overlap on one workspace race. */
int64_t oi_gemm_workspace_bytes(const oi_weights *w, int32_t n);
int oi_gemm_launch(const oi_weights *w, const uint16_t *x_dev, int32_t n, float *c_dev, void *workspace,
                   int64_t workspace_bytes, void *stream);

/* Host-memory convenience form of oi_gemm_launch (synchronous). */
int oi_gemm(int32_t type, const void *host_blocks, int64_t rows, int64_t cols, const uint16_t *x, int32_t n,
            float *c);

/* ------------------------------------------- Qwen3.5 linear-attention step --- */

/* Shape of a gated DeltaNet layer (qwen3_5/model.odin: lin_n_k_heads,
 * lin_n_v_heads, lin_head_k_dim, lin_head_v_dim, lin_conv_kernel; rms_eps).
 * conv_dim = 2 * n_k_heads * head_k_dim + n_v_heads * head_v_dim. */
typedef struct {
    int32_t n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel;
    float eps;
} oi_deltanet_dims;

/* One token of forward_linear_layer (qwen3_5/forward.odin:172-219) between the
 * input projections and the output projection: conv1d_step + silu over the
 * in_qkv projection (qwen3_5/ops.odin:97-117), l2norm of q and k per k head with q
 * scaled by 1/sqrt(head_k_dim), beta = sigmoid(b), decay = exp(ssm_a *
 * softplus(a + dt_bias)) (ssm_a already -exp(A_log)), the gated delta rule on
 * each value head's state with k head vh % n_k_heads (qwen3_5/ops.odin:120-153), and
 * the gated RMSNorm rmsnorm(o) * norm_w * silu(z).  Device pointers:
 * qkv [conv_dim], z [n_v_heads*head_v_dim], b and a [n_v_heads], conv_w
 * [conv_dim][conv_kernel], a_decay (ssm_a) and dt_bias [n_v_heads], norm_w
 * [head_v_dim]; conv_state [conv_dim][conv_kernel-1] and rec_state
 * [n_v_heads][head_k_dim][head_v_dim] are updated in place; scratch holds
 * conv_dim floats; out [n_v_heads*head_v_dim].  head_k_dim and head_v_dim
 * must be 128.  Enqueued on `stream`. */
int oi_deltanet_step_launch(const oi_deltanet_dims *d, const float *qkv, const float *z, const float *b,
                            const float *a, const float *conv_w, const float *a_decay, const float *dt_bias,
                            const float *norm_w, float *conv_state, float *rec_state, float *scratch, float *out,
                            void *stream);

/* Host-memory form over a trajectory of n_tokens steps (synchronous): inputs
 * qkv [n][conv_dim], z [n][n_v*head_v_dim], b and a [n][n_v_heads]; states in
 * and out in host memory; out [n][n_v_heads*head_v_dim]. */
int oi_deltanet_steps(const oi_deltanet_dims *d, int32_t n_tokens, const float *qkv, const float *z, const float *b,
                      const float *a, const float *conv_w, const float *a_decay, const float *dt_bias,
                      const float *norm_w, float *conv_state, float *rec_state, float *out);

/* The same trajectory through the batched prefill kernels, all n_tokens at
 * once: the conv over the whole trajectory, l2norm and gates per token, the
 * delta rule token by token in one launch (chunk 0) or in its chunked form
 * over chunks of 16, 32 or 64 tokens (chunk 16 / 32 / 64, the last on the
 * matrix cores; qwen3_5/metal.odin:416-468
 * chunked_delta, which the reference builds but does not dispatch,
 * qwen3_5/metal.odin:1583-1586), the gated norm (qwen3_5/metal.odin:1582-1618, the linear
 * layer of forward_gpu_batch).  Host memory as oi_deltanet_steps; head dims
 * 128, conv kernel 4, n_tokens >= conv_kernel - 1. */
int oi_deltanet_steps_batched(const oi_deltanet_dims *d, int32_t n_tokens, int32_t chunk, const float *qkv,
                              const float *z, const float *b, const float *a, const float *conv_w,
                              const float *a_decay, const float *dt_bias, const float *norm_w, float *conv_state,
                              float *rec_state, float *out);

/* ------------------------------------------ Qwen3.5 full-attention step --- */

/* Shape of a Qwen3.5 full-attention layer (qwen3_5/model.odin: n_heads,
 * n_kv_heads, head_dim, rotary_dim; seq_len of the cache; rms_eps). */
typedef struct {
    int32_t n_heads, n_kv_heads, head_dim, rotary_dim, seq_len;
    float eps;
} oi_qwen35_attn_dims;

/* Device scratch bytes that oi_qwen35_attn_step_launch needs. */
int64_t oi_qwen35_attn_workspace_bytes(const oi_qwen35_attn_dims *d);

/* The attention of forward_full_layer (qwen3_5/forward.odin:69-127) for one
 * token at `pos`, between the q/k/v projections and wo: per head q = the first
 * head_dim values of its [q | gate] slice of qproj, RMSNorm with q_norm; k
 * heads RMSNorm with k_norm; RoPE on the first rotary_dim dimensions only
 * (pairs i, i + rotary_dim/2; angle pos * inv_freq[i], qwen3_5/ops.odin:77-89); k and v
 * stored as f16 in the cache [n_kv_heads][seq_len][head_dim] at pos; scores
 * q.k * (1/sqrt(head_dim)) over positions 0..pos, softmax, weighted sum of v;
 * out = that sum * sigmoid(gate).  head_dim 128 or 256.  Device pointers;
 * enqueued on `stream`. */
int oi_qwen35_attn_step_launch(const oi_qwen35_attn_dims *d, int32_t pos, const float *qproj, const float *k,
                               const float *v, const float *q_norm, const float *k_norm, const float *inv_freq,
                               uint16_t *k_cache, uint16_t *v_cache, void *workspace, float *out, void *stream);

/* Host-memory form over n_tokens consecutive positions pos0.. (synchronous):
 * qproj [n][n_heads*2*head_dim], k and v [n][n_kv_heads*head_dim]; the caches
 * (f16 bits, [n_kv_heads][seq_len][head_dim]) in and out in host memory;
 * out [n][n_heads*head_dim]. */
int oi_qwen35_attn_steps(const oi_qwen35_attn_dims *d, int32_t n_tokens, int32_t pos0, const float *qproj,
                         const float *k, const float *v, const float *q_norm, const float *k_norm,
                         const float *inv_freq, uint16_t *k_cache, uint16_t *v_cache, float *out);

/* --------------------------------------------------- mixture of experts --- */

/* Shape of a routed-expert FFN: n_experts, experts per token, model dim,
 * expert inner dim, and whether the chosen router probabilities are
 * renormalized to sum 1. */
typedef struct {
    int32_t n_experts, top_k, dim, inter, norm_topk_prob;
} oi_moe_dims;

/* Device scratch bytes that oi_moe_ffn_launch needs. */
int64_t oi_moe_workspace_bytes(const oi_moe_dims *d);

/* One token through a routed-expert SwiGLU FFN.  No counterpart in the
 * reference (its Qwen3.5 MLP is dense, qwen3_5/model.odin:80-82,
 * qwen3_5/forward.odin:227-243); the convention is HF Qwen3-MoE's: logits = router x,
 * p = softmax over all experts, the top_k largest p (ties to the lower id),
 * weights p or p / sum (norm_topk_prob), y = sum_k w_k down_e(silu(gate_e x) *
 * up_e x).  router [n_experts][dim]; gate and up stacked [n_experts*inter][dim];
 * down stacked [n_experts*dim][inter] (oi_weights of any GEMV type).  The
 * experts are chosen on the device; only the chosen experts' rows are read.
 * x_dev, y_dev [dim]; workspace of oi_moe_workspace_bytes.  Enqueued on
 * `stream`. */
int oi_moe_ffn_launch(const oi_moe_dims *d, const oi_weights *router, const oi_weights *gate, const oi_weights *up,
                      const oi_weights *down, const float *x_dev, void *workspace, float *y_dev, void *stream);

/* oi_moe_ffn_launch for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments and result as
 * oi_moe_ffn_launch without the workspace: the library uses a fixed 512 KiB
 * device array of its own, one per GPU, held until the process ends, and
 * rejects dims whose oi_moe_workspace_bytes exceed it (OI_E_ARG).  It calls
 * no hipMalloc/hipFree.  Calls on one GPU share the array, so calls that
 * overlap on one GPU (two streams or two threads) race.  The array's device
 * address is looked up once per GPU and kept: do not call it across a
 * hipDeviceReset of that GPU (the code object, and the array with it, may
 * move). */
int oi_moe_ffn_launch_noalloc(const oi_moe_dims *d, const oi_weights *router, const oi_weights *gate,
                              const oi_weights *up, const oi_weights *down, const float *x_dev, float *y_dev,
                              void *stream);

/* Host-memory form (synchronous); also returns the chosen ids and weights
 * (ids_out, w_out: top_k each, may be NULL). */
int oi_moe_ffn(const oi_moe_dims *d, int32_t router_type, const void *router_blocks, int32_t expert_type,
               const void *gate_blocks, const void *up_blocks, const void *down_blocks, const float *x, float *y,
               int32_t *ids_out, float *w_out);

#ifdef __cplusplus
}
#endif
#endif /* OI_H */
