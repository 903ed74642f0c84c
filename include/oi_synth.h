/*
 * oi_synth.h -- seeded synthetic GGUF models and quantizers (host only).
 *
 * The reference has no writer and no quantizer (it only dequantizes:
 * ggml/quant.odin:76-282) and ships no model files.  This library writes the
 * GGUF files that the parity tests and the benchmark load.  It emits exactly
 * the metadata keys and tensor names that the reference's dense Qwen3 loader
 * reads (infer/model.odin:99-179; ggml/gguf.odin:167-229).
 *
 * Weights: every 2-D weight is N(0, sigma) from a generator seeded by
 * (seed, tensor name, row); F32 norm weights are 1 + N(0, norm_sigma).
 * Quantizers produce valid blocks; bit-exactness is a property of dequant,
 * not of the quantizer.
 */
#ifndef OI_SYNTH_H
#define OI_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oi_synth_spec {
    int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim;
    int64_t vocab_size, context_length;
    float rope_theta, rms_eps;
    int32_t type_default;  /* ggml type of attn_q/k/output, ffn_gate/up */
    int32_t type_attn_v;   /* ggml type of attn_v */
    int32_t type_ffn_down; /* ggml type of ffn_down */
    int32_t type_embd;     /* ggml type of token_embd */
    int32_t type_output;   /* ggml type of output.weight; -1 = tied (no tensor) */
    float sigma;           /* stddev of 2-D weights */
    float norm_sigma;      /* stddev around 1.0 of F32 norm weights */
    uint64_t seed;
    int32_t n_threads;
    /* Architecture: 0 = dense Qwen3 ("qwen3"); 1 = Qwen3-MoE ("qwen3moe": the
     * FFN of every layer is n_experts routed experts of expert_ffn, top
     * n_experts_used, router ffn_gate_inp); 2 = Qwen3.5 hybrid ("qwen35", the
     * layout qwen3_5/model.odin:225-364 reads: every full_attn_interval-th layer
     * full attention with [q | gate] heads and partial RoPE, the others gated
     * DeltaNet; the FFN dense, or routed experts plus a shared expert of
     * shared_expert_ffn with a sigmoid gate when n_experts > 0). */
    int32_t arch;
    int32_t n_experts, n_experts_used, expert_ffn, shared_expert_ffn;
    int32_t type_router;   /* ggml type of ffn_gate_inp (and ffn_gate_inp_shexp) */
    int32_t full_attn_interval, rotary_dim;
    int32_t lin_n_k_heads, lin_n_v_heads, lin_head_k_dim, lin_head_v_dim, lin_conv_kernel;
} oi_synth_spec;

/* Write a GGUF v3 file of spec->arch. Returns 0 or a negative code. */
int oi_synth_write_gguf(const char *path, const oi_synth_spec *spec);

/* Quantize nrows x ncols f32 (row-major) to `type` blocks (GGUF layout).
 * Types: F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q6_K. */
int oi_quantize_rows(int32_t type, const float *src, int64_t nrows, int64_t ncols, uint8_t *dst);

/* n samples of N(0,1)*scale from `seed` (deterministic, multithreaded). */
void oi_synth_normal_f32(uint64_t seed, int64_t n, float scale, float *out, int32_t n_threads);
/* Same, rounded to binary16 (round to nearest even), as raw bits. */
void oi_synth_normal_f16(uint64_t seed, int64_t n, float scale, uint16_t *out, int32_t n_threads);

/* The weights that oi_synth_write_gguf stores for `name` before quantization
 * (rows x cols f32), for tests that need the unquantized values. */
void oi_synth_tensor_f32(uint64_t seed, const char *name, int64_t rows, int64_t cols, float sigma,
                         float mean, float *out, int32_t n_threads);

#ifdef __cplusplus
}
#endif
#endif /* OI_SYNTH_H */
