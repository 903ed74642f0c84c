// engine_internal.h -- the engine's device state, shared by the sources of
// liboi_hip.so that operate on a loaded engine (engine.cpp, state.cpp).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "oi.h"
#include "oi_kernels.h"

namespace oi {

struct Arena {
    uint8_t *base = nullptr;
    size_t size = 0, used = 0;
    uint8_t *take(size_t n) {
        size_t at = (used + 255) & ~(size_t)255;
        if (at + n > size) return nullptr;
        used = at + n;
        return base + at;
    }
};

// Layer kinds: Qwen3 attention (infer/forward.odin:45-121), Qwen3.5 full
// attention (qwen3_5/forward.odin:46-135), Qwen3.5 gated DeltaNet (:137-225).
enum { LK_QWEN3 = 0, LK_FULL = 1, LK_LINEAR = 2 };

struct LayerDev {
    int kind = LK_QWEN3;
    bool moe = false, shared = false;  // routed-expert FFN (with a shared expert)
    bool shared_merged = false;        // the shared expert stored as expert n_experts of the stacks
    DMat wq{}, wk{}, wv{}, wo{}, w1{}, w2{}, w3{};
    const float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    DMat router{}, gexp{}, uexp{}, dexp{}, sh_inp{}, sh_gate{}, sh_up{}, sh_down{};
    DMat in_qkv{}, in_z{}, in_b{}, in_a{}, ssm_out{};
    const float *conv_w = nullptr, *dt_bias = nullptr, *ssm_a = nullptr, *ssm_norm = nullptr;
    float *conv_state = nullptr, *rec_state = nullptr;
};

// One launch of the token step: a GEMV (dense or routed-expert), an attention
// or a DeltaNet step.  `role` is the kernel id of oi_engine_time_kernel.
enum { OP_GEMV = 0, OP_MOE_ROWS, OP_MOE_COLS, OP_ATTN, OP_Q35, OP_DN, OP_MOE_ROWS_R };
struct Op {
    int kind = OP_GEMV, role = 0;
    double bytes = 0;  // algorithmic HBM bytes per launch (attention: without the cache rows)
    GemvArgs g{};
    AttnArgs at{};
    Q35Args q{};
    DnArgs dn{};
};

// The host half of a weight upload: the GGUF matrix `src` (rows x cols of
// `type`) repacked into the device layout in `stage`.  OI_OK, or OI_E_ARG
// when a row is not a whole number of blocks.  Separate so that the sanitizer
// build can run it on files without a device.
int repack_matrix_host(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols, std::vector<uint8_t> &stage);

}  // namespace oi

enum { K_QKV = 0, K_ATTN = 1, K_WO = 2, K_GATEUP = 3, K_DOWN = 4, K_OUTPUT = 5, K_TOKEN = 6, K_ROUTER = 7,
       K_LIN_IN = 8, K_DELTANET = 9, K_LIN_OUT = 10, K_SHARED = 11, K_LAST = 11 };

struct oi_engine {
    oi_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    oi::Arena arena;
    std::vector<oi::LayerDev> layers;
    oi::DMat tok_embd{}, output{};
    const float *output_norm = nullptr;
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *hb = nullptr;
    float *logits = nullptr, *part = nullptr, *am_val = nullptr;
    int32_t *am_idx = nullptr, *state = nullptr, *tokens = nullptr;
    int n_partials = 0;
    bool use_graph = true;
    float2 *rope_cs = nullptr;
    float *logits_host = nullptr;
    int32_t *state_host = nullptr;
    int chunk = 64, max_splits = 0;
    int arch = 0;  // 0 qwen3, 1 qwen3moe, 2 qwen35
    int64_t n_experts = 0, top_k = 0, expert_ffn = 0, shared_ffn = 0;
    int64_t rotary_dim = 0, lin_nk = 0, lin_nv = 0, lin_hk = 0, lin_hv = 0, lin_kernel = 0, full_interval = 0;
    std::vector<std::vector<oi::Op>> ops;  // per layer, in launch order
    oi::GemvArgs g_out{};
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    // sampled decoding: the sampler's device state, its probability scratch
    // [vocab], and the token step + sampler graph
    oi::SampleState *samp = nullptr;
    float *samp_p = nullptr;
    void *samp_work = nullptr;
    hipGraph_t graph_s[3] = {nullptr, nullptr, nullptr};  // the step + sampler, per sample_mode
    hipGraphExec_t gexec_s[3] = {nullptr, nullptr, nullptr};
    int last_pos = 0;
    size_t weight_bytes = 0;
    float *inv_freq = nullptr;  // Qwen3.5 partial RoPE frequencies [rotary_dim / 2]
    // batched prefill buffers (allocated on the first prefill): token ids,
    // residual [T][dim], rotated q [T][q_dim], f16 projection inputs
    // [T][max(dim, q_dim, hidden, value_dim)], four buffers of partial
    // products; the Qwen3.5 attention gate [T][q_dim]; the DeltaNet scratch
    // (conv outputs, normalized q / k, gates, outputs); the routed-expert
    // scratch (normalized x in f32, router logits, chosen ids / weights, pair
    // lists, work items, SwiGLU rows and down rows per pair)
    void *pf_mem = nullptr;
    int32_t *pf_tok = nullptr;
    float *pf_x = nullptr, *pf_q = nullptr, *pf_p[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t pf_pbytes[4] = {0, 0, 0, 0};
    uint16_t *pf_xb = nullptr;
    float *pf_gate = nullptr;
    float *pf_conv = nullptr, *pf_qk = nullptr, *pf_gates = nullptr, *pf_o = nullptr;
    float *pf_dc = nullptr;  // the chunked delta rule's Tb and M per value head and 64-token chunk
    float *pf_xn = nullptr, *pf_lg = nullptr, *pf_w = nullptr, *pf_h = nullptr, *pf_yd = nullptr;
    float *pf_h2 = nullptr;  // up rows of the routed experts (few-pair items)
    int32_t *pf_ids = nullptr, *pf_list = nullptr, *pf_off = nullptr, *pf_cnt = nullptr, *pf_fill = nullptr;
    int32_t *pf_items_gu = nullptr, *pf_items_dn = nullptr, *pf_nitems = nullptr;
    // the router's work items for mt_q4i8_kernel: list, items, then off / cnt / count (filled for pf_rt_T tokens)
    int32_t *pf_rt = nullptr;
    int pf_rt_T = 0;
    // the chunk's normalized rows quantized once for the int8 router and
    // gate/up items (launch_qi_rows): operand slots, group sums, scales
    void *pf_xq = nullptr;
    float *pf_xq_sum = nullptr, *pf_xq_scale = nullptr;
    bool pf_xq_on = true;  // OI_PREFILL_XQ=0: every int8 item quantizes its x rows itself (tests)
    bool pf_fused = true;  // gate/up GEMM with the SwiGLU epilogue where it applies (OI_PREFILL_UNFUSED=1: off)
    int pf_experts = 0;  // routed experts of a prefill: 0 the default kernels, 1 the multi-token GEMV, 2 f32 MFMA
                         // only, 3 no few-pair items, 4 few-pair items on MFMA (OI_PREFILL_EXPERTS=gemv / f32 /
                         // wide / fewmfma)
    bool dn_fused = false;  // token loop: the one-launch DeltaNet step instead of the split one (OI_DN_FUSED)
    bool router_fused = false;  // token loop: the router inside the routed gate/up launch where it applies
                                // (OI_MOE_ROUTER=fused; measured slower at config 4 than its own launch)
    int pf_dn_chunk = 64;  // delta rule of a prefill chunk: 0 token by token, 16 / 32 / 64 chunked (OI_PREFILL_DN_CHUNK)
    // engine_verify_batch: the logits of every position, [rows][vocab] on the
    // device and in pinned host memory (allocated on first use, grown as needed)
    float *vf_dev = nullptr, *vf_host = nullptr;
    int64_t vf_rows = 0;
};

