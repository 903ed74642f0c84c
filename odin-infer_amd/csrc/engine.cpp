// engine.cpp -- the C ABI (include/oi.h): engine load / forward / destroy on
// one gfx950 GPU, plus the kernel test and bench hooks.
//
// One engine = one HIP stream, one device arena holding every weight matrix
// (in the GEMV layout, oi_kernels.h), the f16 KV cache, activations and the
// small device state [token, pos, step, capacity].  A token step is recorded
// once into a hipGraph (5 kernels per layer + embedding + output) and
// replayed; token and pos live in device memory so the same graph serves
// every position and the device-side greedy loop.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <climits>
#include <cstddef>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gguf.h"
#include "oi.h"
#include "oi_kernels.h"
#include "engine_internal.h"

using namespace oi;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(OI_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

bool device_type_ok(uint32_t t) {
    return t == T_F32 || t == T_F16 || t == T_Q8_0 || t == T_Q4_K || t == T_Q6_K || t == T_Q4_0 || t == T_Q4_1 ||
           t == T_Q5_0 || t == T_Q5_1;
}

const char *type_name(uint32_t t) {
    switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 12: return "Q4_K";
    case 14: return "Q6_K";
    default: return "other";
    }
}

int check_device(int dev) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(OI_E_DEVICE, "no HIP device visible");
    if (dev < 0 || dev >= n) return fail(OI_E_DEVICE, "device ordinal out of range");
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return fail(OI_E_DEVICE, "hipGetDeviceProperties failed");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(OI_E_DEVICE, std::string("this library is built for gfx950; device is ") + p.gcnArchName);
    if (hipSetDevice(dev) != hipSuccess) return fail(OI_E_DEVICE, "hipSetDevice failed");
    return OI_OK;
}

// Bytes of a matrix in GGUF layout (= bytes in the device layout).
bool matrix_bytes(uint32_t type, int64_t rows, int64_t cols, size_t &bytes) {
    int e, b;
    if (!block_info(type, e, b) || cols % e) return false;
    bytes = (size_t)(rows * (cols / e) * b);
    return true;
}

}  // namespace

namespace oi {
// Q4_K super-block header in the device form: d, dmin, then the 6-bit
// (scale, min) of each group pair p as one 24-bit field at bits 24p of the
// tail.  The values are those of get_scale_min_k4 (ggml/quant.odin:64-73).
void q4k_header(const uint8_t *blk, uint8_t *out) {
    const uint8_t *q = blk + 4;
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = q[j] & 63;
            mn[j] = q[j + 4] & 63;
        } else {
            sc[j] = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
            mn[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
        }
    }
    std::memcpy(out, blk, 4);
    uint64_t lo = 0, hi = 0;  // 96-bit tail as two words
    for (int p = 0; p < 4; p++) {
        const uint64_t f = (uint64_t)sc[2 * p] | (uint64_t)mn[2 * p] << 6 | (uint64_t)sc[2 * p + 1] << 12 |
                           (uint64_t)mn[2 * p + 1] << 18;
        const int bit = 24 * p;
        if (bit >= 64) {
            hi |= f << (bit - 64);
        } else {
            lo |= f << bit;
            if (bit + 24 > 64) hi |= f >> (64 - bit);
        }
    }
    std::memcpy(out + 4, &lo, 8);
    std::memcpy(out + 12, &hi, 4);
}

// Records a failure for oi_last_error() from the library's other sources.
int set_error(int code, const char *msg) { return fail(code, msg); }

}  // namespace oi

namespace {

// Repack one GGUF matrix into the device layout (see DMat in oi_kernels.h).
// Writes into `dst` (bytes from matrix_bytes) and returns the region offsets.
struct Regions { size_t q = 0, plane = 0, s = 0, d = 0; };
Regions repack(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols, uint8_t *dst) {
    Regions r;
    const int64_t U = cols / 64, NSB = cols / 256, NB = cols / 32;
    if (type == T_Q4_K) {
        r.plane = (size_t)(rows * U * 16);
        r.s = 2 * r.plane;
        for (int64_t row = 0; row < rows; row++)
            for (int64_t sb = 0; sb < NSB; sb++) {
                const uint8_t *b = src + (row * NSB + sb) * 144;
                q4k_header(b, dst + r.s + (row * NSB + sb) * 16);
                for (int p = 0; p < 4; p++) {
                    const size_t u = (size_t)(row * U + 4 * sb + p);
                    std::memcpy(dst + u * 16, b + 16 + 32 * p, 16);
                    std::memcpy(dst + r.plane + u * 16, b + 32 + 32 * p, 16);
                }
            }
    } else if (type == T_Q6_K) {
        r.plane = (size_t)(rows * U * 16);
        r.s = 3 * r.plane;
        r.d = r.s + (size_t)(rows * NSB * 16);
        for (int64_t row = 0; row < rows; row++)
            for (int64_t sb = 0; sb < NSB; sb++) {
                const uint8_t *b = src + (row * NSB + sb) * 210;  // ql[128] qh[64] sc[16] d
                std::memcpy(dst + r.s + (row * NSB + sb) * 16, b + 192, 16);
                std::memcpy(dst + r.d + (row * NSB + sb) * 2, b + 208, 2);
                for (int h = 0; h < 2; h++)
                    for (int half = 0; half < 2; half++) {
                        const int l0 = 16 * half;
                        const size_t u = (size_t)(row * U + 4 * sb + 2 * h + half);
                        std::memcpy(dst + u * 16, b + 64 * h + l0, 16);
                        std::memcpy(dst + r.plane + u * 16, b + 64 * h + 32 + l0, 16);
                        std::memcpy(dst + 2 * r.plane + u * 16, b + 128 + 32 * h + l0, 16);
                    }
            }
    } else if (type == T_Q8_0) {
        r.plane = (size_t)(rows * U * 16);
        r.d = 4 * r.plane;
        for (int64_t row = 0; row < rows; row++)
            for (int64_t blk = 0; blk < NB; blk++) {
                const uint8_t *b = src + (row * NB + blk) * 34;
                std::memcpy(dst + r.d + (row * NB + blk) * 2, b, 2);
                const size_t u = (size_t)(row * U + blk / 2);
                for (int h = 0; h < 2; h++)
                    std::memcpy(dst + (size_t)(2 * (blk & 1) + h) * r.plane + u * 16, b + 2 + 16 * h, 16);
            }
    } else {
        size_t bytes = 0;
        matrix_bytes(type, rows, cols, bytes);
        std::memcpy(dst, src, bytes);
    }
    return r;
}

DMat make_dmat(uint32_t type, int64_t rows, int64_t cols, const uint8_t *dev, const Regions &r) {
    DMat m{};
    m.type = (int32_t)type;
    m.rows = (int32_t)rows;
    m.cols = (int32_t)cols;
    m.q = dev + r.q;
    m.plane = (int64_t)r.plane;
    m.s = dev + r.s;
    m.d = (const uint16_t *)(dev + r.d);
    return m;
}

// Rows [r0, r0 + n) of a device matrix as a matrix of its own (the planes
// keep their stride; the per-row regions move by r0 rows).
DMat dmat_rows(const DMat &m, int64_t r0, int64_t n) {
    DMat v = m;
    v.rows = (int32_t)n;
    const size_t r = (size_t)r0, c = (size_t)m.cols;
    switch (m.type) {
    case T_Q4_K: v.q += r * (c / 64) * 16; v.s += r * (c / 256) * 16; break;
    case T_Q6_K: v.q += r * (c / 64) * 16; v.s += r * (c / 256) * 16; v.d += r * (c / 256); break;
    case T_Q8_0: v.q += r * (c / 64) * 16; v.d += r * (c / 32); break;
    case T_F16: v.q += r * c * 2; break;
    case T_Q4_0: v.q += r * (c / 32) * 18; break;
    case T_Q4_1: v.q += r * (c / 32) * 20; break;
    case T_Q5_0: v.q += r * (c / 32) * 22; break;
    case T_Q5_1: v.q += r * (c / 32) * 24; break;
    default: v.q += r * c * 4; break;
    }
    return v;
}

// Host staging of a repacked matrix, then one copy into device memory.
int upload_matrix(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols, uint8_t *dev, hipStream_t st,
                  std::vector<uint8_t> &stage, DMat &out) {
    size_t bytes;
    if (!matrix_bytes(type, rows, cols, bytes)) return fail(OI_E_ARG, "matrix size not a whole number of blocks");
    stage.resize(bytes);
    Regions r = repack(type, src, rows, cols, stage.data());
    HIP_TRY(hipMemcpyAsync(dev, stage.data(), bytes, hipMemcpyHostToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));
    out = make_dmat(type, rows, cols, dev, r);
    return OI_OK;
}

}  // namespace

namespace oi {
int repack_matrix_host(uint32_t type, const uint8_t *src, int64_t rows, int64_t cols, std::vector<uint8_t> &stage) {
    size_t bytes;
    if (!matrix_bytes(type, rows, cols, bytes)) return fail(OI_E_ARG, "matrix size not a whole number of blocks");
    stage.resize(bytes);
    (void)repack(type, src, rows, cols, stage.data());
    return OI_OK;
}
}  // namespace oi

namespace {

hipError_t launch_op(const oi_engine *e, const Op &o, hipStream_t st) {
    switch (o.kind) {
    case OP_MOE_ROWS: return launch_gemv_q_moe(o.g, MOE_ROWS, st);
    case OP_MOE_ROWS_R: return launch_gemv_q_moe(o.g, MOE_ROWS_R, st);
    case OP_MOE_COLS: return launch_gemv_q_moe(o.g, MOE_COLS, st);
    case OP_ATTN: return launch_attn(o.at, (int)e->cfg.head_dim, st);
    case OP_Q35: return launch_q35_attn(o.q, (int)e->cfg.head_dim, st);
    case OP_DN: return launch_deltanet(o.dn, st);
    default: return launch_gemv(o.g, st);
    }
}

int enqueue_token(oi_engine *e) {
    const hipStream_t st = e->stream;
    HIP_TRY(launch_embed(e->tok_embd, e->state, e->x, (int32_t)e->cfg.vocab_size, e->am_val, e->am_idx, e->tokens,
                         0, st));
    for (const auto &layer : e->ops)
        for (const Op &o : layer) HIP_TRY(launch_op(e, o, st));
    HIP_TRY(launch_gemv(e->g_out, st));
    return OI_OK;
}

int ensure_graph(oi_engine *e) {
    if (e->gexec || !e->use_graph) return OI_OK;
    HIP_TRY(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_token(e);
    hipGraph_t g = nullptr;
    hipError_t ec = hipStreamEndCapture(e->stream, &g);
    if (rc) return rc;
    if (ec != hipSuccess) return fail(OI_E_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(ec));
    e->graph = g;
    HIP_TRY(hipGraphInstantiate(&e->gexec, g, nullptr, nullptr, 0));
    return OI_OK;
}

int set_state(oi_engine *e, int32_t token, int32_t pos, int32_t cap) {
    for (int i = 0; i < ST_WORDS; i++) e->state_host[i] = 0;
    e->state_host[ST_TOKEN] = token;
    e->state_host[ST_POS] = pos;
    e->state_host[ST_CAP] = cap;
    e->state_host[ST_NPART] = e->n_partials;
    HIP_TRY(hipMemcpyAsync(e->state, e->state_host, ST_WORDS * 4, hipMemcpyHostToDevice, e->stream));
    return OI_OK;
}

// One token step: the captured graph, or its launches issued directly
// (OI_NO_GRAPH=1, e.g. under tools that do not follow graph capture).
int run_token(oi_engine *e) {
    if (e->use_graph) {
        HIP_TRY(hipGraphLaunch(e->gexec, e->stream));
        return OI_OK;
    }
    return enqueue_token(e);
}

GemvArgs gemv_args(int mode, int K, const float *x, const float *norm_w, float eps) {
    GemvArgs a{};
    a.mode = mode;
    a.K = K;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    return a;
}


// Mean time of one token step (the token kernel, or the multi-kernel graph)
// over `iters` consecutive greedy steps from the last forward/decode position
// (moved back so the steps stay inside the context), HIP events on the
// engine stream.  *bytes: algorithmic HBM bytes of one step at the mean
// position (weights read once, f16 K/V read and written, logits written).
int time_token(oi_engine *e, int iters, double *avg_us, double *bytes) {
    const oi_config &c = e->cfg;
    if (iters >= c.seq_len) return fail(OI_E_ARG, "iters exceeds the context");
    const int start = (int)std::min<int64_t>(e->last_pos, c.seq_len - 1 - iters);
    int rc = ensure_graph(e);
    if (rc) return rc;
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    for (int pass = 0; pass < 2; pass++) {  // warm-up pass, then the timed pass
        if ((rc = set_state(e, 0, start, 0))) return rc;
        if (pass) HIP_TRY(hipEventRecord(e0, e->stream));
        for (int i = 0; i < iters; i++)
            if ((rc = run_token(e))) return rc;
        if (pass) HIP_TRY(hipEventRecord(e1, e->stream));
    }
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    *avg_us = ms * 1000.0 / iters;
    // every launch's algorithmic bytes (weights read once: routed experts only
    // the chosen ones), the cache rows read at the mean position, the classifier
    size_t b = 0;
    matrix_bytes((uint32_t)e->output.type, e->output.rows, e->output.cols, b);
    double w = (double)b + 4.0 * c.dim + 4.0 * c.vocab_size;  // + output_norm, logits
    size_t erow = 0;
    matrix_bytes((uint32_t)e->tok_embd.type, 1, e->tok_embd.cols, erow);
    w += (double)erow;
    const double kvd = (double)(c.n_kv_heads * c.head_dim), mean_pos = start + (iters - 1) / 2.0;
    for (const auto &layer : e->ops)
        for (const Op &o : layer) {
            w += o.bytes;
            if (o.kind == OP_ATTN || o.kind == OP_Q35) w += 2 * kvd * 2 * (mean_pos + 1);
        }
    *bytes = w;
    e->last_pos = start + iters - 1;
    return OI_OK;
}

}  // namespace

extern "C" {

const char *oi_last_error(void) { return g_err.c_str(); }

void oi_engine_destroy(oi_engine *e) {
    if (!e) return;
    hipSetDevice(e->device);
    if (e->stream) hipStreamSynchronize(e->stream);
    if (e->gexec) hipGraphExecDestroy(e->gexec);
    if (e->graph) hipGraphDestroy(e->graph);
    for (int m = 0; m < 3; m++) {
        if (e->gexec_s[m]) hipGraphExecDestroy(e->gexec_s[m]);
        if (e->graph_s[m]) hipGraphDestroy(e->graph_s[m]);
    }
    if (e->arena.base) hipFree(e->arena.base);
    if (e->pf_mem) hipFree(e->pf_mem);
    if (e->logits_host) hipHostFree(e->logits_host);
    if (e->state_host) hipHostFree(e->state_host);
    if (e->vf_dev) hipFree(e->vf_dev);
    if (e->vf_host) hipHostFree(e->vf_host);
    if (e->stream) hipStreamDestroy(e->stream);
    delete e;
}

int oi_engine_load(const char *path, const oi_opts *opts, oi_engine **out) {
    if (!path || !opts || !out) return fail(OI_E_ARG, "null argument");
    *out = nullptr;
    if (!opts->use_hip) return fail(OI_E_ARG, "use_hip must be set: this library has no CPU path");
    if (opts->max_ctx <= 0) return fail(OI_E_ARG, "max_ctx must be positive");

    // the file and the model are checked first, as the reference builds the
    // transformer before it initialises the GPU (infer/engine.odin:21-25)
    GgufFile g;
    std::string err;
    int rc = g.open(path, err);
    if (rc) return fail(rc, err);

    // load_config (infer/model.odin:99-139; qwen3_5/model.odin:225-304): the
    // metadata keys carry the architecture name as their prefix
    auto *am = g.meta("general.architecture");
    const std::string arch = am ? am->str : "";
    std::unique_ptr<oi_engine> e(new oi_engine());
    e->arch = arch == "qwen3moe" ? 1 : arch == "qwen35" ? 2 : 0;
    if (e->arch == 0 && arch != "qwen3")
        std::fprintf(stderr, "warning: architecture is '%s', expected 'qwen3'\n", arch.c_str());
    const std::string a = (e->arch == 0 ? std::string("qwen3") : arch) + ".";
    auto key = [&](const char *k, int64_t &v) -> int {
        auto *m = g.meta(a + k);
        if (!m) return fail(OI_E_MODEL, "missing metadata key: " + a + k);
        v = (int64_t)m->u;
        return OI_OK;
    };
    e->device = opts->device;
    oi_config &c = e->cfg;
    if ((rc = key("embedding_length", c.dim)) || (rc = key("feed_forward_length", c.hidden_dim)) ||
        (rc = key("block_count", c.n_layers)) || (rc = key("attention.head_count", c.n_heads)) ||
        (rc = key("attention.head_count_kv", c.n_kv_heads)) || (rc = key("context_length", c.max_seq)) ||
        (rc = key("attention.key_length", c.head_dim)))
        return rc;
    const bool moe = e->arch == 1 || (e->arch == 2 && g.meta(a + "expert_count"));
    if (moe) {
        if ((rc = key("expert_count", e->n_experts)) || (rc = key("expert_used_count", e->top_k)) ||
            (rc = key("expert_feed_forward_length", e->expert_ffn)))
            return rc;
        if (auto *m = g.meta(a + "expert_shared_feed_forward_length")) e->shared_ffn = (int64_t)m->u;
        c.hidden_dim = e->expert_ffn;
    }
    if (e->arch == 2) {
        int64_t inner = 0;
        if ((rc = key("ssm.group_count", e->lin_nk)) || (rc = key("ssm.time_step_rank", e->lin_nv)) ||
            (rc = key("ssm.state_size", e->lin_hk)) || (rc = key("ssm.inner_size", inner)) ||
            (rc = key("ssm.conv_kernel", e->lin_kernel)) || (rc = key("full_attention_interval", e->full_interval)) ||
            (rc = key("rope.dimension_count", e->rotary_dim)))
            return rc;
        e->lin_hv = e->lin_nv > 0 ? inner / e->lin_nv : 0;
    }
    auto *rf = g.meta(a + "rope.freq_base");
    c.rope_freq = rf ? (float)rf->f : (e->arch == 2 ? 10000000.0f : 1000000.0f);
    auto *re = g.meta(a + "attention.layer_norm_rms_epsilon");
    c.rms_eps = re ? (float)re->f : 1e-6f;

    auto require = [&](const std::string &name, const GgufTensor *&t) -> int {
        t = g.tensor(name);
        if (!t) return fail(OI_E_MODEL, "missing required tensor: " + name);
        if (!device_type_ok(t->kind))
            return fail(OI_E_UNSUPPORTED, "tensor " + name + " has quant type " + type_name(t->kind) +
                                              " (supported on this path: F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q6_K)");
        return OI_OK;
    };
    const GgufTensor *emb;
    if ((rc = require("token_embd.weight", emb))) return rc;
    c.vocab_size = (int64_t)emb->dims.back();  // infer/model.odin:137-138
    c.seq_len = std::min<int64_t>(c.max_seq, opts->max_ctx);  // infer/model.odin:220-223
    if (c.seq_len <= 0) c.seq_len = opts->max_ctx;

    if (c.dim <= 0 || c.dim % 256 || c.dim > 15360 || c.hidden_dim <= 0 || c.hidden_dim % 256 ||
        c.hidden_dim > 15360 || c.n_layers <= 0 || c.n_layers > 4096 || c.n_heads <= 0 || c.n_heads > 4096 ||
        c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads)
        return fail(OI_E_MODEL, "model dimensions outside what this path supports");
    const int G = (int)(c.n_heads / c.n_kv_heads);
    if (!((c.head_dim == 128 || c.head_dim == 256) && (G == 1 || G == 2 || G == 4 || G == 8)))
        return fail(OI_E_UNSUPPORTED, "head_dim / GQA group not supported (head_dim 128 or 256, group 1, 2, 4 or 8)");
    if (c.n_heads * c.head_dim > 15360) return fail(OI_E_MODEL, "n_heads*head_dim too large");
    if (moe && (e->n_experts < 1 || e->n_experts > 1024 || e->top_k < 1 || e->top_k > 32 ||
                e->top_k > e->n_experts || e->shared_ffn % 256 || e->shared_ffn > 15360))
        return fail(OI_E_UNSUPPORTED, "expert configuration not supported (<= 1024 experts, top_k <= 32, "
                                      "inner sizes multiples of 256)");
    if (e->arch == 2 && (e->full_interval < 1 || e->lin_hk != 128 || e->lin_hv != 128 || e->lin_nk < 1 ||
                         e->lin_nk > 4096 || e->lin_nv < 1 || e->lin_nv > 4096 || e->lin_nv % e->lin_nk || e->lin_kernel < 1 || e->lin_kernel > 8 ||
                         e->rotary_dim < 0 || e->rotary_dim > c.head_dim || e->rotary_dim % 2))
        return fail(OI_E_UNSUPPORTED, "hybrid configuration not supported (DeltaNet head dims 128, value heads a "
                                      "multiple of key heads, conv kernel <= 8)");

    // tensors (infer/model.odin:141-179; qwen3_5/model.odin:306-364): shapes checked against the config
    // append: a tensor uploaded as more rows of this one (a shared expert as
    // expert n_experts of the stacked matrices); merged_into: this tensor is
    // those rows, a view from row view_r0 of that entry
    struct Want {
        std::string name;
        int64_t rows, cols;
        bool f32;
        const GgufTensor *t;
        const GgufTensor *append = nullptr;
        int merged_into = -1;
        int64_t view_r0 = 0;
    };
    std::vector<Want> want;
    const int64_t D = c.dim, H = c.hidden_dim, QD = c.n_heads * c.head_dim, KVD = c.n_kv_heads * c.head_dim;
    const int64_t E = e->n_experts, EF = e->expert_ffn, SF = e->shared_ffn;
    const int64_t KD = e->lin_nk * e->lin_hk, VD = e->lin_nv * e->lin_hv, CD = 2 * KD + VD;
    want.push_back({"token_embd.weight", c.vocab_size, D, false, nullptr});
    want.push_back({"output_norm.weight", 1, D, true, nullptr});
    const bool tied = g.tensor("output.weight") == nullptr;  // infer/model.odin:149-158
    if (!tied) want.push_back({"output.weight", c.vocab_size, D, false, nullptr});
    std::vector<int> kinds((size_t)c.n_layers);
    std::vector<char> shared((size_t)c.n_layers, 0);
    std::vector<int> exp_at, shx_at;  // want index of each layer's routed / shared gate matrix
    for (int64_t l = 0; l < c.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        // qwen3_5/model.odin:289-300: full attention at layers interval-1, 2 interval-1, ...
        const int kind = e->arch != 2 ? LK_QWEN3 : ((l + 1) % e->full_interval == 0 ? LK_FULL : LK_LINEAR);
        kinds[(size_t)l] = kind;
        want.push_back({p + "attn_norm.weight", 1, D, true, nullptr});
        want.push_back({p + (e->arch == 2 ? "post_attention_norm.weight" : "ffn_norm.weight"), 1, D, true, nullptr});
        if (kind != LK_LINEAR) {
            want.push_back({p + "attn_q_norm.weight", 1, c.head_dim, true, nullptr});
            want.push_back({p + "attn_k_norm.weight", 1, c.head_dim, true, nullptr});
            want.push_back({p + "attn_q.weight", kind == LK_FULL ? 2 * QD : QD, D, false, nullptr});
            want.push_back({p + "attn_k.weight", KVD, D, false, nullptr});
            want.push_back({p + "attn_v.weight", KVD, D, false, nullptr});
            want.push_back({p + "attn_output.weight", D, QD, false, nullptr});
        } else {
            want.push_back({p + "attn_qkv.weight", CD, D, false, nullptr});
            want.push_back({p + "attn_gate.weight", VD, D, false, nullptr});
            want.push_back({p + "ssm_beta.weight", e->lin_nv, D, false, nullptr});
            want.push_back({p + "ssm_alpha.weight", e->lin_nv, D, false, nullptr});
            want.push_back({p + "ssm_conv1d.weight", CD, e->lin_kernel, true, nullptr});
            want.push_back({p + "ssm_dt.bias", 1, e->lin_nv, true, nullptr});
            want.push_back({p + "ssm_a", 1, e->lin_nv, true, nullptr});
            want.push_back({p + "ssm_norm.weight", 1, e->lin_hv, true, nullptr});
            want.push_back({p + "ssm_out.weight", D, VD, false, nullptr});
        }
        if (!moe) {
            want.push_back({p + "ffn_gate.weight", H, D, false, nullptr});
            want.push_back({p + "ffn_down.weight", D, H, false, nullptr});
            want.push_back({p + "ffn_up.weight", H, D, false, nullptr});
        } else {
            want.push_back({p + "ffn_gate_inp.weight", E, D, false, nullptr});
            exp_at.push_back((int)want.size());
            want.push_back({p + "ffn_gate_exps.weight", E * EF, D, false, nullptr});
            want.push_back({p + "ffn_up_exps.weight", E * EF, D, false, nullptr});
            want.push_back({p + "ffn_down_exps.weight", E * D, EF, false, nullptr});
            if (SF > 0 && g.tensor(p + "ffn_gate_inp_shexp.weight")) {
                shared[(size_t)l] = 1;
                shx_at.push_back((int)want.size() + 1);
                want.push_back({p + "ffn_gate_inp_shexp.weight", 1, D, false, nullptr});
                want.push_back({p + "ffn_gate_shexp.weight", SF, D, false, nullptr});
                want.push_back({p + "ffn_up_shexp.weight", SF, D, false, nullptr});
                want.push_back({p + "ffn_down_shexp.weight", D, SF, false, nullptr});
            }
        }
    }
    size_t wbytes = 0;
    for (auto &w : want) {
        if ((rc = require(w.name, w.t))) return rc;
        if (w.f32 && w.t->kind != T_F32) return fail(OI_E_MODEL, "expected F32 tensor for " + w.name);
        if (w.t->nelems() != (uint64_t)(w.rows * w.cols) || w.t->dims[0] != (uint64_t)w.cols)
            return fail(OI_E_MODEL, "tensor " + w.name + " has an unexpected shape");
        wbytes += ((size_t)w.t->nbytes + 255) & ~(size_t)255;
    }
    e->weight_bytes = wbytes;
    e->n_experts = E;
    // a shared expert with the routed experts' inner size and types becomes
    // expert E of the stacked matrices, so the routed gate/up and down launches
    // take it as one more chosen expert (weight sigmoid of its router row)
    std::vector<char> merged((size_t)c.n_layers, 0);
    {
        size_t si = 0;
        for (int64_t l = 0, ei = 0; l < c.n_layers && moe; l++, ei++) {
            if (!shared[(size_t)l]) continue;
            const int xg = exp_at[(size_t)ei], sg = shx_at[si++];
            bool ok = SF == EF;
            for (int m = 0; m < 3 && ok; m++) ok = want[(size_t)(xg + m)].t->kind == want[(size_t)(sg + m)].t->kind;
            if (!ok) continue;
            merged[(size_t)l] = 1;
            for (int m = 0; m < 3; m++) {
                Want &x = want[(size_t)(xg + m)], &sh = want[(size_t)(sg + m)];
                sh.merged_into = xg + m;
                sh.view_r0 = x.rows;  // E * EF (gate, up) or E * D (down)
                x.append = sh.t;
                x.rows += sh.rows;
            }
        }
    }
    if ((rc = check_device(opts->device))) return rc;

    // device memory plan
    int n_attn = 0, n_lin = 0;
    for (int k : kinds) (k == LK_LINEAR ? n_lin : n_attn)++;
    // decode attention at head_dim 128: the lane-per-position kernel over
    // splits of 64 (default), or OI_ATTN=mfma, the matrix-core kernel over
    // splits sized from pos (the same arithmetic; measured no faster at C3)
    const char *af = std::getenv("OI_ATTN");
    e->max_splits = attn_plan((int)c.head_dim, (int)c.n_kv_heads, (int)c.seq_len, &e->chunk,
                              !(af && std::strcmp(af, "mfma") == 0));
    if (e->max_splits > attn_max_splits())
        return fail(OI_E_UNSUPPORTED, "seq_len " + std::to_string(c.seq_len) + " needs " +
                                          std::to_string(e->max_splits) + " attention splits (at most " +
                                          std::to_string(attn_max_splits()) + ")");
    const int q35_splits = e->arch == 2 ? q35_max_splits((int)c.seq_len) : 0;
    const size_t kv_layer = (size_t)c.n_kv_heads * c.seq_len * c.head_dim * 2;
    const size_t conv_layer = (size_t)CD * (e->lin_kernel > 0 ? e->lin_kernel - 1 : 0) * 4;
    const size_t rec_layer = (size_t)e->lin_nv * e->lin_hk * e->lin_hv * 4;
    auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t out_rows = (size_t)c.vocab_size;
    GemvArgs probe = gemv_args(GEMV_ARGMAX, (int)D, nullptr, nullptr, 0.f);
    probe.nseg = 1;
    probe.seg[0].m.type = (int32_t)(tied ? emb->kind : g.tensor("output.weight")->kind);
    probe.seg[0].m.rows = (int32_t)out_rows;
    probe.seg[0].m.cols = (int32_t)D;
    plan_gemv(probe);
    const size_t hb_n = std::max<size_t>({(size_t)H, (size_t)((e->top_k + 1) * EF), (size_t)SF, 1});
    const size_t part_n = std::max((size_t)c.n_heads * e->max_splits * (c.head_dim + 4),
                                   (size_t)c.n_heads * q35_splits * (c.head_dim + 2));
    size_t act = al(D * 4) + al(2 * QD * 4) + 2 * al(KVD * 4) + al(QD * 4) + al(hb_n * 4) + al(out_rows * 4) +
                 al(part_n * 4) + 2 * al((size_t)probe.total_wgs * 4) +
                 al(ST_WORDS * 4) + al((size_t)(c.seq_len + 1) * 4) +
                 al((size_t)c.seq_len * (c.head_dim / 2) * 8);
    if (e->arch == 2)
        act += al(QD * 4) + al((size_t)(e->rotary_dim / 2 + 1) * 4) + 2 * al((size_t)CD * 4) + 2 * al((size_t)VD * 4) +
               2 * al((size_t)e->lin_nv * 4) + al((size_t)e->lin_nv * 16);
    if (moe) act += al((size_t)E * 4) + 3 * al(64 * 4) + al((size_t)SF * 4 + 4);
    act += al(sizeof(SampleState)) + al((size_t)c.vocab_size * 4) + al(sample_work_bytes());  // the sampler
    e->arena.size = wbytes + 2 * kv_layer * n_attn + (conv_layer + rec_layer + 512) * n_lin + act + 8192;
    hipError_t he = hipMalloc(&e->arena.base, e->arena.size);
    if (he != hipSuccess) return fail(OI_E_NOMEM, "hipMalloc of " + std::to_string(e->arena.size) + " bytes failed");
    HIP_TRY(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    HIP_TRY(hipMemsetAsync(e->arena.base, 0, e->arena.size, e->stream));

    // weights
    std::vector<uint8_t> stage;
    std::vector<DMat> mats(want.size());
    std::vector<const float *> f32s(want.size(), nullptr);
    std::vector<uint8_t> cat;
    for (size_t i = 0; i < want.size(); i++) {
        const GgufTensor *t = want[i].t;
        if (want[i].merged_into >= 0) continue;  // uploaded with the tensor it extends
        const size_t nb = (size_t)t->nbytes + (want[i].append ? (size_t)want[i].append->nbytes : 0);
        uint8_t *dev = e->arena.take(nb);
        if (!dev) return fail(OI_E_NOMEM, "arena exhausted");
        const uint8_t *src = t->data;
        if (want[i].append) {  // the GGUF rows of both, one after the other
            cat.resize(nb);
            std::memcpy(cat.data(), t->data, (size_t)t->nbytes);
            std::memcpy(cat.data() + t->nbytes, want[i].append->data, (size_t)want[i].append->nbytes);
            src = cat.data();
        }
        if ((rc = upload_matrix(t->kind, src, want[i].rows, want[i].cols, dev, e->stream, stage, mats[i])))
            return rc;
        f32s[i] = (const float *)dev;
    }
    for (size_t i = 0; i < want.size(); i++)
        if (want[i].merged_into >= 0) mats[i] = dmat_rows(mats[(size_t)want[i].merged_into], want[i].view_r0, want[i].rows);
    std::vector<uint8_t>().swap(cat);
    size_t wi = 0;
    e->tok_embd = mats[wi++];
    e->output_norm = f32s[wi++];
    e->output = tied ? e->tok_embd : mats[wi++];
    e->layers.resize((size_t)c.n_layers);
    for (size_t l = 0; l < e->layers.size(); l++) {
        LayerDev &L = e->layers[l];
        L.kind = kinds[l];
        L.moe = moe;
        L.shared = shared[l] != 0;
        L.shared_merged = merged[l] != 0;
        L.attn_norm = f32s[wi++];
        L.ffn_norm = f32s[wi++];
        if (L.kind != LK_LINEAR) {
            L.q_norm = f32s[wi++];
            L.k_norm = f32s[wi++];
            L.wq = mats[wi++];
            L.wk = mats[wi++];
            L.wv = mats[wi++];
            L.wo = mats[wi++];
        } else {
            L.in_qkv = mats[wi++];
            L.in_z = mats[wi++];
            L.in_b = mats[wi++];
            L.in_a = mats[wi++];
            L.conv_w = f32s[wi++];
            L.dt_bias = f32s[wi++];
            L.ssm_a = f32s[wi++];
            L.ssm_norm = f32s[wi++];
            L.ssm_out = mats[wi++];
        }
        if (!moe) {
            L.w1 = mats[wi++];
            L.w2 = mats[wi++];
            L.w3 = mats[wi++];
        } else {
            L.router = mats[wi++];
            L.gexp = mats[wi++];
            L.uexp = mats[wi++];
            L.dexp = mats[wi++];
            if (L.shared) {
                L.sh_inp = mats[wi++];
                L.sh_gate = mats[wi++];
                L.sh_up = mats[wi++];
                L.sh_down = mats[wi++];
            }
        }
    }
    for (auto &L : e->layers) {
        if (L.kind != LK_LINEAR) {
            L.kc = (uint16_t *)e->arena.take(kv_layer);
            L.vc = (uint16_t *)e->arena.take(kv_layer);
        } else {
            L.conv_state = (float *)e->arena.take(conv_layer + 4);
            L.rec_state = (float *)e->arena.take(rec_layer);
        }
    }
    e->x = (float *)e->arena.take(D * 4);
    e->q = (float *)e->arena.take(2 * QD * 4);  // q, or [q | gate] per head (Qwen3.5)
    e->k = (float *)e->arena.take(KVD * 4);
    e->v = (float *)e->arena.take(KVD * 4);
    e->att = (float *)e->arena.take(QD * 4);
    e->hb = (float *)e->arena.take(hb_n * 4);
    e->logits = (float *)e->arena.take(out_rows * 4);
    e->part = (float *)e->arena.take(part_n * 4);
    e->am_val = (float *)e->arena.take((size_t)probe.total_wgs * 4);
    e->am_idx = (int32_t *)e->arena.take((size_t)probe.total_wgs * 4);
    e->state = (int32_t *)e->arena.take(ST_WORDS * 4);
    e->tokens = (int32_t *)e->arena.take((size_t)(c.seq_len + 1) * 4);
    e->samp = (SampleState *)e->arena.take(sizeof(SampleState));
    e->samp_p = (float *)e->arena.take((size_t)c.vocab_size * 4);
    e->samp_work = e->arena.take(sample_work_bytes());
    e->rope_cs = (float2 *)e->arena.take((size_t)c.seq_len * (c.head_dim / 2) * 8);
    float *qbuf = nullptr, *inv_freq = nullptr, *lin_qkv = nullptr, *lin_conv = nullptr, *lin_z = nullptr;
    float *lin_out = nullptr, *lin_b = nullptr, *lin_a = nullptr, *lin_ssq = nullptr;
    if (e->arch == 2) {
        qbuf = (float *)e->arena.take(QD * 4);
        inv_freq = (float *)e->arena.take((size_t)(e->rotary_dim / 2 + 1) * 4);
        e->inv_freq = inv_freq;
        lin_qkv = (float *)e->arena.take((size_t)CD * 4);
        lin_conv = (float *)e->arena.take((size_t)CD * 4);
        lin_z = (float *)e->arena.take((size_t)VD * 4);
        lin_out = (float *)e->arena.take((size_t)VD * 4);
        lin_b = (float *)e->arena.take((size_t)e->lin_nv * 4);
        lin_a = (float *)e->arena.take((size_t)e->lin_nv * 4);
        lin_ssq = (float *)e->arena.take((size_t)e->lin_nv * 4 * 4);  // [n_vh][hv / 32] (hv 128 on that path)
    }
    float *mo_logits = nullptr, *mo_w = nullptr, *mo_sg = nullptr;
    int32_t *mo_ids = nullptr;
    if (moe) {
        mo_logits = (float *)e->arena.take((size_t)E * 4);
        mo_ids = (int32_t *)e->arena.take(64 * 4);
        mo_w = (float *)e->arena.take(64 * 4);
        mo_sg = (float *)e->arena.take(64 * 4);
    }
    float *sh_h = moe ? (float *)e->arena.take((size_t)SF * 4 + 4) : nullptr;
    if (!e->rope_cs || (e->arch == 2 && !lin_ssq) || (moe && !sh_h))
        return fail(OI_E_NOMEM, "arena exhausted (activations)");

    // RoPE table, same f32 formula as infer/forward.odin:127-130
    {
        const int hd2 = (int)c.head_dim / 2;
        std::vector<float> freq((size_t)hd2);
        for (int i = 0; i < hd2; i++) freq[(size_t)i] = 1.0f / powf(c.rope_freq, (float)i / (float)hd2);
        std::vector<float2> cs((size_t)c.seq_len * hd2);
        for (int64_t p = 0; p < c.seq_len; p++)
            for (int i = 0; i < hd2; i++) {
                const float ang = (float)p * freq[(size_t)i];
                cs[(size_t)p * hd2 + i] = make_float2(cosf(ang), sinf(ang));
            }
        HIP_TRY(hipMemcpyAsync(e->rope_cs, cs.data(), cs.size() * 8, hipMemcpyHostToDevice, e->stream));
        HIP_TRY(hipStreamSynchronize(e->stream));
    }
    if (e->arch == 2) {  // partial-rotary inverse frequencies (qwen3_5/ops.odin:163-168)
        const int half = (int)e->rotary_dim / 2;
        std::vector<float> inv((size_t)half + 1, 0.f);
        const float rd = (float)e->rotary_dim;
        for (int i = 0; i < half; i++) inv[(size_t)i] = 1.0f / powf(c.rope_freq, (float)i / (rd / 2.0f));
        HIP_TRY(hipMemcpyAsync(inv_freq, inv.data(), inv.size() * 4, hipMemcpyHostToDevice, e->stream));
        HIP_TRY(hipStreamSynchronize(e->stream));
    }
    HIP_TRY(hipHostMalloc((void **)&e->logits_host, out_rows * 4, hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&e->state_host, ST_WORDS * 4, hipHostMallocDefault));

    // launch plans
    const float eps = c.rms_eps;
    auto mbytes = [](const DMat &m) {
        size_t b = 0;
        matrix_bytes((uint32_t)m.type, m.rows, m.cols, b);
        return (double)b;
    };
    auto gemv_op = [&](int role, GemvArgs ga) -> Op {
        Op o;
        o.kind = OP_GEMV;
        o.role = role;
        if (!plan_gemv(ga)) fail(OI_E_DEVICE, "internal: GEMV plan");
        o.g = ga;
        const int n = ga.mode == GEMV_SWIGLU ? 2 : ga.nseg;
        double rows = 0;
        for (int i = 0; i < n; i++) {
            o.bytes += mbytes(ga.seg[i].m);
            rows += ga.seg[i].m.rows;
        }
        o.bytes += 4.0 * ga.K + (ga.norm_w ? 4.0 * ga.K : 0) + 4.0 * (ga.mode == GEMV_SWIGLU ? rows / 2 : rows) *
                                                               (ga.mode == GEMV_ADD ? 2 : 1);
        return o;
    };
    e->dn_fused = std::getenv("OI_DN_FUSED") != nullptr;  // the one-launch DeltaNet step in the token loop
    {
        const char *mr = std::getenv("OI_MOE_ROUTER");
        e->router_fused = mr && std::strcmp(mr, "fused") == 0;
    }
    e->ops.assign((size_t)c.n_layers, {});
    for (size_t l = 0; l < e->layers.size(); l++) {
        LayerDev &L = e->layers[l];
        std::vector<Op> &ops = e->ops[l];
        if (L.kind == LK_QWEN3 || L.kind == LK_FULL) {
            GemvArgs q = gemv_args(GEMV_STORE, (int)D, e->x, L.attn_norm, eps);
            q.nseg = 3;
            q.seg[0].m = L.wq; q.seg[0].y = e->q;
            q.seg[1].m = L.wk; q.seg[1].y = e->k;
            q.seg[2].m = L.wv; q.seg[2].y = e->v;
            ops.push_back(gemv_op(K_QKV, q));
            Op at;
            at.role = K_ATTN;
            at.bytes = (QD * 2.0 + 2 * KVD) * 4 + 2.0 * c.head_dim * 4 + 2.0 * KVD * 2;
            if (L.kind == LK_QWEN3) {
                at.kind = OP_ATTN;
                AttnArgs &t = at.at;
                t.q = e->q; t.k = e->k; t.v = e->v;
                t.q_norm = L.q_norm; t.k_norm = L.k_norm; t.eps = eps;
                t.seq_len = (int32_t)c.seq_len;
                t.rope_cs = e->rope_cs;
                t.kc = L.kc; t.vc = L.vc;
                t.state = e->state;
                t.chunk = e->chunk;
                t.max_splits = e->max_splits;
                t.part = e->part;
                t.out = e->att;
                t.n_heads = (int32_t)c.n_heads;
                t.n_kv_heads = (int32_t)c.n_kv_heads;
            } else {
                at.kind = OP_Q35;
                Q35Args &t = at.q;
                t.qproj = e->q; t.k = e->k; t.v = e->v;
                t.q_norm = L.q_norm; t.k_norm = L.k_norm;
                t.inv_freq = inv_freq;
                t.eps = eps;
                t.rotary_dim = (int32_t)e->rotary_dim;
                t.pos = 0;
                t.state = e->state;  // pos from the device state
                t.seq_len = (int32_t)c.seq_len;
                t.n_heads = (int32_t)c.n_heads;
                t.n_kv_heads = (int32_t)c.n_kv_heads;
                t.max_splits = q35_splits;
                t.kc = L.kc; t.vc = L.vc;
                t.qbuf = qbuf;
                t.part = e->part;
                t.out = e->att;
            }
            ops.push_back(at);
            GemvArgs o = gemv_args(GEMV_ADD, (int)QD, e->att, nullptr, eps);
            o.nseg = 1;
            o.seg[0].m = L.wo; o.seg[0].y = e->x;
            ops.push_back(gemv_op(K_WO, o));
        } else {
            GemvArgs in = gemv_args(GEMV_STORE, (int)D, e->x, L.attn_norm, eps);
            in.nseg = 4;
            in.seg[0].m = L.in_qkv; in.seg[0].y = lin_qkv;
            in.seg[1].m = L.in_z; in.seg[1].y = lin_z;
            in.seg[2].m = L.in_b; in.seg[2].y = lin_b;
            in.seg[3].m = L.in_a; in.seg[3].y = lin_a;
            GemvArgs o = gemv_args(GEMV_ADD, (int)VD, lin_out, nullptr, eps);
            o.nseg = 1;
            o.seg[0].m = L.ssm_out; o.seg[0].y = e->x;
            // the split step when both GEMVs take their part: the conv as the
            // in_qkv rows' epilogue, the delta rule on n_vh x 4 workgroups,
            // the gated norm as the output GEMV's prologue
            GemvArgs in2 = in, o2 = o;
            in2.seg[0].y = lin_conv;
            in2.conv_w = L.conv_w; in2.conv_state = L.conv_state; in2.conv_kernel = (int32_t)e->lin_kernel;
            o2.norm_w = L.ssm_norm; o2.gss = lin_ssq;
            const bool split = !e->dn_fused && e->lin_hk == 128 && e->lin_hv == 128 && plan_gemv(in2) &&
                               in2.kernel == 1 && plan_gemv(o2) && o2.kernel == 1;
            ops.push_back(gemv_op(K_LIN_IN, split ? in2 : in));
            Op dn;
            dn.kind = OP_DN;
            dn.role = K_DELTANET;
            DnArgs &t = dn.dn;
            t.qkv = lin_qkv; t.z = lin_z; t.b = lin_b; t.a = lin_a;
            t.conv_w = L.conv_w; t.a_decay = L.ssm_a; t.dt_bias = L.dt_bias; t.norm_w = L.ssm_norm;
            t.eps = eps;
            t.conv_state = L.conv_state;
            t.state = L.rec_state;
            t.conv_out = lin_conv;
            t.out = lin_out;
            t.n_kh = (int32_t)e->lin_nk; t.n_vh = (int32_t)e->lin_nv;
            t.hk = (int32_t)e->lin_hk; t.hv = (int32_t)e->lin_hv; t.kernel = (int32_t)e->lin_kernel;
            t.cols = split ? 1 : 0;
            t.ssq = lin_ssq;
            dn.bytes = split ? 2.0 * rec_layer + (2.0 * KD + VD) * 4 + 2.0 * VD * 4
                             : 2.0 * rec_layer + 2.0 * conv_layer + (double)CD * e->lin_kernel * 4 + (CD + 3.0 * VD) * 4;
            ops.push_back(dn);
            ops.push_back(gemv_op(K_LIN_OUT, split ? o2 : o));
        }
        if (!L.moe) {
            GemvArgs gu = gemv_args(GEMV_SWIGLU, (int)D, e->x, L.ffn_norm, eps);
            gu.nseg = 2;
            gu.seg[0].m = L.w1; gu.seg[0].y = e->hb;
            gu.seg[1].m = L.w3; gu.seg[1].y = e->hb;
            ops.push_back(gemv_op(K_GATEUP, gu));
            GemvArgs dw = gemv_args(GEMV_ADD, (int)H, e->hb, nullptr, eps);
            dw.nseg = 1;
            dw.seg[0].m = L.w2; dw.seg[0].y = e->x;
            ops.push_back(gemv_op(K_DOWN, dw));
            continue;
        }
        // routed experts: router (+ the shared expert's gate row), the chosen
        // experts' gate/up with the routing in its prologue, the shared expert's
        // gate/up, then the two down projections adding into x (the shared one
        // scaled by sigmoid of its gate)
        // a merged shared expert is expert E: one more part of the routed launches
        const int sx = L.shared_merged ? 1 : 0;
        const int64_t KP = e->top_k + sx;  // parts: the chosen experts (+ the shared one)
        Op gu;
        gu.kind = OP_MOE_ROWS;
        gu.role = K_GATEUP;
        GemvArgs &ga = gu.g;
        ga = gemv_args(GEMV_SWIGLU, (int)D, e->x, L.ffn_norm, eps);
        ga.nseg = 2;
        ga.seg[0].m = L.gexp; ga.seg[1].m = L.uexp;
        ga.seg[0].m.rows = ga.seg[1].m.rows = (int32_t)(KP * EF);  // the chosen experts' rows
        ga.seg[0].y = ga.seg[1].y = e->hb;
        ga.moe_logits = mo_logits;
        ga.moe_ids_out = mo_ids;
        ga.moe_w_out = mo_w;
        ga.moe_norm = 1;  // Qwen3-MoE / Qwen3-Next renormalize the chosen weights
        ga.moe_k = (int32_t)KP;
        ga.moe_n = (int32_t)E;
        ga.moe_blk = (int32_t)EF;
        if (sx) {
            ga.moe_sel = (int32_t)e->top_k;
            ga.moe_nblk = (int32_t)E + 1;
            ga.moe_sgate = mo_sg;
        }
        if (!gemv_q_moe_supported(ga, MOE_ROWS))
            return fail(OI_E_UNSUPPORTED, "routed experts: type or shape not supported by the expert GEMV "
                                          "(Q4_K / Q6_K / Q8_0, dim <= 4096, inner a multiple of 256)");
        gu.bytes = 2.0 * KP * mbytes(L.gexp) / (E + sx) + 4.0 * D + 4.0 * E + 4.0 * KP * EF;
        // a router GEMV (+ the shared expert's gate row) first; or, with
        // OI_MOE_ROUTER=fused, the router inside the gate/up launch (each
        // workgroup computes the logits from its normalized x) where the router
        // fits it -- no shared expert, the experts' type.  Config 4: gate/up
        // 16.7 us fused against 5.6 + 9.8 us as two launches (every workgroup
        // reads the router and routes before its first expert row is requested)
        GemvArgs fr = ga;
        fr.moe_logits = nullptr;
        fr.moe_router = L.router;
        if (e->router_fused && !L.shared && gemv_q_moe_supported(fr, MOE_ROWS_R)) {
            ga = fr;
            gu.kind = OP_MOE_ROWS_R;
            gu.bytes += mbytes(L.router);
        } else {
            GemvArgs r = gemv_args(GEMV_STORE, (int)D, e->x, L.ffn_norm, eps);
            r.nseg = L.shared ? 2 : 1;
            r.seg[0].m = L.router; r.seg[0].y = mo_logits;
            if (L.shared) { r.seg[1].m = L.sh_inp; r.seg[1].y = mo_sg; }
            ops.push_back(gemv_op(K_ROUTER, r));
        }
        plan_gemv_q(ga);
        ops.push_back(gu);
        // the shared expert's gate/up reads the same normalized x, so it runs
        // before either down projection adds into x
        if (L.shared && !sx) {
            GemvArgs su = gemv_args(GEMV_SWIGLU, (int)D, e->x, L.ffn_norm, eps);
            su.nseg = 2;
            su.seg[0].m = L.sh_gate; su.seg[0].y = sh_h;
            su.seg[1].m = L.sh_up; su.seg[1].y = sh_h;
            ops.push_back(gemv_op(K_SHARED, su));
        }
        Op dn;
        dn.kind = OP_MOE_COLS;
        dn.role = K_DOWN;
        GemvArgs &gd = dn.g;
        gd = gemv_args(GEMV_ADD, (int)(KP * EF), e->hb, nullptr, eps);
        gd.nseg = 1;
        gd.seg[0].m = L.dexp;
        gd.seg[0].m.rows = (int32_t)D;  // row r of every expert
        gd.seg[0].y = e->x;
        gd.moe_ids = mo_ids;
        gd.moe_w = mo_w;
        gd.moe_k = (int32_t)KP;
        gd.moe_n = (int32_t)E;
        gd.moe_blk = (int32_t)(EF / 64);
        if (sx) gd.moe_nblk = (int32_t)E + 1;
        if (!gemv_q_moe_supported(gd, MOE_COLS))
            return fail(OI_E_UNSUPPORTED, "routed experts: down projection not supported by the expert GEMV");
        plan_gemv_q(gd);
        dn.bytes = KP * mbytes(L.dexp) / (E + sx) + 4.0 * KP * EF + 8.0 * D;
        ops.push_back(dn);
        if (L.shared && !sx) {
            GemvArgs sd = gemv_args(GEMV_ADD, (int)SF, sh_h, nullptr, eps);
            sd.nseg = 1;
            sd.seg[0].m = L.sh_down; sd.seg[0].y = e->x;
            sd.ygate = mo_sg;  // x += sigmoid(gate . x) * shared(x)
            ops.push_back(gemv_op(K_SHARED, sd));
        }
    }
    if (!g_err.empty() && g_err == "internal: GEMV plan") return OI_E_DEVICE;
    GemvArgs ao = gemv_args(GEMV_ARGMAX, (int)D, e->x, e->output_norm, eps);
    ao.nseg = 1;
    ao.seg[0].m = e->output; ao.seg[0].y = e->logits;
    plan_gemv(ao);
    ao.am_val = e->am_val;
    ao.am_idx = e->am_idx;
    ao.state = e->state;
    if (ao.total_wgs != probe.total_wgs) return fail(OI_E_DEVICE, "internal: output plan mismatch");
    e->n_partials = ao.total_wgs;
    e->g_out = ao;
    const char *ng = std::getenv("OI_NO_GRAPH");
    e->use_graph = !(ng && ng[0] == '1');
    const char *pu = std::getenv("OI_PREFILL_UNFUSED");
    e->pf_fused = !(pu && pu[0] == '1');
    const char *pm = std::getenv("OI_PREFILL_EXPERTS");  // "gemv" / "f32": the other expert kernels (tests)
    e->pf_experts = !pm                            ? 0
                    : std::strcmp(pm, "gemv") == 0  ? 1
                    : std::strcmp(pm, "f32") == 0   ? 2
                    : std::strcmp(pm, "wide") == 0  ? 3
                    : std::strcmp(pm, "fewmfma") == 0 ? 4
                    : std::strcmp(pm, "dot4") == 0 ? 5
                    : std::strcmp(pm, "i8") == 0 ? 6
                                                    : 0;
    // the delta rule of a prefill chunk: in its chunked form over 64 tokens on
    // the matrix cores (default), token by token ("0"), or the lane-level
    // chunked form over 16 / 32 tokens
    const char *pq = std::getenv("OI_PREFILL_XQ");
    e->pf_xq_on = !(pq && pq[0] == '0');
    const char *pc = std::getenv("OI_PREFILL_DN_CHUNK");
    e->pf_dn_chunk = !pc                          ? 64
                     : std::strcmp(pc, "16") == 0 ? 16
                     : std::strcmp(pc, "32") == 0 ? 32
                     : std::strcmp(pc, "0") == 0  ? 0
                                                  : 64;

    std::printf("model: %s dim=%lld layers=%lld (attention %d, linear %d) heads=%lld/%lld hidden=%lld vocab=%lld "
                "ctx=%lld/%lld experts=%lld/%lld  weights=%.0f MB  KV cache (f16)=%.0f MB  [gfx950]\n",
                e->arch == 0 ? "qwen3" : arch.c_str(), (long long)c.dim, (long long)c.n_layers, n_attn, n_lin,
                (long long)c.n_heads, (long long)c.n_kv_heads, (long long)c.hidden_dim, (long long)c.vocab_size,
                (long long)c.seq_len, (long long)c.max_seq, (long long)e->top_k, (long long)E, wbytes / 1048576.0,
                2.0 * kv_layer * n_attn / 1048576.0);
    HIP_TRY(hipStreamSynchronize(e->stream));
    *out = e.release();
    return OI_OK;
}

int oi_engine_config(const oi_engine *e, oi_config *out) {
    if (!e || !out) return fail(OI_E_ARG, "null argument");
    *out = e->cfg;
    return OI_OK;
}

static_assert(sizeof(oi_qwen35_config) == 160, "oi_qwen35_config layout (the Odin binding mirrors it)");

int oi_engine_config_qwen35(const oi_engine *e, oi_qwen35_config *out) {
    if (!e || !out) return fail(OI_E_ARG, "null argument");
    const oi_config &c = e->cfg;
    oi_qwen35_config q{};
    q.dim = c.dim;
    q.hidden_dim = c.hidden_dim;
    q.n_layers = c.n_layers;
    q.n_heads = c.n_heads;
    q.n_kv_heads = c.n_kv_heads;
    q.head_dim = c.head_dim;
    q.vocab_size = c.vocab_size;
    q.seq_len = c.seq_len;
    q.max_seq = c.max_seq;
    q.rms_eps = c.rms_eps;
    q.rope_theta = c.rope_freq;
    // a hybrid file's partial RoPE (qwen3_5/model.odin:277-286); every other
    // layout rotates the whole head and has no DeltaNet layers
    const bool hybrid = e->arch == 2;
    q.rotary_dim = hybrid ? e->rotary_dim : c.head_dim;
    q.partial_rotary = (float)q.rotary_dim / (float)std::max<int64_t>(c.head_dim, 1);
    q.lin_n_k_heads = hybrid ? e->lin_nk : 0;
    q.lin_n_v_heads = hybrid ? e->lin_nv : 0;
    q.lin_head_k_dim = hybrid ? e->lin_hk : 0;
    q.lin_head_v_dim = hybrid ? e->lin_hv : 0;
    q.lin_conv_kernel = hybrid ? e->lin_kernel : 0;
    q.full_attn_interval = hybrid ? e->full_interval : 1;
    for (const LayerDev &L : e->layers) {
        if (L.kind == LK_LINEAR) q.n_linear++;
        else q.n_full++;
    }
    *out = q;
    return OI_OK;
}

int oi_engine_layer_types(const oi_engine *e, int32_t *out, int32_t n) {
    if (!e || (!out && n > 0)) return fail(OI_E_ARG, "null argument");
    if (n != (int32_t)e->layers.size())
        return fail(OI_E_ARG, "layer_types: " + std::to_string(n) + " entries for " +
                                  std::to_string(e->layers.size()) + " layers");
    for (int32_t l = 0; l < n; l++) out[l] = e->layers[(size_t)l].kind == LK_LINEAR ? 1 : 0;
    return OI_OK;
}

const float *oi_engine_forward(oi_engine *e, int32_t token, int32_t pos) {
    if (!e) {
        fail(OI_E_ARG, "null engine");
        return nullptr;
    }
    // infer/forward.odin:22-29
    if (pos < 0 || pos >= e->cfg.seq_len) {
        fail(OI_E_RANGE, "forward: pos=" + std::to_string(pos) + " out of range (seq_len=" +
                             std::to_string(e->cfg.seq_len) + ")");
        return nullptr;
    }
    if (token < 0 || token >= e->cfg.vocab_size) {
        fail(OI_E_RANGE, "forward: token=" + std::to_string(token) + " out of range (vocab=" +
                             std::to_string(e->cfg.vocab_size) + ")");
        return nullptr;
    }
    if (hipSetDevice(e->device) != hipSuccess || ensure_graph(e) || set_state(e, token, pos, 0) || run_token(e))
        return nullptr;
    hipError_t r = hipSuccess;
    if (r == hipSuccess)
        r = hipMemcpyAsync(e->logits_host, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost, e->stream);
    if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
    if (r != hipSuccess) {
        fail(OI_E_DEVICE, std::string("forward: ") + hipGetErrorString(r));
        return nullptr;
    }
    e->last_pos = pos;
    return e->logits_host;
}

// ------------------------------------------------------ batched prefill --
// Max tokens per batched chunk and the chunking rule of the reference
// (qwen3_5/metal.odin:22 MAX_BATCH_T; qwen3_5/engine.odin:66-93: chunks of a multiple
// of 8 tokens, the trailing 1-7 tokens one at a time).
constexpr int PF_MAX_T = 512;

namespace {

bool prefill_batched_ok(const oi_engine *e) {
    // every layout of the reference's batched path (the dense decoder and the
    // Qwen3.5 hybrid, forward_gpu_batch) and the routed-expert FFN; a layout
    // a kernel here does not take runs its prompt token by token (the
    // reference's fallback, qwen3_5/engine.odin:86-91)
    const oi_config &c = e->cfg;
    if ((c.head_dim != 128 && c.head_dim != 256) || c.dim > 16384) return false;
    for (const LayerDev &L : e->layers) {
        std::vector<const DMat *> g;
        if (L.kind == LK_LINEAR) {
            if (!pf_dn_supported((int)e->lin_hk, (int)e->lin_hv, (int)e->lin_kernel) || e->lin_nv % e->lin_nk) return false;
            g = {&L.in_qkv, &L.in_z, &L.in_b, &L.in_a, &L.ssm_out};
        } else {
            if (L.kind == LK_FULL && (e->rotary_dim > c.head_dim || e->rotary_dim % 2)) return false;
            g = {&L.wq, &L.wk, &L.wv, &L.wo};
        }
        if (!L.moe) {
            g.push_back(&L.w1); g.push_back(&L.w2); g.push_back(&L.w3);
        } else {
            const int32_t D = (int32_t)c.dim, EF = (int32_t)e->expert_ffn;
            if ((L.shared && !L.shared_merged) || e->n_experts + 1 > 1024 || e->top_k > MOE_MAX_K) return false;
            if (!mt_gemv_supported(L.router, D) || !mt_gemv_supported(L.gexp, D) || !mt_gemv_supported(L.uexp, D) ||
                !mt_gemv_supported(L.dexp, EF) || (L.shared && !mt_gemv_supported(L.sh_inp, D)))
                return false;
        }
        for (const DMat *m : g)
            if (!gemm_supported(*m)) return false;
    }
    return true;
}

size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

int prefill_alloc(oi_engine *e) {
    if (e->pf_mem) return OI_OK;
    const oi_config &c = e->cfg;
    const size_t T = PF_MAX_T, D = (size_t)c.dim, QD = (size_t)c.n_heads * c.head_dim, H = (size_t)c.hidden_dim;
    const size_t KD = (size_t)(e->lin_nk * e->lin_hk), VD = (size_t)(e->lin_nv * e->lin_hv), CD = 2 * KD + VD;
    bool full = false, lin = false, moe = false;
    // partial products: buffer 0 takes q, wo, gate, down, in_qkv and ssm_out,
    // buffer 1 k, up and in_z, buffer 2 v and in_b, buffer 3 in_a; each sized
    // for the largest K split of any chunk length
    size_t need[4] = {0, 0, 0, 0};
    for (const LayerDev &L : e->layers) {
        full |= L.kind == LK_FULL;
        lin |= L.kind == LK_LINEAR;
        moe |= L.moe;
        std::vector<std::pair<const DMat *, int>> uses;
        if (L.kind == LK_LINEAR) uses = {{&L.in_qkv, 0}, {&L.ssm_out, 0}, {&L.in_z, 1}, {&L.in_b, 2}, {&L.in_a, 3}};
        else uses = {{&L.wq, 0}, {&L.wo, 0}, {&L.wk, 1}, {&L.wv, 2}};
        if (!L.moe) {
            uses.push_back({&L.w1, 0}); uses.push_back({&L.w2, 0}); uses.push_back({&L.w3, 1});
        }
        for (const auto &u : uses)
            for (int n = 8; n <= PF_MAX_T; n += 8)
                need[u.second] = std::max(need[u.second],
                                          (size_t)gemm_split(*u.first, n, SIZE_MAX) * n * u.first->rows * 4);
    }
    need[0] = std::max(need[0], T * D * 4);  // the routed experts' weighted sums
    const size_t xb = T * std::max({D, QD, H, VD}) * 2;
    const size_t NE = (size_t)(e->n_experts + 1), KP = (size_t)(e->top_k + 1), EF = (size_t)e->expert_ffn;
    // work items: row tiles x pair slices, for either expert kernel
    size_t tg = 0, td = 0;
    if (moe) {
        const size_t rg = (size_t)mt_gemv_tile_rows((int32_t)D, (int32_t)EF), rd = (size_t)mt_gemv_tile_rows((int32_t)EF, (int32_t)D);
        tg = std::max((EF + rg - 1) / rg * (NE + (T * KP + MT_PAIR_SLICE - 1) / MT_PAIR_SLICE),
                      (EF + MT_MFMA_ROWS - 1) / MT_MFMA_ROWS * (NE + (T * KP + MT_MFMA_FEW - 1) / MT_MFMA_FEW));
        td = std::max((D + rd - 1) / rd * (NE + (T * KP + MT_PAIR_SLICE - 1) / MT_PAIR_SLICE),
                      (D + MT_MFMA_ROWS - 1) / MT_MFMA_ROWS * (NE + (T * KP + MT_MFMA_FEW - 1) / MT_MFMA_FEW));
    }
    std::vector<size_t> sizes = {T * 4, T * D * 4, T * QD * 4 * 2, xb, need[0], need[1], need[2], need[3],
                                 full ? T * QD * 4 : 0,
                                 lin ? T * CD * 4 : 0, lin ? T * 2 * KD * 4 : 0, lin ? T * 3 * (size_t)e->lin_nv * 4 : 0,
                                 lin ? T * VD * 4 : 0,
                                 lin ? pf_dc_scratch_floats((int)e->lin_nv, (int)T) * 4 : 0,
                                 moe ? T * D * 4 : 0, moe ? T * (size_t)e->n_experts * 4 : 0,
                                 moe ? T * KP * 4 : 0, moe ? T * KP * EF * 4 : 0, moe ? T * KP * EF * 4 : 0,
                                 moe ? T * KP * D * 4 : 0,
                                 moe ? T * KP * 4 : 0, moe ? T * KP * 4 : 0, moe ? NE * 4 : 0, moe ? NE * 4 : 0,
                                 moe ? NE * 4 : 0, 8 * tg, 8 * td, moe ? (size_t)8 : 0,
                                 moe ? (T + 2 * ((T + MT_MFMA_FEW - 1) / MT_MFMA_FEW) * 16 + 4) * 4 : 0,
                                 moe ? T * D * 4 : 0, moe ? T * (D / 32) * 4 : 0, moe ? T * 4 : 0};
    size_t total = 0;
    for (size_t b : sizes) total += al256(b);
    HIP_TRY(hipMalloc(&e->pf_mem, total));
    uint8_t *p = (uint8_t *)e->pf_mem;
    size_t k = 0;
    auto take = [&]() {
        uint8_t *r = sizes[k] ? p : nullptr;
        p += al256(sizes[k++]);
        return r;
    };
    e->pf_tok = (int32_t *)take();
    e->pf_x = (float *)take();
    e->pf_q = (float *)take();
    e->pf_xb = (uint16_t *)take();
    for (int i = 0; i < 4; i++) {
        e->pf_pbytes[i] = sizes[k];
        e->pf_p[i] = (float *)take();
    }
    e->pf_gate = (float *)take();
    e->pf_conv = (float *)take();
    e->pf_qk = (float *)take();
    e->pf_gates = (float *)take();
    e->pf_o = (float *)take();
    e->pf_dc = (float *)take();
    e->pf_xn = (float *)take();
    e->pf_lg = (float *)take();
    e->pf_w = (float *)take();
    e->pf_h = (float *)take();
    e->pf_h2 = (float *)take();
    e->pf_yd = (float *)take();
    e->pf_ids = (int32_t *)take();
    e->pf_list = (int32_t *)take();
    e->pf_off = (int32_t *)take();
    e->pf_cnt = (int32_t *)take();
    e->pf_fill = (int32_t *)take();
    e->pf_items_gu = (int32_t *)take();
    e->pf_items_dn = (int32_t *)take();
    e->pf_nitems = (int32_t *)take();
    e->pf_rt = (int32_t *)take();
    e->pf_rt_T = 0;
    e->pf_xq = take();
    e->pf_xq_sum = (float *)take();
    e->pf_xq_scale = (float *)take();
    return OI_OK;
}

// The routed-expert FFN of the chunk (no counterpart in the reference: its
// batched path has a dense MLP), in f32 as the per-token path: router logits
// (and the shared expert's gate logit) by a multi-token GEMV of the f32 norm
// output, softmax + top-k per token, the pairs grouped by expert, the chosen
// experts' SwiGLU rows and down rows per pair, their weighted sum per token
// into partial-product buffer 0.
// combine = false: the pair rows and weights stay in pf_yd / pf_w for the next
// residual add + norm, which sums them (launch_pf_addnorm16's myd)
// The MoE FFN's normalized rows are also quantized for the int8 router and
// gate/up items (by launch_pf_addnorm16, instead of by each item)
static bool pf_xq_used(const oi_engine *e) {
    const int64_t D = e->cfg.dim;
    return e->pf_xq_on && (e->pf_experts == 0 || e->pf_experts == 6) && e->pf_xq && D % 256 == 0 && D <= 4096;
}

int prefill_moe(oi_engine *e, const LayerDev &L, int T, bool combine = true) {
    const hipStream_t st = e->stream;
    const int32_t D = (int32_t)e->cfg.dim, E = (int32_t)e->n_experts, EF = (int32_t)e->expert_ffn;
    const int sx = L.shared_merged ? 1 : 0, KP = (int)e->top_k + sx, NE = E + sx;
    // router: slices of 8 tokens (the multi-token GEMV's x staging holds 8 rows
    // of 2048), so each workgroup stages its x once and the grid fills the GPU
    const int rps = D <= 2048 ? 8 : MT_PAIR_SLICE;
    const int slices = (T + rps - 1) / rps, pairs = T * KP;
    // the normalized rows, quantized once by the residual add + norm that
    // wrote them, for the int8 kernels below (router, gate/up)
    const bool xq = pf_xq_used(e);
    MtGemvArgs r{};
    r.m = L.router;
    r.K = D;
    r.rows = E;
    r.xdiv = 1;
    r.x = e->pf_xn;
    r.y = e->pf_lg;
    // on int8 MFMA (the experts' kernel, x to 2^-25 of its row maximum) in
    // items of 4 tokens and 128-row tiles where the router allows (200 tokens
    // of config 5: 62 -> 14 us per layer; the 2048-token prompt 489 -> 477 ms
    // at 64-token chunks, 198 -> 177 ms at 512), else the multi-token GEMV
    const int tiles_r = std::max(1, std::min(16, E / 128));
    const int px0 = e->pf_experts;
    if ((px0 == 0 || px0 == 6) && E % tiles_r == 0 && T <= 16 * MT_MFMA_FEW * 0x7FF &&
        mt_q4i8_supported(L.router, D, E / tiles_r)) {
        const int nsr = (T + MT_MFMA_FEW - 1) / MT_MFMA_FEW;
        int32_t *rl = e->pf_rt, *ri = rl + T, *rh = ri + 2 * nsr * 16;
        if (e->pf_rt_T != T) {  // the items depend on T only (tiles_r <= 16 fits the buffer)
            HIP_TRY(launch_pf_router_items(T, tiles_r, rl, ri, rh, st));
            e->pf_rt_T = T;
        }
        r.tiles = tiles_r;
        r.pair_slice = MT_MFMA_FEW;
        r.list = rl; r.items = ri; r.off = rh; r.cnt = rh + 1; r.nitems = rh + 2;
        if (xq) {
            r.xq = e->pf_xq; r.xq_sum = e->pf_xq_sum; r.xq_scale = e->pf_xq_scale;
        }
        HIP_TRY(launch_mt_q4i8(r, nsr * tiles_r, st));
    } else {
        r.tile_rows = std::max(1, mt_gemv_tile_rows(D, E) / 8);  // one pass of the lane groups: more workgroups
        r.tiles = (E + r.tile_rows - 1) / r.tile_rows;
        r.dense_n = T;
        r.pair_slice = rps;
        HIP_TRY(launch_mt_gemv(r, r.tiles * slices, st));
    }
    // the chosen experts on the matrix cores where their type allows (f32 MFMA),
    // else the multi-token GEMV
    const bool mm = e->pf_experts != 1 && mt_mfma_supported(L.gexp, D, EF) && mt_mfma_supported(L.uexp, D, EF) &&
                    L.gexp.type == L.uexp.type && mt_mfma_supported(L.dexp, EF, D);
    const int tr_gu = mm ? MT_MFMA_ROWS : mt_gemv_tile_rows(D, EF), tr_dn = mm ? MT_MFMA_ROWS : mt_gemv_tile_rows(EF, D);
    // few pairs per expert (a short chunk: ~1.4 at 64 tokens of top 10 of 512):
    // items of MT_MFMA_FEW pairs with the x rows staged once
    const int px = e->pf_experts;
    // int8 MFMA items stay ahead of the 16-pair f16 items at any chunk size
    // (200 tokens of config 5, ~4.3 pairs per expert: 304 against 669 us per
    // layer), so with it the few-pair items are used whatever the pair count
    const int tiles_qi = D % 128 == 0 ? 2 : 1, tiles_qg = EF % 128 == 0 ? 2 : 1;
    const bool i8_all = (px == 0 || px == 6) && mt_q4i8_supported(L.gexp, D, EF / tiles_qg) &&
                        mt_q4i8_supported(L.uexp, D, EF / tiles_qg) && mt_q4i8_supported(L.dexp, EF, D / tiles_qi);
    const bool few = mm && (px == 0 || px == 4 || px == 5 || px == 6) && L.gexp.type == T_Q4_K &&
                     L.dexp.type == T_Q4_K && (pairs <= MT_MFMA_FEW * NE || i8_all) && D <= 4096 && EF <= 4096 &&
                     D % MT_MFMA_ROWS == 0 && EF % MT_MFMA_ROWS == 0;
    const int ps = few ? MT_MFMA_FEW : mm ? MT_MFMA_PAIRS : MT_PAIR_SLICE;
    // few pairs, where the shapes allow: int8 planes of x on the matrix cores
    // with items of half the rows (64 tokens of config 5: gate/up 120 us, down
    // 58 us per layer, against 141 / 94 us on the token loop's int8 dot4
    // arithmetic); OI_PREFILL_EXPERTS=dot4: dot4, fewmfma: f16 MFMA
    const bool i8_gu = few && mt_q4i8_supported(L.gexp, D, EF / tiles_qg) && mt_q4i8_supported(L.uexp, D, EF / tiles_qg);
    const bool d4_gu = few && mt_dot4_supported(L.gexp, D, EF) && mt_dot4_supported(L.uexp, D, EF);
    const bool gu_i8 = i8_gu && (px == 0 || px == 6);
    const bool gu_d4 = !gu_i8 && d4_gu && (px == 0 || px == 5);
    const bool dn_i8 = few && mt_q4i8_supported(L.dexp, EF, D / tiles_qi) && (px == 0 || px == 6);
    const bool dn_d4 = !dn_i8 && few && mt_dot4_supported(L.dexp, EF, D) && (px == 0 || px == 5);
    PfMoeArgs ma{};
    ma.logits = e->pf_lg;
    if (L.shared) ma.sh_inp = L.sh_inp;
    ma.xn = e->pf_xn;
    ma.ids = e->pf_ids;
    ma.w = e->pf_w;
    ma.list = e->pf_list; ma.off = e->pf_off; ma.cnt = e->pf_cnt; ma.fill = e->pf_fill;
    ma.items_gu = e->pf_items_gu; ma.items_dn = e->pf_items_dn; ma.nitems = e->pf_nitems;
    ma.yd = e->pf_yd;
    ma.out = e->pf_p[0];
    ma.T = T; ma.n_experts = E; ma.top_k = (int32_t)e->top_k; ma.kp = KP;
    ma.norm_topk = 1;  // Qwen3-MoE / Qwen3-Next renormalize the chosen weights
    // a few-pair item covers every row tile, or half the rows on int8 MFMA
    ma.tiles_gu = gu_i8 ? tiles_qg : few ? 1 : (EF + tr_gu - 1) / tr_gu;
    ma.tiles_dn = dn_i8 ? tiles_qi : few ? 1 : (D + tr_dn - 1) / tr_dn;
    ma.dim = D;
    ma.pair_slice = ps;
    HIP_TRY(launch_pf_moe_route(ma, st));
    const int item_tiles = NE + (pairs + ps - 1) / ps;  // bound on the pair slices
    MtGemvArgs g{};
    g.m = L.gexp; g.m2 = L.uexp;
    g.swiglu = 1;
    g.K = D; g.rows = EF; g.xdiv = KP; g.tile_rows = tr_gu;
    g.x = e->pf_xn; g.y = e->pf_h;
    if (few) {  // gate rows to pf_h, up rows to pf_h2; the down launch applies the SwiGLU
        g.y2 = e->pf_h2;
        g.tiles = ma.tiles_gu;
    }
    g.list = e->pf_list; g.off = e->pf_off; g.cnt = e->pf_cnt;
    g.items = e->pf_items_gu; g.nitems = e->pf_nitems;
    g.pair_slice = ps;
    if (xq && gu_i8) {
        g.xq = e->pf_xq; g.xq_sum = e->pf_xq_sum; g.xq_scale = e->pf_xq_scale;
    }
    HIP_TRY(gu_i8 ? launch_mt_q4i8(g, item_tiles * ma.tiles_gu, st)
            : gu_d4 ? launch_mt_dot4(g, item_tiles, st)
            : mm ? launch_mt_mfma(g, item_tiles * ma.tiles_gu, st, e->pf_experts == 2)
                 : launch_mt_gemv(g, item_tiles * ma.tiles_gu, st));
    MtGemvArgs d{};
    d.m = L.dexp;
    d.K = EF; d.rows = D; d.xdiv = 1; d.tile_rows = tr_dn;
    d.x = e->pf_h; d.y = e->pf_yd;
    if (few) {
        d.x2 = e->pf_h2;
        d.tiles = ma.tiles_dn;
    }
    d.list = e->pf_list; d.off = e->pf_off; d.cnt = e->pf_cnt;
    d.items = e->pf_items_dn; d.nitems = e->pf_nitems + 1;
    d.pair_slice = ps;
    HIP_TRY(dn_i8 ? launch_mt_q4i8(d, item_tiles * ma.tiles_dn, st)
            : dn_d4 ? launch_mt_dot4(d, item_tiles, st)
            : mm ? launch_mt_mfma(d, item_tiles * ma.tiles_dn, st, e->pf_experts == 2)
                 : launch_mt_gemv(d, item_tiles * ma.tiles_dn, st));
    if (combine) HIP_TRY(launch_pf_moe_combine(ma, st));
    return OI_OK;
}

// One batched chunk of T tokens at positions pos .. pos+T-1 (forward_gpu_batch,
// qwen3_5/metal.odin:1472-1654): per layer the attention sublayer (Qwen3
// attention; Qwen3.5 full attention with the [q | gate] projection, partial
// RoPE and the sigmoid output gate; or the Qwen3.5 DeltaNet: conv, delta
// rule over the chunk's tokens in order, gated RMSNorm), then the FFN (dense
// SwiGLU, or routed experts), all over the T tokens; at the end the final
// norm and classifier of the last token.
// rows != nullptr: the classifier of every token of the chunk, token t's
// logits to rows + t * vocab (engine_verify_batch); otherwise the last token's
// logits to e->logits.
// Projections of the same f16 input into partial-product buffers P[idx[i]]
// (slice counts to split[i]): consecutive matrices of one type share a launch
// (launch_gemm_parts_multi; the same blocks and results as a launch each).
int prefill_projections(oi_engine *e, const DMat *const *m, const int *idx, int n, int T, int *split) {
    for (int i = 0; i < n;) {
        int j = i + 1;
        while (j < n && j - i < 4 && m[j]->type == m[i]->type && m[j]->cols == m[i]->cols) j++;
        float *part[4];
        size_t pb[4];
        for (int k = i; k < j; k++) {
            part[k - i] = e->pf_p[idx[k]];
            pb[k - i] = e->pf_pbytes[idx[k]];
        }
        if (j - i == 1) HIP_TRY(launch_gemm_parts(*m[i], e->pf_xb, T, part[0], pb[0], &split[i], e->stream));
        else HIP_TRY(launch_gemm_parts_multi(m + i, part, pb, j - i, e->pf_xb, T, split + i, e->stream));
        i = j;
    }
    return OI_OK;
}

int prefill_chunk(oi_engine *e, const int32_t *tokens, int T, int pos, float *rows = nullptr) {
    const hipStream_t st = e->stream;
    const oi_config &c = e->cfg;
    const int D = (int)c.dim, H = (int)c.hidden_dim, hd = (int)c.head_dim;
    const float eps = c.rms_eps;
    HIP_TRY(hipMemcpyAsync(e->pf_tok, tokens, (size_t)T * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(launch_embed_rows(e->tok_embd, e->pf_tok, T, e->pf_x, st));
    float *const *P = e->pf_p;
    const size_t *PB = e->pf_pbytes;
    // each residual add is fused with the next sublayer's RMSNorm
    HIP_TRY(launch_pf_addnorm16(e->pf_x, nullptr, 1, e->layers[0].attn_norm, eps, D, T, e->pf_xb, st));
    for (size_t l = 0; l < e->layers.size(); l++) {
        const LayerDev &L = e->layers[l];
        int qs = 1, ks = 1, vs = 1, s0 = 1, s1 = 1, s2 = 1, s3 = 1;
        if (L.kind == LK_QWEN3 || L.kind == LK_FULL) {
            const DMat *pm[3] = {&L.wq, &L.wk, &L.wv};
            const int pi[3] = {0, 1, 2};
            int sp[3];
            if (prefill_projections(e, pm, pi, 3, T, sp)) return -1;
            qs = sp[0]; ks = sp[1]; vs = sp[2];
        }
        if (L.kind == LK_QWEN3) {
            PfQkvArgs qa{P[0], P[1], P[2], qs, ks, vs, L.q_norm, L.k_norm, eps, e->rope_cs, L.kc, L.vc, e->pf_q,
                         T, pos, (int32_t)c.seq_len, (int32_t)c.n_heads, (int32_t)c.n_kv_heads};
            HIP_TRY(launch_pf_qkv(qa, hd, st));
            HIP_TRY(launch_pf_attn(e->pf_q, L.kc, L.vc, e->pf_xb, T, pos, (int)c.seq_len, (int)c.n_heads,
                                   (int)c.n_kv_heads, hd, st));
            HIP_TRY(launch_gemm_parts(L.wo, e->pf_xb, T, P[0], PB[0], &s0, st));
        } else if (L.kind == LK_FULL) {
            PfQ35Args qa{P[0], P[1], P[2], qs, ks, vs, L.q_norm, L.k_norm, e->inv_freq, eps, (int32_t)e->rotary_dim,
                         L.kc, L.vc, e->pf_q, e->pf_gate, T, pos, (int32_t)c.seq_len, (int32_t)c.n_heads,
                         (int32_t)c.n_kv_heads};
            HIP_TRY(launch_pf_q35_qkv(qa, hd, st));
            // the k / v partial products are consumed: their buffer is the
            // attention's scratch
            HIP_TRY(launch_pf_attn(e->pf_q, L.kc, L.vc, e->pf_xb, T, pos, (int)c.seq_len, (int)c.n_heads,
                                   (int)c.n_kv_heads, hd, st, e->pf_gate, P[1], PB[1]));
            HIP_TRY(launch_gemm_parts(L.wo, e->pf_xb, T, P[0], PB[0], &s0, st));
        } else {
            const DMat *pm[4] = {&L.in_qkv, &L.in_z, &L.in_b, &L.in_a};
            const int pi[4] = {0, 1, 2, 3};
            int sp[4];
            if (prefill_projections(e, pm, pi, 4, T, sp)) return -1;
            s0 = sp[0]; s1 = sp[1]; s2 = sp[2]; s3 = sp[3];
            PfDnArgs da{};
            da.qkv = P[0]; da.z = P[1]; da.b = P[2]; da.a = P[3];
            da.qkvs = s0; da.zs = s1; da.bs = s2; da.as = s3;
            da.conv_w = L.conv_w; da.a_decay = L.ssm_a; da.dt_bias = L.dt_bias; da.norm_w = L.ssm_norm;
            da.eps = eps;
            da.conv_state = L.conv_state;
            da.state = L.rec_state;
            da.conv_out = e->pf_conv; da.qk = e->pf_qk; da.gates = e->pf_gates; da.o = e->pf_o;
            da.out16 = e->pf_xb;  // the in_* projections have read it
            da.T = T;
            da.n_kh = (int32_t)e->lin_nk; da.n_vh = (int32_t)e->lin_nv;
            da.hk = (int32_t)e->lin_hk; da.hv = (int32_t)e->lin_hv; da.kernel = (int32_t)e->lin_kernel;
            da.chunk = e->pf_dn_chunk;
            da.dc = e->pf_dc;
            HIP_TRY(launch_pf_deltanet(da, st));
            HIP_TRY(launch_gemm_parts(L.ssm_out, e->pf_xb, T, P[0], PB[0], &s0, st));
        }
        const bool xq = L.moe && pf_xq_used(e);
        HIP_TRY(launch_pf_addnorm16(e->pf_x, P[0], s0, L.ffn_norm, eps, D, T, e->pf_xb, st,
                                    L.moe ? e->pf_xn : nullptr, nullptr, nullptr, 0, xq ? e->pf_xq : nullptr,
                                    e->pf_xq_sum, e->pf_xq_scale));
        const bool last = l + 1 == e->layers.size();
        if (L.moe) {
            if (prefill_moe(e, L, T, last)) return -1;
            s0 = 1;
            if (!last) {  // the expert combine summed in the next layer's residual add + norm
                const int KP = (int)e->top_k + (L.shared_merged ? 1 : 0);
                HIP_TRY(launch_pf_addnorm16(e->pf_x, nullptr, 1, e->layers[l + 1].attn_norm, eps, D, T, e->pf_xb, st,
                                            nullptr, e->pf_w, e->pf_yd, KP));
                continue;
            }
        } else if (e->pf_fused && gemm_swiglu_supported(L.w1, L.w3, T)) {
            // gate and up in one pass, SwiGLU in its epilogue; h goes to the up
            // partials' buffer (unsplit, it holds T x H floats)
            uint16_t *hb = (uint16_t *)P[1];
            HIP_TRY(launch_gemm_swiglu(L.w1, L.w3, e->pf_xb, T, hb, st));
            HIP_TRY(launch_gemm_parts(L.w2, hb, T, P[0], PB[0], &s0, st));
        } else {
            HIP_TRY(launch_gemm_parts(L.w1, e->pf_xb, T, P[0], PB[0], &s0, st));
            HIP_TRY(launch_gemm_parts(L.w3, e->pf_xb, T, P[1], PB[1], &s1, st));
            HIP_TRY(launch_pf_swiglu16(P[0], s0, P[1], s1, (int64_t)T * H, e->pf_xb, st));
            HIP_TRY(launch_gemm_parts(L.w2, e->pf_xb, T, P[0], PB[0], &s0, st));
        }
        if (l + 1 < e->layers.size())
            HIP_TRY(launch_pf_addnorm16(e->pf_x, P[0], s0, e->layers[l + 1].attn_norm, eps, D, T, e->pf_xb, st));
        else
            HIP_TRY(launch_pf_add(e->pf_x, P[0], s0, (int64_t)T * D, st));
    }
    // the final norm and classifier (qwen3_5/metal.odin:1637-1641 for the last token;
    // metal_verify_batch_logits, qwen3_5/metal.odin:1707-1747, for every token): the
    // decode path's f32 GEMV with the RMSNorm prologue, one row at a time
    for (int t = rows ? 0 : T - 1; t < T; t++) {
        GemvArgs a = gemv_args(GEMV_STORE, D, e->pf_x + (size_t)t * D, e->output_norm, eps);
        a.nseg = 1;
        a.seg[0].m = e->output;
        a.seg[0].y = rows ? rows + (size_t)t * c.vocab_size : e->logits;
        if (!plan_gemv(a)) return fail(OI_E_DEVICE, "internal: classifier plan");
        HIP_TRY(launch_gemv(a, st));
    }
    return OI_OK;
}

}  // namespace

namespace {

// engine_forward_batch over tokens[0, n) at pos0 (chunks of a multiple of 8
// up to PF_MAX_T batched, the trailing 1-7 through the decode path).  rows ==
// nullptr: the last token's logits in e->logits; otherwise every token's
// logits, token i at rows + i * vocab (device memory).  Returns 0 or a code.
int prefill_run(oi_engine *e, const int32_t *tokens, int32_t n, int32_t pos0, float *rows) {
    const char *what = rows ? "verify_batch" : "prefill";
    if (n <= 0) return fail(OI_E_ARG, std::string(what) + ": no tokens");
    if (pos0 < 0 || (int64_t)pos0 + n > e->cfg.seq_len)
        return fail(OI_E_RANGE, std::string(what) + ": positions [" + std::to_string(pos0) + ", " +
                                    std::to_string((int64_t)pos0 + n) + ") out of range (seq_len=" +
                                    std::to_string(e->cfg.seq_len) + ")");
    for (int32_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= e->cfg.vocab_size)
            return fail(OI_E_RANGE, std::string(what) + ": token=" + std::to_string(tokens[i]) +
                                        " out of range (vocab=" + std::to_string(e->cfg.vocab_size) + ")");
    if (hipSetDevice(e->device) != hipSuccess) return fail(OI_E_DEVICE, "hipSetDevice failed");
    const bool batched = prefill_batched_ok(e);
    if (batched && prefill_alloc(e)) return -1;
    if (ensure_graph(e)) return -1;
    const size_t V = (size_t)e->cfg.vocab_size;
    int i = 0;
    while (i < n) {
        const int rem = n - i;
        if (batched && rem >= 8) {
            int chunk = std::min(PF_MAX_T, rem);
            chunk -= chunk % 8;
            if (prefill_chunk(e, tokens + i, chunk, pos0 + i, rows ? rows + (size_t)i * V : nullptr)) return -1;
            i += chunk;
        } else {  // one token through the decode path
            if (set_state(e, tokens[i], pos0 + i, 0) || run_token(e)) return -1;
            hipError_t r = hipSuccess;
            if (rows) r = hipMemcpyAsync(rows + (size_t)i * V, e->logits, V * 4, hipMemcpyDeviceToDevice, e->stream);
            // the state copy reads pinned host memory when the stream reaches
            // it: the next token's state must not be written before that
            if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
            if (r != hipSuccess) return fail(OI_E_DEVICE, std::string(what) + ": " + hipGetErrorString(r));
            i += 1;
        }
    }
    return OI_OK;
}

}  // namespace

int32_t oi_engine_batch_max(void) { return PF_MAX_T; }

const float *oi_engine_verify_batch(oi_engine *e, const int32_t *tokens, int32_t n, int32_t pos0) {
    if (!e || !tokens) {
        fail(OI_E_ARG, "null argument");
        return nullptr;
    }
    if (n > 0 && n > e->vf_rows) {
        if (hipSetDevice(e->device) != hipSuccess) {
            fail(OI_E_DEVICE, "hipSetDevice failed");
            return nullptr;
        }
        if (e->vf_dev) hipFree(e->vf_dev);
        if (e->vf_host) hipHostFree(e->vf_host);
        e->vf_dev = e->vf_host = nullptr;
        e->vf_rows = 0;
        const size_t bytes = (size_t)n * (size_t)e->cfg.vocab_size * 4;
        if (hipMalloc((void **)&e->vf_dev, bytes) != hipSuccess ||
            hipHostMalloc((void **)&e->vf_host, bytes, hipHostMallocDefault) != hipSuccess) {
            fail(OI_E_NOMEM, "verify_batch: cannot allocate the logits of " + std::to_string(n) + " positions");
            return nullptr;
        }
        e->vf_rows = n;
    }
    if (prefill_run(e, tokens, n, pos0, e->vf_dev)) return nullptr;
    const size_t bytes = (size_t)n * (size_t)e->cfg.vocab_size * 4;
    hipError_t r = hipMemcpyAsync(e->vf_host, e->vf_dev, bytes, hipMemcpyDeviceToHost, e->stream);
    if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
    if (r != hipSuccess) {
        fail(OI_E_DEVICE, std::string("verify_batch: ") + hipGetErrorString(r));
        return nullptr;
    }
    e->last_pos = pos0 + n - 1;
    return e->vf_host;
}

const float *oi_engine_prefill(oi_engine *e, const int32_t *tokens, int32_t n, int32_t pos0) {
    if (!e || !tokens) {
        fail(OI_E_ARG, "null argument");
        return nullptr;
    }
    if (prefill_run(e, tokens, n, pos0, nullptr)) return nullptr;
    hipError_t r = hipMemcpyAsync(e->logits_host, e->logits, (size_t)e->cfg.vocab_size * 4, hipMemcpyDeviceToHost,
                                  e->stream);
    if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
    if (r != hipSuccess) {
        fail(OI_E_DEVICE, std::string("prefill: ") + hipGetErrorString(r));
        return nullptr;
    }
    e->last_pos = pos0 + n - 1;
    return e->logits_host;
}

int oi_engine_decode_greedy(oi_engine *e, int32_t token, int32_t pos, int32_t n_steps, int32_t *out_tokens) {
    if (!e || !out_tokens || n_steps < 0) return fail(OI_E_ARG, "bad argument");
    if (pos < 0 || (int64_t)pos + n_steps > e->cfg.seq_len)
        return fail(OI_E_RANGE, "decode: positions [" + std::to_string(pos) + ", " + std::to_string(pos + n_steps) +
                                    ") exceed seq_len=" + std::to_string(e->cfg.seq_len));
    if (token < 0 || token >= e->cfg.vocab_size) return fail(OI_E_RANGE, "decode: token out of range");
    if (n_steps == 0) return OI_OK;
    HIP_TRY(hipSetDevice(e->device));
    int rc = ensure_graph(e);
    if (rc) return rc;
    if ((rc = set_state(e, token, pos, n_steps))) return rc;
    for (int i = 0; i < n_steps; i++)
        if ((rc = run_token(e))) return rc;
    // the last step's argmax is still pending: reduce it
    HIP_TRY(launch_embed(e->tok_embd, e->state, e->x, (int32_t)e->cfg.vocab_size, e->am_val, e->am_idx, e->tokens,
                         1, e->stream));
    HIP_TRY(hipMemcpyAsync(out_tokens, e->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, e->stream));
    HIP_TRY(hipStreamSynchronize(e->stream));
    e->last_pos = pos + n_steps - 1;
    return OI_OK;
}

static_assert(sizeof(oi_sampler) == sizeof(SampleState) && offsetof(oi_sampler, rng_state) == offsetof(SampleState, rng) &&
                  offsetof(oi_sampler, last) == offsetof(SampleState, last),
              "oi_sampler is copied to the device as SampleState");

int oi_engine_decode_sample(oi_engine *e, int32_t token, int32_t pos, int32_t n_steps, oi_sampler *s,
                            int32_t *out_tokens) {
    if (!e) return fail(OI_E_ARG, "null engine");
    if (!s || (n_steps > 0 && !out_tokens) || n_steps < 0) return fail(OI_E_ARG, "bad argument");
    if (pos < 0 || (int64_t)pos + n_steps > e->cfg.seq_len)
        return fail(OI_E_RANGE, "decode: positions [" + std::to_string(pos) + ", " + std::to_string(pos + n_steps) +
                                    ") exceed seq_len=" + std::to_string(e->cfg.seq_len));
    if (token < 0 || token >= e->cfg.vocab_size) return fail(OI_E_RANGE, "decode: token out of range");
    if (s->n_last < 0 || s->n_last > SAMPLE_WINDOW) return fail(OI_E_ARG, "sampler: n_last outside [0, 64]");
    if (e->cfg.vocab_size > sample_max_vocab())
        return fail(OI_E_UNSUPPORTED, "sampler: vocabulary larger than " + std::to_string(sample_max_vocab()));
    if (n_steps == 0) return OI_OK;
    HIP_TRY(hipSetDevice(e->device));
    const int V = (int)e->cfg.vocab_size;
    // the token step followed by the sampler's launches for this mode,
    // captured once per mode
    const int mode = sample_mode(s->temperature, s->topp, V);
    if (e->use_graph && !e->gexec_s[mode]) {
        HIP_TRY(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_token(e);
        const hipError_t le = rc ? hipSuccess
                                 : launch_sample(e->logits, e->samp_p, V, e->samp, mode, e->samp_work, e->state,
                                                 e->tokens, nullptr, e->stream);
        hipGraph_t g = nullptr;
        const hipError_t ec = hipStreamEndCapture(e->stream, &g);
        if (rc) return rc;
        if (le != hipSuccess) return fail(OI_E_DEVICE, std::string("launch_sample: ") + hipGetErrorString(le));
        if (ec != hipSuccess) return fail(OI_E_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(ec));
        e->graph_s[mode] = g;
        HIP_TRY(hipGraphInstantiate(&e->gexec_s[mode], g, nullptr, nullptr, 0));
    }
    HIP_TRY(hipMemcpyAsync(e->samp, s, sizeof(SampleState), hipMemcpyHostToDevice, e->stream));
    int rc = set_state(e, token, pos, n_steps);
    if (rc) return rc;
    for (int i = 0; i < n_steps; i++) {
        if (e->use_graph) {
            HIP_TRY(hipGraphLaunch(e->gexec_s[mode], e->stream));
        } else {
            if ((rc = enqueue_token(e))) return rc;
            HIP_TRY(launch_sample(e->logits, e->samp_p, V, e->samp, mode, e->samp_work, e->state, e->tokens, nullptr,
                                  e->stream));
        }
    }
    HIP_TRY(hipMemcpyAsync(out_tokens, e->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, e->stream));
    HIP_TRY(hipMemcpyAsync(s, e->samp, sizeof(SampleState), hipMemcpyDeviceToHost, e->stream));
    HIP_TRY(hipStreamSynchronize(e->stream));
    e->last_pos = pos + n_steps - 1;
    return OI_OK;
}

int oi_sample(const float *logits, int32_t n, oi_sampler *s, int32_t *out_token) {
    if (!logits || !s || !out_token || n <= 0) return fail(OI_E_ARG, "bad argument");
    if (n > sample_max_vocab()) return fail(OI_E_UNSUPPORTED, "sampler: n larger than " + std::to_string(sample_max_vocab()));
    if (s->n_last < 0 || s->n_last > SAMPLE_WINDOW) return fail(OI_E_ARG, "sampler: n_last outside [0, 64]");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    const size_t lb = (size_t)n * 4, al = (lb + 255) & ~(size_t)255, wb = (sample_work_bytes() + 255) & ~(size_t)255;
    uint8_t *buf = nullptr;
    HIP_TRY(hipMalloc((void **)&buf, 2 * al + wb + sizeof(SampleState) + 256));
    std::unique_ptr<uint8_t, void (*)(uint8_t *)> guard(buf, [](uint8_t *b) { (void)hipFree(b); });
    float *dl = (float *)buf, *dp = (float *)(buf + al);
    void *work = buf + 2 * al;
    SampleState *ds = (SampleState *)(buf + 2 * al + wb);
    int32_t *dpick = (int32_t *)(buf + 2 * al + wb + sizeof(SampleState));
    HIP_TRY(hipMemcpy(dl, logits, lb, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(ds, s, sizeof(SampleState), hipMemcpyHostToDevice));
    HIP_TRY(launch_sample(dl, dp, n, ds, sample_mode(s->temperature, s->topp, n), work, nullptr, nullptr, dpick,
                          nullptr));
    HIP_TRY(hipMemcpy(out_token, dpick, 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(s, ds, sizeof(SampleState), hipMemcpyDeviceToHost));
    return OI_OK;
}

int oi_engine_kv_fill(oi_engine *e, int32_t layer0, int32_t nlayers, int32_t pos0, int32_t npos, const uint16_t *k,
                      const uint16_t *v) {
    if (!e || !k || !v) return fail(OI_E_ARG, "null argument");
    const oi_config &c = e->cfg;
    if (layer0 < 0 || nlayers < 0 || layer0 + nlayers > c.n_layers || pos0 < 0 || npos < 0 ||
        (int64_t)pos0 + npos > c.seq_len)
        return fail(OI_E_RANGE, "kv_fill range out of bounds");
    HIP_TRY(hipSetDevice(e->device));
    const size_t hd = (size_t)c.head_dim;
    for (int l = 0; l < nlayers; l++)
        for (int h = 0; h < c.n_kv_heads && e->layers[(size_t)(layer0 + l)].kc; h++) {  // DeltaNet layers: no cache
            const size_t src = (((size_t)l * c.n_kv_heads + h) * npos) * hd;
            const size_t dst = ((size_t)h * c.seq_len + pos0) * hd;
            HIP_TRY(hipMemcpyAsync(e->layers[(size_t)(layer0 + l)].kc + dst, k + src, (size_t)npos * hd * 2,
                                   hipMemcpyHostToDevice, e->stream));
            HIP_TRY(hipMemcpyAsync(e->layers[(size_t)(layer0 + l)].vc + dst, v + src, (size_t)npos * hd * 2,
                                   hipMemcpyHostToDevice, e->stream));
        }
    HIP_TRY(hipStreamSynchronize(e->stream));
    return OI_OK;
}

int oi_engine_reset_state(oi_engine *e) {
    if (!e) return fail(OI_E_ARG, "null engine");
    HIP_TRY(hipSetDevice(e->device));
    const oi_config &c = e->cfg;
    const size_t kv_layer = (size_t)c.n_kv_heads * c.seq_len * c.head_dim * 2;
    const size_t conv_layer = (size_t)(2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv) *
                              (e->lin_kernel > 0 ? e->lin_kernel - 1 : 0) * 4;
    const size_t rec_layer = (size_t)e->lin_nv * e->lin_hk * e->lin_hv * 4;
    for (const LayerDev &L : e->layers) {
        if (L.kc) HIP_TRY(hipMemsetAsync(L.kc, 0, kv_layer, e->stream));
        if (L.vc) HIP_TRY(hipMemsetAsync(L.vc, 0, kv_layer, e->stream));
        if (L.conv_state && conv_layer) HIP_TRY(hipMemsetAsync(L.conv_state, 0, conv_layer, e->stream));
        if (L.rec_state) HIP_TRY(hipMemsetAsync(L.rec_state, 0, rec_layer, e->stream));
    }
    HIP_TRY(hipStreamSynchronize(e->stream));
    e->last_pos = 0;
    return OI_OK;
}

const float *oi_engine_logits_device(oi_engine *e) { return e ? e->logits : nullptr; }
void *oi_engine_stream(oi_engine *e) { return e ? (void *)e->stream : nullptr; }

int oi_engine_time_kernel(oi_engine *e, int32_t kernel, int32_t iters, double *avg_us, double *bytes) {
    if (!e || !avg_us || !bytes || iters <= 0 || kernel < K_QKV || kernel > K_LAST)
        return fail(OI_E_ARG, "bad argument");
    if (kernel == K_TOKEN) return time_token(e, iters, avg_us, bytes);
    HIP_TRY(hipSetDevice(e->device));
    const oi_config &c = e->cfg;
    // the launches of this role in every layer, in layer order
    std::vector<const Op *> sel;
    for (const auto &layer : e->ops)
        for (const Op &o : layer)
            if (o.role == kernel) sel.push_back(&o);
    Op out;
    if (kernel == K_OUTPUT) {
        out.g = e->g_out;
        size_t b = 0;
        matrix_bytes((uint32_t)e->output.type, e->output.rows, e->output.cols, b);
        out.bytes = (double)b + 8.0 * c.dim + 4.0 * c.vocab_size;
        sel.push_back(&out);
    }
    if (sel.empty()) return fail(OI_E_ARG, "this model has no launch of that kernel");
    const double pos = e->last_pos;
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    auto run = [&]() -> int {
        for (int it = 0; it < iters; it++) {
            const hipError_t r = launch_op(e, *sel[(size_t)it % sel.size()], e->stream);
            if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("launch: ") + hipGetErrorString(r));
        }
        return OI_OK;
    };
    int rc;
    if ((rc = set_state(e, 0, e->last_pos, 0))) return rc;
    if ((rc = run())) return rc;
    HIP_TRY(hipEventRecord(e0, e->stream));
    if ((rc = run())) return rc;
    HIP_TRY(hipEventRecord(e1, e->stream));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    *avg_us = ms * 1000.0 / iters;
    // mean algorithmic bytes over the launches timed; attention adds the
    // cache rows read at the timed position
    double total = 0;
    for (int it = 0; it < iters; it++) {
        const Op &o = *sel[(size_t)it % sel.size()];
        double b = o.bytes;
        if (o.kind == OP_ATTN || o.kind == OP_Q35) b += 2.0 * c.n_kv_heads * c.head_dim * 2 * (pos + 1);
        total += b;
    }
    *bytes = total / iters;
    return OI_OK;
}

// ------------------------------------------------------------ kernel hooks --

struct oi_weights {
    DMat m{};
    uint8_t *dev = nullptr;
    size_t bytes = 0;
};

int oi_weights_upload(int32_t type, const void *host_blocks, int64_t rows, int64_t cols, oi_weights **out) {
    if (!host_blocks || !out || rows <= 0 || cols <= 0 || rows > INT32_MAX || cols > 15360)
        return fail(OI_E_ARG, "bad argument");
    if (!device_type_ok((uint32_t)type)) return fail(OI_E_UNSUPPORTED, "type not supported by the GEMV kernels");
    if (cols % 64 || ((type == T_Q4_K || type == T_Q6_K) && cols % 256))
        return fail(OI_E_ARG, "cols must be a multiple of 64 (256 for K-quants)");
    int rc = check_device(0);
    if (rc) return rc;
    std::unique_ptr<oi_weights> w(new oi_weights());
    if (!matrix_bytes((uint32_t)type, rows, cols, w->bytes)) return fail(OI_E_ARG, "bad size");
    if (hipMalloc(&w->dev, w->bytes) != hipSuccess) return fail(OI_E_NOMEM, "hipMalloc failed");
    std::vector<uint8_t> stage;
    rc = upload_matrix((uint32_t)type, (const uint8_t *)host_blocks, rows, cols, w->dev, nullptr, stage, w->m);
    if (rc) {
        hipFree(w->dev);
        return rc;
    }
    *out = w.release();
    return OI_OK;
}

void oi_weights_free(oi_weights *w) {
    if (!w) return;
    if (w->dev) hipFree(w->dev);
    delete w;
}

int64_t oi_weights_bytes(const oi_weights *w) { return w ? (int64_t)w->bytes : 0; }

int oi_gemv_launch(const oi_weights *w, const float *x_dev, float *y_dev, void *stream) {
    if (!w || !x_dev || !y_dev) return fail(OI_E_ARG, "null argument");
    GemvArgs a = gemv_args(GEMV_STORE, w->m.cols, x_dev, nullptr, 0.f);
    a.nseg = 1;
    a.seg[0].m = w->m;
    a.seg[0].y = y_dev;
    if (!plan_gemv(a)) return fail(OI_E_ARG, "cols not a multiple of 64");
    hipError_t r = launch_gemv(a, (hipStream_t)stream);
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("gemv launch: ") + hipGetErrorString(r));
    return OI_OK;
}

int64_t oi_gemm_workspace_bytes(const oi_weights *w, int32_t n) {
    if (!w || n <= 0 || !gemm_supported(w->m)) return 0;
    const int split = gemm_split(w->m, n, SIZE_MAX);
    return split > 1 ? (int64_t)split * n * w->m.rows * 4 : 0;
}

int oi_gemm_launch(const oi_weights *w, const uint16_t *x_dev, int32_t n, float *c_dev, void *workspace,
                   int64_t workspace_bytes, void *stream) {
    if (!w || !x_dev || !c_dev) return fail(OI_E_ARG, "null argument");
    if (n <= 0) return fail(OI_E_ARG, "n must be positive");
    if (workspace_bytes < 0) return fail(OI_E_ARG, "negative workspace size");
    if (!gemm_supported(w->m)) return fail(OI_E_UNSUPPORTED, "type / row length not supported by the GEMM kernel");
    const hipError_t r = launch_gemm(w->m, x_dev, n, c_dev, (float *)workspace, workspace ? (size_t)workspace_bytes : 0,
                                     (hipStream_t)stream);
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("gemm launch: ") + hipGetErrorString(r));
    return OI_OK;
}

int oi_gemm(int32_t type, const void *host_blocks, int64_t rows, int64_t cols, const uint16_t *x, int32_t n,
            float *c) {
    if (!x || !c) return fail(OI_E_ARG, "null argument");
    if (n <= 0) return fail(OI_E_ARG, "n must be positive");
    oi_weights *w = nullptr;
    int rc = oi_weights_upload(type, host_blocks, rows, cols, &w);
    if (rc) return rc;
    uint16_t *dx = nullptr;
    float *dc = nullptr;
    void *ws = nullptr;
    const int64_t wsb = oi_gemm_workspace_bytes(w, n);
    hipError_t r = hipMalloc(&dx, (size_t)n * cols * 2);
    if (r == hipSuccess) r = hipMalloc(&dc, (size_t)n * rows * 4);
    if (r == hipSuccess && wsb) r = hipMalloc(&ws, (size_t)wsb);
    if (r == hipSuccess) r = hipMemcpy(dx, x, (size_t)n * cols * 2, hipMemcpyHostToDevice);
    if (r == hipSuccess) {
        rc = oi_gemm_launch(w, dx, n, dc, ws, wsb, nullptr);
        if (!rc) r = hipMemcpy(c, dc, (size_t)n * rows * 4, hipMemcpyDeviceToHost);
    }
    if (dx) hipFree(dx);
    if (dc) hipFree(dc);
    if (ws) hipFree(ws);
    oi_weights_free(w);
    if (rc) return rc;
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("gemm: ") + hipGetErrorString(r));
    return OI_OK;
}

int oi_gemv(int32_t type, const void *host_blocks, int64_t rows, int64_t cols, const float *x, float *y) {
    if (!x || !y) return fail(OI_E_ARG, "null argument");
    oi_weights *w = nullptr;
    int rc = oi_weights_upload(type, host_blocks, rows, cols, &w);
    if (rc) return rc;
    float *dx = nullptr, *dy = nullptr;
    hipError_t r = hipMalloc(&dx, (size_t)cols * 4);
    if (r == hipSuccess) r = hipMalloc(&dy, (size_t)rows * 4);
    if (r == hipSuccess) r = hipMemcpy(dx, x, (size_t)cols * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) {
        rc = oi_gemv_launch(w, dx, dy, nullptr);
        if (!rc) r = hipMemcpy(y, dy, (size_t)rows * 4, hipMemcpyDeviceToHost);
    }
    if (dx) hipFree(dx);
    if (dy) hipFree(dy);
    oi_weights_free(w);
    if (rc) return rc;
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("gemv: ") + hipGetErrorString(r));
    return OI_OK;
}

int oi_dequant(int32_t type, const void *blocks, int64_t n, float *out) {
    if (!blocks || !out || n <= 0) return fail(OI_E_ARG, "bad argument");
    if (!device_type_ok((uint32_t)type)) return fail(OI_E_UNSUPPORTED, "type not supported on the device");
    // one row of n elements; the kernels work in units of 64
    if (n % 64 || ((type == T_Q4_K || type == T_Q6_K) && n % 256))
        return fail(OI_E_ARG, "n must be a multiple of 64 (256 for K-quants)");
    // long inputs are cut into rows of at most 15360 elements
    int64_t cols = n;
    while (cols > 15360 && cols % 2 == 0 && (cols / 2) % 256 == 0) cols /= 2;
    const int64_t rows = n / cols;
    oi_weights *w = nullptr;
    int rc = oi_weights_upload(type, blocks, rows, cols, &w);
    if (rc) return rc;
    float *dy = nullptr;
    hipError_t r = hipMalloc(&dy, (size_t)n * 4);
    if (r == hipSuccess) r = launch_dequant(w->m, dy, nullptr);
    if (r == hipSuccess) r = hipMemcpy(out, dy, (size_t)n * 4, hipMemcpyDeviceToHost);
    if (dy) hipFree(dy);
    oi_weights_free(w);
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("dequant: ") + hipGetErrorString(r));
    return OI_OK;
}


}  // extern "C"

// ------------------------------------------------- gated DeltaNet step --
namespace {
bool dn_dims_ok(const oi_deltanet_dims *d) {
    return d && d->n_k_heads > 0 && d->n_v_heads > 0 && d->n_v_heads % d->n_k_heads == 0 && d->head_k_dim == 128 &&
           d->head_v_dim == 128 && d->conv_kernel >= 1 && d->conv_kernel <= 16;
}
DnArgs dn_args(const oi_deltanet_dims *d) {
    DnArgs a{};
    a.eps = d->eps;
    a.n_kh = d->n_k_heads;
    a.n_vh = d->n_v_heads;
    a.hk = d->head_k_dim;
    a.hv = d->head_v_dim;
    a.kernel = d->conv_kernel;
    return a;
}
}  // namespace

int oi_deltanet_step_launch(const oi_deltanet_dims *d, const float *qkv, const float *z, const float *b,
                            const float *a, const float *conv_w, const float *a_decay, const float *dt_bias,
                            const float *norm_w, float *conv_state, float *rec_state, float *scratch, float *out,
                            void *stream) {
    if (!dn_dims_ok(d)) return fail(OI_E_ARG, "deltanet: head dims must be 128, n_v_heads a multiple of n_k_heads");
    if (!qkv || !z || !b || !a || !conv_w || !a_decay || !dt_bias || !norm_w || !rec_state || !scratch || !out ||
        (d->conv_kernel > 1 && !conv_state))
        return fail(OI_E_ARG, "null argument");
    DnArgs g = dn_args(d);
    g.qkv = qkv; g.z = z; g.b = b; g.a = a;
    g.conv_w = conv_w; g.a_decay = a_decay; g.dt_bias = dt_bias; g.norm_w = norm_w;
    g.conv_state = conv_state; g.state = rec_state; g.conv_out = scratch; g.out = out;
    HIP_TRY(launch_deltanet(g, (hipStream_t)stream));
    return OI_OK;
}

int oi_deltanet_steps(const oi_deltanet_dims *d, int32_t n_tokens, const float *qkv, const float *z, const float *b,
                      const float *a, const float *conv_w, const float *a_decay, const float *dt_bias,
                      const float *norm_w, float *conv_state, float *rec_state, float *out) {
    if (!dn_dims_ok(d)) return fail(OI_E_ARG, "deltanet: head dims must be 128, n_v_heads a multiple of n_k_heads");
    if (n_tokens <= 0 || !qkv || !z || !b || !a || !conv_w || !a_decay || !dt_bias || !norm_w || !rec_state || !out ||
        (d->conv_kernel > 1 && !conv_state))
        return fail(OI_E_ARG, "bad argument");
    const size_t kd = (size_t)d->n_k_heads * d->head_k_dim, vd = (size_t)d->n_v_heads * d->head_v_dim;
    const size_t cd = 2 * kd + vd, nvh = (size_t)d->n_v_heads, km1 = (size_t)d->conv_kernel - 1;
    const size_t st_n = nvh * d->head_k_dim * d->head_v_dim;
    // one device block: inputs of all tokens, parameters, states, scratch, outputs
    const size_t n = (size_t)n_tokens;
    const size_t floats = n * (cd + vd + 2 * nvh) + cd * d->conv_kernel + 2 * nvh + d->head_v_dim + cd * km1 + st_n +
                          cd + n * vd;
    float *dev = nullptr;
    HIP_TRY(hipMalloc(&dev, floats * 4));
    float *p = dev;
    auto put = [&](const float *src, size_t cnt) {
        float *r = p;
        p += cnt;
        return std::make_pair(r, src ? hipMemcpy(r, src, cnt * 4, hipMemcpyHostToDevice) : hipSuccess);
    };
    hipError_t r = hipSuccess;
    float *dq, *dz, *db, *da, *dcw, *dad, *ddt, *dnw, *dcs, *drs, *dsc, *dout;
    {
        auto t = put(qkv, n * cd); dq = t.first; r = t.second;
        if (r == hipSuccess) { t = put(z, n * vd); dz = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(b, n * nvh); db = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(a, n * nvh); da = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(conv_w, cd * d->conv_kernel); dcw = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(a_decay, nvh); dad = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(dt_bias, nvh); ddt = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(norm_w, d->head_v_dim); dnw = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(km1 ? conv_state : nullptr, cd * km1); dcs = t.first; r = t.second; }
        if (r == hipSuccess) { t = put(rec_state, st_n); drs = t.first; r = t.second; }
        if (r == hipSuccess) { dsc = p; p += cd; dout = p; }
    }
    int rc = OI_OK;
    for (size_t i = 0; r == hipSuccess && !rc && i < n; i++)
        rc = oi_deltanet_step_launch(d, dq + i * cd, dz + i * vd, db + i * nvh, da + i * nvh, dcw, dad, ddt, dnw, dcs,
                                     drs, dsc, dout + i * vd, nullptr);
    if (r == hipSuccess && !rc) r = hipMemcpy(out, dout, n * vd * 4, hipMemcpyDeviceToHost);
    if (r == hipSuccess && !rc && km1) r = hipMemcpy(conv_state, dcs, cd * km1 * 4, hipMemcpyDeviceToHost);
    if (r == hipSuccess && !rc) r = hipMemcpy(rec_state, drs, st_n * 4, hipMemcpyDeviceToHost);
    hipFree(dev);
    if (rc) return rc;
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("deltanet: ") + hipGetErrorString(r));
    return OI_OK;
}

int oi_deltanet_steps_batched(const oi_deltanet_dims *d, int32_t n_tokens, int32_t chunk, const float *qkv,
                              const float *z, const float *b, const float *a, const float *conv_w,
                              const float *a_decay, const float *dt_bias, const float *norm_w, float *conv_state,
                              float *rec_state, float *out) {
    if (!dn_dims_ok(d) || !pf_dn_supported(d->head_k_dim, d->head_v_dim, d->conv_kernel))
        return fail(OI_E_ARG, "deltanet batched: head dims 128, conv kernel 4, n_v_heads a multiple of n_k_heads");
    if (chunk != 0 && chunk != 16 && chunk != 32 && chunk != 64)
        return fail(OI_E_ARG, "deltanet batched: chunk must be 0, 16, 32 or 64");
    if (n_tokens < d->conv_kernel - 1 || !qkv || !z || !b || !a || !conv_w || !a_decay || !dt_bias || !norm_w ||
        !conv_state || !rec_state || !out)
        return fail(OI_E_ARG, "deltanet batched: bad argument (n_tokens must be at least conv_kernel - 1)");
    const size_t n = (size_t)n_tokens, nvh = (size_t)d->n_v_heads, kd = (size_t)d->n_k_heads * d->head_k_dim;
    const size_t vd = nvh * d->head_v_dim, cd = 2 * kd + vd, km1 = (size_t)d->conv_kernel - 1;
    const size_t st_n = nvh * d->head_k_dim * d->head_v_dim;
    // inputs, parameters, states, then the kernels' scratch (conv out, q/k, gates, o) and out
    const size_t in_f[] = {n * cd, n * vd, n * nvh, n * nvh, cd * d->conv_kernel, nvh, nvh, (size_t)d->head_v_dim,
                           cd * km1, st_n};
    const float *in_p[] = {qkv, z, b, a, conv_w, a_decay, dt_bias, norm_w, conv_state, rec_state};
    const size_t dcf = chunk == 64 ? pf_dc_scratch_floats((int)nvh, (int)n) : 0;
    size_t floats = n * cd + n * 2 * kd + n * 3 * nvh + n * vd + n * vd + dcf;
    for (size_t x : in_f) floats += x;
    float *dev = nullptr;
    HIP_TRY(hipMalloc(&dev, floats * 4));
    float *dp[10], *p = dev;
    hipError_t r = hipSuccess;
    for (int i = 0; i < 10; i++) {
        dp[i] = p;
        p += in_f[i];
        if (r == hipSuccess) r = hipMemcpy(dp[i], in_p[i], in_f[i] * 4, hipMemcpyHostToDevice);
    }
    PfDnArgs da{};
    da.qkv = dp[0]; da.z = dp[1]; da.b = dp[2]; da.a = dp[3];
    da.qkvs = da.zs = da.bs = da.as = 1;
    da.conv_w = dp[4]; da.a_decay = dp[5]; da.dt_bias = dp[6]; da.norm_w = dp[7];
    da.eps = d->eps;
    da.conv_state = dp[8]; da.state = dp[9];
    da.conv_out = p; p += n * cd;
    da.qk = p; p += n * 2 * kd;
    da.gates = p; p += n * 3 * nvh;
    da.o = p; p += n * vd;
    da.dc = dcf ? p : nullptr; p += dcf;
    da.out32 = p;
    da.T = n_tokens;
    da.n_kh = d->n_k_heads; da.n_vh = d->n_v_heads;
    da.hk = d->head_k_dim; da.hv = d->head_v_dim; da.kernel = d->conv_kernel;
    da.chunk = chunk;
    if (r == hipSuccess) r = launch_pf_deltanet(da, nullptr);
    if (r == hipSuccess) r = hipMemcpy(out, da.out32, n * vd * 4, hipMemcpyDeviceToHost);
    if (r == hipSuccess) r = hipMemcpy(conv_state, dp[8], cd * km1 * 4, hipMemcpyDeviceToHost);
    if (r == hipSuccess) r = hipMemcpy(rec_state, dp[9], st_n * 4, hipMemcpyDeviceToHost);
    hipFree(dev);
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("deltanet batched: ") + hipGetErrorString(r));
    return OI_OK;
}

// ------------------------------------------------ Qwen3.5 full attention --
namespace {
bool q35_dims_ok(const oi_qwen35_attn_dims *d) {
    return d && d->n_heads > 0 && d->n_kv_heads > 0 && d->n_heads % d->n_kv_heads == 0 &&
           (d->head_dim == 128 || d->head_dim == 256) && d->rotary_dim >= 0 && d->rotary_dim <= d->head_dim &&
           d->rotary_dim % 2 == 0 && d->seq_len > 0;
}
}  // namespace

int64_t oi_qwen35_attn_workspace_bytes(const oi_qwen35_attn_dims *d) {
    if (!q35_dims_ok(d)) return 0;
    return ((int64_t)d->n_heads * d->head_dim + (int64_t)d->n_heads * q35_max_splits(d->seq_len) * (d->head_dim + 2)) *
           4;
}

int oi_qwen35_attn_step_launch(const oi_qwen35_attn_dims *d, int32_t pos, const float *qproj, const float *k,
                               const float *v, const float *q_norm, const float *k_norm, const float *inv_freq,
                               uint16_t *k_cache, uint16_t *v_cache, void *workspace, float *out, void *stream) {
    if (!q35_dims_ok(d)) return fail(OI_E_ARG, "qwen35 attention: bad dims");
    if (pos < 0 || pos >= d->seq_len)
        return fail(OI_E_RANGE, "qwen35 attention: pos=" + std::to_string(pos) + " out of range (seq_len=" +
                                    std::to_string(d->seq_len) + ")");
    if (!qproj || !k || !v || !q_norm || !k_norm || (d->rotary_dim && !inv_freq) || !k_cache || !v_cache ||
        !workspace || !out)
        return fail(OI_E_ARG, "null argument");
    Q35Args a{};
    a.qproj = qproj; a.k = k; a.v = v; a.q_norm = q_norm; a.k_norm = k_norm; a.inv_freq = inv_freq;
    a.eps = d->eps; a.rotary_dim = d->rotary_dim; a.pos = pos; a.seq_len = d->seq_len;
    a.n_heads = d->n_heads; a.n_kv_heads = d->n_kv_heads; a.max_splits = q35_max_splits(d->seq_len);
    a.kc = k_cache; a.vc = v_cache;
    a.qbuf = (float *)workspace;
    a.part = a.qbuf + (size_t)d->n_heads * d->head_dim;
    a.out = out;
    HIP_TRY(launch_q35_attn(a, d->head_dim, (hipStream_t)stream));
    return OI_OK;
}

int oi_qwen35_attn_steps(const oi_qwen35_attn_dims *d, int32_t n_tokens, int32_t pos0, const float *qproj,
                         const float *k, const float *v, const float *q_norm, const float *k_norm,
                         const float *inv_freq, uint16_t *k_cache, uint16_t *v_cache, float *out) {
    if (!q35_dims_ok(d)) return fail(OI_E_ARG, "qwen35 attention: bad dims");
    if (n_tokens <= 0 || pos0 < 0 || (int64_t)pos0 + n_tokens > d->seq_len)
        return fail(OI_E_RANGE, "qwen35 attention: positions out of range");
    if (!qproj || !k || !v || !q_norm || !k_norm || (d->rotary_dim && !inv_freq) || !k_cache || !v_cache || !out)
        return fail(OI_E_ARG, "null argument");
    const size_t n = (size_t)n_tokens, hd = (size_t)d->head_dim, qd = (size_t)d->n_heads * hd,
                 kvd = (size_t)d->n_kv_heads * hd, cache = kvd * (size_t)d->seq_len;
    const size_t ws = (size_t)oi_qwen35_attn_workspace_bytes(d);
    const size_t fl = n * (2 * qd + 2 * kvd) + 2 * hd + (size_t)d->rotary_dim / 2 + n * qd;
    uint8_t *dev = nullptr;
    HIP_TRY(hipMalloc((void **)&dev, fl * 4 + 2 * cache * 2 + ws + 256));
    float *p = (float *)dev;
    float *dq = p; p += n * 2 * qd;
    float *dk = p; p += n * kvd;
    float *dv = p; p += n * kvd;
    float *dqn = p; p += hd;
    float *dkn = p; p += hd;
    float *dif = p; p += d->rotary_dim / 2;
    float *dout = p; p += n * qd;
    uint16_t *dkc = (uint16_t *)p, *dvc = dkc + cache;
    void *dws = (void *)(((uintptr_t)(dvc + cache) + 255) & ~(uintptr_t)255);
    hipError_t r = hipMemcpy(dq, qproj, n * 2 * qd * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dk, k, n * kvd * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dv, v, n * kvd * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dqn, q_norm, hd * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dkn, k_norm, hd * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess && d->rotary_dim) r = hipMemcpy(dif, inv_freq, (size_t)d->rotary_dim / 2 * 4, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dkc, k_cache, cache * 2, hipMemcpyHostToDevice);
    if (r == hipSuccess) r = hipMemcpy(dvc, v_cache, cache * 2, hipMemcpyHostToDevice);
    int rc = OI_OK;
    for (size_t i = 0; r == hipSuccess && !rc && i < n; i++)
        rc = oi_qwen35_attn_step_launch(d, pos0 + (int32_t)i, dq + i * 2 * qd, dk + i * kvd, dv + i * kvd, dqn, dkn,
                                        dif, dkc, dvc, dws, dout + i * qd, nullptr);
    if (r == hipSuccess && !rc) r = hipMemcpy(out, dout, n * qd * 4, hipMemcpyDeviceToHost);
    if (r == hipSuccess && !rc) r = hipMemcpy(k_cache, dkc, cache * 2, hipMemcpyDeviceToHost);
    if (r == hipSuccess && !rc) r = hipMemcpy(v_cache, dvc, cache * 2, hipMemcpyDeviceToHost);
    hipFree(dev);
    if (rc) return rc;
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("qwen35 attention: ") + hipGetErrorString(r));
    return OI_OK;
}

// ---------------------------------------------------- mixture of experts --
namespace {
bool moe_dims_ok(const oi_moe_dims *d) {
    return d && d->n_experts > 0 && d->n_experts <= MOE_MAX_EXPERTS && d->top_k >= 1 && d->top_k <= MOE_MAX_K &&
           d->top_k <= d->n_experts && d->dim > 0 && d->dim % 64 == 0 && d->inter > 0 && d->inter % 64 == 0 &&
           d->inter <= 64 * MOE_MAX_K * 4 && d->dim <= 15360;
}
size_t moe_ws_floats(const oi_moe_dims *d) {
    return (size_t)d->n_experts + 2 * (size_t)d->top_k + (size_t)d->top_k * d->inter;
}
}  // namespace

int64_t oi_moe_workspace_bytes(const oi_moe_dims *d) { return moe_dims_ok(d) ? (int64_t)moe_ws_floats(d) * 4 : 0; }

int oi_moe_ffn_launch(const oi_moe_dims *d, const oi_weights *router, const oi_weights *gate, const oi_weights *up,
                      const oi_weights *down, const float *x_dev, void *workspace, float *y_dev, void *stream) {
    if (!moe_dims_ok(d)) return fail(OI_E_ARG, "moe: bad dims (dim and inter multiples of 64, top_k <= 32)");
    if (!router || !gate || !up || !down || !x_dev || !workspace || !y_dev) return fail(OI_E_ARG, "null argument");
    const int64_t E = d->n_experts;
    if (router->m.rows != E || router->m.cols != d->dim || gate->m.rows != E * d->inter || gate->m.cols != d->dim ||
        up->m.rows != E * d->inter || up->m.cols != d->dim || down->m.rows != E * d->dim || down->m.cols != d->inter ||
        gate->m.type != up->m.type)
        return fail(OI_E_ARG, "moe: weight shapes do not match the dims");
    float *ws = (float *)workspace;
    MoeArgs a{};
    a.gate = gate->m; a.up = up->m; a.down = down->m;
    a.x = x_dev;
    a.logits = ws;
    a.ids = (int32_t *)(ws + E);
    a.w = ws + E + d->top_k;
    a.h = ws + E + 2 * d->top_k;
    a.y = y_dev;
    a.n_experts = d->n_experts; a.top_k = d->top_k; a.dim = d->dim; a.inter = d->inter;
    a.norm_topk = d->norm_topk_prob;
    GemvArgs g = gemv_args(GEMV_STORE, d->dim, x_dev, nullptr, 0.f);
    g.nseg = 1;
    g.seg[0].m = router->m;
    g.seg[0].y = ws;
    if (!plan_gemv(g)) return fail(OI_E_UNSUPPORTED, "moe: router row length not supported");
    // gate/up and down on the quantized GEMV kernel with the experts chosen on
    // the device, where the type and shapes allow; the generic kernels otherwise
    GemvArgs gu = gemv_args(GEMV_SWIGLU, d->dim, x_dev, nullptr, 0.f);
    gu.nseg = 2;
    gu.seg[0].m = gate->m;
    gu.seg[1].m = up->m;
    gu.seg[0].m.rows = gu.seg[1].m.rows = d->top_k * d->inter;  // the chosen experts' rows
    gu.seg[0].y = gu.seg[1].y = a.h;
    gu.moe_logits = a.logits;  // routed inside the gate/up kernel
    gu.moe_ids_out = a.ids;
    gu.moe_w_out = a.w;
    gu.moe_norm = d->norm_topk_prob;
    gu.moe_k = d->top_k;
    gu.moe_n = d->n_experts;
    gu.moe_blk = d->inter;
    const bool gu_ok = gemv_q_moe_supported(gu, MOE_ROWS);
    if (gu_ok) plan_gemv_q(gu);
    GemvArgs dn = gemv_args(GEMV_STORE, d->top_k * d->inter, a.h, nullptr, 0.f);
    dn.nseg = 1;
    dn.seg[0].m = down->m;
    dn.seg[0].m.rows = d->dim;  // row r of every expert
    dn.seg[0].y = y_dev;
    dn.moe_ids = a.ids;
    dn.moe_w = a.w;
    dn.moe_k = d->top_k;
    dn.moe_n = d->n_experts;
    dn.moe_blk = d->inter / 64;
    const bool dn_ok = gemv_q_moe_supported(dn, MOE_COLS);
    if (dn_ok) plan_gemv_q(dn);
    HIP_TRY(launch_moe(a, g, gu_ok ? &gu : nullptr, dn_ok ? &dn : nullptr, (hipStream_t)stream));
    return OI_OK;
}

int oi_moe_ffn(const oi_moe_dims *d, int32_t router_type, const void *router_blocks, int32_t expert_type,
               const void *gate_blocks, const void *up_blocks, const void *down_blocks, const float *x, float *y,
               int32_t *ids_out, float *w_out) {
    if (!moe_dims_ok(d)) return fail(OI_E_ARG, "moe: bad dims (dim and inter multiples of 64, top_k <= 32)");
    if (!router_blocks || !gate_blocks || !up_blocks || !down_blocks || !x || !y) return fail(OI_E_ARG, "null argument");
    const int64_t E = d->n_experts;
    oi_weights *wr = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
    int rc = oi_weights_upload(router_type, router_blocks, E, d->dim, &wr);
    if (!rc) rc = oi_weights_upload(expert_type, gate_blocks, E * d->inter, d->dim, &wg);
    if (!rc) rc = oi_weights_upload(expert_type, up_blocks, E * d->inter, d->dim, &wu);
    if (!rc) rc = oi_weights_upload(expert_type, down_blocks, E * d->dim, d->inter, &wd);
    float *dx = nullptr, *dy = nullptr, *dws = nullptr;
    hipError_t r = hipSuccess;
    if (!rc) {
        r = hipMalloc(&dx, (size_t)d->dim * 4);
        if (r == hipSuccess) r = hipMalloc(&dy, (size_t)d->dim * 4);
        if (r == hipSuccess) r = hipMalloc(&dws, moe_ws_floats(d) * 4);
        if (r == hipSuccess) r = hipMemcpy(dx, x, (size_t)d->dim * 4, hipMemcpyHostToDevice);
        if (r == hipSuccess) {
            rc = oi_moe_ffn_launch(d, wr, wg, wu, wd, dx, dws, dy, nullptr);
            if (!rc) r = hipMemcpy(y, dy, (size_t)d->dim * 4, hipMemcpyDeviceToHost);
            if (!rc && r == hipSuccess && ids_out)
                r = hipMemcpy(ids_out, dws + E, (size_t)d->top_k * 4, hipMemcpyDeviceToHost);
            if (!rc && r == hipSuccess && w_out)
                r = hipMemcpy(w_out, dws + E + d->top_k, (size_t)d->top_k * 4, hipMemcpyDeviceToHost);
        }
    }
    if (dx) hipFree(dx);
    if (dy) hipFree(dy);
    if (dws) hipFree(dws);
    oi_weights_free(wr);
    oi_weights_free(wg);
    oi_weights_free(wu);
    oi_weights_free(wd);
    if (rc) return rc;
    if (r != hipSuccess) return fail(OI_E_DEVICE, std::string("moe: ") + hipGetErrorString(r));
    return OI_OK;
}
