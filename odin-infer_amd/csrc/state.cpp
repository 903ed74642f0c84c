// state.cpp -- persistence of the engine's position-evolving state: the
// .oikv v1 file (reference: qwen3_5/kv_persist.odin:1-381 and the Metal
// conversion qwen3_5/metal.odin:780-962) and in-memory snapshots
// (qwen3_5/engine.odin:139-165, qwen3_5/metal.odin:1655-1700).
//
// The state lives in HBM: per attention layer an f16 head-major cache
// [n_kv][seq_len][hd] for K and for V, per DeltaNet layer its conv window
// [conv_dim][kernel-1] and recurrent state [n_v][hk][hv] (f32).  The file holds
// f32 rows [pos][n_kv * hd]; the conversion runs on the device
// (launch_kv_convert), one layer at a time through a staging buffer, and the
// file is streamed (no whole-file buffer: a Qwen3-8B cache at 4096 positions
// is 1.2 GB of f32).  Snapshots are plain byte copies of the device layout
// into caller memory, host or device.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "engine_internal.h"
#include "oikv.h"

using namespace oi;

namespace {

int fail(int code, const std::string &msg) { return set_error(code, msg.c_str()); }

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(OI_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

// What the engine holds, in the header's terms.
struct Shape {
    std::vector<const LayerDev *> attn, lin;  // layers with a K/V cache / with DeltaNet states, in order
    int64_t kv_dim = 0, conv_dim = 0, km1 = 0, rec_floats = 0;
    size_t kv_layer_bytes = 0;  // one f16 cache tensor of one layer
};

Shape shape_of(const oi_engine *e) {
    Shape s;
    const oi_config &c = e->cfg;
    for (const LayerDev &L : e->layers) {
        if (L.kc) s.attn.push_back(&L);
        if (L.rec_state) s.lin.push_back(&L);
    }
    s.kv_dim = c.n_kv_heads * c.head_dim;
    s.kv_layer_bytes = (size_t)c.n_kv_heads * c.seq_len * c.head_dim * 2;
    s.conv_dim = 2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv;
    s.km1 = e->lin_kernel > 0 ? e->lin_kernel - 1 : 0;
    s.rec_floats = e->lin_nv * e->lin_hk * e->lin_hv;
    return s;
}

// model_fingerprint (kv_persist.odin:74-93): FNV-1a 64 over the identifying
// Config fields, each mixed as one 64-bit word.
uint64_t fingerprint(const oi_engine *e) {
    const oi_config &c = e->cfg;
    uint64_t h = 0xcbf29ce484222325ull;
    for (int64_t v : {c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, e->lin_nk, e->lin_nv, e->lin_hk,
                      e->lin_hv, e->lin_kernel, c.vocab_size})
        h = (h ^ (uint64_t)v) * 0x100000001b3ull;
    return h;
}

// arch field: the reference's KV_ARCH_QWEN3_5 = 2 for the hybrid layout
uint32_t arch_code(const oi_engine *e) { return e->arch == 2 ? 2u : e->arch == 1 ? 3u : 1u; }

OikvHeader header_of(const oi_engine *e, const Shape &s, uint32_t n_valid) {
    OikvHeader h{};
    h.magic = OIKV_MAGIC;
    h.version = OIKV_VERSION;
    h.arch = arch_code(e);
    h.fingerprint = fingerprint(e);
    h.n_valid_pos = n_valid;
    h.seq_len = (uint32_t)e->cfg.seq_len;
    h.n_full = (uint32_t)s.attn.size();
    h.n_linear = (uint32_t)s.lin.size();
    h.kv_dim = (uint32_t)s.kv_dim;
    h.conv_dim = (uint32_t)s.conv_dim;
    h.conv_kernel = (uint32_t)e->lin_kernel;
    h.n_v_heads = (uint32_t)e->lin_nv;
    h.head_k_dim = (uint32_t)e->lin_hk;
    h.head_v_dim = (uint32_t)e->lin_hv;
    return h;
}

struct FileCloser {
    void operator()(FILE *f) const {
        if (f) std::fclose(f);
    }
};
using File = std::unique_ptr<FILE, FileCloser>;

// Device staging of one tensor's f32 rows and its pinned host copy.
struct Staging {
    float *dev = nullptr, *host = nullptr;
    ~Staging() {
        if (dev) (void)hipFree(dev);
        if (host) (void)hipHostFree(host);
    }
    int alloc(size_t bytes) {
        if (bytes == 0) return OI_OK;
        if (hipMalloc((void **)&dev, bytes) != hipSuccess || hipHostMalloc((void **)&host, bytes, 0) != hipSuccess)
            return fail(OI_E_NOMEM, "kv: staging allocation failed");
        return OI_OK;
    }
};

}  // namespace

extern "C" {

int oi_engine_save_kv(oi_engine *e, const char *path, int32_t n_valid_pos) {
    if (!e || !path) return fail(OI_E_ARG, "null argument");
    const oi_config &c = e->cfg;
    if (n_valid_pos < 0 || n_valid_pos > c.seq_len)  // kv_persist.odin:221-224
        return fail(OI_E_RANGE, "kv: n_valid_pos " + std::to_string(n_valid_pos) + " > seq_len " +
                                    std::to_string(c.seq_len));
    HIP_TRY(hipSetDevice(e->device));
    const Shape s = shape_of(e);
    const OikvHeader h = header_of(e, s, (uint32_t)n_valid_pos);
    File f(std::fopen(path, "wb"));
    if (!f) return fail(OI_E_IO, std::string("kv: cannot open ") + path + " for write");
    Crc32 crc;
    auto put = [&](const void *p, size_t n) -> bool {
        crc.add(p, n);
        return std::fwrite(p, 1, n, f.get()) == n;
    };
    uint8_t hb[OIKV_HEADER_BYTES];
    oikv_encode(h, hb);
    if (!put(hb, sizeof hb)) return fail(OI_E_IO, "kv: header write failed");

    const size_t rows = (size_t)n_valid_pos * s.kv_dim * 4;
    const size_t conv_b = (size_t)(s.conv_dim * s.km1) * 4, rec_b = (size_t)s.rec_floats * 4;
    Staging st;
    int rc = st.alloc(std::max(rows, std::max(conv_b, rec_b)));
    if (rc) return rc;
    for (size_t l = 0; l < s.attn.size(); l++) {
        for (uint16_t *cache : {s.attn[l]->kc, s.attn[l]->vc}) {
            if (!rows) continue;
            HIP_TRY(launch_kv_convert(true, cache, st.dev, n_valid_pos, (int)c.n_kv_heads, (int)c.seq_len,
                                      (int)c.head_dim, e->stream));
            HIP_TRY(hipMemcpyAsync(st.host, st.dev, rows, hipMemcpyDeviceToHost, e->stream));
            HIP_TRY(hipStreamSynchronize(e->stream));
            if (!put(st.host, rows))
                return fail(OI_E_IO, std::string("kv: write failed at ") + (cache == s.attn[l]->kc ? "K" : "V") +
                                         " layer " + std::to_string(l));
        }
    }
    for (int part = 0; part < 2; part++)  // every conv state, then every recurrent state
        for (const LayerDev *L : s.lin) {
            const size_t b = part == 0 ? conv_b : rec_b;
            if (!b) continue;
            HIP_TRY(hipMemcpyAsync(st.host, part == 0 ? L->conv_state : L->rec_state, b, hipMemcpyDeviceToHost,
                                   e->stream));
            HIP_TRY(hipStreamSynchronize(e->stream));
            if (!put(st.host, b))
                return fail(OI_E_IO, part == 0 ? "kv: conv_states write failed" : "kv: recurrent_states write failed");
        }
    uint8_t cb[4], *p = cb;
    oikv_put_u32(p, crc.value());
    if (std::fwrite(cb, 1, 4, f.get()) != 4 || std::fflush(f.get()) != 0)
        return fail(OI_E_IO, "kv: crc append failed");
    if (std::fclose(f.release()) != 0) return fail(OI_E_IO, "kv: close failed");
    return OI_OK;
}

int oi_engine_load_kv(oi_engine *e, const char *path, int32_t *n_valid_pos) {
    if (!e || !path) return fail(OI_E_ARG, "null argument");
    const oi_config &c = e->cfg;
    HIP_TRY(hipSetDevice(e->device));
    File f(std::fopen(path, "rb"));
    if (!f) return fail(OI_E_IO, std::string("kv: cannot open ") + path);
    const Shape s = shape_of(e);
    // the reference's checks, in its order, then the size and the CRC over
    // header + body before any state changes (kv_persist.odin:278-310)
    OikvHeader h;
    std::string msg;
    int rc = oikv_open_checked(f.get(), header_of(e, s, 0), h, msg);
    if (rc != OI_OK) return fail(rc, msg);

    const int n = (int)h.n_valid_pos;
    const size_t rows = (size_t)n * s.kv_dim * 4;
    const size_t conv_b = (size_t)(s.conv_dim * s.km1) * 4, rec_b = (size_t)s.rec_floats * 4;
    Staging st;
    rc = st.alloc(std::max(rows, std::max(conv_b, rec_b)));
    if (rc) return rc;
    // everything past n_valid_pos is stale: zero the caches first (qwen3_5/metal.odin:912-916)
    for (const LayerDev *L : s.attn) {
        HIP_TRY(hipMemsetAsync(L->kc, 0, s.kv_layer_bytes, e->stream));
        HIP_TRY(hipMemsetAsync(L->vc, 0, s.kv_layer_bytes, e->stream));
    }
    for (size_t l = 0; l < s.attn.size(); l++)
        for (uint16_t *cache : {s.attn[l]->kc, s.attn[l]->vc}) {
            if (!rows) continue;
            // the previous conversion must have read the staging buffer before it is refilled
            HIP_TRY(hipStreamSynchronize(e->stream));
            if (std::fread(st.host, 1, rows, f.get()) != rows)
                return fail(OI_E_IO, std::string("kv: read failed at ") + (cache == s.attn[l]->kc ? "K" : "V") +
                                         " layer " + std::to_string(l));
            HIP_TRY(hipMemcpyAsync(st.dev, st.host, rows, hipMemcpyHostToDevice, e->stream));
            HIP_TRY(launch_kv_convert(false, cache, st.dev, n, (int)c.n_kv_heads, (int)c.seq_len, (int)c.head_dim,
                                      e->stream));
        }
    for (int part = 0; part < 2; part++)
        for (const LayerDev *L : s.lin) {
            const size_t b = part == 0 ? conv_b : rec_b;
            if (!b) continue;
            HIP_TRY(hipStreamSynchronize(e->stream));
            if (std::fread(st.host, 1, b, f.get()) != b)
                return fail(OI_E_IO, part == 0 ? "kv: conv_states read failed" : "kv: recurrent_states read failed");
            HIP_TRY(hipMemcpyAsync(part == 0 ? L->conv_state : L->rec_state, st.host, b, hipMemcpyHostToDevice,
                                   e->stream));
        }
    HIP_TRY(hipStreamSynchronize(e->stream));
    e->last_pos = n;
    if (n_valid_pos) *n_valid_pos = n;
    return OI_OK;
}

int oi_engine_state_sizes(oi_engine *e, int64_t sizes[4]) {
    if (!e || !sizes) return fail(OI_E_ARG, "null argument");
    const Shape s = shape_of(e);
    sizes[0] = sizes[1] = (int64_t)(s.attn.size() * s.kv_layer_bytes);
    sizes[2] = (int64_t)s.lin.size() * s.conv_dim * s.km1 * 4;
    sizes[3] = (int64_t)s.lin.size() * s.rec_floats * 4;
    return OI_OK;
}

}  // extern "C"

namespace {

// Copies between the engine's per-layer buffers and one contiguous caller
// buffer per kind (host or device memory: hipMemcpyDefault).
int copy_state(oi_engine *e, bool save, void *kv_k, void *kv_v, void *conv, void *rec, bool with_kv) {
    if (!e) return fail(OI_E_ARG, "null engine");
    const Shape s = shape_of(e);
    const size_t conv_b = (size_t)(s.conv_dim * s.km1) * 4, rec_b = (size_t)s.rec_floats * 4;
    if ((with_kv && !s.attn.empty() && (!kv_k || !kv_v)) || (!s.lin.empty() && ((conv_b && !conv) || !rec)))
        return fail(OI_E_ARG, "null state buffer");
    HIP_TRY(hipSetDevice(e->device));
    auto cp = [&](void *buf, size_t off, void *dev, size_t n) -> hipError_t {
        uint8_t *b = (uint8_t *)buf + off;
        return save ? hipMemcpyAsync(b, dev, n, hipMemcpyDefault, e->stream)
                    : hipMemcpyAsync(dev, b, n, hipMemcpyDefault, e->stream);
    };
    if (with_kv)
        for (size_t l = 0; l < s.attn.size(); l++) {
            HIP_TRY(cp(kv_k, l * s.kv_layer_bytes, s.attn[l]->kc, s.kv_layer_bytes));
            HIP_TRY(cp(kv_v, l * s.kv_layer_bytes, s.attn[l]->vc, s.kv_layer_bytes));
        }
    for (size_t l = 0; l < s.lin.size(); l++) {
        if (conv_b) HIP_TRY(cp(conv, l * conv_b, s.lin[l]->conv_state, conv_b));
        HIP_TRY(cp(rec, l * rec_b, s.lin[l]->rec_state, rec_b));
    }
    HIP_TRY(hipStreamSynchronize(e->stream));
    return OI_OK;
}

}  // namespace

extern "C" {

int oi_engine_save_full_state(oi_engine *e, void *kv_k, void *kv_v, void *conv, void *rec) {
    return copy_state(e, true, kv_k, kv_v, conv, rec, true);
}

int oi_engine_restore_full_state(oi_engine *e, const void *kv_k, const void *kv_v, const void *conv,
                                 const void *rec) {
    return copy_state(e, false, const_cast<void *>(kv_k), const_cast<void *>(kv_v), const_cast<void *>(conv),
                      const_cast<void *>(rec), true);
}

int oi_engine_save_spec_state(oi_engine *e, void *conv, void *rec) {
    return copy_state(e, true, nullptr, nullptr, conv, rec, false);
}

int oi_engine_restore_spec_state(oi_engine *e, const void *conv, const void *rec) {
    return copy_state(e, false, nullptr, nullptr, const_cast<void *>(conv), const_cast<void *>(rec), false);
}

}  // extern "C"
