// state.cpp -- persistence of the engine's position-evolving state: the
// .oikv v1 file (reference: qwen3_5/kv_persist.odin:1-381 and the Metal
// conversion qwen3_5/metal.odin:780-962) and in-memory snapshots
// (qwen3_5/engine.odin:139-165, metal.odin:1655-1700).
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

using namespace oi;

namespace {

int fail(int code, const std::string &msg) { return set_error(code, msg.c_str()); }

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(OI_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

constexpr uint32_t KV_MAGIC = 0x4F494B56u;  // 'O','I','K','V' little-endian
constexpr uint32_t KV_VERSION = 1;
constexpr size_t HEADER_BYTES = 60;  // the fields as written by write_header (kv_persist.odin:141-156)

// IEEE 802.3 CRC-32 (reflected polynomial 0xEDB88320, initial and final
// complement), the checksum of core:hash crc32 over header + body.
struct Crc32 {
    uint32_t table[256];
    uint32_t v = 0xFFFFFFFFu;
    Crc32() {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
    }
    void add(const void *p, size_t n) {
        const uint8_t *b = (const uint8_t *)p;
        for (size_t i = 0; i < n; i++) v = table[(v ^ b[i]) & 0xFF] ^ (v >> 8);
    }
    uint32_t value() const { return v ^ 0xFFFFFFFFu; }
};

// Header fields in file order (kv_persist.odin:55-70, 95-113).
struct Header {
    uint32_t magic, version, arch;
    uint64_t fingerprint;
    uint32_t n_valid_pos, seq_len, n_full, n_linear, kv_dim, conv_dim, conv_kernel, n_v_heads, head_k_dim,
        head_v_dim;
};

void put_u32(uint8_t *&p, uint32_t v) {
    for (int i = 0; i < 4; i++) *p++ = (uint8_t)(v >> (8 * i));
}
void put_u64(uint8_t *&p, uint64_t v) {
    for (int i = 0; i < 8; i++) *p++ = (uint8_t)(v >> (8 * i));
}
uint32_t get_u32(const uint8_t *&p) {
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) v |= (uint32_t)*p++ << (8 * i);
    return v;
}
uint64_t get_u64(const uint8_t *&p) {
    uint64_t v = 0;
    for (int i = 0; i < 8; i++) v |= (uint64_t)*p++ << (8 * i);
    return v;
}

void encode(const Header &h, uint8_t out[HEADER_BYTES]) {
    uint8_t *p = out;
    put_u32(p, h.magic);
    put_u32(p, h.version);
    put_u32(p, h.arch);
    put_u64(p, h.fingerprint);
    for (uint32_t v : {h.n_valid_pos, h.seq_len, h.n_full, h.n_linear, h.kv_dim, h.conv_dim, h.conv_kernel,
                       h.n_v_heads, h.head_k_dim, h.head_v_dim})
        put_u32(p, v);
}

Header decode(const uint8_t in[HEADER_BYTES]) {
    const uint8_t *p = in;
    Header h{};
    h.magic = get_u32(p);
    h.version = get_u32(p);
    h.arch = get_u32(p);
    h.fingerprint = get_u64(p);
    h.n_valid_pos = get_u32(p);
    h.seq_len = get_u32(p);
    h.n_full = get_u32(p);
    h.n_linear = get_u32(p);
    h.kv_dim = get_u32(p);
    h.conv_dim = get_u32(p);
    h.conv_kernel = get_u32(p);
    h.n_v_heads = get_u32(p);
    h.head_k_dim = get_u32(p);
    h.head_v_dim = get_u32(p);
    return h;
}

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

Header header_of(const oi_engine *e, const Shape &s, uint32_t n_valid) {
    Header h{};
    h.magic = KV_MAGIC;
    h.version = KV_VERSION;
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

// body bytes after the header (kv_bytes / conv_bytes / rec_bytes, kv_persist.odin:116-128)
uint64_t body_bytes(const Header &h) {
    const uint64_t kv = 2ull * h.n_full * h.n_valid_pos * h.kv_dim * 4;
    const uint64_t conv = h.conv_kernel == 0 ? 0 : (uint64_t)h.n_linear * h.conv_dim * (h.conv_kernel - 1) * 4;
    const uint64_t rec = (uint64_t)h.n_linear * h.n_v_heads * h.head_k_dim * h.head_v_dim * 4;
    return kv + conv + rec;
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
    const Header h = header_of(e, s, (uint32_t)n_valid_pos);
    File f(std::fopen(path, "wb"));
    if (!f) return fail(OI_E_IO, std::string("kv: cannot open ") + path + " for write");
    Crc32 crc;
    auto put = [&](const void *p, size_t n) -> bool {
        crc.add(p, n);
        return std::fwrite(p, 1, n, f.get()) == n;
    };
    uint8_t hb[HEADER_BYTES];
    encode(h, hb);
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
    put_u32(p, crc.value());
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
    uint8_t hb[HEADER_BYTES];
    if (std::fread(hb, 1, sizeof hb, f.get()) != sizeof hb) return fail(OI_E_FORMAT, "kv: header truncated");
    const Header h = decode(hb);
    const Shape s = shape_of(e);
    const Header mine = header_of(e, s, 0);
    char msg[160];
    // the reference's checks, in its order (kv_persist.odin:278-305)
    if (h.magic != KV_MAGIC) {
        std::snprintf(msg, sizeof msg, "kv: bad magic 0x%08x", h.magic);
        return fail(OI_E_FORMAT, msg);
    }
    if (h.version != KV_VERSION) {
        std::snprintf(msg, sizeof msg, "kv: version mismatch (file=%u, supported=%u)", h.version, KV_VERSION);
        return fail(OI_E_FORMAT, msg);
    }
    if (h.arch != mine.arch) {
        std::snprintf(msg, sizeof msg, "kv: arch mismatch (file=%u, expected %u)", h.arch, mine.arch);
        return fail(OI_E_FORMAT, msg);
    }
    if (h.fingerprint != mine.fingerprint) {
        std::snprintf(msg, sizeof msg, "kv: fingerprint mismatch (file=0x%016llx, model=0x%016llx) — wrong model?",
                      (unsigned long long)h.fingerprint, (unsigned long long)mine.fingerprint);
        return fail(OI_E_FORMAT, msg);
    }
    if (h.seq_len != mine.seq_len) {
        std::snprintf(msg, sizeof msg, "kv: seq_len mismatch (file=%u, engine=%u) — use same -c", h.seq_len,
                      mine.seq_len);
        return fail(OI_E_FORMAT, msg);
    }
    if (h.n_valid_pos > mine.seq_len) {
        std::snprintf(msg, sizeof msg, "kv: file n_valid_pos %u > engine seq_len %u", h.n_valid_pos, mine.seq_len);
        return fail(OI_E_FORMAT, msg);
    }
    // layer dims (the fingerprint implies them; a file that disagrees is corrupt)
    if (h.n_full != mine.n_full || h.n_linear != mine.n_linear || h.kv_dim != mine.kv_dim ||
        h.conv_dim != mine.conv_dim || h.conv_kernel != mine.conv_kernel || h.n_v_heads != mine.n_v_heads ||
        h.head_k_dim != mine.head_k_dim || h.head_v_dim != mine.head_v_dim)
        return fail(OI_E_FORMAT, "kv: layer dimensions differ from the engine's");
    const uint64_t body = body_bytes(h);
    if (std::fseek(f.get(), 0, SEEK_END) != 0) return fail(OI_E_IO, "kv: seek failed");
    const long size = std::ftell(f.get());
    if (size < 0 || (uint64_t)size != HEADER_BYTES + body + 4) {
        std::snprintf(msg, sizeof msg, "kv: file is %ld bytes, the header implies %llu", size,
                      (unsigned long long)(HEADER_BYTES + body + 4));
        return fail(OI_E_FORMAT, msg);
    }
    // CRC over header + body before any state changes (kv_persist.odin:307-310)
    {
        Crc32 crc;
        std::vector<uint8_t> buf(8u << 20);
        std::rewind(f.get());
        uint64_t left = HEADER_BYTES + body;
        while (left) {
            const size_t n = (size_t)std::min<uint64_t>(left, buf.size());
            if (std::fread(buf.data(), 1, n, f.get()) != n) return fail(OI_E_IO, "kv: read failed");
            crc.add(buf.data(), n);
            left -= n;
        }
        uint8_t cb[4];
        if (std::fread(cb, 1, 4, f.get()) != 4) return fail(OI_E_IO, "kv: read failed");
        const uint8_t *p = cb;
        if (get_u32(p) != crc.value()) return fail(OI_E_FORMAT, "kv: CRC mismatch — file corrupted");
    }
    if (std::fseek(f.get(), (long)HEADER_BYTES, SEEK_SET) != 0) return fail(OI_E_IO, "kv: seek failed");

    const int n = (int)h.n_valid_pos;
    const size_t rows = (size_t)n * s.kv_dim * 4;
    const size_t conv_b = (size_t)(s.conv_dim * s.km1) * 4, rec_b = (size_t)s.rec_floats * 4;
    Staging st;
    int rc = st.alloc(std::max(rows, std::max(conv_b, rec_b)));
    if (rc) return rc;
    // everything past n_valid_pos is stale: zero the caches first (metal.odin:912-916)
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
