// oikv.cpp -- see oikv.h.
#include "oikv.h"

#include <algorithm>
#include <cstring>
#include <vector>

#include "oi.h"

namespace oi {

Crc32::Crc32() {
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
        table[i] = c;
    }
}

void Crc32::add(const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    for (size_t i = 0; i < n; i++) v = table[(v ^ b[i]) & 0xFF] ^ (v >> 8);
}

void oikv_put_u32(uint8_t *&p, uint32_t v) {
    for (int i = 0; i < 4; i++) *p++ = (uint8_t)(v >> (8 * i));
}

static void put_u64(uint8_t *&p, uint64_t v) {
    for (int i = 0; i < 8; i++) *p++ = (uint8_t)(v >> (8 * i));
}

uint32_t oikv_get_u32(const uint8_t *&p) {
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) v |= (uint32_t)*p++ << (8 * i);
    return v;
}

static uint64_t get_u64(const uint8_t *&p) {
    uint64_t v = 0;
    for (int i = 0; i < 8; i++) v |= (uint64_t)*p++ << (8 * i);
    return v;
}

void oikv_encode(const OikvHeader &h, uint8_t out[OIKV_HEADER_BYTES]) {
    uint8_t *p = out;
    oikv_put_u32(p, h.magic);
    oikv_put_u32(p, h.version);
    oikv_put_u32(p, h.arch);
    put_u64(p, h.fingerprint);
    for (uint32_t v : {h.n_valid_pos, h.seq_len, h.n_full, h.n_linear, h.kv_dim, h.conv_dim, h.conv_kernel,
                       h.n_v_heads, h.head_k_dim, h.head_v_dim})
        oikv_put_u32(p, v);
}

OikvHeader oikv_decode(const uint8_t in[OIKV_HEADER_BYTES]) {
    const uint8_t *p = in;
    OikvHeader h{};
    h.magic = oikv_get_u32(p);
    h.version = oikv_get_u32(p);
    h.arch = oikv_get_u32(p);
    h.fingerprint = get_u64(p);
    h.n_valid_pos = oikv_get_u32(p);
    h.seq_len = oikv_get_u32(p);
    h.n_full = oikv_get_u32(p);
    h.n_linear = oikv_get_u32(p);
    h.kv_dim = oikv_get_u32(p);
    h.conv_dim = oikv_get_u32(p);
    h.conv_kernel = oikv_get_u32(p);
    h.n_v_heads = oikv_get_u32(p);
    h.head_k_dim = oikv_get_u32(p);
    h.head_v_dim = oikv_get_u32(p);
    return h;
}

uint64_t oikv_body_bytes(const OikvHeader &h) {
    const uint64_t kv = 2ull * h.n_full * h.n_valid_pos * h.kv_dim * 4;
    const uint64_t conv = h.conv_kernel == 0 ? 0 : (uint64_t)h.n_linear * h.conv_dim * (h.conv_kernel - 1) * 4;
    const uint64_t rec = (uint64_t)h.n_linear * h.n_v_heads * h.head_k_dim * h.head_v_dim * 4;
    return kv + conv + rec;
}

int oikv_check_header(const OikvHeader &h, const OikvHeader &mine, uint64_t file_size, std::string &msg) {
    char b[160];
    auto bad = [&](void) {
        msg = b;
        return OI_E_FORMAT;
    };
    if (h.magic != OIKV_MAGIC) {
        std::snprintf(b, sizeof b, "kv: bad magic 0x%08x", h.magic);
        return bad();
    }
    if (h.version != OIKV_VERSION) {
        std::snprintf(b, sizeof b, "kv: version mismatch (file=%u, supported=%u)", h.version, OIKV_VERSION);
        return bad();
    }
    if (h.arch != mine.arch) {
        std::snprintf(b, sizeof b, "kv: arch mismatch (file=%u, expected %u)", h.arch, mine.arch);
        return bad();
    }
    if (h.fingerprint != mine.fingerprint) {
        std::snprintf(b, sizeof b, "kv: fingerprint mismatch (file=0x%016llx, model=0x%016llx) — wrong model?",
                      (unsigned long long)h.fingerprint, (unsigned long long)mine.fingerprint);
        return bad();
    }
    if (h.seq_len != mine.seq_len) {
        std::snprintf(b, sizeof b, "kv: seq_len mismatch (file=%u, engine=%u) — use same -c", h.seq_len,
                      mine.seq_len);
        return bad();
    }
    if (h.n_valid_pos > mine.seq_len) {
        std::snprintf(b, sizeof b, "kv: file n_valid_pos %u > engine seq_len %u", h.n_valid_pos, mine.seq_len);
        return bad();
    }
    // layer dims (the fingerprint implies them; a file that disagrees is corrupt)
    if (h.n_full != mine.n_full || h.n_linear != mine.n_linear || h.kv_dim != mine.kv_dim ||
        h.conv_dim != mine.conv_dim || h.conv_kernel != mine.conv_kernel || h.n_v_heads != mine.n_v_heads ||
        h.head_k_dim != mine.head_k_dim || h.head_v_dim != mine.head_v_dim) {
        std::snprintf(b, sizeof b, "kv: layer dimensions differ from the engine's");
        return bad();
    }
    // every field that sizes the body now equals the engine's, so the sum cannot overflow
    const uint64_t want = OIKV_HEADER_BYTES + oikv_body_bytes(h) + 4;
    if (file_size != want) {
        std::snprintf(b, sizeof b, "kv: file is %llu bytes, the header implies %llu", (unsigned long long)file_size,
                      (unsigned long long)want);
        return bad();
    }
    return OI_OK;
}

int oikv_verify_crc(FILE *f, uint64_t covered, std::string &msg) {
    Crc32 crc;
    std::vector<uint8_t> buf(8u << 20);
    std::rewind(f);
    uint64_t left = covered;
    while (left) {
        const size_t n = (size_t)std::min<uint64_t>(left, buf.size());
        if (std::fread(buf.data(), 1, n, f) != n) {
            msg = "kv: read failed";
            return OI_E_IO;
        }
        crc.add(buf.data(), n);
        left -= n;
    }
    uint8_t cb[4];
    if (std::fread(cb, 1, 4, f) != 4) {
        msg = "kv: read failed";
        return OI_E_IO;
    }
    const uint8_t *p = cb;
    if (oikv_get_u32(p) != crc.value()) {
        msg = "kv: CRC mismatch — file corrupted";
        return OI_E_FORMAT;
    }
    return OI_OK;
}

int oikv_open_checked(FILE *f, const OikvHeader &mine, OikvHeader &h, std::string &msg) {
    uint8_t hb[OIKV_HEADER_BYTES];
    if (std::fread(hb, 1, sizeof hb, f) != sizeof hb) {
        msg = "kv: header truncated";
        return OI_E_FORMAT;
    }
    h = oikv_decode(hb);
    if (std::fseek(f, 0, SEEK_END) != 0) {
        msg = "kv: seek failed";
        return OI_E_IO;
    }
    const long size = std::ftell(f);
    if (size < 0) {
        msg = "kv: tell failed";
        return OI_E_IO;
    }
    int rc = oikv_check_header(h, mine, (uint64_t)size, msg);
    if (rc == OI_OK) rc = oikv_verify_crc(f, OIKV_HEADER_BYTES + oikv_body_bytes(h), msg);
    if (rc != OI_OK) return rc;
    if (std::fseek(f, (long)OIKV_HEADER_BYTES, SEEK_SET) != 0) {
        msg = "kv: seek failed";
        return OI_E_IO;
    }
    return OI_OK;
}

}  // namespace oi
