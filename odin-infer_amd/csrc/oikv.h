// oikv.h -- the .oikv v1 state-file format, host side only: header layout,
// CRC-32, body size, and the load-time checks (reference:
// qwen3_5/kv_persist.odin:55-156 for the layout, :278-310 for the checks and
// their order).  state.cpp streams the body to and from the device; this part
// reads nothing but the file's bytes, so it also builds without HIP (the
// sanitizer build under tests/sanitize runs it on malformed files).
#pragma once
#include <stdint.h>
#include <stdio.h>

#include <string>

namespace oi {

constexpr uint32_t OIKV_MAGIC = 0x4F494B56u;  // 'O','I','K','V' little-endian
constexpr uint32_t OIKV_VERSION = 1;
constexpr size_t OIKV_HEADER_BYTES = 60;  // the fields as written by write_header (kv_persist.odin:141-156)

// Header fields in file order (kv_persist.odin:55-70, 95-113).
struct OikvHeader {
    uint32_t magic, version, arch;
    uint64_t fingerprint;
    uint32_t n_valid_pos, seq_len, n_full, n_linear, kv_dim, conv_dim, conv_kernel, n_v_heads, head_k_dim,
        head_v_dim;
};

// IEEE 802.3 CRC-32 (reflected polynomial 0xEDB88320, initial and final
// complement), the checksum of core:hash crc32 over header + body.
struct Crc32 {
    uint32_t table[256];
    uint32_t v = 0xFFFFFFFFu;
    Crc32();
    void add(const void *p, size_t n);
    uint32_t value() const { return v ^ 0xFFFFFFFFu; }
};

void oikv_put_u32(uint8_t *&p, uint32_t v);
uint32_t oikv_get_u32(const uint8_t *&p);
void oikv_encode(const OikvHeader &h, uint8_t out[OIKV_HEADER_BYTES]);
OikvHeader oikv_decode(const uint8_t in[OIKV_HEADER_BYTES]);

// body bytes after the header (kv_bytes / conv_bytes / rec_bytes, kv_persist.odin:116-128)
uint64_t oikv_body_bytes(const OikvHeader &h);

// The reference's header checks against the engine's own header `mine`
// (kv_persist.odin:278-305, same order and messages), then the layer
// dimensions, then the file size against header + body + CRC.  OI_OK, or
// OI_E_FORMAT with `msg` set.
int oikv_check_header(const OikvHeader &file, const OikvHeader &mine, uint64_t file_size, std::string &msg);

// CRC over the first `covered` bytes of `f` (header + body) against the
// 4-byte value stored after them (kv_persist.odin:307-310).  Reads from the
// start; OI_OK, OI_E_IO or OI_E_FORMAT with `msg` set.
int oikv_verify_crc(FILE *f, uint64_t covered, std::string &msg);

// Everything a load does before it touches state: read and decode the
// header, the checks above against `mine`, the CRC, then position `f` at the
// body.  OI_OK with `h` filled, else OI_E_FORMAT / OI_E_IO with `msg` set.
int oikv_open_checked(FILE *f, const OikvHeader &mine, OikvHeader &h, std::string &msg);

}  // namespace oi
