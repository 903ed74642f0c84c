// gguf.cpp -- see gguf.h.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "oi.h"

namespace oi {

bool block_info(uint32_t kind, int &elems, int &bytes) {
    switch (kind) {
    case 0: elems = 1; bytes = 4; return true;      // F32
    case 1: elems = 1; bytes = 2; return true;      // F16
    case 2: elems = 32; bytes = 18; return true;    // Q4_0
    case 3: elems = 32; bytes = 20; return true;    // Q4_1
    case 6: elems = 32; bytes = 22; return true;    // Q5_0
    case 7: elems = 32; bytes = 24; return true;    // Q5_1
    case 8: elems = 32; bytes = 34; return true;    // Q8_0
    case 9: elems = 32; bytes = 36; return true;    // Q8_1
    case 10: elems = 256; bytes = 84; return true;  // Q2_K
    case 11: elems = 256; bytes = 110; return true; // Q3_K
    case 12: elems = 256; bytes = 144; return true; // Q4_K
    case 13: elems = 256; bytes = 176; return true; // Q5_K
    case 14: elems = 256; bytes = 210; return true; // Q6_K
    case 15: elems = 256; bytes = 292; return true; // Q8_K
    default: return false;
    }
}

uint64_t GgufTensor::nelems() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
}

namespace {

struct Cursor {
    const uint8_t *p;
    size_t len, pos = 0;
    bool bad = false;
    bool take(size_t n) {
        if (bad || n > len - pos) {
            bad = true;
            return false;
        }
        return true;
    }
    uint64_t le(int n) {
        if (!take((size_t)n)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < n; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += (size_t)n;
        return v;
    }
    std::string str() {
        uint64_t n = le(8);
        if (!take(n)) return {};
        std::string s((const char *)p + pos, (size_t)n);
        pos += n;
        return s;
    }
    void skip(uint32_t t, int depth) {
        if (depth > 8) {
            bad = true;
            return;
        }
        switch (t) {
        case 0: case 1: case 7: le(1); break;
        case 2: case 3: le(2); break;
        case 4: case 5: case 6: le(4); break;
        case 10: case 11: case 12: le(8); break;
        case 8: {
            uint64_t n = le(8);
            if (take(n)) pos += n;
            break;
        }
        case 9: {
            uint32_t et = (uint32_t)le(4);
            uint64_t c = le(8);
            for (uint64_t i = 0; i < c && !bad; i++) skip(et, depth + 1);
            break;
        }
        default: bad = true;
        }
    }
};

}  // namespace

GgufFile::~GgufFile() {
    if (map_) munmap(map_, len_);
}

int GgufFile::open(const std::string &path, std::string &err) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        err = "cannot open " + path + ": " + std::strerror(errno);
        return OI_E_IO;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        err = "not a GGUF file (too short): " + path;
        return OI_E_FORMAT;
    }
    len_ = (size_t)st.st_size;
    void *m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        err = "mmap failed for " + path;
        return OI_E_IO;
    }
    map_ = (uint8_t *)m;
    Cursor c{map_, len_};
    uint32_t magic = (uint32_t)c.le(4);
    if (magic != 0x46554747u) {
        err = "not a GGUF file (bad magic)";
        return OI_E_FORMAT;
    }
    uint32_t version = (uint32_t)c.le(4);
    if (version != 2 && version != 3) {
        err = "unsupported GGUF version " + std::to_string(version);
        return OI_E_FORMAT;
    }
    uint64_t n_tensors = c.le(8), n_meta = c.le(8);
    if (n_tensors > (1u << 24) || n_meta > (1u << 24)) {
        err = "corrupt GGUF header";
        return OI_E_FORMAT;
    }
    for (uint64_t i = 0; i < n_meta && !c.bad; i++) {
        std::string key = c.str();
        GgufValue v;
        v.type = (uint32_t)c.le(4);
        switch (v.type) {
        case 0: case 1: case 7: v.u = c.le(1); break;
        case 2: case 3: v.u = c.le(2); break;
        case 4: case 5: v.u = c.le(4); break;
        case 10: case 11: v.u = c.le(8); break;
        case 6: {
            uint32_t b = (uint32_t)c.le(4);
            float f;
            std::memcpy(&f, &b, 4);
            v.f = f;
            break;
        }
        case 12: {
            uint64_t b = c.le(8);
            std::memcpy(&v.f, &b, 8);
            break;
        }
        case 8: v.str = c.str(); break;
        case 9: {
            uint32_t et = (uint32_t)c.le(4);
            uint64_t cnt = c.le(8);
            for (uint64_t j = 0; j < cnt && !c.bad; j++) c.skip(et, 1);
            break;
        }
        default: c.bad = true;
        }
        if (!c.bad) meta_[key] = v;
    }
    for (uint64_t i = 0; i < n_tensors && !c.bad; i++) {
        GgufTensor t;
        t.name = c.str();
        uint32_t nd = (uint32_t)c.le(4);
        if (nd == 0 || nd > 4) {
            c.bad = true;
            break;
        }
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.le(8));
        t.kind = (uint32_t)c.le(4);
        t.offset = c.le(8);
        index_[t.name] = tensors_.size();
        tensors_.push_back(std::move(t));
    }
    if (c.bad) {
        err = "truncated or corrupt GGUF";
        return OI_E_FORMAT;
    }
    uint64_t align = 32;
    if (auto *a = meta("general.alignment")) align = a->u;
    if (align == 0 || (align & (align - 1)) || align > len_) {
        err = "bad general.alignment";
        return OI_E_FORMAT;
    }
    const uint64_t base = ((uint64_t)c.pos + align - 1) & ~(align - 1);
    for (auto &t : tensors_) {
        int e, b;
        if (!block_info(t.kind, e, b)) {
            err = "tensor " + t.name + " has unknown type " + std::to_string(t.kind);
            return OI_E_FORMAT;
        }
        // the element count must not wrap and the row must hold whole blocks
        uint64_t n = 1;
        for (uint64_t d : t.dims)
            if (d != 0 && n > UINT64_MAX / d) {
                err = "tensor " + t.name + " has an element count beyond 2^64";
                return OI_E_FORMAT;
            } else {
                n *= d;
            }
        if (t.dims[0] % (uint64_t)e != 0) {
            err = "tensor " + t.name + " has rows of " + std::to_string(t.dims[0]) + " elements, not a multiple of " +
                  std::to_string(e);
            return OI_E_FORMAT;
        }
        // GGUF places every tensor at a multiple of the alignment (the
        // reference does not check it; f32 and f16 data must be aligned)
        if (t.offset % align != 0) {
            err = "tensor " + t.name + " is not aligned to " + std::to_string(align) + " bytes";
            return OI_E_FORMAT;
        }
        if (n / (uint64_t)e > UINT64_MAX / (uint64_t)b || t.offset > len_ || base > len_ - t.offset) {
            err = "tensor " + t.name + " extends past the end of the file";
            return OI_E_FORMAT;
        }
        t.nbytes = n / (uint64_t)e * (uint64_t)b;
        const uint64_t start = base + t.offset;
        if (t.nbytes > len_ - start) {
            err = "tensor " + t.name + " extends past the end of the file";
            return OI_E_FORMAT;
        }
        t.data = map_ + start;
    }
    return OI_OK;
}

const GgufValue *GgufFile::meta(const std::string &key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

const GgufTensor *GgufFile::tensor(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

}  // namespace oi
