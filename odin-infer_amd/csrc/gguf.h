// gguf.h -- read-only GGUF v2/v3 reader over a memory-mapped file.
//
// Same semantics as the reference parser (ggml/gguf.odin:167-229): metadata
// scalars and strings are kept, arrays are skipped, tensor data offsets are
// relative to the data section, which starts at the header end rounded up to
// `general.alignment` (default 32).  Unlike the reference, malformed input is
// reported as an error instead of exiting, and every tensor is bounds-checked
// against the file size.
#pragma once
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace oi {

struct GgufValue {
    uint32_t type = 0;
    uint64_t u = 0;   // integers and bools
    double f = 0.0;   // floats
    std::string str;  // strings
};

struct GgufTensor {
    std::string name;
    uint32_t kind = 0;
    std::vector<uint64_t> dims;  // dims[0] = row length
    uint64_t offset = 0;
    const uint8_t *data = nullptr;
    uint64_t nbytes = 0;
    uint64_t nelems() const;
};

class GgufFile {
  public:
    ~GgufFile();
    // 0 on success; otherwise a negative OI_E_* code and `err` is set.
    int open(const std::string &path, std::string &err);
    const GgufValue *meta(const std::string &key) const;
    const GgufTensor *tensor(const std::string &name) const;
    const std::vector<GgufTensor> &tensors() const { return tensors_; }

  private:
    uint8_t *map_ = nullptr;
    size_t len_ = 0;
    std::map<std::string, GgufValue> meta_;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, size_t> index_;
};

// ggml_block_info (ggml/quant.odin:10-42); returns false for unknown ids.
bool block_info(uint32_t kind, int &elems, int &bytes);

}  // namespace oi
