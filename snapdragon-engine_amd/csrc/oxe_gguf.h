// GGUF v2/v3 reader (host): the file is memory-mapped, the header, metadata and tensor table are
// parsed, tensor payloads are read only by the caller. Semantics of the reference's narrow reader
// (crates/gguf/src/lib.rs:268-400): long metadata arrays (> 4096 items) are counted, not kept; the
// data section starts at the next multiple of general.alignment (default 32, a power of two); every
// count, dimension and byte size is checked arithmetic, and every tensor must lie inside the file.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/oxe_model.h"

namespace oxe {

// ggml tensor types: (name, block elements, block bytes) (gguf/src/lib.rs:42-86)
struct GgmlTypeInfo {
    const char *name;
    uint64_t blk, size;
};
bool ggml_type_info(uint32_t ty, GgmlTypeInfo *out);
constexpr uint32_t GGML_F32 = 0, GGML_F16 = 1, GGML_Q8_0 = 8, GGML_BF16 = 30;

enum GgufVType : uint32_t {
    GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64
};

struct GgufValue {
    uint32_t type = GV_U8;
    uint64_t u = 0;      // unsigned bits of integer / bool values
    int64_t i = 0;       // signed value of integer types
    double f = 0.0;      // F32 / F64
    std::string s;
    std::vector<GgufValue> arr;
    bool long_array = false;   // more than 4096 items: only item_type and len kept
    uint32_t item_type = 0;
    uint64_t len = 0;
    bool as_u64(uint64_t *out) const;
    bool as_f64(double *out) const;
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> shape;   // shape[0] is the contiguous dimension
    uint32_t type = 0;
    uint64_t offset = 0;           // relative to the data section
    uint64_t elements() const;
    uint64_t bytes() const;        // UINT64_MAX on an unknown type or overflow
};

struct Gguf {
    std::string path;
    uint32_t version = 0;
    std::vector<std::pair<std::string, GgufValue>> meta;
    std::vector<GgufTensor> tensors;
    uint64_t data_offset = 0, header_bytes = 0, file_bytes = 0;
    const uint8_t *map = nullptr;
    size_t map_len = 0;
    ~Gguf();
    const GgufValue *get(const std::string &key) const;
    const GgufTensor *tensor(const std::string &name) const;
    const uint8_t *data(const GgufTensor &t) const { return map + data_offset + t.offset; }
};

// parse a header from a file image (nothing is read beyond buf[0, len)); "" on success
std::string gguf_parse(const uint8_t *buf, size_t len, Gguf &g);
// open + map + parse + bounds check; "" on success
std::string gguf_open(const char *path, Gguf &g);
// ModelDesc::from_header + check (crates/model/src/desc.rs:69-178); "" on success
std::string gguf_model_desc(const Gguf &g, oxe_model_desc *d);

}  // namespace oxe
