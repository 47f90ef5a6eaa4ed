// GGUF v2/v3 container: key/value table, tensor table, byte mapping.
// Internal to the host library (gguf.cpp implements it, qwen35.cpp reads
// models through it). Format facts it follows:
//   type ids, block sizes, row bytes   src/xiaoju-pipe/core/gguf.c:12-50
//   header layout, alignment key,      src/xiaoju-pipe/core/gguf.c:106-186
//   data offset = header end rounded up to the alignment
//   integer keys of any width, bool    src/xiaoju-pipe/core/gguf.c:276-300
//   as 0/1, floats from F32/F64/ints
#pragma once

#include "xj_hip.h"

#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

struct xj_gguf_file;

namespace xjg {

// GGUF value type ids.
enum VType : uint32_t { U8 = 0, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 };

// Width in bytes of a scalar value type, 0 for strings and arrays.
int scalar_width(uint32_t t);

// A key's value as stored in the header: its type and where its bytes start.
// For arrays, elem/count describe the elements and body points at the first
// one (after the 12-byte element-type + count prefix).
struct Value {
    uint32_t type = 0;
    uint32_t elem = 0;
    uint64_t count = 0;
    const uint8_t *at = nullptr;   // first byte of the value
    const uint8_t *body = nullptr; // arrays: first element

    bool as_uint(uint32_t *out) const;            // any integer width, bool as 0/1
    bool as_float(float *out) const;              // F32, F64 narrowed, integers converted
    bool as_string(std::string_view *out) const;  // STR only
    bool uint_at(uint64_t i, uint32_t *out) const; // element i of an integer/bool array
    // Calls f(index, text) for every element of a string array; false if this is not one.
    template <class F> bool each_string(F &&f) const;
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;   // relative to the data section
    uint64_t nbytes = 0;   // 0 for block types this library does not know
};

}  // namespace xjg

// The opened file. Tensor data is reached through ptr(); with a header-only
// open nothing is mapped until map_range().
struct xj_gguf_file {
    int fd = -1;
    const uint8_t *map = nullptr;       // file bytes [map_off, map_off + map_len)
    uint64_t map_off = 0, map_len = 0;
    uint64_t size = 0, data_off = 0;
    uint32_t alignment = 32;
    std::vector<uint8_t> header;        // owned header bytes (header-only open)
    std::vector<xjg::Tensor> tensors;   // file order
    std::unordered_map<std::string, xjg::Value> keys;
    std::unordered_map<std::string, size_t> by_name;

    const xjg::Value *key(const char *k) const {
        auto it = keys.find(k);
        return it == keys.end() ? nullptr : &it->second;
    }
    const xjg::Tensor *tensor(const std::string &n) const {
        auto it = by_name.find(n);
        return it == by_name.end() ? nullptr : &tensors[it->second];
    }
    // File offset -> pointer into the mapping; NULL when [off, off + n) is not mapped.
    const void *ptr(uint64_t off, uint64_t n) const {
        if (!map || off < map_off || off + n > map_off + map_len) return nullptr;
        return map + (off - map_off);
    }
    ~xj_gguf_file();
};

namespace xjg {

// Whole file mapped; every tensor must lie inside the file.
xj_gguf_file *open_mapped(const char *path, char *err, size_t errlen);
// Header only (read with pread); tensors may lie past the end of a partial file.
xj_gguf_file *open_header(const char *path, char *err, size_t errlen);
// Map file bytes [lo, hi) of a header-only file, starting on the page below lo.
bool map_range(xj_gguf_file *f, uint64_t lo, uint64_t hi, char *err, size_t errlen);

template <class F> bool Value::each_string(F &&f) const {
    if (type != ARR || elem != STR) return false;
    const uint8_t *p = body;
    for (uint64_t i = 0; i < count; i++) {
        uint64_t n;
        __builtin_memcpy(&n, p, 8);
        f(i, std::string_view((const char *)p + 8, n));
        p += 8 + n;
    }
    return true;
}

}  // namespace xjg
