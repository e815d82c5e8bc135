// GGUF v3 container reader (host only): the header's metadata and tensor
// descriptors, the aligned data section mapped read-only, split models read
// shard by shard. It follows recipe's reader (mod gguf, recipe.rs:9783-10327):
// the same magic, version, value types, alignment rule
// (general.alignment, default 32, a power of two), data offset (the header's
// end rounded up to the alignment), bounds checks and split naming
// (<prefix>-<n>-of-<count>.gguf with split.count / split.no /
// split.tensors.count).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <memory>
#include <string>
#include <vector>

namespace rq {

struct GgufValue {
    uint32_t type = 0;  // GGUF value type id (0..12)
    uint64_t u = 0;     // unsigned integers and bool
    int64_t i = 0;      // signed integers
    double f = 0.0;     // F32 / F64
    std::string s;      // STRING
    uint32_t array_type = 0;
    std::vector<GgufValue> array;  // ARRAY
    bool integer(uint64_t* out) const;  // a nonnegative integer of any width
    bool real(double* out) const;       // F32 or F64
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> shape;  // GGML order: shape[0] is the row width
    uint32_t type = 0;            // GGML type id
    uint64_t offset = 0;          // within the shard's data section
    uint64_t bytes = 0;
    int shard = 0;
};

struct GgufMapping {
    const uint8_t* data = nullptr;
    size_t length = 0;
    ~GgufMapping();
};

struct GgufFile {
    std::vector<std::unique_ptr<GgufMapping>> shards;
    std::vector<uint64_t> data_start;  // per shard
    std::vector<std::pair<std::string, GgufValue>> metadata;  // the first shard's, in file order
    std::vector<GgufTensor> tensors;                           // every shard's, in file order
    const GgufValue* value(const std::string& key) const;
    const GgufTensor* tensor(const std::string& name) const;
    const uint8_t* bytes(const GgufTensor& t) const;
};

// GGML type id -> elements and bytes per block; false for an unsupported id.
bool ggml_block(uint32_t type, uint64_t* elements, uint64_t* bytes);

// Opens `path` (and its sibling shards when it declares a split). On failure
// returns null and sets `error`.
std::unique_ptr<GgufFile> gguf_open(const std::string& path, std::string* error);

}  // namespace rq
