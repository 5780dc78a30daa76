// safetensors.h — a sharded safetensors checkpoint opened for reading: the
// index (model.safetensors.index.json "weight_map": tensor name -> shard
// file), every shard's header (8-byte little-endian length, then a JSON object
// name -> {dtype, shape, data_offsets}), and positional reads of one tensor's
// bytes. Host-only; the C ABI (wl_st_*) is in include/windlass_moe.h.
//
// Reference: st::open / st::info / st::read_bytes (src/safetensors_io.cuh:
// 89-230). Differences, all on the side of refusing a malformed file rather
// than reading past it: the header is parsed as JSON (not searched for
// substrings), each tensor's byte range is checked against its shard's size
// and, for the fixed-width dtypes, against its shape; a directory without an
// index but with model.safetensors, or a path to one .safetensors file, is a
// one-shard checkpoint.
#pragma once
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/windlass_moe.h"

namespace wl {
namespace json {

// A parsed JSON value (enough for safetensors headers and index files).
struct Value {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    std::string s;         // Str: the decoded string
    bool is_uint = false;  // Num: a non-negative integer that fits 64 bits (then u holds it)
    uint64_t u = 0;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;  // in document order
    const Value* get(const std::string& key) const;
};

// Parses text[0, n) as one JSON value surrounded by optional whitespace.
// Returns false and a message (with the byte offset) on malformed input,
// nesting deeper than 64 levels, or a duplicate key in one object.
bool parse(const char* text, size_t n, Value* out, std::string* err);

}  // namespace json

// Element size of a safetensors dtype name, 0 if unknown.
uint32_t st_dtype_size(const std::string& dtype);

}  // namespace wl

struct wl_st {
    struct Shard {
        std::string file;    // as named by the index
        std::string path;
        int fd = -1;         // -1: absent (allow_missing_shards)
        uint64_t size = 0;   // file size
        uint64_t base = 0;   // first data byte: 8 + header length
    };
    struct Tensor {
        uint32_t shard = 0;
        uint64_t offset = 0;  // absolute file offset
        uint64_t nbytes = 0;
        std::string dtype;
        std::vector<uint64_t> shape;
    };
    std::string root;
    std::vector<Shard> shards;
    std::unordered_map<std::string, Tensor> tensors;
    std::vector<std::string> names;  // sorted
    std::string err;

    ~wl_st();
    const Tensor* find(const std::string& name) const;
    // Opens `path` (a checkpoint directory or one .safetensors file).
    // WL_ERR_IO (a file cannot be opened or read) or WL_ERR_FORMAT (a
    // malformed index or header) with err set on failure.
    wl_status open(const std::string& path, bool allow_missing_shards);
    // Reads bytes [off, off + n) of tensor t into dst: WL_ERR_INVALID for a
    // range outside the tensor, WL_ERR_IO on a short read, err set.
    wl_status read(const Tensor& t, uint64_t off, uint64_t n, void* dst, const std::string& name);
};
