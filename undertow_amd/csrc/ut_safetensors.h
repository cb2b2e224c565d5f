// ut_safetensors.h -- reading safetensors checkpoints from disk (host code).
//
// The checkpoint layout undertow's converter writes (undertow-convert/src/
// lib.rs:273-345): `experts-{layer:05}.safetensors` shards with every routed
// expert of a layer, `dense.safetensors` with the rest, and
// `model.safetensors.index.json` mapping tensor names to shard files; or a
// single `model.safetensors`.  Quantized weights are `<name>` (U8 payload)
// plus `<name>.scales` (one per output row: F32, or BF16 / F16 read as f32).
//
// Headers are untrusted input, validated as undertow-io's parse_header does
// (undertow-io/src/reader.rs:78-143): every entry needs a known dtype, a
// shape whose byte size matches its data_offsets without overflow, and an
// extent inside the file; the header itself is at most 100 MB.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace ut {
namespace st {

enum Dtype { ST_F32, ST_F16, ST_BF16, ST_U8, ST_I8 };

inline int dtype_size(int d) { return d == ST_F32 ? 4 : (d == ST_F16 || d == ST_BF16) ? 2 : 1; }

// A JSON value: just what safetensors headers and index files hold.
struct Json {
    enum Kind { Null, Bool, Int, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json *get(const std::string &key) const {
        for (auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

// Parses text[0, n) as one JSON value (trailing whitespace allowed).
bool parse_json(const char *text, size_t n, Json &out, std::string &err);

struct Entry {
    int dtype = ST_F32;
    std::vector<int64_t> shape;
    uint64_t offset = 0;  // absolute offset of the data in its file
    uint64_t nbytes = 0;
    int shard = 0;
};

struct Shard {
    std::string path;
    int fd = -1;
    uint64_t file_len = 0;
};

// The tensors of a model directory, indexed at open (headers only).
struct Index {
    std::vector<Shard> shards;
    std::unordered_map<std::string, Entry> tensors;
    ~Index();
    const Entry *find(const std::string &name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

// ShardedModelReader::open (reader.rs:300-363): the index file if present,
// else the single model.safetensors.  Returns false with err set.
bool open_dir(const std::string &dir, Index &idx, std::string &err);

// pread of [offset, offset + n) from a shard, retried until complete.
bool read_at(const Shard &s, void *dst, uint64_t n, uint64_t offset, std::string &err);

// decode_f32 of a 16-bit float run (reader.rs:256-276): n bf16 or f16
// values widened exactly to f32 bits (every half is a float).
void widen_halves(const uint16_t *src, uint64_t n, bool bf16, uint32_t *dst);

// A tensor's elements as f32 into dst (F32 read as is, BF16 / F16 widened),
// staging halves through `tmp`; false (err set) for other dtypes.
bool read_f32_at(const Shard &s, const Entry &e, float *dst, std::vector<uint16_t> &tmp,
                 std::string &err);

}  // namespace st
}  // namespace ut
