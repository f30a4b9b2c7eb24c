// Minimal GGUF v3 reader over a memory-mapped file (public GGUF specification). The reference reads GGUF through
// antirez/gguf-tools (pinned commit a3257ff3); this is an independent reader of the same format.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace gguf
{

enum ValueType : uint32_t
{
    T_UINT8 = 0,
    T_INT8 = 1,
    T_UINT16 = 2,
    T_INT16 = 3,
    T_UINT32 = 4,
    T_INT32 = 5,
    T_FLOAT32 = 6,
    T_BOOL = 7,
    T_STRING = 8,
    T_ARRAY = 9,
    T_UINT64 = 10,
    T_INT64 = 11,
    T_FLOAT64 = 12
};

enum TensorType : uint32_t
{
    GGML_F32 = 0,
    GGML_F16 = 1
};

struct KV
{
    std::string key;
    uint32_t type = 0;
    // scalar payload (raw little-endian bytes, zero-extended) for scalar types
    uint64_t u64 = 0;
    double f64 = 0.0;
    std::string str;
    // arrays
    uint32_t arr_type = 0;
    uint64_t arr_len = 0;
    const uint8_t *arr_data = nullptr; // first element in the mapped file
    const uint8_t *arr_end = nullptr;  // one past the last element's bytes
};

struct TensorInfo
{
    std::string name;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;  // from the data section
    const uint8_t *data = nullptr;
    uint64_t bytes = 0;   // for F32/F16: elements * size; otherwise up to the next tensor
};

struct File
{
    int fd = -1;
    const uint8_t *base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    std::vector<KV> kvs;
    std::vector<TensorInfo> tensors;

    ~File();
    // false on a missing file or malformed header
    bool open(const char *path, std::string *err);
    const KV *find(const char *key) const;
};

// iterate the elements of an array KV of strings
std::vector<std::string> string_array(const KV &kv);
std::vector<float> f32_array(const KV &kv);
std::vector<int32_t> i32_array(const KV &kv);

} // namespace gguf
