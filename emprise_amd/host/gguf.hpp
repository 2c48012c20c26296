// GGUF v2/v3 reader (the reference's Gguf, include/emprise/gguf.hpp:12-51,
// src/gguf.cpp:72-191). The file is memory-mapped read-only; tensor bytes are handed
// to the device backend straight from the mapping.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace emprise {

enum class WeightType : uint32_t { f32 = 0, f16 = 1, q4_k = 12, q6_k = 14, bf16 = 30 };

struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;  // GGUF order: fastest-varying dimension first
    WeightType type = WeightType::f32;
    uint64_t offset = 0, bytes = 0, elements = 0;
};

struct MetaValue {
    uint32_t type = 0;  // GGUF metadata type id
    double number = 0;  // numeric scalars and booleans
    std::string text;   // strings
    uint64_t array_len = 0;
    bool is_array = false;
    uint32_t array_type = 0;           // element type of an array
    std::vector<std::string> strings;  // elements of a string array
    std::vector<int64_t> integers;     // elements of an integer array
};

uint64_t encoded_bytes(WeightType type, uint64_t elements);  // the reference's gguf.cpp:72-85 (throws)

class Gguf {
public:
    explicit Gguf(const std::string& path);
    ~Gguf();
    Gguf(const Gguf&) = delete;
    Gguf& operator=(const Gguf&) = delete;
    const std::vector<Tensor>& tensors() const noexcept { return tensors_; }
    const Tensor& tensor(const std::string& name) const;
    bool has(const std::string& name) const { return index_.count(name) != 0; }
    const MetaValue* meta(const std::string& key) const;
    size_t metadata_count() const noexcept { return meta_.size(); }
    int meta_int(const std::string& key) const;
    float meta_float(const std::string& key) const;
    const uint8_t* data(const Tensor& t) const { return base_ + data_offset_ + t.offset; }
    uint64_t data_bytes() const noexcept { return file_bytes_ - data_offset_; }

private:
    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    uint64_t file_bytes_ = 0, data_offset_ = 0;
    std::vector<Tensor> tensors_;
    std::unordered_map<std::string, size_t> index_;
    std::map<std::string, MetaValue> meta_;
};

}  // namespace emprise
