// GGUF reader over a read-only memory map: header, key/value section, tensor table and
// the format's invariants (the checks the reference makes in src/gguf.cpp:87-147, each
// stated from the GGUF layout itself).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace emprise {

namespace {
uint64_t checked_mul(uint64_t a, uint64_t b) {
    if (b && a > std::numeric_limits<uint64_t>::max() / b) throw std::runtime_error("GGUF: a tensor size overflows 64 bits");
    return a * b;
}

class Cursor {
public:
    Cursor(const uint8_t* p, uint64_t size) : p_(p), size_(size) {}
    template <class T> T scalar() {
        if (pos_ > size_ || size_ - pos_ < sizeof(T)) throw std::runtime_error("GGUF: the file ends inside its header");
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string string() {
        const uint64_t n = scalar<uint64_t>();
        if (n > size_ - pos_ || n > 64ull * 1024 * 1024)
            throw std::runtime_error("GGUF: a string of " + std::to_string(n) + " bytes runs past the header");
        std::string s(reinterpret_cast<const char*>(p_ + pos_), n);
        pos_ += n;
        return s;
    }
    MetaValue value(uint32_t type, int depth = 0) {
        if (depth > 4) throw std::runtime_error("GGUF: metadata arrays nested deeper than 4");
        MetaValue v;
        v.type = type;
        switch (type) {
        case 0: v.number = scalar<uint8_t>(); break;
        case 1: v.number = scalar<int8_t>(); break;
        case 2: v.number = scalar<uint16_t>(); break;
        case 3: v.number = scalar<int16_t>(); break;
        case 4: v.number = scalar<uint32_t>(); break;
        case 5: v.number = scalar<int32_t>(); break;
        case 6: v.number = scalar<float>(); break;
        case 7: {
            const auto b = scalar<uint8_t>();
            if (b > 1) throw std::runtime_error("GGUF: a boolean value other than 0 or 1");
            v.number = b;
            break;
        }
        case 8: v.text = string(); break;
        case 9: {
            const auto sub = scalar<uint32_t>();
            const auto count = scalar<uint64_t>();
            if (count > size_ - pos_) throw std::runtime_error("GGUF: a metadata array longer than the file");
            // string and integer arrays are kept (the tokenizer's vocabulary, merges and
            // token types); others are validated and skipped
            const bool integer = sub <= 5 || sub == 10 || sub == 11;
            if (sub == 8) v.strings.reserve(count);
            if (integer) v.integers.reserve(count);
            for (uint64_t i = 0; i < count; ++i) {
                MetaValue e = value(sub, depth + 1);
                if (sub == 8) v.strings.push_back(std::move(e.text));
                else if (integer) v.integers.push_back(static_cast<int64_t>(e.number));
            }
            v.is_array = true;
            v.array_len = count;
            v.array_type = sub;
            break;
        }
        case 10: v.number = (double)scalar<uint64_t>(); break;
        case 11: v.number = (double)scalar<int64_t>(); break;
        case 12: v.number = scalar<double>(); break;
        default: throw std::runtime_error("GGUF: metadata value type " + std::to_string(type) + " is undefined");
        }
        return v;
    }
    uint64_t pos() const { return pos_; }

private:
    const uint8_t* p_;
    uint64_t size_, pos_ = 0;
};
}  // namespace

// Bytes a tensor of `n` elements occupies in the file. Block encodings (Q6_K: 210 bytes
// per 256 values, Q4_K: 144 per 256) only hold whole blocks.
uint64_t encoded_bytes(WeightType type, uint64_t n) {
    uint64_t per_block = 0, block = 1;
    switch (type) {
    case WeightType::f32: per_block = 4; break;
    case WeightType::f16:
    case WeightType::bf16: per_block = 2; break;
    case WeightType::q6_k: per_block = 210, block = 256; break;
    case WeightType::q4_k: per_block = 144, block = 256; break;
    default:
        throw std::runtime_error("GGUF: tensor encoding " + std::to_string(static_cast<uint32_t>(type)) +
                                 " is not one this reader decodes (F32, F16, BF16, Q4_K, Q6_K)");
    }
    if (n % block) throw std::runtime_error("GGUF: " + std::to_string(n) + " values are not whole 256-value blocks");
    return checked_mul(n / block, per_block);
}

namespace {

// The format's invariants over the tensor table, once every entry is read:
// - each tensor's bytes lie inside the data section, which starts at the first
//   `alignment` boundary after the table, and starts on such a boundary itself;
// - a block-encoded tensor's rows (its first dimension) are whole blocks;
// - names are unique and no two tensors share a byte.
void check_table(const std::vector<Tensor>& tensors, uint64_t alignment, uint64_t data_bytes) {
    std::vector<std::pair<uint64_t, const Tensor*>> by_offset;
    by_offset.reserve(tensors.size());
    for (const Tensor& t : tensors) {
        const bool blocked = t.type == WeightType::q6_k || t.type == WeightType::q4_k;
        if (blocked && t.shape[0] % 256)
            throw std::runtime_error("GGUF: rows of '" + t.name + "' (" + std::to_string(t.shape[0]) +
                                     " values) split a 256-value block");
        if (t.offset % alignment)
            throw std::runtime_error("GGUF: '" + t.name + "' starts off the " + std::to_string(alignment) +
                                     "-byte alignment");
        if (t.offset > data_bytes || data_bytes - t.offset < t.bytes)
            throw std::runtime_error("GGUF: '" + t.name + "' runs past the end of the file");
        by_offset.emplace_back(t.offset, &t);
    }
    std::sort(by_offset.begin(), by_offset.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
    for (size_t i = 1; i < by_offset.size(); ++i) {
        const Tensor& prev = *by_offset[i - 1].second;
        if (prev.offset + prev.bytes > by_offset[i].first)
            throw std::runtime_error("GGUF: '" + prev.name + "' and '" + by_offset[i].second->name + "' overlap");
    }
}

}  // namespace

Gguf::Gguf(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("Cannot open model: " + path);
    struct stat st;
    if (fstat(fd_, &st) != 0) {
        ::close(fd_);
        throw std::runtime_error("Cannot determine model size");
    }
    file_bytes_ = static_cast<uint64_t>(st.st_size);
    if (file_bytes_) {
        void* p = mmap(nullptr, file_bytes_, PROT_READ, MAP_PRIVATE, fd_, 0);
        if (p == MAP_FAILED) {
            ::close(fd_);
            throw std::runtime_error("Cannot map model: " + path);
        }
        base_ = static_cast<const uint8_t*>(p);
    }
    try {
        // header: magic "GGUF", version 2 or 3, tensor count, key/value count
        Cursor r(base_, file_bytes_);
        if (r.scalar<uint32_t>() != 0x46554747u) throw std::runtime_error("GGUF: missing the 'GGUF' magic");
        const auto version = r.scalar<uint32_t>();
        if (version != 2 && version != 3)
            throw std::runtime_error("GGUF: version " + std::to_string(version) + " (2 and 3 are read)");
        const auto tensor_count = r.scalar<uint64_t>(), kv_count = r.scalar<uint64_t>();
        // each entry takes at least 8 bytes, so counts beyond the file size are corrupt
        if (tensor_count > file_bytes_ / 8 || kv_count > file_bytes_ / 8)
            throw std::runtime_error("GGUF: header counts exceed the file size");
        // key/value section
        for (uint64_t i = 0; i < kv_count; ++i) {
            std::string key = r.string();
            const auto type = r.scalar<uint32_t>();
            if (!meta_.emplace(std::move(key), r.value(type)).second) throw std::runtime_error("GGUF: repeated key");
        }
        uint64_t alignment = 32;  // the format's default
        if (const MetaValue* a = meta("general.alignment")) alignment = static_cast<uint64_t>(a->number);
        if (alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20))
            throw std::runtime_error("GGUF: general.alignment must be a power of two up to 1 MiB");
        // tensor table: name, rank (1..4), dimensions, encoding, offset in the data section
        tensors_.reserve(tensor_count);
        for (uint64_t i = 0; i < tensor_count; ++i) {
            Tensor t;
            t.name = r.string();
            const auto rank = r.scalar<uint32_t>();
            if (rank < 1 || rank > 4) throw std::runtime_error("GGUF: '" + t.name + "' has rank " + std::to_string(rank));
            t.elements = 1;
            for (uint32_t d = 0; d < rank; ++d) {
                const auto n = r.scalar<uint64_t>();
                if (n == 0) throw std::runtime_error("GGUF: '" + t.name + "' has an empty dimension");
                t.shape.push_back(n);
                t.elements = checked_mul(t.elements, n);
            }
            t.type = static_cast<WeightType>(r.scalar<uint32_t>());
            t.bytes = encoded_bytes(t.type, t.elements);
            t.offset = r.scalar<uint64_t>();
            if (!index_.emplace(t.name, tensors_.size()).second)
                throw std::runtime_error("GGUF: tensor name '" + t.name + "' repeats");
            tensors_.push_back(std::move(t));
        }
        data_offset_ = (r.pos() + alignment - 1) / alignment * alignment;
        if (data_offset_ > file_bytes_) throw std::runtime_error("GGUF: the data section is missing");
        check_table(tensors_, alignment, data_bytes());
    } catch (...) {
        if (base_) munmap(const_cast<uint8_t*>(base_), file_bytes_);
        ::close(fd_);
        throw;
    }
}

Gguf::~Gguf() {
    if (base_) munmap(const_cast<uint8_t*>(base_), file_bytes_);
    if (fd_ >= 0) ::close(fd_);
}

const Tensor& Gguf::tensor(const std::string& name) const {
    auto it = index_.find(name);
    if (it == index_.end()) throw std::runtime_error("Missing tensor: " + name);
    return tensors_[it->second];
}

const MetaValue* Gguf::meta(const std::string& key) const {
    auto it = meta_.find(key);
    return it == meta_.end() ? nullptr : &it->second;
}

int Gguf::meta_int(const std::string& key) const {
    const MetaValue* v = meta(key);
    if (!v || v->is_array || v->type == 8) throw std::runtime_error("Missing metadata: " + key);
    return static_cast<int>(v->number);
}

float Gguf::meta_float(const std::string& key) const {
    const MetaValue* v = meta(key);
    if (!v || v->is_array || v->type == 8) throw std::runtime_error("Missing metadata: " + key);
    return static_cast<float>(v->number);
}

}  // namespace emprise
