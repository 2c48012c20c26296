// GGUF reader: header, metadata, tensor table and the validation rules of the
// reference (src/gguf.cpp:87-147), over a read-only memory map.
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
    if (b && a > std::numeric_limits<uint64_t>::max() / b) throw std::runtime_error("GGUF dimension overflow");
    return a * b;
}

class Cursor {
public:
    Cursor(const uint8_t* p, uint64_t size) : p_(p), size_(size) {}
    template <class T> T scalar() {
        if (size_ - pos_ < sizeof(T) || pos_ > size_) throw std::runtime_error("Truncated GGUF header");
        T v;
        std::memcpy(&v, p_ + pos_, sizeof(T));
        pos_ += sizeof(T);
        return v;
    }
    std::string string() {
        const uint64_t n = scalar<uint64_t>();
        if (n > size_ - pos_ || n > 64ull * 1024 * 1024)
            throw std::runtime_error("Invalid GGUF string length: " + std::to_string(n));
        std::string s(reinterpret_cast<const char*>(p_ + pos_), n);
        pos_ += n;
        return s;
    }
    MetaValue value(uint32_t type, int depth = 0) {
        if (depth > 4) throw std::runtime_error("Excessive metadata nesting");
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
            if (b > 1) throw std::runtime_error("Invalid boolean metadata");
            v.number = b;
            break;
        }
        case 8: v.text = string(); break;
        case 9: {
            const auto sub = scalar<uint32_t>();
            const auto count = scalar<uint64_t>();
            if (count > size_ || count > 10000000) throw std::runtime_error("Invalid metadata array");
            for (uint64_t i = 0; i < count; ++i) (void)value(sub, depth + 1);
            v.is_array = true;
            v.array_len = count;
            break;
        }
        case 10: v.number = (double)scalar<uint64_t>(); break;
        case 11: v.number = (double)scalar<int64_t>(); break;
        case 12: v.number = scalar<double>(); break;
        default: throw std::runtime_error("Unknown GGUF metadata type");
        }
        return v;
    }
    uint64_t pos() const { return pos_; }

private:
    const uint8_t* p_;
    uint64_t size_, pos_ = 0;
};
}  // namespace

uint64_t encoded_bytes(WeightType type, uint64_t n) {
    switch (type) {
    case WeightType::f32: return checked_mul(n, 4);
    case WeightType::f16:
    case WeightType::bf16: return checked_mul(n, 2);
    case WeightType::q6_k:
        if (n % 256) throw std::runtime_error("Q6_K requires blocks of 256 elements");
        return checked_mul(n / 256, 210);
    case WeightType::q4_k:
        if (n % 256) throw std::runtime_error("Q4_K requires blocks of 256 elements");
        return checked_mul(n / 256, 144);
    default: throw std::runtime_error("Unsupported GGUF tensor encoding: " + std::to_string(static_cast<uint32_t>(type)));
    }
}

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
        Cursor r(base_, file_bytes_);
        if (r.scalar<uint32_t>() != 0x46554747u) throw std::runtime_error("Not a GGUF file");
        const auto version = r.scalar<uint32_t>();
        if (version != 2 && version != 3) throw std::runtime_error("Unsupported GGUF version");
        const auto nt = r.scalar<uint64_t>(), nkv = r.scalar<uint64_t>();
        if (nt > 1000000 || nkv > 1000000) throw std::runtime_error("Excessive header entries");
        for (uint64_t i = 0; i < nkv; ++i) {
            auto key = r.string();
            if (meta_.count(key)) throw std::runtime_error("Duplicate metadata key");
            const auto type = r.scalar<uint32_t>();
            meta_[key] = r.value(type);
        }
        uint64_t alignment = 32;
        if (auto* a = meta("general.alignment")) alignment = static_cast<uint64_t>(a->number);
        if (!alignment || alignment > 1024 * 1024 || (alignment & (alignment - 1)))
            throw std::runtime_error("Invalid GGUF alignment");
        tensors_.reserve(nt);
        for (uint64_t i = 0; i < nt; ++i) {
            Tensor t;
            t.name = r.string();
            const auto nd = r.scalar<uint32_t>();
            if (!nd || nd > 4) throw std::runtime_error("Unsupported tensor rank");
            t.elements = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const auto n = r.scalar<uint64_t>();
                if (!n) throw std::runtime_error("Zero tensor dimension");
                t.shape.push_back(n);
                t.elements = checked_mul(t.elements, n);
            }
            t.type = static_cast<WeightType>(r.scalar<uint32_t>());
            t.bytes = encoded_bytes(t.type, t.elements);
            if ((t.type == WeightType::q6_k || t.type == WeightType::q4_k) && t.shape[0] % 256)
                throw std::runtime_error("Q6_K row must contain whole blocks");
            t.offset = r.scalar<uint64_t>();
            if (t.offset % alignment) throw std::runtime_error("Misaligned tensor offset");
            if (!index_.emplace(t.name, tensors_.size()).second) throw std::runtime_error("Duplicate tensor name");
            tensors_.push_back(std::move(t));
        }
        data_offset_ = (r.pos() + alignment - 1) / alignment * alignment;
        if (data_offset_ > file_bytes_) throw std::runtime_error("Missing tensor data");
        std::vector<std::pair<uint64_t, uint64_t>> extents;
        for (const auto& t : tensors_) {
            if (t.offset > data_bytes() || t.bytes > data_bytes() - t.offset)
                throw std::runtime_error("Truncated tensor: " + t.name);
            extents.emplace_back(t.offset, t.offset + t.bytes);
        }
        std::sort(extents.begin(), extents.end());
        for (size_t i = 1; i < extents.size(); ++i)
            if (extents[i].first < extents[i - 1].second) throw std::runtime_error("Overlapping tensor extents");
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
