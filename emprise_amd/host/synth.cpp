// Deterministic synthetic qwen35 GGUF writer (benchmark/test inputs).
//
// Every tensor draws from its own counter-based SplitMix64 stream, keyed by the seed
// and the tensor name, so the bytes are the same for any thread count or host.
// Normals are Irwin-Hall sums of twelve 16-bit uniforms (IEEE adds only).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "emprise_host.h"
#include "tokenizer.hpp"

namespace emprise {

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Stream {
    uint64_t key;
    uint64_t word(uint64_t i) const { return mix(key + (i + 1) * kGolden); }
    // N(0,1) approximation: twelve 16-bit uniforms from three words
    double normal(uint64_t i) const {
        double s = 0;
        for (int w = 0; w < 3; ++w) {
            const uint64_t v = word(i * 3 + w);
            for (int k = 0; k < 4; ++k) s += (double((v >> (16 * k)) & 0xffff) + 0.5) / 65536.0;
        }
        return s - 6.0;
    }
};

Stream stream_for(uint64_t seed, const std::string& name) {
    uint64_t h = 0xcbf29ce484222325ull;  // FNV-1a of the tensor name
    for (unsigned char c : name) h = (h ^ c) * 0x100000001b3ull;
    return Stream{mix(seed ^ h)};
}

// fp32 -> fp16 bits, round to nearest even (values here are finite and >= 0).
uint16_t half_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000;
    x &= 0x7fffffff;
    if (x >= 0x47800000) return static_cast<uint16_t>(sign | 0x7c00);  // overflow -> inf
    if (x < 0x38800000) {                                                // subnormal half
        if (x < 0x33000000) return static_cast<uint16_t>(sign);
        const uint32_t mant = (x & 0x7fffff) | 0x800000;
        const int shift = 113 - static_cast<int>(x >> 23) + 13;
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return static_cast<uint16_t>(sign | h);
    }
    uint32_t h = ((x - 0x38000000) >> 13);
    const uint32_t rem = x & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h;
    return static_cast<uint16_t>(sign | h);
}

struct TensorSpec {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t type;
    int kind;  // 0 matrix, 1 norm (1+0.02N), 2 ssm_a, 3 dt, 4 conv
    uint64_t offset = 0, bytes = 0;
};

uint64_t elements(const TensorSpec& t) {
    uint64_t n = 1;
    for (auto s : t.shape) n *= s;
    return n;
}

uint64_t bytes_of(uint32_t type, uint64_t n) {
    switch (type) {
    case EMPRISE_F32: return n * 4;
    case EMPRISE_Q6_K: return n / 256 * 210;
    case EMPRISE_Q4_K: return n / 256 * 144;
    default: throw std::runtime_error("synthetic writer: unsupported type");
    }
}

void fill(const TensorSpec& t, uint64_t seed, uint8_t* out) {
    const Stream s = stream_for(seed, t.name);
    const Stream sn{mix(s.key ^ 0xD1B54A32D192ED03ull)};  // normals of the block scales
    const uint64_t n = elements(t);
    if (t.type == EMPRISE_Q6_K) {
        const int64_t blocks = static_cast<int64_t>(n / 256);
#pragma omp parallel for schedule(static)
        for (int64_t b = 0; b < blocks; ++b) {
            uint8_t* blk = out + b * 210;
            const uint64_t w0 = static_cast<uint64_t>(b) * 26;
            for (int i = 0; i < 24; ++i) {  // ql[128] qh[64]: uniform bytes
                const uint64_t v = s.word(w0 + i);
                std::memcpy(blk + 8 * i, &v, 8);
            }
            for (int i = 0; i < 2; ++i) {  // sub-scales uniform in [-32, 31]
                const uint64_t v = s.word(w0 + 24 + i);
                for (int k = 0; k < 8; ++k) blk[192 + 8 * i + k] = static_cast<uint8_t>(int8_t(int((v >> (8 * k)) & 63) - 32));
            }
            const uint16_t d = half_rne(static_cast<float>(std::fabs(sn.normal(static_cast<uint64_t>(b))) * 2e-4));
            std::memcpy(blk + 208, &d, 2);
        }
    } else if (t.type == EMPRISE_Q4_K) {
        const int64_t blocks = static_cast<int64_t>(n / 256);
#pragma omp parallel for schedule(static)
        for (int64_t b = 0; b < blocks; ++b) {
            uint8_t* blk = out + b * 144;
            const uint64_t w0 = static_cast<uint64_t>(b) * 18;
            for (int i = 0; i < 18; ++i) {  // everything uniform first
                const uint64_t v = s.word(w0 + i);
                std::memcpy(blk + 8 * i, &v, 8);
            }
            const uint16_t d = half_rne(static_cast<float>(std::fabs(sn.normal(2 * static_cast<uint64_t>(b))) * 1e-3));
            const uint16_t dm = half_rne(static_cast<float>(std::fabs(sn.normal(2 * static_cast<uint64_t>(b) + 1)) * 1e-3));
            std::memcpy(blk, &d, 2);
            std::memcpy(blk + 2, &dm, 2);
        }
    } else {
        std::vector<float> v(n);
        for (uint64_t i = 0; i < n; ++i) {
            const double z = s.normal(i);
            double x = 0;
            switch (t.kind) {
            case 1: x = 1.0 + 0.02 * z; break;
            case 2: x = -std::exp(0.5 * z - 2.0); break;
            case 3: x = 0.5 * z - 1.0; break;
            case 4: x = 0.5 * z; break;
            default: x = 0.05 * z; break;
            }
            v[i] = static_cast<float>(x);
        }
        std::memcpy(out, v.data(), n * 4);
    }
}

// The synthetic tokenizer: GPT-2's byte encoder strings for the 256 bytes, then the
// merges of a byte-pair training run on kCorpus (the most frequent adjacent pair over
// the pre-tokenizer's pieces, ties to the smaller pair string), then the chat template's
// special tokens, then numbered control tokens up to `vocab`.
const char* const kCorpus =
    "The quick brown fox jumps over the lazy dog. The dog sleeps; the fox runs away!\n"
    "Explain how a refrigerator works. A refrigerator moves heat from the inside to the "
    "outside: the compressor squeezes the refrigerant, which gets hot, and the coils let "
    "the heat go. It's cold inside because the liquid evaporates and takes heat with it.\n"
    "In 2024 there were 365 days, 12 months and 52 weeks; 3.14159 is pi, 2.71828 is e.\n"
    "    def add(a, b):\n        return a + b  # they'll add, we've seen it, I'd say\n"
    "Grüße aus München! Ça va? Numbers: 0 1 2 3 4 5 6 7 8 9, 10 100 1000.\n\n";
const char* const kSpecials[] = {"<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>"};

struct SynthVocab {
    std::vector<std::string> tokens, merges;
    std::vector<int32_t> types;
};

SynthVocab synth_vocab(int vocab) {
    SynthVocab v;
    std::string enc[256];
    int extra = 256;
    for (int b = 0; b < 256; ++b) {
        const bool direct = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
        const uint32_t c = direct ? static_cast<uint32_t>(b) : static_cast<uint32_t>(extra++);
        enc[b] = c < 0x80 ? std::string(1, static_cast<char>(c))
                          : std::string{static_cast<char>(0xC0 | (c >> 6)), static_cast<char>(0x80 | (c & 0x3F))};
        v.tokens.push_back(enc[b]);
        v.types.push_back(1);
    }
    // words of the corpus as sequences of byte-encoded symbols, with their counts
    const std::string text = kCorpus;
    std::map<std::vector<std::string>, int> words;
    size_t start = 0;
    for (size_t end : pretokenize(text)) {
        std::vector<std::string> w;
        for (size_t i = start; i < end; ++i) w.push_back(enc[static_cast<uint8_t>(text[i])]);
        ++words[w];
        start = end;
    }
    const int specials = static_cast<int>(sizeof kSpecials / sizeof kSpecials[0]);
    const int budget = std::min(400, vocab - 256 - specials);
    for (int m = 0; m < budget; ++m) {
        std::map<std::pair<std::string, std::string>, int> freq;
        for (const auto& [w, n] : words)
            for (size_t i = 0; i + 1 < w.size(); ++i) freq[{w[i], w[i + 1]}] += n;
        if (freq.empty()) break;
        auto best = freq.begin();
        for (auto it = freq.begin(); it != freq.end(); ++it)
            if (it->second > best->second) best = it;  // map order: ties keep the smaller pair
        const auto [a, b] = best->first;
        v.merges.push_back(a + " " + b);
        v.tokens.push_back(a + b);
        v.types.push_back(1);
        std::map<std::vector<std::string>, int> next;
        for (const auto& [w, n] : words) {
            std::vector<std::string> r;
            for (size_t i = 0; i < w.size(); ++i) {
                if (i + 1 < w.size() && w[i] == a && w[i + 1] == b) {
                    r.push_back(a + b);
                    ++i;
                } else {
                    r.push_back(w[i]);
                }
            }
            next[r] += n;
        }
        words.swap(next);
    }
    for (const char* sp : kSpecials) {
        v.tokens.push_back(sp);
        v.types.push_back(3);
    }
    for (int i = 0; static_cast<int>(v.tokens.size()) < vocab; ++i) {
        v.tokens.push_back("<|control_" + std::to_string(i) + "|>");
        v.types.push_back(3);
    }
    if (static_cast<int>(v.tokens.size()) != vocab) throw std::invalid_argument("synthetic vocabulary too small");
    return v;
}

struct Writer {
    FILE* f;
    void raw(const void* p, size_t n) {
        if (fwrite(p, 1, n, f) != n) throw std::runtime_error("synthetic writer: write failed");
    }
    template <class T> void put(T v) { raw(&v, sizeof v); }
    void str(const std::string& s) {
        put<uint64_t>(s.size());
        raw(s.data(), s.size());
    }
    void kv_u32(const std::string& k, uint32_t v) {
        str(k);
        put<uint32_t>(4);
        put<uint32_t>(v);
    }
    void kv_f32(const std::string& k, float v) {
        str(k);
        put<uint32_t>(6);
        put<float>(v);
    }
    void kv_str(const std::string& k, const std::string& v) {
        str(k);
        put<uint32_t>(8);
        str(v);
    }
    void kv_u64(const std::string& k, uint64_t v) {
        str(k);
        put<uint32_t>(10);
        put<uint64_t>(v);
    }
    void kv_strings(const std::string& k, const std::vector<std::string>& v) {
        str(k);
        put<uint32_t>(9);
        put<uint32_t>(8);
        put<uint64_t>(v.size());
        for (const auto& e : v) str(e);
    }
    void kv_i32s(const std::string& k, const std::vector<int32_t>& v) {
        str(k);
        put<uint32_t>(9);
        put<uint32_t>(5);
        put<uint64_t>(v.size());
        for (int32_t e : v) put<int32_t>(e);
    }
};

}  // namespace

void synth_write(const emprise_synth_config& c, const std::string& path) {
    if (c.hidden % 256 || c.ffn % 256 || (c.value_heads * c.state_dim) % 256 || (c.heads * c.head_dim) % 256)
        throw std::invalid_argument("synthetic shapes must keep matrix rows in whole 256-blocks");
    if (c.full_attention_interval < 1 || c.layers < 1) throw std::invalid_argument("bad layer pattern");
    const uint64_t H = c.hidden, kd = uint64_t(c.key_heads) * c.state_dim, vd = uint64_t(c.value_heads) * c.state_dim;
    const uint64_t ch = 2 * kd + vd, qd = uint64_t(c.heads) * c.head_dim * 2, kvd = uint64_t(c.kv_heads) * c.head_dim;
    auto mtype = [&](const std::string& n) -> uint32_t {
        if (c.q4_k_m_mix) return (n.find("attn_v.") != std::string::npos || n.find("ffn_down.") != std::string::npos)
                                     ? EMPRISE_Q6_K : EMPRISE_Q4_K;
        return c.matrix_type;
    };
    std::vector<TensorSpec> ts;
    auto mat = [&](const std::string& n, uint64_t cols, uint64_t rows) { ts.push_back({n, {cols, rows}, mtype(n), 0}); };
    auto vec = [&](const std::string& n, std::vector<uint64_t> shape, int kind) { ts.push_back({n, shape, EMPRISE_F32, kind}); };
    mat("token_embd.weight", H, c.vocab);
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const bool attn = (l + 1) % c.full_attention_interval == 0;
        vec(p + "attn_norm.weight", {H}, 1);
        if (attn) {
            mat(p + "attn_q.weight", H, qd);
            mat(p + "attn_k.weight", H, kvd);
            mat(p + "attn_v.weight", H, kvd);
            mat(p + "attn_output.weight", uint64_t(c.heads) * c.head_dim, H);
            vec(p + "attn_q_norm.weight", {uint64_t(c.head_dim)}, 1);
            vec(p + "attn_k_norm.weight", {uint64_t(c.head_dim)}, 1);
        } else {
            mat(p + "attn_qkv.weight", H, ch);
            mat(p + "attn_gate.weight", H, vd);
            mat(p + "ssm_alpha.weight", H, c.value_heads);
            mat(p + "ssm_beta.weight", H, c.value_heads);
            mat(p + "ssm_out.weight", vd, H);
            vec(p + "ssm_conv1d.weight", {uint64_t(c.conv_width), ch}, 4);
            vec(p + "ssm_a", {uint64_t(c.value_heads)}, 2);
            vec(p + "ssm_dt.bias", {uint64_t(c.value_heads)}, 3);
            vec(p + "ssm_norm.weight", {uint64_t(c.state_dim)}, 1);
        }
        vec(p + "post_attention_norm.weight", {H}, 1);
        mat(p + "ffn_gate.weight", H, c.ffn);
        mat(p + "ffn_up.weight", H, c.ffn);
        mat(p + "ffn_down.weight", c.ffn, H);
    }
    if (c.mtp) {
        // the next-n block after the main layers: an attention layer + FFN, fed by
        // eh_proj over [enorm(embedding) | hnorm(hidden)]
        const std::string p = "blk." + std::to_string(c.layers) + ".";
        vec(p + "nextn.enorm.weight", {H}, 1);
        vec(p + "nextn.hnorm.weight", {H}, 1);
        mat(p + "nextn.eh_proj.weight", 2 * H, H);
        vec(p + "nextn.shared_head_norm.weight", {H}, 1);
        vec(p + "attn_norm.weight", {H}, 1);
        mat(p + "attn_q.weight", H, qd);
        mat(p + "attn_k.weight", H, kvd);
        mat(p + "attn_v.weight", H, kvd);
        mat(p + "attn_output.weight", uint64_t(c.heads) * c.head_dim, H);
        vec(p + "attn_q_norm.weight", {uint64_t(c.head_dim)}, 1);
        vec(p + "attn_k_norm.weight", {uint64_t(c.head_dim)}, 1);
        vec(p + "post_attention_norm.weight", {H}, 1);
        mat(p + "ffn_gate.weight", H, c.ffn);
        mat(p + "ffn_up.weight", H, c.ffn);
        mat(p + "ffn_down.weight", c.ffn, H);
    }
    vec("output_norm.weight", {H}, 1);
    mat("output.weight", H, c.vocab);
    const uint64_t align = 32;
    uint64_t off = 0;
    for (auto& t : ts) {
        t.bytes = bytes_of(t.type, elements(t));
        t.offset = off;
        off = (off + t.bytes + align - 1) / align * align;
    }

    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("Cannot write " + path);
    Writer w{f};
    try {
        SynthVocab sv;
        if (c.tokenizer) sv = synth_vocab(c.vocab);
        const int kv_count = 22 + (c.mtp ? 1 : 0) + (c.tokenizer ? 4 : 0);
        w.put<uint32_t>(0x46554747u);
        w.put<uint32_t>(3);
        w.put<uint64_t>(ts.size());
        w.put<uint64_t>(kv_count);
        w.kv_str("general.architecture", "qwen35");
        w.kv_u32("general.alignment", static_cast<uint32_t>(align));
        w.kv_u64("emprise.synthetic.seed", c.seed);
        w.kv_u32("qwen35.embedding_length", static_cast<uint32_t>(c.hidden));
        w.kv_u32("qwen35.block_count", static_cast<uint32_t>(c.layers + (c.mtp ? 1 : 0)));
        if (c.mtp) w.kv_u32("qwen35.nextn_predict_layers", 1);
        w.kv_u32("qwen35.feed_forward_length", static_cast<uint32_t>(c.ffn));
        w.kv_u32("qwen35.context_length", static_cast<uint32_t>(c.context_length));
        w.kv_u32("qwen35.attention.head_count", static_cast<uint32_t>(c.heads));
        w.kv_u32("qwen35.attention.head_count_kv", static_cast<uint32_t>(c.kv_heads));
        w.kv_u32("qwen35.attention.key_length", static_cast<uint32_t>(c.head_dim));
        w.kv_u32("qwen35.attention.value_length", static_cast<uint32_t>(c.head_dim));
        w.kv_u32("qwen35.rope.dimension_count", static_cast<uint32_t>(c.rotary));
        w.kv_f32("qwen35.rope.freq_base", c.rope_base);
        w.kv_f32("qwen35.attention.layer_norm_rms_epsilon", c.eps);
        w.kv_u32("qwen35.ssm.group_count", static_cast<uint32_t>(c.key_heads));
        w.kv_u32("qwen35.ssm.time_step_rank", static_cast<uint32_t>(c.value_heads));
        w.kv_u32("qwen35.ssm.state_size", static_cast<uint32_t>(c.state_dim));
        w.kv_u32("qwen35.ssm.conv_kernel", static_cast<uint32_t>(c.conv_width));
        w.kv_u32("qwen35.ssm.inner_size", static_cast<uint32_t>(vd));
        w.kv_u32("qwen35.full_attention_interval", static_cast<uint32_t>(c.full_attention_interval));
        w.kv_u32("tokenizer.ggml.eos_token_id", static_cast<uint32_t>(c.eos));
        if (c.tokenizer) {
            w.kv_str("tokenizer.ggml.model", "gpt2");
            w.kv_str("tokenizer.ggml.pre", "qwen35");
            w.kv_strings("tokenizer.ggml.tokens", sv.tokens);
            w.kv_i32s("tokenizer.ggml.token_type", sv.types);
            w.kv_strings("tokenizer.ggml.merges", sv.merges);
        } else {
            w.kv_str("tokenizer.ggml.model", "none");
        }
        for (const auto& t : ts) {
            w.str(t.name);
            w.put<uint32_t>(static_cast<uint32_t>(t.shape.size()));
            for (auto s : t.shape) w.put<uint64_t>(s);
            w.put<uint32_t>(t.type);
            w.put<uint64_t>(t.offset);
        }
        long pos = std::ftell(f);
        const uint64_t data_start = (static_cast<uint64_t>(pos) + align - 1) / align * align;
        std::vector<uint8_t> pad(align, 0);
        w.raw(pad.data(), data_start - static_cast<uint64_t>(pos));
        uint64_t written = 0;
        std::vector<uint8_t> buf;
        for (const auto& t : ts) {
            if (written < t.offset) {
                w.raw(pad.data(), t.offset - written);
                written = t.offset;
            }
            buf.resize(t.bytes);
            fill(t, c.seed, buf.data());
            w.raw(buf.data(), buf.size());
            written += t.bytes;
        }
        const uint64_t end = (written + align - 1) / align * align;
        if (end > written) w.raw(pad.data(), end - written);
    } catch (...) {
        std::fclose(f);
        throw;
    }
    if (std::fclose(f) != 0) throw std::runtime_error("synthetic writer: close failed");
}

void synth_prompt(uint64_t seed, int vocab, size_t n, int* ids) {
    const Stream s = stream_for(seed, "prompt");
    for (size_t i = 0; i < n; ++i) ids[i] = static_cast<int>(s.word(i) % static_cast<uint64_t>(vocab));
}

}  // namespace emprise
