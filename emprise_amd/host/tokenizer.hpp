// The qwen35 GPT-2 byte-level BPE tokenizer over a GGUF's tokenizer metadata (reference
// include/emprise/tokenizer.hpp, src/tokenizer.cpp:18-129). The reference splits text
// with a PCRE2 pattern (tokenizer.cpp:112); here the same pattern's alternatives are a
// hand-written scanner over generated Unicode class tables (unicode_tables.cpp).
#pragma once
#include <array>
#include <cstddef>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace emprise {

class Gguf;

class Tokenizer {
public:
    // Throws std::runtime_error unless tokenizer.ggml.model is "gpt2" and
    // tokenizer.ggml.pre is "qwen35" (tokenizer.cpp:62-63).
    explicit Tokenizer(const Gguf& g);
    // Tokenizer::encode (tokenizer.cpp:114-131): with parse_special, special tokens
    // (token types 3 and 4) found verbatim in the text are emitted as their ids, the
    // earliest first and the longest at one position; the text between them is split by
    // the pre-tokenizer and byte-pair merged by rank.
    std::vector<int> encode(const std::string& text, bool parse_special) const;
    // Tokenizer::decode (tokenizer.cpp:132-135): the token's bytes.
    std::string decode(int token) const;
    // Tokenizer::chat_prompt (tokenizer.cpp:136-139): the single-turn text template.
    std::string chat_prompt(const std::string& user) const;
    size_t size() const { return decoded_.size(); }

private:
    void ordinary(const std::string& text, std::vector<int>& out) const;
    std::vector<std::string> decoded_;
    std::vector<std::pair<std::string, int>> special_;
    std::unordered_map<std::string, int> ids_, rank_;
    std::array<std::string, 256> byte_encoder_;
};

// The pre-tokenizer alone: the byte offsets at which the pieces of `text` end (the
// pattern of tokenizer.cpp:112 matched repeatedly, anchored at the previous end). Throws
// std::runtime_error on invalid UTF-8.
std::vector<size_t> pretokenize(const std::string& text);

}  // namespace emprise
