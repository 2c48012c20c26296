// qwen35 GPT-2 byte-level BPE (reference src/tokenizer.cpp).
#include "tokenizer.hpp"

#include <algorithm>
#include <cstdint>
#include <limits>
#include <stdexcept>

#include "gguf.hpp"
#include "unicode_tables.hpp"

namespace emprise {

namespace {

std::string utf8(uint32_t cp) {
    std::string s;
    if (cp < 0x80) {
        s += static_cast<char>(cp);
    } else if (cp < 0x800) {
        s += static_cast<char>(0xC0 | (cp >> 6));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        s += static_cast<char>(0xE0 | (cp >> 12));
        s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
        s += static_cast<char>(0xF0 | (cp >> 18));
        s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
        s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    }
    return s;
}

// One UTF-8 sequence at s[i]: its code point and length, or 0 when it is not well
// formed (overlong forms, surrogates, values past U+10FFFF, bad or missing continuation
// bytes -- what PCRE2's UTF check rejects).
size_t next_utf8(const std::string& s, size_t i, uint32_t& cp) {
    const auto b = [&](size_t k) { return static_cast<uint8_t>(s[k]); };
    const uint8_t c = b(i);
    size_t n;
    uint32_t min;
    if (c < 0x80) {
        cp = c;
        return 1;
    } else if ((c & 0xE0) == 0xC0) {
        n = 2, cp = c & 0x1F, min = 0x80;
    } else if ((c & 0xF0) == 0xE0) {
        n = 3, cp = c & 0x0F, min = 0x800;
    } else if ((c & 0xF8) == 0xF0) {
        n = 4, cp = c & 0x07, min = 0x10000;
    } else {
        return 0;
    }
    if (i + n > s.size()) return 0;
    for (size_t k = 1; k < n; ++k) {
        if ((b(i + k) & 0xC0) != 0x80) return 0;
        cp = (cp << 6) | (b(i + k) & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return 0;
    return n;
}

bool in(const CodeRange* r, size_t n, uint32_t cp) {
    const CodeRange* e = r + n;
    const CodeRange* it = std::upper_bound(r, e, cp, [](uint32_t v, const CodeRange& x) { return v < x.lo; });
    return it != r && cp <= (it - 1)->hi;
}
bool letter(uint32_t c) { return in(k_letter, k_letter_count, c); }
bool mark(uint32_t c) { return in(k_mark, k_mark_count, c); }
bool number(uint32_t c) { return in(k_number, k_number_count, c); }
bool space(uint32_t c) { return in(k_space, k_space_count, c); }
bool newline(uint32_t c) { return c == '\r' || c == '\n'; }

// Case folding for the contraction alternative: the letters it names fold from their
// ASCII capitals, and 's' also from U+017F LATIN SMALL LETTER LONG S.
uint32_t fold(uint32_t c) {
    if (c >= 'A' && c <= 'Z') return c + 32;
    return c == 0x17F ? 's' : c;
}

// End (code-point index) of the pattern's match at i; the alternatives are tried in the
// pattern's order and the first that matches is taken, as PCRE2 does:
//   (?i:'s|'t|'re|'ve|'m|'ll|'d) | [^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+ | \p{N}
//   | ' '?[^\s\p{L}\p{M}\p{N}]+[\r\n]* | \s*[\r\n]+ | \s+(?!\S) | \s+
size_t match_at(const std::vector<uint32_t>& cp, size_t i) {
    const size_t n = cp.size();
    if (cp[i] == '\'' && i + 1 < n) {
        const uint32_t a = fold(cp[i + 1]);
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return i + 2;
        if (i + 2 < n) {
            const uint32_t b = fold(cp[i + 2]);
            if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return i + 3;
        }
    }
    const auto lm = [&](size_t k) { return k < n && (letter(cp[k]) || mark(cp[k])); };
    if (!newline(cp[i]) && !letter(cp[i]) && !number(cp[i]) && lm(i + 1)) {
        size_t j = i + 1;
        while (lm(j)) ++j;
        return j;
    }
    if (lm(i)) {
        size_t j = i;
        while (lm(j)) ++j;
        return j;
    }
    if (number(cp[i])) return i + 1;
    const auto other = [&](size_t k) {
        return k < n && !space(cp[k]) && !letter(cp[k]) && !mark(cp[k]) && !number(cp[k]);
    };
    {
        size_t j = cp[i] == ' ' && other(i + 1) ? i + 1 : i;
        if (other(j)) {
            while (other(j)) ++j;
            while (j < n && newline(cp[j])) ++j;
            return j;
        }
    }
    size_t w = i;
    while (w < n && space(cp[w])) ++w;
    if (w > i) {
        // \s*[\r\n]+: backtracking from the whole whitespace run, the last line break in it
        for (size_t k = w; k-- > i;)
            if (newline(cp[k])) return k + 1;
        // \s+(?!\S): the run, or all but its last character when text follows
        if (w == n) return w;
        if (w - i >= 2) return w - 1;
        return w;  // \s+
    }
    return i + 1;  // not reached: every code point falls in one of the classes above
}

}  // namespace

std::vector<size_t> pretokenize(const std::string& text) {
    std::vector<uint32_t> cp;
    std::vector<size_t> off;
    for (size_t i = 0; i < text.size();) {
        uint32_t c;
        const size_t len = next_utf8(text, i, c);
        if (!len) throw std::runtime_error("Invalid UTF-8 or unsupported tokenization input");
        cp.push_back(c);
        off.push_back(i);
        i += len;
    }
    off.push_back(text.size());
    std::vector<size_t> ends;
    for (size_t i = 0; i < cp.size();) {
        i = match_at(cp, i);
        ends.push_back(off[i]);
    }
    return ends;
}

Tokenizer::Tokenizer(const Gguf& g) {
    const MetaValue* model = g.meta("tokenizer.ggml.model");
    const MetaValue* pre = g.meta("tokenizer.ggml.pre");
    if (!model || model->text != "gpt2" || !pre || pre->text != "qwen35")
        throw std::runtime_error("Tokenizer currently supports qwen35 GPT-2 BPE only");
    const MetaValue* tokens = g.meta("tokenizer.ggml.tokens");
    const MetaValue* types = g.meta("tokenizer.ggml.token_type");
    const MetaValue* merges = g.meta("tokenizer.ggml.merges");
    if (!tokens || !types || !merges || tokens->array_type != 8 || merges->array_type != 8 ||
        types->integers.size() != types->array_len)
        throw std::runtime_error("Missing tokenizer metadata");
    if (types->integers.size() != tokens->strings.size()) throw std::runtime_error("Vocabulary/type size mismatch");
    for (size_t i = 0; i < merges->strings.size(); ++i) rank_.emplace(merges->strings[i], static_cast<int>(i));
    // GPT-2's byte encoder: printable Latin-1 bytes stand for themselves, the others map
    // to U+0100 on in byte order (tokenizer.cpp:68-74)
    std::unordered_map<uint32_t, uint8_t> reverse;
    uint32_t extra = 256;
    for (int b = 0; b < 256; ++b) {
        const bool direct = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
        const uint32_t c = direct ? static_cast<uint32_t>(b) : extra++;
        byte_encoder_[b] = utf8(c);
        reverse[c] = static_cast<uint8_t>(b);
    }
    const auto& vocab = tokens->strings;
    decoded_.reserve(vocab.size());
    for (size_t i = 0; i < vocab.size(); ++i) {
        const std::string& token = vocab[i];
        ids_.emplace(token, static_cast<int>(i));
        const int64_t type = types->integers[i];
        if (type == 3 || type == 4) {
            special_.emplace_back(token, static_cast<int>(i));
            decoded_.push_back(token);
            continue;
        }
        std::string bytes;
        for (size_t pos = 0; pos < token.size();) {
            uint32_t c;
            const size_t len = next_utf8(token, pos, c);
            if (!len) throw std::runtime_error("Invalid vocabulary UTF-8");
            const auto it = reverse.find(c);
            if (it == reverse.end()) {  // not byte-encoded: an unused vocabulary entry
                bytes = token;
                break;
            }
            bytes.push_back(static_cast<char>(it->second));
            pos += len;
        }
        decoded_.push_back(std::move(bytes));
    }
}

void Tokenizer::ordinary(const std::string& text, std::vector<int>& out) const {
    size_t start = 0;
    for (size_t end : pretokenize(text)) {
        std::vector<std::string> pieces;
        for (size_t i = start; i < end; ++i) pieces.push_back(byte_encoder_[static_cast<uint8_t>(text[i])]);
        // the lowest-ranked adjacent pair merges first, the leftmost of equal pairs
        while (pieces.size() > 1) {
            int best_rank = std::numeric_limits<int>::max();
            size_t best = pieces.size();
            for (size_t i = 0; i + 1 < pieces.size(); ++i) {
                const auto found = rank_.find(pieces[i] + ' ' + pieces[i + 1]);
                if (found != rank_.end() && found->second < best_rank) {
                    best_rank = found->second;
                    best = i;
                }
            }
            if (best == pieces.size()) break;
            pieces[best] += pieces[best + 1];
            pieces.erase(pieces.begin() + static_cast<std::ptrdiff_t>(best + 1));
        }
        for (const auto& piece : pieces) {
            const auto found = ids_.find(piece);
            if (found == ids_.end()) throw std::runtime_error("BPE piece missing from vocabulary");
            out.push_back(found->second);
        }
        start = end;
    }
}

std::vector<int> Tokenizer::encode(const std::string& text, bool parse_special) const {
    std::vector<int> out;
    size_t offset = 0;
    while (offset < text.size()) {
        size_t next = text.size(), length = 0;
        int id = -1;
        if (parse_special)
            for (const auto& [s, token] : special_) {
                const size_t pos = text.find(s, offset);
                if (pos < next || (pos == next && s.size() > length)) {
                    next = pos;
                    length = s.size();
                    id = token;
                }
            }
        ordinary(text.substr(offset, next - offset), out);
        if (id < 0) break;
        out.push_back(id);
        offset = next + length;
    }
    return out;
}

std::string Tokenizer::decode(int token) const {
    if (token < 0 || static_cast<size_t>(token) >= decoded_.size()) throw std::out_of_range("Invalid token ID");
    return decoded_[static_cast<size_t>(token)];
}

std::string Tokenizer::chat_prompt(const std::string& user) const {
    return "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n";
}

}  // namespace emprise
