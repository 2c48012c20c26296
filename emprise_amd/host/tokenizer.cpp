// qwen35 GPT-2 byte-level BPE (reference src/tokenizer.cpp).
#include "tokenizer.hpp"

#include <algorithm>
#include <cstdint>
#include <functional>
#include <queue>
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

// The byte-level alphabet of GPT-2 BPE: a byte whose Latin-1 character is printable and
// not a space ('!'..'~', U+00A1..U+00AC, U+00AE..U+00FF) is written as that character;
// the other 68 bytes, taken in increasing order, are written as U+0100, U+0101, ... so
// every byte has a visible single-code-point spelling.
std::array<uint32_t, 256> byte_alphabet() {
    std::array<uint32_t, 256> cp{};
    uint32_t spare = 0x100;
    for (uint32_t b = 0; b < 256; ++b) {
        const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || b >= 0xAE;
        cp[b] = printable ? b : spare++;
    }
    return cp;
}

Tokenizer::Tokenizer(const Gguf& g) {
    const MetaValue* kind = g.meta("tokenizer.ggml.model");
    const MetaValue* pre = g.meta("tokenizer.ggml.pre");
    if (!kind || kind->text != "gpt2" || !pre || pre->text != "qwen35")
        throw std::runtime_error("tokenizer: only qwen35 GPT-2 BPE vocabularies are supported");
    const MetaValue* vocab = g.meta("tokenizer.ggml.tokens");
    const MetaValue* kinds = g.meta("tokenizer.ggml.token_type");
    const MetaValue* merges = g.meta("tokenizer.ggml.merges");
    if (!vocab || !kinds || !merges || vocab->array_type != 8 || merges->array_type != 8 ||
        kinds->integers.size() != kinds->array_len)
        throw std::runtime_error("tokenizer: tokens, token types or merges missing from the metadata");
    if (kinds->integers.size() != vocab->strings.size())
        throw std::runtime_error("tokenizer: token and token-type arrays differ in length");

    // merge rank = index in the merges list ("left right", one space)
    rank_.reserve(merges->strings.size());
    for (size_t r = 0; r < merges->strings.size(); ++r) rank_.emplace(merges->strings[r], static_cast<int>(r));

    const std::array<uint32_t, 256> alphabet = byte_alphabet();
    std::unordered_map<uint32_t, uint8_t> byte_of;
    for (int b = 0; b < 256; ++b) {
        byte_encoder_[b] = utf8(alphabet[b]);
        byte_of.emplace(alphabet[b], static_cast<uint8_t>(b));
    }

    // id of every vocabulary string; the bytes each id decodes to. Control (3) and
    // user-defined (4) tokens are matched and decoded as their literal text; an ordinary
    // entry that is not spelled in the byte alphabet decodes as its own text too.
    const auto& words = vocab->strings;
    ids_.reserve(words.size());
    decoded_.resize(words.size());
    for (size_t id = 0; id < words.size(); ++id) {
        const std::string& w = words[id];
        ids_.emplace(w, static_cast<int>(id));
        const int64_t kind_id = kinds->integers[id];
        if (kind_id == 3 || kind_id == 4) {
            special_.emplace_back(w, static_cast<int>(id));
            decoded_[id] = w;
            continue;
        }
        std::string raw;
        bool in_alphabet = true;
        for (size_t at = 0; at < w.size() && in_alphabet;) {
            uint32_t c = 0;
            const size_t len = next_utf8(w, at, c);
            if (!len) throw std::runtime_error("tokenizer: a vocabulary entry is not well-formed UTF-8");
            const auto hit = byte_of.find(c);
            in_alphabet = hit != byte_of.end();
            if (in_alphabet) raw.push_back(static_cast<char>(hit->second));
            at += len;
        }
        decoded_[id] = in_alphabet ? std::move(raw) : w;
    }
    // longest first, so the first special token that matches at a position is its longest
    std::stable_sort(special_.begin(), special_.end(),
                     [](const auto& x, const auto& y) { return x.first.size() > y.first.size(); });
}

// Byte-pair merging of one pre-tokenized piece. The piece starts as its bytes in the byte
// alphabet; the merge of lowest rank among all adjacent symbol pairs is applied, to the
// leftmost such pair, until no adjacent pair has a rank. Symbols sit in a doubly linked
// list in their original order; candidate pairs wait in a min-heap ordered by (rank,
// position of the left symbol), and a popped candidate is skipped when either symbol has
// changed since it was pushed.
void Tokenizer::ordinary(const std::string& text, std::vector<int>& out) const {
    struct Sym {
        std::string s;
        int prev, next;
        uint32_t version;  // bumped on every change, invalidating queued pairs
    };
    struct Cand {
        int rank, left;
        uint32_t vl, vr;
        bool operator>(const Cand& o) const { return rank != o.rank ? rank > o.rank : left > o.left; }
    };
    size_t start = 0;
    for (size_t end : pretokenize(text)) {
        const int n = static_cast<int>(end - start);
        std::vector<Sym> sym(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i)
            sym[i] = {byte_encoder_[static_cast<uint8_t>(text[start + static_cast<size_t>(i)])], i - 1,
                      i + 1 < n ? i + 1 : -1, 0};
        std::priority_queue<Cand, std::vector<Cand>, std::greater<Cand>> heap;
        auto offer = [&](int l) {
            const int r = l >= 0 ? sym[l].next : -1;
            if (l < 0 || r < 0) return;
            const auto hit = rank_.find(sym[l].s + ' ' + sym[r].s);
            if (hit != rank_.end()) heap.push({hit->second, l, sym[l].version, sym[r].version});
        };
        for (int i = 0; i + 1 < n; ++i) offer(i);
        while (!heap.empty()) {
            const Cand c = heap.top();
            heap.pop();
            const int r = sym[c.left].next;
            if (r < 0 || sym[c.left].version != c.vl || sym[r].version != c.vr || sym[c.left].s.empty()) continue;
            // merge r into its left neighbour
            sym[c.left].s += sym[r].s;
            ++sym[c.left].version;
            sym[r].s.clear();
            ++sym[r].version;
            sym[c.left].next = sym[r].next;
            if (sym[r].next >= 0) sym[sym[r].next].prev = c.left;
            offer(sym[c.left].prev);
            offer(c.left);
        }
        for (int i = n ? 0 : -1; i >= 0; i = sym[i].next) {
            const auto hit = ids_.find(sym[i].s);
            if (hit == ids_.end()) throw std::runtime_error("tokenizer: a merged piece has no vocabulary id");
            out.push_back(hit->second);
        }
        start = end;
    }
}

// Special tokens are taken where they occur in the text (the earliest occurrence first,
// the longest token where several start at one byte); the text between them goes through
// the pre-tokenizer and the merges.
std::vector<int> Tokenizer::encode(const std::string& text, bool parse_special) const {
    std::vector<int> out;
    size_t plain = 0;  // start of the text not yet encoded
    if (parse_special && !special_.empty()) {
        for (size_t at = 0; at < text.size();) {
            int hit = -1;
            for (size_t k = 0; k < special_.size() && hit < 0; ++k) {
                const std::string& w = special_[k].first;
                if (!w.empty() && text.compare(at, w.size(), w) == 0) hit = static_cast<int>(k);
            }
            if (hit < 0) {
                ++at;
                continue;
            }
            ordinary(text.substr(plain, at - plain), out);
            out.push_back(special_[static_cast<size_t>(hit)].second);
            at += special_[static_cast<size_t>(hit)].first.size();
            plain = at;
        }
    }
    ordinary(text.substr(plain), out);
    return out;
}

std::string Tokenizer::decode(int token) const {
    if (token < 0 || static_cast<size_t>(token) >= decoded_.size()) throw std::out_of_range("Invalid token ID");
    return decoded_[static_cast<size_t>(token)];
}

// The single-turn template (tokenizer.cpp:136-139): the user turn, then an assistant turn
// that opens with an empty thinking block.
std::string Tokenizer::chat_prompt(const std::string& user) const {
    static const std::string open = "<|im_start|>user\n";
    static const std::string close = "<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n";
    return open + user + close;
}

}  // namespace emprise
