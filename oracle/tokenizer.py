"""CPU restatement of the reference's qwen35 GPT-2 byte-level BPE tokenizer
(v1.1 src/tokenizer.cpp:18-139), over a GGUF's tokenizer.ggml.* metadata.

TEST INFRASTRUCTURE ONLY: the checker of emprise_amd's C++ tokenizer in tests/. The
product never imports it.

The pre-tokenizer is the reference's PCRE2 pattern (tokenizer.cpp:112) run by the
`regex` module, with \\s spelled out as PCRE2's UCP space (\\p{Z} plus \\h and \\v:
U+0009-000D, U+0085, U+180E), which is not exactly `regex`'s own \\s. The merge loop,
special-token search, byte encoder and decode table follow tokenizer.cpp:25-52, :60-105
and :114-139 step by step. Pinned by tests/test_oracle_refmodel.py against the
reference's own compiled tokenizer.cpp (where oracle/_ref is built), by
tests/test_tokenizer.py against the HF `tokenizers` library (an independent byte-level
BPE) on the same vocabulary and merges, by the byte round trip, and by pre-tokenizer
splits derived by hand from the pattern.
"""
import struct

import regex

_S = r"\p{Z}\t\n\u000b\f\r\u0085\u180e"
PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
           r"| ?[^" + _S + r"\p{L}\p{M}\p{N}]+[\r\n]*|[" + _S + r"]*[\r\n]+|[" + _S + r"]+(?![^" + _S + r"])"
           r"|[" + _S + r"]+")
_RX = regex.compile(PATTERN)


def read_metadata(path) -> dict:
    """The key/value section of a GGUF file (scalars, strings, arrays of either)."""
    with open(path, "rb") as f:
        data = f.read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, data, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0]

    def string():
        nonlocal pos
        n = take("Q")
        s = data[pos:pos + n].decode()
        pos += n
        return s

    fmts = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            sub, n = take("I"), take("Q")
            return [value(sub) for _ in range(n)]
        return take(fmts[t])

    magic, _version, _n_tensors, n_kv = struct.unpack_from("<IIQQ", data, 0)
    assert magic == 0x46554747
    pos = 24
    out = {}
    for _ in range(n_kv):
        k = string()
        out[k] = value(take("I"))
    return out


def bytes_to_unicode():
    """GPT-2's byte encoder (tokenizer.cpp:68-74): printable Latin-1 bytes stand for
    themselves, the others take U+0100 on in byte order."""
    enc, extra = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or b >= 174:
            enc.append(chr(b))
        else:
            enc.append(chr(extra))
            extra += 1
    return enc


class Tokenizer:
    def __init__(self, meta: dict):
        if meta.get("tokenizer.ggml.model") != "gpt2" or meta.get("tokenizer.ggml.pre") != "qwen35":
            raise ValueError("Tokenizer currently supports qwen35 GPT-2 BPE only")
        vocab, types = meta["tokenizer.ggml.tokens"], meta["tokenizer.ggml.token_type"]
        if len(types) != len(vocab):
            raise ValueError("Vocabulary/type size mismatch")
        self.rank = {}
        for i, m in enumerate(meta["tokenizer.ggml.merges"]):
            self.rank.setdefault(m, i)
        self.enc = bytes_to_unicode()
        reverse = {c: b for b, c in enumerate(self.enc)}
        self.ids, self.special, self.decoded = {}, [], []
        for i, (tok, ty) in enumerate(zip(vocab, types)):
            self.ids.setdefault(tok, i)
            if ty in (3, 4):
                self.special.append((tok.encode(), i))
                self.decoded.append(tok.encode())
                continue
            if all(c in reverse for c in tok):
                self.decoded.append(bytes(reverse[c] for c in tok))
            else:
                self.decoded.append(tok.encode())  # not byte-encoded: an unused entry

    @classmethod
    def from_file(cls, path):
        return cls(read_metadata(path))

    @staticmethod
    def pretokenize(text: str):
        """The pattern matched repeatedly, anchored at the previous end."""
        pieces, pos = [], 0
        while pos < len(text):
            m = _RX.match(text, pos)
            if not m or m.end() <= pos:
                raise ValueError("Tokenizer made no progress")
            pieces.append(m.group())
            pos = m.end()
        return pieces

    def _ordinary(self, data: bytes, out: list):
        text = data.decode("utf-8")  # strict: what PCRE2's UTF check rejects raises
        for piece in self.pretokenize(text):
            parts = [self.enc[b] for b in piece.encode()]
            while len(parts) > 1:
                best, best_rank = None, None
                for i in range(len(parts) - 1):
                    r = self.rank.get(parts[i] + " " + parts[i + 1])
                    if r is not None and (best_rank is None or r < best_rank):
                        best, best_rank = i, r
                if best is None:
                    break
                parts[best:best + 2] = [parts[best] + parts[best + 1]]
            for p in parts:
                if p not in self.ids:
                    raise ValueError("BPE piece missing from vocabulary")
                out.append(self.ids[p])

    def encode(self, text, parse_special: bool = True) -> list:
        data = text.encode() if isinstance(text, str) else bytes(text)
        out, offset = [], 0
        while offset < len(data):
            nxt, length, tid = len(data), 0, -1
            if parse_special:
                for s, i in self.special:
                    p = data.find(s, offset)
                    if p >= 0 and (p < nxt or (p == nxt and len(s) > length)):
                        nxt, length, tid = p, len(s), i
            self._ordinary(data[offset:nxt], out)
            if tid < 0:
                break
            out.append(tid)
            offset = nxt + length
        return out

    def decode(self, token: int) -> bytes:
        if not 0 <= token < len(self.decoded):
            raise IndexError("Invalid token ID")
        return self.decoded[token]

    @staticmethod
    def chat_prompt(user: str) -> str:
        return "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n"
