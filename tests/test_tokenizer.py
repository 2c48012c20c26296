"""The C++ host tokenizer (emprise_amd/host/tokenizer.cpp; reference src/tokenizer.cpp)
against the CPU oracle (oracle/tokenizer.py), and the oracle against the HF `tokenizers`
library -- an independent byte-level BPE -- on the same vocabulary and merges. CPU only.

The vocabulary is the synthetic one emprise_synth_write adds (256 byte tokens, merges
trained on a built-in text, the chat template's special tokens). The text corpus covers
each alternative of the pre-tokenizer pattern (tokenizer.cpp:112): contractions in both
cases (and U+017F, which folds to 's'), letters with and without marks, digits, runs of
punctuation with and without a leading space and trailing line breaks, whitespace runs
with and without line breaks, before text and at the end, PCRE2's UCP spaces (U+0085,
U+00A0, U+180E, U+2028, U+3000), several scripts, and special tokens inside text.
"""
import random
import subprocess
from pathlib import Path

import pytest

from emprise_amd import InvalidArgument, TINY, Tokenizer, synth_write
from oracle.tokenizer import PATTERN, Tokenizer as Oracle, read_metadata

CHAT = Path(__file__).resolve().parent.parent / "emprise_amd" / "emprise-chat"

CORPUS = [
    "", "a", " ", "  ", "\n", "Hello world!", "The quick brown fox jumps over the lazy dog.",
    "It's 2024, they'll see; we've done it, I'd say, you're right, I'M SURE IT'S FINE.",
    "'S 'T 'RE 'VE 'M 'LL 'D 's 't 're 've 'm 'll 'd 'x 'ſ 'Re",
    "don't  can't\tshan't\n", "x'll", "''s", "'",
    "3.14159 2.71828 1000000 ½ ² ٣ Ⅻ", "abc123def", "a1b2c3",
    "!!!  ???\n\n... --- ***\r\n", " !\n", "(foo) [bar] {baz} <qux>", "#include <stdio.h>\nint main() { return 0; }",
    "    def add(a, b):\n        return a + b\n", "\t\ttabs\t", "line\r\nbreaks\rmixed\n\n\n",
    "trailing spaces   ", "   leading", "a  b   c    d", "x \n y", " \n\n ", "\n \n \n",
    "Grüße aus München! Ça va? naïve café", "é ä ́̂ x̧y", "́start",
    "日本語のテキスト、句読点。", "中文测试：你好，世界！", "한국어 텍스트", "Ελληνικά κείμενα", "Русский текст!",
    "العربية نص", "हिन्दी पाठ", "emoji 😀🎉👍 mixed😀text", "\u0085nel nbsp᠎mvs ls　ideo",
    "\x0bvt\x0cff", "<|im_start|>user\nhi<|im_end|>\n", "<|im_start|><|im_end|><think></think>",
    "a<|endoftext|>b", "<|im_st", "<|im_start|", "text <think>\n\n</think>\n\nanswer",
]

POOLS = [list("abcXYZéüñßçøåæ"), list("日本語中文한국"), ["́", "̈", "̧", "ि"],
         list("0123456789½²٣"), [" ", " ", " ", "\t", "\n", "\r", "\r\n", " ", "　", " ", "\u0085"],
         list("!?.,;:-_()[]{}<>\"#$%&*+/=@\\^`|~"), ["'s", "'t", "'re", "'LL", "'", "ſ"], ["😀", "🎉", "\U00010348"],
         ["<|im_start|>", "<|im_end|>", "<think>", "</think>", "<|endoftext|>", "<|im_"]]


def _random_texts(n=400, seed=5):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        k = rng.randint(1, 40)
        out.append("".join(rng.choice(rng.choice(POOLS)) for _ in range(k)))
    return out


@pytest.fixture(scope="module")
def tok_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("tok") / "tiny_tok.gguf"
    synth_write(p, seed=0, tokenizer=True, **TINY)
    return p


@pytest.fixture(scope="module")
def pair(tok_path):
    with Tokenizer(tok_path) as t:
        yield t, Oracle.from_file(tok_path)


def _hf(meta, specials):
    from tokenizers import AddedToken, Regex, models, pre_tokenizers
    from tokenizers import Tokenizer as HF
    vocab = {}
    for i, t in enumerate(meta["tokenizer.ggml.tokens"]):
        vocab.setdefault(t, i)
    merges = [tuple(m.split(" ")) for m in meta["tokenizer.ggml.merges"]]
    hf = HF(models.BPE(vocab=vocab, merges=merges))
    hf.pre_tokenizer = pre_tokenizers.Sequence([pre_tokenizers.Split(Regex(PATTERN), behavior="isolated"),
                                                pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    hf.add_special_tokens([AddedToken(s, special=True, normalized=False) for s in specials])
    return hf


def test_oracle_matches_hf_tokenizers(tok_path):
    """The pin of the oracle: HF's byte-level BPE with the same pattern, vocabulary,
    merges and special tokens gives the same ids on the corpus and 400 random texts."""
    pytest.importorskip("tokenizers")
    meta = read_metadata(tok_path)
    specials = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>"]
    hf = _hf(meta, specials)
    o = Oracle(meta)
    for text in CORPUS + _random_texts():
        assert o.encode(text) == hf.encode(text, add_special_tokens=False).ids, repr(text)


def test_pretokenizer_splits_from_the_pattern():
    """Splits worked out by hand from the pattern's alternatives and PCRE2's backtracking."""
    cases = {
        "  \n  x": ["  \n", " ", " x"],                # \s*[\r\n]+ to the last break, \s+(?!\S), then ' x'
        "don't": ["don", "'t"],
        "DON'T": ["DON", "'T"],
        "x'LL y": ["x", "'LL", " y"],
        "a ſ'ſ": ["a", " ſ", "'ſ"],                    # U+017F folds to s (and is a letter)
        "abc123": ["abc", "1", "2", "3"],
        " !!\n\nx": [" !!\n\n", "x"],                  # ' '?[^\s\pL\pM\pN]+[\r\n]*
        "a   ": ["a", "   "],                           # \s+ at the end
        "a   b": ["a", "  ", " b"],                     # \s+(?!\S) leaves one space for ' b'
        "́e": ["́e"],                         # a mark opens [^\r\n\pL\pN]?[\pL\pM]+
        "x\r\n\r\ny": ["x", "\r\n\r\n", "y"],
        "\t\ty": ["\t", "\ty"],                         # the optional char may be a tab
        "　x": ["　x"],                         # ... or an ideographic space
    }
    for text, want in cases.items():
        assert Oracle.pretokenize(text) == want, repr(text)


def test_cpp_matches_oracle(pair):
    t, o = pair
    for text in CORPUS + _random_texts(seed=9):
        for special in (True, False):
            assert t.encode(text, special) == o.encode(text, special), (repr(text), special)


def test_decode_table_matches_oracle_and_round_trips(pair):
    t, o = pair
    for i in range(len(o.decoded)):
        assert t.decode(i) == o.decode(i)
    for text in CORPUS + _random_texts(seed=11):
        assert b"".join(t.decode(i) for i in t.encode(text)) == text.encode(), repr(text)


def test_chat_prompt_and_specials(pair):
    t, o = pair
    p = t.chat_prompt("Explain how a refrigerator works.")
    assert p == Oracle.chat_prompt("Explain how a refrigerator works.")
    ids = t.encode(p)
    assert ids == o.encode(p) and t.decode(ids[0]) == b"<|im_start|>"
    # without special-token parsing the markers are ordinary text
    assert t.encode("<|im_end|>", False) != t.encode("<|im_end|>", True)


def test_rejects_bad_input(pair, tmp_path):
    t, o = pair
    for bad in (b"\xff", b"ab\xc3", b"\xed\xa0\x80", b"\xc0\xaf", b"\xf4\x90\x80\x80"):
        with pytest.raises(InvalidArgument, match="UTF-8"):
            t.encode(bad)
        with pytest.raises(UnicodeDecodeError):
            o.encode(bad)
    with pytest.raises(InvalidArgument):
        t.decode(len(o.decoded))
    plain = tmp_path / "plain.gguf"
    synth_write(plain, seed=0, **TINY)
    with pytest.raises(InvalidArgument, match="qwen35 GPT-2 BPE"):
        Tokenizer(plain)


def test_cli_tokenize(tok_path):
    """emprise-chat --tokenize (chat.cpp:47-52): the chat template's ids, or the raw
    text's with --raw; no device is touched."""
    o = Oracle.from_file(tok_path)
    text = "Explain how a refrigerator works."
    for raw in (False, True):
        cmd = [str(CHAT), "--model", str(tok_path), "--prompt", text, "--tokenize"] + (["--raw"] if raw else [])
        out = subprocess.run(cmd, capture_output=True, text=True, check=True).stdout.strip()
        want = o.encode(text if raw else o.chat_prompt(text))
        assert out == "[" + ",".join(map(str, want)) + "]"
