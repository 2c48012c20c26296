"""The oracle's whole model, and the tokenizers, against the reference's own compiled
Model and Tokenizer (oracle/_ref/libemprise_refmodel.so: v1.1 model.cpp, tokenizer.cpp
and the rest of its library built unchanged, PCRE2 and utf8proc from its third_party/,
on its CPU backend). Skipped where that library was not built (it needs the reference
tree). CPU only.

These pin what the op-level comparisons of test_oracle_ref.py cannot reach: the model
composition (the gated attention with its q/k norms and RoPE, the layer order, the
residuals, the output head; model.cpp:121-259), the trace points (model.cpp:118-120), the
hidden vectors the model keeps, the MTP head (model.cpp:376-397), evaluate_block and
prefill (model.cpp:274-366), and the tokenizer (tokenizer.cpp)."""
import numpy as np
import pytest

import oracle
from emprise_amd import TINY, Tokenizer, synth_prompt, synth_write
from oracle.tokenizer import Tokenizer as OracleTokenizer

pytestmark = pytest.mark.skipif(not oracle.ref_model_available(),
                                reason="oracle/_ref/libemprise_refmodel.so not built (reference tree absent)")


def _bits_equal(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=["q6k", "q4km"])
def model_path(request, tmp_path_factory):
    p = tmp_path_factory.mktemp("refmodel") / f"tiny_{request.param}.gguf"
    synth_write(p, seed=0, tokenizer=True, q4_k_m_mix=(request.param == "q4km"), **TINY)
    return str(p)


def test_oracle_model_is_the_reference_model_bit_for_bit(model_path):
    """Sixteen positions (every fourth without logits): every traced tensor, the logits and
    the kept hidden vectors (raw and normed) of the oracle equal the reference Model's
    bit for bit, and the trace points come in the same order with the same names."""
    ref, eo = oracle.RefModel(model_path, context=64), oracle.Model(model_path, context=64)
    a, b = {}, {}
    ref.set_trace(a)
    eo.set_trace(b)
    for pos, tok in enumerate(synth_prompt(5, TINY["vocab"], 16)):
        logits = pos % 4 != 3
        x, y = ref.evaluate(tok, logits), eo.evaluate(tok, logits)
        if logits:
            assert _bits_equal(x, y), f"logits at position {pos}"
        assert _bits_equal(ref.last_hidden(), eo.last_hidden()), f"raw hidden after position {pos}"
        assert _bits_equal(ref.last_hidden(normed=True), eo.last_hidden(normed=True))
    assert list(a) == list(b)
    bad = [k for k in a if not _bits_equal(a[k], b[k])]
    assert not bad, f"{len(bad)} traced tensors differ, first {bad[0]}"
    ref.close()
    eo.close()


def test_oracle_block_and_prefill_are_the_reference_paths(model_path):
    """evaluate_block's rows and prefill's logits (the reference's batched chunks of 4) against
    the oracle evaluating the same positions one at a time: equal bit for bit (the
    reference's CPU batch projections are per-position matvecs)."""
    toks = synth_prompt(6, TINY["vocab"], 11)
    ref, eo = oracle.RefModel(model_path, context=64), oracle.Model(model_path, context=64)
    rows = ref.evaluate_block(toks[:7])
    for i, t in enumerate(toks[:7]):
        assert _bits_equal(rows[i], eo.evaluate(t)), f"block row {i}"
    assert _bits_equal(ref.last_hidden(), eo.last_hidden())
    ref.reset()
    eo.reset()
    last = ref.prefill(toks)
    for t in toks[:-1]:
        eo.evaluate(t, False)
    assert _bits_equal(last, eo.evaluate(toks[-1]))
    ref.close()
    eo.close()


def test_oracle_mtp_head_is_the_reference_head(tmp_path):
    """The MTP draft head (model.cpp:376-397) over chained drafts from the model's own
    hidden vectors: logits and the block's output hidden, bit for bit. The reference names
    the head's tensors blk.32.nextn.* (model.cpp:379-395), so the model here has 32 main
    layers at the tiny widths; the oracle and the device take blk.<layers>."""
    p = tmp_path / "tiny_mtp.gguf"
    synth_write(p, seed=3, tokenizer=True, mtp=True, **dict(TINY, layers=32))
    ref, eo = oracle.RefModel(str(p), context=64), oracle.Model(str(p), context=64)
    toks = synth_prompt(7, TINY["vocab"], 6)
    for t in toks:
        ref.evaluate(t)
        eo.evaluate(t)
    h = eo.last_hidden(normed=True)
    assert _bits_equal(ref.last_hidden(normed=True), h)
    pos = len(toks)
    for step, tok in enumerate([11, 12, 13]):
        lr, le = ref.mtp_draft(h, tok, pos + step), eo.mtp_draft(h, tok, pos + step)
        assert _bits_equal(lr, le), f"draft {step}"
        hr, he = ref.mtp_hidden(), eo.mtp_hidden()
        assert _bits_equal(hr, he)
        h = he
    ref.close()
    eo.close()


def test_tokenizers_are_the_reference_tokenizer(tmp_path):
    """tokenizer.cpp itself against the oracle's restatement (oracle/tokenizer.py) and the
    product's tokenizer (host/tokenizer.cpp): the same ids on the tokenizer tests' corpus
    and random texts, with and without special tokens; the same bytes for every id; the
    same chat prompt."""
    from test_tokenizer import CORPUS, _random_texts
    p = tmp_path / "tiny_tok.gguf"
    synth_write(p, seed=0, tokenizer=True, **TINY)
    ref = oracle.RefModel(str(p), context=8)
    orc = OracleTokenizer.from_file(p)
    with Tokenizer(p) as cpp:
        for special in (True, False):
            for text in CORPUS + _random_texts(200, seed=11):
                want = ref.encode(text, special)
                assert orc.encode(text, special) == want, repr(text)
                assert cpp.encode(text, special) == want, repr(text)
        for i in range(TINY["vocab"]):
            assert cpp.decode(i) == ref.decode(i), i
        assert cpp.chat_prompt("hi there") == ref.chat_prompt("hi there")
    ref.close()
