"""The MTP (next-n) draft head, Model::evaluate_block and Model::last_hidden on the GPU
against the CPU oracle (model.cpp:376-397, :274-354, :483-487), on the tiny synthetic
qwen35 with its MTP block (blk.4, the layout of the 9B's blk.32) and at the 9B width.

Bars: the draft is one embedding row, three RMSNorm pairs, seven projections, one
attention and an FFN -- a composite like one decoder layer -- so its logits are held to
the per-step bar of the tiny model's teacher-forced test (max-abs 2e-4 of max|ref|), its
argmax to the CPU's wherever the CPU's top-2 margin exceeds 1e-3.

The acceptance loop is tests/mtp_check.cpp's: after the prompt, each greedy step t1 is
drafted from the previous hidden (raw or output-normed) and from the current one, and a
draft counts when its argmax equals the next greedy token t2; the GPU's counts must be
the CPU's.
"""
import numpy as np
import pytest

import oracle
from emprise_amd import InvalidArgument, Model, NINE_B, TINY, synth_prompt, synth_write

pytestmark = pytest.mark.gpu

MARGIN = 1e-3


@pytest.fixture(scope="module")
def mtp_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("models") / "tiny_mtp.gguf"
    synth_write(p, seed=4, mtp=True, **TINY)
    return str(p)


def _check(got, want, what):
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    assert err <= 2e-4 * float(np.max(np.abs(want))), f"{what}: max-abs {err:.3e}"
    top = np.argsort(want)[-2:]
    if want[top[1]] - want[top[0]] > MARGIN:
        assert int(np.argmax(got)) == int(top[1]), what


def test_mtp_draft_matches_oracle(mtp_path):
    """Drafts chained without reset (the block's cache grows to 6 rows), then after
    reset_mtp, from raw and output-normed hidden vectors; mtp_hidden with them."""
    prompt = synth_prompt(5, TINY["vocab"], 20)
    ref = oracle.Model(mtp_path, context=256)
    with Model(mtp_path, context=256) as m:
        assert m.has_mtp and ref.has_mtp
        for t in prompt[:-1]:
            ref.evaluate(t, logits=False)
            m.evaluate(t, logits=False)
        want_l, got_l = ref.evaluate(prompt[-1]), m.evaluate(prompt[-1])
        pos = len(prompt)
        for normed in (False, True):
            h_ref = ref.last_hidden(normed=normed)
            h_gpu = m.last_hidden(normed=normed)
            _check(h_gpu, h_ref, f"last_hidden normed={normed}")
            ref.reset_mtp()
            m.reset_mtp()
            tok = int(np.argmax(want_l))
            for step in range(6):
                # both sides draft from the CPU's hidden vector, so only the block differs
                want = ref.mtp_draft(h_ref, tok, pos + step)
                got = m.mtp_draft(h_ref, tok, pos + step)
                _check(got, want, f"draft {step} normed={normed}")
                _check(m.mtp_hidden(), ref.mtp_hidden(), f"mtp_hidden {step}")
                h_ref = ref.mtp_hidden()
                tok = int(np.argmax(want))
        assert np.all(np.isfinite(got_l))


def test_mtp_check_acceptance_counts(mtp_path):
    """tests/mtp_check.cpp's four conventions (A: raw previous hidden, B: normed previous,
    C: raw current, D: normed current), each draft from a reset cache at the step's
    position; the GPU counts the same matches as the CPU."""
    prompt = synth_prompt(6, TINY["vocab"], 16)
    steps = 12

    def run(model):
        for t in prompt[:-1]:
            model.evaluate(t, logits=False)
        logits = model.evaluate(prompt[-1])
        prev_raw, prev = model.last_hidden(), model.last_hidden(normed=True)
        match = np.zeros(4, int)
        drafts, greedy = [], []
        position = len(prompt)
        for _ in range(steps):
            t1 = int(np.argmax(logits))
            logits1 = model.evaluate(t1)
            cur_raw, cur = model.last_hidden(), model.last_hidden(normed=True)
            t2 = int(np.argmax(logits1))
            greedy.append((t1, t2))
            for i, h in enumerate((prev_raw, prev, cur_raw, cur)):
                model.reset_mtp()
                d = model.mtp_draft(h, t1, position)
                match[i] += int(np.argmax(d)) == t2
                drafts.append(d)
            logits, prev_raw, prev = logits1, cur_raw, cur
            position += 1
        return match, drafts, greedy

    ref_match, ref_drafts, ref_greedy = run(oracle.Model(mtp_path, context=256))
    with Model(mtp_path, context=256) as m:
        gpu_match, gpu_drafts, gpu_greedy = run(m)
    print(f"acceptance A/B/C/D over {steps} steps: cpu {ref_match.tolist()}, gpu {gpu_match.tolist()}")
    assert gpu_greedy == ref_greedy
    for i, (g, w) in enumerate(zip(gpu_drafts, ref_drafts)):
        _check(g, w, f"draft {i // 4} convention {'ABCD'[i % 4]}")
    margins = [float(np.diff(np.sort(w)[-2:])[0]) for w in ref_drafts]
    if min(margins) > MARGIN:
        assert gpu_match.tolist() == ref_match.tolist()


@pytest.mark.parametrize("n", [2, 5, 9])
def test_evaluate_block_matches_oracle(mtp_path, n):
    """Every position's logits of an n-token block after a 12-token prefix, the block in one
    batched pass (small-batch matvec projections up to 7 positions, GEMM from 8), and the
    state it leaves: the next decode step and last_hidden match the CPU's."""
    toks = synth_prompt(8, TINY["vocab"], 12 + n + 1)
    ref = oracle.Model(mtp_path, context=256)
    with Model(mtp_path, context=256) as m:
        m.prefill(toks[:12], logits=False)
        for t in toks[:12]:
            ref.evaluate(t, logits=False)
        got = m.evaluate_block(toks[12:12 + n])
        assert got.shape == (n, TINY["vocab"])
        for i, t in enumerate(toks[12:12 + n]):
            _check(got[i], ref.evaluate(t), f"block row {i}")
        _check(m.last_hidden(), ref.last_hidden(), "last_hidden after the block")
        _check(m.evaluate(toks[-1]), ref.evaluate(toks[-1]), "decode step after the block")


def test_mtp_errors(tmp_path, mtp_path):
    p = tmp_path / "plain.gguf"
    synth_write(p, seed=0, **TINY)
    with Model(str(p), context=64) as m:
        assert not m.has_mtp
        with pytest.raises(InvalidArgument):
            m.mtp_draft(np.zeros(TINY["hidden"], np.float32), 1, 0)
    with Model(mtp_path, context=64) as m:
        with pytest.raises(InvalidArgument):
            m.mtp_draft(np.zeros(TINY["hidden"], np.float32), TINY["vocab"], 0)  # token id
        with pytest.raises(InvalidArgument):
            m.mtp_draft(np.zeros(TINY["hidden"], np.float32), 1, 64)  # rotary position past the context


def test_mtp_9b_width_matches_oracle(tmp_path):
    """The block at the 9B width (hidden 4096, 16 Q / 4 KV heads of 256, FFN 12288,
    vocab 151936; two main layers so the file stays small): three chained drafts."""
    shape = dict(NINE_B, layers=4, vocab=151936)
    p = tmp_path / "w9b_mtp.gguf"
    synth_write(p, seed=2, mtp=True, **shape)
    prompt = synth_prompt(9, shape["vocab"], 6)
    ref = oracle.Model(str(p), context=64)
    with Model(str(p), context=64) as m:
        for t in prompt:
            want = ref.evaluate(t)
            m.evaluate(t)
        h = ref.last_hidden()
        tok = int(np.argmax(want))
        for step in range(3):
            w = ref.mtp_draft(h, tok, len(prompt) + step)
            g = m.mtp_draft(h, tok, len(prompt) + step)
            _check(g, w, f"9B-width draft {step}")
            tok = int(np.argmax(w))
