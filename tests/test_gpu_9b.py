"""The 9B-shape models of benchmark configs 3 and 4 on the GPU against golden fixtures
written by the CPU oracle (tests/golden/make_golden_9b.py; the oracle restates the
reference's CPU path and is pinned to the reference's own compiled code).

Bars (north star): greedy tokens identical wherever the reference's top-2 logit margin
exceeds 1e-3; the batched prefill's logits within the reference's batched-vs-sequential
bar (tests/block_check.cpp:43-67: relative L2 <= 1e-3, same argmax).

The synthetic GGUFs are regenerated here (seeded, the bytes bench.py writes) and their
SHA-256 checked against the fixture's.
"""
import hashlib
import json
import os
import tempfile
from pathlib import Path

import numpy as np
import pytest

from emprise_amd import NINE_B, Model, synth_write

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
MARGIN = 1e-3


def _golden(name):
    p = GOLD / f"{name}.json"
    if not p.exists():
        pytest.skip(f"{p.name} not generated (tests/golden/make_golden_9b.py)")
    g = json.loads(p.read_text())
    z = GOLD / f"{name}.npz"
    logits = np.load(z)["logits"] if z.exists() else None
    return g, logits


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for b in iter(lambda: f.read(1 << 24), b""):
            h.update(b)
    return h.hexdigest()


_checked = {}


def _model_file(kind, want_sha):
    d = Path(os.environ.get("EMPRISE_BENCH_DIR", tempfile.gettempdir()))
    p = d / f"emprise_{kind}_seed0.gguf"
    if not p.exists():
        tmp = p.with_suffix(".tmp")
        synth_write(tmp, seed=0, q4_k_m_mix=(kind == "9b_q4km"), **NINE_B)
        os.replace(tmp, p)
    if str(p) not in _checked:
        _checked[str(p)] = _sha256(p)
    assert _checked[str(p)] == want_sha, f"{p.name} differs from the fixture's model"
    return str(p)


def _rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


def _teacher_forced(m, g, want_prompt_logits=None, margin=MARGIN):
    """Evaluates the golden prompt and tokens position by position; returns the number
    of picks compared and the prompt-end logits."""
    prompt, tokens, margins = g["prompt"], g["tokens"], g["margins"]
    for t in prompt[:-1]:
        m.evaluate(t, logits=False)
    logits = m.evaluate(prompt[-1])
    first = logits.copy()
    compared = 0
    for i, (tok, mg) in enumerate(zip(tokens, margins)):
        if mg > margin:
            assert int(np.argmax(logits)) == tok, f"pick {i}: gpu {int(np.argmax(logits))} != cpu {tok} (margin {mg:.3g})"
            compared += 1
        if i + 1 < len(tokens):
            logits = m.evaluate(tok)
    return compared, first


def test_c3_9b_q6k_teacher_forced():
    """Config 3 (9B shape, Q6_K): every greedy pick of the 512 + 128 token run, each
    position evaluated as a decode step; the prompt-end logits against the CPU's."""
    g, want = _golden("c3_9b_q6k")
    path = _model_file("9b_q6k", g["gguf_sha256"])
    with Model(path, context=g["context"]) as m:
        compared, first = _teacher_forced(m, g)
    rel = _rel_l2(first, want)
    print(f"C3 teacher-forced: {compared} of {len(g['tokens'])} picks compared, prompt-end logits rel L2 {rel:.3e}, "
          f"max-abs {np.max(np.abs(first - want)) / np.max(np.abs(want)):.3e} of max|ref|")
    assert rel <= 1e-3
    assert int(np.argmax(first)) == g["tokens"][0]
    assert compared >= len(g["tokens"]) - 4


def test_c3_9b_q6k_generate():
    """Config 3 through the benchmark's path: batched prefill of the 512-token prompt,
    then 128 greedy tokens from the replayed step graph, identical to the CPU's up to
    the first pick whose CPU margin is <= 1e-3."""
    g, _ = _golden("c3_9b_q6k")
    path = _model_file("9b_q6k", g["gguf_sha256"])
    with Model(path, context=g["context"]) as m:
        tokens, _ = m.generate(g["prompt"], len(g["tokens"]))
    n = 0
    for i, (a, b) in enumerate(zip(tokens, g["tokens"])):
        if g["margins"][i] <= MARGIN:
            break
        assert a == b, f"token {i}: gpu {a} != cpu {b}"
        n += 1
    print(f"C3 generate: {n} of {len(g['tokens'])} tokens identical before the first low-margin pick")
    assert n >= 16 or n == len(g["tokens"]) or g["margins"][n] <= MARGIN


def test_c4a_9b_q4km_batched_prefill():
    """Config 4a (9B shape, Q4_K_M mix): the 2048-token prompt prefilled in one batch
    (GEMM projections on the matrix cores), then the prompt-end logits (relative L2 <=
    1e-3 and the same argmax, block_check.cpp:43-67) and 16 greedy tokens."""
    g, want = _golden("c4a_9b_q4km")
    path = _model_file("9b_q4km", g["gguf_sha256"])
    with Model(path, context=g["context"]) as m:
        got = m.prefill(g["prompt"])
        assert int(np.argmax(got)) == int(np.argmax(want)) == g["tokens"][0]
        rel = _rel_l2(got, want)
        print(f"C4a prompt-end logits after the batched prefill: rel L2 {rel:.3e}")
        assert rel <= 1e-3
        tokens, _ = m.generate(g["prompt"], len(g["tokens"]))
    for i, (a, b) in enumerate(zip(tokens, g["tokens"])):
        if g["margins"][i] <= MARGIN:
            break
        assert a == b, f"token {i}: gpu {a} != cpu {b}"


def test_c4b_9b_q4km_fast_q8_teacher_forced():
    """Config 4b (Q4_K_M mix, --fast-q8) against the oracle's Q8 mode, teacher-forced.
    The GPU quantises its own activations, which differ from the CPU's in the last bits,
    so an input can fall one quantum (amax/127) away from the CPU's; over 32 layers that
    moves logits by ~1e-4 of their scale. Picks are compared where the CPU margin exceeds
    1e-2."""
    g, _ = _golden("c4b_9b_q4km_q8")
    path = _model_file("9b_q4km", g["gguf_sha256"])
    with Model(path, context=g["context"], fast_q8=True) as m:
        assert "Q8" in m.backend_name
        compared, _ = _teacher_forced(m, g, margin=1e-2)
    print(f"C4b teacher-forced: {compared} of {len(g['tokens'])} picks compared")
    assert compared >= len(g["tokens"]) - 4
