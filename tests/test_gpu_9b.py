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


def _step_values(logits, tok):
    """The GPU's logit at the CPU's pick and its largest logit elsewhere: the two numbers
    the fixture records per step as top1 / top2 (index-free, so a low-margin step where
    the two paths rank the top pair differently is still compared value for value)."""
    rest = logits.copy()
    rest[tok] = -np.inf
    return float(logits[tok]), float(rest.max())


def _teacher_forced(m, g, margin=MARGIN):
    """Evaluates the golden prompt and tokens position by position, each position as one
    decode step. Returns the number of picks compared (CPU margin > `margin`), the
    prompt-end logits and the largest per-step deviation of the top-1 / top-2 logit
    values from the fixture's, relative to that step's logit scale max(|top1|, |top2|)."""
    prompt, tokens, margins = g["prompt"], g["tokens"], g["margins"]
    for t in prompt[:-1]:
        m.evaluate(t, logits=False)
    logits = m.evaluate(prompt[-1])
    first = logits.copy()
    compared, worst = 0, 0.0
    for i, (tok, mg) in enumerate(zip(tokens, margins)):
        if mg > margin:
            assert int(np.argmax(logits)) == tok, f"pick {i}: gpu {int(np.argmax(logits))} != cpu {tok} (margin {mg:.3g})"
            compared += 1
        v1, v2 = _step_values(logits, tok)
        scale = max(abs(g["top1"][i]), abs(g["top2"][i]))
        dev = max(abs(v1 - g["top1"][i]), abs(v2 - g["top2"][i])) / scale
        worst = max(worst, dev)
        if i + 1 < len(tokens):
            logits = m.evaluate(tok)
    return compared, first, worst


# Per-step bar on the top-1 / top-2 logit values (FP32 paths): 1e-3 of the step's logit
# scale. The prompt-end logits of C3 sit at a relative L2 of ~2e-5 from the CPU's; the
# per-op bar is 1e-4 of max|ref| per op, and 32 layers of it accumulate to ~1e-3 at most.
STEP_BAR = 1e-3


def test_c3_9b_q6k_teacher_forced():
    """Config 3 (9B shape, Q6_K): every greedy pick of the 512 + 128 token run, each
    position evaluated as a decode step; per step the logit at the CPU's pick and the
    largest other logit against the CPU's values; the prompt-end logits against the
    CPU's."""
    g, want = _golden("c3_9b_q6k")
    path = _model_file("9b_q6k", g["gguf_sha256"])
    with Model(path, context=g["context"]) as m:
        compared, first, worst = _teacher_forced(m, g)
    rel = _rel_l2(first, want)
    print(f"C3 teacher-forced: {compared} of {len(g['tokens'])} picks compared, prompt-end logits rel L2 {rel:.3e}, "
          f"max-abs {np.max(np.abs(first - want)) / np.max(np.abs(want)):.3e} of max|ref|, "
          f"per-step top-1/top-2 values within {worst:.3e} of the step's scale")
    assert rel <= 1e-3
    assert int(np.argmax(first)) == g["tokens"][0]
    assert compared >= len(g["tokens"]) - 4
    assert worst <= STEP_BAR


def test_c3_9b_q6k_generate():
    """Config 3 through the benchmark's path: batched prefill of the 512-token prompt,
    then 128 greedy tokens from the replayed step graph, identical to the CPU's up to
    the first pick whose CPU margin is <= 1e-3 (beyond it the two runs may follow
    different, equally valid continuations)."""
    g, _ = _golden("c3_9b_q6k")
    path = _model_file("9b_q6k", g["gguf_sha256"])
    with Model(path, context=g["context"]) as m:
        tokens, _ = m.generate(g["prompt"], len(g["tokens"]))
    low = [i for i, mg in enumerate(g["margins"]) if mg <= MARGIN]
    n = low[0] if low else len(g["tokens"])
    print(f"C3 generate: {n} of {len(g['tokens'])} tokens compared (up to the first low-margin pick)")
    assert len(tokens) == len(g["tokens"])
    assert tokens[:n] == g["tokens"][:n], next(f"token {i}: gpu {a} != cpu {b}" for i, (a, b) in
                                                enumerate(zip(tokens[:n], g["tokens"][:n])) if a != b)
    assert n >= 100  # the fixture's first low-margin pick is at 113: most of the run is compared


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
        # the 16 decode steps after the batched prefill, teacher-forced: top-1 / top-2 values
        logits, worst = got, 0.0
        for i, tok in enumerate(g["tokens"]):
            v1, v2 = _step_values(logits, tok)
            scale = max(abs(g["top1"][i]), abs(g["top2"][i]))
            worst = max(worst, abs(v1 - g["top1"][i]) / scale, abs(v2 - g["top2"][i]) / scale)
            if i + 1 < len(g["tokens"]):
                logits = m.evaluate(tok)
        print(f"C4a prompt-end logits after the batched prefill: rel L2 {rel:.3e}; per-step top-1/top-2 values "
              f"within {worst:.3e} of the step's scale")
        assert rel <= 1e-3
        assert worst <= STEP_BAR
        m.reset()
        tokens, _ = m.generate(g["prompt"], len(g["tokens"]))
    for i, (a, b) in enumerate(zip(tokens, g["tokens"])):
        if g["margins"][i] <= MARGIN:
            break
        assert a == b, f"token {i}: gpu {a} != cpu {b}"


def test_c4b_9b_q4km_fast_q8_teacher_forced():
    """Config 4b (Q4_K_M mix, --fast-q8) against the oracle's Q8 mode, teacher-forced over
    the config's 512-token prompt and 256 tokens. The GPU quantises its own activations,
    which differ from the CPU's in the last bits, so an input can land one quantum
    (amax/127 of its 32-value block) away from the CPU's. One such flip moves a projection
    output by about |w| * amax/127 in one of its 4096 terms; summed over the ~1% of inputs
    near a rounding boundary and 32 layers, the logits move by ~1e-4 to 1e-3 of their
    scale. Bars: picks compared where the CPU margin exceeds 1e-2, the prompt-end logits
    within a relative L2 of 5e-3, and each step's top-1 / top-2 logit values within 5e-3
    of the step's scale -- a Q8 path off by 1% (a wrong scale, a dropped zero point)
    fails both."""
    g, want = _golden("c4b_9b_q4km_q8")
    path = _model_file("9b_q4km", g["gguf_sha256"])
    with Model(path, context=g["context"], fast_q8=True) as m:
        assert "Q8" in m.backend_name
        compared, first, worst = _teacher_forced(m, g, margin=1e-2)
    rel = _rel_l2(first, want)
    print(f"C4b teacher-forced: {compared} of {len(g['tokens'])} picks compared, prompt-end logits rel L2 {rel:.3e}, "
          f"per-step top-1/top-2 values within {worst:.3e} of the step's scale")
    assert len(g["prompt"]) == 512 and len(g["tokens"]) == 256
    assert compared >= len(g["tokens"]) - 8
    assert rel <= 5e-3
    assert worst <= 5e-3


def test_c3_9b_trace_layer_by_layer():
    """The per-tensor trace hook (model.hpp:18-19) at the 9B shape: the first positions of
    the C3 prompt on the device and in the CPU oracle (run here, on the same GGUF), every
    traced tensor compared -- attn_norm-L, attn_residual-L and l_out-L of all 32 layers,
    result_norm and logits. Each within a relative L2 of 1e-4 (the prompt-end logits of
    the 512-position C3 run are at ~2e-5); the worst tensor and the drift of the residual
    stream through the layers are printed, which is what the hook is for: finding the
    layer where two paths part."""
    import oracle
    g, _ = _golden("c3_9b_q6k")
    path = _model_file("9b_q6k", g["gguf_sha256"])
    prompt = g["prompt"][:4]
    ref = oracle.Model(path, context=64)
    want = {}
    ref.set_trace(want)
    for t in prompt:
        ref.evaluate(t, True)
    ref.close()
    got = {}
    with Model(path, context=64) as m:
        m.set_trace(lambda pos, name, x: got.__setitem__(f"{pos}.{name}", x))
        for t in prompt:
            m.evaluate(t)
    assert set(got) == set(want) and len(want) == len(prompt) * (3 * NINE_B["layers"] + 2)
    rel = {k: _rel_l2(got[k], w) for k, w in want.items()}
    worst = max(rel, key=rel.get)
    last = len(prompt) - 1
    drift = [rel[f"{last}.l_out-{layer}"] for layer in range(NINE_B["layers"])]
    print(f"9B trace: {len(rel)} tensors over {len(prompt)} positions, worst {worst} at rel L2 {rel[worst]:.3e}; "
          f"position {last} l_out rel L2 by layer: " + " ".join(f"{d:.1e}" for d in drift) +
          f"; logits {rel[f'{last}.logits']:.3e}")
    assert rel[worst] <= 1e-4, f"{worst}: rel L2 {rel[worst]:.3e}"
