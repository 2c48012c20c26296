"""The oracle against fixtures written from the reference's own compiled code by
tests/golden/make_golden.py (so the pin holds where oracle/_ref is not built). CPU only."""
import json
from pathlib import Path

import numpy as np

import oracle
from oracle import Q4_K, Q6_K

GOLD = Path(__file__).resolve().parent / "golden"


def test_ref_ops_fixture():
    z = np.load(GOLD / "ref_ops.npz")
    for name, wtype in (("q6k", Q6_K), ("q4k", Q4_K)):
        raw = z[f"{name}_raw"].tobytes()
        assert np.array_equal(oracle.dequantize(wtype, raw, 4 * 512).view(np.uint32), z[f"{name}_dequant"].view(np.uint32))
        assert np.array_equal(oracle.matvec(wtype, raw, z[f"{name}_x"], 4).view(np.uint32), z[f"{name}_y"].view(np.uint32))
    kh, vh, sd, cw = (int(v) for v in z["dn_dims"])
    cs, rs = z["dn_conv_state"].copy(), z["dn_rec_state"].copy()
    out = oracle.delta_net(kh, vh, sd, cw, np.float32(1e-6), z["dn_qkv"], z["dn_gate"], z["dn_alpha"], z["dn_beta"],
                           z["dn_conv"], z["dn_ssm_a"], z["dn_dt"], z["dn_norm"], cs, rs)
    assert np.array_equal(out.view(np.uint32), z["dn_out"].view(np.uint32))
    assert np.array_equal(rs.view(np.uint32), z["dn_rec_state_after"].view(np.uint32))
    assert np.array_equal(cs, z["dn_conv_state_after"])


def test_tiny_model_tokens_match_reference_composition(tmp_path):
    """64 greedy tokens of the tiny model: the oracle's own decode loop reproduces the
    decode composed from reference-built projections, FFNs and recurrent blocks."""
    from emprise_amd import synth_write
    g = json.loads((GOLD / "tiny_generate.json").read_text())
    p = tmp_path / "tiny.gguf"
    synth_write(p, seed=g["seed"], **g["config"])
    m = oracle.Model(str(p), context=g["context"])
    tokens, margins = m.generate(g["prompt"], len(g["tokens"]))
    assert tokens == g["tokens"]
    assert np.allclose(margins, g["margins"], rtol=0, atol=0)


def test_evaluate_many_has_the_bits_of_single_positions(tmp_path):
    """The batched prompt evaluation that writes the 9B fixtures (eo_model_evaluate_many)
    against the position-by-position evaluate pinned above: logits, the last residual and
    the state it leaves (the next position's logits) all bit for bit, across a 64-position
    tile boundary, from position 0 and from a later position, plain and with --fast-q8,
    on the all-Q6_K and the Q4_K_M-mix tiny models."""
    from emprise_amd import TINY, synth_prompt, synth_write
    prompt = synth_prompt(5, TINY["vocab"], 75)
    for mix in (False, True):
        p = tmp_path / f"tiny_{mix}.gguf"
        synth_write(p, seed=3, q4_k_m_mix=mix, **TINY)
        for q8 in (False, True):
            ref = oracle.Model(str(p), context=128, fast_q8=q8)
            many = oracle.Model(str(p), context=128, fast_q8=q8)
            for start, stop in ((0, 1), (1, 70), (70, 75)):
                for t in prompt[start:stop]:
                    want = ref.evaluate(t)
                got = many.evaluate_many(prompt[start:stop])
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (mix, q8, start)
                assert np.array_equal(many.last_hidden().view(np.uint32), ref.last_hidden().view(np.uint32))
            nxt = prompt[0]
            assert np.array_equal(many.evaluate(nxt).view(np.uint32), ref.evaluate(nxt).view(np.uint32))
            ref.close()
            many.close()
