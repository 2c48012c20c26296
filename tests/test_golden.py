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
