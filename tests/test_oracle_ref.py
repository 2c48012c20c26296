"""The C oracle against the reference's own compiled CPU code (oracle/_ref: v1.1
quant.cpp, gguf.cpp, backend.cpp built unchanged). Skipped where _ref was not built
(it needs the reference tree); the committed fixtures in tests/golden carry the same
checks to machines without it (test_golden.py). CPU only."""
import ctypes
import json

import numpy as np
import pytest

import oracle
from oracle import BF16, F16, F32, Q4_K, Q6_K
from synth import matrix, q4k_blocks, q6k_blocks

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (reference tree absent)")

_fp = ctypes.POINTER(ctypes.c_float)


def _f(a):
    return a.ctypes.data_as(_fp)


def ref_dequantize(wtype, raw, n):
    buf = np.frombuffer(raw, dtype=np.uint8)
    out = np.empty(n, np.float32)
    assert oracle.ref().ref_dequantize(wtype, buf.ctypes.data, buf.nbytes, _f(out), n) == 0
    return out


def ref_matvec(wtype, raw, x, rows):
    buf = np.frombuffer(raw, dtype=np.uint8)
    y = np.empty(rows, np.float32)
    assert oracle.ref().ref_matvec(wtype, buf.ctypes.data, buf.nbytes, _f(x), x.size, _f(y), rows) == 0
    return y


def test_half_to_float_all_inputs_bit_exact():
    R, L = oracle.ref(), oracle.lib()
    for b in range(65536):
        r, o = R.ref_half_to_float(b), L.eo_half_to_float(b)
        assert (r == o and np.float32(r).view(np.uint32) == np.float32(o).view(np.uint32)) or (r != r and o != o), b


@pytest.mark.parametrize("wtype", [Q6_K, Q4_K, F16, BF16, F32])
def test_dequantize_bit_exact(wtype):
    rng = np.random.default_rng(10 + wtype)
    raw = matrix(rng, wtype, 64, 512)
    assert np.array_equal(oracle.dequantize(wtype, raw, 64 * 512).view(np.uint32),
                          ref_dequantize(wtype, raw, 64 * 512).view(np.uint32))


@pytest.mark.parametrize("wtype,rows,cols", [(Q6_K, 300, 4096), (Q4_K, 300, 4096), (Q6_K, 64, 12288),
                                             (F16, 50, 1024), (BF16, 50, 1024), (F32, 33, 768)])
def test_matvec_bit_exact(wtype, rows, cols):
    rng = np.random.default_rng(rows + cols + wtype)
    raw = matrix(rng, wtype, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    assert np.array_equal(oracle.matvec(wtype, raw, x, rows).view(np.uint32), ref_matvec(wtype, raw, x, rows).view(np.uint32))


def test_encoded_bytes_agree():
    R, L = oracle.ref(), oracle.lib()
    out = ctypes.c_uint64()
    for t, n in [(Q6_K, 256), (Q6_K, 255), (Q4_K, 4096), (F32, 3), (F16, 5), (BF16, 7), (9, 256)]:
        rc = R.ref_encoded_bytes(t, n, ctypes.byref(out))
        mine = L.eo_encoded_bytes(t, n)
        assert (rc != 0 and mine == 0) or (rc == 0 and out.value == mine)


@pytest.mark.parametrize("kh,vh,sd,cw", [(4, 8, 64, 4), (16, 32, 128, 4), (2, 6, 64, 3)])
def test_delta_net_bit_exact(kh, vh, sd, cw, tmp_path):
    from emprise_amd import TINY, synth_write
    path = tmp_path / "any.gguf"  # the CPU delta_net ignores its Gguf argument
    synth_write(path, seed=0, **TINY)
    m = oracle.ref().ref_open(str(path).encode(), 1 << 30)
    assert m
    rng = np.random.default_rng(kh * vh)
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    conv = (rng.standard_normal(ch * cw) * 0.5).astype(np.float32)
    a = (-np.exp(rng.standard_normal(vh) * 0.5 - 2)).astype(np.float32)
    dt = (rng.standard_normal(vh) * 0.5 - 1).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(sd)).astype(np.float32)
    cs_r, rs_r = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    cs_o, rs_o = cs_r.copy(), rs_r.copy()
    for step in range(4):
        qkv, gate = rng.standard_normal(ch).astype(np.float32), rng.standard_normal(vd).astype(np.float32)
        al, be = rng.standard_normal(vh).astype(np.float32), rng.standard_normal(vh).astype(np.float32)
        out_r = np.empty(vd, np.float32)
        assert oracle.ref().ref_delta_net(m, kh, vh, sd, cw, 1e-6, _f(qkv), _f(gate), _f(al), _f(be), _f(conv), _f(a),
                                          _f(dt), _f(nw), _f(cs_r), _f(rs_r), _f(out_r)) == 0
        out_o = oracle.delta_net(kh, vh, sd, cw, 1e-6, qkv, gate, al, be, conv, a, dt, nw, cs_o, rs_o)
        assert np.array_equal(out_o.view(np.uint32), out_r.view(np.uint32)), f"step {step}"
        assert np.array_equal(rs_o.view(np.uint32), rs_r.view(np.uint32))
        assert np.array_equal(cs_o, cs_r)
    oracle.ref().ref_close(m)


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from emprise_amd import TINY, synth_write
    path = tmp_path_factory.mktemp("m") / "tiny.gguf"
    synth_write(path, seed=0, **TINY)
    m = oracle.ref().ref_open(str(path).encode(), 1 << 30)
    assert m, oracle.ref().ref_last_error()
    yield str(path), m
    oracle.ref().ref_close(m)


def _tensor(m, name):
    R = oracle.ref()
    t, nd, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    shape = (ctypes.c_uint64 * 4)()
    assert R.ref_tensor_info(m, name.encode(), ctypes.byref(t), shape, ctypes.byref(nd), ctypes.byref(nb)) == 0
    raw = np.empty(nb.value, np.uint8)
    assert R.ref_tensor_read(m, name.encode(), raw.ctypes.data, nb.value) == 0
    return t.value, list(shape[:nd.value]), raw.tobytes()


def test_reference_loader_accepts_synthetic_gguf(tiny):
    """The reference's own GGUF parser (gguf.cpp:87-147) reads the synthetic file."""
    path, m = tiny
    buf = ctypes.create_string_buffer(1 << 16)
    assert oracle.ref().ref_metadata_json(m, buf, len(buf)) == 0
    meta = json.loads(buf.value.decode())
    assert meta["general.architecture"] == "qwen35"
    assert meta["qwen35.embedding_length"] == 512 and meta["qwen35.ssm.state_size"] == 64
    t, shape, raw = _tensor(m, "blk.0.attn_qkv.weight")
    assert t == Q6_K and shape == [512, 2 * 4 * 64 + 8 * 64] and len(raw) == 1024 * 512 // 256 * 210


def test_linear_and_feed_forward_bit_exact(tiny):
    """Cpu::linear and Backend::feed_forward (backend.cpp:91-122) vs the oracle."""
    path, m = tiny
    R = oracle.ref()
    rng = np.random.default_rng(4)
    x = rng.standard_normal(512).astype(np.float32)
    t, shape, raw = _tensor(m, "blk.1.attn_qkv.weight")
    y = np.empty(shape[1], np.float32)
    assert R.ref_linear(m, b"blk.1.attn_qkv.weight", _f(x), 512, _f(y), shape[1]) == 0
    assert np.array_equal(y, oracle.matvec(t, raw, x, shape[1]))
    yr = np.empty(512, np.float32)
    assert R.ref_feed_forward(m, b"blk.2.ffn_gate.weight", b"blk.2.ffn_up.weight", b"blk.2.ffn_down.weight", _f(x), 512,
                              _f(yr)) == 0
    tg, _, g = _tensor(m, "blk.2.ffn_gate.weight")
    tu, _, u = _tensor(m, "blk.2.ffn_up.weight")
    td, _, d = _tensor(m, "blk.2.ffn_down.weight")
    yo = np.empty(512, np.float32)
    gb, ub, db = (np.frombuffer(b, np.uint8) for b in (g, u, d))
    assert oracle.lib().eo_feed_forward(tg, gb.ctypes.data, tu, ub.ctypes.data, td, db.ctypes.data, 512, 1536,
                                        _f(x), _f(yo)) == 0
    assert np.array_equal(yo, yr)


def test_recurrent_block_bit_exact(tiny):
    """Backend::recurrent_block (backend.cpp:61-77) vs oracle projections + delta_net."""
    path, m = tiny
    R = oracle.ref()
    kh, vh, sd, cw = 4, 8, 64, 4
    ch = 2 * kh * sd + vh * sd
    p = "blk.0."
    conv = np.frombuffer(_tensor(m, p + "ssm_conv1d.weight")[2], np.float32).copy()
    a = np.frombuffer(_tensor(m, p + "ssm_a")[2], np.float32).copy()
    dt = np.frombuffer(_tensor(m, p + "ssm_dt.bias")[2], np.float32).copy()
    nw = np.frombuffer(_tensor(m, p + "ssm_norm.weight")[2], np.float32).copy()
    cs_r, rs_r = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    cs_o, rs_o = cs_r.copy(), rs_r.copy()
    rng = np.random.default_rng(5)
    for step in range(3):
        x = rng.standard_normal(512).astype(np.float32)
        out_r = np.empty(512, np.float32)
        assert R.ref_recurrent_block(m, p.encode(), kh, vh, sd, cw, 1e-6, _f(conv), _f(a), _f(dt), _f(nw), _f(x), 512,
                                     _f(cs_r), _f(rs_r), _f(out_r)) == 0
        proj = {}
        for name in ("attn_qkv", "attn_gate", "ssm_alpha", "ssm_beta"):
            t, shape, raw = _tensor(m, p + name + ".weight")
            proj[name] = oracle.matvec(t, raw, x, shape[1])
        dn = oracle.delta_net(kh, vh, sd, cw, 1e-6, proj["attn_qkv"], proj["attn_gate"], proj["ssm_alpha"],
                              proj["ssm_beta"], conv, a, dt, nw, cs_o, rs_o)
        t, shape, raw = _tensor(m, p + "ssm_out.weight")
        out_o = oracle.matvec(t, raw, dn, 512)
        assert np.array_equal(out_o, out_r), f"step {step}"
