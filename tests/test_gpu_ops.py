"""Decode-step mixer and small ops on the GPU through the C ABI, against the CPU oracle.

Tolerance: max-abs error <= 1e-4 * max|ref| per FP32 output (north star); state
buffers carried across several tokens are held to the same bar at every step.
"""
import numpy as np
import pytest

import oracle
from emprise_amd import (F32, Q4_K, Q6_K, AttentionParams, DeltaNetParams, Input, InvalidArgument,
                         RecurrentParams)
from synth import matrix, quantize_like_reference

pytestmark = pytest.mark.gpu


def _close(got, ref, tol=1e-4, what=""):
    err = np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))
    bound = tol * max(np.max(np.abs(ref)), 1e-30)
    assert err <= bound, f"{what} max abs err {err:.3e} > {bound:.3e}"


def test_rmsnorm_rows_and_embed_rows(backend):
    """Row-wise forms used by batched prefill: every row matches the one-row op."""
    rng = np.random.default_rng(2)
    n, rows = 1536, 37
    x = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    xd, wd, od = backend.to_device(x), backend.vector(w), backend.alloc(rows * n * 4)
    backend.rmsnorm_rows(xd, wd, od, n, rows, 1e-6)
    got = backend.download(od, (rows, n))
    for r in range(rows):
        _close(got[r], oracle.rms(x[r], w, 1e-6), what=f"row {r}")
    vocab, cols = 300, 512
    raw = matrix(rng, Q6_K, vocab, cols)
    emb = backend.upload_weight(Q6_K, cols, vocab, raw)
    table = oracle.dequantize(Q6_K, raw, vocab * cols).reshape(vocab, cols)
    toks = np.array([5, 0, 299, 17, 5], np.int32)
    td, ed = backend.to_device(toks), backend.alloc(len(toks) * cols * 4)
    backend.embed_rows(emb, td, len(toks), ed)
    assert np.array_equal(backend.download(ed, (len(toks), cols)), table[toks])
    # the residual add fused into the norm's pass: x and out bit-equal to add + rmsnorm_rows
    delta = rng.standard_normal((rows, n)).astype(np.float32)
    x2, dd, o2 = backend.to_device(x), backend.to_device(delta), backend.alloc(rows * n * 4)
    backend.add_rmsnorm_rows(x2, dd, wd, o2, n, rows, 1e-6)
    x3 = backend.to_device(x)
    backend.add(x3, dd, rows * n)
    backend.rmsnorm_rows(x3, wd, od, n, rows, 1e-6)
    assert np.array_equal(backend.download(x2, (rows, n)), x + delta)
    assert np.array_equal(backend.download(x2, (rows, n)), backend.download(x3, (rows, n)))
    assert np.array_equal(backend.download(o2, (rows, n)), backend.download(od, (rows, n)))
    with pytest.raises(InvalidArgument):
        backend.add_rmsnorm_rows(x2, dd, wd, x2, n, rows, 1e-6)  # out aliasing x
    for b in (xd, od, td, ed, x2, dd, o2, x3):
        backend.free(b)
    backend.weight_free(emb)
    backend.weight_free(wd)


def test_rmsnorm_add_swiglu(backend):
    rng = np.random.default_rng(1)
    n = 4096
    x = rng.standard_normal(n).astype(np.float32) * 3
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    xd, wd, od = backend.to_device(x), backend.vector(w), backend.alloc(n * 4)
    backend.rmsnorm(xd, wd, od, n, 1e-6)
    _close(backend.download(od, n), oracle.rms(x, w, 1e-6))
    y = rng.standard_normal(n).astype(np.float32)
    yd = backend.to_device(y)
    backend.add(xd, yd, n)
    assert np.array_equal(backend.download(xd, n), x + y)
    g = (rng.standard_normal(n) * 8).astype(np.float32)
    gd = backend.to_device(g)
    backend.swiglu(gd, yd, n)
    ref = np.array([oracle.lib().eo_silu(float(v)) for v in g], dtype=np.float32) * y
    _close(backend.download(gd, n), ref)


@pytest.mark.parametrize("wtype,cols,rows", [(Q6_K, 4096, 151936), (Q6_K, 512, 4096), (Q4_K, 4096, 1000)])
def test_embed_row(backend, wtype, cols, rows):
    rng = np.random.default_rng(2)
    raw = matrix(rng, wtype, rows, cols)
    w = backend.upload_weight(wtype, cols, rows, raw)
    rb = len(raw) // rows
    out, tok = backend.alloc(cols * 4), backend.alloc(4)
    for t in (0, rows // 3, rows - 1):
        backend.upload(tok, np.array([t], np.int32))
        backend.embed(w, tok, out)
        ref = oracle.dequantize(wtype, raw[t * rb:(t + 1) * rb], cols)
        assert np.array_equal(backend.download(out, cols).view(np.uint32), ref.view(np.uint32))
    backend.weight_free(w)


def test_argmax_first_maximum(backend):
    rng = np.random.default_rng(4)
    v = rng.standard_normal(151936).astype(np.float32)
    v[[10, 5000, 90000]] = 9.0  # ties: std::max_element keeps the first
    d, idx = backend.to_device(v), backend.alloc(4)
    backend.argmax(d, v.size, idx)
    assert backend.download(idx, 1, np.int32)[0] == 10
    v2 = -np.abs(v) - 1
    backend.upload(d, v2)
    backend.argmax(d, v2.size, idx)
    assert backend.download(idx, 1, np.int32)[0] == int(np.argmax(v2))


def test_quantize_q8_matches_reference_rule(backend):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    x[64:96] = 0.0  # an all-zero block keeps scale 0 and codes 0
    xd, qd, sd = backend.to_device(x), backend.alloc(4096), backend.alloc(4096 // 32 * 4)
    backend.quantize_q8(xd, 4096, qd, sd)
    q = backend.download(qd, 4096, np.int8)
    s = backend.download(sd, 128)
    for b in range(128):
        blk = x[b * 32:(b + 1) * 32]
        sc = np.float32(np.max(np.abs(blk)) / np.float32(127))
        assert s[b] == np.float32(np.float16(sc))
        if sc == 0:
            assert np.all(q[b * 32:(b + 1) * 32] == 0)
            continue
        r = blk / sc
        exp = np.where(np.abs(r - np.trunc(r)) == 0.5, np.trunc(r) + np.sign(r), np.round(r)).astype(np.int8)
        assert np.array_equal(q[b * 32:(b + 1) * 32], exp)


def _gdn_inputs(rng, kh, vh, sd, cw):
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    return dict(
        conv=(rng.standard_normal(ch * cw) * 0.5).astype(np.float32),
        ssm_a=(-np.exp(rng.standard_normal(vh) * 0.5 - 2)).astype(np.float32),
        dt=(rng.standard_normal(vh) * 0.5 - 1).astype(np.float32),
        norm=(1 + 0.02 * rng.standard_normal(sd)).astype(np.float32),
    )


@pytest.mark.parametrize("kh,vh,sd,cw", [(16, 32, 128, 4), (4, 8, 64, 4)])
def test_delta_net_steps(backend, kh, vh, sd, cw):
    """Config 2a: GDN recurrent update over several tokens (state carried)."""
    rng = np.random.default_rng(6)
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = _gdn_inputs(rng, kh, vh, sd, cw)
    eps = 1e-6
    conv_c = np.zeros(ch * cw, np.float32)
    rec_c = np.zeros(vh * sd * sd, np.float32)
    conv_g, rec_g = backend.to_device(conv_c), backend.to_device(rec_c)
    wconv, wa, wdt, wn = (backend.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    bufs = {k: backend.alloc(n * 4) for k, n in (("qkv", ch), ("gate", vd), ("alpha", vh), ("beta", vh), ("out", vd))}
    for step in range(5):
        qkv = rng.standard_normal(ch).astype(np.float32)
        gate = rng.standard_normal(vd).astype(np.float32)
        alpha = rng.standard_normal(vh).astype(np.float32)
        beta = rng.standard_normal(vh).astype(np.float32)
        for k, v in (("qkv", qkv), ("gate", gate), ("alpha", alpha), ("beta", beta)):
            backend.upload(bufs[k], v)
        p = DeltaNetParams(kh, vh, sd, cw, eps, bufs["qkv"], bufs["gate"], bufs["alpha"], bufs["beta"], wconv, wa,
                           wdt, wn, conv_g, rec_g, bufs["out"])
        backend.delta_net(p)
        ref = oracle.delta_net(kh, vh, sd, cw, eps, qkv, gate, alpha, beta, prm["conv"], prm["ssm_a"], prm["dt"],
                               prm["norm"], conv_c, rec_c)
        _close(backend.download(bufs["out"], vd), ref, what=f"step {step} out")
        _close(backend.download(rec_g, vh * sd * sd), rec_c, what=f"step {step} state")
        assert np.array_equal(backend.download(conv_g, ch * cw), conv_c)  # conv history is a copy


# counts: one position; fewer than conv_width - 1; within one 64-position block of the
# scan; over three blocks (both register sets of the scan, a partial last block)
@pytest.mark.parametrize("kh,vh,sd,cw,count", [(16, 32, 128, 4, 37), (4, 8, 64, 4, 9), (4, 8, 64, 3, 1),
                                               (16, 32, 128, 4, 1), (4, 8, 64, 4, 2), (16, 32, 128, 4, 150),
                                               (4, 8, 64, 2, 130)])
def test_delta_net_batch_matches_steps(backend, kh, vh, sd, cw, count):
    """emprise_hip_delta_net_batch (the prefill scan over `count` positions, rows in a
    strided [qkv | gate | alpha | beta] layout) against `count` calls of delta_net, from a
    nonzero starting state: every output row and both final states bit for bit; the first
    steps are also checked against the oracle."""
    rng = np.random.default_rng(11)
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    W = ch + vd + 2 * vh + 5  # padded row stride
    prm = _gdn_inputs(rng, kh, vh, sd, cw)
    eps = 1e-6
    conv0 = (rng.standard_normal(ch * cw) * 0.3).astype(np.float32)
    rec0 = (rng.standard_normal(vh * sd * sd) * 0.05).astype(np.float32)
    rows = rng.standard_normal((count, W)).astype(np.float32)
    wconv, wa, wdt, wn = (backend.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    # position by position
    conv_s, rec_s = backend.to_device(conv0), backend.to_device(rec0)
    bufs = {k: backend.alloc(n * 4) for k, n in (("qkv", ch), ("gate", vd), ("alpha", vh), ("beta", vh), ("out", vd))}
    seq = np.zeros((count, vd), np.float32)
    conv_c, rec_c = conv0.copy(), rec0.copy()
    for t in range(count):
        r = rows[t]
        parts = (("qkv", r[:ch]), ("gate", r[ch:ch + vd]), ("alpha", r[ch + vd:ch + vd + vh]),
                 ("beta", r[ch + vd + vh:ch + vd + 2 * vh]))
        for k, v in parts:
            backend.upload(bufs[k], np.ascontiguousarray(v))
        p = DeltaNetParams(kh, vh, sd, cw, eps, bufs["qkv"], bufs["gate"], bufs["alpha"], bufs["beta"], wconv, wa,
                           wdt, wn, conv_s, rec_s, bufs["out"])
        backend.delta_net(p)
        seq[t] = backend.download(bufs["out"], vd)
        if t < 2:
            ref = oracle.delta_net(kh, vh, sd, cw, eps, r[:ch], r[ch:ch + vd], r[ch + vd:ch + vd + vh],
                                   r[ch + vd + vh:ch + vd + 2 * vh], prm["conv"], prm["ssm_a"], prm["dt"], prm["norm"],
                                   conv_c, rec_c)
            _close(seq[t], ref, what=f"step {t} vs oracle")
    # one batched call over the strided rows
    conv_b, rec_b = backend.to_device(conv0), backend.to_device(rec0)
    rows_d = backend.to_device(rows)
    out_stride = vd + 3
    out_d = backend.alloc(count * out_stride * 4)
    p = DeltaNetParams(kh, vh, sd, cw, eps, rows_d, rows_d + ch * 4, rows_d + (ch + vd) * 4,
                       rows_d + (ch + vd + vh) * 4, wconv, wa, wdt, wn, conv_b, rec_b, out_d)
    backend.delta_net_batch(p, count, W, out_stride)
    got = backend.download(out_d, count * out_stride).reshape(count, out_stride)[:, :vd]
    assert np.array_equal(got, seq)
    assert np.array_equal(backend.download(rec_b, vh * sd * sd), backend.download(rec_s, vh * sd * sd))
    assert np.array_equal(backend.download(conv_b, ch * cw), backend.download(conv_s, ch * cw))
    assert np.array_equal(backend.download(rows_d, count * W).reshape(count, W), rows)  # inputs untouched


def test_delta_net_batch_rejects_bad_strides_and_state(backend):
    kh, vh, sd, cw = 4, 8, 64, 4
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = _gdn_inputs(np.random.default_rng(0), kh, vh, sd, cw)
    wconv, wa, wdt, wn = (backend.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    buf = backend.alloc(4 * (ch + vd + 2 * vh))
    st = backend.alloc(4 * (ch * cw + vh * sd * sd))
    p = DeltaNetParams(kh, vh, sd, cw, 1e-6, buf, buf, buf, buf, wconv, wa, wdt, wn, st, st, buf)
    for count, stride, out_stride in ((0, ch, vd), (2, ch - 1, vd), (2, ch, vd - 1), ((1 << 19) + 1, ch, vd)):
        with pytest.raises(InvalidArgument):
            backend.delta_net_batch(p, count, stride, out_stride)
    # the recurrent state's rows move as 16-byte accesses: a state 4 bytes off is refused
    # by every entry point that takes one, before anything runs
    bad = DeltaNetParams(kh, vh, sd, cw, 1e-6, buf, buf, buf, buf, wconv, wa, wdt, wn, st, st + 4, buf)
    for call in (lambda: backend.delta_net(bad), lambda: backend.delta_net_noalloc(bad),
                 lambda: backend.delta_net_batch(bad, 2, ch, vd)):
        with pytest.raises(InvalidArgument):
            call()


@pytest.mark.parametrize("H,kh,vh,sd,positions", [(512, 4, 8, 64, 40), (4096, 16, 32, 128, 2048)])
def test_delta_net_prefill_then_recurrent_shares_state(backend, H, kh, vh, sd, positions):
    """The reference adapter's call order: the reference prefill calls
    Backend::delta_net once per prompt position with the layer slot (model.cpp:301-306 ->
    :162-183) and decode calls recurrent_block on the same slot, whose state the CUDA
    backend keeps on the device (cuda.cpp:934-984). Here: emprise_hip_delta_net per
    position, then emprise_hip_recurrent, on one pair of state buffers, against the CPU
    oracle doing the same. The 2048-position case issues the eager per-position
    delta_net launches of a 2048-token prompt."""
    rng = np.random.default_rng(31)
    cw, eps = 4, 1e-6
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = _gdn_inputs(rng, kh, vh, sd, cw)
    wconv, wa, wdt, wn = (backend.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    conv_c, rec_c = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    conv_g, rec_g = backend.to_device(conv_c), backend.to_device(rec_c)
    bufs = {k: backend.alloc(n * 4) for k, n in (("qkv", ch), ("gate", vd), ("alpha", vh), ("beta", vh), ("out", vd))}
    p = DeltaNetParams(kh, vh, sd, cw, eps, bufs["qkv"], bufs["gate"], bufs["alpha"], bufs["beta"], wconv, wa, wdt,
                       wn, conv_g, rec_g, bufs["out"])
    check = {0, 1, positions // 2, positions - 1}
    for t in range(positions):
        qkv = rng.standard_normal(ch).astype(np.float32)
        gate = rng.standard_normal(vd).astype(np.float32)
        alpha = rng.standard_normal(vh).astype(np.float32)
        beta = rng.standard_normal(vh).astype(np.float32)
        for k, v in (("qkv", qkv), ("gate", gate), ("alpha", alpha), ("beta", beta)):
            backend.upload(bufs[k], v)
        backend.delta_net(p)
        ref = oracle.delta_net(kh, vh, sd, cw, eps, qkv, gate, alpha, beta, prm["conv"], prm["ssm_a"], prm["dt"],
                               prm["norm"], conv_c, rec_c)
        if t in check:
            _close(backend.download(bufs["out"], vd), ref, what=f"prefill position {t}")
    _close(backend.download(rec_g, vh * sd * sd), rec_c, what="state after the prefill")
    raws = {"qkv": (ch, H), "gate": (vd, H), "alpha": (vh, H), "beta": (vh, H), "out": (H, vd)}
    raws = {k: (r, c, matrix(rng, Q6_K, r, c)) for k, (r, c) in raws.items()}
    ws = {k: backend.upload_weight(Q6_K, c, r, raw) for k, (r, c, raw) in raws.items()}
    rp = RecurrentParams(ws["qkv"], ws["gate"], ws["alpha"], ws["beta"], ws["out"], wconv, wa, wdt, wn, kh, vh, sd,
                         cw, eps, conv_g, rec_g)
    xd, yd = backend.alloc(H * 4), backend.alloc(H * 4)
    for step in range(3):
        x = rng.standard_normal(H).astype(np.float32)
        backend.upload(xd, x)
        backend.recurrent(rp, xd, yd)
        proj = {k: oracle.matvec(Q6_K, raws[k][2], x, raws[k][0]) for k in ("qkv", "gate", "alpha", "beta")}
        dn = oracle.delta_net(kh, vh, sd, cw, eps, proj["qkv"], proj["gate"], proj["alpha"], proj["beta"],
                              prm["conv"], prm["ssm_a"], prm["dt"], prm["norm"], conv_c, rec_c)
        _close(backend.download(yd, H), oracle.matvec(Q6_K, raws["out"][2], dn, H), what=f"decode step {step}")
        _close(backend.download(rec_g, vh * sd * sd), rec_c, what=f"decode step {step} state")
    for w in ws.values():
        backend.weight_free(w)
    for b in list(bufs.values()) + [xd, yd, conv_g, rec_g]:
        backend.free(b)


@pytest.mark.parametrize("wtype,kh,vh,sd", [(Q6_K, 16, 32, 128), (Q4_K, 16, 32, 128), (Q6_K, 16, 64, 64)])
def test_recurrent_block(backend, wtype, kh, vh, sd):
    """dev_recurrent: fused projections + conv epilogue + scan + out projection. With a
    4096-wide chunked out weight the state update runs split per head and the per-head
    RMSNorm x SiLU(gate) runs in the out projection's input staging."""
    rng = np.random.default_rng(7)
    H, cw, eps = 4096, 4, 1e-6
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = _gdn_inputs(rng, kh, vh, sd, cw)
    raws = {"qkv": (ch, H), "gate": (vd, H), "alpha": (vh, H), "beta": (vh, H), "out": (H, vd)}
    raws = {k: (r, c, matrix(rng, wtype, r, c)) for k, (r, c) in raws.items()}
    ws = {k: backend.upload_weight(wtype, c, r, raw) for k, (r, c, raw) in raws.items()}
    wconv, wa, wdt, wn = (backend.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    conv_c, rec_c = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    conv_g, rec_g = backend.to_device(conv_c), backend.to_device(rec_c)
    p = RecurrentParams(ws["qkv"], ws["gate"], ws["alpha"], ws["beta"], ws["out"], wconv, wa, wdt, wn, kh, vh, sd,
                        cw, eps, conv_g, rec_g)
    xd, yd = backend.alloc(H * 4), backend.alloc(H * 4)
    for step in range(3):
        x = rng.standard_normal(H).astype(np.float32)
        backend.upload(xd, x)
        backend.recurrent(p, xd, yd)
        proj = {k: oracle.matvec(wtype, raws[k][2], x, raws[k][0]) for k in ("qkv", "gate", "alpha", "beta")}
        dn = oracle.delta_net(kh, vh, sd, cw, eps, proj["qkv"], proj["gate"], proj["alpha"], proj["beta"],
                              prm["conv"], prm["ssm_a"], prm["dt"], prm["norm"], conv_c, rec_c)
        ref = oracle.matvec(wtype, raws["out"][2], dn, H)
        _close(backend.download(yd, H), ref, what=f"step {step}")
        _close(backend.download(rec_g, vh * sd * sd), rec_c, what=f"step {step} state")


@pytest.mark.parametrize("H,kh,vh,sd", [(4096, 16, 32, 128), (512, 4, 8, 64)])
def test_recurrent_block_q8(backend_q8, H, kh, vh, sd):
    """--fast-q8 on the 9B and tiny recurrent shapes: every Q6_K projection quantises its
    input (core.cpp:119-125), the out projection after the per-head norm x gate of its
    staging. Tolerance: the Q8 matvec bound, plus one +-1 rounding flip of a quantised dn
    value (dn differs from the CPU's in the last bits before quantisation)."""
    rng = np.random.default_rng(17)
    cw, eps = 4, 1e-6
    kd, vd = kh * sd, vh * sd
    ch = 2 * kd + vd
    prm = _gdn_inputs(rng, kh, vh, sd, cw)
    raws = {"qkv": (ch, H), "gate": (vd, H), "alpha": (vh, H), "beta": (vh, H), "out": (H, vd)}
    raws = {k: (r, c, matrix(rng, Q6_K, r, c)) for k, (r, c) in raws.items()}
    ws = {k: backend_q8.upload_weight(Q6_K, c, r, raw) for k, (r, c, raw) in raws.items()}
    wconv, wa, wdt, wn = (backend_q8.vector(prm[k]) for k in ("conv", "ssm_a", "dt", "norm"))
    conv_c, rec_c = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    conv_g, rec_g = backend_q8.to_device(conv_c), backend_q8.to_device(rec_c)
    p = RecurrentParams(ws["qkv"], ws["gate"], ws["alpha"], ws["beta"], ws["out"], wconv, wa, wdt, wn, kh, vh, sd,
                        cw, eps, conv_g, rec_g)
    xd, yd = backend_q8.alloc(H * 4), backend_q8.alloc(H * 4)
    wout = oracle.dequantize(Q6_K, raws["out"][2], H * vd).reshape(H, vd)
    for step in range(3):
        x = rng.standard_normal(H).astype(np.float32)
        backend_q8.upload(xd, x)
        backend_q8.recurrent(p, xd, yd)
        xq = quantize_like_reference(x)
        proj = {k: oracle.matvec(Q6_K, raws[k][2], xq, raws[k][0]) for k in ("qkv", "gate", "alpha", "beta")}
        dn = oracle.delta_net(kh, vh, sd, cw, eps, proj["qkv"], proj["gate"], proj["alpha"], proj["beta"],
                              prm["conv"], prm["ssm_a"], prm["dt"], prm["norm"], conv_c, rec_c)
        ref = oracle.matvec(Q6_K, raws["out"][2], quantize_like_reference(dn), H)
        got = backend_q8.download(yd, H)
        step_q = np.repeat(np.max(np.abs(dn.reshape(-1, 32)), axis=1) / 127, 32)  # one quantum per column
        flip = np.max(np.abs(wout) * step_q[None, :], axis=1)
        bad = np.abs(got - ref) > 1e-3 + 1e-4 * np.abs(ref) + flip
        assert not bad.any(), (step, int(bad.sum()), float(np.max(np.abs(got - ref))))
        _close(backend_q8.download(rec_g, vh * sd * sd), rec_c, tol=2e-4, what=f"step {step} state")


def _attention_case(backend, heads, kv, hd, rot, L, context, seed, base=1e7, eps=1e-6):
    rng = np.random.default_rng(seed)
    kvd = kv * hd
    qn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    keys = np.zeros((context, kvd), np.float32)
    values = np.zeros((context, kvd), np.float32)
    keys[:L - 1] = rng.standard_normal((L - 1, kvd)).astype(np.float32)
    values[:L - 1] = rng.standard_normal((L - 1, kvd)).astype(np.float32)
    qg = rng.standard_normal(heads * hd * 2).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    kd_, vd_ = backend.to_device(keys), backend.to_device(values)
    qkv = backend.to_device(np.concatenate([qg, k, v]))
    pos = backend.to_device(np.array([L - 1], np.int32))
    out = backend.alloc(heads * hd * 4)
    p = AttentionParams(heads, kv, hd, rot, context, eps, base, backend.vector(qn), backend.vector(kn), kd_, vd_, pos)
    backend.attention(p, qkv, out)
    got = backend.download(out, heads * hd)
    ref = oracle.attention(heads, kv, hd, rot, base, eps, qn, kn, qg, k, v, keys, values, L, L - 1)
    _close(got, ref, what=f"L={L}")
    # the new k/v landed at row L-1 of the caches
    _close(backend.download(kd_, (context, kvd))[L - 1], keys[L - 1])
    assert np.array_equal(backend.download(vd_, (context, kvd))[L - 1], v)
    for b in (kd_, vd_, qkv, pos, out):
        backend.free(b)


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 129, 512, 1025, 2048, 4095, 4096])
def test_attention_config2b(backend, L):
    """Config 2b: 16 Q / 4 KV heads, head_dim 256, partial RoPE over 64 dims."""
    _attention_case(backend, 16, 4, 256, 64, L, 4096, seed=L)


@pytest.mark.parametrize("L", [1, 7, 130])
def test_attention_tiny(backend, L):
    _attention_case(backend, 8, 2, 64, 16, L, 512, seed=100 + L)


@pytest.mark.parametrize("heads,kv,hd,rot,first,count,context", [(16, 4, 256, 64, 0, 40, 4096),
                                                                (16, 4, 256, 64, 100, 37, 4096),
                                                                (8, 2, 64, 16, 0, 130, 512), (8, 2, 64, 16, 5, 1, 512)])
def test_attention_batch_matches_steps(backend, heads, kv, hd, rot, first, count, context):
    """emprise_hip_attention_batch over positions first..first+count-1 (strided qkv rows,
    caches holding `first` earlier rows) against `count` decode attention calls on a copy
    of the caches: outputs within the per-op bar (GEMM summation order), appended K/V rows
    equal; two outputs also against the oracle."""
    rng = np.random.default_rng(3 + first + count)
    kvd, qd = kv * hd, heads * hd * 2
    W = qd + 2 * kvd + 4
    qn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    keys = np.zeros((context, kvd), np.float32)
    values = np.zeros((context, kvd), np.float32)
    keys[:first] = rng.standard_normal((first, kvd)).astype(np.float32)
    values[:first] = rng.standard_normal((first, kvd)).astype(np.float32)
    rows = rng.standard_normal((count, W)).astype(np.float32)
    qnv, knv = backend.vector(qn), backend.vector(kn)
    # position by position
    ks, vs = backend.to_device(keys), backend.to_device(values)
    qkv1, pos, out1 = backend.alloc(W * 4), backend.alloc(4), backend.alloc(heads * hd * 4)
    seq = np.zeros((count, heads * hd), np.float32)
    for t in range(count):
        backend.upload(qkv1, rows[t])
        backend.upload(pos, np.array([first + t], np.int32))
        p = AttentionParams(heads, kv, hd, rot, context, 1e-6, 1e7, qnv, knv, ks, vs, pos)
        backend.attention(p, qkv1, out1)
        seq[t] = backend.download(out1, heads * hd)
    # batched
    kb, vb = backend.to_device(keys), backend.to_device(values)
    rows_d = backend.to_device(rows)
    out_stride = heads * hd + 8
    ob = backend.alloc(count * out_stride * 4)
    p = AttentionParams(heads, kv, hd, rot, context, 1e-6, 1e7, qnv, knv, kb, vb, 0)
    backend.attention_batch(p, rows_d, count, W, first, ob, out_stride)
    got = backend.download(ob, count * out_stride).reshape(count, out_stride)[:, :heads * hd]
    for t in range(count):
        _close(got[t], seq[t], what=f"position {first + t}")
    n = first + count
    _close(backend.download(kb, (context, kvd))[:n], backend.download(ks, (context, kvd))[:n], what="keys")
    assert np.array_equal(backend.download(vb, (context, kvd))[:n], backend.download(vs, (context, kvd))[:n])
    for t in (0, count - 1):
        r = rows[t]
        kc = backend.download(kb, (context, kvd)).copy()
        vc = backend.download(vb, (context, kvd)).copy()
        ref = oracle.attention(heads, kv, hd, rot, 1e7, 1e-6, qn, kn, r[:qd], r[qd:qd + kvd], r[qd + kvd:qd + 2 * kvd],
                               kc, vc, first + t + 1, first + t)
        _close(got[t], ref, what=f"position {first + t} vs oracle")


def test_attention_rejects_bad_shape(backend):
    p = AttentionParams(16, 5, 256, 64, 64, 1e-6, 1e7, backend.vector(np.ones(256, np.float32)),
                        backend.vector(np.ones(256, np.float32)), 1, 1, 1)
    with pytest.raises(InvalidArgument):
        backend.attention(p, 1, 1)


def test_graph_replay_matches_eager(backend):
    """A captured linear_norm + argmax sequence replayed several times (with eager
    work between replays) gives the eager result each time."""
    rng = np.random.default_rng(9)
    cols, rows = 4096, 20000
    raw = matrix(rng, Q6_K, rows, cols)
    w = backend.upload_weight(Q6_K, cols, rows, raw)
    nw = backend.vector((1 + 0.02 * rng.standard_normal(cols)).astype(np.float32))
    xd, dd, xo, yd, idx = (backend.alloc(cols * 4), backend.alloc(cols * 4), backend.alloc(cols * 4),
                           backend.alloc(rows * 4), backend.alloc(4))
    inp = Input(xd, dd, xo, nw, 1e-6)
    backend.upload(xd, rng.standard_normal(cols).astype(np.float32))
    backend.upload(dd, rng.standard_normal(cols).astype(np.float32))
    backend.linear_norm(inp, [w], [yd])
    backend.argmax(yd, rows, idx)
    eager_y, eager_i = backend.download(yd, rows), backend.download(idx, 1, np.int32)
    backend.graph_begin()
    backend.linear_norm(inp, [w], [yd])
    backend.argmax(yd, rows, idx)
    g = backend.graph_end()
    for _ in range(4):
        backend.fill(yd, 0.0, rows)
        backend.upload(idx, np.array([-1], np.int32))
        backend.graph_launch(g)
        backend.sync()
        assert np.array_equal(backend.download(yd, rows), eager_y)
        assert backend.download(idx, 1, np.int32)[0] == eager_i[0]
    backend.graph_destroy(g)
    backend.weight_free(w)


def test_stream_read_sees_every_word(backend):
    """The read-bandwidth probe (bench.py's achievable-HBM figure) reads every byte: the
    XOR of its per-workgroup words is the XOR of the buffer, for a buffer of more 4 KiB
    pieces than waves (several pieces each) and one of fewer; sizes that are not whole
    pieces are refused."""
    rng = np.random.default_rng(11)
    sink = backend.alloc(4096 * 4)
    for pieces in (3000, 5):
        data = rng.integers(0, 2**32, size=pieces * 4096, dtype=np.uint32)
        src = backend.to_device(data)
        backend.fill(sink, 0.0, 4096)
        backend.stream_read(src, data.nbytes, sink)
        words = backend.download(sink, (4096,), np.uint32)
        assert np.bitwise_xor.reduce(words) == np.bitwise_xor.reduce(data), pieces
        with pytest.raises(InvalidArgument):
            backend.stream_read(src, data.nbytes - 4, sink)
        backend.free(src)
    backend.free(sink)


def _q8_reference(x):
    """quantize_x's rule in numpy: per 32 values s = amax / 127 (FP32), codes round(v / s)
    with ties away from zero on the IEEE FP32 quotient, scale kept as fp16(s)."""
    blocks = x.reshape(-1, 32)
    s = (np.max(np.abs(blocks), axis=1) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = (blocks / s[:, None]).astype(np.float32)
    q = np.where(np.abs(r - np.trunc(r)) == 0.5, np.trunc(r) + np.sign(r), np.round(r))
    q = np.where(s[:, None] == 0, 0, q).astype(np.int8).reshape(-1)
    return q, s.astype(np.float16).astype(np.float32)


def test_quantize_q8_exact_on_ties_and_scales(backend):
    """The quantiser's quotient v / s (computed from one reciprocal per block and a
    correction step, not a division per value) equals the IEEE quotient: blocks whose scale
    is a power of two with values exactly on every half-integer code boundary (ties away
    from zero), their FP32 neighbours on both sides, random blocks over scales from 1e-30
    to 1e30, a block whose scale is below 2^-125 (the per-value division path) and a zero
    block; codes and kept scales equal numpy's bit for bit."""
    rng = np.random.default_rng(17)
    blocks = []
    for e in range(-40, 41, 5):  # s = 2^e exactly: amax = 127 * 2^e
        base = np.float32(2.0 ** e)
        for lo in range(-127, 127, 31):
            ties = (np.arange(lo, lo + 31, dtype=np.float64) + 0.5) * float(base)
            b = np.concatenate([[127 * float(base)], ties]).astype(np.float32)
            blocks += [b, np.nextafter(b, np.float32(np.inf)), np.nextafter(b, np.float32(-np.inf))]
            blocks[-2][0] = blocks[-1][0] = b[0]  # keep amax, so s stays 2^e
    for mag in (1e-30, 1e-12, 1e-3, 1.0, 7.5, 1e6, 1e30):
        blocks += list((rng.standard_normal((64, 32)) * mag).astype(np.float32))
    tiny = (rng.uniform(-1, 1, 32) * 2e-36).astype(np.float32)  # s ~ 1.6e-38 < 2^-125: the division path
    tiny[5] = np.float32(2e-36)
    blocks += [tiny, np.zeros(32, np.float32)]
    x = np.concatenate(blocks).astype(np.float32)
    n = x.size
    xd, qd, sd = backend.to_device(x), backend.alloc(n), backend.alloc(n // 32 * 4)
    backend.quantize_q8(xd, n, qd, sd)
    q = backend.download(qd, n, np.int8)
    s = backend.download(sd, n // 32)
    q_ref, s_ref = _q8_reference(x)
    bad = np.nonzero(q != q_ref)[0]
    assert bad.size == 0, f"{bad.size} codes differ, first at {bad[0]}: x {x[bad[0]]!r} got {q[bad[0]]} want {q_ref[bad[0]]}"
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    for b in (xd, qd, sd):
        backend.free(b)
