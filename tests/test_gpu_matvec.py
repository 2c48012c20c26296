"""Dequant-matvec parity on the GPU through the C ABI against the CPU oracle.

Bars (north star): dequantised weights bit-exact; FP32 outputs within max-abs error
1e-4 * max|ref|; the Q8 path within 1e-3 + 1e-4*|ref| of the CPU matvec on the
explicitly quantised input (reference tests/core.cpp:115, :119-129).
"""
import numpy as np
import pytest

import oracle
from emprise_amd import BF16, F16, F32, Q4_K, Q6_K, Input, InvalidArgument
from synth import quantize_like_reference, matrix

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _close(got, ref, tol=TOL):
    err = np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))
    bound = tol * max(np.max(np.abs(ref)), 1e-30)
    assert err <= bound, f"max abs err {err:.3e} > {bound:.3e}"


def _run_linear(be, wtype, rows, cols, seed, x=None):
    rng = np.random.default_rng(seed)
    raw = matrix(rng, wtype, rows, cols)
    if x is None:
        x = rng.standard_normal(cols).astype(np.float32)
    w = be.upload_weight(wtype, cols, rows, raw)
    xd, yd = be.to_device(x), be.alloc(rows * 4)
    be.linear(w, xd, yd)
    y = be.download(yd, rows)
    be.free(xd)
    be.free(yd)
    be.weight_free(w)
    return raw, x, y


@pytest.mark.parametrize("wtype", [Q6_K, Q4_K, F32, F16, BF16])
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 512), (64, 1536), (129, 4096), (33, 12288)])
def test_linear_small_vs_oracle(backend, wtype, rows, cols):
    raw, x, y = _run_linear(backend, wtype, rows, cols, seed=rows * 7 + cols + wtype)
    _close(y, oracle.matvec(wtype, raw, x, rows))


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (12288, 4096), (4096, 12288)])
@pytest.mark.parametrize("wtype", [Q6_K, Q4_K])
def test_linear_config1_shapes(backend, wtype, rows, cols):
    raw, x, y = _run_linear(backend, wtype, rows, cols, seed=rows + cols + wtype)
    _close(y, oracle.matvec(wtype, raw, x, rows))


@pytest.mark.parametrize("wtype", [Q6_K, Q4_K])
def test_linear_lm_head(backend, wtype):
    rows, cols = 151936, 4096
    raw, x, y = _run_linear(backend, wtype, rows, cols, seed=5 + wtype)
    row_bytes = len(raw) // rows
    # oracle on three row windows: first, middle, last (rows are independent)
    for r0 in (0, rows // 2 - 700, rows - 1500):
        n = 1500
        ref = oracle.matvec(wtype, raw[r0 * row_bytes:(r0 + n) * row_bytes], x, n)
        _close(y[r0:r0 + n], ref)
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("wtype,K,rows,cols", [(Q6_K, 3, 64, 512), (Q6_K, 37, 300, 512), (Q4_K, 130, 257, 4096),
                                               (F32, 9, 33, 256), (Q6_K, 64, 512, 12288), (F16, 20, 40, 1536),
                                               (Q6_K, 2, 4096, 4096), (Q4_K, 4, 1000, 4096), (Q6_K, 5, 333, 8192),
                                               (Q6_K, 7, 257, 12288), (Q4_K, 4, 4096, 12288), (Q6_K, 3, 151936, 4096),
                                               (Q6_K, 8, 4096, 4096), (Q6_K, 200, 300, 4096), (Q4_K, 129, 1000, 8192),
                                               (Q6_K, 40, 130, 12288), (Q4_K, 8, 128, 4096)])
def test_linear_batch(backend, wtype, K, rows, cols):
    """Backend::linear_batch (backend.hpp:20-24): Y[k] = W X[k]. From 8 tokens up it runs
    on the matrix cores -- chunked Q6_K/Q4_K weights on exact fp16 pieces of weights and
    activations with FP32 sums, other weights as an FP32 GEMM on exactly dequantised
    weights; from 2 to 7 through a chunked Q6_K/Q4_K matrix as the small-batch matvec (up
    to 4 inputs per launch, 3 at 12288 columns, the weights read once per launch); every
    token must match the CPU matvec, and the single-token projection, to the per-op bar
    (batched == sequential, reference tests/core.cpp:149-164). Token and row counts off
    the 128 x 128 tiles included."""
    rng = np.random.default_rng(K * 131 + rows + cols + wtype)
    raw = matrix(rng, wtype, rows, cols)
    X = rng.standard_normal((K, cols)).astype(np.float32)
    w = backend.upload_weight(wtype, cols, rows, raw)
    xd, yd = backend.to_device(X), backend.alloc(K * rows * 4)
    backend.linear_batch(w, xd, yd, K)
    Y = backend.download(yd, (K, rows))
    x1, y1 = backend.alloc(cols * 4), backend.alloc(rows * 4)
    for k in range(K):
        ref = oracle.matvec(wtype, raw, X[k], rows)
        _close(Y[k], ref)
        if k in (0, K - 1):
            backend.upload(x1, X[k])
            backend.linear(w, x1, y1)
            _close(Y[k], backend.download(y1, rows))
    for b in (xd, yd, x1, y1):
        backend.free(b)
    backend.weight_free(w)


@pytest.mark.parametrize("wtype", [Q6_K, Q4_K])
def test_linear_batch_wide_range(backend, wtype):
    """The fp16 GEMM scales each token row by a power of two before splitting it into fp16
    pieces: rows of 1e6-sized, 1e-6-sized, mixed and all-zero activations (and one whose
    values would overflow fp16 unscaled) all meet the per-op bar against the CPU matvec."""
    rows, cols = 200, 4096
    rng = np.random.default_rng(wtype + 5)
    raw = matrix(rng, wtype, rows, cols)
    X = rng.standard_normal((12, cols)).astype(np.float32)
    X[0] *= 1e6
    X[1] *= 1e-6
    X[2, ::2] *= 1e5
    X[3] = 0.0
    X[4] *= 7e4  # beyond fp16's 65504 without the row scale
    X[5, :100] = 0.0
    w = backend.upload_weight(wtype, cols, rows, raw)
    xd, yd = backend.to_device(X), backend.alloc(len(X) * rows * 4)
    backend.linear_batch(w, xd, yd, len(X))
    Y = backend.download(yd, (len(X), rows))
    for k in range(len(X)):
        ref = oracle.matvec(wtype, raw, X[k], rows)
        if not np.any(ref):
            assert np.all(Y[k] == 0.0), k
        else:
            _close(Y[k], ref)
    backend.free(xd)
    backend.free(yd)
    backend.weight_free(w)


# (type, K, F, cols, ldy pad): the paired GEMM (8+ tokens, chunked Q6_K/Q4_K), tile-ragged
# token and row counts, the 9B FFN shape; fewer than 8 tokens and F32 weights take the
# two-projection path
@pytest.mark.parametrize("wtype,K,F,cols,pad", [(Q6_K, 8, 1000, 4096, 0), (Q4_K, 129, 1000, 4096, 3),
                                                (Q6_K, 200, 12288, 4096, 0), (Q4_K, 300, 64, 8192, 5),
                                                (Q6_K, 3, 700, 4096, 1), (F32, 40, 96, 512, 2)])
def test_ffn_gate_up_batch(backend, wtype, K, F, cols, pad):
    """emprise_hip_ffn_gate_up_batch: Y[k] = silu(G X[k]) * (U X[k]) equals the two
    projections of linear_batch_strided followed by swiglu, bit for bit (the paired
    GEMM interleaves gate and up rows and forms the SwiGLU in its epilogue), and the
    per-op bar against the CPU matvecs for the first and last token."""
    rng = np.random.default_rng(K * 7 + F + wtype)
    if wtype == F32:
        rg = rng.standard_normal((F, cols)).astype(np.float32) * 0.05
        ru = rng.standard_normal((F, cols)).astype(np.float32) * 0.05
        g = backend.upload_weight(F32, cols, F, rg.tobytes())
        u = backend.upload_weight(F32, cols, F, ru.tobytes())
    else:
        rg, ru = matrix(rng, wtype, F, cols), matrix(rng, wtype, F, cols)
        g, u = backend.upload_weight(wtype, cols, F, rg), backend.upload_weight(wtype, cols, F, ru)
    X = rng.standard_normal((K, cols)).astype(np.float32)
    ldy = F + pad
    xd, yd = backend.to_device(X), backend.alloc(K * ldy * 4)
    backend.ffn_gate_up_batch(g, u, xd, cols, yd, ldy, K)
    Y = backend.download(yd, (K, ldy))[:, :F]
    gd, ud = backend.alloc(K * F * 4), backend.alloc(K * F * 4)
    backend.linear_batch_strided(g, xd, cols, gd, F, K)
    backend.linear_batch_strided(u, xd, cols, ud, F, K)
    backend.swiglu(gd, ud, K * F)
    assert np.array_equal(Y, backend.download(gd, (K, F)))
    for k in (0, K - 1):
        if wtype == F32:
            gr, ur = rg @ X[k], ru @ X[k]
        else:
            gr, ur = oracle.matvec(wtype, rg, X[k], F), oracle.matvec(wtype, ru, X[k], F)
        ref = (gr / (1 + np.exp(-gr.astype(np.float64))) * ur).astype(np.float32)
        _close(Y[k], ref)
    for b in (xd, yd, gd, ud):
        backend.free(b)
    backend.weight_free(g)
    backend.weight_free(u)


@pytest.mark.parametrize("K", [3, 40])
def test_linear_batch_strided(backend, K):
    """Strided batched projection writes its rows into a slice of wider output rows."""
    rows, cols, ldy, off = 96, 512, 300, 37
    rng = np.random.default_rng(K)
    raw = matrix(rng, Q6_K, rows, cols)
    X = rng.standard_normal((K, cols + 16)).astype(np.float32)
    w = backend.upload_weight(Q6_K, cols, rows, raw)
    xd = backend.to_device(X)
    Y0 = np.full((K, ldy), 7.0, np.float32)
    yd = backend.to_device(Y0)
    backend.linear_batch_strided(w, xd, cols + 16, yd + off * 4, ldy, K)
    Y = backend.download(yd, (K, ldy))
    for k in range(K):
        _close(Y[k, off:off + rows], oracle.matvec(Q6_K, raw, X[k, :cols], rows))
    assert np.all(Y[:, :off] == 7.0) and np.all(Y[:, off + rows:] == 7.0)
    backend.free(xd)
    backend.free(yd)
    backend.weight_free(w)


@pytest.mark.parametrize("K", [3, 40])
def test_linear_batch_many(backend, K):
    """Stacked weights (mixed types) in one batched call: each weight's rows land after
    the previous weight's, equal to the oracle and bit-equal to one call per weight."""
    cols, ldy, off = 4096, 700, 11
    specs = [(Q6_K, 200), (Q4_K, 32), (F32, 16), (Q6_K, 300)]
    rng = np.random.default_rng(K + 1)
    raws = [(t, r, matrix(rng, t, r, cols)) for t, r in specs]
    ws = [backend.upload_weight(t, cols, r, raw) for t, r, raw in raws]
    X = rng.standard_normal((K, cols)).astype(np.float32)
    xd = backend.to_device(X)
    Y0 = np.full((K, ldy), 7.0, np.float32)
    yd, y1 = backend.to_device(Y0), backend.to_device(Y0)
    backend.linear_batch_many(ws, xd, cols, yd + off * 4, ldy, K)
    Y = backend.download(yd, (K, ldy))
    o = off
    for (t, r, raw), w in zip(raws, ws):
        backend.linear_batch_strided(w, xd, cols, y1 + o * 4, ldy, K)
        for k in range(K):
            _close(Y[k, o:o + r], oracle.matvec(t, raw, X[k], r))
        o += r
    assert np.array_equal(Y, backend.download(y1, (K, ldy)))
    assert np.all(Y[:, :off] == 7.0) and np.all(Y[:, o:] == 7.0)
    wn = backend.upload_weight(Q6_K, 2048, 16, matrix(rng, Q6_K, 16, 2048))
    with pytest.raises(InvalidArgument):  # input widths differ
        backend.linear_batch_many([ws[0], wn], xd, cols, yd, ldy, K)
    for b in (xd, yd, y1):
        backend.free(b)
    for w in ws + [wn]:
        backend.weight_free(w)


def test_linear_batch_many_over_scratch_blocks(backend):
    """Stacked rows beyond one dequantisation block (16384 rows of 4096): the second
    weight straddles the block boundary; bit-equal to one call per weight."""
    cols, K = 4096, 8
    rng = np.random.default_rng(5)
    specs = [(Q6_K, 12000), (Q4_K, 6000)]
    ws = [backend.upload_weight(t, cols, r, matrix(rng, t, r, cols)) for t, r in specs]
    ldy = sum(r for _, r in specs)
    xd = backend.to_device(rng.standard_normal((K, cols)).astype(np.float32))
    yd, y1 = backend.alloc(K * ldy * 4), backend.alloc(K * ldy * 4)
    backend.linear_batch_many(ws, xd, cols, yd, ldy, K)
    backend.linear_batch_strided(ws[0], xd, cols, y1, ldy, K)
    backend.linear_batch_strided(ws[1], xd, cols, y1 + specs[0][1] * 4, ldy, K)
    assert np.array_equal(backend.download(yd, (K, ldy)), backend.download(y1, (K, ldy)))
    for b in (xd, yd, y1):
        backend.free(b)
    for w in ws:
        backend.weight_free(w)


# widths: chunked layout (one and two 4096-column chunks), multiples of 1024, others
@pytest.mark.parametrize("wtype,rows,cols", [(Q6_K, 300, 4096), (Q4_K, 300, 4096), (Q6_K, 5, 1536), (Q4_K, 7, 512),
                                             (Q6_K, 3, 8192), (Q4_K, 5, 8192), (Q6_K, 6, 2048), (Q4_K, 6, 3072),
                                             (F16, 9, 512), (BF16, 9, 512), (F32, 9, 256), (F32, 4, 1024)])
def test_dequantize_bit_exact(backend, wtype, rows, cols):
    rng = np.random.default_rng(11)
    raw = matrix(rng, wtype, rows, cols)
    w = backend.upload_weight(wtype, cols, rows, raw)
    out = backend.alloc(rows * cols * 4)
    backend.dequantize_rows(w, 0, rows, out)
    got = backend.download(out, rows * cols)
    ref = oracle.dequantize(wtype, raw, rows * cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a block of rows starting past row 0 (the GEMM path dequantises in blocks)
    r0, n = rows // 3, rows - rows // 3 - 1
    backend.dequantize_rows(w, r0, n, out)
    got = backend.download(out, n * cols)
    assert np.array_equal(got.view(np.uint32), ref[r0 * cols:(r0 + n) * cols].view(np.uint32))
    # the device re-layout is lossless: reading it back restores the GGUF bytes
    assert backend.weight_download_gguf(w, len(raw)) == raw
    backend.free(out)
    backend.weight_free(w)


def test_q6k_subnormal_and_extreme_scales(backend):
    """fp16 d subnormal/largest and sc at -32/31 keep exact products (no flush)."""
    rng = np.random.default_rng(3)
    from synth import q6k_blocks
    b = q6k_blocks(rng, 64)
    d_bits = np.array([0x0001, 0x03ff, 0x0400, 0x7bff, 0x3c00, 0x8001, 0x0200, 0x0010] * 8, dtype=np.uint16)
    b[:, 208:210] = d_bits.view(np.uint8).reshape(64, 2)
    b[::2, 192:208] = np.int8(-32).view(np.uint8)
    b[1::2, 192:208] = np.int8(31).view(np.uint8)
    raw = b.tobytes()
    rows, cols = 4, 4096
    w = backend.upload_weight(Q6_K, cols, rows, raw)
    out = backend.alloc(rows * cols * 4)
    backend.dequantize_rows(w, 0, rows, out)
    got = backend.download(out, rows * cols)
    ref = oracle.dequantize(Q6_K, raw, rows * cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    backend.free(out)
    backend.weight_free(w)


def test_linear_many_matches_single(backend):
    rng = np.random.default_rng(21)
    cols = 4096
    shapes = [8192, 4096, 32, 32]  # GDN qkv, gate, alpha, beta
    raws = [matrix(rng, Q6_K, r, cols) for r in shapes]
    x = rng.standard_normal(cols).astype(np.float32)
    ws = [backend.upload_weight(Q6_K, cols, r, raw) for r, raw in zip(shapes, raws)]
    xd = backend.to_device(x)
    ys = [backend.alloc(r * 4) for r in shapes]
    backend.linear_many(ws, xd, ys)
    many = [backend.download(y, r) for y, r in zip(ys, shapes)]
    for w, y, r, got in zip(ws, ys, shapes, many):
        backend.linear(w, xd, y)
        assert np.array_equal(backend.download(y, r), got)
    for raw, r, got in zip(raws, shapes, many):
        _close(got, oracle.matvec(Q6_K, raw, x, r))


def test_linear_norm_fuses_add_and_rmsnorm(backend):
    rng = np.random.default_rng(22)
    cols, rows, eps = 4096, 1024, 1e-6
    raw = matrix(rng, Q6_K, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    delta = rng.standard_normal(cols).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    w = backend.upload_weight(Q6_K, cols, rows, raw)
    nwd = backend.vector(nw)
    xd, dd, xo, yd = backend.to_device(x), backend.to_device(delta), backend.alloc(cols * 4), backend.alloc(rows * 4)
    backend.linear_norm(Input(xd, dd, xo, nwd, eps), [w], [yd])
    v = x + delta
    assert np.array_equal(backend.download(xo, cols), v)
    ref = oracle.matvec(Q6_K, raw, oracle.rms(v, nw, eps), rows)
    _close(backend.download(yd, rows), ref)


@pytest.mark.parametrize("wtype", [Q6_K, Q4_K])
def test_feed_forward(backend, wtype):
    rng = np.random.default_rng(23)
    hidden, ffn = 4096, 12288
    graw, uraw, draw = matrix(rng, wtype, ffn, hidden), matrix(rng, wtype, ffn, hidden), matrix(rng, Q6_K, hidden, ffn)
    x = rng.standard_normal(hidden).astype(np.float32)
    g = backend.upload_weight(wtype, hidden, ffn, graw)
    u = backend.upload_weight(wtype, hidden, ffn, uraw)
    d = backend.upload_weight(Q6_K, ffn, hidden, draw)
    xd, yd = backend.to_device(x), backend.alloc(hidden * 4)
    backend.feed_forward(g, u, d, xd, yd)
    got = backend.download(yd, hidden)
    gr, ur = oracle.matvec(wtype, graw, x, ffn), oracle.matvec(wtype, uraw, x, ffn)
    e = np.exp(-np.abs(gr))
    s = np.where(gr >= 0, 1 / (1 + e), e / (1 + e)).astype(np.float32)
    h = (gr * s * ur).astype(np.float32)
    _close(got, oracle.matvec(Q6_K, draw, h, hidden))
    for w in (g, u, d):
        backend.weight_free(w)


@pytest.mark.parametrize("rows,cols", [(256, 4096), (4096, 4096), (1024, 12288), (12288, 4096), (4096, 12288),
                                       (151936, 4096), (64, 512), (1536, 512), (512, 1536)])
def test_q8_path(backend_q8, rows, cols):
    raw, x, got = _run_linear(backend_q8, Q6_K, rows, cols, seed=rows + cols)
    ref = oracle.matvec(Q6_K, raw, quantize_like_reference(x), rows)
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-4 * np.abs(ref)), np.max(np.abs(got - ref))
    assert "Q8" in backend_q8.name


def test_q8_leaves_q4k_on_fp32(backend_q8):
    """--fast-q8 quantises activations for Q6_K only (cuda.cpp:709-718)."""
    raw, x, y = _run_linear(backend_q8, Q4_K, 64, 4096, seed=77)
    _close(y, oracle.matvec(Q4_K, raw, x, 64))


def test_shape_errors(backend):
    with pytest.raises(InvalidArgument):
        backend.upload_weight(Q6_K, 255, 1, b"\0" * 210)
    with pytest.raises(InvalidArgument):
        backend.upload_weight(Q6_K, 256, 1, b"\0" * 209)
    with pytest.raises(InvalidArgument):
        backend.upload_weight(7, 256, 1, b"\0" * 1024)
    w1 = backend.upload_weight(F32, 512, 2, np.zeros(1024, np.float32).tobytes())
    w2 = backend.upload_weight(F32, 256, 2, np.zeros(512, np.float32).tobytes())
    x, y = backend.alloc(4096), backend.alloc(4096)
    with pytest.raises(InvalidArgument):
        backend.linear_many([w1, w2], x, [y, y])
    backend.weight_free(w1)
    backend.weight_free(w2)


def test_core_fp32_2x2(backend):
    """core.cpp:92-98: [[1,2],[-3,4]] . [2,3] = [8,6] on the device."""
    w = backend.upload_weight(F32, 2, 2, np.array([1, 2, -3, 4], np.float32).tobytes())
    x, y = backend.to_device(np.array([2, 3], np.float32)), backend.alloc(8)
    backend.linear(w, x, y)
    assert backend.download(y, 2).tolist() == [8.0, 6.0]


def test_budget_exhaustion():
    from emprise_amd import ENOMEM, EmpriseError, HipBackend
    with HipBackend(0, weight_budget=1000) as be:
        with pytest.raises(EmpriseError) as e:
            be.upload_weight(Q6_K, 4096, 1, b"\0" * 3360)
        assert e.value.status == ENOMEM


def _q8_check(got, raw, rows, cols, xin):
    """The Q8 bar of core.cpp:119-129 (CPU matvec on round(x/s)*fp16(s), within
    1e-3 + 1e-4|ref|), plus one quantum of the input (s = amax/127 of its 32-block) times
    the largest weight of each row: the GPU quantises its own FP32 input, which can differ
    from the CPU's in the last bits and round one step the other way."""
    ref = oracle.matvec(Q6_K, raw, quantize_like_reference(xin), rows)
    w = np.abs(oracle.dequantize(Q6_K, raw, rows * cols).reshape(rows, cols))
    step = np.repeat(np.max(np.abs(xin.reshape(-1, 32)), axis=1) / 127, 32)
    flip = np.max(w * step[None, :], axis=1)
    bad = np.abs(got - ref) > 1e-3 + 1e-4 * np.abs(ref) + flip
    assert not bad.any(), (int(bad.sum()), float(np.max(np.abs(got - ref))))
    return ref


@pytest.mark.parametrize("rows,cols", [(1536, 512), (1024, 4096)])
def test_linear_norm_q8(backend_q8, rows, cols):
    """--fast-q8 with the residual add + RMSNorm prologue: the normalised input is what
    gets quantised (device_linear after dev_add + dev_rmsnorm, cuda.cpp:707-712)."""
    rng = np.random.default_rng(rows + cols)
    eps = 1e-6
    raw = matrix(rng, Q6_K, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    delta = rng.standard_normal(cols).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    be = backend_q8
    w, nwd = be.upload_weight(Q6_K, cols, rows, raw), be.vector(nw)
    xd, dd, xo, yd = be.to_device(x), be.to_device(delta), be.alloc(cols * 4), be.alloc(rows * 4)
    be.linear_norm(Input(xd, dd, xo, nwd, eps), [w], [yd])
    _q8_check(be.download(yd, rows), raw, rows, cols, oracle.rms(x + delta, nw, eps))
    for b in (xd, dd, xo, yd):
        be.free(b)
    be.weight_free(w)


@pytest.mark.parametrize("hidden,ffn", [(512, 1536), (4096, 12288)])
def test_feed_forward_q8(backend_q8, hidden, ffn):
    """--fast-q8 SwiGLU FFN (cuda.cpp:897-927): gate and up on the quantised input, down
    on the quantised SwiGLU output."""
    rng = np.random.default_rng(hidden + 7)
    be = backend_q8
    graw, uraw, draw = matrix(rng, Q6_K, ffn, hidden), matrix(rng, Q6_K, ffn, hidden), matrix(rng, Q6_K, hidden, ffn)
    x = rng.standard_normal(hidden).astype(np.float32)
    g, u, d = (be.upload_weight(Q6_K, c, r, raw) for r, c, raw in ((ffn, hidden, graw), (ffn, hidden, uraw),
                                                                     (hidden, ffn, draw)))
    xd, yd = be.to_device(x), be.alloc(hidden * 4)
    be.feed_forward(g, u, d, xd, yd)
    xq = quantize_like_reference(x)
    gr, ur = oracle.matvec(Q6_K, graw, xq, ffn), oracle.matvec(Q6_K, uraw, xq, ffn)
    e = np.exp(-np.abs(gr))
    s = np.where(gr >= 0, 1 / (1 + e), e / (1 + e)).astype(np.float32)
    h = (gr * s * ur).astype(np.float32)
    _q8_check(be.download(yd, hidden), draw, hidden, ffn, h)
    for wt in (g, u, d):
        be.weight_free(wt)
    be.free(xd)
    be.free(yd)


@pytest.mark.parametrize("vocab,hidden", [(4096, 512), (151936, 4096)])
def test_lm_head_q8(backend_q8, vocab, hidden):
    """--fast-q8 output head: RMSNorm of x + delta, quantised, Q6_K matvec, argmax."""
    rng = np.random.default_rng(vocab)
    be = backend_q8
    eps = 1e-6
    raw = matrix(rng, Q6_K, vocab, hidden)
    x = rng.standard_normal(hidden).astype(np.float32)
    delta = rng.standard_normal(hidden).astype(np.float32)
    nw = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    w, nwd = be.upload_weight(Q6_K, hidden, vocab, raw), be.vector(nw)
    xd, dd, xo = be.to_device(x), be.to_device(delta), be.alloc(hidden * 4)
    ld, idx = be.alloc(vocab * 4), be.alloc(4)
    be.lm_head(Input(xd, dd, xo, nwd, eps), w, ld, idx)
    got = be.download(ld, vocab)
    _q8_check(got, raw, vocab, hidden, oracle.rms(x + delta, nw, eps))
    assert int(be.download(idx, 1, np.int32)[0]) == int(np.argmax(got))
    for b in (xd, dd, xo, ld, idx):
        be.free(b)
    be.weight_free(w)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (12288, 4096), (1024, 12288)])
def test_q8_register_quantiser_matches_lds_pass(backend_q8, rows, cols):
    """The quantiser in the fused-norm staging (from registers) against the generic
    staging's LDS pass, bit for bit. The input has mean(v^2) = 1 exactly (5/8 of the
    entries +-0.5, 3/8 +-1.5, in a seeded order) and the norm weights are 1 with eps = 0,
    so rms(v) * norm = v exactly and both paths quantise the same floats: once as
    x = v - delta, delta with the residual add, once as plain v without the norm."""
    rng = np.random.default_rng(rows * 3 + cols)
    mag = np.where(np.arange(cols) < cols * 5 // 8, 0.5, 1.5)
    v = (rng.permutation(mag) * rng.choice([-1.0, 1.0], cols)).astype(np.float32)
    delta = (rng.integers(-8, 9, cols) * 0.25).astype(np.float32)  # v - delta exact in FP32
    x = (v - delta).astype(np.float32)
    assert np.array_equal((x + delta).astype(np.float32), v) and float(np.mean(v.astype(np.float64) ** 2)) == 1.0
    be = backend_q8
    raw = matrix(rng, Q6_K, rows, cols)
    w, ones = be.upload_weight(Q6_K, cols, rows, raw), be.vector(np.ones(cols, np.float32))
    vd, xd, dd, xo = be.to_device(v), be.to_device(x), be.to_device(delta), be.alloc(cols * 4)
    y_plain, y_norm, y_delta = be.alloc(rows * 4), be.alloc(rows * 4), be.alloc(rows * 4)
    be.linear(w, vd, y_plain)
    be.linear_norm(Input(vd, 0, 0, ones, 0.0), [w], [y_norm])
    be.linear_norm(Input(xd, dd, xo, ones, 0.0), [w], [y_delta])
    a, b, c = (be.download(y, rows) for y in (y_plain, y_norm, y_delta))
    assert np.array_equal(be.download(xo, cols), v)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    _q8_check(a, raw, rows, cols, v)
    for t in (vd, xd, dd, xo, y_plain, y_norm, y_delta):
        be.free(t)
    be.weight_free(w)
