"""Closed forms and invariants that pin the oracle functions the reference's compiled
code does not expose (RMSNorm, RoPE and attention live in model.cpp's private
Model::Impl). Each check is chosen so a dropped term, wrong sign/index or transposed
operand fails it. CPU only."""
import numpy as np

import oracle


def test_rms_closed_form():
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    got = oracle.rms(x, w, 0.0)
    s = 1 / np.sqrt(12.5)  # mean of squares (9 + 16) / 2
    assert np.allclose(got, [3 * s, 8 * s], rtol=1e-7)
    # eps enters under the root, not outside
    assert np.allclose(oracle.rms(np.zeros(4, np.float32), np.ones(4, np.float32), 1.0), 0)
    assert np.allclose(oracle.rms(np.ones(4, np.float32), np.ones(4, np.float32), 3.0), 0.5)


def test_rope_identity_at_position_zero_and_norm_preserving():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 16, 0, 1e7), x)
    y = oracle.rope(x, 16, 37, 1e7)
    # rotation of pairs (i, i+8) for i < 8; the other 48 dims untouched
    assert np.array_equal(y[16:], x[16:])
    for i in range(8):
        a, b = x[i], x[i + 8]
        assert abs(np.hypot(y[i], y[i + 8]) - np.hypot(a, b)) < 1e-5
        ang = 37 / np.power(1e7, 2 * i / 16)
        assert np.allclose([y[i], y[i + 8]], [a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)],
                           atol=2e-5)


def _attn(heads, kv, hd, rot, L, rng, keys=None, values=None, qg=None, k=None, v=None):
    ctx = L
    qn, kn = np.ones(hd, np.float32), np.ones(hd, np.float32)
    if keys is None:
        keys = np.zeros((ctx, kv * hd), np.float32)
        values = np.zeros((ctx, kv * hd), np.float32)
        keys[:L - 1] = rng.standard_normal((L - 1, kv * hd))
        values[:L - 1] = rng.standard_normal((L - 1, kv * hd))
    qg = rng.standard_normal(heads * hd * 2).astype(np.float32) if qg is None else qg
    k = rng.standard_normal(kv * hd).astype(np.float32) if k is None else k
    v = rng.standard_normal(kv * hd).astype(np.float32) if v is None else v
    out = oracle.attention(heads, kv, hd, rot, 1e7, 1e-6, qn, kn, qg, k, v, keys, values, L, L - 1)
    return out, keys, values, qg, k, v


def _sig(x):
    return 1 / (1 + np.exp(-x.astype(np.float64)))


def test_attention_single_position_is_gated_value():
    """L = 1: softmax over one key is 1, so o = v[kv head] * sigmoid(gate)."""
    rng = np.random.default_rng(1)
    heads, kv, hd = 4, 2, 64
    out, keys, values, qg, k, v = _attn(heads, kv, hd, 16, 1, rng)
    for h in range(heads):
        kh = h // (heads // kv)
        gate = qg[h * hd * 2 + hd:(h + 1) * hd * 2]
        assert np.allclose(out[h * hd:(h + 1) * hd], v[kh * hd:(kh + 1) * hd] * _sig(gate), rtol=1e-5, atol=1e-6)
    # the new key was normalised and stored (RoPE at pos 0 is the identity)
    kh0 = k[:hd] / np.sqrt(np.mean(k[:hd].astype(np.float64) ** 2) + 1e-6)
    assert np.allclose(keys[0, :hd], kh0, rtol=1e-5)


def test_attention_equal_keys_average_values():
    """Identical keys give uniform weights: o = mean of v over positions (GQA head map)."""
    rng = np.random.default_rng(2)
    heads, kv, hd, L = 4, 2, 64, 9
    base = rng.standard_normal(kv * hd).astype(np.float32)
    keys = np.zeros((L, kv * hd), np.float32)
    values = rng.standard_normal((L, kv * hd)).astype(np.float32)
    # the stored keys are post-norm; the new one is normalised with unit weights, so store
    # the normalised version of `base` at every earlier position (RoPE differs by position,
    # so use rotary = 0 to keep every key identical)
    kn = np.concatenate([base[i * hd:(i + 1) * hd] / np.sqrt(np.mean(base[i * hd:(i + 1) * hd].astype(np.float64) ** 2) + 1e-6)
                         for i in range(kv)]).astype(np.float32)
    keys[:L - 1] = kn
    v_new = values[L - 1].copy()
    qg = rng.standard_normal(heads * hd * 2).astype(np.float32)
    out = oracle.attention(heads, kv, hd, 0, 1e7, 1e-6, np.ones(hd, np.float32), np.ones(hd, np.float32), qg, base,
                           v_new, keys, values, L, L - 1)
    for h in range(heads):
        kh = h // (heads // kv)
        gate = qg[h * hd * 2 + hd:(h + 1) * hd * 2]
        want = values[:, kh * hd:(kh + 1) * hd].astype(np.float64).mean(0) * _sig(gate)
        assert np.allclose(out[h * hd:(h + 1) * hd], want, rtol=1e-4, atol=1e-5)


def test_attention_float64_brute_force():
    rng = np.random.default_rng(3)
    heads, kv, hd, rot, L = 8, 2, 64, 16, 40
    out, keys, values, qg, k, v = _attn(heads, kv, hd, rot, L, rng)
    pos = L - 1
    for h in range(heads):
        kh = h // (heads // kv)
        q = qg[h * hd * 2:h * hd * 2 + hd].astype(np.float64)
        q = q / np.sqrt(np.mean(q ** 2) + 1e-6)
        half = rot // 2
        ang = pos / np.power(1e7, 2 * np.arange(half) / rot)
        a, b = q[:half].copy(), q[half:rot].copy()
        q[:half], q[half:rot] = a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)
        K = keys[:L, kh * hd:(kh + 1) * hd].astype(np.float64)
        V = values[:L, kh * hd:(kh + 1) * hd].astype(np.float64)
        s = K @ q / np.sqrt(hd)
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ V * _sig(qg[h * hd * 2 + hd:(h + 1) * hd * 2])
        assert np.allclose(out[h * hd:(h + 1) * hd], want, rtol=1e-4, atol=1e-5)


def _dn(kh, vh, sd, cw, qkv, gate, alpha, beta, conv, a, dt, nw, cs, rs):
    return oracle.delta_net(kh, vh, sd, cw, 1e-6, qkv, gate, alpha, beta, conv, a, dt, nw, cs, rs)


def test_delta_net_zero_state_closed_form():
    """Zero state: S = b * v k^T, so o_d = b v_d (k.q) before the norm/gate; with
    beta -> -inf (b = 0) the state stays zero and the output is zero."""
    rng = np.random.default_rng(4)
    kh, vh, sd, cw = 1, 2, 64, 4
    ch = 2 * kh * sd + vh * sd
    conv = np.zeros(ch * cw, np.float32)
    conv[cw - 1::cw] = 1.0  # taps pick the newest input: conv output = silu(x)
    qkv = rng.standard_normal(ch).astype(np.float32)
    gate = np.full(vh * sd, 30.0, np.float32)  # silu(30) = 30 (sigmoid ~ 1)
    a = np.full(vh, -1.0, np.float32)
    dt = np.zeros(vh, np.float32)
    nw = np.ones(sd, np.float32)
    alpha = np.zeros(vh, np.float32)
    beta = np.array([40.0, -40.0], np.float32)  # b = 1 for head 0, b ~ 0 for head 1
    cs, rs = np.zeros(ch * cw, np.float32), np.zeros(vh * sd * sd, np.float32)
    out = _dn(kh, vh, sd, cw, qkv, gate, alpha, beta, conv, a, dt, nw, cs, rs)
    silu = lambda x: x / (1 + np.exp(-x.astype(np.float64)))
    c = silu(qkv)
    q, k, v = c[:sd], c[sd:2 * sd], c[2 * sd:]
    qh = q / np.sqrt((q ** 2).sum() + 1e-6) / np.sqrt(sd)
    kn = k / np.sqrt((k ** 2).sum() + 1e-6)
    o0 = v[:sd] * (kn @ qh)
    o0 = o0 / np.sqrt(np.mean(o0 ** 2) + 1e-6) * 30.0
    assert np.allclose(out[:sd], o0, rtol=2e-4, atol=1e-5)
    S0 = np.outer(v[:sd], kn)
    assert np.allclose(rs[:sd * sd].reshape(sd, sd), S0, rtol=1e-5, atol=1e-6)
    assert np.max(np.abs(rs[sd * sd:])) < 1e-15 * 0 + 1e-16


def test_delta_net_decay_only_when_beta_closed():
    """b = 0: the state is only multiplied by decay = exp(a * softplus(alpha + dt))."""
    rng = np.random.default_rng(5)
    kh, vh, sd, cw = 1, 1, 64, 4
    ch = 2 * kh * sd + vh * sd
    rs = rng.standard_normal(sd * sd).astype(np.float32)
    before = rs.copy()
    cs = np.zeros(ch * cw, np.float32)
    a, dt, alpha = np.array([-0.7], np.float32), np.array([0.3], np.float32), np.array([0.2], np.float32)
    _dn(kh, vh, sd, cw, rng.standard_normal(ch).astype(np.float32), np.ones(sd, np.float32), alpha,
        np.array([-200.0], np.float32), np.ones(ch * cw, np.float32), a, dt, np.ones(sd, np.float32), cs, rs)
    decay = np.exp(-0.7 * np.log1p(np.exp(0.5)))
    assert np.allclose(rs, before * decay, rtol=1e-6)


def test_delta_net_conv_history_shifts():
    """The conv state is the last conv_width inputs per channel, oldest first."""
    kh, vh, sd, cw = 1, 1, 64, 3
    ch = 2 * kh * sd + vh * sd
    cs, rs = np.zeros(ch * cw, np.float32), np.zeros(sd * sd, np.float32)
    ones = np.ones(ch * cw, np.float32)
    for t in range(4):
        qkv = np.full(ch, float(t + 1), np.float32)
        _dn(kh, vh, sd, cw, qkv, np.ones(sd, np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32), ones,
            np.full(1, -1.0, np.float32), np.zeros(1, np.float32), np.ones(sd, np.float32), cs, rs)
    assert np.array_equal(cs.reshape(ch, cw)[0], [2.0, 3.0, 4.0])


def test_attention_softmax_temperature_two_keys():
    """Two keys with a closed-form score pins the 1/sqrt(head_dim) temperature
    (model.cpp:143-148): q and the keys are axis vectors, so after the per-head RMSNorm
    (unit weights) q.k is known exactly and the softmax weight of key 0 is
    e^s / (e^s + 1) with s = q.k / sqrt(hd). A temperature of 1 or 1/hd misses it."""
    eps = 1e-6
    for hd in (4, 16):
        qg = np.zeros(2 * hd, np.float32)
        qg[2] = 1.0  # q = e_2; gate 0 -> sigmoid 1/2
        k_new = np.zeros(hd, np.float32)
        k_new[3] = 1.0  # new key e_3, orthogonal to q
        keys = np.zeros((2, hd), np.float32)
        values = np.zeros((2, hd), np.float32)
        norm = 1 / np.sqrt(1 / hd + eps)  # RMSNorm scale of an axis vector
        keys[0, 2] = norm  # key 0 already stored in its normalised form
        values[0, 0] = 1.0
        v_new = np.zeros(hd, np.float32)
        v_new[1] = 1.0
        out = oracle.attention(1, 1, hd, 0, 1e7, eps, np.ones(hd, np.float32), np.ones(hd, np.float32), qg, k_new,
                               v_new, keys, values, 2, 1)
        s = norm * norm / np.sqrt(hd)
        p0 = np.exp(s) / (np.exp(s) + 1)
        want = np.zeros(hd)
        want[0], want[1] = 0.5 * p0, 0.5 * (1 - p0)
        assert np.allclose(out, want, rtol=1e-5, atol=1e-7), (hd, out[:2], want[:2])
        for wrong in (s * np.sqrt(hd), s / np.sqrt(hd)):
            pw = np.exp(wrong) / (np.exp(wrong) + 1)
            assert abs(out[0] - 0.5 * pw) > 1e-3


def test_quantize_q8_matches_core_rule():
    """eo_quantize_q8 (the fast-q8 input of core.cpp:119-125) against the numpy statement
    of the same rule (tests/synth.py: float16 cast for fp16(s), ties away from zero by
    hand), bit for bit, over blocks that hit exact .5 ties, zero blocks, fp16-subnormal
    scales and large values; plus closed forms."""
    from synth import quantize_like_reference
    rng = np.random.default_rng(4)
    blocks = [rng.standard_normal(32) * 10.0 ** rng.uniform(-9, 4) for _ in range(200)]
    tie = np.arange(32, dtype=np.float64) - 15.5
    tie[0] = 127.0  # s = 1: every other value is an exact .5 tie
    blocks += [np.zeros(32), tie, -tie, np.full(32, 1e-9), np.full(32, 3e4)]
    x = np.concatenate(blocks).astype(np.float32)
    got = oracle.quantize_q8(x)
    assert np.array_equal(got.view(np.uint32), quantize_like_reference(x).view(np.uint32))
    # closed forms: s = 1 rounds half away from zero; a zero block stays zero
    t = got[201 * 32:202 * 32]
    assert t[1] == -15.0 and t[16] == 1.0 and t[15] == -1.0 and t[31] == 16.0
    assert not got[200 * 32:201 * 32].any()


# ---- the MTP draft head (model.cpp:376-397) on F32 models built to reduce it to closed forms

def _mtp_model(tmp_path, rng, eh="hidden", attn_out=False, ffn=False, name="mtp.gguf"):
    """One attention layer (unused by the draft) + the MTP block blk.1, H = 8 = 2 heads x 4,
    1 kv head, ffn 8, vocab 16. eh_proj selects one half of [enorm(e) | hnorm(h)]; the
    block's attention output and FFN down projections are zero unless asked for."""
    from gguf_f32 import write
    H, V, F, hd = 8, 16, 8, 4
    meta = {"embedding_length": H, "block_count": 2, "nextn_predict_layers": 1, "feed_forward_length": F,
            "context_length": 64, "attention.head_count": 2, "attention.head_count_kv": 1,
            "attention.key_length": hd, "attention.value_length": hd, "rope.dimension_count": 2,
            "rope.freq_base": 10000.0, "attention.layer_norm_rms_epsilon": 1e-6, "ssm.group_count": 1,
            "ssm.time_step_rank": 1, "ssm.state_size": 4, "ssm.conv_kernel": 4, "eos": V}
    n = lambda *s: rng.standard_normal(s).astype(np.float32)
    w = lambda: (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    t = {"token_embd.weight": n(V, H), "output_norm.weight": w(), "output.weight": n(V, H)}
    for p in ("blk.0.", "blk.1."):
        t.update({p + "attn_norm.weight": w(), p + "post_attention_norm.weight": w(),
                  p + "attn_q.weight": n(2 * 2 * hd, H), p + "attn_k.weight": n(hd, H), p + "attn_v.weight": n(hd, H),
                  p + "attn_q_norm.weight": w()[:hd].copy(), p + "attn_k_norm.weight": w()[:hd].copy(),
                  p + "ffn_gate.weight": n(F, H), p + "ffn_up.weight": n(F, H)})
    t["blk.0.attn_output.weight"], t["blk.0.ffn_down.weight"] = n(H, H), n(H, F)
    t["blk.1.attn_output.weight"] = np.eye(H, dtype=np.float32) if attn_out else np.zeros((H, H), np.float32)
    t["blk.1.ffn_down.weight"] = n(H, F) if ffn else np.zeros((H, F), np.float32)
    sel = np.zeros((H, 2 * H), np.float32)
    sel[:, H:] = np.eye(H) if eh == "hidden" else 0
    sel[:, :H] = np.eye(H) if eh == "embedding" else 0
    t["blk.1.nextn.eh_proj.weight"] = sel
    t.update({"blk.1.nextn.enorm.weight": w(), "blk.1.nextn.hnorm.weight": w(),
              "blk.1.nextn.shared_head_norm.weight": w()})
    p = tmp_path / name
    write(p, meta, t)
    return p, t


def _rms64(x, w, eps=1e-6):
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * w


def _close64(got, want, rel=1e-5):
    assert np.max(np.abs(got - want)) <= rel * np.max(np.abs(want)), (got, want)


def test_mtp_hidden_half_and_head(tmp_path):
    """eh_proj = [0 | I], attention output and FFN down zero: the block's output is
    hnorm(hidden) and the logits are output . head_norm(hnorm(hidden)). The embedding half
    and the block's residual branches contribute nothing."""
    rng = np.random.default_rng(7)
    path, t = _mtp_model(tmp_path, rng, eh="hidden")
    m = oracle.Model(str(path), context=64)
    assert m.has_mtp
    h = rng.standard_normal(8).astype(np.float32)
    logits = m.mtp_draft(h, 3, 5)
    cur = _rms64(h, t["blk.1.nextn.hnorm.weight"])
    _close64(m.mtp_hidden(), cur)
    _close64(logits, t["output.weight"] @ _rms64(cur, t["blk.1.nextn.shared_head_norm.weight"]))


def test_mtp_embedding_half(tmp_path):
    """eh_proj = [I | 0]: the block's output is enorm(embedding row of the token),
    whatever the hidden vector."""
    rng = np.random.default_rng(8)
    path, t = _mtp_model(tmp_path, rng, eh="embedding")
    m = oracle.Model(str(path), context=64)
    for token in (0, 11):
        m.reset_mtp()
        m.mtp_draft(rng.standard_normal(8).astype(np.float32), token, 9)
        _close64(m.mtp_hidden(), _rms64(t["token_embd.weight"][token], t["blk.1.nextn.enorm.weight"]))


def test_mtp_attention_first_row(tmp_path):
    """The first draft after reset_mtp attends over one row, so each head's output is
    v of its kv head times sigmoid of its gate (the second half of the head's q
    projection); with attn_output = I it is added to the block's input."""
    rng = np.random.default_rng(9)
    path, t = _mtp_model(tmp_path, rng, eh="embedding", attn_out=True)
    m = oracle.Model(str(path), context=64)
    token = 5
    m.mtp_draft(rng.standard_normal(8).astype(np.float32), token, 17)
    cur = _rms64(t["token_embd.weight"][token], t["blk.1.nextn.enorm.weight"])
    a = _rms64(cur, t["blk.1.attn_norm.weight"])
    qg = t["blk.1.attn_q.weight"].astype(np.float64) @ a
    v = t["blk.1.attn_v.weight"].astype(np.float64) @ a
    o = np.concatenate([v / (1 + np.exp(-qg[h * 8 + 4:h * 8 + 8])) for h in range(2)])
    _close64(m.mtp_hidden(), cur + o)


def test_mtp_feed_forward(tmp_path):
    """With the attention output zero, the block adds down(silu(gate p) * up p) with p =
    post_norm(rms(block input))."""
    rng = np.random.default_rng(10)
    path, t = _mtp_model(tmp_path, rng, eh="hidden", ffn=True)
    m = oracle.Model(str(path), context=64)
    h = rng.standard_normal(8).astype(np.float32)
    m.mtp_draft(h, 2, 3)
    cur = _rms64(h, t["blk.1.nextn.hnorm.weight"])
    p = _rms64(cur, t["blk.1.post_attention_norm.weight"])
    g, u = t["blk.1.ffn_gate.weight"] @ p, t["blk.1.ffn_up.weight"] @ p
    _close64(m.mtp_hidden(), cur + t["blk.1.ffn_down.weight"].astype(np.float64) @ (g / (1 + np.exp(-g)) * u))


def test_mtp_cache_grows_until_reset(tmp_path):
    """Without reset_mtp the block's cache keeps every draft's row: a draft of token 9
    after one of token 4 attends over both rows and differs from the same draft on an
    empty cache; after reset_mtp a repeated draft gives the first one's bits."""
    rng = np.random.default_rng(11)
    path, _ = _mtp_model(tmp_path, rng, eh="embedding", attn_out=True)
    m = oracle.Model(str(path), context=64)
    h = rng.standard_normal(8).astype(np.float32)
    first = m.mtp_draft(h, 4, 6)
    chained = m.mtp_draft(h, 9, 7)
    m.reset_mtp()
    alone = m.mtp_draft(h, 9, 7)
    assert not np.allclose(chained, alone)
    m.reset_mtp()
    assert np.array_equal(m.mtp_draft(h, 4, 6).view(np.uint32), first.view(np.uint32))


def test_last_hidden_normed_is_output_norm_of_raw(tmp_path):
    """Model::last_hidden is the last residual through the output norm."""
    rng = np.random.default_rng(12)
    path, t = _mtp_model(tmp_path, rng)
    m = oracle.Model(str(path), context=64)
    m.evaluate(1)
    _close64(m.last_hidden(normed=True), _rms64(m.last_hidden(), t["output_norm.weight"]))
