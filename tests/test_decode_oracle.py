"""Pins of the numpy decode-glue oracle (oracle/decode.py) against the
reference's own transformer tests and closed forms."""
import math

import numpy as np

from oracle import decode as od


def test_rope_reference_kats():
    # rope_test.zig:4-14
    np.testing.assert_allclose(od.rope_half(np.array([1, 0, 0, 1], np.float32), 0, 10000.0), [1, 0, 0, 1], atol=1e-6)
    np.testing.assert_allclose(od.rope_half(np.array([1, 0], np.float32), 1, 1.0), [math.cos(1.0), math.sin(1.0)],
                               atol=1e-6)


def test_rope_is_a_rotation_that_composes():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128)
    a = od.rope_half(x, 37, 1e6)
    # each pair keeps its length, and rotating by p then q is rotating by p+q
    half = 64
    np.testing.assert_allclose(np.hypot(a[:half], a[half:]), np.hypot(x[:half], x[half:]), rtol=1e-12)
    # (angles are f32 products, so composing positions holds to f32 rounding)
    np.testing.assert_allclose(od.rope_half(od.rope_half(x, 5, 1e6), 7, 1e6), od.rope_half(x, 12, 1e6), atol=2e-6)
    # the frequencies: pair i turns by pos * base^(-2i/hd)
    e = np.zeros(128)
    e[3] = 1.0
    r = od.rope_half(e, 10, 1e4)
    ang = 10 * 1e4 ** (-2 * 3 / 128)
    assert abs(r[3] - math.cos(ang)) < 1e-6 and abs(r[3 + half] - math.sin(ang)) < 1e-6


def test_rope_angle_is_the_f32_product_at_long_positions():
    # RopeTable (rope.zig:46-104) stores inv_freq as f32 and forms t * inv_freq
    # in f32; at position 32767 that angle is far (up to ~2e-3 rad) from the
    # exact one, and the oracle must rotate by the f32 angle
    half, pos = 64, 32767
    for i in (0, 1, 7, 40):
        e = np.zeros(2 * half)
        e[i] = 1.0
        r = od.rope_half(e, pos, 1e6)
        got = math.atan2(r[i + half], r[i])
        inv32 = np.float32(np.power(np.float32(1e6), np.float32(-2.0 * i / (2 * half))))
        want = float(np.float32(np.float32(pos) * inv32))
        exact = pos * 1e6 ** (-2.0 * i / (2 * half))
        d = (got - want + math.pi) % (2 * math.pi) - math.pi
        assert abs(d) < 1e-9, (i, d)
        if i == 0:  # pos * 1 is exact in f32 ...
            assert want == exact
        if i == 1:  # ... but pos * base^(-1/64) is not
            assert abs(want - exact) > 1e-5


def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(4096).astype(np.float32) * 5
    y = od.rms_norm(x, np.ones(4096, np.float32), 0.0)
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-5
    w = rng.standard_normal(4096).astype(np.float32)
    np.testing.assert_allclose(od.rms_norm(x, w, 1e-6), y * w, rtol=1e-5, atol=1e-6)


def test_write_kv_and_attend_reference_kat():
    # attention_test.zig:5-31: 4 q heads, 2 kv heads, head_dim 2, max_seq 4
    kc = np.zeros((2, 4, 2), np.float16)
    vc = np.zeros((2, 4, 2), np.float16)
    od.write_kv(np.array([1, 0, 0, 1], np.float32), np.array([2, 3, 4, 5], np.float32), kc, vc, 0)
    assert kc.reshape(-1)[0] == 1 and vc.reshape(-1)[1] == 3 and vc.reshape(-1)[8] == 4
    q = np.zeros(8, np.float32)
    q[:2] = [1, 0]
    out = od.attend(q, kc, vc, 4, 0, 1 / math.sqrt(2))
    np.testing.assert_allclose(out[:2], [2, 3], atol=1e-4)


def test_attend_invariants():
    rng = np.random.default_rng(3)
    kc = np.repeat(rng.standard_normal((1, 1, 8)), 5, axis=1).astype(np.float16)  # identical keys
    vc = rng.standard_normal((1, 5, 8)).astype(np.float16)
    out = od.attend(rng.standard_normal(16), kc, vc, 2, 4, 0.3)
    mean = vc[0].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(out[:8], mean, atol=1e-12)
    np.testing.assert_allclose(out[8:], mean, atol=1e-12)
    # one dominant score selects its value row
    kc2 = np.zeros((1, 5, 8), np.float16)
    kc2[0, 2, 0] = 60.0
    q = np.zeros(8)
    q[0] = 1.0
    np.testing.assert_allclose(od.attend(q, kc2, vc, 1, 4, 1.0), vc[0, 2].astype(np.float64), atol=1e-12)


def test_silu_mul_closed_forms_and_c_oracle():
    import oracle

    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 0.5, -2.5], np.float64)
    u = np.array([3.0, 2.0, 2.0, 0.5, 0.5, -4.0, 1.5], np.float64)
    y = od.silu_mul(g, u)
    assert y[0] == 0.0  # silu(0) = 0
    assert abs(y[1] - 2.0 / (1.0 + math.exp(-1.0))) < 1e-15
    # silu(-g) = silu(g) - g
    assert abs(y[2] / u[2] - (y[1] / u[1] - 1.0)) < 1e-15
    assert abs(y[3] - 15.0) < 1e-11 and abs(y[4]) < 1e-11  # saturation: silu(g) -> g, -> 0
    # against the C oracle's ActivationKind.silu.apply (f32), elementwise
    rng = np.random.default_rng(11)
    gg = (rng.standard_normal(256) * 4).astype(np.float32)
    uu = rng.standard_normal(256).astype(np.float32)
    c = np.array([oracle.act_apply(0, float(a), float(b)) for a, b in zip(gg, uu)], np.float64)
    np.testing.assert_allclose(od.silu_mul(gg, uu), c, rtol=2e-6, atol=1e-7)


def _qkv(rng, nh, nkv, hd):
    return (rng.standard_normal((nh + 2 * nkv) * hd) * 2).astype(np.float32)


def test_qk_norm_rope_structure():
    nh, nkv, hd, eps, base = 8, 2, 128, 1e-6, 1e6
    rng = np.random.default_rng(5)
    qkv = _qkv(rng, nh, nkv, hd)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    q0, k0, v0 = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 0)
    # v passes through untouched
    np.testing.assert_array_equal(v0, qkv[(nh + nkv) * hd:])
    # at position 0 the rotation is the identity: each head is RMS-normed with
    # its own weights (q heads by q_norm, k heads by k_norm)
    ones = np.ones(hd, np.float32)
    for h in range(nh):
        x = qkv[h * hd:(h + 1) * hd].astype(np.float64)
        unit = x / np.sqrt(np.mean(x * x) + eps)
        np.testing.assert_allclose(q0[h * hd:(h + 1) * hd], unit * qn, rtol=2e-6, atol=2e-6)
        np.testing.assert_allclose(od.rms_norm(x.astype(np.float32), ones, eps), unit, rtol=2e-6, atol=2e-6)
    for h in range(nkv):
        x = qkv[(nh + h) * hd:(nh + h + 1) * hd].astype(np.float64)
        np.testing.assert_allclose(k0[h * hd:(h + 1) * hd], x / np.sqrt(np.mean(x * x) + eps) * kn, rtol=2e-6,
                                   atol=2e-6)
    # at any position the pairs (i, i + hd/2) keep their lengths
    q9, k9, _ = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 9)
    half = hd // 2
    for a, b in ((q0, q9), (k0, k9)):
        a2, b2 = a.reshape(-1, hd).astype(np.float64), b.reshape(-1, hd).astype(np.float64)
        np.testing.assert_allclose(np.hypot(b2[:, :half], b2[:, half:]), np.hypot(a2[:, :half], a2[:, half:]),
                                   rtol=1e-5)
    # relative position: the q.k score of a q at m and a k at n depends on m - n only
    qa, _, _ = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 10)
    _, ka, _ = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 3)
    qb, _, _ = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 1007)
    _, kb, _ = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, 1000)
    sa = qa.reshape(nh, hd).astype(np.float64) @ ka.reshape(nkv, hd).astype(np.float64).T
    sb = qb.reshape(nh, hd).astype(np.float64) @ kb.reshape(nkv, hd).astype(np.float64).T
    np.testing.assert_allclose(sa, sb, rtol=1e-4, atol=1e-4)
    # heads are independent: swapping two q heads in the input swaps them in the output
    sw = qkv.copy()
    sw[0:hd], sw[3 * hd:4 * hd] = qkv[3 * hd:4 * hd], qkv[0:hd]
    qs, _, _ = od.qk_norm_rope(sw, qn, kn, nh, nkv, hd, eps, base, 9)
    np.testing.assert_array_equal(qs[0:hd], q9[3 * hd:4 * hd])
    np.testing.assert_array_equal(qs[3 * hd:4 * hd], q9[0:hd])


def _zero_scales(w, block_bytes):
    """Q4_0 / Q8_0 raw bytes with every block scale d = 0 (an all-zero matrix)."""
    z = w.reshape(-1, block_bytes).copy()
    z[:, 0:2] = 0
    return z.reshape(-1)


class _Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _small_model(cfg, rng):
    from zlm_amd import synth

    layers = []
    for i in range(cfg.n_layers):
        layers.append({
            "qkv": synth.weights(synth.Q4_0, (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim, cfg.hidden, 10 * i + 1),
            "o": synth.weights(synth.Q4_0, cfg.hidden, cfg.n_heads * cfg.head_dim, 10 * i + 2),
            "gate": synth.weights(synth.Q4_0, cfg.ffn, cfg.hidden, 10 * i + 3),
            "up": synth.weights(synth.Q4_0, cfg.ffn, cfg.hidden, 10 * i + 4),
            "down": synth.weights(synth.Q4_0, cfg.hidden, cfg.ffn, 10 * i + 5),
            "attn_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
            "ffn_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
            "q_norm": (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32),
            "k_norm": (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32),
        })
    return layers


def test_decode_step_with_zero_residual_branches_is_the_lm_head_of_the_input():
    """o and down all zero: every layer adds exactly 0 to the hidden state, so
    the logits are lm_head(RMSNorm(x_in, out_norm)) whatever the attention and
    MLP compute."""
    import oracle
    from zlm_amd import synth

    cfg = _Cfg(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=300, max_seq=16,
               eps=1e-6, freq_base=1e4)
    rng = np.random.default_rng(21)
    layers = _small_model(cfg, rng)
    for L in layers:
        L["o"] = _zero_scales(L["o"], 18)
        L["down"] = _zero_scales(L["down"], 18)
    lm = synth.weights(synth.Q8_0, cfg.vocab, cfg.hidden, 99)
    out_norm = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    x = rng.standard_normal(cfg.hidden).astype(np.float32)
    shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
    kc = [np.zeros(shape, np.float16) for _ in range(cfg.n_layers)]
    vc = [np.zeros(shape, np.float16) for _ in range(cfg.n_layers)]
    got = od.decode_step(cfg, layers, out_norm, lm, synth.Q8_0, synth.Q4_0, x, 3, kc, vc)
    want = oracle.matvec(synth.Q8_0, lm, cfg.hidden, cfg.vocab, od.rms_norm(x, out_norm, cfg.eps))
    np.testing.assert_array_equal(got, want)
    # the K/V append still happened at the step's position (and only there)
    assert np.any(kc[0][:, 3] != 0) and not np.any(kc[0][:, :3]) and not np.any(kc[0][:, 4:])


def test_decode_step_at_position_zero_attends_to_its_own_value():
    """At position 0 softmax runs over one score, so each q head's attention
    output is its kv head's value row (as stored in the f16 cache); with down
    all zero, one layer's logits are lm_head(RMSNorm(x + W_o . att))."""
    import oracle
    from zlm_amd import synth

    cfg = _Cfg(n_layers=1, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=200, max_seq=8,
               eps=1e-6, freq_base=1e4)
    rng = np.random.default_rng(22)
    layers = _small_model(cfg, rng)
    layers[0]["down"] = _zero_scales(layers[0]["down"], 18)
    lm = synth.weights(synth.Q8_0, cfg.vocab, cfg.hidden, 98)
    out_norm = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    x = rng.standard_normal(cfg.hidden).astype(np.float32)
    shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
    kc, vc = [np.zeros(shape, np.float16)], [np.zeros(shape, np.float16)]
    got = od.decode_step(cfg, layers, out_norm, lm, synth.Q8_0, synth.Q4_0, x, 0, kc, vc)
    v16 = vc[0][:, 0, :].astype(np.float32)  # the value rows the step stored, per kv head
    group = cfg.n_heads // cfg.n_kv_heads
    att = np.concatenate([v16[h // group] for h in range(cfg.n_heads)])
    # the stored value rows are the v part of the q;k;v projection of the normed input
    n = od.rms_norm(x, layers[0]["attn_norm"], cfg.eps)
    qkv = oracle.matvec(synth.Q4_0, layers[0]["qkv"], cfg.hidden, (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim, n)
    v = qkv[(cfg.n_heads + cfg.n_kv_heads) * cfg.head_dim:]
    np.testing.assert_array_equal(v16.reshape(-1), v.astype(np.float16).astype(np.float32))
    h1 = (x + oracle.matvec(synth.Q4_0, layers[0]["o"], cfg.n_heads * cfg.head_dim, cfg.hidden, att)).astype(
        np.float32)
    want = oracle.matvec(synth.Q8_0, lm, cfg.hidden, cfg.vocab, od.rms_norm(h1, out_norm, cfg.eps))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
