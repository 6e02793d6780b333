"""GPU parity of the decode-step glue and of whole decode steps.

* q/k head RMSNorm + RoPE + cache append, and split-K attention, against the
  numpy restatement (oracle/decode.py) of reference transformer/norm.zig,
  rope.zig and attention.zig (relative L2 <= 1e-4 in fp32; the f16 cache rows
  within one f16 rounding);
* a small Qwen3-shaped model (2 layers, 4 q / 2 kv heads of 128) stepped
  through positions 0, 1, 2 and 70 against the oracle's layer sequence
  (block.zig:20-41), eager and replayed from one captured HIP graph:
  logits relative L2 <= 1e-3;
* the configs[2] model (Qwen3-8B shapes, weights synthesised in HBM): an eager
  step and graph replays give bit-identical, finite logits.
"""
import math
import sys

import numpy as np
import pytest

from oracle import decode as od
from tests.helpers import rel_l2
from zlm_amd import decode as zdec
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _vec(dev, a):
    p = dev.dev_malloc(max(16, a.nbytes))
    dev.dev_upload(p, np.ascontiguousarray(a))
    return p


@pytest.mark.parametrize("pos", [0, 5, 2047])
def test_qk_norm_rope_kv_matches_oracle(dev, pos):
    nh, nkv, hd, max_seq, eps, base = 32, 8, 128, 2048, 1e-6, 1e6
    _say(f"qk_norm_rope pos={pos}")
    rng = np.random.default_rng(pos)
    qkv = (rng.standard_normal((nh + 2 * nkv) * hd) * 2).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    vc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    d_qkv, d_qn, d_kn, d_kc, d_vc = (_vec(dev, a) for a in (qkv, qn, kn, kc0, vc0))
    d_q = dev.dev_malloc(nh * hd * 4)
    d_pos = _vec(dev, np.array([pos, 0, 0, 0], np.int32))
    assert dev.qk_norm_rope_kv_enqueue(d_qkv, d_q, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc, d_vc, max_seq), \
        dev.last_error()
    q = np.zeros(nh * hd, np.float32)
    kc, vc = np.zeros_like(kc0), np.zeros_like(vc0)
    dev.dev_download(q, d_q)
    dev.dev_download(kc, d_kc)
    dev.dev_download(vc, d_vc)
    wq, wk, wv = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, pos)
    assert rel_l2(q, wq) <= 1e-4
    kref, vref = kc0.copy(), vc0.copy()
    od.write_kv(wk, wv, kref, vref, pos)
    # rows other than pos untouched; row pos within one f16 rounding
    others = np.ones(max_seq, bool)
    others[pos] = False
    np.testing.assert_array_equal(kc[:, others], kc0[:, others])
    np.testing.assert_array_equal(vc[:, others], vc0[:, others])
    np.testing.assert_array_equal(vc[:, pos], vref[:, pos])
    np.testing.assert_allclose(kc[:, pos].astype(np.float32), kref[:, pos].astype(np.float32), rtol=2e-3, atol=1e-3)
    for p in (d_qkv, d_qn, d_kn, d_kc, d_vc, d_q, d_pos):
        dev.dev_free(p)


@pytest.mark.parametrize("nh,nkv,L", [(32, 8, 1), (32, 8, 63), (32, 8, 64), (32, 8, 65), (32, 8, 2048),
                                      (16, 16, 300), (8, 4, 129)])
def test_attention_matches_oracle(dev, nh, nkv, L):
    hd, max_seq = 128, 2048
    _say(f"attention nh={nh} nkv={nkv} L={L}")
    rng = np.random.default_rng(L + nh)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    vc = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    scale = 1.0 / math.sqrt(hd)
    d_q, d_kc, d_vc = _vec(dev, q), _vec(dev, kc), _vec(dev, vc)
    d_pos = _vec(dev, np.array([L - 1, 0, 0, 0], np.int32))
    d_out = dev.dev_malloc(nh * hd * 4)
    assert dev.attention_enqueue(d_q, d_kc, d_vc, nh, nkv, hd, d_pos, max_seq, scale, d_out), dev.last_error()
    out = np.zeros(nh * hd, np.float32)
    dev.dev_download(out, d_out)
    want = od.attend(q, kc, vc, nh, L - 1, scale)
    assert rel_l2(out, want) <= 1e-4
    for p in (d_q, d_kc, d_vc, d_pos, d_out):
        dev.dev_free(p)


FUSED_CASES = [(32, 8, 0, 2048), (32, 8, 63, 2048), (32, 8, 64, 2048), (32, 8, 700, 2048), (32, 8, 2047, 2048),
               (8, 4, 129, 2048), (16, 16, 5, 2048),
               # past 64 splits the 16-wave merge runs: 94 splits (2 per wave
               # for most waves), 512 (one chunk of 32 per wave) and 625 (two
               # chunks, the running rescale); the later positions hold the
               # larger scores
               (32, 8, 5999, 6000), (8, 2, 4100, 6000), (32, 8, 32767, 32768), (8, 2, 39999, 40000),
               # 65 splits (the first wide case), the new row alone in the last
               (32, 8, 4096, 4100)]


@pytest.mark.parametrize("nh,nkv,pos,max_seq", FUSED_CASES)
def test_fused_attention_decode_matches_oracle(dev, nh, nkv, pos, max_seq):
    """q/k head norm + RoPE, K/V append at pos and attention in one launch, then the merge."""
    hd, eps, base = 128, 1e-6, 1e6
    _say(f"attention_decode nh={nh} nkv={nkv} pos={pos} max_seq={max_seq}")
    rng = np.random.default_rng(pos + nh)
    qkv = (rng.standard_normal((nh + 2 * nkv) * hd) * 2).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    vc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    if max_seq > 2048:
        kc0[:, 2048:] *= np.float16(1.5)
        # a mean offset keeps the output from being a near-cancelling average
        # of thousands of zero-mean rows, whose fp32 rounding alone would be
        # ~5e-4 of it at 32768 positions (the same for either merge kernel)
        vc0 += np.float16(0.5)
    scale = 1.0 / math.sqrt(hd)
    d_qkv, d_qn, d_kn, d_kc, d_vc = (_vec(dev, a) for a in (qkv, qn, kn, kc0, vc0))
    d_pos = _vec(dev, np.array([pos, 0, 0, 0], np.int32))
    d_out = dev.dev_malloc(nh * hd * 4)
    q, k, v = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, pos)
    kref, vref = kc0.copy(), vc0.copy()
    od.write_kv(k, v, kref, vref, pos)
    want = od.attend(q, kref, vref, nh, pos, scale)
    for rep in range(3):  # later calls over the appended caches give the same result
        assert dev.attention_decode_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc, d_vc, max_seq,
                                            scale, d_out), dev.last_error()
        out = np.zeros(nh * hd, np.float32)
        dev.dev_download(out, d_out)
        assert rel_l2(out, want) <= 1e-4, rep
    kc, vc = np.zeros_like(kc0), np.zeros_like(vc0)
    dev.dev_download(kc, d_kc)
    dev.dev_download(vc, d_vc)
    np.testing.assert_array_equal(vc, vref)
    # the new K row is rotated by f32 angles pos * base^(-2i/hd); one ulp of
    # the f32 pow moves the angle by ~pos * 6e-8 rad (2e-3 at 32767), so long
    # caches get that much slack on the row
    atol = 1e-3 if pos < 4096 else 4 * pos * 6e-8
    np.testing.assert_allclose(kc.astype(np.float32), kref.astype(np.float32), rtol=2e-3, atol=atol)
    for p in (d_qkv, d_qn, d_kn, d_kc, d_vc, d_pos, d_out):
        dev.dev_free(p)


def test_attention_rejects_unsupported_shapes(dev):
    p = dev.dev_malloc(1 << 16)
    assert not dev.attention_enqueue(p, p, p, 32, 8, 64, p, 16, 1.0, p)  # head_dim
    assert not dev.attention_enqueue(p, p, p, 40, 8, 128, p, 16, 1.0, p)  # 5 q heads per kv head
    assert not dev.attention_enqueue(p, p, p, 30, 8, 128, p, 16, 1.0, p)  # not a multiple
    dev.dev_free(p)


TINY = zdec.DecodeConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768, vocab=1000,
                         max_seq=80)


def _tiny_host(cfg, seed=7):
    rng = np.random.default_rng(seed)
    layers = []
    for i in range(cfg.n_layers):
        s = seed * 100 + 10 * i
        layers.append({
            "qkv": synth.weights(synth.Q4_0, cfg.qkv_rows, cfg.hidden, s + 1),
            "o": synth.weights(synth.Q4_0, cfg.hidden, cfg.n_heads * cfg.head_dim, s + 2),
            "gate": synth.weights(synth.Q4_0, cfg.ffn, cfg.hidden, s + 3),
            "up": synth.weights(synth.Q4_0, cfg.ffn, cfg.hidden, s + 4),
            "down": synth.weights(synth.Q4_0, cfg.hidden, cfg.ffn, s + 5),
            "attn_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
            "ffn_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
            "q_norm": (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32),
            "k_norm": (1 + 0.1 * rng.standard_normal(cfg.head_dim)).astype(np.float32),
        })
    return {"layers": layers, "lm_head": synth.weights(synth.Q8_0, cfg.vocab, cfg.hidden, seed + 99),
            "out_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)}


def test_tiny_decode_steps_match_oracle(dev):
    cfg = TINY
    host = _tiny_host(cfg)
    model = zdec.DecodeModel(dev, cfg, host=host)
    shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
    kref = [np.zeros(shape, np.float16) for _ in range(cfg.n_layers)]
    vref = [np.zeros(shape, np.float16) for _ in range(cfg.n_layers)]
    graph = None
    try:
        for step, pos in enumerate([0, 1, 2, 70]):
            _say(f"tiny decode pos={pos}")
            x = synth.activation(100 + pos, cfg.hidden)
            want = od.decode_step(cfg, host["layers"], host["out_norm"], host["lm_head"], synth.Q8_0, synth.Q4_0, x,
                                  pos, kref, vref)
            if step < 2:
                got = model.step(x, pos)
            else:  # replay the graph captured after the eager steps
                if graph is None:
                    graph = model.capture()
                model.set_input(x, pos)
                dev.graph_launch(graph, 1)
                got = model.logits_host()
            assert np.all(np.isfinite(got))
            assert rel_l2(got, want) <= 1e-3, (pos, rel_l2(got, want))
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        model.free()


def test_qwen3_8b_step_matches_oracle_and_graph_replays_match_eager(dev):
    """configs[2] at full size: weights synthesised in HBM, caches holding a
    2047-token history; the step at position 2047 (attention over 2048) against
    the oracle's 36-layer sequence over the same weights and caches (read back
    from HBM; the GEMVs through the oracle's pooled production sweep,
    bit-identical to its scalar one), relative L2 <= 1e-3 on the logits; then
    graph replays equal the eager step bit for bit."""
    cfg = zdec.QWEN3_8B
    _say("qwen3-8b decode: building the model in HBM")
    model = zdec.DecodeModel(dev, cfg)
    graph = None
    try:
        x = synth.activation(0x5A4C4D02, cfg.hidden)
        host = model.host_copy()
        _say("qwen3-8b decode: eager step")
        eager = model.step(x, cfg.max_seq - 1)
        assert np.all(np.isfinite(eager))
        _say("qwen3-8b decode: oracle step")
        import oracle
        kref = [L.pop("k_cache") for L in host["layers"]]
        vref = [L.pop("v_cache") for L in host["layers"]]
        want = od.decode_step(cfg, host["layers"], host["out_norm"], host["lm_head"], cfg.lm_type, cfg.proj_type,
                              x, cfg.max_seq - 1, kref, vref, matvec=oracle.pooled_matvec)
        del host
        assert rel_l2(eager, want) <= 1e-3, rel_l2(eager, want)
        graph = model.capture()
        for _ in range(3):
            model.set_input(x, cfg.max_seq - 1)
            dev.graph_launch(graph, 1)
            np.testing.assert_array_equal(model.logits_host(), eager)
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        model.free()


# (nh, nkv, pos, max_seq, window): the attention over a window of the caches,
# one split (64), the 128 bucket, a window of 1024 in a 32768 cache, and a
# window past 64 splits (the wide merge) in a 40000 cache
WINDOW_CASES = [(32, 8, 5, 2048, 64), (32, 8, 100, 2048, 128), (32, 8, 700, 32768, 1024),
                (8, 2, 4100, 40000, 8192)]


@pytest.mark.parametrize("nh,nkv,pos,max_seq,window", WINDOW_CASES)
def test_windowed_attention_decode(dev, nh, nkv, pos, max_seq, window):
    """The fused attention over positions [0, window) only: against the oracle,
    and equal to the full-cache call bit for bit where both merges take the
    same kernel (at most 64 splits); a position at or past the window gives
    NaN heads instead of a shortened attention."""
    hd, eps, base = 128, 1e-6, 1e6
    _say(f"windowed attention nh={nh} nkv={nkv} pos={pos} max_seq={max_seq} window={window}")
    rng = np.random.default_rng(pos + window)
    qkv = (rng.standard_normal((nh + 2 * nkv) * hd) * 2).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    vc0 = rng.standard_normal((nkv, max_seq, hd)).astype(np.float16)
    scale = 1.0 / math.sqrt(hd)
    q, k, v = od.qk_norm_rope(qkv, qn, kn, nh, nkv, hd, eps, base, pos)
    kref, vref = kc0.copy(), vc0.copy()
    od.write_kv(k, v, kref, vref, pos)
    want = od.attend(q, kref, vref, nh, pos, scale)
    bufs = [_vec(dev, a) for a in (qkv, qn, kn, kc0, vc0, np.array([pos, 0, 0, 0], np.int32))]
    d_qkv, d_qn, d_kn, d_kc, d_vc, d_pos = bufs
    d_out = dev.dev_malloc(nh * hd * 4)
    try:
        assert dev.attention_decode_window_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc, d_vc,
                                                   max_seq, window, scale, d_out), dev.last_error()
        got = np.zeros(nh * hd, np.float32)
        dev.dev_download(got, d_out)
        assert rel_l2(got, want) <= 1e-4
        assert dev.attention_decode_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc, d_vc, max_seq,
                                            scale, d_out), dev.last_error()
        full = np.zeros(nh * hd, np.float32)
        dev.dev_download(full, d_out)
        if (max_seq + 63) // 64 <= 64:
            np.testing.assert_array_equal(got.view(np.uint32), full.view(np.uint32))
        else:
            assert rel_l2(got, full) <= 1e-6
        # the window must hold the position
        dev.dev_upload(d_pos, np.array([window, 0, 0, 0], np.int32))
        assert dev.attention_decode_window_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc, d_vc,
                                                   max_seq, window, scale, d_out), dev.last_error()
        past = np.zeros(nh * hd, np.float32)
        dev.dev_download(past, d_out)
        assert np.all(np.isnan(past))
        # windows outside 1..max_seq are refused
        assert not dev.attention_decode_window_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc,
                                                       d_vc, max_seq, max_seq + 1, scale, d_out)
        assert not dev.attention_decode_window_enqueue(d_qkv, d_qn, d_kn, nh, nkv, hd, eps, base, d_pos, d_kc,
                                                       d_vc, max_seq, 0, scale, d_out)
    finally:
        for p in bufs + [d_out]:
            dev.dev_free(p)


def test_windowed_decode_step_graph_matches_the_full_step(dev):
    """A two-layer model at Qwen3-8B dimensions with a 2048-position cache: the
    step at position 100 through the graph captured for its window bucket
    (128) equals the full-cache step bit for bit, replay after replay."""
    import dataclasses
    cfg = dataclasses.replace(zdec.QWEN3_8B, n_layers=2)
    model = zdec.DecodeModel(dev, cfg)
    graph = None
    try:
        x = synth.activation(0x5A4C4D03, cfg.hidden)
        pos = 100
        assert model.window_for(pos) == 128 and model.window_for(127) == 128 and model.window_for(128) == 256
        assert model.window_for(cfg.max_seq - 1) == cfg.max_seq and model.window_for(0) == 128
        full = model.step(x, pos)
        assert np.all(np.isfinite(full))
        windowed = model.step(x, pos, model.window_for(pos))
        np.testing.assert_array_equal(windowed.view(np.uint32), full.view(np.uint32))
        graph = model.capture(model.window_for(pos))
        for _ in range(3):
            model.set_input(x, pos)
            dev.graph_launch(graph, 1)
            np.testing.assert_array_equal(model.logits_host().view(np.uint32), full.view(np.uint32))
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        model.free()
