"""GPU parity at the benchmark configurations' full dimensions.

* The lm_head GEMVs (reference lmHeadRows,
  src/kernels/linear/matvec/form/single.zig:294-360) at their real sizes:
  configs[2]'s Q8_0 151936 x 4096 and configs[3]'s Q6_K 262144 x 3840, the
  plain contract op (host x in, host logits out) and the RMSNorm-fused device
  form the decode step uses, against the oracle's lmHeadRows restatement
  (relative L2 <= 1e-3).  These shapes take the tall instances the host picks
  from 65536 rows; a ragged 65573-row Q8_0 case covers the last partial tile.
* The configs[2] decode step at Qwen3-8B dimensions (hidden 4096, 32 q / 8 kv
  heads of 128, FFN 12288, vocab 151936, Q4_0 projections, Q8_0 lm_head, fp16
  KV of 2048), two layers, caches holding a 2047-token history: the step at
  position 2047 (attention over all 2048 positions) eager, then a replay of
  the captured graph at position 1500, each against the oracle's layer
  sequence (oracle/decode.py decode_step over the same weights and caches).
  Logits relative L2 <= 1e-3.  This reaches every kernel the 36-layer
  benchmark step runs: the 16-wave normed gate_up, the split-K residual down
  at k = 12288, the two-row o projection and the tall normed lm_head.
"""
import sys

import numpy as np
import pytest

import oracle
from oracle import decode as od
from tests.helpers import rel_l2
from zlm_amd import decode as zdec
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dev_vec(dev, a):
    a = np.ascontiguousarray(a)
    p = dev.dev_malloc(max(16, a.nbytes))
    dev.dev_upload(p, a)
    return p


LM_HEADS = [
    ("c2_lm_head_q8_0", synth.Q8_0, 151936, 4096),
    ("c3_lm_head_q6_k", synth.Q6_K, 262144, 3840),
    ("tall_ragged_q8_0", synth.Q8_0, 65536 + 37, 4096),
]


@pytest.mark.parametrize("name,qt,rows,k", LM_HEADS, ids=[c[0] for c in LM_HEADS])
def test_lm_head_full_size_matches_oracle(dev, name, qt, rows, k):
    _say(f"lm_head {name} {rows}x{k}: synthesising")
    eps = 1e-6
    w = synth.weights(qt, rows, k, seed=0x5A4C4D40 + rows)
    x = synth.activation(0x5A4C4D0A, k)
    nw = (1.0 + 0.1 * synth.activation(0x5A4C4D0B, k)).astype(np.float32)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    try:
        _say(f"lm_head {name}: plain contract op")
        want = oracle.lm_head_rows(qt, w, k, rows, x)
        out = np.full(rows, np.nan, np.float32)
        assert dev.mat_vec_resident(res, zd.quant(qt), rows, k, x, out), dev.last_error()
        assert np.all(np.isfinite(out))
        err = rel_l2(out, want)
        assert err <= REL_L2, f"plain rel-L2 {err:.3e}"
        _say(f"lm_head {name}: RMSNorm-fused form (plain rel-L2 {err:.2e})")
        xn = od.rms_norm(x, nw, eps)
        want_n = oracle.lm_head_rows(qt, w, k, rows, xn)
        xd, nwd, yd = _dev_vec(dev, x), _dev_vec(dev, nw), dev.dev_malloc(rows * 4)
        try:
            assert dev.gemv_op_enqueue(zd.FORM_NORM, zd.quant(qt), res, rows, k, xd, yd, norm_w=nwd, eps=eps), \
                dev.last_error()
            got = np.full(rows, np.nan, np.float32)
            dev.dev_download(got, yd)
            err_n = rel_l2(got, want_n)
            assert err_n <= REL_L2, f"norm form rel-L2 {err_n:.3e}"
        finally:
            for p in (xd, nwd, yd):
                dev.dev_free(p)
    finally:
        dev.free_resident(res)


# configs[2] dimensions with two layers (the per-layer kernels are the same in
# every layer; two layers also check that layer i+1 reads layer i's output).
QWEN3_8B_2L = zdec.DecodeConfig(n_layers=2, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288,
                                vocab=151936, max_seq=2048)


def _host_model(cfg, seed=0x5A4C4D52):
    rng = np.random.default_rng(seed)
    shape = (cfg.n_kv_heads, cfg.max_seq, cfg.head_dim)
    layers = []
    for i in range(cfg.n_layers):
        s = seed + 100 * i
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
            # a 2047-token history (row 2047 is written by the step at that position)
            "k_cache": rng.standard_normal(shape).astype(np.float16),
            "v_cache": rng.standard_normal(shape).astype(np.float16),
        })
    return {"layers": layers, "lm_head": synth.weights(synth.Q8_0, cfg.vocab, cfg.hidden, seed + 99),
            "out_norm": (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)}


def test_qwen3_8b_dims_decode_matches_oracle(dev):
    cfg = QWEN3_8B_2L
    _say("qwen3-8b dims decode: synthesising 2 layers + lm_head on the host")
    host = _host_model(cfg)
    kref = [L["k_cache"].copy() for L in host["layers"]]
    vref = [L["v_cache"].copy() for L in host["layers"]]
    model = zdec.DecodeModel(dev, cfg, host=host)
    graph = None
    try:
        for step, pos in enumerate([cfg.max_seq - 1, 1500]):
            x = synth.activation(0x5A4C4D60 + pos, cfg.hidden)
            _say(f"qwen3-8b dims decode: oracle step at pos {pos}")
            want = od.decode_step(cfg, host["layers"], host["out_norm"], host["lm_head"], synth.Q8_0, synth.Q4_0, x,
                                  pos, kref, vref)
            if step == 0:
                _say("qwen3-8b dims decode: eager GPU step")
                got = model.step(x, pos)
            else:
                _say("qwen3-8b dims decode: captured graph replay")
                graph = model.capture()
                model.set_input(x, pos)
                dev.graph_launch(graph, 1)
                got = model.logits_host()
            assert np.all(np.isfinite(got))
            err = rel_l2(got, want)
            _say(f"qwen3-8b dims decode pos {pos}: logits rel-L2 {err:.2e}")
            assert err <= REL_L2, (pos, err)
        # the K/V rows both steps appended (layer 0: its k is normed and rotated, v as projected)
        kc = np.zeros_like(kref[0])
        vc = np.zeros_like(vref[0])
        dev.dev_download(kc, model.layers[0].k_cache)
        dev.dev_download(vc, model.layers[0].v_cache)
        for pos in (cfg.max_seq - 1, 1500):
            assert rel_l2(vc[:, pos].astype(np.float32), vref[0][:, pos].astype(np.float32)) <= 2e-3
            assert rel_l2(kc[:, pos].astype(np.float32), kref[0][:, pos].astype(np.float32)) <= 2e-3
        untouched = np.ones(cfg.max_seq, bool)
        untouched[[1500, cfg.max_seq - 1]] = False
        np.testing.assert_array_equal(kc[:, untouched], host["layers"][0]["k_cache"][:, untouched])
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        model.free()
