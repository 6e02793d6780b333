"""Every launch of a decode step, and of the prefill GEMM and the long-cache
attention, within what a kernel-dispatch (AQL) packet can carry.

The library checks each launch on the host before it reaches the queue
(workgroup of 64..1024 work-items in whole waves; grid x workgroup below 2^32
work-items in x; at most 65536 workgroups in y and z; static LDS <= 160 KiB)
and fails with the parameters otherwise.  Here the launch log records every
launch of: one eager decode step of the small Qwen3-shaped model and of a
two-layer model at Qwen3-8B dimensions (the same launches, per layer, as the
36-layer configs[2] step; the reference's decode loop is
runtime/executor.zig:45-86), the same step while it is captured into a graph,
the configs[4] prefill GEMM with its small-M and GEMV routes, and the attention
at a 40000-position cache (the wide merge).  Each record must sit within the
limits, and the step's launch count must be 1 + 6 layers + 1.
"""
import dataclasses
import math
import sys

import numpy as np
import pytest

from zlm_amd import decode as zdec
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(records):
    assert records
    for r in records:
        assert 64 <= r["block"] <= 1024 and r["block"] % 64 == 0, r
        assert r["grid_x"] >= 1 and r["grid_y"] >= 1 and r["grid_z"] >= 1, r
        assert r["grid_x"] * r["block"] < 2 ** 32, r
        assert r["grid_y"] <= 65536 and r["grid_z"] <= 65536, r
        assert r["lds_bytes"] <= 160 * 1024, r


@pytest.mark.parametrize("cfg", [
    zdec.DecodeConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768, vocab=1000,
                      max_seq=80),
    dataclasses.replace(zdec.QWEN3_8B, n_layers=2),
], ids=["tiny", "qwen3_8b_dims_2_layers"])
def test_decode_step_launches_within_dispatch_limits(dev, cfg):
    _say(f"launch limits: decode {cfg.n_layers} layers hidden {cfg.hidden}")
    model = zdec.DecodeModel(dev, cfg)
    graph = None
    try:
        x = synth.activation(3, cfg.hidden)
        model.step(x, 0)  # first step converts layouts and sizes scratch
        assert dev.launch_log(True)
        model.step(x, cfg.max_seq - 1)
        eager = dev.launch_log_read()
        _check(eager)
        assert len(eager) == 1 + 6 * cfg.n_layers + 1, [r["what"] for r in eager]
        # the same launches recorded into a graph
        assert dev.launch_log(True)
        graph = model.capture()
        captured = dev.launch_log_read()
        assert [(r["what"], r["grid_x"], r["grid_y"], r["block"]) for r in captured] == \
            [(r["what"], r["grid_x"], r["grid_y"], r["block"]) for r in eager]
    finally:
        dev.launch_log(False)
        if graph is not None:
            dev.graph_destroy(graph)
        model.free()


def test_gemm_and_long_attention_launches_within_dispatch_limits(dev):
    rows, k = 12288, 4096
    res = dev.synth_resident(zd.Q4_0, rows * k // 32, 5, 0.02)
    assert res is not None, dev.last_error()
    x = dev.dev_malloc(512 * k * 4)
    out = dev.dev_malloc(512 * rows * 4)
    dev.dev_upload(x, synth.activation(4, 512 * k))
    try:
        assert dev.launch_log(True)
        for m in (1, 2, 3, 5, 32, 33, 512):
            _say(f"launch limits: matMul m={m}")
            assert dev.mat_mul_enqueue(res, zd.quant(zd.Q4_0), rows, k, m, x, out), dev.last_error()
        dev.sync()
        _check(dev.launch_log_read())
    finally:
        dev.launch_log(False)
        dev.dev_free(x)
        dev.dev_free(out)
        dev.free_resident(res)
    nh, nkv, hd, max_seq = 32, 8, 128, 40000
    q = dev.dev_malloc((nh + 2 * nkv) * hd * 4)
    kc = dev.dev_malloc(nkv * max_seq * hd * 2)
    vc = dev.dev_malloc(nkv * max_seq * hd * 2)
    nw = dev.dev_malloc(hd * 4)
    pos = dev.dev_malloc(16)
    o = dev.dev_malloc(nh * hd * 4)
    try:
        dev.dev_upload(q, np.ones((nh + 2 * nkv) * hd, np.float32))
        dev.dev_upload(nw, np.ones(hd, np.float32))
        dev.dev_upload(pos, np.array([max_seq - 1, 0, 0, 0], np.int32))
        dev.dev_upload(kc, np.zeros(nkv * max_seq * hd, np.float16))
        dev.dev_upload(vc, np.zeros(nkv * max_seq * hd, np.float16))
        assert dev.launch_log(True)
        _say("launch limits: attention at 40000 positions")
        assert dev.attention_decode_enqueue(q, nw, nw, nh, nkv, hd, 1e-6, 1e6, pos, kc, vc, max_seq,
                                            1.0 / math.sqrt(hd), o), dev.last_error()
        dev.sync()
        recs = dev.launch_log_read()
        _check(recs)
        assert [r["what"] for r in recs] == ["attention decode", "attention combine wide"]
    finally:
        dev.launch_log(False)
        for p in (q, kc, vc, nw, pos, o):
            dev.dev_free(p)
