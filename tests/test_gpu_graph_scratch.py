"""Library scratch versus captured graphs.

A HIP graph replays with the device addresses it was captured with, so the
library must not free or replace scratch that a live graph references.  On a
fresh device (so these calls size the scratch themselves):

* attention: an eager call sizes the partials, a capture records the same call,
  an eager call that needs more partials is refused while the graph lives, the
  replays still equal the oracle (oracle/decode.py), and after the graph is
  destroyed the larger call runs and matches the oracle;
* matMul (the prefill GEMM): the same with the activation scratch and a
  resident's GEMM tiles, replays checked against the eager result and the
  oracle's int path (oracle.matmul_int);
* the host-buffer contract ops refuse to run under capture.
"""
import math
import sys

import numpy as np
import pytest

import oracle
from oracle import decode as od
from tests.helpers import rel_l2
from zlm_amd import device as zd
from zlm_amd import synth

pytestmark = pytest.mark.gpu

HD, EPS, BASE = 128, 1e-6, 1e6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture()
def fresh():
    d = zd.Device()
    if not d.available():
        pytest.fail(f"HIP backend unavailable: {d.last_error()}")
    yield d
    d.deinit()


class _Attn:
    def __init__(self, dev, nh, nkv, max_seq, pos, seed):
        rng = np.random.default_rng(seed)
        self.dev, self.nh, self.nkv, self.max_seq, self.pos_v = dev, nh, nkv, max_seq, pos
        self.scale = 1.0 / math.sqrt(HD)
        self.qkv_h = (rng.standard_normal((nh + 2 * nkv) * HD) * 2).astype(np.float32)
        self.qn_h = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
        self.kn_h = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
        self.kc0 = rng.standard_normal((nkv, max_seq, HD)).astype(np.float16)
        self.vc0 = rng.standard_normal((nkv, max_seq, HD)).astype(np.float16)
        self.bufs = []
        self.qkv, self.qn, self.kn = self._vec(self.qkv_h), self._vec(self.qn_h), self._vec(self.kn_h)
        self.pos = self._vec(np.array([pos, 0, 0, 0], np.int32))
        self.kc, self.vc = self._vec(self.kc0), self._vec(self.vc0)
        self.out = self._vec(np.zeros(nh * HD, np.float32))

    def _vec(self, a):
        p = self.dev.dev_malloc(max(16, a.nbytes))
        self.dev.dev_upload(p, np.ascontiguousarray(a))
        self.bufs.append(p)
        return p

    def enqueue(self):
        return self.dev.attention_decode_enqueue(self.qkv, self.qn, self.kn, self.nh, self.nkv, HD, EPS, BASE,
                                                 self.pos, self.kc, self.vc, self.max_seq, self.scale, self.out)

    def want(self):
        q, k, v = od.qk_norm_rope(self.qkv_h, self.qn_h, self.kn_h, self.nh, self.nkv, HD, EPS, BASE, self.pos_v)
        kref, vref = self.kc0.copy(), self.vc0.copy()
        od.write_kv(k, v, kref, vref, self.pos_v)
        return od.attend(q, kref, vref, self.nh, self.pos_v, self.scale)

    def got(self):
        out = np.zeros(self.nh * HD, np.float32)
        self.dev.dev_download(out, self.out)
        return out

    def free(self):
        for p in self.bufs:
            self.dev.dev_free(p)


def test_attention_scratch_outlives_its_graph(fresh):
    dev = fresh
    small = _Attn(dev, 32, 8, 2048, 1000, seed=1)
    big = _Attn(dev, 32, 8, 8192, 6000, seed=2)  # 128 splits per head against 32
    graph = None
    try:
        _say("graph scratch: eager attention sizes the partials")
        assert small.enqueue(), dev.last_error()
        grown = dev.scratch_device_bytes()
        assert grown >= 32 * 32 * 130 * 4
        assert dev.capture_begin(), dev.last_error()
        try:
            ok = small.enqueue()
        finally:
            graph = dev.capture_end()
        assert ok and graph is not None, dev.last_error()
        _say("graph scratch: a larger eager call is refused while the graph lives")
        assert not big.enqueue()
        assert "captured graph" in dev.last_error(), dev.last_error()
        assert dev.scratch_device_bytes() == grown
        want = small.want()
        for rep in range(3):
            dev.dev_upload(small.out, np.zeros(32 * HD, np.float32))
            dev.graph_launch(graph, 1)
            assert rel_l2(small.got(), want) <= 1e-4, rep
        dev.graph_destroy(graph)
        graph = None
        _say("graph scratch: after the graph is destroyed the larger call runs")
        assert big.enqueue(), dev.last_error()
        assert rel_l2(big.got(), big.want()) <= 1e-4
        assert dev.scratch_device_bytes() > grown
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        small.free()
        big.free()


def test_gemm_scratch_outlives_its_graph(fresh):
    dev = fresh
    rows, k = 256, 1024
    q = zd.quant(zd.Q4_0)
    w = synth.weights(synth.Q4_0, rows, k, seed=31)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    m_small, m_big = 64, 256
    x_small = np.random.default_rng(3).standard_normal(m_small * k).astype(np.float32)
    x_big = np.random.default_rng(4).standard_normal(m_big * k).astype(np.float32)
    d_xs, d_xb = dev.dev_malloc(x_small.nbytes), dev.dev_malloc(x_big.nbytes)
    d_os, d_ob = dev.dev_malloc(m_small * rows * 4), dev.dev_malloc(m_big * rows * 4)
    dev.dev_upload(d_xs, x_small)
    dev.dev_upload(d_xb, x_big)
    graph = None
    try:
        _say("graph scratch: eager matMul builds the tiles and the activation scratch")
        assert dev.mat_mul_enqueue(res, q, rows, k, m_small, d_xs, d_os), dev.last_error()
        eager = np.zeros(m_small * rows, np.float32)
        dev.dev_download(eager, d_os)
        want = oracle.matmul_int(synth.Q4_0, w, k, rows, m_small, x_small)
        assert rel_l2(eager.reshape(m_small, rows), want) <= 1e-5
        assert dev.capture_begin(), dev.last_error()
        try:
            ok = dev.mat_mul_enqueue(res, q, rows, k, m_small, d_xs, d_os)
        finally:
            graph = dev.capture_end()
        assert ok and graph is not None, dev.last_error()
        _say("graph scratch: larger matMul, tile rebuild and tile release are refused while the graph lives")
        assert not dev.mat_mul_enqueue(res, q, rows, k, m_big, d_xb, d_ob)
        assert "captured graph" in dev.last_error(), dev.last_error()
        assert not dev.release_gemm_tiles(res)
        assert not dev.mat_mul_enqueue(res, q, rows, k // 2, m_small, d_xs, d_os)  # another k: new tiles
        for rep in range(3):
            dev.dev_upload(d_os, np.zeros(m_small * rows, np.float32))
            dev.graph_launch(graph, 1)
            got = np.zeros(m_small * rows, np.float32)
            dev.dev_download(got, d_os)
            np.testing.assert_array_equal(got.view(np.uint32), eager.view(np.uint32))
        dev.graph_destroy(graph)
        graph = None
        _say("graph scratch: after the graph is destroyed the larger matMul runs")
        assert dev.mat_mul_enqueue(res, q, rows, k, m_big, d_xb, d_ob), dev.last_error()
        got = np.zeros(m_big * rows, np.float32)
        dev.dev_download(got, d_ob)
        assert rel_l2(got.reshape(m_big, rows), oracle.matmul_int(synth.Q4_0, w, k, rows, m_big, x_big)) <= 1e-5
        assert dev.release_gemm_tiles(res), dev.last_error()
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        for p in (d_xs, d_xb, d_os, d_ob):
            dev.dev_free(p)
        dev.free_resident(res)


def test_host_buffer_ops_refuse_capture(fresh):
    dev = fresh
    rows, k = 64, 256
    w = synth.weights(synth.Q4_0, rows, k, seed=9)
    x = synth.activation(9, k)
    res = dev.upload_resident(w)
    assert res is not None, dev.last_error()
    out = np.zeros(rows, np.float32)
    q = zd.quant(zd.Q4_0)
    assert dev.mat_vec_resident(res, q, rows, k, x, out), dev.last_error()
    graph = None
    assert dev.capture_begin(), dev.last_error()
    try:
        assert not dev.mat_vec_resident(res, q, rows, k, x, out)
        assert "capture" in dev.last_error()
        assert dev.mat_vec_resident_burst_async(res, q, rows, k, x, True) is None
        assert dev.upload_resident(w) is None
    finally:
        graph = dev.capture_end()
    if graph is not None:
        dev.graph_destroy(graph)
    # the device works normally afterwards
    assert dev.mat_vec_resident(res, q, rows, k, x, out), dev.last_error()
    assert rel_l2(out, oracle.matvec(synth.Q4_0, w, k, rows, x)) <= 1e-3
    dev.free_resident(res)
