"""The no-allocation decode attention entry point against the allocating one.

zlm_gpu_attention_decode_enqueue_noalloc runs the same kernels as
zlm_gpu_attention_decode_enqueue with the split partials in the library's
fixed static scratch, so its outputs and cache appends must equal the
allocating entry point's bit for bit: two calls in a row (the second on a
smaller shape, so it reuses the array the first left behind), a HIP graph
captured as the first op of a fresh device handle and replayed with other work
between the replays (the library's own scratch stays at zero bytes through the
capture and the replay), and the size limit refused on the host.
"""
import math
import sys

import numpy as np
import pytest

from zlm_amd import device as zd

pytestmark = pytest.mark.gpu

HD, EPS, BASE = 128, 1e-6, 1e6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class _Case:
    """Device buffers of one attention call: q;k;v, norm weights, the position
    and two identical copies of the caches (one per entry point)."""

    def __init__(self, dev, nh, nkv, max_seq, pos, seed):
        rng = np.random.default_rng(seed)
        self.dev, self.nh, self.nkv, self.max_seq = dev, nh, nkv, max_seq
        self.scale = 1.0 / math.sqrt(HD)
        qkv = (rng.standard_normal((nh + 2 * nkv) * HD) * 2).astype(np.float32)
        qn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
        kn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
        self.kc0 = rng.standard_normal((nkv, max_seq, HD)).astype(np.float16)
        self.vc0 = rng.standard_normal((nkv, max_seq, HD)).astype(np.float16)
        self.bufs = []
        self.qkv, self.qn, self.kn = self._vec(qkv), self._vec(qn), self._vec(kn)
        self.pos = self._vec(np.array([pos, 0, 0, 0], np.int32))
        self.kc = [self._vec(self.kc0), self._vec(self.kc0)]
        self.vc = [self._vec(self.vc0), self._vec(self.vc0)]
        self.out = [self._vec(np.zeros(nh * HD, np.float32)), self._vec(np.zeros(nh * HD, np.float32))]

    def _vec(self, a):
        p = self.dev.dev_malloc(max(16, a.nbytes))
        self.dev.dev_upload(p, np.ascontiguousarray(a))
        self.bufs.append(p)
        return p

    def enqueue(self, which, noalloc):
        fn = self.dev.attention_decode_enqueue_noalloc if noalloc else self.dev.attention_decode_enqueue
        return fn(self.qkv, self.qn, self.kn, self.nh, self.nkv, HD, EPS, BASE, self.pos, self.kc[which],
                  self.vc[which], self.max_seq, self.scale, self.out[which])

    def host(self, which):
        out = np.zeros(self.nh * HD, np.float32)
        kc, vc = np.zeros_like(self.kc0), np.zeros_like(self.vc0)
        self.dev.dev_download(out, self.out[which])
        self.dev.dev_download(kc, self.kc[which])
        self.dev.dev_download(vc, self.vc[which])
        return out, kc, vc

    def free(self):
        for p in self.bufs:
            self.dev.dev_free(p)
        self.bufs = []


def _assert_same(a, b):
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x.view(np.uint32 if x.dtype == np.float32 else np.uint16),
                                      y.view(np.uint32 if y.dtype == np.float32 else np.uint16))


def test_noalloc_attention_matches_allocating_entry_point(dev):
    # the second case is smaller than the first (fewer heads, fewer splits)
    for nh, nkv, max_seq, pos in ((32, 8, 2048, 2047), (8, 4, 300, 129)):
        _say(f"no-alloc attention nh={nh} nkv={nkv} max_seq={max_seq} pos={pos}")
        c = _Case(dev, nh, nkv, max_seq, pos, seed=nh + max_seq)
        try:
            assert c.enqueue(0, noalloc=False), dev.last_error()
            assert c.enqueue(1, noalloc=True), dev.last_error()
            want, got = c.host(0), c.host(1)
            assert np.all(np.isfinite(got[0]))
            _assert_same(got, want)
        finally:
            c.free()


def test_noalloc_attention_in_a_graph_captured_before_any_eager_call():
    # a fresh device handle: the capture is its first op, so no library
    # scratch was sized before it, and the no-alloc path must not size any
    dev = zd.Device()
    if not dev.available():
        pytest.fail(f"HIP backend unavailable: {dev.last_error()}")
    nh, nkv, max_seq, pos = 16, 4, 1000, 777
    _say(f"no-alloc attention graph nh={nh} nkv={nkv} max_seq={max_seq} pos={pos}")
    c = _Case(dev, nh, nkv, max_seq, pos, seed=5)
    other = _Case(dev, 32, 8, 2048, 1500, seed=6)
    graph = None
    try:
        assert dev.scratch_device_bytes() == 0
        assert dev.capture_begin(), dev.last_error()
        try:
            ok = c.enqueue(1, noalloc=True)
        finally:
            graph = dev.capture_end()
        assert ok and graph is not None, dev.last_error()
        dev.graph_launch(graph, 1)
        assert dev.scratch_device_bytes() == 0, "the no-alloc path allocated library scratch"
        # the allocating entry point on the same handle sizes its own partials
        # (this graph does not reference them, so that is allowed while it lives)
        assert c.enqueue(0, noalloc=False), dev.last_error()
        assert dev.scratch_device_bytes() > 0
        want = c.host(0)
        for rep in range(3):
            # other work on the same array between the replays
            assert other.enqueue(1, noalloc=True), dev.last_error()
            dev.sync()
            dev.graph_launch(graph, 1)
            _assert_same(c.host(1), want)
    finally:
        if graph is not None:
            dev.graph_destroy(graph)
        c.free()
        other.free()
        dev.deinit()


def test_noalloc_attention_refuses_shapes_beyond_its_array(dev):
    p = dev.dev_malloc(1 << 16)
    try:
        # 32 heads x ceil(40000 / 64) = 20000 head-splits > 16384: refused before any launch
        assert not dev.attention_decode_enqueue_noalloc(p, p, p, 32, 8, HD, EPS, BASE, p, p, p, 40000, 1.0, p)
        assert "at most 16384" in dev.last_error()
        assert not dev.attention_decode_enqueue_noalloc(p, p, p, 32, 8, 64, EPS, BASE, p, p, p, 16, 1.0, p)  # head_dim
    finally:
        dev.dev_free(p)
