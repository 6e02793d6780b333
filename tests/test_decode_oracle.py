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
    np.testing.assert_allclose(od.rope_half(od.rope_half(x, 5, 1e6), 7, 1e6), od.rope_half(x, 12, 1e6), atol=1e-9)
    # the frequencies: pair i turns by pos * base^(-2i/hd)
    e = np.zeros(128)
    e[3] = 1.0
    r = od.rope_half(e, 10, 1e4)
    ang = 10 * 1e4 ** (-2 * 3 / 128)
    assert abs(r[3] - math.cos(ang)) < 1e-9 and abs(r[3 + half] - math.sin(ang)) < 1e-9


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
