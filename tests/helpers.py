"""Test helpers: tolerance checks and reference-style fixtures."""
from __future__ import annotations

import numpy as np

from zlm_amd import synth


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


def assert_close_ref(cpu, gpu, abs_tol=1e-4, rel_tol=1e-4):
    """The reference GPU parity check (gpu/root_test.zig:33-50): per element
    |c - g| <= abs_tol + rel_tol*|c|."""
    cpu = np.asarray(cpu, np.float64)
    gpu = np.asarray(gpu, np.float64)
    tol = abs_tol + rel_tol * np.abs(cpu)
    bad = np.abs(cpu - gpu) > tol
    assert not bad.any(), f"{bad.sum()} elements out of tolerance; worst {np.max(np.abs(cpu - gpu) - tol)}"


def ref_x(k: int) -> np.ndarray:
    """The reference GPU tests' activation x[i] = (i % 11)*0.1 - 0.5 (gpu/root_test.zig:62-64)."""
    i = np.arange(k)
    return ((i % 11).astype(np.float32) * np.float32(0.1) - np.float32(0.5)).astype(np.float32)


def fill_weights(qtype: int, rows: int, k: int, seed: int = 0x9E3779B9) -> np.ndarray:
    """The shape of the reference's `fillWeights` (gpu/backend/root.zig:734-786):
    random payload bytes with the f16 scale fields overwritten (q4_0/q8_0 d=0.05,
    q4_1 d=0.05 m=0.02, q4_k d=0.05 dmin=0.02, q6_k d=0.02); the float types get
    the reference's deterministic ramp f32(i % 13) * 0.05 - 0.3 (f16 rounded,
    bf16 truncated).  The random bytes come from this repository's splitmix
    stream, not Zig's PRNG."""
    if qtype in (synth.F32, synth.F16, synth.BF16):
        i = np.arange(rows * k)
        v = (i % 13).astype(np.float32) * np.float32(0.05) - np.float32(0.3)
        if qtype == synth.F32:
            return v.astype(np.float32).view(np.uint8).copy()
        if qtype == synth.F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    be, bb = synth.BLOCK_ELEMS[qtype], synth.BLOCK_BYTES[qtype]
    nblk = rows * (k // be)
    w = synth.random_bytes(seed, 7, nblk * bb).reshape(nblk, bb)
    h05 = np.frombuffer(np.float16(0.05).tobytes(), np.uint8)
    h02 = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
    if qtype in (synth.Q4_0, synth.Q8_0):
        w[:, 0:2] = h05
    elif qtype in (synth.Q4_1, synth.Q4_K):
        w[:, 0:2] = h05
        w[:, 2:4] = h02
    elif qtype == synth.Q6_K:
        w[:, 208:210] = h02
    return w.reshape(-1).copy()
