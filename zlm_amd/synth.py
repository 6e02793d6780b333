"""Seeded synthetic GGUF weights and activations for the benchmark configs.

A counter-based splitmix64 stream: value ``i`` of stream ``s`` under seed
``seed`` is ``mix(base(seed, s) + (i + 1) * GAMMA)``, so any slice of a stream
can be produced independently (and on the GPU, if ever needed).  Normals are
Box-Muller over two uniforms.  Each tensor draws its scales, its quant bytes and
the activation from separate streams.

Distributions follow the benchmark configurations:
  * Q4_0: per 32-block ``d = f16(|N(0,1)| * 0.02)``, 16 uniform bytes (nibbles
    uniform on 0..15), value ``(q - 8) * d``.
  * Q8_0: ``d = f16(|N(0,1)| * 0.01)``, int8 quants uniform on [-127, 127].
  * Q4_K: ``d``, ``dmin`` = ``f16(|N(0,1)| * 0.02)``; 12 scale bytes and 128
    quant bytes uniform.
  * Q6_K: ``ql``, ``qh`` and ``sc`` uniform bytes, ``d = f16(|N(0,1)| * 0.02)``.
  * F32 / F16 / BF16: elements ``N(0,1) * 0.02`` rounded to the type
    (round-to-nearest-even).
  * activations: fp32 N(0, 1).

The raw byte layout is GGUF's (block formats as in the reference's
``src/kernels/linear/quant/types.zig:6-53`` and ``gguf/format.zig:135-159``).
"""
from __future__ import annotations

import os

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_STREAM = np.uint64(0xD1B54A32D192ED03)

# GGML type codes (reference gguf/format.zig:41-77).
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
BLOCK_ELEMS = {Q4_0: 32, Q4_1: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256, F32: 1, F16: 1, BF16: 1}
BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q4_K: 144, Q6_K: 210, F32: 4, F16: 2, BF16: 2}
TYPE_NAMES = {Q4_0: "q4_0", Q4_1: "q4_1", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", F32: "f32", F16: "f16",
              BF16: "bf16"}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _base(seed: int, stream: int) -> np.uint64:
    s = np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    with np.errstate(over="ignore"):
        b = _mix(s + GAMMA)[0] ^ (np.uint64(stream) * _STREAM)
    return np.uint64(b)


def u64(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """``n`` uint64 values of stream ``stream`` starting at counter ``offset``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(_base(seed, stream) + i * GAMMA)


def random_bytes(seed: int, stream: int, n: int) -> np.ndarray:
    words = u64(seed, stream, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def uniform01(seed: int, stream: int, n: int) -> np.ndarray:
    """float64 uniforms on [0, 1)."""
    return (u64(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    """float64 N(0, 1) by Box-Muller over counters (2i, 2i+1)."""
    w = u64(seed, stream, 2 * n)
    a = (w[0::2] >> np.uint64(11)).astype(np.float64)
    b = (w[1::2] >> np.uint64(11)).astype(np.float64)
    u1 = (a + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
    u2 = b * (1.0 / 9007199254740992.0)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def activation(seed: int, n: int, stream: int = 9) -> np.ndarray:
    """fp32 N(0, 1) activation of length ``n``."""
    return normal(seed, stream, n).astype(np.float32)


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def _bf16_bytes(v: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(v.astype(np.float32)).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return r.view(np.uint8).reshape(-1, 2)


def _bytes_at(seed: int, stream: int, byte0: int, n: int) -> np.ndarray:
    """Bytes [byte0, byte0 + n) of stream ``stream`` (what ``random_bytes``
    returns for the whole stream, sliced)."""
    w0 = byte0 // 8
    words = u64(seed, stream, (byte0 + n + 7) // 8 - w0, offset=w0)
    lo = byte0 - 8 * w0
    return words.view(np.uint8)[lo:lo + n]


def _normal_at(seed: int, stream: int, i0: int, n: int) -> np.ndarray:
    """Values [i0, i0 + n) of ``normal(seed, stream, ...)``."""
    w = u64(seed, stream, 2 * n, offset=2 * i0)
    a = (w[0::2] >> np.uint64(11)).astype(np.float64)
    b = (w[1::2] >> np.uint64(11)).astype(np.float64)
    u1 = (a + 1.0) * (1.0 / 9007199254740992.0)
    u2 = b * (1.0 / 9007199254740992.0)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def _fill_blocks(out: np.ndarray, qtype: int, seed: int, b0: int) -> None:
    """Blocks [b0, b0 + len(out)) of a weight stream into ``out`` (n x block bytes)."""
    n = out.shape[0]
    if qtype == Q4_0:
        out[:, 0:2] = _f16_bytes(np.abs(_normal_at(seed, 1, b0, n)) * 0.02)
        out[:, 2:18] = _bytes_at(seed, 2, 16 * b0, 16 * n).reshape(n, 16)
    elif qtype == Q8_0:
        out[:, 0:2] = _f16_bytes(np.abs(_normal_at(seed, 1, b0, n)) * 0.01)
        r = _bytes_at(seed, 2, 64 * b0, 64 * n).view(np.uint16).astype(np.uint32)
        q = ((r * 255) >> 16).astype(np.int32) - 127
        out[:, 2:34] = q.astype(np.int8).view(np.uint8).reshape(n, 32)
    elif qtype == Q4_1:
        out[:, 0:2] = _f16_bytes(np.abs(_normal_at(seed, 1, b0, n)) * 0.02)
        out[:, 2:4] = _f16_bytes(-np.abs(_normal_at(seed, 3, b0, n)) * 0.1)
        out[:, 4:20] = _bytes_at(seed, 2, 16 * b0, 16 * n).reshape(n, 16)
    elif qtype == Q4_K:
        out[:, 0:2] = _f16_bytes(np.abs(_normal_at(seed, 1, b0, n)) * 0.02)
        out[:, 2:4] = _f16_bytes(np.abs(_normal_at(seed, 3, b0, n)) * 0.02)
        out[:, 4:144] = _bytes_at(seed, 2, 140 * b0, 140 * n).reshape(n, 140)
    elif qtype == Q6_K:
        out[:, 0:208] = _bytes_at(seed, 2, 208 * b0, 208 * n).reshape(n, 208)
        out[:, 208:210] = _f16_bytes(np.abs(_normal_at(seed, 1, b0, n)) * 0.02)
    elif qtype == F32:
        out[:] = np.ascontiguousarray((_normal_at(seed, 1, b0, n) * 0.02).astype(np.float32)).view(
            np.uint8).reshape(n, 4)
    elif qtype == F16:
        out[:] = _f16_bytes(_normal_at(seed, 1, b0, n) * 0.02)
    elif qtype == BF16:
        out[:] = _bf16_bytes(_normal_at(seed, 1, b0, n) * 0.02)
    else:
        raise ValueError(f"unsupported type {qtype}")


_CHUNK_BYTES = 16 << 20


def weights(qtype: int, rows: int, k: int, seed: int) -> np.ndarray:
    """Raw GGUF bytes of a ``rows x k`` weight (row-major blocks), uint8.
    Large tensors are generated in chunks on a few threads (numpy releases
    the GIL); the bytes do not depend on the chunking."""
    if qtype not in BLOCK_ELEMS:
        raise ValueError(f"unsupported type {qtype}")
    be, bb = BLOCK_ELEMS[qtype], BLOCK_BYTES[qtype]
    if k % be:
        raise ValueError(f"k={k} is not a multiple of the {TYPE_NAMES[qtype]} block ({be})")
    nblk = rows * (k // be)
    out = np.empty((nblk, bb), dtype=np.uint8)
    per = max(1, _CHUNK_BYTES // bb)
    starts = list(range(0, nblk, per))
    if len(starts) <= 1:
        _fill_blocks(out, qtype, seed, 0)
    else:
        from concurrent.futures import ThreadPoolExecutor

        workers = max(1, min(8, len(os.sched_getaffinity(0)), len(starts)))
        with ThreadPoolExecutor(workers) as pool:
            list(pool.map(lambda b0: _fill_blocks(out[b0:b0 + per], qtype, seed, b0), starts))
    return out.reshape(-1)


def row_bytes(qtype: int, k: int) -> int:
    return (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]


def weight_bytes(qtype: int, rows: int, k: int) -> int:
    return rows * row_bytes(qtype, k)
