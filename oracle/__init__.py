"""CPU oracle for the zlm quantized GEMV/GEMM path -- TEST INFRASTRUCTURE ONLY.

A ctypes view of ``liboracle.so`` (built from ``zlm_oracle.c`` by this
directory's Makefile), the C restatement of zlm's CPU kernels.  Only the tests,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this
module; the product (``zlm_amd``) never does.

Each wrapper names the reference routine it restates; the C definitions carry
the file:line citations.  ``lanes`` is the Zig ``simd.native`` width being
emulated (4, 8 or 16).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

DEFAULT_LANES = 8

ERRORS = {
    -1: "TruncatedData",
    -2: "ShapeMismatch",
    -3: "InvalidRange",
    -4: "UnsupportedType",
}


class OracleError(RuntimeError):
    def __init__(self, code: int):
        super().__init__(ERRORS.get(code, f"error {code}"))
        self.code = code
        self.name = ERRORS.get(code, str(code))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle` or __graft_entry__.build()")
        L = ctypes.CDLL(_LIB_PATH)
        P, S, I, U, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32, ctypes.c_float
        L.orc_f16_to_f32.restype = F
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [F]
        L.orc_block_elems.restype = S
        L.orc_block_elems.argtypes = [U]
        L.orc_block_bytes.restype = S
        L.orc_block_bytes.argtypes = [U]
        L.orc_tensor_byte_length.restype = ctypes.c_int64
        L.orc_tensor_byte_length.argtypes = [U, ctypes.c_uint64]
        L.orc_get_scale_min_k4.restype = None
        L.orc_get_scale_min_k4.argtypes = [I, P, P, P]
        L.orc_dequant.restype = I
        L.orc_dequant.argtypes = [U, P, S, P, S]
        for name in ("orc_matvec", "orc_lm_head_rows", "orc_matvec_int"):
            fn = getattr(L, name)
            fn.restype = I
            fn.argtypes = [U, P, S, S, S, P, P, S, S, I]
        L.orc_quantize_act_q8.restype = None
        L.orc_quantize_act_q8.argtypes = [P, S, P, P, P]
        for name in ("orc_matmul_rows", "orc_matmul_int"):
            fn = getattr(L, name)
            fn.restype = I
            fn.argtypes = [U, P, S, S, S, S, P, P, S, S, I]
        L.orc_act_apply.restype = F
        L.orc_act_apply.argtypes = [I, F, F]
        L.orc_gate_up.restype = I
        L.orc_gate_up.argtypes = [U, P, P, S, S, S, P, I, P, S, S, I]
        L.orc_range_of.restype = None
        L.orc_range_of.argtypes = [S, S, S, P, P]
        L.orc_time_matvec.restype = ctypes.c_double
        L.orc_time_matvec.argtypes = [U, P, S, S, S, P, P, I, I, I]
        L.orc_time_matmul_int.restype = ctypes.c_double
        L.orc_time_matmul_int.argtypes = [U, P, S, S, S, S, P, P, I, I, I]
        L.orc_fast_native_lanes.restype = I
        L.orc_fast_native_lanes.argtypes = []
        for name in ("orc_fast_matvec", "orc_fast_matvec_int"):
            fn = getattr(L, name)
            fn.restype = I
            fn.argtypes = [U, P, S, S, S, P, P, S, S, I]
        L.orc_physical_cores.restype = I
        L.orc_physical_cores.argtypes = [P, I]
        L.orc_pool_start.restype = I
        L.orc_pool_start.argtypes = [I]
        L.orc_pool_stop.restype = None
        L.orc_pool_stop.argtypes = []
        L.orc_pool_threads.restype = I
        L.orc_pool_threads.argtypes = []
        L.orc_fast_time_matvec.restype = ctypes.c_double
        L.orc_fast_time_matvec.argtypes = [U, P, S, S, S, P, P, I, I, I]
        L.orc_fast_time_matvec_copies.restype = ctypes.c_double
        L.orc_fast_time_matvec_copies.argtypes = [U, P, I, S, S, S, P, P, I, I, I]
        L.orc_fast_time_matmul_int.restype = ctypes.c_double
        L.orc_fast_time_matmul_int.argtypes = [U, P, S, S, S, S, P, P, I, I, I]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint8).reshape(-1))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(rc)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def block_elems(t: int) -> int:
    return lib().orc_block_elems(t)


def block_bytes(t: int) -> int:
    return lib().orc_block_bytes(t)


def tensor_byte_length(t: int, n: int) -> int:
    """gguf/format.zig:170-174 (-1 for an unsupported type)."""
    return lib().orc_tensor_byte_length(t, n)


def get_scale_min_k4(j: int, scales) -> tuple[int, int]:
    s = _u8(scales)
    d = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().orc_get_scale_min_k4(j, _ptr(s), _ptr(d), _ptr(m))
    return int(d[0]), int(m[0])


def dequant(t: int, data, n: int) -> np.ndarray:
    """quant/root.zig:44-57 dequantTo."""
    d = _u8(data)
    out = np.zeros(n, np.float32)
    _check(lib().orc_dequant(t, _ptr(d), d.size, _ptr(out), n))
    return out


def matvec(t: int, w, k: int, rows: int, x, lanes: int = DEFAULT_LANES, begin: int = 0,
           end: int | None = None) -> np.ndarray:
    """matVecRowsWithPlan(.production) (form/single.zig:168-205)."""
    wb, xf = _u8(w), _f32(x)
    if xf.size != k:
        raise OracleError(-2)
    end = rows if end is None else end
    out = np.zeros(rows, np.float32)
    _check(lib().orc_matvec(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), begin, end, lanes))
    return out


def lm_head_rows(t: int, w, k: int, rows: int, x, lanes: int = DEFAULT_LANES) -> np.ndarray:
    """lmHeadRows (form/single.zig:294-360)."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().orc_lm_head_rows(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), 0, rows, lanes))
    return out


def matvec_int(t: int, w, k: int, rows: int, x, lanes: int = DEFAULT_LANES) -> np.ndarray:
    """The `.int` sweep over q8 activations (form/single.zig:65-73)."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().orc_matvec_int(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), 0, rows, lanes))
    return out


def quantize_act_q8(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """quantizeActivationQ8Sum (matvec/layout.zig:458-476)."""
    xf = _f32(x)
    if xf.size % 32:
        raise ValueError("activation length must be a multiple of 32")
    blocks = xf.size // 32
    qx = np.zeros(xf.size, np.int8)
    dx = np.zeros(blocks, np.float32)
    sums = np.zeros(blocks, np.int32)
    lib().orc_quantize_act_q8(_ptr(xf), blocks, _ptr(qx), _ptr(dx), _ptr(sums))
    return qx, dx, sums


def matmul_rows(t: int, w, k: int, rows: int, m: int, x, lanes: int = DEFAULT_LANES) -> np.ndarray:
    """matMulRows (form/single.zig:213-292): out[t, r], token-major."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(m * rows, np.float32)
    _check(lib().orc_matmul_rows(t, _ptr(wb), wb.size, k, rows, m, _ptr(xf), _ptr(out), 0, rows, lanes))
    return out.reshape(m, rows)


def matmul_int(t: int, w, k: int, rows: int, m: int, x, lanes: int = DEFAULT_LANES) -> np.ndarray:
    """Per-token q8 int sweep (the prefill int oracle), token-major."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(m * rows, np.float32)
    _check(lib().orc_matmul_int(t, _ptr(wb), wb.size, k, rows, m, _ptr(xf), _ptr(out), 0, rows, lanes))
    return out.reshape(m, rows)


def act_apply(act: int, g: float, u: float) -> float:
    """ActivationKind.apply (transformer/activation.zig:4-14); 0 = silu, 1 = gelu_tanh."""
    return lib().orc_act_apply(act, g, u)


def gate_up(t: int, wg, wu, k: int, rows: int, x, act: int, lanes: int = DEFAULT_LANES) -> np.ndarray:
    """fusedGateUpRows generic path (form/fused.zig:27-86)."""
    g, u, xf = _u8(wg), _u8(wu), _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().orc_gate_up(t, _ptr(g), _ptr(u), min(g.size, u.size), k, rows, _ptr(xf), act,
                             _ptr(out), 0, rows, lanes))
    return out


def range_of(total: int, parts: int, idx: int) -> tuple[int, int]:
    """Pool.rangeOf (runtime/pool.zig:52-66)."""
    b = ctypes.c_size_t(0)
    e = ctypes.c_size_t(0)
    lib().orc_range_of(total, parts, idx, ctypes.addressof(b), ctypes.addressof(e))
    return b.value, e.value


def time_matvec(t: int, w, k: int, rows: int, x, threads: int, reps: int,
                lanes: int = DEFAULT_LANES) -> float:
    """Min-of-reps wall seconds of the production sweep over `threads` row ranges."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(rows, np.float32)
    return lib().orc_time_matvec(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), threads, reps, lanes)


def time_matmul_int(t: int, w, k: int, rows: int, m: int, x, threads: int, reps: int,
                    lanes: int = DEFAULT_LANES) -> float:
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(m * rows, np.float32)
    return lib().orc_time_matmul_int(t, _ptr(wb), wb.size, k, rows, m, _ptr(xf), _ptr(out), threads,
                                     reps, lanes)


# ---- the speed-faithful sweep (zlm_cpu_sweep.c / zlm_cpu_pool.c) -------------

def fast_native_lanes() -> int:
    """The width zlm's simd.native picks on this host: 16 (AVX-512), 8 (AVX2) or 0."""
    return int(lib().orc_fast_native_lanes())


def fast_matvec(t: int, w, k: int, rows: int, x, lanes: int = 0, begin: int = 0, end: int = -1) -> np.ndarray:
    """The production sweep at zlm's speed; bit-identical to matvec(..., lanes)."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().orc_fast_matvec(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), begin,
                                 rows if end < 0 else end, lanes))
    return out


def fast_matvec_int(t: int, w, k: int, rows: int, x, lanes: int = 0) -> np.ndarray:
    """The int sweep (q8 activations) at zlm's speed; bit-identical to matvec_int."""
    wb, xf = _u8(w), _f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().orc_fast_matvec_int(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), 0, rows, lanes))
    return out


def physical_cores() -> list[int]:
    """One logical CPU per physical core of this process's affinity mask."""
    buf = (ctypes.c_int * 1024)()
    n = lib().orc_physical_cores(ctypes.addressof(buf), 1024)
    return list(buf[:n])


def fast_time_matvec(t: int, w, k: int, rows: int, x, threads: int, reps: int, lanes: int = 0,
                     out: np.ndarray | None = None) -> float:
    """Min-of-reps wall seconds of one GEMV over the pinned persistent pool
    (the results land in `out` when given)."""
    wb, xf = _u8(w), _f32(x)
    if out is None:
        out = np.zeros(rows, np.float32)
    assert out.dtype == np.float32 and out.size >= rows
    return lib().orc_fast_time_matvec(t, _ptr(wb), wb.size, k, rows, _ptr(xf), _ptr(out), threads, reps, lanes)


def fast_time_matvec_copies(t: int, copies, k: int, rows: int, x, threads: int, reps: int, lanes: int = 0,
                            out: np.ndarray | None = None) -> float:
    """fast_time_matvec with call r reading copies[r % len(copies)] (distinct
    buffers of the same weight, their total past the host's last level cache)."""
    cb = [_u8(c) for c in copies]
    n = min(c.size for c in cb)
    ptrs = (ctypes.c_void_p * len(cb))(*[_ptr(c) for c in cb])
    xf = _f32(x)
    if out is None:
        out = np.zeros(rows, np.float32)
    assert out.dtype == np.float32 and out.size >= rows
    return lib().orc_fast_time_matvec_copies(t, ctypes.addressof(ptrs), len(cb), n, k, rows, _ptr(xf), _ptr(out),
                                             threads, reps, lanes)


def last_level_cache_bytes() -> int:
    """Total last-level cache of the CPUs this process may run on (distinct
    cache instances summed), from sysfs; 0 if unknown."""
    seen, total = set(), 0
    for c in sorted(os.sched_getaffinity(0)):
        base = f"/sys/devices/system/cpu/cpu{c}/cache"
        try:
            idx = sorted(d for d in os.listdir(base) if d.startswith("index"))
        except OSError:
            continue
        best = None
        for d in idx:
            try:
                with open(f"{base}/{d}/level") as f:
                    level = int(f.read())
                with open(f"{base}/{d}/size") as f:
                    size = f.read().strip()
                with open(f"{base}/{d}/shared_cpu_list") as f:
                    shared = f.read().strip()
            except (OSError, ValueError):
                continue
            mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(size[-1:], 1)
            nbytes = int(size.rstrip("KMG")) * mult
            if best is None or level > best[0]:
                best = (level, nbytes, shared)
        if best and best[2] not in seen:
            seen.add(best[2])
            total += best[1]
    return total


def fast_time_matmul_int(t: int, w, k: int, rows: int, m: int, x, threads: int, reps: int,
                         lanes: int = 0, out: np.ndarray | None = None) -> float:
    wb, xf = _u8(w), _f32(x)
    if out is None:
        out = np.zeros(m * rows, np.float32)
    assert out.dtype == np.float32 and out.size >= m * rows
    return lib().orc_fast_time_matmul_int(t, _ptr(wb), wb.size, k, rows, m, _ptr(xf), _ptr(out), threads, reps,
                                          lanes)


def pool_threads() -> int:
    return int(lib().orc_pool_threads())


def pooled_matvec(t: int, w, k: int, rows: int, x, lanes: int = DEFAULT_LANES, threads: int = 16) -> np.ndarray:
    """matvec(t, w, k, rows, x, lanes) computed by the speed-faithful sweep over
    the pinned pool (bit-identical to matvec at the same lanes); for checking
    model-sized GEMVs in seconds."""
    out = np.zeros(rows, np.float32)
    cores = max(1, len(physical_cores()))
    if fast_time_matvec(t, w, k, rows, x, min(threads, cores), 1, lanes=lanes, out=out) < 0:
        raise OracleError(-4)
    return out
