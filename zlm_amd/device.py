"""Python mirror of zlm's GPU ``Device`` over the HIP backend's C ABI.

The method names are the reference contract's ops in snake_case
(reference ``src/gpu/backend/root.zig:299-311``), with the same argument
meaning and the same failure convention: an op that did not run on the device
returns ``False`` (or ``None`` for a handle/resident) and the caller runs the
CPU kernel.  ``Device()`` never raises for a missing GPU; it is then inert
(``available() is False``).  A missing *library*, however, is an installation
error and raises immediately.

Buffers are numpy arrays: weights ``uint8`` (raw GGUF blocks), activations and
outputs ``float32``, all C-contiguous.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libzlm_gpu_hip.so")
CODE_OBJECT_PATH = os.path.join(LIB_DIR, "zlm_kernels_gfx950.hsaco")
# Every code object the library loads: the common kernels and one GEMV object per quant.
CODE_OBJECT_PATHS = [CODE_OBJECT_PATH] + [os.path.join(LIB_DIR, f"zlm_gemv_{q}_gfx950.hsaco")
                                          for q in ("q4_0", "q8_0", "q4_k", "q6_k", "q4_1", "f32", "f16", "bf16")]

RING_SIZE = 8
NULL_HANDLE = -1

# GGML type codes (reference gguf/format.zig:41-77).
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 30
# GpuVariant codes (reference gpu/kernels/grid.zig:14).
PLAIN, U4, U8, SUB, UN2, UN4, W32, W128 = range(8)
VARIANT_NAMES = ("plain", "u4", "u8", "sub", "un2", "un4", "w32", "w128")
# GateUpAct (reference gpu/backend/root.zig:225).
SILU, GELU = 0, 1
# GEMV forms of zlm_gemv_op (device-level; see include/zlm_gpu_hip.h).
FORM_PLAIN, FORM_PAIR, FORM_NORM, FORM_NORMPAIR, FORM_RESID = range(5)


def layout_bytes(quant_code: int, rows: int, k: int, with_gemm: bool) -> int:
    """HBM of a rows x k weight once converted (+ its GEMM tiled copy); no GPU needed."""
    return int(lib().zlm_gpu_layout_bytes(quant_code, rows, k, with_gemm))


def quant(ggml_type: int, variant: int = PLAIN) -> int:
    """The C ABI's quant code: GGML type in bits 0..7, GpuVariant in 8..15."""
    return (ggml_type & 0xFF) | ((variant & 0xFF) << 8)


class _ResidentOp(ctypes.Structure):
    _fields_ = [
        ("res", ctypes.c_void_p),
        ("quant", ctypes.c_uint32),
        ("rows", ctypes.c_size_t),
        ("out", ctypes.c_void_p),
        ("out_len", ctypes.c_size_t),
    ]


class _GemvDesc(ctypes.Structure):
    _fields_ = [
        ("res", ctypes.c_void_p),
        ("quant", ctypes.c_uint32),
        ("rows", ctypes.c_size_t),
        ("k", ctypes.c_size_t),
        ("x_dev", ctypes.c_void_p),
        ("y_dev", ctypes.c_void_p),
        ("with_next", ctypes.c_uint32),
    ]


class _GemvOp(ctypes.Structure):
    _fields_ = [
        ("form", ctypes.c_uint32),
        ("quant", ctypes.c_uint32),
        ("w", ctypes.c_void_p),
        ("w_up", ctypes.c_void_p),
        ("rows", ctypes.c_size_t),
        ("k", ctypes.c_size_t),
        ("x", ctypes.c_void_p),
        ("norm_w", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("act", ctypes.c_uint32),
        ("res", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
    ]


class LaunchRecord(ctypes.Structure):
    """zlm_launch_record: one logged kernel launch."""
    _fields_ = [("what", ctypes.c_char_p), ("grid_x", ctypes.c_uint32), ("grid_y", ctypes.c_uint32),
                ("grid_z", ctypes.c_uint32), ("block", ctypes.c_uint32), ("lds_bytes", ctypes.c_uint32)]


class _Probe(ctypes.Structure):
    _fields_ = [
        ("gemv_gbps", ctypes.c_double),
        ("gemv_streamed_gbps", ctypes.c_double),
        ("matmul_gbps", ctypes.c_double),
        ("q4_0_variant", ctypes.c_uint8),
        ("q4_1_variant", ctypes.c_uint8),
        ("q8_0_variant", ctypes.c_uint8),
        ("q6_k_variant", ctypes.c_uint8),
        ("q4_k_variant", ctypes.c_uint8),
        ("f32_variant", ctypes.c_uint8),
        ("f16_variant", ctypes.c_uint8),
        ("bf16_variant", ctypes.c_uint8),
        ("gate_up_variant", ctypes.c_uint8),
        ("gate_up_q4_1_variant", ctypes.c_uint8),
        ("gate_up_q8_0_variant", ctypes.c_uint8),
        ("q4_0_u4_gbps", ctypes.c_double),
        ("q4_0_sub_gbps", ctypes.c_double),
        ("q4_0_un2_gbps", ctypes.c_double),
        ("q4_0_un4_gbps", ctypes.c_double),
        ("q4_0_w32_gbps", ctypes.c_double),
        ("q4_0_w128_gbps", ctypes.c_double),
        ("q4_k_gbps", ctypes.c_double),
        ("q4_k_u4_gbps", ctypes.c_double),
        ("gate_up_gbps", ctypes.c_double),
        ("gate_up_u4_gbps", ctypes.c_double),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded C-ABI library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"HIP backend library missing: {LIB_PATH} (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, S, B, U, I32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_bool, ctypes.c_uint32, ctypes.c_int32
    sig = {
        "zlm_gpu_init": (P, []),
        "zlm_gpu_deinit": (None, [P]),
        "zlm_gpu_available": (B, [P]),
        "zlm_gpu_backend_name": (ctypes.c_char_p, [P]),
        "zlm_gpu_device_name": (ctypes.c_char_p, [P]),
        "zlm_gpu_is_uma": (B, [P]),
        "zlm_gpu_mat_vec": (B, [P, U, P, S, S, S, P, S, P, S]),
        "zlm_gpu_mat_mul_batch": (B, [P, U, P, S, S, S, S, P, S, P, S]),
        "zlm_gpu_mat_mul_resident": (B, [P, P, U, S, S, S, P, S, P, S]),
        "zlm_gpu_mat_vec_resident": (B, [P, P, U, S, S, P, S, P, S]),
        "zlm_gpu_mat_vec_resident_async": (I32, [P, P, U, S, S, P, S]),
        "zlm_gpu_mat_vec_resident_burst_async": (I32, [P, P, U, S, S, P, S, B]),
        "zlm_gpu_mat_vec_gate_up_resident_burst_async": (I32, [P, P, P, U, S, S, P, S, U, U, B]),
        "zlm_gpu_mat_vec_mlp_resident_burst_async": (I32, [P, P, P, P, U, S, S, S, P, S, U, U, B]),
        "zlm_gpu_mat_vec_mlp_pair_resident_burst_async": (I32, [P, P, P, P, U, U, S, S, S, P, S, U, U, B]),
        "zlm_gpu_wait_resident": (B, [P, I32, P, S, S]),
        "zlm_gpu_mat_vec_resident_batch": (B, [P, S, P, S, P, S]),
        "zlm_gpu_upload_resident": (P, [P, P, S]),
        "zlm_gpu_free_resident": (None, [P, P]),
        "zlm_gpu_sync": (None, [P]),
        "zlm_gpu_probe": (None, [P, S, S, S, P]),
        "zlm_gpu_resident_bytes": (ctypes.c_uint64, [P]),
        "zlm_gpu_resident_read_raw": (B, [P, P, P, S]),
        "zlm_gpu_last_error": (ctypes.c_char_p, [P]),
        "zlm_gpu_cu_count": (ctypes.c_int, [P]),
        "zlm_gpu_vram_info": (B, [P, P, P]),
        "zlm_gpu_dev_malloc": (P, [P, S]),
        "zlm_gpu_dev_free": (None, [P, P]),
        "zlm_gpu_dev_upload": (B, [P, P, P, S]),
        "zlm_gpu_dev_download": (B, [P, P, P, S]),
        "zlm_gpu_dev_copy": (B, [P, P, P, S]),
        "zlm_gpu_dev_copy_enqueue": (B, [P, P, P, S]),
        "zlm_gpu_mat_vec_enqueue": (B, [P, P, U, S, S, P, P]),
        "zlm_gpu_mat_vec_batch_enqueue": (B, [P, P, U, P, S, S, P, P]),
        "zlm_gpu_time_mat_vec": (B, [P, P, S, U, S, S, P, P, ctypes.c_int, P]),
        "zlm_gpu_mat_mul_enqueue": (B, [P, P, U, S, S, S, P, P]),
        "zlm_gpu_time_mat_mul": (B, [P, P, S, U, S, S, S, P, P, ctypes.c_int, P]),
        "zlm_gpu_time_gemv_sequence": (B, [P, P, S, ctypes.c_int, P]),
        "zlm_gpu_dequant_resident": (B, [P, P, U, S, P]),
        "zlm_gpu_gemv_op_enqueue": (B, [P, P]),
        "zlm_gpu_qk_norm_rope_kv_enqueue": (B, [P, P, P, P, P, U, U, U, ctypes.c_float, ctypes.c_float, P, P, P,
                                                U]),
        "zlm_gpu_attention_enqueue": (B, [P, P, P, P, U, U, U, P, U, ctypes.c_float, P]),
        "zlm_gpu_attention_decode_enqueue": (B, [P, P, P, P, U, U, U, ctypes.c_float, ctypes.c_float, P, P, P, U,
                                                 ctypes.c_float, P]),
        "zlm_gpu_attention_decode_enqueue_noalloc": (B, [P, P, P, P, U, U, U, ctypes.c_float, ctypes.c_float, P, P,
                                                         P, U, ctypes.c_float, P]),
        "zlm_gpu_attention_decode_window_enqueue": (B, [P, P, P, P, U, U, U, ctypes.c_float, ctypes.c_float, P, P,
                                                        P, U, U, ctypes.c_float, P]),
        "zlm_gpu_resident_device_bytes": (ctypes.c_uint64, [P]),
        "zlm_gpu_layout_bytes": (ctypes.c_uint64, [U, S, S, ctypes.c_bool]),
        "zlm_gpu_release_gemm_tiles": (B, [P, P]),
        "zlm_gpu_probe_rates": (B, [P, U, ctypes.c_bool, S, S, P]),
        "zlm_gpu_time_contract_gemv": (B, [P, P, S, U, S, S, ctypes.c_int, P]),
        "zlm_gpu_time_contract_gemv_split": (B, [P, P, S, U, S, S, ctypes.c_int, P]),
        "zlm_gpu_time_contract_decode": (B, [P, P, S, U, S, S, S, S, P, U, S, ctypes.c_int, P]),
        "zlm_gpu_capture_begin": (B, [P]),
        "zlm_gpu_capture_end": (P, [P]),
        "zlm_gpu_graph_launch": (B, [P, P, ctypes.c_int, P]),
        "zlm_gpu_graph_destroy": (None, [P, P]),
        "zlm_gpu_profiler_loaded": (B, [ctypes.c_char_p]),
        "zlm_gpu_kernel_convention": (B, [ctypes.c_char_p, P, P]),
        "zlm_gpu_launch_log": (B, [P, B]),
        "zlm_gpu_launch_log_read": (S, [P, P, S]),
        "zlm_gpu_scratch_device_bytes": (ctypes.c_uint64, [P]),
        "zlm_gpu_synth_resident": (P, [P, U, S, ctypes.c_uint64, ctypes.c_float]),
        "zlm_gpu_synth_f16": (B, [P, P, S, ctypes.c_uint64, ctypes.c_float]),
        "zlm_gpu_quantize_act_q8": (B, [P, P, S, P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def _f32(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError("expected a C-contiguous float32 array")
    return a


def _u8(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.uint8 or not a.flags.c_contiguous:
        raise TypeError("expected a C-contiguous uint8 array")
    return a


class Resident:
    """A weight uploaded once into HBM (reference ``Resident``, root.zig:241-244)."""

    def __init__(self, dev: "Device", ptr: int):
        self._dev = dev
        self.ptr = ptr

    @property
    def bytes(self) -> int:
        return int(lib().zlm_gpu_resident_bytes(self.ptr))


@dataclass
class ResidentOp:
    """One resident GEMV of a batch (reference ``ResidentOp``, root.zig:249-254)."""

    res: Resident
    quant: int
    rows: int
    out: np.ndarray


@dataclass
class Probe:
    """Measured co-processor rates (reference ``Probe``, root.zig:260-295)."""

    fields: dict = field(default_factory=dict)

    def __getattr__(self, name):
        try:
            return self.fields[name]
        except KeyError as e:
            raise AttributeError(name) from e


class Device:
    """The HIP co-processor; inert (``available() is False``) without a gfx950 GPU."""

    def __init__(self) -> None:
        self._L = lib()
        self._h = self._L.zlm_gpu_init()
        if not self._h:
            raise MemoryError("zlm_gpu_init returned NULL")

    # -- lifecycle / identity -------------------------------------------------
    def deinit(self) -> None:
        if self._h:
            self._L.zlm_gpu_deinit(self._h)
            self._h = None

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass

    def available(self) -> bool:
        return bool(self._h) and bool(self._L.zlm_gpu_available(self._h))

    def backend_name(self) -> str:
        return self._L.zlm_gpu_backend_name(self._h).decode()

    def device_name(self) -> str:
        return self._L.zlm_gpu_device_name(self._h).decode()

    def is_uma(self) -> bool:
        return bool(self._L.zlm_gpu_is_uma(self._h))

    def last_error(self) -> str:
        return self._L.zlm_gpu_last_error(self._h).decode()

    def vram_info(self) -> Optional[tuple]:
        """(free, total) HBM bytes, or None when inert."""
        f, t = ctypes.c_uint64(0), ctypes.c_uint64(0)
        if not self._L.zlm_gpu_vram_info(self._h, ctypes.addressof(f), ctypes.addressof(t)):
            return None
        return f.value, t.value

    def cu_count(self) -> int:
        return int(self._L.zlm_gpu_cu_count(self._h))

    # -- GEMV / GEMM -----------------------------------------------------------
    def mat_vec(self, quant: int, weight: np.ndarray, rows: int, k: int, x: np.ndarray, out: np.ndarray) -> bool:
        w, x, out = _u8(weight), _f32(x), _f32(out)
        return bool(self._L.zlm_gpu_mat_vec(self._h, quant, _p(w), w.size, rows, k, _p(x), x.size, _p(out), out.size))

    def mat_mul_batch(self, quant: int, weight: np.ndarray, rows: int, k: int, m: int, x: np.ndarray,
                      out: np.ndarray) -> bool:
        w, x, out = _u8(weight), _f32(x), _f32(out)
        return bool(self._L.zlm_gpu_mat_mul_batch(self._h, quant, _p(w), w.size, rows, k, m, _p(x), x.size,
                                                  _p(out), out.size))

    def mat_mul_resident(self, res: Resident, quant: int, rows: int, k: int, m: int, x: np.ndarray,
                         out: np.ndarray) -> bool:
        x, out = _f32(x), _f32(out)
        return bool(self._L.zlm_gpu_mat_mul_resident(self._h, res.ptr, quant, rows, k, m, _p(x), x.size, _p(out),
                                                     out.size))

    def mat_vec_resident(self, res: Resident, quant: int, rows: int, k: int, x: np.ndarray,
                         out: np.ndarray) -> bool:
        x, out = _f32(x), _f32(out)
        return bool(self._L.zlm_gpu_mat_vec_resident(self._h, res.ptr, quant, rows, k, _p(x), x.size, _p(out),
                                                     out.size))

    @staticmethod
    def _handle(h: int) -> Optional[int]:
        return None if h < 0 else int(h)

    def mat_vec_resident_async(self, res: Resident, quant: int, rows: int, k: int, x: np.ndarray) -> Optional[int]:
        x = _f32(x)
        return self._handle(self._L.zlm_gpu_mat_vec_resident_async(self._h, res.ptr, quant, rows, k, _p(x), x.size))

    def mat_vec_resident_burst_async(self, res: Resident, quant: int, rows: int, k: int, x: np.ndarray,
                                     first: bool) -> Optional[int]:
        x = _f32(x)
        return self._handle(self._L.zlm_gpu_mat_vec_resident_burst_async(self._h, res.ptr, quant, rows, k, _p(x),
                                                                         x.size, first))

    def mat_vec_gate_up_resident_burst_async(self, res_gate: Resident, res_up: Resident, quant: int, rows: int,
                                             k: int, x: np.ndarray, act: int, variant: int,
                                             first: bool) -> Optional[int]:
        x = _f32(x)
        return self._handle(self._L.zlm_gpu_mat_vec_gate_up_resident_burst_async(
            self._h, res_gate.ptr, res_up.ptr, quant, rows, k, _p(x), x.size, act, variant, first))

    def mat_vec_mlp_resident_burst_async(self, res_gate: Resident, res_up: Resident, res_down: Resident,
                                         quant: int, rows: int, k: int, ffn: int, x: np.ndarray, act: int,
                                         variant: int, first: bool) -> Optional[int]:
        x = _f32(x)
        return self._handle(self._L.zlm_gpu_mat_vec_mlp_resident_burst_async(
            self._h, res_gate.ptr, res_up.ptr, res_down.ptr, quant, rows, k, ffn, _p(x), x.size, act, variant,
            first))

    def mat_vec_mlp_pair_resident_burst_async(self, res_gate: Resident, res_up: Resident, res_down: Resident,
                                              gu_quant: int, down_quant: int, rows: int, k: int, ffn: int,
                                              x: np.ndarray, act: int, variant: int,
                                              first: bool) -> Optional[int]:
        x = _f32(x)
        return self._handle(self._L.zlm_gpu_mat_vec_mlp_pair_resident_burst_async(
            self._h, res_gate.ptr, res_up.ptr, res_down.ptr, gu_quant, down_quant, rows, k, ffn, _p(x), x.size,
            act, variant, first))

    def wait_resident(self, h: int, out: np.ndarray, rows: int) -> bool:
        out = _f32(out)
        return bool(self._L.zlm_gpu_wait_resident(self._h, h, _p(out), out.size, rows))

    def mat_vec_resident_batch(self, k: int, x: np.ndarray, ops: Sequence[ResidentOp]) -> bool:
        x = _f32(x)
        arr = (_ResidentOp * max(1, len(ops)))()
        for i, op in enumerate(ops):
            o = _f32(op.out)
            arr[i] = _ResidentOp(op.res.ptr, op.quant, op.rows, _p(o), o.size)
        return bool(self._L.zlm_gpu_mat_vec_resident_batch(self._h, k, _p(x), x.size, ctypes.addressof(arr),
                                                           len(ops)))

    # -- residency -------------------------------------------------------------
    def upload_resident(self, data: np.ndarray) -> Optional[Resident]:
        d = _u8(data)
        ptr = self._L.zlm_gpu_upload_resident(self._h, _p(d), d.size)
        return Resident(self, ptr) if ptr else None

    def free_resident(self, res: Resident) -> None:
        if res is not None and res.ptr:
            self._L.zlm_gpu_free_resident(self._h, res.ptr)
            res.ptr = None

    def sync(self) -> None:
        self._L.zlm_gpu_sync(self._h)

    def probe_gpu(self, rows: int, k: int, m: int) -> Probe:
        p = _Probe()
        self._L.zlm_gpu_probe(self._h, rows, k, m, ctypes.addressof(p))
        return Probe({name: getattr(p, name) for name, _ in _Probe._fields_})

    # -- device-level helpers (no reference counterpart) -----------------------
    def dev_malloc(self, nbytes: int) -> int:
        p = self._L.zlm_gpu_dev_malloc(self._h, nbytes)
        if not p:
            raise MemoryError(self.last_error())
        return p

    def dev_free(self, ptr: int) -> None:
        self._L.zlm_gpu_dev_free(self._h, ptr)

    def dev_upload(self, dst: int, src: np.ndarray) -> None:
        src = np.ascontiguousarray(src)
        if not self._L.zlm_gpu_dev_upload(self._h, dst, _p(src), src.nbytes):
            raise RuntimeError(self.last_error())

    def dev_download(self, dst: np.ndarray, src: int) -> None:
        if not dst.flags.c_contiguous:
            raise TypeError("destination must be contiguous")
        if not self._L.zlm_gpu_dev_download(self._h, _p(dst), src, dst.nbytes):
            raise RuntimeError(self.last_error())

    def dev_copy(self, dst: int, src: int, nbytes: int) -> None:
        if not self._L.zlm_gpu_dev_copy(self._h, dst, src, nbytes):
            raise RuntimeError(self.last_error())

    def dev_copy_enqueue(self, dst: int, src: int, nbytes: int) -> bool:
        return bool(self._L.zlm_gpu_dev_copy_enqueue(self._h, dst, src, nbytes))

    def mat_vec_enqueue(self, res: Resident, quant: int, rows: int, k: int, x_dev: int, y_dev: int) -> bool:
        return bool(self._L.zlm_gpu_mat_vec_enqueue(self._h, res.ptr, quant, rows, k, x_dev, y_dev))

    def mat_vec_batch_enqueue(self, residents: Sequence[Resident], quant: int, rows: Sequence[int], k: int,
                              x_dev: int, y_devs: Sequence[int]) -> bool:
        """One launch of up to RING_SIZE GEMVs over one device x (no wait)."""
        n = len(residents)
        ra = (ctypes.c_void_p * max(1, n))(*[r.ptr for r in residents])
        rw = (ctypes.c_size_t * max(1, n))(*rows)
        ya = (ctypes.c_void_p * max(1, n))(*y_devs)
        return bool(self._L.zlm_gpu_mat_vec_batch_enqueue(self._h, ctypes.addressof(ra), quant, ctypes.addressof(rw),
                                                          n, k, x_dev, ctypes.addressof(ya)))

    def time_mat_vec(self, residents: Sequence[Resident], quant: int, rows: int, k: int, x_dev: int, y_dev: int,
                     iters: int) -> float:
        """GPU milliseconds for `iters` GEMVs rotating over `residents` (HIP events)."""
        arr = (ctypes.c_void_p * len(residents))(*[r.ptr for r in residents])
        ms = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_time_mat_vec(self._h, ctypes.addressof(arr), len(residents), quant, rows, k, x_dev,
                                            y_dev, iters, ctypes.addressof(ms)):
            raise RuntimeError(self.last_error())
        return ms.value

    def mat_mul_enqueue(self, res: Resident, quant: int, rows: int, k: int, m: int, x_dev: int, out_dev: int) -> bool:
        return bool(self._L.zlm_gpu_mat_mul_enqueue(self._h, res.ptr, quant, rows, k, m, x_dev, out_dev))

    def time_mat_mul(self, residents: Sequence[Resident], quant: int, rows: int, k: int, m: int, x_dev: int,
                     out_dev: int, iters: int) -> float:
        """GPU milliseconds for `iters` prefill GEMMs (quantizer + GEMM) rotating over `residents`."""
        arr = (ctypes.c_void_p * len(residents))(*[r.ptr for r in residents])
        ms = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_time_mat_mul(self._h, ctypes.addressof(arr), len(residents), quant, rows, k, m, x_dev,
                                            out_dev, iters, ctypes.addressof(ms)):
            raise RuntimeError(self.last_error())
        return ms.value

    def time_gemv_sequence(self, descs: Sequence[tuple], iters: int) -> float:
        """GPU milliseconds for `iters` passes over descs = [(res, quant, rows, k, x_dev, y_dev[, with_next]), ...];
        with_next joins a GEMV and the next into one batch launch."""
        arr = (_GemvDesc * len(descs))()
        for i, d in enumerate(descs):
            res, q, rows, k, xd, yd = d[:6]
            arr[i] = _GemvDesc(res.ptr, q, rows, k, xd, yd, int(d[6]) if len(d) > 6 else 0)
        ms = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_time_gemv_sequence(self._h, ctypes.addressof(arr), len(descs), iters,
                                                  ctypes.addressof(ms)):
            raise RuntimeError(self.last_error())
        return ms.value

    def gemv_op_enqueue(self, form: int, quant: int, w: Resident, rows: int, k: int, x_dev: int, y_dev: int,
                        w_up: Optional[Resident] = None, norm_w: int = 0, eps: float = 0.0, act: int = SILU,
                        res: int = 0) -> bool:
        """Enqueue one GEMV form on device buffers (no wait); see zlm_gemv_op."""
        op = _GemvOp(form, quant, w.ptr if w else None, w_up.ptr if w_up else None, rows, k, x_dev,
                     norm_w or None, eps, act, res or None, y_dev)
        return bool(self._L.zlm_gpu_gemv_op_enqueue(self._h, ctypes.byref(op)))

    # -- decode-step glue, graphs, synthetic data ------------------------------
    def qk_norm_rope_kv_enqueue(self, qkv: int, q_out: int, q_norm_w: int, k_norm_w: int, n_heads: int,
                                n_kv_heads: int, head_dim: int, eps: float, freq_base: float, pos: int,
                                k_cache: int, v_cache: int, max_seq: int) -> bool:
        return bool(self._L.zlm_gpu_qk_norm_rope_kv_enqueue(self._h, qkv, q_out, q_norm_w, k_norm_w, n_heads,
                                                            n_kv_heads, head_dim, eps, freq_base, pos, k_cache,
                                                            v_cache, max_seq))

    def attention_enqueue(self, q: int, k_cache: int, v_cache: int, n_heads: int, n_kv_heads: int, head_dim: int,
                          pos: int, max_seq: int, scale: float, out: int) -> bool:
        return bool(self._L.zlm_gpu_attention_enqueue(self._h, q, k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                                      pos, max_seq, scale, out))

    def attention_decode_enqueue(self, qkv: int, q_norm_w: int, k_norm_w: int, n_heads: int, n_kv_heads: int,
                                 head_dim: int, eps: float, freq_base: float, pos: int, k_cache: int, v_cache: int,
                                 max_seq: int, scale: float, out: int) -> bool:
        return bool(self._L.zlm_gpu_attention_decode_enqueue(self._h, qkv, q_norm_w, k_norm_w, n_heads, n_kv_heads,
                                                             head_dim, eps, freq_base, pos, k_cache, v_cache,
                                                             max_seq, scale, out))

    def attention_decode_window_enqueue(self, qkv: int, q_norm_w: int, k_norm_w: int, n_heads: int,
                                        n_kv_heads: int, head_dim: int, eps: float, freq_base: float, pos: int,
                                        k_cache: int, v_cache: int, max_seq: int, window: int, scale: float,
                                        out: int) -> bool:
        """attention_decode_enqueue over positions [0, window) only (a position
        at or past the window gives NaN heads)."""
        return bool(self._L.zlm_gpu_attention_decode_window_enqueue(self._h, qkv, q_norm_w, k_norm_w, n_heads,
                                                                    n_kv_heads, head_dim, eps, freq_base, pos,
                                                                    k_cache, v_cache, max_seq, window, scale, out))

    def attention_decode_enqueue_noalloc(self, qkv: int, q_norm_w: int, k_norm_w: int, n_heads: int,
                                         n_kv_heads: int, head_dim: int, eps: float, freq_base: float, pos: int,
                                         k_cache: int, v_cache: int, max_seq: int, scale: float, out: int) -> bool:
        """attention_decode_enqueue with its partials in the library's fixed
        static scratch: allocates nothing (see the C header for the limit)."""
        return bool(self._L.zlm_gpu_attention_decode_enqueue_noalloc(self._h, qkv, q_norm_w, k_norm_w, n_heads,
                                                                     n_kv_heads, head_dim, eps, freq_base, pos,
                                                                     k_cache, v_cache, max_seq, scale, out))

    def probe_rates(self, ggml_type: int, gate_up: bool, rows: int, k: int) -> Optional[np.ndarray]:
        """GB/s of each GpuVariant for one quant (resident GEMV or fused gate_up); None if one did not run."""
        r = np.zeros(8, np.float64)
        if not self._L.zlm_gpu_probe_rates(self._h, ggml_type, gate_up, rows, k, _p(r)):
            return None
        return r

    def time_contract_gemv(self, residents: Sequence[Resident], quant: int, rows: int, k: int, iters: int) -> float:
        """Host-wall us per contract GEMV (burst of one + waitResident, host x and y)."""
        arr = (ctypes.c_void_p * len(residents))(*[r.ptr for r in residents])
        us = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_time_contract_gemv(self._h, arr, len(residents), quant, rows, k, iters,
                                                  ctypes.addressof(us)):
            raise RuntimeError(self.last_error())
        return us.value

    def time_contract_gemv_split(self, residents: Sequence[Resident], quant: int, rows: int, k: int,
                                 iters: int) -> dict:
        """Per-op host microseconds of a contract GEMV: total, submit, wait, and the GPU's own time."""
        arr = (ctypes.c_void_p * len(residents))(*[r.ptr for r in residents])
        out = (ctypes.c_double * 4)()
        if not self._L.zlm_gpu_time_contract_gemv_split(self._h, arr, len(residents), quant, rows, k, iters,
                                                        ctypes.addressof(out)):
            raise RuntimeError(self.last_error())
        return {"total_us": out[0], "submit_us": out[1], "wait_us": out[2], "gpu_us": out[3]}

    def time_contract_decode(self, layers: Sequence[Sequence[Resident]], quant: int, hidden: int, q_rows: int,
                             kv_rows: int, ffn: int, lm_head: Resident, lm_quant: int, vocab: int, iters: int) -> float:
        """Host-wall ms per token of the projections driven through the contract ops
        (layers[i] = (q, k, v, o, gate, up, down) residents)."""
        Arr = ctypes.c_void_p * (7 * len(layers))
        arr = Arr(*[r.ptr for layer in layers for r in layer])
        ms = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_time_contract_decode(self._h, arr, len(layers), quant, hidden, q_rows, kv_rows, ffn,
                                                    lm_head.ptr, lm_quant, vocab, iters, ctypes.addressof(ms)):
            raise RuntimeError(self.last_error())
        return ms.value

    def resident_read_raw(self, res: Resident) -> np.ndarray:
        """The resident's raw GGUF bytes (only before its first op)."""
        out = np.empty(res.bytes, np.uint8)
        if not self._L.zlm_gpu_resident_read_raw(self._h, res.ptr, _p(out), out.size):
            raise RuntimeError(self.last_error())
        return out

    def resident_device_bytes(self, res: Resident) -> int:
        """HBM the resident holds now (raw bytes, device layout, GEMM tiles)."""
        return int(self._L.zlm_gpu_resident_device_bytes(res.ptr))

    def release_gemm_tiles(self, res: Resident) -> bool:
        return bool(self._L.zlm_gpu_release_gemm_tiles(self._h, res.ptr))

    def capture_begin(self) -> bool:
        return bool(self._L.zlm_gpu_capture_begin(self._h))

    def capture_end(self) -> Optional[int]:
        g = self._L.zlm_gpu_capture_end(self._h)
        return g or None

    def graph_launch(self, graph: int, iters: int = 1) -> float:
        """Launch a captured graph `iters` times; returns GPU milliseconds for all of them."""
        ms = ctypes.c_double(0.0)
        if not self._L.zlm_gpu_graph_launch(self._h, graph, iters, ctypes.addressof(ms)):
            raise RuntimeError(self.last_error())
        return ms.value

    def graph_destroy(self, graph: int) -> None:
        self._L.zlm_gpu_graph_destroy(self._h, graph)

    def launch_log(self, enable: bool) -> bool:
        """Turn the launch log on or off (either clears it)."""
        return bool(self._L.zlm_gpu_launch_log(self._h, enable))

    def launch_log_read(self) -> list:
        """The logged launches as dicts (what, grid_x/y/z, block, lds_bytes)."""
        n = int(self._L.zlm_gpu_launch_log_read(self._h, None, 0))
        arr = (LaunchRecord * max(1, n))()
        self._L.zlm_gpu_launch_log_read(self._h, ctypes.addressof(arr), n)
        return [{"what": r.what.decode(), "grid_x": r.grid_x, "grid_y": r.grid_y, "grid_z": r.grid_z,
                 "block": r.block, "lds_bytes": r.lds_bytes} for r in arr[:n]]

    def scratch_device_bytes(self) -> int:
        """Device bytes the library holds for staging and scratch (not residents)."""
        return int(self._L.zlm_gpu_scratch_device_bytes(self._h))

    def synth_resident(self, ggml_type: int, n_blocks: int, seed: int, scale: float) -> Optional[Resident]:
        p = self._L.zlm_gpu_synth_resident(self._h, ggml_type, n_blocks, seed & 0xFFFFFFFFFFFFFFFF, scale)
        return Resident(self, p) if p else None

    def synth_f16(self, dst: int, n: int, seed: int, scale: float) -> None:
        if not self._L.zlm_gpu_synth_f16(self._h, dst, n, seed & 0xFFFFFFFFFFFFFFFF, scale):
            raise RuntimeError(self.last_error())

    def dequant_resident(self, res: Resident, quant: int, n: int) -> Optional[np.ndarray]:
        out = np.zeros(n, np.float32)
        if not self._L.zlm_gpu_dequant_resident(self._h, res.ptr, quant, n, _p(out)):
            return None
        return out

    def quantize_act_q8(self, x: np.ndarray):
        x = _f32(x)
        n = x.size
        qx = np.zeros(n, np.int8)
        dx = np.zeros(n // 32, np.float32)
        sums = np.zeros(n // 32, np.int32)
        if not self._L.zlm_gpu_quantize_act_q8(self._h, _p(x), n, _p(qx), _p(dx), _p(sums)):
            return None
        return qx, dx, sums


def profiler_loaded(maps_path: Optional[str] = None) -> bool:
    """Whether a rocprofiler library is mapped (this process, or a maps-format file)."""
    return bool(lib().zlm_gpu_profiler_loaded(None if maps_path is None else maps_path.encode()))


def kernel_convention(name: str) -> Optional[tuple]:
    """(role, takes one GemvArgs block) as the host reads them from a GEMV
    entry point's name, or None for a name outside zlm_gemv_<quant>_...; no
    device needed."""
    role = ctypes.c_int32(0)
    st = ctypes.c_bool(False)
    if not lib().zlm_gpu_kernel_convention(name.encode(), ctypes.addressof(role), ctypes.addressof(st)):
        return None
    return int(role.value), bool(st.value)
