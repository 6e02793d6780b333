"""zlm_amd -- MI355X (gfx950) HIP backend for zlm's quantized GEMV/GEMM path.

``zlm_amd.device.Device`` mirrors the reference co-processor contract
(``src/gpu/backend/root.zig:299-311``) over ``lib/libzlm_gpu_hip.so``;
``zlm_amd.synth`` generates the seeded synthetic weights and activations of the
benchmark configurations.
"""
from . import synth  # noqa: F401
from .device import (  # noqa: F401
    BF16, F16, F32, GELU, NULL_HANDLE, PLAIN, Q4_0, Q4_1, Q4_K, Q6_K, Q8_0, RING_SIZE, SILU, SUB, U4, U8, UN2,
    UN4, W32, W128, Device, Probe, Resident, ResidentOp, quant,
)

__all__ = [
    "Device", "Resident", "ResidentOp", "Probe", "quant", "synth",
    "F32", "F16", "BF16", "Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q6_K",
    "PLAIN", "U4", "U8", "SUB", "UN2", "UN4", "W32", "W128", "SILU", "GELU", "RING_SIZE", "NULL_HANDLE",
]
