"""probeGpu (reference gpu/backend/root.zig:357-498) on the HIP device: every
rate the backend can measure is filled (GB/s of weight bytes over host wall
time, min of 5), every variant field names a GpuVariant, and the quants this
backend does not run stay at the contract's "unmeasured" (0 / plain)."""
import pytest

from zlm_amd import device as zd

pytestmark = pytest.mark.gpu


def test_probe_fills_measured_fields(dev):
    p = dev.probe_gpu(4096, 4096, 4)
    for name in ("gemv_gbps", "gemv_streamed_gbps", "matmul_gbps", "q4_0_u4_gbps", "q4_0_sub_gbps",
                 "q4_0_un2_gbps", "q4_0_un4_gbps", "q4_0_w32_gbps", "q4_0_w128_gbps", "q4_k_gbps", "q4_k_u4_gbps",
                 "gate_up_gbps", "gate_up_u4_gbps"):
        v = getattr(p, name)
        assert 0.0 < v < 8000.0, (name, v)
    # a resident GEMV beats the streamed one (no weight upload per call)
    assert p.gemv_gbps > p.gemv_streamed_gbps
    for name in ("q4_0_variant", "q8_0_variant", "q6_k_variant", "q4_k_variant", "gate_up_variant",
                 "gate_up_q8_0_variant"):
        assert 0 <= getattr(p, name) < 8, name
    for name in ("q4_1_variant", "f32_variant", "f16_variant", "bf16_variant", "gate_up_q4_1_variant"):
        assert getattr(p, name) == zd.PLAIN, name


def test_probe_clamps_its_shape(dev):
    p = dev.probe_gpu(1 << 20, 1 << 20, 0)  # clamped to 12288 x 4096, m >= 2
    assert p.gemv_gbps > 0 and p.matmul_gbps > 0
    z = dev.probe_gpu(0, 4096, 2)
    assert z.gemv_gbps == 0 and z.q4_0_variant == zd.PLAIN


def test_vram_info_tracks_residents(dev):
    free0, total = dev.vram_info()
    assert 0 < free0 <= total
    big = dev.dev_malloc(1 << 30)
    free1, _ = dev.vram_info()
    assert free1 <= free0 - (1 << 30) + (64 << 20)
    dev.dev_free(big)
