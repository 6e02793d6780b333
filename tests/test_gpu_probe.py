"""probeGpu (reference gpu/backend/root.zig:357-498) on the HIP device: every
rate the probe reports is filled (GB/s of weight bytes over host wall time,
min of 5), every quant the backend runs is probed -- q4_0, q4_1, q8_0, q4_k,
q6_k, f32, f16, bf16 and the fused gate_up over q4_0, q8_0 and q4_1, as the
reference's probe does (:440-498) -- and each recorded winner is a variant
whose rate was measured."""
import pytest

from zlm_amd import device as zd

pytestmark = pytest.mark.gpu

VARIANT_FIELDS = ("q4_0_variant", "q4_1_variant", "q8_0_variant", "q6_k_variant", "q4_k_variant", "f32_variant",
                  "f16_variant", "bf16_variant", "gate_up_variant", "gate_up_q4_1_variant", "gate_up_q8_0_variant")


def test_probe_fills_measured_fields(dev):
    p = dev.probe_gpu(4096, 4096, 4)
    for name in ("gemv_gbps", "gemv_streamed_gbps", "matmul_gbps", "q4_0_u4_gbps", "q4_0_sub_gbps",
                 "q4_0_un2_gbps", "q4_0_un4_gbps", "q4_0_w32_gbps", "q4_0_w128_gbps", "q4_k_gbps", "q4_k_u4_gbps",
                 "gate_up_gbps", "gate_up_u4_gbps"):
        v = getattr(p, name)
        assert 0.0 < v < 8000.0, (name, v)
    # a resident GEMV beats the streamed one (no weight upload per call)
    assert p.gemv_gbps > p.gemv_streamed_gbps
    for name in VARIANT_FIELDS:
        assert 0 <= getattr(p, name) < 8, name


@pytest.mark.parametrize("qt,gate_up", [(zd.Q4_0, False), (zd.Q4_1, False), (zd.Q8_0, False), (zd.Q4_K, False),
                                        (zd.Q6_K, False), (zd.F32, False), (zd.F16, False), (zd.BF16, False),
                                        (zd.Q4_0, True), (zd.Q8_0, True), (zd.Q4_1, True)])
def test_every_probed_variant_is_measured(dev, qt, gate_up):
    """The rate table behind each probe entry: all eight GpuVariants ran and
    got a rate, so the probe's winner (their fastest) is a measured one."""
    rates = dev.probe_rates(qt, gate_up, 4096, 4096)
    assert rates is not None, dev.last_error()
    assert all(0.0 < r < 8000.0 for r in rates), rates


def test_probe_clamps_its_shape(dev):
    p = dev.probe_gpu(1 << 20, 1 << 20, 0)  # clamped to 12288 x 4096, m >= 2
    assert p.gemv_gbps > 0 and p.matmul_gbps > 0
    z = dev.probe_gpu(0, 4096, 2)
    assert z.gemv_gbps == 0 and z.q4_0_variant == zd.PLAIN
    assert dev.probe_rates(77, False, 64, 256) is None  # unknown type


def test_vram_info_tracks_residents(dev):
    free0, total = dev.vram_info()
    assert 0 < free0 <= total
    big = dev.dev_malloc(1 << 30)
    free1, _ = dev.vram_info()
    assert free1 <= free0 - (1 << 30) + (64 << 20)
    dev.dev_free(big)
