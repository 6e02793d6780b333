"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and without a GPU the device is inert (the reference's
`available() == false`, every op refused) -- gpu/root_test.zig:328-336."""
import os
import re

import numpy as np
import pytest

from zlm_amd import device as zd
from zlm_amd import synth

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "zlm_gpu_hip.h")

# The reference contract's op names (gpu/backend/root.zig:299-311) and the C symbol each maps to.
REQUIRED_OPS = {
    "init": "zlm_gpu_init",
    "deinit": "zlm_gpu_deinit",
    "available": "zlm_gpu_available",
    "backendName": "zlm_gpu_backend_name",
    "deviceName": "zlm_gpu_device_name",
    "isUma": "zlm_gpu_is_uma",
    "matVec": "zlm_gpu_mat_vec",
    "matMulBatch": "zlm_gpu_mat_mul_batch",
    "matMulResident": "zlm_gpu_mat_mul_resident",
    "matVecResident": "zlm_gpu_mat_vec_resident",
    "matVecResidentAsync": "zlm_gpu_mat_vec_resident_async",
    "matVecResidentBurstAsync": "zlm_gpu_mat_vec_resident_burst_async",
    "matVecGateUpResidentBurstAsync": "zlm_gpu_mat_vec_gate_up_resident_burst_async",
    "matVecMlpResidentBurstAsync": "zlm_gpu_mat_vec_mlp_resident_burst_async",
    "matVecMlpPairResidentBurstAsync": "zlm_gpu_mat_vec_mlp_pair_resident_burst_async",
    "waitResident": "zlm_gpu_wait_resident",
    "matVecResidentBatch": "zlm_gpu_mat_vec_resident_batch",
    "uploadResident": "zlm_gpu_upload_resident",
    "freeResident": "zlm_gpu_free_resident",
    "sync": "zlm_gpu_sync",
    "probeGpu": "zlm_gpu_probe",
}


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zlm_gpu_\w+)\s*\(", text)))


def test_header_declares_every_required_op():
    names = declared_functions()
    for op, sym in REQUIRED_OPS.items():
        assert sym in names, f"contract op {op} has no C entry point"


def test_library_exports_every_declared_symbol():
    L = zd.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_code_objects_built_for_gfx950():
    for path in zd.CODE_OBJECT_PATHS:
        assert os.path.exists(path), path
        blob = open(path, "rb").read()
        # hipcc --genco writes an offload bundle around the gfx950 ELF
        assert blob[:4] == b"\x7fELF" or blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
        assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_quant_encoding():
    assert zd.quant(zd.Q4_0) == 2
    assert zd.quant(zd.Q8_0, zd.U4) == 8 | (1 << 8)
    assert zd.quant(zd.Q6_K, zd.W128) == 14 | (7 << 8)


def test_inert_device_refuses_everything():
    dev = zd.Device()
    if dev.available():
        pytest.skip("a GPU is present; the inert-device contract is checked on GPU-less hosts")
    assert dev.backend_name() == "off" and dev.device_name() == "off" and not dev.is_uma()
    rows, k = 8, 64
    w = synth.weights(synth.Q4_0, rows, k, seed=1)
    x = synth.activation(1, k)
    out = np.zeros(rows, np.float32)
    assert not dev.mat_vec(zd.quant(zd.Q4_0), w, rows, k, x, out)
    assert not dev.mat_mul_batch(zd.quant(zd.Q4_0), w, rows, k, 2, np.zeros(2 * k, np.float32),
                                 np.zeros(2 * rows, np.float32))
    assert dev.upload_resident(w) is None
    fake = zd.Resident(dev, None)
    assert not dev.mat_vec_resident(fake, zd.quant(zd.Q4_0), rows, k, x, out)
    assert dev.mat_vec_resident_async(fake, zd.quant(zd.Q4_0), rows, k, x) is None
    assert dev.mat_vec_resident_burst_async(fake, zd.quant(zd.Q4_0), rows, k, x, True) is None
    assert dev.mat_vec_gate_up_resident_burst_async(fake, fake, zd.quant(zd.Q4_0), rows, k, x, zd.SILU, 0,
                                                    True) is None
    assert not dev.wait_resident(0, out, rows)
    assert not dev.mat_vec_resident_batch(k, x, [zd.ResidentOp(fake, zd.quant(zd.Q4_0), rows, out)])
    assert dev.vram_info() is None
    p = dev.probe_gpu(rows, k, 2)
    assert p.gemv_gbps == 0 and p.matmul_gbps == 0 and p.q4_0_variant == 0
    dev.sync()
    dev.free_resident(fake)
    dev.deinit()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(zd, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(zd, "_lib", None)
    with pytest.raises(ImportError):
        zd.Device()


def test_layout_bytes_for_the_residency_budget():
    """zlm_gpu_layout_bytes (host arithmetic, no GPU): the device layout of a
    weight (payload rounded to 256 bytes, then the split scales or records,
    then 256 bytes of slack) and the prefill GEMM's tiled copy."""
    nblk = 4096 * 4096 // 32
    q4 = 16 * nblk + 2 * nblk + 256
    assert zd.layout_bytes(zd.quant(zd.Q4_0), 4096, 4096, False) == q4
    tiles = 128 * 128 * 32 * 16 + 128 * 128 * 32 * 2  # 32-row tiles x blocks x (16 nibble bytes + f16 scale)
    assert zd.layout_bytes(zd.quant(zd.Q4_0), 4096, 4096, True) == q4 + tiles
    # q4_k: 128-byte qs blocks + 20-byte records; its tiles carry a (scale, min) float pair per 32 elements
    kb = 15360 * 3840 // 256
    q4k = 128 * kb + 20 * kb + 256
    assert zd.layout_bytes(zd.quant(zd.Q4_K), 15360, 3840, False) == q4k
    assert zd.layout_bytes(zd.quant(zd.Q4_K), 15360, 3840, True) == q4k + 480 * 120 * 32 * (16 + 8)
    # q6_k has no GEMM: with_gemm adds nothing; the float types keep their raw rows
    q6 = zd.layout_bytes(zd.quant(zd.Q6_K), 3840, 15360, False)
    assert q6 == zd.layout_bytes(zd.quant(zd.Q6_K), 3840, 15360, True) == 128 * 230400 + 84 * 230400 + 256
    assert zd.layout_bytes(zd.quant(zd.F16), 64, 256, True) == 64 * 256 * 2
    assert zd.layout_bytes(zd.quant(zd.Q4_0), 64, 100, False) == 0  # k not whole blocks
    assert zd.layout_bytes(77, 64, 256, False) == 0  # unknown type


def test_profiler_check_reads_the_process_map(tmp_path):
    """Graph replays are refused while a profiler library is mapped: the check
    matches rocprofiler-sdk (what rocprofv3 preloads) and the older
    librocprofiler64, not the HIP runtime's own librocprofiler-register or
    torch's roctracer / roctx, which every process maps."""
    base = ("7f0000000000-7f0000001000 r-xp 00000000 08:01 1 /opt/rocm/lib/libamdhip64.so.7\n"
            "7f0000001000-7f0000002000 r-xp 00000000 08:01 2 /opt/rocm/lib/librocprofiler-register.so.0.6.0\n"
            "7f0000002000-7f0000003000 r-xp 00000000 08:01 3 /usr/lib/torch/lib/libroctracer64.so\n"
            "7f0000003000-7f0000004000 r-xp 00000000 08:01 4 /usr/lib/torch/lib/libroctx64.so\n")
    plain = tmp_path / "plain"
    plain.write_text(base)
    assert not zd.profiler_loaded(str(plain))
    for lib_name in ("/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so.1",
                     "/opt/rocm/lib/librocprofiler-sdk.so.1.1.0", "/opt/rocm/lib/librocprofiler64.so.2"):
        traced = tmp_path / "traced"
        traced.write_text(base + f"7f0000005000-7f0000006000 r-xp 00000000 08:01 5 {lib_name}\n")
        assert zd.profiler_loaded(str(traced)), lib_name
    assert not zd.profiler_loaded(str(tmp_path / "missing"))
    # this test process runs without a profiler
    assert not zd.profiler_loaded()


def _kernel_args(path):
    """{kernel name: [sizes of its explicit arguments]} from a code object's
    metadata (the ROCm LLVM tools read the bundle and the ELF notes)."""
    import subprocess
    import tempfile
    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not (os.path.exists(bundler) and os.path.exists(readelf)):
        pytest.skip("ROCm LLVM tools not installed")
    with tempfile.TemporaryDirectory() as tmp:
        elf = os.path.join(tmp, "k.o")
        subprocess.run([bundler, "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={path}", f"--output={elf}"], check=True)
        notes = subprocess.run([readelf, "--notes", elf], capture_output=True, text=True, check=True).stdout
    out = {}
    for entry in re.split(r"\n\s+- \.agpr_count:", notes[notes.find("amdhsa.kernels:"):])[1:]:
        name = re.search(r"\n\s+\.name:\s+(\S+)", entry).group(1)
        args = entry[entry.find(".args:"):entry.find(".group_segment_fixed_size")]
        sizes = [int(x) for x in re.findall(r"\.size:\s+(\d+)", args)]
        kinds = re.findall(r"\.value_kind:\s+(\S+)", args)
        out[name] = [s for s, k in zip(sizes, kinds) if not k.startswith("hidden")]
    return out


def test_kernel_conventions_match_the_code_objects():
    """The host launches a GEMV entry point with the argument convention and
    checks the role it reads from the kernel's name (a kernel picked for one
    form must never run as another).  For every entry point in the GEMV code
    objects, that parse must agree with the compiled kernel: one 88-byte
    GemvArgs block (the batch kernel: its own block), or the plain GEMV's six
    arguments; and the name families map to their roles."""
    gemv_args_bytes = 88  # sizeof(GemvArgsHost) in zlm_gpu_hip.cpp
    families = {"multi_": 16, "tok2_": 17, "q8tok": 18, "pair_": 1, "norm_": 2, "normpair_": 3, "resid_": 4}
    seen = 0
    for q in ("q4_0", "q8_0", "q4_k", "q6_k", "q4_1", "f32", "f16", "bf16"):
        path = os.path.join(zd.LIB_DIR, f"zlm_gemv_{q}_gfx950.hsaco")
        for name, sizes in _kernel_args(path).items():
            conv = zd.kernel_convention(name)
            assert conv is not None, name
            role, struct_args = conv
            rest = name[len(f"zlm_gemv_{q}_"):]
            want_role = next((r for p, r in families.items() if rest.startswith(p)), 0)
            assert role == want_role, (name, role)
            if struct_args:
                assert len(sizes) == 1, (name, sizes)
                if role != 16:
                    assert sizes == [gemv_args_bytes], (name, sizes)
            else:
                assert sizes == [8, 8, 8, 8, 4, 4], (name, sizes)
            seen += 1
    assert seen > 300
    assert zd.kernel_convention("zlm_attn_decode") is None
