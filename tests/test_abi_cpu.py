"""The C-ABI library loads, exports every symbol include/mer_hip.h declares,
and its host-only sizing / validation agrees with the oracle.  CPU only:
nothing here launches GPU work."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mer_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mer_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_surface():
    names = declared_functions()
    for must in ("mer_hip_init", "mer_hip_expert_forward", "mer_hip_moe_forward", "mer_hip_dequantize",
                 "mer_hip_q4_0_matvec", "mer_expert_weight_bytes"):
        assert must in names


def test_library_exports_every_declared_symbol(mer):
    lib = mer._lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers exactly the declared set
    assert sorted(mer._lib.SIGNATURES) == declared_functions()


def test_abi_version(mer):
    assert mer._lib.lib().mer_hip_abi_version() == 1


def test_uninitialised_calls_fail_cleanly(mer):
    lib = mer._lib.lib()
    rc = lib.mer_hip_expert_forward(4, None, 0, None, 0, 32, 32, None, 0, None)
    assert rc == mer._lib.Status.NOT_INITIALIZED
    assert b"mer_hip_init" in lib.mer_last_error()
    h = ctypes.c_void_p()
    assert lib.mer_slot_cache_create(4, 64, 64, 2, 4, ctypes.byref(h)) == mer._lib.Status.NOT_INITIALIZED
    assert h.value is None
    # null handles are rejected before any device work
    assert lib.mer_slot_cache_prepare(None, None, None, None, 0, None) == mer._lib.Status.INVALID_LAYOUT
    assert lib.mer_slot_cache_table(None) is None
    assert lib.mer_slot_cache_destroy(None) == 0


@pytest.mark.parametrize("dtype,dm,dff", [(4, 8, 8), (4, 10, 10), (5, 8, 8), (4, 4096, 14336), (4, 7168, 2048),
                                          (5, 2048, 768), (5, 37, 45), (4, 0, 5)])
def test_expert_weight_bytes_matches_oracle(mer, oracle, dtype, dm, dff):
    assert mer.expert_weight_bytes_for(dm, dff, mer.WeightDtype(dtype)) == oracle.expert_weight_bytes(dtype, dm, dff)


def test_expert_weight_bytes_saturates(mer):
    assert mer.expert_weight_bytes_for(2**63, 2**63, mer.WeightDtype.Q4_0) == 2**64 - 1


def _status(mer, fn):
    try:
        fn()
    except mer.ExpertWeightsError as e:
        return int(e.status), e
    return 0, None


def test_q8_validation_matches_oracle(mer, oracle):
    cases = [
        (0, 0, 0, 0, 2), (10, 31, 32, 32, 32), (0, 2**63, 2**63, 2**63, 2),
    ]
    need = oracle.expert_weight_bytes(5, 32, 64)
    cases += [(need - 1, 32, 32, 32, 64), (need, 32, 32, 32, 64), (need + 7, 32, 32, 32, 64)]
    small = oracle.expert_weight_bytes(5, 32, 32)
    cases += [(small - 1, 32, 32, 32, 32)]
    for length, xl, yl, dm, dff in cases:
        st, _ = _status(mer, lambda: mer.validate_expert(mer.WeightDtype.Q8_0, length, xl, yl, dm, dff))
        assert st == oracle.validate_q8_direct(length, xl, yl, dm, dff), (length, xl, yl, dm, dff)


def test_q4_validation_matches_oracle_and_reports_fields(mer, oracle):
    dm, dff = 4096, 14336
    need = oracle.expert_weight_bytes(4, dm, dff)
    for length in (need, need + 1, need - 1, need - 4096, need - 4097, 0):
        st, err = _status(mer, lambda: mer.validate_expert(mer.WeightDtype.Q4_0, length, dm, dm, dm, dff))
        assert st == oracle.validate_q4_0(length, dm, dff), length
        if st in (1, 5):
            assert (err.have, err.need, err.d_model, err.d_ff) == (length, need, dm, dff)
    # x length mismatch is the Candle shape error of forward_candle
    st, _ = _status(mer, lambda: mer.validate_expert(mer.WeightDtype.Q4_0, need, dm - 1, dm, dm, dff))
    assert st == mer._lib.Status.COMPUTE
    assert isinstance(_status(mer, lambda: mer.validate_expert(mer.WeightDtype.Q4_0, 107, 8, 8, 8, 8))[1],
                      mer.BufferTooSmall)
    assert isinstance(
        _status(mer, lambda: mer.validate_expert(mer.WeightDtype.Q4_0, need - 10, dm, dm, dm, dff))[1],
        mer.TruncatedPayload)


def test_gpu_compatibility_rule(mer):
    mer.routed_expert_gpu_compatibility(mer.WeightDtype.Q4_0, 4096, 14336)
    mer.routed_expert_gpu_compatibility(mer.WeightDtype.Q8_0, 2048, 768)
    mer.routed_expert_gpu_compatibility(mer.WeightDtype.Q4_0, 16384, 16384)
    with pytest.raises(mer.RoutedExpertGpuIncompatibility):
        mer.routed_expert_gpu_compatibility(mer.WeightDtype.Q4_0, 16385, 32)
    with pytest.raises(mer.RoutedExpertGpuIncompatibility):
        mer._lib.lib().mer_routed_expert_gpu_compatibility(3, 32, 32) and mer.errors.raise_for_status(
            mer._lib.lib().mer_routed_expert_gpu_compatibility(3, 32, 32))


def test_dispatch_error_kind_names(mer):
    k = mer.GpuExpertDispatchErrorKind
    assert str(k.ResidencyMiss) == "residency-miss" and str(k.DeviceLost) == "device-lost"
    assert int(k.ResidencyMiss.value) == 16


def test_product_package_does_not_reference_oracle():
    pkg = os.path.join(ROOT, "micro-expert-router-ssd-streamed-moe-mer_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "mer_oracle" not in text and "oracle/" not in text, f


def test_output_digest_matches_oracle_and_hand_case(mer, oracle):
    """mer_output_digest = summarise_output (inference.rs:3087-3106): equal to
    the oracle's (pinned by its closed form) on random, signed-zero and
    non-finite vectors, and on y = [1.0] worked by hand: one xor of the bit
    pattern 0x3f800000 into the seed, one multiplication by the FNV prime."""
    import numpy as np

    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(4096).astype(np.float32), np.array([-0.0, 0.0, np.inf, -np.inf, np.nan], np.float32),
             np.zeros(0, np.float32)]
    for i, y in enumerate(cases):
        got = mer.summarise_output(7 + i, 3 * i, y)
        want = oracle.output_digest(7 + i, 3 * i, y)
        assert got[0] == want[0]
        assert (np.isnan(got[1]) and np.isnan(want[1])) or got[1] == want[1]
    d, norm = mer.summarise_output(2, 5, np.array([1.0], np.float32))
    assert d == (((0xCBF29CE484222325 ^ 2 ^ 5) ^ 0x3F800000) * 0x100000001B3) % (1 << 64)
    assert norm == 1.0


def test_join_u32_does_not_sign_extend(tmp_path):
    """The kernels rebuild 64-bit values (launch epochs, blob pointers) from
    two halves taken through __builtin_amdgcn_readfirstlane, which returns
    int; mer::join_u32 takes the halves as uint32_t, so a low half with bit
    31 set stays in the low 32 bits.  The helper is __host__ __device__ and
    is checked here in a host build."""
    import shutil
    import subprocess

    hipcc = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else shutil.which("hipcc")
    if not hipcc:
        pytest.skip("hipcc not available")
    src = tmp_path / "join.hip"
    src.write_text(
        '#include "mer_device.hpp"\n'
        "#include <stdio.h>\n"
        "int main() {\n"
        "  const int lo = (int)0x80000001u;  // what readfirstlane hands back\n"
        "  const unsigned long long v = mer::join_u32(0x12345678u, (uint32_t)lo);\n"
        "  static_assert(mer::join_u32(1u, 0x80000000u) == 0x180000000ull, \"join\");\n"
        '  printf("%llx\\n", v);\n'
        "  return v == 0x1234567880000001ull ? 0 : 1;\n"
        "}\n")
    exe = tmp_path / "join"
    csrc = os.path.join(ROOT, "micro-expert-router-ssd-streamed-moe-mer_amd", "csrc")
    r = subprocess.run([hipcc, "-std=c++17", "--offload-arch=gfx950", "-I", csrc, str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "1234567880000001", out.stdout


def test_header_is_plain_c_and_links_from_c(mer, tmp_path):
    """include/mer_hip.h compiles as strict C99 and C++11, and a C program
    links against libmer_hip.so and calls its host-only entry points (what a
    cgo / FFI binding does): the byte size of a Mixtral Q4_0 expert, the
    ABI version, and a refused call before mer_hip_init."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    inc = os.path.join(ROOT, "include")
    libdir = os.path.dirname(mer._lib.LIB_PATH)
    src = tmp_path / "use.c"
    src.write_text(
        '#include "mer_hip.h"\n'
        "#include <stdio.h>\n"
        "int main(void) {\n"
        "  size_t n = mer_expert_weight_bytes(MER_DTYPE_Q4_0, 4096, 14336);\n"
        "  int rc = mer_hip_expert_forward_qmm(NULL, 0, NULL, 0, 4096, 14336, NULL, 0, NULL);\n"
        '  printf("%zu %d %d\\n", n, mer_hip_abi_version(), rc);\n'
        "  return n == 99090432u && rc == MER_ERR_NOT_INITIALIZED ? 0 : 1;\n"
        "}\n")
    for std in (["-std=c99"], ["-x", "c++", "-std=c++11"]):
        r = subprocess.run([gcc, *std, "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", inc, "-c", str(src),
                            "-o", str(tmp_path / "use.o")], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
    exe = tmp_path / "use"
    r = subprocess.run([gcc, "-std=c99", "-I", inc, str(src), "-o", str(exe), "-L", libdir, "-lmer_hip",
                        f"-Wl,-rpath,{libdir}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.split()[:2] == ["99090432", "1"]
