"""CPU checks of the native artefacts: the C-ABI library loads and exports
every symbol include/wush_int4.h declares; argument validation rejects bad
calls before any device work; the torch module exposes the reference's 16 ops
(reference csrc/bindings.cpp:28-68) and rejects CPU tensors like the
reference does.  No kernel is launched here (there is no GPU)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wush_int4.h")
INVALID = 1  # hipErrorInvalidValue

REFERENCE_OPS = [
    "quant_int4_tensor_scale", "quant_int4_tensor_scale_dev", "quant_int4", "w4a4_gemm",
    "w4a4_gemm_v1", "w4a4_gemm_cutlass", "w4a4_gemm_cutlass_dev", "w4a4_gemm_s4",
    "s4_atom_selftest", "w4a4_gemv", "w4a4_gemv_multi", "fused_transform_quant_int4_v3",
    "fused_transform_quant_int4_smallm", "fused_transform_quant_int4", "w4a4_gemm_v2",
    "fused_transform_quant_int4_wmma",
]


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(wush_[a-z0-9_]+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def capi():
    import torch  # noqa: F401
    from wush_int4_kernel_amd import capi as c
    c.load()
    return c


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for s in ["wush_quant_int4", "wush_fused_tq", "wush_gemv_int4", "wush_gemm_s4",
              "wush_gemm_s4_workspace_bytes", "wush_mfma_selftest", "wush_quant_int4_tensor_scale",
              "wush_gemm_s4_tensor_scale", "wush_abi_version", "wush_error_string",
              "wush_gemv_int4_supported"]:
        assert s in syms, s


def test_library_exports_every_declared_symbol(capi):
    lib = capi.load()
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(declared_symbols()) == set(capi.SIGNATURES)
    assert lib.wush_abi_version() == 1


def test_library_exports_no_undeclared_c_symbols():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(ROOT, "wush_int4_kernel_amd", "libwush_int4.so")],
                         capture_output=True, text=True).stdout
    exported = sorted(set(re.findall(r" T (wush_[a-z0-9_]+)$", out, re.M)))
    assert exported == declared_symbols()


def test_argument_validation_without_device(capi):
    lib = capi.load()
    P = ctypes.c_void_p
    # empty work succeeds without touching the device
    assert lib.wush_quant_int4(None, 0, None, None, 0, None) == 0
    assert lib.wush_fused_tq(None, None, None, None, 0, 32, None) == 0
    assert lib.wush_gemm_s4(None, None, None, None, None, 0, 8, 64, None, 0, None) == 0
    # bad arguments are rejected before any launch
    assert lib.wush_quant_int4(None, 0, None, None, 4, None) == INVALID
    assert lib.wush_quant_int4(P(16), 9, P(16), P(16), 4, None) == INVALID       # dtype
    assert lib.wush_quant_int4(P(8), 0, P(16), P(16), 4, None) == INVALID        # misaligned x
    assert lib.wush_fused_tq(P(16), P(16), P(16), P(16), 1, 48, None) == INVALID  # K % 32
    assert lib.wush_gemv_int4(P(16), P(16), P(16), P(16), P(16), 9, 4, 64, None) == INVALID  # M > 8
    assert lib.wush_gemv_int4(P(16), P(16), P(16), P(16), P(16), 8, 4, 1 << 20, None) == INVALID  # LDS
    assert lib.wush_gemm_s4(P(16), P(16), P(16), P(16), P(16), 4, 4, 40, None, 0, None) == INVALID
    assert lib.wush_gemm_s4_tensor_scale(P(16), P(16), P(16), 4, 4, 1 << 21, 1.0, None, None) == INVALID
    # int32 bound of the per-tensor GEMM: 256 * 64 * K < 2^31 for K <= 131040
    assert 256 * 64 * 131040 < 2 ** 31 <= 256 * 64 * (131040 + 32)
    assert lib.wush_gemm_s4_tensor_scale(P(16), P(16), P(16), 4, 4, 131040 + 32, 1.0, None, None) == INVALID
    assert lib.wush_gemm_s4_tensor_scale(P(16), P(16), P(16), 0, 4, 131040, 1.0, None, None) == 0  # empty, valid
    assert lib.wush_quant_int4_tensor_scale(P(16), P(16), 40, 1.0, None, None) == INVALID
    assert lib.wush_mfma_selftest(None, None, None, None) == INVALID
    assert b"invalid argument" in lib.wush_error_string(INVALID)


def test_workspace_plan_is_host_only(capi):
    # split-K across workgroups only for skinny shapes with few row blocks and
    # a long K (each wavefront of the in-workgroup K split keeps >= 2 stages)
    assert capi.gemm_s4_workspace_bytes(8, 1024, 16384) > 0
    assert capi.gemm_s4_workspace_bytes(8, 4096, 4096) == 0
    assert capi.gemm_s4_workspace_bytes(4096, 4096, 4096) == 0
    assert capi.gemm_s4_workspace_bytes(0, 4096, 4096) == 0
    assert capi.gemm_s4_workspace_bytes(8, 4096, 40) == 0


def test_torch_module_exposes_reference_ops():
    from my_int4 import _C
    import my_int4
    from wush_int4_kernel_amd import _C as C2
    for op in REFERENCE_OPS:
        assert callable(getattr(_C, op)), op
        assert getattr(_C, op) is getattr(C2, op)
    assert my_int4.quant_int4 is C2.quant_int4
    assert _C.abi_version() == 1


def test_torch_ops_reject_cpu_tensors():
    import torch
    from my_int4 import _C
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA"):
        _C.quant_int4(x)
    with pytest.raises(RuntimeError, match="CUDA"):
        _C.fused_transform_quant_int4(x, torch.zeros(2, 32, 32, dtype=torch.bfloat16))
    q = torch.zeros(4, 32, dtype=torch.uint8)
    s = torch.zeros(4, 2, dtype=torch.bfloat16)
    for op in ["w4a4_gemm_s4", "w4a4_gemv_multi", "w4a4_gemm", "w4a4_gemm_v1", "w4a4_gemm_v2"]:
        with pytest.raises(RuntimeError, match="CUDA"):
            getattr(_C, op)(q, s, q, s)
    with pytest.raises(RuntimeError, match="CUDA"):
        _C.w4a4_gemm_cutlass(q, q, 1.0)


def test_reference_python_modules_exposed():
    # reference my_int4/rtn_int4.py and my_int4/wush_transform.py: same names
    # and parameters; rtn_int4's quant/product refuse CPU tensors (no CPU path)
    import inspect
    import torch
    from my_int4 import rtn_int4, wush_transform
    assert list(inspect.signature(rtn_int4.quant_int4).parameters) == ["x", "group_size"]
    assert list(inspect.signature(rtn_int4.dequant_int4).parameters) == ["q_byte", "scale", "group_size"]
    assert list(inspect.signature(rtn_int4.w4a4_matmul_reference).parameters) == ["x_q", "x_s", "w_q", "w_s"]
    for name in ("compute_wush_transform", "transform_weights", "transform_activations_reference"):
        assert callable(getattr(wush_transform, name))
    assert list(inspect.signature(wush_transform.compute_wush_transform).parameters)[:4] == \
        ["X_cal", "W", "group_size", "use_hadamard"]
    with pytest.raises(RuntimeError, match="GPU"):
        rtn_int4.quant_int4(torch.zeros(2, 64, dtype=torch.bfloat16))
    # dequant decodes the packed format: byte 0xD3 = codes (+3, -3), scale 0.5
    q = torch.tensor([[0xD3] * 16], dtype=torch.uint8)
    s = torch.tensor([[0.5]], dtype=torch.bfloat16)
    d = rtn_int4.dequant_int4(q, s)
    assert d.shape == (1, 32) and d[0, 0].item() == 1.5 and d[0, 1].item() == -1.5


def test_tuning_defines_parsing(monkeypatch):
    # WUSH_DEFINES becomes -D flags on the hipcc lines; only WUSH_* names with
    # plain values pass, so the variable cannot smuggle other compiler flags in
    from wush_int4_kernel_amd import _build

    monkeypatch.setenv("WUSH_DEFINES", "WUSH_TQ_SMALLM_PAIRS=0  WUSH_GEMV_WAVES=8 WUSH_X")
    assert _build.tuning_defines() == ["-DWUSH_TQ_SMALLM_PAIRS=0", "-DWUSH_GEMV_WAVES=8", "-DWUSH_X"]
    monkeypatch.delenv("WUSH_DEFINES")
    assert _build.tuning_defines() == []
    for bad in ("-fsanitize=address", "WUSH_A=1;rm", "OTHER=1", "WUSH_A=$(x)", "wush_a=1"):
        monkeypatch.setenv("WUSH_DEFINES", bad)
        with pytest.raises(ValueError):
            _build.tuning_defines()


# (M, N, K) on both sides of every term of the GEMV shape rule: the staged
# kernel's 64 KiB LDS limit, the K-split kernel's M, N and K bounds
GEMV_RULE_SHAPES = [(M, N, K) for M in (1, 4, 6, 7, 8, 9) for N in (4096, 32768, 32769, 57344)
                    for K in (4096, 8192, 16384, 32768, 34816, 65536)] + [(0, 4096, 4096), (8, 57344, 8200)]


def _check_gemv_rule(lib):
    """wush_gemv_int4 rejects (before touching a device) exactly the shapes
    wush_gemv_int4_supported reports as unsupported; returns the supported set."""
    P = ctypes.c_void_p
    lib.wush_gemv_int4_supported.argtypes = [ctypes.c_int64] * 3
    lib.wush_gemv_int4.argtypes = [P] * 5 + [ctypes.c_int64] * 3 + [P]
    ok = set()
    for M, N, K in GEMV_RULE_SHAPES:
        sup = lib.wush_gemv_int4_supported(M, N, K)
        st = lib.wush_gemv_int4(P(16), P(16), P(16), P(16), P(16), M, N, K, None)
        assert sup in (0, 1)
        assert (st == INVALID) == (sup == 0), (M, N, K, sup, st)
        if sup:
            ok.add((M, N, K))
    return ok


def test_gemv_rule_is_the_librarys(capi, tmp_path):
    # The _C product ops route to wush_gemv_int4 only where the library says
    # it runs the shape (bindings.cpp asks wush_gemv_int4_supported), so a
    # build with other tuning macros cannot send a shape the GEMV rejects.
    # Default build: the K-split kernel takes M = 7, 8 at L70 and K = 16384.
    default = _check_gemv_rule(capi.load())
    assert (8, 57344, 8192) in default and (8, 57344, 16384) in default and (7, 32769, 32768) in default
    assert (8, 32768, 16384) not in default and (6, 57344, 16384) not in default
    assert (1, 4096, 65536) in default and (4, 4096, 16384) in default and (6, 4096, 16384) not in default
    # A build with the K-split kernel off (WUSH_GEMV_KS_MIN_M=9, the documented
    # off value) keeps only the LDS-staged shapes.
    from wush_int4_kernel_amd import _build
    lib_path = str(tmp_path / "libwush_int4_ks_off.so")
    _build.build_capi(lib_path=lib_path, build_dir=str(tmp_path / "obj"), defines="WUSH_GEMV_KS_MIN_M=9")
    off = _check_gemv_rule(ctypes.CDLL(lib_path))
    assert (8, 57344, 16384) not in off and (7, 57344, 32768) not in off and (7, 57344, 8192) in off
    assert off == {s for s in default if s[0] * (s[2] // 2) + s[0] * (s[2] // 32) * 8 <= 64 * 1024}
