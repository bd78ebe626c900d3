"""ctypes view of the C ABI in ``libwush_int4.so`` (``include/wush_int4.h``).

This is how a non-torch host (or a test) reaches the kernels: plain device
pointers, sizes and a HIP stream handle.  Every wrapper raises
``RuntimeError`` with the library's message on a non-zero status.  torch is
used by callers only for device memory and streams.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libwush_int4.so")

# Every symbol include/wush_int4.h declares, with its ctypes signature.
_P, _I64, _I, _F, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "wush_abi_version": ([], _I),
    "wush_init": ([], _I),
    "wush_error_string": ([_I], ctypes.c_char_p),
    "wush_quant_int4": ([_P, _I, _P, _P, _I64, _P], _I),
    "wush_fused_tq": ([_P, _P, _P, _P, _I64, _I64, _P], _I),
    "wush_fused_tq_transform32": ([_P, _P, _P, _I64, _P], _I),
    "wush_gemv_int4": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "wush_gemv_int4_supported": ([_I64, _I64, _I64], _I),
    "wush_gemm_s4_workspace_bytes": ([_I64, _I64, _I64], _SZ),
    "wush_gemm_s4": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "wush_gemm_s4_noalloc": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "wush_mfma_selftest": ([_P, _P, _P, _P], _I),
    "wush_quant_int4_tensor_scale": ([_P, _P, _I64, _F, _P, _P], _I),
    "wush_gemm_s4_tensor_scale": ([_P, _P, _P, _I64, _I64, _I64, _F, _P, _P], _I),
}

DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2
_lib = None


def load() -> ctypes.CDLL:
    """Load libwush_int4.so (torch, if imported first, supplies the HIP runtime)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is not built; run `python -m wush_int4_kernel_amd._build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def init() -> None:
    """Per-device one-time set-up (call before capturing entry points in a graph)."""
    _check(load().wush_init(), "wush_init")


def _check(status: int, op: str) -> None:
    if status != 0:
        msg = load().wush_error_string(status).decode()
        raise RuntimeError(f"{op}: {msg} (status {status})")


def quant_int4(x_ptr, dtype, q_ptr, s_ptr, n_groups, stream) -> None:
    _check(load().wush_quant_int4(x_ptr, dtype, q_ptr, s_ptr, n_groups, stream), "wush_quant_int4")


def fused_tq(x_ptr, t_ptr, q_ptr, s_ptr, rows, K, stream) -> None:
    _check(load().wush_fused_tq(x_ptr, t_ptr, q_ptr, s_ptr, rows, K, stream), "wush_fused_tq")


def gemv_int4(xq, xs, wq, ws, y, M, N, K, stream) -> None:
    _check(load().wush_gemv_int4(xq, xs, wq, ws, y, M, N, K, stream), "wush_gemv_int4")


def gemv_int4_supported(M, N, K) -> bool:
    return bool(load().wush_gemv_int4_supported(M, N, K))


def gemm_s4_workspace_bytes(M, N, K) -> int:
    return int(load().wush_gemm_s4_workspace_bytes(M, N, K))


def gemm_s4(xq, xs, wq, ws, y, M, N, K, workspace, workspace_bytes, stream) -> None:
    _check(load().wush_gemm_s4(xq, xs, wq, ws, y, M, N, K, workspace, workspace_bytes, stream),
           "wush_gemm_s4")


GEMM_SCRATCH_BYTES = 64 << 20          # WUSH_GEMM_SCRATCH_BYTES
ERROR_SCRATCH_TOO_SMALL = 0x57550001   # WUSH_ERROR_SCRATCH_TOO_SMALL


def gemm_s4_noalloc(xq, xs, wq, ws, y, M, N, K, stream) -> None:
    _check(load().wush_gemm_s4_noalloc(xq, xs, wq, ws, y, M, N, K, stream), "wush_gemm_s4_noalloc")


def fused_tq_transform32(x, t, xp, rows, stream) -> None:
    _check(load().wush_fused_tq_transform32(x, t, xp, rows, stream), "wush_fused_tq_transform32")


def mfma_selftest(a, b, c, stream) -> None:
    _check(load().wush_mfma_selftest(a, b, c, stream), "wush_mfma_selftest")


def quant_int4_tensor_scale(x, q, n, inv_scale, inv_scale_dev, stream) -> None:
    _check(load().wush_quant_int4_tensor_scale(x, q, n, inv_scale, inv_scale_dev, stream),
           "wush_quant_int4_tensor_scale")


def gemm_s4_tensor_scale(xq, wq, y, M, N, K, alpha, alpha_dev, stream) -> None:
    _check(load().wush_gemm_s4_tensor_scale(xq, wq, y, M, N, K, alpha, alpha_dev, stream),
           "wush_gemm_s4_tensor_scale")
