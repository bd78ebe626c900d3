"""CPU oracle for the WUSH INT4 W4A4 path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg import this package, and only as the checker.  The product
(``wush_int4_kernel_amd`` and the ``my_int4`` package) never imports, links or
calls it: those fail loudly when the HIP library is missing.

Two independent restatements of the reference semantics live here:

* ``wush_oracle.c`` (built by ``oracle/Makefile`` into ``oracle/_build/``),
  reached through :mod:`ctypes` -- the fast checker used by the GPU tests;
* the numpy functions in :mod:`oracle.rtn_np` -- written separately from the C
  code so the two can be compared bit for bit;
* :mod:`oracle.rtn_torch` -- the reference's eager torch CPU ops, checked bit
  for bit against the C code; ``bench.py``'s ``cpu_baseline`` leg times it.

Reference semantics followed (paths relative to the reference repo root):
``my_int4/rtn_int4.py:15-75`` (quant / dequant / matmul),
``csrc/quant_int4.cu:59-100`` (operation order, rounding),
``tests/test_sw2.py:12-24`` and ``csrc/fused_tq_int4.cu:38-84`` (transform),
``csrc/gemm_int4.cu:63-82`` (group-int-then-scale GEMM formula),
``tests/test_p12.py:21-26`` (per-tensor quant mirror).

How each function is pinned (closed forms, the reference tests' known answers,
an exact-rational fp32 emulation, brute force) is listed in
``tests/test_oracle_pinning.py``; ``oracle_transform`` / ``fused_tq`` are
pinned by permutation / diagonal / identity transforms, the GEMM pieces by
brute-force integer products.  The oracle has no WUSH T solve: the
reference builds T with an un-vendored third-party module, and the product
side's own closed form (``wush_int4_kernel_amd.wush_transform``) is parity
unpinned beyond the invariants in ``tests/test_transform_invariants.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import rtn_np  # noqa: F401  (re-exported restatement)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build(verbose: bool = False) -> str:
    """Compile ``wush_oracle.c`` with ``make`` into ``oracle/_build``."""
    out = subprocess.run(["make", "-s", "-C", _HERE], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if verbose and out.stdout:
        print(out.stdout)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """The C oracle, building it on first use if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, f32, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        sig = {
            "oracle_quant_f32": [p, p, p, i64],
            "oracle_quant_bf16": [p, p, p, i64],
            "oracle_quant_f16": [p, p, p, i64],
            "oracle_transform_bf16": [p, p, p, i64, i64],
            "oracle_fused_tq_bf16": [p, p, p, p, i64, i64],
            "oracle_dequant": [p, p, p, i64],
            "oracle_group_dots": [p, p, p, i64, i64, i64],
            "oracle_gemm_f64": [p, p, p, p, p, i64, i64, i64],
            "oracle_quant_tensor_scale_bf16": [p, p, i64, f32],
            "oracle_gemm_tensor_scale_f64": [p, p, f64, p, i64, i64, i64],
            "oracle_int_matmul_8x32x8": [p, p, p],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- bit helpers
def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = (((u[nan] >> 16) & 0x8000) | 0x7FC0).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------ C-backed API
def quant(x: np.ndarray, dtype: str = "f32"):
    """rtn_int4.quant_int4: x (..., K) -> (q uint8 (..., K/2), s bf16-bits uint16 (..., K/32)).

    ``dtype`` names how ``x`` is stored: "f32" (float32 array), "bf16" or
    "f16" (uint16 bit patterns)."""
    x = np.ascontiguousarray(x)
    K = x.shape[-1]
    assert K % 32 == 0
    n_groups = x.size // 32
    q = np.empty(x.shape[:-1] + (K // 2,), np.uint8)
    s = np.empty(x.shape[:-1] + (K // 32,), np.uint16)
    if dtype == "f32":
        x = np.ascontiguousarray(x, dtype=np.float32)
        lib().oracle_quant_f32(_ptr(x), _ptr(q), _ptr(s), n_groups)
    elif dtype == "bf16":
        assert x.dtype == np.uint16
        lib().oracle_quant_bf16(_ptr(x), _ptr(q), _ptr(s), n_groups)
    elif dtype == "f16":
        assert x.dtype in (np.uint16, np.float16)
        x = x.view(np.uint16)
        lib().oracle_quant_f16(_ptr(x), _ptr(q), _ptr(s), n_groups)
    else:
        raise ValueError(dtype)
    return q, s


def transform(x_bf16: np.ndarray, t_bf16: np.ndarray) -> np.ndarray:
    """x' = X T^T per 32-block in fp32, i ascending, mul then add (test_sw2.py:12-24)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    t = np.ascontiguousarray(t_bf16, dtype=np.uint16)
    K = x.shape[-1]
    rows = x.size // K
    assert t.shape == (K // 32, 32, 32)
    out = np.empty(x.shape, np.float32)
    lib().oracle_transform_bf16(_ptr(x), _ptr(t), _ptr(out), rows, K)
    return out


def fused_tq(x_bf16: np.ndarray, t_bf16: np.ndarray):
    """fused_transform_quant_int4 (fused_tq_int4.cu:27-85) on bf16 bit patterns."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    t = np.ascontiguousarray(t_bf16, dtype=np.uint16)
    K = x.shape[-1]
    rows = x.size // K
    assert t.shape == (K // 32, 32, 32)
    q = np.empty(x.shape[:-1] + (K // 2,), np.uint8)
    s = np.empty(x.shape[:-1] + (K // 32,), np.uint16)
    lib().oracle_fused_tq_bf16(_ptr(x), _ptr(t), _ptr(q), _ptr(s), rows, K)
    return q, s


def dequant(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """dequant_int4 (rtn_int4.py:58-68) -> fp32 (..., K)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    out = np.empty(q.shape[:-1] + (q.shape[-1] * 2,), np.float32)
    lib().oracle_dequant(_ptr(q), _ptr(s), _ptr(out), s.size)
    return out


def group_dots(xq: np.ndarray, wq: np.ndarray) -> np.ndarray:
    """Exact int32 D[m, n, g] = sum_{k in g} qx*qw."""
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1, xq.shape[-1])
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    M, K2 = xq.shape
    N = wq.shape[0]
    D = np.empty((M, N, K2 // 16), np.int32)
    lib().oracle_group_dots(_ptr(xq), _ptr(wq), _ptr(D), M, N, 2 * K2)
    return D


def gemm_f64(xq, xs, wq, ws) -> np.ndarray:
    """fp64 value of dequant(xq,xs) @ dequant(wq,ws)^T (test_p13.py:22)."""
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1, xq.shape[-1])
    xs = np.ascontiguousarray(xs, dtype=np.uint16).reshape(xq.shape[0], -1)
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.uint16)
    M, K2 = xq.shape
    N = wq.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().oracle_gemm_f64(_ptr(xq), _ptr(xs), _ptr(wq), _ptr(ws), _ptr(Y), M, N, 2 * K2)
    return Y


def quant_tensor_scale(x_bf16: np.ndarray, inv_scale) -> np.ndarray:
    """Per-tensor quant mirror (test_p12.py:21-26): flat packed uint8 (numel/2)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1)
    q = np.empty(x.size // 2, np.uint8)
    lib().oracle_quant_tensor_scale_bf16(_ptr(x), _ptr(q), x.size, float(np.float32(inv_scale)))
    return q


def gemm_tensor_scale_f64(xq, wq, alpha: float) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    N, K2 = wq.shape
    xq = np.ascontiguousarray(xq, dtype=np.uint8).reshape(-1, K2)
    M = xq.shape[0]
    Y = np.empty((M, N), np.float64)
    lib().oracle_gemm_tensor_scale_f64(_ptr(xq), _ptr(wq), float(alpha), _ptr(Y), M, N, 2 * K2)
    return Y


def int_matmul_8x32x8(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    assert a.shape == (8, 32) and b.shape == (32, 8)
    c = np.empty((8, 8), np.int32)
    lib().oracle_int_matmul_8x32x8(_ptr(a), _ptr(b), _ptr(c))
    return c
