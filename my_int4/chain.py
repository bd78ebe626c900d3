"""M-dispatched decode/prefill layer step and its graph capture.

The reference builds the layer step of its benchmarks with ``make_chain``
(bench/exp_p13_official.py:31-39) and captures it with ``graphed``
(:24-29); its tests check a replay against eager (tests/test_p13.py:45-66).
This module provides the same two helpers over ``my_int4._C`` so a caller
gets the reference's dispatch by M without copying benchmark code:

  M == 1       fused_transform_quant_int4_smallm -> w4a4_gemv       (y: (N,))
  M <= 4       fused_transform_quant_int4_smallm -> w4a4_gemv_multi (y: (M, N))
  M <= 32      fused_transform_quant_int4_smallm -> w4a4_gemm_s4
  otherwise    fused_transform_quant_int4_v3     -> w4a4_gemm_s4

Every op allocates its outputs with torch and launches on the current stream,
and none of them synchronizes or allocates device memory behind torch's back,
so the step can be captured in a CUDA (HIP) graph.  In this build every op is
deterministic (split-K partials are summed in a fixed order, no atomics), so a
replay equals the eager result bit for bit.
"""
from __future__ import annotations

from typing import Callable, Tuple

from my_int4 import _C

# (quantizer, product) op names per M range, bench/exp_p13_official.py:33-39
_ROUTES = (
    (1, "fused_transform_quant_int4_smallm", "w4a4_gemv"),
    (4, "fused_transform_quant_int4_smallm", "w4a4_gemv_multi"),
    (32, "fused_transform_quant_int4_smallm", "w4a4_gemm_s4"),
)
_PREFILL = ("fused_transform_quant_int4_v3", "w4a4_gemm_s4")


def route(M: int) -> Tuple[str, str]:
    """Names of the (transform+quant, product) ops make_chain uses for M rows."""
    if M < 1:
        raise ValueError(f"M must be >= 1, got {M}")
    for bound, quant_op, prod_op in _ROUTES:
        if M <= bound:
            return quant_op, prod_op
    return _PREFILL


def make_chain(X, T, wq, ws, M: int | None = None) -> Callable[[], "object"]:
    """The layer step y = W4A4(fused_tq(X, T), wq, ws) for X (M, K) bf16.

    Same contract as the reference's make_chain (bench/exp_p13_official.py:31-39):
    X bf16 (M, K), T bf16 (K/32, 32, 32), wq uint8 (N, K/2), ws bf16 (N, K/32);
    the returned callable computes and returns y (fp16; (N,) at M == 1,
    (M, N) otherwise)."""
    if M is None:
        M = X.shape[0] if X.dim() > 1 else 1
    quant_op, prod_op = (getattr(_C, n) for n in route(M))
    return lambda: prod_op(*quant_op(X, T), wq, ws)


def graphed(step: Callable[[], "object"], warmup: int = 3):
    """Capture ``step`` in a CUDA graph after ``warmup`` eager calls
    (bench/exp_p13_official.py:24-29).  Returns (graph, out): ``graph.replay()``
    recomputes ``out`` in place."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    return g, out
