"""GPU test of wush_gemm_s4_noalloc, the entry point that allocates nothing
(split-K partials in the library's static per-device scratch).

It must give the same result as wush_gemm_s4 with a caller workspace of
WUSH_GEMM_SCRATCH_BYTES -- the plan the no-alloc entry point runs -- bit for
bit (every kernel is deterministic): on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents); on a shape whose
partials fill the scratch exactly; and on a shape whose full split of K would
need more partials than the scratch holds, which then runs fewer K slices.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from _util import f16_tensor_f64, outlier_activations, rel_fro, rng, to_dev_bf16, to_dev_u8

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def capi():
    import torch  # noqa: F401  (HIP runtime first)
    from wush_int4_kernel_amd import capi as c
    c.load()
    c.init()
    return c


def _operands(g, M, N, K):
    from _util import f32_to_bf16_bits
    xq, xs = oracle.quant(outlier_activations(g, M, K), "bf16")
    wq, ws = oracle.quant(f32_to_bf16_bits(g.standard_normal((N, K)) * 0.02), "bf16")
    return xq, xs, wq, ws


def _both(capi, xq, xs, wq, ws, ws_cap=None):
    """y of wush_gemm_s4_noalloc and of wush_gemm_s4 with a workspace of
    min(its full need, ws_cap) bytes; returns (full need, y, y_ref)."""
    import torch
    M, N, K = xq.shape[0], wq.shape[0], 2 * xq.shape[1]
    dx, dxs, dw, dws = to_dev_u8(xq), to_dev_bf16(xs), to_dev_u8(wq), to_dev_bf16(ws)
    stream = torch.cuda.current_stream().cuda_stream
    need = capi.gemm_s4_workspace_bytes(M, N, K)
    wsb = need if ws_cap is None else min(need, ws_cap)
    work = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    y_ref = torch.empty(M, N, dtype=torch.float16, device="cuda")
    capi.gemm_s4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y_ref.data_ptr(), M, N, K,
                 work.data_ptr() if wsb else None, wsb, stream)
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    capi.gemm_s4_noalloc(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y.data_ptr(), M, N, K,
                         stream)
    torch.cuda.synchronize()
    return need, f16_tensor_f64(y), f16_tensor_f64(y_ref)


# (M, N, K): a K-split prefill plan whose partials fill the scratch exactly
# (4 slices of M*N fp32 = 64 MiB), then a smaller K-split streaming plan; then
# a larger and a smaller decode plan
CASES = [[(1024, 4096, 4096), (16, 2048, 16384)], [(8, 1024, 16384), (4, 512, 8192)]]


@pytest.mark.parametrize("pair", CASES)
def test_noalloc_matches_workspace_entry_point(capi, pair):
    g = rng(9100 + pair[0][0])
    needs = []
    for M, N, K in pair:
        xq, xs, wq, ws = _operands(g, M, N, K)
        need, y, y_ref = _both(capi, xq, xs, wq, ws)
        needs.append(need)
        assert need <= capi.GEMM_SCRATCH_BYTES
        assert np.array_equal(y, y_ref), (M, N, K)
        rows = np.arange(0, M, max(1, M // 16))
        ref = oracle.gemm_f64(xq[rows], xs[rows], wq, ws)
        assert rel_fro(y[rows], ref) < 2e-3
    assert needs[0] > needs[1] > 0      # both calls split K; the second uses less scratch
    if pair[0] == (1024, 4096, 4096):
        assert needs[0] == capi.GEMM_SCRATCH_BYTES


def test_noalloc_splits_less_beyond_scratch(capi):
    # fp16 tiles at 768 x 4096 x 8192 split K 8 ways (32 groups each) with a
    # full workspace: 96 MiB of partials.  Within the 64 MiB scratch the plan
    # takes fewer slices: the same as wush_gemm_s4 given 64 MiB of workspace.
    M, N, K = 768, 4096, 8192
    assert capi.gemm_s4_workspace_bytes(M, N, K) > capi.GEMM_SCRATCH_BYTES
    g = rng(9200)
    xq, xs, wq, ws = _operands(g, M, N, K)
    _, y, y_ref = _both(capi, xq, xs, wq, ws, ws_cap=capi.GEMM_SCRATCH_BYTES)
    assert np.array_equal(y, y_ref)
    rows = np.arange(0, M, 48)
    ref = oracle.gemm_f64(xq[rows], xs[rows], wq, ws)
    assert rel_fro(y[rows], ref) < 2e-3
    lib = capi.load()
    assert b"WUSH_GEMM_SCRATCH_BYTES" in lib.wush_error_string(capi.ERROR_SCRATCH_TOO_SMALL)
