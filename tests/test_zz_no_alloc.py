"""GPU test of wush_gemm_s4_noalloc, the entry point that allocates nothing
(split-K partials in the library's static per-device scratch).

It must give the same result as wush_gemm_s4 with a caller workspace of
wush_gemm_s4_workspace_bytes(M, N, K) bytes -- the same split of K and the
same kernels on these shapes (N < 8192: no activations converted into the
workspace), every kernel deterministic, so bit for bit -- on two calls in a
row, the second with a smaller input (the scratch keeps the first call's
contents), and reject a shape whose partials need more than
WUSH_GEMM_SCRATCH_BYTES.
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


def _both(capi, xq, xs, wq, ws):
    import torch
    M, N, K = xq.shape[0], wq.shape[0], 2 * xq.shape[1]
    dx, dxs, dw, dws = to_dev_u8(xq), to_dev_bf16(xs), to_dev_u8(wq), to_dev_bf16(ws)
    stream = torch.cuda.current_stream().cuda_stream
    need = capi.gemm_s4_workspace_bytes(M, N, K)
    work = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    y_ref = torch.empty(M, N, dtype=torch.float16, device="cuda")
    capi.gemm_s4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y_ref.data_ptr(), M, N, K,
                 work.data_ptr() if need else None, need, stream)
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    capi.gemm_s4_noalloc(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y.data_ptr(), M, N, K,
                         stream)
    torch.cuda.synchronize()
    return need, f16_tensor_f64(y), f16_tensor_f64(y_ref)


# (M, N, K): a K-split prefill plan that fills the scratch exactly (64 MiB),
# then a smaller K-split streaming plan; then a larger and a smaller decode plan
CASES = [[(512, 4096, 4096), (16, 2048, 16384)], [(8, 1024, 16384), (4, 512, 8192)]]


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


def test_noalloc_rejects_plans_beyond_scratch(capi):
    import torch
    M, N, K = 768, 4096, 8192           # fp16 tiles split K 8 ways (32 groups each): 96 MiB of partials
    need = capi.gemm_s4_workspace_bytes(M, N, K)
    assert need > capi.GEMM_SCRATCH_BYTES
    lib = capi.load()
    x = torch.zeros(M * K // 2, dtype=torch.uint8, device="cuda")
    s = torch.zeros(M * K // 32, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(N * K // 2, dtype=torch.uint8, device="cuda")
    ws = torch.zeros(N * K // 32, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(M * N, dtype=torch.float16, device="cuda")
    st = lib.wush_gemm_s4_noalloc(x.data_ptr(), s.data_ptr(), w.data_ptr(), ws.data_ptr(), y.data_ptr(),
                                  M, N, K, torch.cuda.current_stream().cuda_stream)
    assert st == capi.ERROR_SCRATCH_TOO_SMALL
    assert b"WUSH_GEMM_SCRATCH_BYTES" in lib.wush_error_string(st)
