"""The reference's own tests, restated against the drop-in ``my_int4._C``.

Each test follows a reference test script (tests/test_s2.py, test_sw2.py,
test_s3.py, test_p13.py, test_p12.py, test_sw3.py, test_final.py of the reference) with the
same inputs, shapes and gates; the truth values come from the CPU oracle
(the reference's rtn_int4 / ref_fused semantics) instead of the torch
reference, and inputs are drawn on the CPU (a GPU RNG stream would not
reproduce a CPU one).  The sigma-clip gates are bit-exact; GEMM gates are the
reference's max-abs < 5% of max|Y| plus the 2e-3 relative Frobenius bar.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from _util import (bf16_bits_to_f32, bf16_tensor_bits, f16_tensor_f64, f32_to_bf16_bits, rel_fro,
                   rng, to_dev_bf16)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from my_int4 import _C
    return _C


def _bf16(g, shape, scale=1.0):
    return f32_to_bf16_bits(g.standard_normal(shape) * scale)


def _check_quant(C, xb, name):
    import torch
    q, s = C.quant_int4(to_dev_bf16(xb))
    torch.cuda.synchronize()
    qo, so = oracle.quant(xb, "bf16")
    assert tuple(q.shape) == qo.shape, name
    assert s.numel() == so.size, name
    assert np.array_equal(q.cpu().numpy(), qo), name
    assert np.array_equal(bf16_tensor_bits(s).reshape(so.shape), so), name


def test_s2_quant_bit_exact(C):
    # reference tests/test_s2.py:23-36
    g = rng(0)
    _check_quant(C, _bf16(g, (4096, 32)), "random 4096 groups")
    _check_quant(C, _bf16(g, (2, 3, 96)), "3-D")
    _check_quant(C, np.zeros((4, 32), np.uint16), "zeros")
    _check_quant(C, _bf16(g, (1 << 17, 128)), "stress 2^24")
    x = np.zeros((2, 32), np.float32)
    x[0, :8] = [7.0, -7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5]
    x[1, :8] = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -6.5], np.float32) * np.float32(0.7)
    _check_quant(C, f32_to_bf16_bits(x), "ties")
    _check_quant(C, f32_to_bf16_bits(np.full((4, 32), 3.3e38, np.float32)), "overflow")


def _check_fused(C, xb, tb, name, fn="fused_transform_quant_int4"):
    import torch
    q, s = getattr(C, fn)(to_dev_bf16(xb), to_dev_bf16(tb))
    torch.cuda.synchronize()
    qo, so = oracle.fused_tq(xb, tb)
    assert q.numel() == qo.size and s.numel() == so.size, name
    assert np.array_equal(q.cpu().numpy().reshape(-1), qo.reshape(-1)), name
    assert np.array_equal(bf16_tensor_bits(s).reshape(-1), so.reshape(-1)), name


@pytest.mark.parametrize("fn", ["fused_transform_quant_int4", "fused_transform_quant_int4_smallm",
                                "fused_transform_quant_int4_v3", "fused_transform_quant_int4_wmma"])
def test_sw2_fused_bit_exact(C, fn):
    # reference tests/test_sw2.py:34-50, for every fused entry point
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform
    import torch
    g = rng(1)
    X = bf16_bits_to_f32(_bf16(g, (256, 128)))
    X[:, 5::32] *= 12.0
    xb = f32_to_bf16_bits(X)
    W = g.standard_normal((64, 128)).astype(np.float32)
    T = compute_wush_transform(torch.from_numpy(bf16_bits_to_f32(xb)).double(),
                               torch.from_numpy(W).double())
    tb = bf16_tensor_bits(T.to(torch.bfloat16))
    _check_fused(C, xb, tb, "WUSH T, 256 rows with outliers", fn)
    _check_fused(C, xb, _bf16(g, tb.shape), "random T", fn)
    _check_fused(C, _bf16(g, (2, 3, 96)), _bf16(g, (3, 32, 32)), "3-D", fn)
    _check_fused(C, np.zeros((4, 64), np.uint16), tb[:2].copy(), "zeros", fn)
    _check_fused(C, _bf16(g, (1 << 16, 64)), tb[:2].copy(), "stress 2^21", fn)


def test_s3_gemm_fp64_arbitration(C):
    # reference tests/test_s3.py:29-47 (w4a4_gemm; K=96 and K=32 cases included)
    import torch
    g = rng(2)
    for (M, N, K) in [(64, 96, 128), (1, 64, 128), (257, 33, 96), (8, 8, 32)]:
        xq, xs = C.quant_int4(to_dev_bf16(_bf16(g, (M, K))))
        wq, ws = C.quant_int4(to_dev_bf16(_bf16(g, (N, K))))
        for fn in ("w4a4_gemm", "w4a4_gemm_v1"):
            y = getattr(C, fn)(xq, xs, wq, ws)
            torch.cuda.synchronize()
            assert tuple(y.shape) == (M, N) and y.dtype == torch.float16
            ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq.cpu().numpy(), bf16_tensor_bits(ws))
            yy = f16_tensor_f64(y)
            assert np.abs(yy - ref).max() < 0.05 * max(1.0, np.abs(ref).max()), (fn, M, N, K)
            assert rel_fro(yy, ref) < 2e-3, (fn, M, N, K)
    X = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    xq, xs = C.quant_int4(X)
    wq, ws = C.quant_int4(to_dev_bf16(_bf16(g, (16, 64))))
    assert (C.w4a4_gemm(xq, xs, wq, ws) == 0).all()


def test_p13_gemm_s4_fp64_arbitration(C):
    # reference tests/test_p13.py:17-28 -- every dispatch branch
    import torch
    g = rng(3)
    for (M, N, K) in [(64, 96, 128), (1, 64, 64), (300, 500, 512), (130, 512, 4096), (8, 4096, 4096)]:
        xq, xs = C.quant_int4(to_dev_bf16(_bf16(g, (M, K))))
        wq, ws = C.quant_int4(to_dev_bf16(_bf16(g, (N, K))))
        for fn in ("w4a4_gemm_s4", "w4a4_gemm_v2"):
            y = getattr(C, fn)(xq, xs, wq, ws)
            torch.cuda.synchronize()
            ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq.cpu().numpy(), bf16_tensor_bits(ws))
            yy = f16_tensor_f64(y)
            assert np.abs(yy - ref).max() < 0.05 * max(1.0, np.abs(ref).max()), (fn, M, N, K)
            assert rel_fro(yy, ref) < 2e-3, (fn, M, N, K)


def test_p13_outlier_e2e_gate(C):
    # reference tests/test_p13.py:29-43: WUSH chain on outlier data <= 8.2%
    # relative Frobenius vs X W^T in fp64.
    import torch
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform, transform_weights
    g = rng(4)
    M, N, K, GT = 2048, 512, 4096, 32
    X = g.standard_normal((M, K)).astype(np.float32)
    X[:, 5::GT] *= 15.0
    W = g.standard_normal((N, K)).astype(np.float32)
    W[:, 12::GT] *= 8.0
    Xb = f32_to_bf16_bits(X)
    Wb = f32_to_bf16_bits(W)
    Xd = torch.from_numpy(bf16_bits_to_f32(Xb)).double()
    Wd = torch.from_numpy(bf16_bits_to_f32(Wb)).double()
    Yt = Xd @ Wd.T
    Xc = g.standard_normal((256, K)).astype(np.float32)
    Xc[:, 5::GT] *= 15.0
    T64 = compute_wush_transform(torch.from_numpy(Xc).double(), Wd)
    Ww = transform_weights(Wd, T64).to(torch.bfloat16).cuda().contiguous()
    wqw, wsw = C.quant_int4(Ww)
    xqw, xsw = C.fused_transform_quant_int4_v3(to_dev_bf16(Xb), T64.to(torch.bfloat16).cuda().contiguous())
    y = C.w4a4_gemm_s4(xqw, xsw, wqw, wsw).double().cpu()
    e = ((y - Yt).norm() / Yt.norm()).item()
    assert e <= 0.082, e


def test_sw3_wmma_chain_and_final_gate(C):
    # reference tests/test_sw3.py:11-38 and tests/test_final.py:61-77: the WMMA
    # fused entry point against v0 (code flips < 2%, scales within 1e-2; here
    # the same bit-exact kernel serves both, so no code flips at all), and the
    # WMMA chain with w4a4_gemm_v1 (T rounded to bf16 on both sides) and with
    # w4a4_gemm_v2 (weights transformed by the fp64 T) under 10% relative
    # Frobenius error against X W^T in fp64.
    import torch
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform, transform_weights
    g = rng(7)
    M, N, K, GT = 2048, 512, 4096, 32
    X = bf16_bits_to_f32(_bf16(g, (M, K)))
    W = bf16_bits_to_f32(_bf16(g, (N, K)))
    X[:, 5::GT] *= 15.0
    W[:, 12::GT] *= 8.0
    Xb, Wb = f32_to_bf16_bits(X), f32_to_bf16_bits(W)
    Xd = torch.from_numpy(bf16_bits_to_f32(Xb)).double()
    Wd = torch.from_numpy(bf16_bits_to_f32(Wb)).double()
    Xc = g.standard_normal((256, K)).astype(np.float32)
    Xc[:, 5::GT] *= 15.0
    T64 = compute_wush_transform(torch.from_numpy(Xc).double(), Wd)
    Tb = T64.to(torch.bfloat16).cuda().contiguous()
    Xg = to_dev_bf16(Xb)
    q0, s0 = C.fused_transform_quant_int4(Xg, Tb)
    q1, s1 = C.fused_transform_quant_int4_wmma(Xg, Tb)
    assert torch.equal(q0, q1) and torch.equal(s0, s1)
    Yt = Xd @ Wd.T
    for w_t, gemm in ((Tb.double().cpu(), "w4a4_gemm_v1"), (T64, "w4a4_gemm_v2")):
        Ww = transform_weights(Wd, w_t).to(torch.bfloat16).cuda().contiguous()
        wqw, wsw = C.quant_int4(Ww)
        y = getattr(C, gemm)(q1, s1, wqw, wsw).double().cpu()
        e = ((y - Yt).norm() / Yt.norm()).item()
        assert e < 0.10, (gemm, e)


def test_p13_graph_capture_replay(C):
    # reference tests/test_p13.py:45-66; our split-K reduction is deterministic,
    # so replay must equal eager bit for bit (stronger than the 0.5 gate).
    import torch
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform, transform_weights
    g = rng(5)
    M, N, K = 8, 4096, 4096
    X = to_dev_bf16(_bf16(g, (M, K)))
    W = torch.from_numpy(g.standard_normal((N, K)).astype(np.float32)).double()
    Xc = torch.from_numpy(g.standard_normal((256, K)).astype(np.float32)).double()
    T64 = compute_wush_transform(Xc, W)
    T = T64.to(torch.bfloat16).cuda().contiguous()
    wqw, wsw = C.quant_int4(transform_weights(W, T64).to(torch.bfloat16).cuda().contiguous())

    def step():
        a, b = C.fused_transform_quant_int4_smallm(X, T)
        return C.w4a4_gemm_s4(a, b, wqw, wsw)

    y0 = step().clone()
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out = step()
    for _ in range(3):
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0)
        step()                       # eager work between replays
        torch.cuda.synchronize()


def test_gemv_ops(C):
    # reference call shapes: w4a4_gemv returns (N,), gemv_multi (M, N)
    import torch
    g = rng(6)
    N, K = 1000, 4096
    wq, ws = C.quant_int4(to_dev_bf16(_bf16(g, (N, K), 0.02)))
    for M in (1, 3, 8):
        xq, xs = C.quant_int4(to_dev_bf16(_bf16(g, (M, K))))
        ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq.cpu().numpy(), bf16_tensor_bits(ws))
        y = C.w4a4_gemv_multi(xq, xs, wq, ws)
        assert tuple(y.shape) == (M, N)
        assert rel_fro(f16_tensor_f64(y), ref) < 2e-3
        if M == 1:
            y1 = C.w4a4_gemv(xq, xs, wq, ws)
            assert tuple(y1.shape) == (N,)
            assert torch.equal(y1, y[0])
    with pytest.raises(RuntimeError, match="1<=M<=8"):
        xq, xs = C.quant_int4(to_dev_bf16(_bf16(g, (9, K))))
        C.w4a4_gemv_multi(xq, xs, wq, ws)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 6, 7, 8])
def test_decode_ops_route_to_either_kernel(C, M):
    # w4a4_gemm_s4 and w4a4_gemv_multi run the dot8 GEMV at M <= 4, and at
    # 5 <= M <= 8 when N > 32768, if its LDS staging (M*K*3/4 bytes) fits in
    # 64 KiB; otherwise the K-split MFMA GEMM (N = 4096 and 32768 at M >= 5,
    # K = 16384 at M >= 6).  Either way the two ops give the same product
    # (checked on sampled columns against the oracle).
    import torch
    g = rng(60 + M)
    for N, K in [(4096, 4096), (32768, 8192), (40000, 4096), (1024, 16384)]:
        wq, ws = C.quant_int4(to_dev_bf16(_bf16(g, (N, K), 0.02)))
        xq, xs = C.quant_int4(to_dev_bf16(_bf16(g, (M, K))))
        cols = torch.from_numpy(np.sort(g.choice(N, size=512, replace=False))).cuda()
        ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq[cols].cpu().numpy(),
                              bf16_tensor_bits(ws[cols]))
        y1 = C.w4a4_gemm_s4(xq, xs, wq, ws)
        y2 = C.w4a4_gemv_multi(xq, xs, wq, ws)
        assert torch.equal(y1, y2), (M, N, K)
        assert rel_fro(f16_tensor_f64(y1[:, cols]), ref) < 2e-3, (M, N, K)


@pytest.mark.parametrize("M", [6, 7, 8])
def test_decode_ops_ksplit_large_k(C, M):
    # K = 16384, N > 32768: at M = 7, 8 both ops run the GEMV's K-split kernel
    # (activations in registers, no LDS staging limit), at M = 6 the GEMM
    # (the staged GEMV would need 72 KiB of LDS); random codes and scales
    import torch
    g = rng(90 + M)
    N, K = 32800, 16384
    wq = torch.from_numpy(g.integers(0, 256, (N, K // 2), dtype=np.uint8)).cuda()
    ws = torch.from_numpy(((g.integers(118, 122, (N, K // 32)) << 7) | g.integers(0, 128, (N, K // 32)))
                          .astype(np.int16)).cuda().view(torch.bfloat16)
    xq = torch.from_numpy(g.integers(0, 256, (M, K // 2), dtype=np.uint8)).cuda()
    xs = torch.from_numpy(((g.integers(124, 128, (M, K // 32)) << 7) | g.integers(0, 128, (M, K // 32)))
                          .astype(np.int16)).cuda().view(torch.bfloat16)
    cols = torch.from_numpy(np.sort(g.choice(N, size=512, replace=False))).cuda()
    ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq[cols].cpu().numpy(), bf16_tensor_bits(ws[cols]))
    y1 = C.w4a4_gemm_s4(xq, xs, wq, ws)
    y2 = C.w4a4_gemv_multi(xq, xs, wq, ws)
    assert torch.equal(y1, y2), M
    assert rel_fro(f16_tensor_f64(y1[:, cols]), ref) < 2e-3, M


def test_rtn_int4_module_on_gpu(C):
    # my_int4.rtn_int4 (reference my_int4/rtn_int4.py:33-75): quant_int4 is
    # the bit-exact kernel, dequant_int4 decodes like the oracle, and
    # w4a4_matmul_reference is the group-scaled product within the 2e-3 bar
    import torch
    from my_int4 import rtn_int4
    g = rng(8)
    xb = _bf16(g, (3, 5, 128))
    wb = _bf16(g, (96, 128), 0.02)
    xq, xs = rtn_int4.quant_int4(to_dev_bf16(xb))
    wq, ws = rtn_int4.quant_int4(to_dev_bf16(wb))
    qo, so = oracle.quant(xb, "bf16")
    assert np.array_equal(xq.cpu().numpy(), qo) and np.array_equal(bf16_tensor_bits(xs), so)
    d = rtn_int4.dequant_int4(xq, xs).cpu().numpy()
    assert np.array_equal(d.reshape(-1, 128), oracle.dequant(qo.reshape(-1, 64), so.reshape(-1, 4)).astype(np.float32))
    y = rtn_int4.w4a4_matmul_reference(xq, xs, wq, ws)
    assert tuple(y.shape) == (3, 5, 96) and y.dtype == torch.float16
    ref = oracle.gemm_f64(qo.reshape(-1, 64), so.reshape(-1, 4), wq.cpu().numpy(), bf16_tensor_bits(ws))
    assert rel_fro(f16_tensor_f64(y.reshape(-1, 96)), ref) < 2e-3


def test_s4_atom_selftest(C):
    import torch
    g = rng(7)
    a = g.integers(-8, 8, (8, 32)).astype(np.int8)
    b = g.integers(-8, 8, (32, 8)).astype(np.int8)
    c = C.s4_atom_selftest(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda())
    assert np.array_equal(c.cpu().numpy(), a.astype(np.int32) @ b.astype(np.int32))


def test_p12_per_tensor_route(C):
    # reference tests/test_p12.py:43-69 (bit mirror), :94-105 (fp64), :142-152 (graph)
    import torch
    g = rng(8)
    for shape in [(1, 4096), (64, 4096), (2048, 512), (96,), (2, 4112)]:
        xb = _bf16(g, shape)
        amax = max(float(np.abs(bf16_bits_to_f32(xb)).max()), 1e-8)
        sx = amax / 7.0
        q = C.quant_int4_tensor_scale(to_dev_bf16(xb), sx)
        qo = oracle.quant_tensor_scale(xb, np.float32(1.0 / sx))
        assert np.array_equal(q.cpu().numpy(), qo), shape
    for (M, N, K) in [(64, 96, 128), (1, 256, 64), (300, 500, 512), (8, 4096, 4096)]:
        X = to_dev_bf16(_bf16(g, (M, K)))
        W = to_dev_bf16(_bf16(g, (N, K)))
        sx = X.float().abs().max().item() / 7.0
        sw = W.float().abs().max().item() / 7.0
        xq = C.quant_int4_tensor_scale(X, sx)
        wq = C.quant_int4_tensor_scale(W, sw).view(N, -1)
        y = C.w4a4_gemm_cutlass(xq, wq, sx * sw)
        ref = oracle.gemm_tensor_scale_f64(xq.cpu().numpy(), wq.cpu().numpy(), np.float32(sx * sw))
        yy = f16_tensor_f64(y)
        assert np.abs(yy - ref).max() < 0.05 * max(1.0, np.abs(ref).max())

    def fast_step(X, wqt, sw_host):
        amax = X.abs().max().float().clamp_(min=1e-8)
        inv = 7.0 / amax
        xq = C.quant_int4_tensor_scale_dev(X, inv.reshape(1))
        alpha = (amax * (sw_host / 7.0)).reshape(1)
        return C.w4a4_gemm_cutlass_dev(xq, wqt, alpha)

    for (M, N, K) in [(64, 4096, 4096), (8, 4096, 4096)]:
        X = to_dev_bf16(_bf16(g, (M, K)))
        W = to_dev_bf16(_bf16(g, (N, K)))
        sw = W.float().abs().max().item() / 7.0
        wqt = C.quant_int4_tensor_scale(W, sw).view(N, -1)
        y0 = fast_step(X, wqt, sw).clone()
        for _ in range(3):
            fast_step(X, wqt, sw)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            out = fast_step(X, wqt, sw)
        for _ in range(2):
            gr.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, y0)


def test_error_behaviour(C):
    import torch
    x = torch.zeros(4, 48, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        C.quant_int4(x)
    with pytest.raises(RuntimeError, match="bf16"):
        C.fused_transform_quant_int4(x.float(), torch.zeros(1, 32, 32, device="cuda"))
    xq = torch.zeros(4, 48, dtype=torch.uint8, device="cuda")
    xs = torch.zeros(4, 3, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 64"):
        C.w4a4_gemm_s4(xq, xs, xq, xs)
    with pytest.raises(RuntimeError, match="single row"):
        C.w4a4_gemv(xq, xs, xq, xs)
