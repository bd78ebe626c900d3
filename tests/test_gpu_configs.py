"""GPU parity at the sizes of every BASELINE.json config, through my_int4._C and
my_int4.chain as a caller of the reference would use them.

Where the CPU oracle finishes in seconds the whole output is compared; at the
Llama-70B and prefill sizes the GPU computes everything and seeded samples of
rows / columns are compared (codes and scales bit-exact, fp16 products within
2e-3 relative Frobenius of the fp64 dequantized product)."""
import numpy as np
import pytest

import oracle
from _util import (bf16_tensor_bits, f16_tensor_f64, f32_to_bf16_bits, outlier_activations, rel_fro, rng,
                   to_dev_bf16)

pytestmark = pytest.mark.gpu
FRO_TOL = 2e-3


@pytest.fixture(scope="module")
def C():
    import torch  # noqa: F401
    from my_int4 import _C
    return _C


def _dev_weights(N, K, seed):
    """N(0, 0.02) bf16 weights generated and quantized on the GPU."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return W


def _check_weight_rows(C, W, wq, ws, rows):
    Wb = bf16_tensor_bits(W[rows])
    qo, so = oracle.quant(Wb, "bf16")
    assert np.array_equal(wq[rows].cpu().numpy(), qo)
    assert np.array_equal(bf16_tensor_bits(ws[rows]), so)


def test_cfg1_cpu_reference_shape(C):
    # X fp16 16x4096 (1% outlier channels x50), W fp16 4096x4096 ~ N(0, 0.02)
    import torch
    g = rng(0)
    M, N, K = 16, 4096, 4096
    x = outlier_activations(g, M, K)
    X = torch.from_numpy((x.astype(np.uint32) << 16).view(np.float32)).half().cuda()
    W = torch.from_numpy((g.standard_normal((N, K)) * 0.02).astype(np.float32)).half().cuda()
    xq, xs = C.quant_int4(X)
    wq, ws = C.quant_int4(W)
    qo, so = oracle.quant(X.cpu().numpy().view(np.uint16), "f16")
    assert np.array_equal(xq.cpu().numpy(), qo) and np.array_equal(bf16_tensor_bits(xs), so)
    qo, so = oracle.quant(W.cpu().numpy().view(np.uint16), "f16")
    assert np.array_equal(wq.cpu().numpy(), qo) and np.array_equal(bf16_tensor_bits(ws), so)
    y = C.w4a4_gemm_s4(xq, xs, wq, ws)
    ref = oracle.gemm_f64(xq.cpu().numpy(), bf16_tensor_bits(xs), wq.cpu().numpy(), bf16_tensor_bits(ws))
    assert rel_fro(f16_tensor_f64(y), ref) < FRO_TOL


def test_cfg2_fused_transform_quant(C):
    # X bf16 2048x4096 with outliers; T: 128 blocks from the block
    # Gram of a seeded 512-row calibration draw (this build's own WUSH T solve)
    import torch
    from wush_int4_kernel_amd.wush_transform import compute_wush_transform
    g = rng(1)
    M, K = 2048, 4096
    xb = outlier_activations(g, M, K)
    xcal = torch.from_numpy(bf16_bits_to_f32_np(outlier_activations(g, 512, K))).double()
    W = torch.from_numpy((g.standard_normal((K, K)) * 0.02).astype(np.float32)).double()
    tb = bf16_tensor_bits(compute_wush_transform(xcal, W).to(torch.bfloat16))
    qo, so = oracle.fused_tq(xb, tb)
    X, T = to_dev_bf16(xb), to_dev_bf16(tb)
    for name in ("fused_transform_quant_int4", "fused_transform_quant_int4_v3",
                 "fused_transform_quant_int4_smallm", "fused_transform_quant_int4_wmma"):
        q, s = getattr(C, name)(X, T)
        assert np.array_equal(q.cpu().numpy(), qo), name
        assert np.array_equal(bf16_tensor_bits(s), so), name


def bf16_bits_to_f32_np(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _chain_case(C, M, N, K, seed, n_rows_checked, n_cols_checked):
    """Full layer through my_int4.chain at (M, N, K); check sampled outputs."""
    import torch
    from my_int4.chain import make_chain
    g = rng(seed)
    W = _dev_weights(N, K, seed)
    wq, ws = C.quant_int4(W)
    xb = outlier_activations(g, M, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    X, T = to_dev_bf16(xb), to_dev_bf16(tb)
    y = make_chain(X, T, wq, ws, M)()
    torch.cuda.synchronize()
    y = y.reshape(M, N)
    rows = np.sort(g.choice(M, size=min(M, n_rows_checked), replace=False))
    cols = np.sort(g.choice(N, size=min(N, n_cols_checked), replace=False))
    _check_weight_rows(C, W, wq, ws, torch.from_numpy(cols).cuda())
    qo, so = oracle.fused_tq(xb[rows], tb)
    wq_s = wq[torch.from_numpy(cols).cuda()].cpu().numpy()
    ws_s = bf16_tensor_bits(ws[torch.from_numpy(cols).cuda()])
    ref = oracle.gemm_f64(qo, so, wq_s, ws_s)
    got = f16_tensor_f64(y[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()])
    assert rel_fro(got, ref) < FRO_TOL, (M, N, K, rel_fro(got, ref))
    return y


@pytest.mark.parametrize("M", [1, 8])
def test_cfg3_llama70b_decode(C, M):
    # W4 K=8192 x N=57344, M = 1 and 8, online transform+quant then GEMV
    _chain_case(C, M, 57344, 8192, 300 + M, 8, 2048)


@pytest.mark.parametrize("M", [1, 8, 32])
def test_cfg4_qwen3_8b_small_batch(C, M):
    # W4 K=4096 x N=24576, M = 1/8/32, fused_tq -> gemm_s4 (split-K)
    _chain_case(C, M, 24576, 4096, 400 + M, 32, 4096)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (4096, 57344, 8192)])
def test_cfg5_prefill(C, M, N, K):
    # K=N=4096 at M=4096 and the Llama-70B FFN at M=4096
    _chain_case(C, M, N, K, 500 + N, 16, 1024)


@pytest.mark.parametrize("M", [1, 8, 32])
def test_l70_exact_properties(C, M):
    # Size-independent properties at the full Llama-70B FFN shape, where the
    # oracle would be slow: (1) doubling every activation scale doubles every
    # output exactly (a power-of-two factor passes through the exact group
    # dots and every fp32 fold and fp16 rounding unchanged); (2) permuting the
    # weight rows permutes the outputs bit for bit (each output's arithmetic
    # does not depend on where its row sits); (3) zero weight rows give zeros.
    import torch
    N, K = 57344, 8192
    g = rng(700 + M)
    W = _dev_weights(N, K, 700 + M)
    wq, ws = C.quant_int4(W)
    del W
    xq, xs = C.quant_int4(to_dev_bf16(outlier_activations(g, M, K)))
    y = C.w4a4_gemm_s4(xq, xs, wq, ws)
    y2 = C.w4a4_gemm_s4(xq, (xs.float() * 2).to(torch.bfloat16), wq, ws)
    assert torch.equal(y2, y * 2), M
    perm = torch.from_numpy(g.permutation(N)).cuda()
    yp = C.w4a4_gemm_s4(xq, xs, wq[perm].contiguous(), ws[perm].contiguous())
    assert torch.equal(yp, y[:, perm]), M
    wz = wq.clone()
    wz[::97] = 0
    yz = C.w4a4_gemm_s4(xq, xs, wz, ws)
    assert (yz[:, ::97] == 0).all() and torch.equal(yz[:, 1::97], y[:, 1::97]), M
