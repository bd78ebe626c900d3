"""GPU parity at the sizes of every BASELINE.json config, through my_int4._C and
my_int4.chain as a caller of the reference would use them.

Whole outputs are compared: every code byte and bf16 scale of the weight and
activation quantizations (bit-exact), and every output of the fp16 products
against the fp64 dequantized product -- within 2e-3 relative Frobenius, and
each output within its own rounding bound (tests/_util.product_check), so a
wrong column cannot hide in the norm.  The one exception is the Llama-70B
prefill product (4096 x 57344 x 8192), whose fp64 reference would take
minutes on the host: there two whole 256-row stripes of the output (an
interior one and the last) are compared, while its weight and activation
codes are still compared whole."""
import numpy as np
import pytest

import oracle
from _util import (bf16_tensor_bits, f16_tensor_f64, f32_to_bf16_bits, outlier_activations, product_check, rng,
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
    err, worst = product_check(f16_tensor_f64(y), xq.cpu().numpy(), bf16_tensor_bits(xs), wq.cpu().numpy(),
                               bf16_tensor_bits(ws), n_terms_for(M, K, N))
    assert err < FRO_TOL and worst <= 1.0, (err, worst)


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


def n_terms_for(M, K, N):
    """Rounded additions per output of the kernel that runs the product:
    the fp16-MFMA kernels (prefill tiles at M >= 256; the streaming kernel at
    32 < M <= 64 on weights about 57344 rows long: this takes the larger
    count for every such M) accumulate all K exact products in fp32 (counted
    twice, for the MFMA's internal adds); the int8 kernels and the GEMV fold
    K/32 exact group terms, plus at most 64 partial-sum additions across
    lanes, wavefronts and K slices."""
    fp16 = M >= 256 or (32 < M <= 64 and N >= 49953 and K % 1024 == 0)
    return 2 * K if fp16 else K // 32 + 64


def _full_weights(C, N, K, seed):
    """Weights generated and quantized on the GPU (_C.quant_int4); every code
    byte and scale is compared with the oracle's quantization of the same
    bf16 values.  Returns the device tensors and the oracle's arrays."""
    W = _dev_weights(N, K, seed)
    wq, ws = C.quant_int4(W)
    Wb = bf16_tensor_bits(W)
    del W
    qo, so = oracle.quant(Wb, "bf16")
    del Wb
    assert np.array_equal(wq.cpu().numpy(), qo), ("weight codes", N, K)
    assert np.array_equal(bf16_tensor_bits(ws), so), ("weight scales", N, K)
    return wq, ws, qo, so


def _chain_case(C, M, N, K, seed, stripes=None):
    """Full layer through my_int4.chain at (M, N, K).  Every weight and
    activation code and scale is compared bit for bit; the product on every
    row (or on the given 256-row stripes) and every column."""
    import torch
    from my_int4.chain import make_chain, route
    print(f"[cfg] M={M} N={N} K={K} seed={seed}", flush=True)
    g = rng(seed)
    wq, ws, qo, so = _full_weights(C, N, K, seed)
    xb = outlier_activations(g, M, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    X, T = to_dev_bf16(xb), to_dev_bf16(tb)
    y = make_chain(X, T, wq, ws, M)()
    # the transform + quant op the chain ran, compared whole
    xq, xs = getattr(C, route(M)[0])(X, T)
    torch.cuda.synchronize()
    y = y.reshape(M, N)
    qx, sx = oracle.fused_tq(xb, tb)
    assert np.array_equal(xq.reshape(M, -1).cpu().numpy(), qx), ("activation codes", M, K)
    assert np.array_equal(bf16_tensor_bits(xs).reshape(M, -1), sx), ("activation scales", M, K)
    rows = np.arange(M) if stripes is None else np.concatenate([np.arange(r, r + 256) for r in stripes])
    got = f16_tensor_f64(y[torch.from_numpy(rows).cuda()])
    err, worst = product_check(got, qx[rows], sx[rows], qo, so, n_terms_for(M, K, N))
    assert err < FRO_TOL and worst <= 1.0, (M, N, K, err, worst)
    return y


@pytest.mark.parametrize("M", [1, 8])
def test_cfg3_llama70b_decode(C, M):
    # W4 K=8192 x N=57344, M = 1 and 8, online transform+quant then GEMV
    _chain_case(C, M, 57344, 8192, 300 + M)


@pytest.mark.parametrize("M", [1, 8, 32])
def test_cfg4_qwen3_8b_small_batch(C, M):
    # W4 K=4096 x N=24576, M = 1/8/32, fused_tq -> gemm_s4 (split-K)
    _chain_case(C, M, 24576, 4096, 400 + M)


def test_cfg5_prefill_square(C):
    # K=N=4096 at M=4096, every output
    _chain_case(C, 4096, 4096, 4096, 500 + 4096)


def test_cfg5_prefill_llama70b(C):
    # the Llama-70B FFN at M=4096: codes whole, the
    # product on an interior 256-row stripe (one row tile of every column
    # tile) and the last one
    _chain_case(C, 4096, 57344, 8192, 500 + 57344, stripes=[256 * int(rng(5).integers(1, 15)), 4096 - 256])


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
