"""GPU parity tests through the C ABI (include/wush_int4.h via ctypes).

torch supplies device memory and the stream only.  Bars:
  * quant_int4 / fused_tq: codes and bf16 scale bits bit-exact vs the oracle
    and the committed fixtures;
  * GEMV / GEMM: the int32 group dots exact (unit scales, |Y| < 2048 so fp16
    holds them exactly) and the fp16 output within 2e-3 relative Frobenius of
    the fp64 dequantized product (the tolerance the north star states);
  * MFMA layout self-test exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from _util import (bf16_bits_to_f32, f16_tensor_f64, f32_to_bf16_bits, outlier_activations,
                   pack_codes, rel_fro, rng, to_dev_bf16, to_dev_u8, unpack_codes)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FRO_TOL = 2e-3


@pytest.fixture(scope="module")
def capi():
    import torch  # noqa: F401  (HIP runtime first)
    from wush_int4_kernel_amd import capi as c
    c.load()
    return c


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def _bits(t) -> np.ndarray:
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_quant(capi, x_np: np.ndarray, dtype: str):
    import torch
    if dtype == "bf16":
        xt = to_dev_bf16(x_np)
        code = capi.DTYPE_BF16
    elif dtype == "f16":
        xt = torch.from_numpy(np.ascontiguousarray(x_np, dtype=np.float16)).cuda()
        code = capi.DTYPE_F16
    else:
        xt = torch.from_numpy(np.ascontiguousarray(x_np, dtype=np.float32)).cuda()
        code = capi.DTYPE_F32
    n_groups = xt.numel() // 32
    q = torch.empty(xt.numel() // 2, dtype=torch.uint8, device="cuda")
    s = torch.empty(n_groups, dtype=torch.bfloat16, device="cuda")
    capi.quant_int4(xt.data_ptr(), code, q.data_ptr(), s.data_ptr(), n_groups, _stream())
    torch.cuda.synchronize()
    K = x_np.shape[-1]
    return q.cpu().numpy().reshape(x_np.shape[:-1] + (K // 2,)), _bits(s).reshape(x_np.shape[:-1] + (K // 32,))


def run_fused(capi, xb: np.ndarray, tb: np.ndarray):
    import torch
    xt = to_dev_bf16(xb)
    tt = to_dev_bf16(tb)
    K = xb.shape[-1]
    rows = xb.size // K
    q = torch.empty(rows * K // 2, dtype=torch.uint8, device="cuda")
    s = torch.empty(rows * K // 32, dtype=torch.bfloat16, device="cuda")
    capi.fused_tq(xt.data_ptr(), tt.data_ptr(), q.data_ptr(), s.data_ptr(), rows, K, _stream())
    torch.cuda.synchronize()
    return q.cpu().numpy().reshape(xb.shape[:-1] + (K // 2,)), _bits(s).reshape(xb.shape[:-1] + (K // 32,))


def _dev_operands(xq, xs, wq, ws):
    return to_dev_u8(xq), to_dev_bf16(xs), to_dev_u8(wq), to_dev_bf16(ws)


def run_gemm(capi, xq, xs, wq, ws, kernel="gemm"):
    import torch
    M, K2 = xq.shape
    N = wq.shape[0]
    K = 2 * K2
    dx, dxs, dw, dws = _dev_operands(xq, xs, wq, ws)
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    if kernel == "gemv":
        capi.gemv_int4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y.data_ptr(),
                       M, N, K, _stream())
    else:
        wsb = capi.gemm_s4_workspace_bytes(M, N, K)
        work = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        capi.gemm_s4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y.data_ptr(),
                     M, N, K, work.data_ptr() if wsb else None, wsb, _stream())
    torch.cuda.synchronize()
    return f16_tensor_f64(y)


# --------------------------------------------------------------------- quant
def test_quant_golden_fixture(capi):
    kat = np.load(os.path.join(GOLDEN, "quant_kat.npz"))
    q, s = run_quant(capi, kat["x_bf16"], "bf16")
    assert np.array_equal(q, kat["q"]) and np.array_equal(s, kat["s"])


@pytest.mark.parametrize("shape", [(4096, 32), (2, 3, 96), (1, 32), (7, 4096), (1 << 17, 128)])
def test_quant_bf16_random(capi, shape):
    g = rng(1000 + len(shape) * 7 + shape[-1])
    x = f32_to_bf16_bits(g.standard_normal(shape).astype(np.float32))
    q, s = run_quant(capi, x, "bf16")
    qo, so = oracle.quant(x, "bf16")
    assert np.array_equal(q, qo), np.argwhere(q != qo)[:5]
    assert np.array_equal(s, so)


def test_quant_outliers_zeros_ties_overflow(capi):
    g = rng(1001)
    blocks = [outlier_activations(g, 64, 4096).reshape(-1, 32)]
    blocks.append(np.zeros((4, 32), np.uint16))
    t = np.zeros((2, 32), np.float32)
    t[0, :8] = [7.0, -7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5]
    t[1, :8] = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -6.5], np.float32) * np.float32(0.7)
    blocks.append(f32_to_bf16_bits(t))
    blocks.append(f32_to_bf16_bits(np.full((4, 32), 3.3e38, np.float32)))
    special = np.zeros((3, 32), np.float32)
    special[0, 3] = np.inf
    special[1, 4] = -np.inf
    special[1, 9] = 2.0
    special[2, :] = g.standard_normal(32)
    special[2, 7] = np.nan
    blocks.append(f32_to_bf16_bits(special))
    blocks.append(f32_to_bf16_bits((g.standard_normal((64, 32)) * 1e-39).astype(np.float32)))  # subnormal
    x = np.concatenate(blocks, axis=0)
    q, s = run_quant(capi, x, "bf16")
    qo, so = oracle.quant(x, "bf16")
    assert np.array_equal(q, qo) and np.array_equal(s, so)


def test_quant_f32_near_ties(capi):
    # fp32 codes come from one fma per element, t = RN(v * RN(1/sf) + 8), and a
    # lane whose t lies within 2^-17 of a half-integer redoes its group with
    # the correctly rounded quotient (wush_device.h, code8_fast).  Groups hold
    # two anchors +-40 that dominate the variance, so the scale sf settles after
    # a few rebuilds, and 30 values h*sf +- k ulps (h a half-integer, |k| <= 3):
    # quotients at and next to rounding ties.  The second half of the groups
    # keeps its values away from ties (the fast path alone).  Codes and scales
    # must match the division bit for bit.
    g = rng(1004)
    n = 512
    x = np.zeros((n, 32), np.float32)
    x[:, 0], x[:, 1] = np.float32(40.0), np.float32(-40.0)
    h = (g.integers(-5, 6, (n, 30)) * 0.5).astype(np.float32)
    h[n // 2:] += g.uniform(-0.4, 0.4, (n // 2, 30)).astype(np.float32)
    k = g.integers(-3, 4, (n, 30))
    sf = np.full(n, 4.0, np.float32)
    for _ in range(10):
        v = (h * sf[:, None]).astype(np.float32)
        for step in range(3):
            v[k > step] = np.nextafter(v[k > step], np.float32(np.inf))
            v[k < -step] = np.nextafter(v[k < -step], np.float32(-np.inf))
        x[:, 2:] = v
        _, so = oracle.quant(x, "f32")
        sf = bf16_bits_to_f32(so.reshape(n))
    q, s = run_quant(capi, x, "f32")
    qo, so = oracle.quant(x, "f32")
    assert np.array_equal(q, qo) and np.array_equal(s, so)
    # the construction must put quotients in the fallback band
    quot = x[:, 2:].astype(np.float64) / bf16_bits_to_f32(so.reshape(n)).astype(np.float64)[:, None]
    near = np.abs(quot - np.floor(quot) - 0.5) < 2.0 ** -17
    assert near[: n // 2].sum() > 1000 and near[n // 2:].sum() == 0


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_quant_other_dtypes(capi, dtype):
    g = rng(1002)
    x = bf16_bits_to_f32(outlier_activations(g, 16, 4096))
    if dtype == "f16":
        x = x.astype(np.float16)
        q, s = run_quant(capi, x, "f16")
        qo, so = oracle.quant(x.view(np.uint16), "f16")
    else:
        x = x * np.float32(1.0001)          # values that are not bf16-representable
        q, s = run_quant(capi, x, "f32")
        qo, so = oracle.quant(x, "f32")
    assert np.array_equal(q, qo) and np.array_equal(s, so)


# --------------------------------------------------------------------- fused
def test_fused_golden_fixture(capi):
    fz = np.load(os.path.join(GOLDEN, "fused_small.npz"))
    q, s = run_fused(capi, fz["x_bf16"], fz["t_bf16"])
    assert np.array_equal(q, fz["q"]) and np.array_equal(s, fz["s"])


# The small-M kernel serves launches of at most 16384 (row, block) pairs; the
# rows kernel the rest (fp32 MFMA steps when a wavefront's values are in
# range).  Shapes cover both, with partial 64-row sets and block counts that
# leave a workgroup's 4 blocks partial.
@pytest.mark.parametrize("rows,K", [(1, 32), (1, 4096), (3, 96), (8, 8192), (63, 256), (64, 256),
                                    (65, 512), (130, 128), (383, 256), (384, 256), (385, 96),
                                    (256, 4096), (200, 4096), (1000, 1056),
                                    (1600, 2080), (1 << 16, 64)])
def test_fused_random(capi, rows, K):
    g = rng(2000 + rows + K)
    xb = outlier_activations(g, rows, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    q, s = run_fused(capi, xb, tb)
    qo, so = oracle.fused_tq(xb, tb)
    assert np.array_equal(q, qo), (rows, K, np.argwhere(q != qo)[:5])
    assert np.array_equal(s, so)


@pytest.mark.parametrize("rows", [5, 2500, 12300])
def test_fused_extreme_operands_both_loops(capi, rows):
    # The rows kernel (2500 and 12300 rows) runs fp32 MFMA steps when every
    # nonzero |x| and |T| of a wavefront lies in [2^-56, 2^51), an fma loop
    # when they lie in [2^-67, 2^51), and the mul-then-add loop otherwise;
    # the small-M kernel (5 rows) the last two.  Plant out-of-range values in
    # some rows and T blocks (tiny, subnormal, huge, inf, NaN, at the range
    # edges) so every loop and the votes between them run; every code and
    # scale must still match the oracle bit for bit.
    g = rng(2003 + rows)
    K = 256
    xb = outlier_activations(g, rows, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    specials = [0x0001, 0x8001, 0x0080, 0x1DFF, 0x1E00, 0x58FF, 0x5900, 0x7F7F, 0x7F80, 0xFF80, 0x7FC0,
                0x2000, 0x0C00, 0x6000, 0x237F, 0xA37F, 0x2380]
    for r in range(0, rows, 7):
        xb[r, g.integers(0, K)] = specials[r % len(specials)]
    tb[1, 3, 5] = 0x0001            # subnormal T entry: block 1 takes mul + add
    tb[2, 0, 0] = 0x1DFF            # just below the range
    tb[3, 7, 9] = 0x58FF            # upper edge, still in range
    tb[4, 1, 1] = 0x5900            # just above the range
    tb[5, 2, 30] = 0x237F           # below the MFMA range, inside the fma loop's
    tb[6, 31, 0] = 0x2380           # lower edge of the MFMA range
    q, s = run_fused(capi, xb, tb)
    qo, so = oracle.fused_tq(xb, tb)
    assert np.array_equal(q, qo), np.argwhere(q != qo)[:5]
    assert np.array_equal(s, so), np.argwhere(s != so)[:5]


def _takes_two_tile(rows: int, K: int, cus: int) -> bool:
    """Whether wush_fused_tq runs a (rows, K) launch on the two-tile rows kernel:
    more than 16384 (row, block) pairs, at least 2 of its 128-row workgroups
    per CU, and no CU with more tiles than the 64-row kernel would give it."""
    C = K // 32
    gx, gy, gy2 = -(-C // 4), -(-rows // 64), -(-rows // 128)
    per_cu1, per_cu2 = -(-gx * gy // cus), -(-gx * gy2 // cus)
    return rows * C > 16384 and gx * gy2 >= 2 * cus and 2 * per_cu2 <= per_cu1


# The two-tile rows kernel (two 64-row tiles per wavefront).  Shapes: cfg2's
# 2048 x 4096, partial 128-row and 4-block sets (3900 x 4128), and a last
# workgroup with a partial first tile and an empty second one (32691 x 256).
# The last shape plants out-of-range values in the first tile only, the second
# only, or neither, of a workgroup's blocks (and in some T blocks), so the
# MFMA steps, the fma loop and the mul-then-add loop meet in every pairing.
@pytest.mark.parametrize("rows,K,special", [(2048, 4096, False), (3900, 4128, False), (32691, 256, True)])
def test_fused_two_tile_kernel(capi, rows, K, special):
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if not _takes_two_tile(rows, K, cus):
        pytest.skip(f"{rows} x {K} does not take the two-tile kernel on {cus} CUs")
    g = rng(2100 + rows + K)
    xb = outlier_activations(g, rows, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.25)
    if special:
        specials = [0x0001, 0x8001, 0x1DFF, 0x1E00, 0x5900, 0x7F80, 0xFF80, 0x7FC0, 0x237F, 0x2000]
        for wg in range(-(-rows // 128)):
            for blk in g.choice(K // 32, size=3, replace=False):
                half = (wg + blk) % 3                  # 0: first tile, 1: second tile, 2: neither
                r = wg * 128 + 64 * half + int(g.integers(0, 64))
                if half < 2 and r < rows:
                    xb[r, blk * 32 + int(g.integers(0, 32))] = specials[(wg + blk) % len(specials)]
        tb[1, 3, 5] = 0x0001                           # whole blocks: mul-then-add
        tb[5, 2, 30] = 0x237F                          # fma loop
    q, s = run_fused(capi, xb, tb)
    qo, so = oracle.fused_tq(xb, tb)
    assert np.array_equal(q, qo), (rows, K, np.argwhere(q != qo)[:5])
    assert np.array_equal(s, so), (rows, K, np.argwhere(s != so)[:5])


def run_transform32(capi, xb: np.ndarray, tb: np.ndarray) -> np.ndarray:
    import torch
    rows = xb.shape[0]
    xt, tt = to_dev_bf16(xb), to_dev_bf16(tb)
    xp = torch.empty(rows * 32, dtype=torch.float32, device="cuda")
    capi.fused_tq_transform32(xt.data_ptr(), tt.data_ptr(), xp.data_ptr(), rows, _stream())
    torch.cuda.synchronize()
    return xp.cpu().numpy().reshape(rows, 32)


def _bf16_exp(g, shape, lo, hi, zeros=0.0):
    """Random bf16 bit patterns: sign, exponent uniform in [lo, hi], 7-bit mantissa."""
    e = g.integers(lo, hi + 1, size=shape) + 127
    b = (g.integers(0, 2, size=shape) << 15) | (e << 7) | g.integers(0, 128, size=shape)
    if zeros:
        b = np.where(g.random(shape) < zeros, 0, b)
    return b.astype(np.uint16)


@pytest.mark.parametrize("family", ["normal", "wide", "ties", "fma_range", "specials"])
def test_fused_transform_stage_bit_exact(capi, family):
    # x' itself, from the rows kernel's transform stage, against the oracle's
    # sequential fp32 sums: every value bit for bit (a NaN matches a NaN).
    # "normal" and "wide" (exponents over the whole MFMA range [2^-56, 2^51),
    # products from 2^-112 up, many roundings and absorptions) and "ties"
    # (a leading product near 1.5, then products of exactly a half, a quarter
    # or three quarters of its ulp: round-half-even decides most sums) run
    # the MFMA steps; "fma_range" (values in [2^-67, 2^-56)) the fma loop;
    # "specials" (subnormal, huge, inf, NaN in some rows) the mul-then-add
    # loop next to MFMA wavefronts.
    g = rng({"normal": 3101, "wide": 3102, "ties": 3103, "fma_range": 3104, "specials": 3105}[family])
    rows = 64 * 7 + 19
    if family == "normal":
        xb = f32_to_bf16_bits(g.standard_normal((rows, 32)) * 3.0)
        tb = f32_to_bf16_bits(g.standard_normal((1, 32, 32)) * 0.25)
    elif family == "wide":
        xb = _bf16_exp(g, (rows, 32), -56, 25, zeros=0.05)
        tb = _bf16_exp(g, (1, 32, 32), -56, 25, zeros=0.05)
    elif family == "ties":
        xb = np.zeros((rows, 32), np.uint16)
        xb[:, 0] = f32_to_bf16_bits(1.5 + g.integers(0, 4, rows) * 0.125)
        xb[:, 1:] = f32_to_bf16_bits(np.ldexp(g.choice([-1.0, 1.0], (rows, 31)), -g.integers(22, 26, (rows, 31))))
        tv = g.choice([1.0, 0.5, 0.75, -1.0, -0.5, 0.0], (1, 32, 32))
        tv[:, :, 0] = 1.0
        tb = f32_to_bf16_bits(tv)
    elif family == "fma_range":
        xb = _bf16_exp(g, (rows, 32), -60, 10)
        xb[::3, 5] = 0x1E80                 # 2^-66: inside the fma loop's range only
        tb = _bf16_exp(g, (1, 32, 32), -20, 5)
    else:
        xb = f32_to_bf16_bits(g.standard_normal((rows, 32)))
        tb = f32_to_bf16_bits(g.standard_normal((1, 32, 32)) * 0.25)
        for r, v in zip(range(3, rows, 37), [0x0001, 0x7F80, 0xFFC0, 0x7F7F, 0x8080, 0x5900]):
            xb[r, (r * 7) % 32] = v
    got = run_transform32(capi, xb, tb)
    want = oracle.transform(xb, tb)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), (family, np.argwhere(~same)[:5], got[~same][:5], want[~same][:5])


def test_fused_permutation_identity_zeros(capi):
    g = rng(2001)
    K = 128
    xb = outlier_activations(g, 70, K)
    T = np.zeros((K // 32, 32, 32), np.float32)
    for c in range(K // 32):
        T[c, np.arange(32), g.permutation(32)] = 1.0
    for tb in (f32_to_bf16_bits(T), f32_to_bf16_bits(np.broadcast_to(np.eye(32), T.shape))):
        for rows in (5, 70):
            q, s = run_fused(capi, xb[:rows], tb)
            qo, so = oracle.fused_tq(xb[:rows], tb)
            assert np.array_equal(q, qo) and np.array_equal(s, so)
    z = np.zeros((4, 64), np.uint16)
    q, s = run_fused(capi, z, f32_to_bf16_bits(g.standard_normal((2, 32, 32))))
    assert (q == 0).all() and (s == 0x322C).all()


def test_fused_3d_shape(capi):
    g = rng(2002)
    xb = f32_to_bf16_bits(g.standard_normal((2, 3, 96)))
    tb = f32_to_bf16_bits(g.standard_normal((3, 32, 32)))
    q, s = run_fused(capi, xb, tb)
    qo, so = oracle.fused_tq(xb, tb)
    assert q.shape == (2, 3, 48) and s.shape == (2, 3, 3)
    assert np.array_equal(q, qo) and np.array_equal(s, so)


# ----------------------------------------------------------------- GEMV/GEMM
def _rand_operands(g, M, N, K):
    xq, xs = oracle.quant(outlier_activations(g, M, K), "bf16")
    wq, ws = oracle.quant(f32_to_bf16_bits(g.standard_normal((N, K)) * 0.02), "bf16")
    return xq, xs, wq, ws


def _unit_scale_operands(g, M, N, K):
    # codes bounded so that |Y| = |sum qx*qw| < 2048 is exact in fp16
    lim = max(1, int(np.sqrt(2000.0 / K)))
    cx = g.integers(-lim, lim + 1, (M, K))
    cw = g.integers(-7, 8, (N, K)) if lim * 7 * K < 2048 else g.integers(-lim, lim + 1, (N, K))
    xs = np.full((M, K // 32), 0x3F80, np.uint16)
    ws = np.full((N, K // 32), 0x3F80, np.uint16)
    return pack_codes(cx), xs, pack_codes(cw), ws, (cx @ cw.T).astype(np.float64)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8])
def test_gemv_matches_oracle(capi, M):
    g = rng(3000 + M)
    for N, K in [(64, 64), (300, 512), (4096, 4096)]:
        xq, xs, wq, ws = _rand_operands(g, M, N, K)
        y = run_gemm(capi, xq, xs, wq, ws, "gemv")
        ref = oracle.gemm_f64(xq, xs, wq, ws)
        assert rel_fro(y, ref) < FRO_TOL, (M, N, K, rel_fro(y, ref))


def _random_code_operands(g, M, N, K, sx_exp=(124, 129), sw_exp=(120, 124)):
    """Any nibbles (including -8) and bf16 scales with exponent fields in the
    given ranges: the product does not care how the codes were quantized."""
    xq = g.integers(0, 256, (M, K // 2), dtype=np.uint8)
    wq = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    xs = ((g.integers(*sx_exp, (M, K // 32)) << 7) | g.integers(0, 128, (M, K // 32))).astype(np.uint16)
    ws = ((g.integers(*sw_exp, (N, K // 32)) << 7) | g.integers(0, 128, (N, K // 32))).astype(np.uint16)
    return xq, xs, wq, ws


@pytest.mark.parametrize("M", [7, 8])
def test_gemv_ksplit_matches_oracle(capi, M):
    # M >= 7, K = 8192 (4 wavefronts per row range) and N > 32768 take the
    # K-split GEMV; ragged N leaves a short last row range
    g = rng(3050 + M)
    N, K = 33000, 8192
    xq, xs, wq, ws = _random_code_operands(g, M, N, K)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    y = run_gemm(capi, xq, xs, wq, ws, "gemv")
    assert rel_fro(y, ref) < FRO_TOL, (M, rel_fro(y, ref))
    y2 = run_gemm(capi, xq, xs, wq, ws, "gemm")
    assert rel_fro(y, y2) < 1e-3


def test_gemv_ksplit_scales_out_of_range(capi):
    # activation scales of 2^61 (above the 2^60 limit of the conversion-free
    # fold) send every wavefront to the conversion form, which rounds the same
    # dot*sx*sw once; tiny weight scales keep the outputs in fp16's range
    g = rng(3060)
    M, N, K = 8, 33000, 8192
    xq, xs, wq, ws = _random_code_operands(g, M, N, K, sx_exp=(188, 189), sw_exp=(64, 66))
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    y = run_gemm(capi, xq, xs, wq, ws, "gemv")
    assert np.isfinite(y).all()
    assert rel_fro(y, ref) < FRO_TOL, rel_fro(y, ref)


@pytest.mark.parametrize("K", [16384, 32768])
def test_gemv_ksplit_more_wavefronts(capi, K):
    # 8 and 16 wavefronts per row range (the largest K-split workgroup)
    g = rng(3070 + K // 16384)
    M, N = 8, 32800
    xq, xs, wq, ws = _random_code_operands(g, M, N, K)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    y = run_gemm(capi, xq, xs, wq, ws, "gemv")
    assert rel_fro(y, ref) < FRO_TOL, (K, rel_fro(y, ref))


def test_gemv_ksplit_mixed_forms(capi):
    # only wavefront 1's groups (64..127) carry activation scales above 2^60:
    # that wavefront takes the conversion form, the other three the
    # conversion-free one, and their partials meet in one sum per output
    g = rng(3080)
    M, N, K = 8, 33000, 8192
    xq, xs, wq, ws = _random_code_operands(g, M, N, K, sw_exp=(64, 66))
    xs[:, :64] = (xs[:, :64] & 0x7F) | (180 << 7)          # 2^53: in range
    xs[:, 64:128] = (xs[:, 64:128] & 0x7F) | (188 << 7)    # 2^61: out of range
    xs[:, 128:] = (xs[:, 128:] & 0x7F) | (180 << 7)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    y = run_gemm(capi, xq, xs, wq, ws, "gemv")
    assert np.isfinite(y).all()
    assert rel_fro(y, ref) < FRO_TOL, rel_fro(y, ref)


@pytest.mark.parametrize("M", [1, 4, 8])
def test_gemv_int_exact(capi, M):
    g = rng(3100 + M)
    xq, xs, wq, ws, yi = _unit_scale_operands(g, M, 200, 256)
    y = run_gemm(capi, xq, xs, wq, ws, "gemv")
    assert np.array_equal(y, yi)


# shapes of the reference's fp64 arbitration (tests/test_p13.py:18) plus edges
GEMM_SHAPES = [(64, 96, 128), (1, 64, 64), (300, 500, 512), (130, 512, 4096), (8, 4096, 4096),
               (33, 200, 96), (257, 33, 96), (8, 32, 32), (32, 1000, 1024), (200, 130, 2048)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_matches_oracle(capi, M, N, K):
    g = rng(4000 + M * 7 + N + K)
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    y = run_gemm(capi, xq, xs, wq, ws)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    assert rel_fro(y, ref) < FRO_TOL, (M, N, K, rel_fro(y, ref))
    # the reference gate (tests/test_p13.py:23-27) holds too
    assert np.abs(y - ref).max() < 0.05 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (8, 300, 256), (40, 130, 128), (150, 260, 96)])
def test_gemm_int_exact(capi, M, N, K):
    g = rng(4100 + M + N + K)
    xq, xs, wq, ws, yi = _unit_scale_operands(g, M, N, K)
    y = run_gemm(capi, xq, xs, wq, ws)
    assert np.array_equal(y, yi)


def test_gemm_group_dots_exact_per_group(capi):
    # One group at a time: scales 1 on group g only, 0 elsewhere -> y = D[:, :, g].
    g = rng(4200)
    M, N, K = 16, 96, 128
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    D = oracle.group_dots(xq, wq)
    for gg in range(K // 32):
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = 0x3F80
        ws[:, gg] = 0x3F80
        for kernel in ("gemm", "gemv"):
            xs_k = xs[:8] if kernel == "gemv" else xs
            xq_k = xq[:8] if kernel == "gemv" else xq
            y = run_gemm(capi, xq_k, xs_k, wq, ws, kernel)
            assert np.array_equal(y, D[: y.shape[0], :, gg].astype(np.float64)), (kernel, gg)


@pytest.mark.parametrize("M", [1, 5, 8])
def test_gemm_decode_many_row_blocks(capi, M):
    # many row blocks with N not a multiple of 32: the last workgroup of the
    # streaming kernel holds a partial block
    g = rng(4270 + M)
    N, K = 33000, 512
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    y = run_gemm(capi, xq, xs, wq, ws)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    assert rel_fro(y, ref) < FRO_TOL, (M, rel_fro(y, ref))


@pytest.mark.parametrize("M", [1, 8, 17, 32, 40, 64])
def test_gemm_scale_alignment_paths_agree(capi, M):
    # Scales that are only 2-byte aligned take the LDS-tiled kernel, 16-byte
    # aligned ones a streaming kernel (M <= 64, K % 256 == 0).  Both fold the
    # same exact group dots; the streaming kernel sums them in another order
    # (per-wavefront K slices added in wavefront order), so the two agree to
    # fp16 rounding.
    import torch
    g = rng(4250 + M)
    N, K = 300, 1024
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    dx, dw = to_dev_u8(xq), to_dev_u8(wq)
    outs = []
    for shift in (0, 1):
        bx = torch.zeros(xs.size + 8, dtype=torch.bfloat16, device="cuda")
        bw = torch.zeros(ws.size + 8, dtype=torch.bfloat16, device="cuda")
        bx[shift:shift + xs.size] = to_dev_bf16(xs).reshape(-1)
        bw[shift:shift + ws.size] = to_dev_bf16(ws).reshape(-1)
        y = torch.empty(M, N, dtype=torch.float16, device="cuda")
        capi.gemm_s4(dx.data_ptr(), bx.data_ptr() + 2 * shift, dw.data_ptr(), bw.data_ptr() + 2 * shift,
                     y.data_ptr(), M, N, K, None, 0, _stream())
        torch.cuda.synchronize()
        outs.append(f16_tensor_f64(y))
        assert rel_fro(outs[-1], ref) < FRO_TOL, (M, shift, rel_fro(outs[-1], ref))
    assert rel_fro(outs[1], outs[0]) < 1e-3


@pytest.mark.parametrize("M,K", [(1, 512), (5, 256), (8, 768), (9, 256), (16, 512), (24, 768), (32, 1024),
                                 (48, 512), (64, 256)])
def test_gemm_stream_group_dots_exact_per_group(capi, M, K):
    # The streaming kernels (16-byte aligned scales, K % 256 == 0): scales 1
    # on group g only and 0 elsewhere -> y = D[:, :, g] exactly, whichever
    # wavefront of the K split holds group g.
    g = rng(4210 + M)
    N = 40
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    D = oracle.group_dots(xq, wq)
    for gg in range(K // 32):
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = 0x3F80
        ws[:, gg] = 0x3F80
        y = run_gemm(capi, xq, xs, wq, ws)
        assert np.array_equal(y, D[:, :, gg].astype(np.float64)), (M, K, gg)


@pytest.mark.parametrize("M,N,K", [(9, 33, 256), (12, 4097, 768), (17, 70, 2048), (31, 1000, 1280),
                                   (32, 8192, 4096), (20, 96, 8192), (33, 500, 512), (40, 1000, 1024),
                                   (57, 33, 256), (64, 4096, 2048)])
def test_gemm_stream_k_split_shapes(capi, M, N, K):
    # in-workgroup K split: stage counts that leave some wavefronts idle
    # (K = 256, 768), ragged N, and global split-K on top (small N, long K)
    g = rng(4280 + M + N)
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    y = run_gemm(capi, xq, xs, wq, ws)
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    assert rel_fro(y, ref) < FRO_TOL, (M, N, K, rel_fro(y, ref))


@pytest.mark.parametrize("M,N,K,groups", [
    # wide weights (4 K ways): 40 stages in runs of 10 per wavefront, so the
    # scale chunks of 4 stages start at stages 0, 4, 8 of a run, the last one
    # clamped; groups at run, chunk and stage boundaries
    (24, 16416, 10240, [0, 31, 32, 63, 64, 72, 79, 80, 239, 240, 319]),
    # 9 stages: runs of 3, 3, 3 and an idle wavefront; ragged last column block
    (9, 16400, 2304, [0, 7, 8, 23, 24, 47, 48, 71]),
])
def test_gemm_stream_wide_exact_per_group(capi, M, N, K, groups):
    # The streaming kernel on wide weights: scales 1 on group g only and 0
    # elsewhere -> y = D[:, :, g] exactly, wherever the stage of g falls in
    # its wavefront's run and in its 4-stage scale chunk.
    g = rng(4290 + M)
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    for gg in groups:
        D = oracle.group_dots(xq[:, 16 * gg:16 * gg + 16], wq[:, 16 * gg:16 * gg + 16])[:, :, 0]
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = 0x3F80
        ws[:, gg] = 0x3F80
        y = run_gemm(capi, xq, xs, wq, ws)
        assert np.array_equal(y, D.astype(np.float64)), (M, N, K, gg)


def test_gemm_random_shapes_all_paths(capi):
    # Seeded random shapes over every planner branch: the streaming kernel
    # (K % 256 == 0, M <= 64, with and without split-K), the LDS tiles (other
    # K, M > 64), ragged N, and 2-byte-aligned scales (the tiles at any M);
    # the GEMV beside them at M <= 8.  Each against the fp64 oracle product.
    import torch
    g = rng(4400)
    for case in range(24):
        M = int(g.choice([1, 2, 3, 5, 8, 9, 16, 23, 31, 32, 33, 47, 64, 65, 100, 200]))
        N = int(g.integers(1, 3000))
        K = 32 * int(g.choice([1, 3, 8, 9, 16, 24, 40, 64, 96, 128]))
        xq, xs, wq, ws = _rand_operands(g, M, N, K)
        ref = oracle.gemm_f64(xq, xs, wq, ws)
        y = run_gemm(capi, xq, xs, wq, ws)
        assert rel_fro(y, ref) < FRO_TOL, (case, M, N, K, rel_fro(y, ref))
        if M <= 8 and M * K * 3 // 4 <= 65536:
            y2 = run_gemm(capi, xq, xs, wq, ws, "gemv")
            assert rel_fro(y2, ref) < FRO_TOL, (case, M, N, K, "gemv")
        # 2-byte-aligned scales take the tiles whatever M and K are
        dx, dw = to_dev_u8(xq), to_dev_u8(wq)
        bx = torch.zeros(xs.size + 8, dtype=torch.bfloat16, device="cuda")
        bw = torch.zeros(ws.size + 8, dtype=torch.bfloat16, device="cuda")
        bx[1:1 + xs.size] = to_dev_bf16(xs).reshape(-1)
        bw[1:1 + ws.size] = to_dev_bf16(ws).reshape(-1)
        y3 = torch.empty(M, N, dtype=torch.float16, device="cuda")
        wsb = capi.gemm_s4_workspace_bytes(M, N, K)
        work = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        capi.gemm_s4(dx.data_ptr(), bx.data_ptr() + 2, dw.data_ptr(), bw.data_ptr() + 2, y3.data_ptr(),
                     M, N, K, work.data_ptr() if wsb else None, wsb, _stream())
        torch.cuda.synchronize()
        assert rel_fro(f16_tensor_f64(y3), ref) < FRO_TOL, (case, M, N, K, "unaligned scales")


# Shapes the planner sends to the 256x256 fp16-MFMA tiles (K % 256 == 0,
# M >= 256, at least 128 tiles): ragged M and N, one and several load batches.
# The last two split K across workgroups (8 and 4 slices of 8 groups).
# prefill plans: no K split, and (the last two) ragged M split into 4 and 2
# slices of 32 groups
# (200, 40000, 1024): 256-row tiles at 128 < M < 256 (157 column tiles, the
# last partial).  The last five take the 128-row tiles (N >= 8192, at least
# 192 workgroups): one row tile of 224 column tiles, K split over 2 slices,
# a partial column tile (2 slices of 64 groups), 256 column tiles of K=256,
# and M = 230 (too few 256-row tiles: two 128-row tiles, the second partial).
H16_SHAPES = [(512, 32768, 256), (700, 30000, 512), (1030, 16400, 1024), (4096, 4096, 2048), (300, 33000, 512),
              (600, 4096, 4096), (1030, 4096, 2048), (200, 40000, 1024),
              (65, 57344, 2048), (100, 24576, 4096), (128, 24400, 4096), (128, 65536, 256), (230, 24600, 2048)]


def _sample(g, n, k):
    """k sorted indices of range(n), always holding the first and the last."""
    idx = set(g.choice(n, size=min(n, k), replace=False).tolist()) | {0, n - 1}
    return np.array(sorted(idx))


def _run_gemm_unaligned(capi, xq, xs, wq, ws):
    """wush_gemm_s4 with both scale tensors at 2-byte (not 16-byte) alignment."""
    import torch
    M, N, K = xq.shape[0], wq.shape[0], 2 * xq.shape[1]
    dx, dw = to_dev_u8(xq), to_dev_u8(wq)
    bx = torch.zeros(xs.size + 8, dtype=torch.bfloat16, device="cuda")
    bw = torch.zeros(ws.size + 8, dtype=torch.bfloat16, device="cuda")
    bx[1:1 + xs.size] = to_dev_bf16(xs).reshape(-1)
    bw[1:1 + ws.size] = to_dev_bf16(ws).reshape(-1)
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    wsb = capi.gemm_s4_workspace_bytes(M, N, K)
    work = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    capi.gemm_s4(dx.data_ptr(), bx.data_ptr() + 2, dw.data_ptr(), bw.data_ptr() + 2, y.data_ptr(),
                 M, N, K, work.data_ptr() if wsb else None, wsb, _stream())
    torch.cuda.synchronize()
    return f16_tensor_f64(y)


@pytest.mark.parametrize("M,N,K", H16_SHAPES)
def test_gemm_h16_matches_oracle(capi, M, N, K):
    # fp16 operands code*scale (exact) with fp32 accumulation over the whole
    # K: seeded samples of rows and columns (first and last always) against
    # the fp64 oracle, for 16-byte and 2-byte aligned scales
    g = rng(4500 + M + N + K)
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    rows, cols = _sample(g, M, 40), _sample(g, N, 1500)
    ref = oracle.gemm_f64(xq[rows], xs[rows], wq[cols], ws[cols])
    for name, y in (("aligned", run_gemm(capi, xq, xs, wq, ws)),
                    ("unaligned", _run_gemm_unaligned(capi, xq, xs, wq, ws))):
        got = y[np.ix_(rows, cols)]
        assert rel_fro(got, ref) < FRO_TOL, (M, N, K, name, rel_fro(got, ref))
        assert np.abs(got - ref).max() < 0.05 * max(1.0, np.abs(ref).max())
        assert np.isfinite(y).all()


def _abs_product(xq, xs, wq, ws):
    """sum over k of |x[m][k] * w[n][k]| (codes times scales), in fp64."""
    cx = np.abs(unpack_codes(xq)).astype(np.float64)
    cw = np.abs(unpack_codes(wq)).astype(np.float64)
    M, K = cx.shape
    N, G = cw.shape[0], K // 32
    d = np.einsum("mgk,ngk->mng", cx.reshape(M, G, 32), cw.reshape(N, G, 32), optimize=True)
    sx = np.abs(bf16_bits_to_f32(xs).astype(np.float64))
    sw = np.abs(bf16_bits_to_f32(ws).astype(np.float64))
    return np.einsum("mng,mg,ng->mn", d, sx, sw, optimize=True)


@pytest.mark.parametrize("M,N,K,wide", [(2048, 8192, 4096, False), (300, 33000, 512, False),
                                         (1030, 16400, 1024, False), (512, 8192, 2048, False),
                                         (512, 8192, 2048, True), (300, 33000, 512, True)])
def test_gemm_h16_preconverted_activations_agree(capi, M, N, K, wide):
    # with a workspace of wush_gemm_s4_workspace_bytes, prefill plans with
    # N >= 8192 convert the activations once into it (h16_prep_a_kernel, then
    # gemm_h16q); without that room they are converted per tile
    # (gemm_h16w8): the same fp16 operands, every product exact in fp32,
    # summed in another order.  So the two outputs differ by at most the two
    # fp32 sums' rounding (2 * K * 2^-24 * sum |x * w|, generous) plus one
    # fp16 rounding, on every sampled output.  (512, 8192, 2048) also splits
    # K (2 slices), compared against the no-alloc entry point, whose scratch
    # holds the partials but not the converted activations.
    import torch
    # wide: activation scales spanning 2^35 within a row, so that tiny ones
    # reach fp16's subnormal range and the per-slice shift matters
    g = rng(4700 + M + N + K + wide)
    if wide:
        xq, xs, wq, ws = _random_code_operands(g, M, N, K, sx_exp=(100, 136), sw_exp=(118, 124))
    else:
        xq, xs, wq, ws = _rand_operands(g, M, N, K)
    dx, dxs, dw, dws = _dev_operands(xq, xs, wq, ws)
    wsb = capi.gemm_s4_workspace_bytes(M, N, K)
    assert wsb >= 2 * M * K, "the plan should hold the converted activations"
    work = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    y_a = torch.empty(M, N, dtype=torch.float16, device="cuda")
    capi.gemm_s4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y_a.data_ptr(), M, N, K,
                 work.data_ptr(), wsb, _stream())
    y_t = torch.empty(M, N, dtype=torch.float16, device="cuda")
    if wsb > 4 * M * K:   # split-K partials too
        capi.gemm_s4_noalloc(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y_t.data_ptr(),
                             M, N, K, _stream())
    else:
        capi.gemm_s4(dx.data_ptr(), dxs.data_ptr(), dw.data_ptr(), dws.data_ptr(), y_t.data_ptr(), M, N, K,
                     None, 0, _stream())
    torch.cuda.synchronize()
    ya, yt = f16_tensor_f64(y_a), f16_tensor_f64(y_t)
    assert np.isfinite(ya).all() and np.isfinite(yt).all()
    rows, cols = _sample(g, M, 24), _sample(g, N, 800)
    a, t = ya[np.ix_(rows, cols)], yt[np.ix_(rows, cols)]
    A = _abs_product(xq[rows], xs[rows], wq[cols], ws[cols])
    ulp = np.spacing(np.maximum(np.abs(a), np.abs(t)).astype(np.float16)).astype(np.float64)
    bound = ulp + 2 * K * 2.0 ** -24 * A
    assert (np.abs(a - t) <= bound).all(), (M, N, K, float((np.abs(a - t) / bound).max()))
    # the two orders round differently on few outputs
    assert np.count_nonzero(ya != yt) < 0.05 * ya.size, (M, N, K, np.count_nonzero(ya != yt))
    ref = oracle.gemm_f64(xq[rows], xs[rows], wq[cols], ws[cols])
    assert rel_fro(a, ref) < FRO_TOL
    assert rel_fro(t, ref) < FRO_TOL


@pytest.mark.parametrize("M,N", [(512, 32768), (128, 65536)])
def test_gemm_h16_int_exact_and_group_dots(capi, M, N):
    # unit scales and small codes: integer sums, exact in fp16; then scales 1
    # on one group only and 0 elsewhere: y = D[:, :, g] exactly (M=128: the
    # 128-row tiles)
    g = rng(4510 + M)
    K = 256
    xq = pack_codes(g.integers(-2, 3, (M, K)))
    wq = pack_codes(g.integers(-2, 3, (N, K)))
    xs = np.full((M, K // 32), 0x3F80, np.uint16)
    ws = np.full((N, K // 32), 0x3F80, np.uint16)
    rows, cols = _sample(g, M, 64), _sample(g, N, 2048)
    y = run_gemm(capi, xq, xs, wq, ws)
    D = oracle.group_dots(xq[rows], wq[cols]).astype(np.float64)
    assert np.array_equal(y[np.ix_(rows, cols)], D.sum(axis=2))
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    D = oracle.group_dots(xq[rows], wq[cols]).astype(np.float64)
    for gg in range(K // 32):
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = 0x3F80
        ws[:, gg] = 0x3F80
        y = run_gemm(capi, xq, xs, wq, ws)
        assert np.array_equal(y[np.ix_(rows, cols)], D[:, :, gg]), gg


def _coarse_bf16(g, shape, emin, emax):
    """bf16 bits of (1 + f/4) * 2^E, f in 0..3, E in [emin, emax]: two fraction
    bits, so products of two scales and a group dot stay exact in fp32."""
    f = g.integers(0, 4, shape)
    E = g.integers(emin, emax + 1, shape)
    return ((E + 127) << 7 | f << 5).astype(np.uint16)


def test_gemm_h16_group_dots_nonunit_scales(capi):
    # one group with non-unit scales, all others 0: y = fp16(sx * sw * D[:, :, g])
    # exactly (the row's only nonzero scale is its largest, so every operand
    # converts exactly and the fp32 sum of the 32 terms is exact)
    g = rng(4515)
    M, N, K = 512, 32768, 256
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    rows, cols = _sample(g, M, 64), _sample(g, N, 2048)
    D = oracle.group_dots(xq[rows], wq[cols]).astype(np.float64)
    for gg in range(K // 32):
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = _coarse_bf16(g, M, -8, 0)
        ws[:, gg] = _coarse_bf16(g, N, -8, 0)
        y = run_gemm(capi, xq, xs, wq, ws)[np.ix_(rows, cols)]
        sx = bf16_bits_to_f32(xs[rows, gg]).astype(np.float64)
        sw = bf16_bits_to_f32(ws[cols, gg]).astype(np.float64)
        exact = (sx[:, None] * sw[None, :] * D[:, :, gg]).astype(np.float16).astype(np.float64)
        assert np.array_equal(y, exact), gg


@pytest.mark.parametrize("M,N", [(512, 32768), (128, 65536)])   # 256-row and 128-row tiles
def test_gemm_h16_group_scale_boundary(capi, M, N):
    # One activation group at 2^-k of its row's largest scale (full 8-bit
    # significands; the largest sits in group 0, whose codes are 0), one weight
    # group nonzero.  The shifted largest scale lies in [2^12, 2^13), so the
    # fp16 scale operand of the tested group keeps all 8 bits (lowest bit at
    # or above 2^-24) down to k = 29: y = fp16(sx * sw * D) exactly.  Below,
    # it rounds to fp16's subnormal spacing: each product term is off by at
    # most 2^-31 * sx_max * sw_max (2^-27 taken: generous), on top of the fp32
    # sum of 32 terms and the fp16 rounding of y.
    g = rng(4516 + M)
    K = 256
    G = K // 32
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    codes = unpack_codes(xq)
    codes[:, :32] = 0
    xq = pack_codes(codes)
    rows, cols = _sample(g, M, 64), _sample(g, N, 2048)
    D = oracle.group_dots(xq[rows], wq[cols]).astype(np.float64)
    A = oracle.group_dots(pack_codes(np.abs(unpack_codes(xq[rows]))),
                          pack_codes(np.abs(unpack_codes(wq[cols])))).astype(np.float64)
    top = (((127 + g.integers(-2, 1, M)) << 7) | g.integers(0, 128, M)).astype(np.uint16)   # [0.25, 2)
    for k in (22, 25, 26, 29, 30, 33):
        gg = 1 + k % (G - 1)
        xs = np.zeros((M, G), np.uint16)
        ws = np.zeros((N, G), np.uint16)
        xs[:, 0] = top
        xs[:, gg] = _bf16_times_pow2(top, -k)
        ws[:, gg] = _coarse_bf16(g, N, -4, 0)
        y = run_gemm(capi, xq, xs, wq, ws)[np.ix_(rows, cols)]
        sx = bf16_bits_to_f32(xs[rows, gg]).astype(np.float64)
        sw = bf16_bits_to_f32(ws[cols, gg]).astype(np.float64)
        exact = sx[:, None] * sw[None, :] * D[:, :, gg]
        if k <= 29:
            assert np.array_equal(y, exact.astype(np.float16).astype(np.float64)), k
        else:
            sx_max = bf16_bits_to_f32(top[rows]).astype(np.float64)
            ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
            bound = (0.5 * ulp + 32 * 2.0 ** -24 * sx[:, None] * sw[None, :] * A[:, :, gg]
                     + 32 * 2.0 ** -27 * sx_max[:, None] * sw[None, :])
            assert (np.abs(y - exact) <= bound).all(), k
            if (np.abs(exact) >= 2.0 ** -22).any():   # some outputs well inside fp16's range
                assert np.count_nonzero(y) > 0, k


def _bf16_times_pow2(bits, e):
    """bf16 bits of positive normal values times 2^e (e broadcast), exactly."""
    b = bits.astype(np.int64) + (np.asarray(e, np.int64) << 7)
    assert ((b >> 7) > 0).all() and ((b >> 7) < 255).all()
    return b.astype(np.uint16)


@pytest.mark.parametrize("M,N,K", [(600, 24000, 1024), (100, 49000, 2048)])   # 256-row and 128-row tiles
def test_gemm_h16_scale_range(capi, M, N, K):
    # Scales far outside fp16's range (activation rows near 2^+40, weight
    # columns near 2^-40, and a spread of 2^-12..2^+12 across the groups of a
    # row) so that every row and column needs its own power-of-two shift; the
    # products stay in fp16 range.  Compared with the oracle after removing
    # each row's and column's factor.
    g = rng(4520 + M)
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    dr = g.integers(-3, 2, M)                    # outputs |y| < 2^11 * 2^2 stay finite in fp16
    dc = g.integers(-3, 2, N)
    spread = g.integers(-12, 13, (M, K // 32))
    xs2 = _bf16_times_pow2(xs, 40 + dr[:, None] + spread)
    ws2 = _bf16_times_pow2(ws, -40 + dc[:, None])
    rows, cols = _sample(g, M, 40), _sample(g, N, 1500)
    xs_ref = _bf16_times_pow2(xs, spread)[rows]
    ref = oracle.gemm_f64(xq[rows], xs_ref, wq[cols], ws[cols])
    y = run_gemm(capi, xq, xs2, wq, ws2)[np.ix_(rows, cols)]
    got = y * np.ldexp(1.0, -(dr[rows][:, None] + dc[cols][None, :]))
    assert rel_fro(got, ref) < FRO_TOL, rel_fro(got, ref)


@pytest.mark.parametrize("M,N", [(512, 32768), (120, 57344)])   # 256-row and 128-row tiles
def test_gemm_h16_nonfinite_scales(capi, M, N):
    # a non-finite activation scale makes its row NaN, a non-finite weight
    # scale its column, as in the dequantized product; the rest is unaffected
    g = rng(4530 + M)
    K = 512
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    bad_r, bad_c = [3, M - 12], [5, 20000]
    xs[bad_r[0], 2] = 0x7F80                     # +inf
    xs[bad_r[1], 15] = 0xFFC0                    # NaN
    ws[bad_c[0], 1] = 0x7FC0                     # NaN
    ws[bad_c[1], 9] = 0xFF80                     # -inf
    y = run_gemm(capi, xq, xs, wq, ws)
    assert np.isnan(y[bad_r]).all() and np.isnan(y[:, bad_c]).all()
    rows = np.array([r for r in _sample(g, M, 40) if r not in bad_r])
    cols = np.array([c for c in _sample(g, N, 1500) if c not in bad_c])
    ref = oracle.gemm_f64(xq[rows], xs[rows], wq[cols], ws[cols])
    got = y[np.ix_(rows, cols)]
    assert rel_fro(got, ref) < FRO_TOL, rel_fro(got, ref)


# Shapes the planner sends to the fp16-MFMA streaming kernel (gemm_h16s:
# 32 < M <= 64, 224-column workgroups filling 7/8 to all of 256 CUs, i.e.
# 49953 <= N <= 57344, K % 1024 == 0, 16-byte aligned operands): two 32-row
# activation blocks, the second ragged; ragged N (a partial last column
# block and workgroup); 4 to 32 batches of 8 groups.
H16S_SHAPES = [(33, 50000, 2048), (37, 57344, 1024), (41, 52000, 1024), (48, 56000, 3072), (64, 57344, 6144),
               (40, 57300, 8192), (57, 57344, 4096)]


@pytest.mark.parametrize("M,N,K", H16S_SHAPES)
def test_gemm_h16s_matches_oracle(capi, M, N, K):
    # fp16 operands code*scale (exact), fp32 accumulation over all of K:
    # seeded samples of columns (first and last always) against the fp64
    # oracle, every row, within each output's own bound (fp16 rounding plus
    # 2K rounded fp32 additions) and the 2e-3 gate
    g = rng(4800 + M + N + K)
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    cols = _sample(g, N, 1500)
    y = run_gemm(capi, xq, xs, wq, ws)
    assert np.isfinite(y).all()
    got = y[:, cols]
    ref = oracle.gemm_f64(xq, xs, wq[cols], ws[cols])
    assert rel_fro(got, ref) < FRO_TOL, (M, N, K, rel_fro(got, ref))
    A = _abs_product(xq, xs, wq[cols], ws[cols])
    bound = (np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) + 2 * K * 2.0 ** -24 * A
             + 2.0 ** -25)
    assert (np.abs(got - ref) <= bound).all(), (M, N, K, float((np.abs(got - ref) / bound).max()))


def test_gemm_h16s_int_exact_and_group_dots(capi):
    # unit scales and small codes: integer sums, exact; then scales 1 on one
    # group only (both lane halves and all four positions of an 8-group
    # batch, first and last batches): y = D[:, :, g] exactly
    g = rng(4810)
    M, N, K = 40, 51200, 2048
    xq = pack_codes(g.integers(-2, 3, (M, K)))
    wq = pack_codes(g.integers(-2, 3, (N, K)))
    xs = np.full((M, K // 32), 0x3F80, np.uint16)
    ws = np.full((N, K // 32), 0x3F80, np.uint16)
    cols = _sample(g, N, 1024)
    y = run_gemm(capi, xq, xs, wq, ws)
    D = oracle.group_dots(xq, wq[cols]).astype(np.float64)
    assert np.array_equal(y[:, cols], D.sum(axis=2))
    xq, _, wq, _ = _rand_operands(g, M, N, K)
    D = oracle.group_dots(xq, wq[cols]).astype(np.float64)
    for gg in (0, 7, 8, 15, 16, 31, 33, 47, 56, 63):
        xs = np.zeros((M, K // 32), np.uint16)
        ws = np.zeros((N, K // 32), np.uint16)
        xs[:, gg] = 0x3F80
        ws[:, gg] = 0x3F80
        y = run_gemm(capi, xq, xs, wq, ws)
        assert np.array_equal(y[:, cols], D[:, :, gg]), gg
        assert np.count_nonzero(np.delete(y, cols, axis=1) != 0) > 0


def test_gemm_h16s_scale_range_and_quarters(capi):
    # Scales far outside fp16's range (rows near 2^+40, columns near 2^-40),
    # and a different order of magnitude in each K quarter of a row (2^-12,
    # 2^0, 2^+6, 2^-6), so that a row's shift comes from one quarter and the
    # others sit up to 2^-18 below it (still exact); the row and column
    # factors (2^-3 .. 2^0) keep every output inside fp16's range.  Compared
    # with the oracle after removing each row's and column's factor.
    g = rng(4820)
    M, N, K = 36, 50400, 4096
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    G = K // 32
    dr = g.integers(-3, 1, M)
    dc = g.integers(-3, 1, N)
    quarter = np.repeat(np.array([-12, 0, 6, -6]), G // 4)[None, :]
    xs2 = _bf16_times_pow2(xs, 40 + dr[:, None] + quarter)
    ws2 = _bf16_times_pow2(ws, -40 + dc[:, None])
    cols = _sample(g, N, 1500)
    ref = oracle.gemm_f64(xq, _bf16_times_pow2(xs, quarter + 0 * dr[:, None]), wq[cols], ws[cols])
    y = run_gemm(capi, xq, xs2, wq, ws2)[:, cols]
    assert np.isfinite(y).all()
    got = y * np.ldexp(1.0, -(dr[:, None] + dc[cols][None, :]))
    assert rel_fro(got, ref) < FRO_TOL, rel_fro(got, ref)


def test_gemm_h16s_nonfinite_scales(capi):
    # a non-finite activation scale makes its row NaN, a non-finite weight
    # scale its column (wherever in K it sits); the rest is unaffected
    g = rng(4830)
    M, N, K = 44, 50500, 2048
    xq, xs, wq, ws = _rand_operands(g, M, N, K)
    xs[3, 2] = 0x7F80                            # +inf, quarter 0
    xs[17, 50] = 0xFFC0                          # NaN, quarter 3
    ws[5, 20] = 0x7FC0                           # NaN, quarter 1
    ws[8400, 40] = 0xFF80                        # -inf, quarter 2
    y = run_gemm(capi, xq, xs, wq, ws)
    bad_r, bad_c = [3, 17], [5, 8400]
    assert np.isnan(y[bad_r]).all() and np.isnan(y[:, bad_c]).all()
    rows = np.array([r for r in range(M) if r not in bad_r])
    cols = np.array([c for c in _sample(g, N, 1500) if c not in bad_c])
    ref = oracle.gemm_f64(xq[rows], xs[rows], wq[cols], ws[cols])
    got = y[np.ix_(rows, cols)]
    assert np.isfinite(got).all()
    assert rel_fro(got, ref) < FRO_TOL, rel_fro(got, ref)


def test_gemm_golden_fixture(capi):
    gm = np.load(os.path.join(GOLDEN, "gemm_small.npz"))
    y = run_gemm(capi, gm["xq"], gm["xs"], gm["wq"], gm["ws"])
    assert rel_fro(y, gm["y_f64"]) < FRO_TOL
    y = run_gemm(capi, gm["xq"], gm["xs"], gm["wq"], gm["ws"], "gemv")
    assert rel_fro(y, gm["y_f64"]) < FRO_TOL


def test_gemm_zero_activations(capi):
    g = rng(4300)
    xq = np.zeros((4, 32), np.uint8)
    xs = np.full((4, 2), 0x322C, np.uint16)
    _, _, wq, ws = _rand_operands(g, 1, 16, 64)
    assert (run_gemm(capi, xq, xs, wq, ws) == 0).all()
    assert (run_gemm(capi, xq, xs, wq, ws, "gemv") == 0).all()


def test_mfma_selftest(capi):
    import torch
    g = rng(5000)
    a = g.integers(-8, 8, (8, 32)).astype(np.int8)
    b = g.integers(-8, 8, (32, 8)).astype(np.int8)
    da = torch.from_numpy(a).cuda()
    db = torch.from_numpy(b).cuda()
    c = torch.zeros(8, 8, dtype=torch.int32, device="cuda")
    capi.mfma_selftest(da.data_ptr(), db.data_ptr(), c.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), oracle.int_matmul_8x32x8(a, b))


# --------------------------------------------------------------- per-tensor
def test_per_tensor_quant_and_gemm(capi):
    import torch
    g = rng(6000)
    for shape in [(1, 4096), (64, 4096), (2048, 512)]:
        x = f32_to_bf16_bits(g.standard_normal(shape))
        amax = float(np.abs(bf16_bits_to_f32(x)).max())
        inv = np.float32(1.0 / (amax / 7.0))
        xt = to_dev_bf16(x)
        q = torch.empty(x.size // 2, dtype=torch.uint8, device="cuda")
        capi.quant_int4_tensor_scale(xt.data_ptr(), q.data_ptr(), x.size, float(inv), None, _stream())
        inv_dev = torch.tensor([inv], dtype=torch.float32, device="cuda")
        q2 = torch.empty_like(q)
        capi.quant_int4_tensor_scale(xt.data_ptr(), q2.data_ptr(), x.size, 0.0, inv_dev.data_ptr(), _stream())
        torch.cuda.synchronize()
        qo = oracle.quant_tensor_scale(x, inv)
        assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(q2.cpu().numpy(), qo)
    for M, N, K in [(64, 96, 128), (1, 256, 64), (300, 500, 512), (8, 4096, 4096)]:
        xq = pack_codes(g.integers(-7, 8, (M, K)))
        wq = pack_codes(g.integers(-7, 8, (N, K)))
        alpha = 1.0 / 64.0
        dx, dw = to_dev_u8(xq), to_dev_u8(wq)
        y = torch.empty(M, N, dtype=torch.float16, device="cuda")
        capi.gemm_s4_tensor_scale(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), M, N, K, alpha, None, _stream())
        a_dev = torch.tensor([alpha], dtype=torch.float32, device="cuda")
        y2 = torch.empty_like(y)
        capi.gemm_s4_tensor_scale(dx.data_ptr(), dw.data_ptr(), y2.data_ptr(), M, N, K, 0.0,
                                  a_dev.data_ptr(), _stream())
        torch.cuda.synchronize()
        ref = oracle.gemm_tensor_scale_f64(xq, wq, alpha)
        assert rel_fro(f16_tensor_f64(y), ref) < FRO_TOL
        assert np.array_equal(f16_tensor_f64(y), f16_tensor_f64(y2))


def test_per_tensor_largest_k(capi):
    """K = 131040, the largest K the per-tensor GEMM admits (256 * 64 * K < 2^31):
    codes of -8 in both operands put every int32 accumulator at its extreme,
    256 * 64 * K; the result must equal the exact product (no wrap-around).
    Random codes in [-8, 7] are checked against the fp64 oracle."""
    import torch
    from wush_int4_kernel_amd import capi as c
    K = 131040
    assert 256 * 64 * K < 2 ** 31
    M, N = 4, 64
    alpha = 2.0 ** -14
    xq = pack_codes(np.full((M, K), -8))
    wq = pack_codes(np.full((N, K), -8))
    dx, dw = to_dev_u8(xq), to_dev_u8(wq)
    y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    c.gemm_s4_tensor_scale(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), M, N, K, alpha, None, _stream())
    torch.cuda.synchronize()
    exact = np.float16(64.0 * K * alpha)
    assert np.all(y.cpu().numpy() == exact), (y.cpu().numpy()[0, :4], exact)
    g = rng(6100)
    xq = pack_codes(g.integers(-8, 8, (M, K)))
    wq = pack_codes(g.integers(-8, 8, (N, K)))
    dx, dw = to_dev_u8(xq), to_dev_u8(wq)
    c.gemm_s4_tensor_scale(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), M, N, K, 1.0 / 1024, None, _stream())
    torch.cuda.synchronize()
    ref = oracle.gemm_tensor_scale_f64(xq, wq, 1.0 / 1024)
    assert rel_fro(f16_tensor_f64(y), ref) < FRO_TOL
    with pytest.raises(RuntimeError, match="invalid argument"):
        c.gemm_s4_tensor_scale(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), M, N, K + 32, 1.0, None, _stream())


def test_invalid_arguments_rejected(capi):
    import torch
    x = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    q = torch.empty(32, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="invalid argument"):
        capi.quant_int4(x.data_ptr(), 7, q.data_ptr(), q.data_ptr(), 2, _stream())
    with pytest.raises(RuntimeError, match="invalid argument"):
        capi.fused_tq(x.data_ptr(), x.data_ptr(), q.data_ptr(), q.data_ptr(), 1, 48, _stream())
    with pytest.raises(RuntimeError, match="invalid argument"):
        capi.gemv_int4(q.data_ptr(), x.data_ptr(), q.data_ptr(), x.data_ptr(), x.data_ptr(), 9, 1, 64, _stream())
