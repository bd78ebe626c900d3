"""CPU tests that pin the oracle before anything is checked against it.

Each oracle function is tied to something other than itself:
  * the reference tests' known answers, recomputed by hand
    (tests/test_rtn_int4.py:9-45, tests/test_s2.py:25-36 of the reference);
  * an exact-rational binary32 emulation of the quantizer (tests/_fp32_exact.py);
  * a second, independently written numpy restatement (oracle/rtn_np.py);
  * closed forms: single-nonzero groups, permutation / diagonal / identity
    transforms, brute-force integer products.
A plausible slip -- a dropped term of the variance, a transposed T, a swapped
nibble, FMA contraction, a wrong rounding mode -- fails at least one of these.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import rtn_np
from _fp32_exact import quant_group as exact_quant_group
from _util import (bf16_bits_to_f32, f32_to_bf16_bits, outlier_activations, pack_codes, rng,
                   unpack_codes)


# --------------------------------------------------------------- known answers
def test_kat_alternating_pm1():
    # reference tests/test_rtn_int4.py:9-20: +-1 alternating -> sigma = 1,
    # scale = C_CLIP (+1e-8 absorbed) -> bf16 0x3EB5 = 0.353515625,
    # 1/0.3535 = 2.83 -> codes +-3 -> bytes 0x3 | 0xD << 4 = 0xD3.
    x = np.zeros((1, 32), np.float32)
    x[0, 0::2] = 1.0
    x[0, 1::2] = -1.0
    q, s = oracle.quant(x)
    assert s[0, 0] == 0x3EB5
    assert (q == 0xD3).all()
    d = oracle.dequant(q, s)
    assert np.array_equal(d[0], np.array([3, -3] * 16, np.float32) * np.float32(0.353515625))


def test_kat_zero_group():
    # reference tests/test_rtn_int4.py:34-38: sigma = 0 -> scale = 1e-8 -> bf16
    # 0x322C, codes 0.
    q, s = oracle.quant(np.zeros((4, 32), np.float32))
    assert (s == 0x322C).all() and (q == 0).all()


def test_kat_overflow_group():
    # reference tests/test_s2.py:31-36: sum x^2 = inf -> var = NaN -> scale 1.0
    # (bf16 0x3F80), codes saturate at +7 -> 0x77.
    x = f32_to_bf16_bits(np.full((4, 32), 3.3e38, np.float32))
    q, s = oracle.quant(x, "bf16")
    assert (s == 0x3F80).all() and (q == 0x77).all()


def test_kat_constants():
    assert np.float32(0.35337862372398376).view(np.uint32) == 0x3EB4EE0B
    assert np.float32(1e-8).view(np.uint32) == 0x322BCC77
    # the stale comment value 2.473650/7 would be a different constant
    assert np.float32(2.473650 / 7).view(np.uint32) != 0x3EB4EE0B


def test_kat_ties_match_exact_emulation():
    # reference tests/test_s2.py:25-29 tie groups
    x = np.zeros((2, 32), np.float32)
    x[0, :8] = [7.0, -7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5]
    x[1, :8] = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -6.5], np.float32) * np.float32(0.7)
    xb = f32_to_bf16_bits(x)
    q, s = oracle.quant(xb, "bf16")
    xv = bf16_bits_to_f32(xb)
    for r in range(2):
        bits, codes = exact_quant_group([float(v) for v in xv[r]])
        assert s[r, 0] == bits
        assert np.array_equal(unpack_codes(q[r]), np.array(codes))


def test_single_nonzero_groups_closed_form():
    # One nonzero v at position p: mean = v/32, var = 31 v^2 / 1024, so
    # |v| / scale = 32 / (sqrt(31) * C_CLIP) = 16.26 > 7: code sign(v)*7 at p and
    # 0 elsewhere (exactly 0/scale).  Every position exercises the nibble order.
    vals = [1.0, -1.0, 3.0, -0.125, 1e-3, -250.0]
    for p in range(32):
        for v in vals:
            x = np.zeros((1, 32), np.float32)
            x[0, p] = v
            q, s = oracle.quant(x)
            codes = unpack_codes(q[0])
            expect = np.zeros(32, np.int32)
            expect[p] = 7 if v > 0 else -7
            assert np.array_equal(codes, expect), (p, v)
            bits, _ = exact_quant_group(list(x[0]))
            assert s[0, 0] == bits


def _exact_check(x: np.ndarray):
    q, s = oracle.quant(x)
    for r in range(x.shape[0]):
        bits, codes = exact_quant_group([float(v) for v in x[r]])
        assert s[r, 0] == bits, (r, hex(s[r, 0]), hex(bits))
        assert np.array_equal(unpack_codes(q[r]), np.array(codes)), r


def test_exact_emulation_random_groups():
    g = rng(11)
    cases = [
        g.standard_normal((40, 32)).astype(np.float32),
        (g.standard_normal((20, 32)) * 1e-20).astype(np.float32),      # tiny values
        (g.standard_normal((20, 32)) * 1e15).astype(np.float32),       # large values
        np.round(g.standard_normal((40, 32)) * 4) / 2,                 # half-integer grid: ties
        (g.integers(-3, 4, (40, 32)) * 0.25).astype(np.float32),       # coarse grid
    ]
    mixed = g.standard_normal((20, 32)).astype(np.float32)
    mixed[:, 3] *= 50.0                                                # outlier channel
    cases.append(mixed)
    for c in cases:
        _exact_check(np.ascontiguousarray(c, dtype=np.float32))


def test_exact_emulation_denormal_inputs():
    g = rng(12)
    x = (g.standard_normal((10, 32)) * 1e-39).astype(np.float32)   # binary32 subnormals
    assert (np.abs(x[x != 0]) < np.finfo(np.float32).tiny).all()
    _exact_check(x)


def test_c_and_numpy_restatements_agree():
    g = rng(13)
    x = bf16_bits_to_f32(outlier_activations(g, 64, 512))
    q1, s1 = oracle.quant(x)
    q2, s2 = rtn_np.quant(x)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    # bf16 and f16 entry points agree with the fp32 one on the same values
    xb = f32_to_bf16_bits(x)
    q3, s3 = oracle.quant(xb, "bf16")
    assert np.array_equal(q1, q3) and np.array_equal(s1, s3)
    xh = x.astype(np.float16)
    q4, s4 = oracle.quant(xh.view(np.uint16), "f16")
    q5, s5 = oracle.quant(xh.astype(np.float32))
    assert np.array_equal(q4, q5) and np.array_equal(s4, s5)


def test_torch_restatement_matches_c_oracle():
    # oracle/rtn_torch.py (the CPU baseline's timed path) bit for bit against
    # the C oracle: outlier activations, ties, overflow, zero, NaN and inf groups
    import torch
    from oracle import rtn_torch
    g = rng(16)
    x = bf16_bits_to_f32(outlier_activations(g, 32, 1024))
    special = np.zeros((6, 32), np.float32)
    special[0] = np.where(np.arange(32) % 2 == 0, 1.0, -1.0)      # test_rtn_int4.py:9-20
    special[2] = 3.3e38                                            # test_s2.py:31-36
    special[3, 5] = np.nan
    special[4, 7] = np.inf
    special[5] = np.float32(0.35353515625) * (np.arange(32) - 15.5)  # many quotients near ties
    for arr in (x, special):
        q1, s1 = oracle.quant(arr)
        q2, s2 = rtn_torch.quant(torch.from_numpy(arr))
        assert np.array_equal(q2.numpy(), q1)
        assert np.array_equal(s2.view(torch.int16).numpy().view(np.uint16), s1)
        d1 = oracle.dequant(q1, s1)
        d2 = rtn_torch.dequant(q2, s2).numpy()
        assert np.array_equal(d1, d2, equal_nan=True)
    wq, ws = oracle.quant(bf16_bits_to_f32(f32_to_bf16_bits(g.standard_normal((64, 1024)) * 0.02)))
    xq, xs = oracle.quant(x[:4])
    y = rtn_torch.w4a4_matmul(torch.from_numpy(xq), torch.from_numpy(xs.view(np.int16)).view(torch.bfloat16),
                              torch.from_numpy(wq), torch.from_numpy(ws.view(np.int16)).view(torch.bfloat16))
    ref = oracle.gemm_f64(xq, xs, wq, ws)
    assert np.abs(y.double().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


def test_dequant_error_bound_and_shapes():
    # reference tests/test_rtn_int4.py:22-32 (|x - dq| <= 6*scale) and :40-45 (shapes)
    g = rng(14)
    x = bf16_bits_to_f32(f32_to_bf16_bits(g.standard_normal((2048, 128))))
    q, s = oracle.quant(x)
    assert q.shape == (2048, 64) and s.shape == (2048, 4)
    d = oracle.dequant(q, s)
    err = np.abs(d - x).reshape(2048, 4, 32)
    assert (err <= bf16_bits_to_f32(s)[..., None] * 6.0).all()
    x3 = g.standard_normal((2, 3, 96)).astype(np.float32)
    q3, s3 = oracle.quant(x3)
    assert q3.shape == (2, 3, 48) and s3.shape == (2, 3, 3)
    assert oracle.dequant(q3, s3).shape == (2, 3, 96)
    # numpy dequant restatement agrees
    assert np.array_equal(rtn_np.dequant(q, s), d)


def test_codes_in_range_and_nan_is_zero():
    g = rng(15)
    x = (g.standard_normal((100, 32)) * 10).astype(np.float32)
    x[0, 5] = np.nan
    q, s = oracle.quant(x)
    c = unpack_codes(q)
    assert c.min() >= -7 and c.max() <= 7
    assert c[0, 5] == 0 and s[0, 0] == 0x3F80          # NaN group: scale 1.0, NaN code 0


# ------------------------------------------------------------------ transform
def _perm_T(g, C):
    """Block permutation matrices with no fixed points and pi != pi^-1."""
    T = np.zeros((C, 32, 32), np.float32)
    perms = []
    for c in range(C):
        while True:
            p = g.permutation(32)
            if (p != np.arange(32)).all() and not np.array_equal(p[p], np.arange(32)):
                break
        T[c, np.arange(32), p] = 1.0            # x'_j = x_{p[j]}
        perms.append(p)
    return T, perms


def test_transform_permutation_closed_form():
    g = rng(21)
    K, C = 128, 4
    xb = outlier_activations(g, 16, K)
    T, perms = _perm_T(g, C)
    xp = oracle.transform(xb, f32_to_bf16_bits(T))
    xv = bf16_bits_to_f32(xb)
    for c in range(C):
        assert np.array_equal(xp[:, c * 32:(c + 1) * 32], xv[:, c * 32 + perms[c]])
    # fused == quant of the permuted activations
    q, s = oracle.fused_tq(xb, f32_to_bf16_bits(T))
    xperm = np.concatenate([xv[:, c * 32 + perms[c]] for c in range(C)], axis=1)
    q2, s2 = oracle.quant(xperm)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_transform_diagonal_and_identity():
    g = rng(22)
    K, C = 96, 3
    xb = outlier_activations(g, 8, K)
    xv = bf16_bits_to_f32(xb)
    d = (2.0 ** g.integers(-3, 4, (C, 32))).astype(np.float32)
    T = np.zeros((C, 32, 32), np.float32)
    for c in range(C):
        T[c] = np.diag(d[c])
    xp = oracle.transform(xb, f32_to_bf16_bits(T))
    assert np.array_equal(xp, xv * d.reshape(-1))
    eye = np.broadcast_to(np.eye(32, dtype=np.float32), (C, 32, 32))
    q, s = oracle.fused_tq(xb, f32_to_bf16_bits(eye))
    q2, s2 = oracle.quant(xb, "bf16")
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_transform_c_vs_numpy_random_T():
    g = rng(23)
    K = 256
    xb = outlier_activations(g, 32, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)))
    xp = oracle.transform(xb, tb)
    xp2 = rtn_np.transform(bf16_bits_to_f32(xb), bf16_bits_to_f32(tb))
    assert np.array_equal(xp, xp2)
    # fp64 closed form X T^T per block (wush_transform.py:54-58) within fp32 rounding
    ref = np.einsum("rci,cji->rcj", bf16_bits_to_f32(xb).reshape(32, -1, 32).astype(np.float64),
                    bf16_bits_to_f32(tb).astype(np.float64)).reshape(32, K)
    assert np.allclose(xp, ref, rtol=1e-5, atol=1e-4 * np.abs(ref).max())


def test_transform_rounding_order_exact_emulation():
    # x'_j = RN(...RN(RN(x_0*T_j0) + RN(x_1*T_j1))...), i ascending, every
    # product and sum rounded (tests/test_sw2.py:12-24), evaluated exactly
    # with Fractions, then the exact quantizer: the C oracle's transform and
    # fused codes/scales must match bit for bit.  Random bf16 T; reversing the
    # order changes x' on this data, so the check sees the order.  A product of
    # two bf16 values is exact in fp32, so contracting to an fma leaves x'
    # unchanged here -- the equivalence the GPU kernel's fma loop relies on.
    from _fp32_exact import transform_block
    g = rng(24)
    rows, K = 3, 128
    xb = outlier_activations(g, rows, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.3)
    xv, tv = bf16_bits_to_f32(xb), bf16_bits_to_f32(tb)
    xp = oracle.transform(xb, tb)
    q, s = oracle.fused_tq(xb, tb)
    exact = np.zeros((rows, K), np.float32)
    rev_differs, fma_same = False, False
    for r in range(rows):
        codes = []
        for c in range(K // 32):
            blk = transform_block(xv[r, c * 32:(c + 1) * 32], tv[c])
            exact[r, c * 32:(c + 1) * 32] = [float(v) for v in blk]
            bits, cq = exact_quant_group(exact[r, c * 32:(c + 1) * 32])
            assert s[r, c] == bits, (r, c)
            codes.extend(cq)
            if r == 0 and c == 0:
                rev = transform_block(xv[r, :32], tv[0], order=range(31, -1, -1))
                fma = transform_block(xv[r, :32], tv[0], fused=True)
                rev_differs = rev != blk
                fma_same = fma == blk
        assert np.array_equal(q[r], pack_codes(np.array(codes))), r
    assert np.array_equal(xp.view(np.uint32), exact.view(np.uint32))
    assert rev_differs and fma_same


# ---------------------------------------------------------------------- GEMM
def test_group_dots_brute_force():
    g = rng(31)
    M, N, K = 3, 5, 96
    cx = g.integers(-7, 8, (M, K))
    cw = g.integers(-7, 8, (N, K))
    D = oracle.group_dots(pack_codes(cx), pack_codes(cw))
    for m in range(M):
        for n in range(N):
            for gg in range(K // 32):
                sl = slice(gg * 32, gg * 32 + 32)
                assert D[m, n, gg] == int(np.dot(cx[m, sl], cw[n, sl]))


def test_gemm_f64_closed_form():
    g = rng(32)
    M, N, K = 7, 9, 128
    xq, xs = oracle.quant(g.standard_normal((M, K)).astype(np.float32))
    wq, ws = oracle.quant((g.standard_normal((N, K)) * 0.02).astype(np.float32))
    Y = oracle.gemm_f64(xq, xs, wq, ws)
    ref = oracle.dequant(xq, xs).astype(np.float64) @ oracle.dequant(wq, ws).astype(np.float64).T
    assert np.allclose(Y, ref, rtol=1e-12, atol=1e-12)
    # unit scales: Y is the plain integer product of the codes
    ones = np.full((M, K // 32), 0x3F80, np.uint16)
    onesw = np.full((N, K // 32), 0x3F80, np.uint16)
    Yi = oracle.gemm_f64(xq, ones, wq, onesw)
    assert np.array_equal(Yi, (unpack_codes(xq) @ unpack_codes(wq).T).astype(np.float64))


def test_per_tensor_quant_mirror():
    # reference tests/test_p12.py:21-26: code = clamp(rint(x * inv), -7, 7)
    x = np.linspace(-8.5, 8.5, 4096, dtype=np.float32)
    xb = f32_to_bf16_bits(x)
    q = oracle.quant_tensor_scale(xb, np.float32(1.0))
    xv = bf16_bits_to_f32(xb).astype(np.float64)
    expect = np.clip(np.array([float(np.rint(v)) for v in xv]), -7, 7).astype(np.int32)
    assert np.array_equal(unpack_codes(q), expect)
    g = rng(33)
    xq = pack_codes(g.integers(-7, 8, (4, 64)))
    wq = pack_codes(g.integers(-7, 8, (6, 64)))
    Y = oracle.gemm_tensor_scale_f64(xq, wq, 0.5)
    assert np.array_equal(Y, 0.5 * (unpack_codes(xq) @ unpack_codes(wq).T))


def test_int_matmul_selftest_reference():
    g = rng(34)
    a = g.integers(-8, 8, (8, 32)).astype(np.int8)
    b = g.integers(-8, 8, (32, 8)).astype(np.int8)
    assert np.array_equal(oracle.int_matmul_8x32x8(a, b), a.astype(np.int32) @ b.astype(np.int32))


# ------------------------------------------------------------------- fixtures
def test_golden_fixtures_match_oracle():
    import os
    here = os.path.join(os.path.dirname(__file__), "golden")
    kat = np.load(os.path.join(here, "quant_kat.npz"))
    q, s = oracle.quant(kat["x_bf16"], "bf16")
    assert np.array_equal(q, kat["q"]) and np.array_equal(s, kat["s"])
    fz = np.load(os.path.join(here, "fused_small.npz"))
    q, s = oracle.fused_tq(fz["x_bf16"], fz["t_bf16"])
    assert np.array_equal(q, fz["q"]) and np.array_equal(s, fz["s"])
    gm = np.load(os.path.join(here, "gemm_small.npz"))
    Y = oracle.gemm_f64(gm["xq"], gm["xs"], gm["wq"], gm["ws"])
    assert np.array_equal(Y, gm["y_f64"])
