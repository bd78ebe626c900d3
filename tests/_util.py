"""Shared helpers for the tests: seeded inputs, bit-pattern conversions,
pack/unpack of the INT4 format.  Inputs are generated on the CPU with numpy's
PCG64 so the same seed gives the same data here and on the GPU box."""
from __future__ import annotations

import numpy as np

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def f32_to_bf16_bits(a) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def outlier_activations(g: np.random.Generator, M: int, K: int, frac: float = 0.01,
                        scale: float = 50.0) -> np.ndarray:
    """N(0,1) activations with round(frac*K) channels scaled by `scale` (bf16 bits)."""
    x = g.standard_normal((M, K), dtype=np.float32)
    n_out = int(round(frac * K))
    ch = g.choice(K, size=n_out, replace=False)
    x[:, ch] *= scale
    return f32_to_bf16_bits(x)


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """int codes (..., K) in [-8, 7] -> packed uint8 (..., K/2), element 2k low nibble."""
    c = codes.astype(np.int8).astype(np.uint8)
    return ((c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_codes(q: np.ndarray) -> np.ndarray:
    lo = (q & 0xF).astype(np.int8)
    hi = (q >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    return np.stack([lo, hi], axis=-1).reshape(q.shape[:-1] + (-1,)).astype(np.int32)


# ------------------------------------------------------------ torch bridges
def to_dev_bf16(bits: np.ndarray, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def to_dev_u8(a: np.ndarray, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)


def bf16_tensor_bits(t) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16_tensor_f64(t) -> np.ndarray:
    return t.detach().cpu().float().numpy().astype(np.float64)


def rel_fro(y: np.ndarray, ref: np.ndarray) -> float:
    num = np.linalg.norm((y - ref).ravel())
    den = np.linalg.norm(ref.ravel())
    return float(num / den) if den > 0 else float(num)


def product_check(y: np.ndarray, xq, xs, wq, ws, n_terms: int, chunk: int = 4096):
    """Whole-output check of a W4A4 product y (M, N) against the fp64 value of
    dequant(xq, xs) @ dequant(wq, ws)^T (the oracle's dequantization, summed in
    fp64 over weight-row chunks).

    Returns (relative Frobenius error, worst ratio of |y - ref| to the
    per-element bound 2^-11 |ref| + 1.01 * n_terms * 2^-24 * (|X| @ |W|^T) +
    2^-25): the fp16 output rounding plus an fp32 summation of at most n_terms
    rounded additions of exact terms, plus half of fp16's smallest subnormal.
    The Frobenius gate alone could hide one wrong column among tens of
    thousands; the bound holds for every output of a correct product."""
    import oracle
    xq = np.ascontiguousarray(xq).reshape(-1, xq.shape[-1])
    M, N = xq.shape[0], wq.shape[0]
    assert y.shape == (M, N), (y.shape, M, N)
    X = oracle.dequant(xq, np.ascontiguousarray(xs).reshape(M, -1)).astype(np.float64)
    Xa = np.abs(X)
    num = den = 0.0
    worst = 0.0
    for c0 in range(0, N, chunk):
        c1 = min(N, c0 + chunk)
        W = oracle.dequant(wq[c0:c1], ws[c0:c1]).astype(np.float64)
        ref = X @ W.T
        A = Xa @ np.abs(W).T
        yy = y[:, c0:c1]
        assert np.isfinite(yy).all() or not np.isfinite(ref).all(), "non-finite output"
        d = np.abs(yy - ref)
        num += float((d * d).sum())
        den += float((ref * ref).sum())
        bound = 2.0 ** -11 * np.abs(ref) + 1.01 * n_terms * 2.0 ** -24 * A + 2.0 ** -25
        worst = max(worst, float((d / bound).max()))
    return (num / den) ** 0.5 if den > 0 else num ** 0.5, worst
