"""Writes the small golden fixtures under tests/golden/.

The reference keeps no stored vectors (its known answers are computed inline
in its tests), so the fixtures are:
  * quant_kat.npz   -- the reference tests' known-answer groups
    (tests/test_rtn_int4.py:9-38, tests/test_s2.py:25-36 of the reference)
    plus single-nonzero groups and a seeded outlier block, with the oracle's
    codes and bf16 scale bits (the known answers themselves are asserted
    independently in tests/test_oracle_pinning.py);
  * fused_small.npz -- seeded activations and a random bf16 T, oracle output;
  * gemm_small.npz  -- seeded codes/scales and the fp64 product.
They freeze the pinned oracle so a later change to it is caught, and they
travel to the GPU box where the GPU tests compare against them directly.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from _util import f32_to_bf16_bits, outlier_activations, rng  # noqa: E402


def kat_inputs() -> np.ndarray:
    rows = []
    a = np.zeros(32, np.float32)
    a[0::2], a[1::2] = 1.0, -1.0
    rows.append(a)                                        # +-1 alternating
    rows.append(np.zeros(32, np.float32))                 # zero group
    rows.append(np.full(32, 3.3e38, np.float32))          # overflow
    t = np.zeros(32, np.float32)
    t[:8] = [7.0, -7.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5]
    rows.append(t)                                        # ties
    t2 = np.zeros(32, np.float32)
    t2[:8] = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -6.5], np.float32) * np.float32(0.7)
    rows.append(t2)
    for p in range(32):                                   # single nonzero at every position
        e = np.zeros(32, np.float32)
        e[p] = (-1.0) ** p * (p + 1) * 0.37
        rows.append(e)
    g = rng(100)
    blk = outlier_activations(g, 8, 256)
    kat = f32_to_bf16_bits(np.stack(rows))
    kat = np.concatenate([kat, blk.reshape(-1, 32)], axis=0)
    return kat


def main():
    x = kat_inputs()
    q, s = oracle.quant(x, "bf16")
    np.savez_compressed(os.path.join(HERE, "quant_kat.npz"), x_bf16=x, q=q, s=s)

    g = rng(101)
    K = 256
    xb = outlier_activations(g, 24, K)
    tb = f32_to_bf16_bits(g.standard_normal((K // 32, 32, 32)) * 0.3)
    q, s = oracle.fused_tq(xb, tb)
    np.savez_compressed(os.path.join(HERE, "fused_small.npz"), x_bf16=xb, t_bf16=tb, q=q, s=s)

    g = rng(102)
    M, N, K = 5, 40, 192
    xq, xs = oracle.quant(outlier_activations(g, M, K), "bf16")
    wq, ws = oracle.quant(f32_to_bf16_bits(g.standard_normal((N, K)) * 0.02), "bf16")
    y = oracle.gemm_f64(xq, xs, wq, ws)
    np.savez_compressed(os.path.join(HERE, "gemm_small.npz"), xq=xq, xs=xs, wq=wq, ws=ws, y_f64=y)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
