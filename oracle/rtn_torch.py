"""torch (CPU) restatement of the reference's rtn path -- TEST INFRASTRUCTURE ONLY.

Used by tests/ as a checker and by bench.py's cpu_baseline leg as the timed CPU
path; never by the product.  It follows my_int4/rtn_int4.py operation for
operation with eager torch CPU ops, which round every operation to nearest even
and do not contract a*b+c:
  * quant_int4 (rtn_int4.py:33-55): a 32-step sequential sum of x and x*x
    (:22-30), mean and variance, scale = sqrt(var)*C_CLIP + 1e-8 (1.0 when
    var < 0 or NaN), the bf16 round trip of the scale, IEEE division, round half
    to even, clamp to [-7, 7], element 2k in the low nibble of byte k;
  * dequant_int4 (:58-68): nibble sign extension by <<12 >>12 on int16, times the
    scale as fp32;
  * w4a4_matmul_reference (:71-75): dequant both operands, fp32 matmul.
The reference's int8 cast of a NaN quotient is left undefined by torch; like
oracle/wush_oracle.c this restatement maps NaN to code 0.  tests/
test_oracle_pinning.py checks it bit for bit against the C oracle.
"""
from __future__ import annotations

import torch

C_CLIP = 0.35337862372398376   # rtn_int4.py:19 (fp32 0x3EB4EE0B)
EPS = 1e-8                     # rtn_int4.py:44


def quant(x: torch.Tensor, group_size: int = 32):
    """-> (q uint8 (..., K/2), s bf16 (..., K/32))."""
    xf = x.float()
    g = xf.reshape(*xf.shape[:-1], -1, group_size)
    s1 = torch.zeros(g.shape[:-1], dtype=torch.float32)
    s2 = torch.zeros(g.shape[:-1], dtype=torch.float32)
    for i in range(group_size):
        v = g[..., i]
        s1 = s1 + v
        s2 = s2 + v * v
    mean = s1 / group_size
    var = s2 / group_size - mean * mean
    c = torch.tensor(C_CLIP, dtype=torch.float32)
    scale = torch.where(var >= 0, torch.sqrt(var) * c + EPS, torch.ones_like(var))
    s = scale.to(torch.bfloat16)
    y = g / s.float().unsqueeze(-1)
    r = torch.clamp(torch.round(y), -7, 7)
    r = torch.where(torch.isnan(r), torch.zeros_like(r), r)
    q = r.to(torch.int8).reshape(*xf.shape[:-1], -1)
    lo = q[..., 0::2].to(torch.int16) & 0xF
    hi = (q[..., 1::2].to(torch.int16) & 0xF) << 4
    return (lo | hi).to(torch.uint8), s


def dequant(q: torch.Tensor, s: torch.Tensor, group_size: int = 32) -> torch.Tensor:
    """-> fp32 (..., K)."""
    qi = q.to(torch.int16)
    lo = ((qi & 0xF) << 12) >> 12
    hi = ((qi >> 4) << 12) >> 12
    d = torch.stack([lo, hi], dim=-1).reshape(*q.shape[:-1], -1, group_size).float()
    return (d * s.float().unsqueeze(-1)).reshape(*q.shape[:-1], -1)


def w4a4_matmul(xq, xs, wq, ws) -> torch.Tensor:
    """dequant(x) @ dequant(w).T in fp32 (the reference then casts to fp16)."""
    return dequant(xq, xs) @ dequant(wq, ws).T
