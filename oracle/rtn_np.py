"""numpy restatement of the reference quantizer -- TEST INFRASTRUCTURE ONLY.

Written independently of ``wush_oracle.c`` so the two can be checked against
each other bit for bit.  numpy float32 ufuncs round every operation to nearest
even and never contract a*b+c, which is the arithmetic of the reference's
eager torch path (my_int4/rtn_int4.py:22-55).
"""
from __future__ import annotations

import numpy as np

C_CLIP = np.float32(0.35337862372398376)  # rtn_int4.py:19 -> fp32 0x3EB4EE0B
EPS = np.float32(1e-8)                    # rtn_int4.py:44 -> fp32 0x322BCC77


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (RNE) -> fp32, returning (bits, value)."""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    bits[nan] = 0x7FC0
    val = (bits.astype(np.uint32) << 16).view(np.float32)
    return bits, val


def quant(x: np.ndarray):
    """rtn_int4.quant_int4 on an fp32 array (..., K)."""
    xf = np.asarray(x, dtype=np.float32)
    g = xf.reshape(xf.shape[:-1] + (-1, 32))
    s1 = np.zeros(g.shape[:-1], np.float32)
    s2 = np.zeros(g.shape[:-1], np.float32)
    for i in range(32):                      # rtn_int4.py:26-29, i ascending
        v = g[..., i]
        s1 = s1 + v
        s2 = s2 + v * v
    with np.errstate(all="ignore"):
        mean = s1 / np.float32(32.0)
        var = s2 / np.float32(32.0) - mean * mean
        scale = np.where(var >= 0, np.sqrt(var) * C_CLIP + EPS, np.float32(1.0)).astype(np.float32)
        bits, sdq = _bf16_round(scale)
        y = g / sdq[..., None]
        r = np.rint(y)
        r = np.where(np.isnan(r), np.float32(0), np.clip(r, -7, 7))
    c = r.astype(np.int8).astype(np.uint8)
    byte = (c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)
    return byte.reshape(xf.shape[:-1] + (-1,)).astype(np.uint8), bits


def dequant(q: np.ndarray, s_bits: np.ndarray) -> np.ndarray:
    """rtn_int4.dequant_int4: nibble sign extension, times float(scale)."""
    q = np.asarray(q, dtype=np.uint8)
    lo = (q & 0xF).astype(np.int16)
    hi = (q >> 4).astype(np.int16)
    lo = ((lo << 12) >> 12).astype(np.int16)   # rtn_int4.py:64-65
    hi = ((hi << 12) >> 12).astype(np.int16)
    d = np.stack([lo, hi], axis=-1).reshape(q.shape[:-1] + (-1, 32)).astype(np.float32)
    sv = (np.asarray(s_bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    return (d * sv[..., None]).reshape(q.shape[:-1] + (-1,))


def transform(x: np.ndarray, t: np.ndarray) -> np.ndarray:
    """ref_fused's transform (test_sw2.py:14-23): fp32, i ascending, mul then add."""
    xf = np.asarray(x, dtype=np.float32)
    tf = np.asarray(t, dtype=np.float32)            # (C, 32, 32) = T[c][j][i]
    g = xf.reshape(xf.shape[:-1] + (-1, 32))         # (..., C, 32)
    out = np.zeros(g.shape, np.float32)
    for i in range(32):
        out = out + g[..., :, i][..., None] * tf[:, :, i]
    return out.reshape(xf.shape)
