"""``my_int4.rtn_int4`` with the reference's names and signatures
(reference my_int4/rtn_int4.py:33-75), for callers that import them.

  quant_int4(x, group_size=32)       -> (q u8 (..., K/2), s bf16 (..., K/32))
  dequant_int4(q, s, group_size=32)  -> fp32 (..., K)
  w4a4_matmul_reference(xq, xs, wq, ws) -> fp16 (..., N)

quant_int4 and w4a4_matmul_reference run this build's HIP kernels
(my_int4._C.quant_int4, bit-exact with the reference's sigma-clip rounding
including ties; my_int4._C.w4a4_gemm_s4, the group-scaled product with exact
int32 group dots) and take GPU tensors only: there is no CPU path in the
product.  dequant_int4 decodes the packed format with tensor ops on the
tensors' own device (element 2k in the low nibble, sign-extended, times the
group's bf16 scale), for inspection and checks."""
from __future__ import annotations

import torch

from my_int4 import _C

INT4_MIN, INT4_MAX = -7, 7      # reference rtn_int4.py:15


def _need_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} runs on the GPU (HIP kernels); got a {t.device} tensor")


def quant_int4(x: torch.Tensor, group_size: int = 32):
    """Per-group sigma-clip INT4 quantization (reference rtn_int4.py:33-55)."""
    if group_size != 32:
        raise ValueError("group_size must be 32 (the kernels' quantization group)")
    _need_gpu(x, "quant_int4")
    return _C.quant_int4(x.contiguous())


def dequant_int4(q_byte: torch.Tensor, scale: torch.Tensor, group_size: int = 32) -> torch.Tensor:
    """(q u8 (..., K/2), s bf16 (..., K/group_size)) -> fp32 (..., K) (reference rtn_int4.py:58-68)."""
    lo = ((q_byte & 0xF).to(torch.int16) << 12) >> 12
    hi = ((q_byte >> 4).to(torch.int16) << 12) >> 12
    d = torch.stack([lo, hi], dim=-1).flatten(-2)
    d = d.unflatten(-1, (-1, group_size)).float() * scale.float().unsqueeze(-1)
    return d.flatten(-2)


def w4a4_matmul_reference(x_q, x_s, w_q, w_s) -> torch.Tensor:
    """Y = X W^T in fp16 from the packed operands (reference rtn_int4.py:71-75),
    computed by the HIP group-scaled GEMM."""
    _need_gpu(x_q, "w4a4_matmul_reference")
    K2 = x_q.shape[-1]
    y = _C.w4a4_gemm_s4(x_q.reshape(-1, K2).contiguous(), x_s.reshape(-1, x_s.shape[-1]).contiguous(),
                        w_q.contiguous(), w_s.contiguous())
    return y.reshape(*x_q.shape[:-1], w_q.shape[0])
