"""Offline WUSH transform preparation (fp64, torch), mirroring the API of the
reference's ``my_int4/wush_transform.py:27-58``:

* ``compute_wush_transform(X_cal, W)`` -> T (K/32, 32, 32) fp64,
* ``transform_weights(W, T)``          -> W' = W T^{-1} per 32-block,
* ``transform_activations_reference(X, T)`` -> X' = X T^T per 32-block.

The reference obtains T from the un-vendored WUSH upstream
(IST-DASLab/WUSH ``src/block_transform.py``, ``src/compute_gram.py``, no pinned
commit; reference wush_transform.py:12-24, :36-40).  It is absent here, so the
construction below is this project's own closed form, built from the same
inputs (per-block Gram matrices of the calibration activations and of the
weights, each divided by its row count, reference wush_transform.py:36-37):

    Gx = X_c^T X_c / M,   Gw = W_c^T W_c / N           (per 32-block c)
    Gw^{1/2} Gx Gw^{1/2} = U S U^T                      (eigendecomposition)
    T = H S^{-1/4} U^T Gw^{1/2}                          (H: normalised Hadamard)

With it the transformed Gram matrices are equal and Hadamard-spread:
T Gx T^T = T^{-T} Gw T^{-1} = H S^{1/2} H^T -- both operands see the same,
flattened second moments, which is what per-group INT4 quantization of both
sides wants.  Any invertible T keeps X'W'^T = XW^T exactly.  T values are
"parity unpinned" against the upstream; the tests pin the invariants
(product invariance, balance, the reference's e2e outlier gate).

Runs on whatever device its inputs are on; nothing here is on the hot path.
"""
from __future__ import annotations

import math

import torch

__all__ = ["block_gram", "hadamard", "compute_wush_transform", "transform_weights",
           "transform_activations_reference"]


def block_gram(x: torch.Tensor, size: int = 32) -> torch.Tensor:
    """Diagonal blocks of x^T x: (K/size, size, size) in fp64."""
    x = x.to(torch.float64)
    M, K = x.shape
    xb = x.reshape(M, K // size, size).transpose(0, 1)          # (C, M, size)
    return xb.transpose(1, 2) @ xb


def hadamard(n: int, dtype=torch.float64, device=None) -> torch.Tensor:
    """Sylvester Hadamard matrix of order n (a power of two), scaled to be orthogonal."""
    assert n & (n - 1) == 0
    H = torch.ones(1, 1, dtype=dtype, device=device)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H / math.sqrt(n)


def _sym_pow(A: torch.Tensor, p: float, floor: float = 0.0) -> torch.Tensor:
    evals, evecs = torch.linalg.eigh(A)
    evals = evals.clamp_min(floor)
    return (evecs * evals.pow(p).unsqueeze(-2)) @ evecs.transpose(-1, -2)


def compute_wush_transform(X_cal: torch.Tensor, W: torch.Tensor, group_size: int = 32,
                           use_hadamard: bool = True, ridge: float = 1e-6) -> torch.Tensor:
    """Per-block transform T (K/gs, gs, gs), fp64.  X_cal: (M, K), W: (N, K)."""
    M, K = X_cal.shape
    N = W.shape[0]
    assert W.shape[1] == K and K % group_size == 0
    dev = X_cal.device
    Gx = block_gram(X_cal, group_size) / M
    Gw = block_gram(W.to(dev), group_size) / N
    eye = torch.eye(group_size, dtype=torch.float64, device=dev)

    def regularise(G):
        mean_diag = G.diagonal(dim1=-2, dim2=-1).mean(-1).clamp_min(1e-30)
        return G + ridge * mean_diag[:, None, None] * eye

    # the (K/32) 32x32 eigenproblems are tiny: solve them on the host
    Gx, Gw = regularise(Gx).cpu(), regularise(Gw).cpu()
    Gw_half = _sym_pow(Gw, 0.5)
    Mmat = Gw_half @ Gx @ Gw_half
    Mmat = 0.5 * (Mmat + Mmat.transpose(-1, -2))
    S, U = torch.linalg.eigh(Mmat)
    S = S.clamp_min(S.amax(-1, keepdim=True) * 1e-12)
    T = (S.pow(-0.25).unsqueeze(-1) * U.transpose(-1, -2)) @ Gw_half
    if use_hadamard:
        T = hadamard(group_size) @ T
    return T.to(dev)


def transform_weights(W: torch.Tensor, T: torch.Tensor) -> torch.Tensor:
    """W' = W T^{-1} per block (reference wush_transform.py:43-51), fp64."""
    W = W.to(torch.float64)
    T = T.to(device=W.device, dtype=torch.float64)
    N, K = W.shape
    C, gs, _ = T.shape
    Tinv = torch.linalg.inv(T.cpu()).to(W.device)               # (C, gs, gs), tiny: host solve
    Wb = W.reshape(N, C, gs).transpose(0, 1).contiguous()       # (C, N, gs)
    return (Wb @ Tinv).transpose(0, 1).reshape(N, K)


def transform_activations_reference(X: torch.Tensor, T: torch.Tensor) -> torch.Tensor:
    """X' = X T^T per block (reference wush_transform.py:54-58), fp64."""
    X = X.to(torch.float64)
    T = T.to(device=X.device, dtype=torch.float64)
    M, K = X.shape[-2], X.shape[-1]
    C, gs, _ = T.shape
    Xb = X.reshape(-1, C, gs).transpose(0, 1).contiguous()     # (C, rows, gs)
    return (Xb @ T.transpose(-1, -2).contiguous()).transpose(0, 1).reshape(X.shape)
