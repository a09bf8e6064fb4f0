"""Math helpers with the reference's names and semantics (scao/utils.py).

These are small tensor utilities, exported for API compatibility.  The
optimizer step does not call them per block: the batched HIP engine
implements quantisation, rank selection and the eigenvalue powers inside
its kernels and its batched refresh.
"""

from __future__ import annotations

import torch
from torch import Tensor


def to_2d(g):
    """scao/utils.py:208-219: 1-D -> (1, n); N-D -> (shape[0], prod(rest))."""
    shape = g.shape
    if g.ndim == 1:
        return g.unsqueeze(0), shape
    if g.ndim == 2:
        return g, shape
    return g.reshape(shape[0], -1), shape


def from_2d(g2: Tensor, shape) -> Tensor:
    """scao/utils.py:222-226."""
    return g2.reshape(shape)


def quantize_sym_int8(x: Tensor):
    """scao/utils.py:170-189: (codes, scale) with scale = max|x|/127 (Python
    float); codes = clamp(round_half_even(x / fp32(scale)), +-127)."""
    amax = x.abs().max().item()
    if amax < 1e-30:
        return torch.zeros_like(x, dtype=torch.int8), 1.0
    scale = amax / 127.0
    return (x / scale).round_().clamp_(-127, 127).to(torch.int8), scale


def dequantize_sym_int8(q: Tensor, scale: float) -> Tensor:
    """scao/utils.py:192-203."""
    return q.to(torch.float32).mul_(scale)


def low_rank_matrix_power_neg_quarter(U: Tensor, S: Tensor, eps: float = 1e-8):
    """scao/utils.py:96-114."""
    return U, S.clamp(min=eps).pow(-0.25)


def matrix_power_neg_quarter(A: Tensor, use_newton_schulz: bool = False, ns_steps: int = 10,
                             eps: float = 1e-8) -> Tensor:
    """scao/utils.py:61-93 (eigendecomposition branch; the Newton-Schulz branch
    is not reachable from the optimizer and is not provided)."""
    if use_newton_schulz:
        raise NotImplementedError("Newton-Schulz root is not part of scao_amd")
    w, V = torch.linalg.eigh(A)
    w = w.clamp(min=eps)
    return (V * w.pow(-0.25).unsqueeze(0)) @ V.T


def adaptive_rank(eigenvalues: Tensor, epsilon: float = 0.05, k_min: int = 4,
                  k_max: int = 128) -> int:
    """scao/utils.py:121-151."""
    total = eigenvalues.sum().item()
    if total < 1e-12:
        return k_min
    thresh = (1.0 - epsilon) * total
    csum = torch.cumsum(eigenvalues, dim=0)
    hits = (csum >= thresh).nonzero(as_tuple=True)[0]
    k = int(hits[0].item()) + 1 if hits.numel() > 0 else len(eigenvalues)
    return int(min(k_max, max(k_min, k)))


def batched_adaptive_rank(S_desc: Tensor, epsilon: Tensor, k_min: Tensor, k_max: Tensor):
    """``adaptive_rank`` for a batch of descending spectra [B, d] on the device.

    Per row: total = sum (fp32), threshold = fp32((1 - eps) * double(total)),
    k = first index with cumsum >= threshold, plus one (d if none); k_min
    when double(total) < 1e-12; clamped to [k_min, k_max].  Returns an int64
    tensor on the device; the caller reads all rows back at once."""
    d = S_desc.shape[1]
    total = S_desc.sum(dim=1)
    thr = ((1.0 - epsilon.double()) * total.double()).float()
    csum = torch.cumsum(S_desc, dim=1)
    hit = csum >= thr.unsqueeze(1)
    first = torch.where(hit.any(dim=1), hit.to(torch.int8).argmax(dim=1) + 1,
                        torch.full_like(total, d, dtype=torch.int64))
    k = torch.minimum(k_max, torch.maximum(k_min, first))
    return torch.where(total.double() < 1e-12, k_min, k)


def batched_adaptive_rank_topk(S_top: Tensor, total: Tensor, dim: int, epsilon: Tensor,
                               k_min: Tensor, k_max: Tensor):
    """``adaptive_rank`` from the kq largest eigenvalues of each spectrum
    (clamped, descending, [B, kq]) and the sum of the whole clamped spectrum
    (float64 [B]): the reference's total is the float32 sum of the clamped
    spectrum, threshold = fp32((1 - eps) * double(total)), k = first index
    whose float32 cumsum reaches it, plus one; when none of the kq does, the
    first index lies beyond them (kq + 1, or dim when kq == dim), above every
    k_max <= kq; k_min when total < 1e-12; clamped to [k_min, k_max]."""
    kq = S_top.shape[1]
    tot = total.float()
    thr = ((1.0 - epsilon.double()) * tot.double()).float()
    csum = torch.cumsum(S_top, dim=1)
    hit = csum >= thr.unsqueeze(1)
    beyond = dim if kq == dim else kq + 1
    first = torch.where(hit.any(dim=1), hit.to(torch.int8).argmax(dim=1) + 1,
                        torch.full_like(tot, beyond, dtype=torch.int64))
    k = torch.minimum(k_max, torch.maximum(k_min, first))
    return torch.where(tot.double() < 1e-12, k_min, k)
