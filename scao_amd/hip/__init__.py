"""Operator surface of the reference's native layer, on gfx950.

Mirrors ``scao.cuda`` (scao/cuda/__init__.py:149-266): the same function
names (fused_kronecker_precond, low_rank_precond_mm, int8_ema_update),
argument meaning and return values.  Unlike the reference there is
no silent fallback: inputs must be float32 tensors on a ROCm device and the
HIP library must be built; otherwise these raise.  (The reference falls back
to PyTorch when its extension is missing -- scao/cuda/__init__.py:56-71,
183-187 -- unless SCAO_FORCE_CUDA_EXT=1; scao_amd always behaves as forced.)
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib as L


def _check(t: Tensor, name: str, dtype=torch.float32) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a ROCm device (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")


def fused_kronecker_precond(U_l: Tensor, s_l_inv4: Tensor, U_r: Tensor, s_r_inv4: Tensor,
                            G: Tensor) -> Tensor:
    """out = G + U_l ((s_l s_r^T - 1) * (U_l^T G U_r)) U_r^T  (reference :149-187).

    G is (m, n) with unit column stride (row stride free, so column slices of
    a larger matrix work); U_l (m, k), U_r (n, k); returns a new (m, n)."""
    for t, nm in ((U_l, "U_l"), (s_l_inv4, "s_l_inv4"), (U_r, "U_r"), (s_r_inv4, "s_r_inv4"),
                  (G, "G")):
        _check(t, nm)
    if G.ndim != 2:
        raise ValueError("G must be 2-D")
    m, n = G.shape
    k = U_l.shape[1]
    if U_l.shape != (m, k) or U_r.shape != (n, k) or s_l_inv4.numel() != k or \
            s_r_inv4.numel() != k:
        raise ValueError(f"shape mismatch: G {tuple(G.shape)}, U_l {tuple(U_l.shape)}, "
                         f"U_r {tuple(U_r.shape)}")
    if G.stride(1) != 1:
        G = G.contiguous()
    U_l, U_r = U_l.contiguous(), U_r.contiguous()
    s_l_inv4, s_r_inv4 = s_l_inv4.contiguous(), s_r_inv4.contiguous()
    out = torch.empty(m, n, dtype=torch.float32, device=G.device)
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.copy_(G)
    ws = torch.empty(L.lib().scao_fused_kronecker_workspace(m, n, k) // 4, dtype=torch.float32,
                     device=G.device)
    L.call("scao_fused_kronecker_precond", U_l.data_ptr(), s_l_inv4.data_ptr(), U_r.data_ptr(),
           s_r_inv4.data_ptr(), G.data_ptr(), G.stride(0), out.data_ptr(), m, n, k,
           ws.data_ptr(), L.stream_ptr(G.device))
    return out


def low_rank_precond_mm(U: Tensor, s: Tensor, G: Tensor, left: bool = True) -> Tensor:
    """left=True: U diag(s) U^T G;  left=False: G U diag(s) U^T
    (reference :190-228; its fallback :102-119 computes (U*s) @ (U^T @ G)
    and (G @ (U*s)) @ U^T).  Not on the optimizer step: two launches of the
    library's strided fp32 GEMM in that order (scao_low_rank_precond_mm)."""
    for t, nm in ((U, "U"), (s, "s"), (G, "G")):
        _check(t, nm)
    if G.ndim != 2 or U.ndim != 2 or s.numel() != U.shape[1]:
        raise ValueError(f"shape mismatch: U {tuple(U.shape)}, s {tuple(s.shape)}, "
                         f"G {tuple(G.shape)}")
    d = G.shape[0] if left else G.shape[1]
    if U.shape[0] != d:
        raise ValueError(f"U has {U.shape[0]} rows, G's {'rows' if left else 'columns'} are {d}")
    m, n = G.shape
    k = U.shape[1]
    out = torch.empty(m, n, dtype=torch.float32, device=G.device)
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.zero_()
    U, s, G = U.contiguous(), s.contiguous(), G.contiguous()
    ws = torch.empty(max(1, L.lib().scao_low_rank_precond_mm_workspace(m, n, k, int(left)) // 4),
                     dtype=torch.float32, device=G.device)
    L.call("scao_low_rank_precond_mm", U.data_ptr(), s.data_ptr(), G.data_ptr(), out.data_ptr(),
           m, n, k, int(left), ws.data_ptr(), L.stream_ptr(G.device))
    return out


def int8_ema_update(ema_q: Tensor, ema_scale: float, new_val: Tensor, rho: float):
    """(q_new, scale_new) for x = rho*dequant(ema_q, ema_scale) + new_val
    (reference :231-266; requantisation multiplies by the fp32 reciprocal of
    the new scale).  Returns a new int8 tensor and a Python float (reading
    the scale back synchronises, as the reference's .item() does)."""
    _check(ema_q, "ema_q", torch.int8)
    _check(new_val, "new_val")
    if ema_q.numel() != new_val.numel():
        raise ValueError("ema_q and new_val must have the same number of elements")
    q = ema_q.contiguous().clone()
    v = new_val.contiguous()
    n = q.numel()
    if n == 0:
        return q, 1.0
    scratch = torch.empty(L.lib().scao_int8_ema_scratch_bytes(n), dtype=torch.uint8,
                          device=q.device)
    scale = torch.empty(1, dtype=torch.float64, device=q.device)
    L.call("scao_int8_ema_update", q.data_ptr(), float(ema_scale), v.data_ptr(), float(rho), n,
           scale.data_ptr(), scratch.data_ptr(), L.stream_ptr(q.device))
    return q.view(ema_q.shape), float(scale.item())
