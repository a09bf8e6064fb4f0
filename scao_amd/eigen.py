"""Top-k eigenpairs of a batch of symmetric matrices on the device.

The eigen stage of the curvature refresh (scao/preconditioner.py:413-451)
needs, per factor, the k_max largest eigenpairs and the sum of the clamped
spectrum (utils.adaptive_rank, scao/utils.py:121-151).  The reference gets
them from a full torch.linalg.eigh.  Here the work is split between the HIP
kernels of csrc/eig.hip and plain batched GEMMs (rocBLAS, through torch):

1. dense -> band with SCAO_EIG_BAND sub-diagonals: for every panel of b
   columns, ``scao_eig_panel_qr`` factors it (Householder, V kept in the
   panel, T returned), then the trailing matrix gets the two-sided update
   A22 <- Q^T A22 Q = A22 - (V W^T + W V^T), W = X - V (T^T V^T X) / 2,
   X = A22 V T.  The next panel's columns are updated first (a thin
   product), the next panel is factored, and one ``scao_eig_sy2sb_update``
   pass over the lower triangle applies the update and forms the next
   panel's A22 V, so each panel reads and writes half the matrix once;
2. ``scao_eig_band_finish`` / ``scao_eig_sb2st``: band -> tridiagonal;
3. ``scao_eig_bisect``: the kq largest eigenvalues and the clamped sum;
4. ``scao_eig_vectors``: eigenvectors of the band matrix;
5. back-transformation Z <- Q_0 (Q_1 (... Q_last Z)): ``scao_eig_back_transform``
   applies the panels' reflectors from the last, each matrix's Z slices held in
   registers for the whole pass.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib as L

NB = L.EIG_BAND
BW = L.EIG_BANDW
MAX_BATCH = 65535   # matrices per call: the batch is a grid dimension


def _call(name: str, *args) -> None:
    """L.call through the engine's launch timing (bench.py's per-kernel
    split of the refresh)."""
    from . import engine
    engine._call(name, *args)


def solver_fits(n: int) -> bool:
    """Whether topk_eigh takes an n x n factor with kernels that need no
    scratch memory: every kernel of the solver keeps its state in registers
    and LDS except the back-transformation when its Z slices exceed the
    register file, which happens above 2048 rows unless n is a multiple of
    16 (kq is, see topk_eigh) and above 4096 rows in any case.  Scratch is
    allocated by the runtime at launch and that can fail when device memory
    is nearly full."""
    return 1 <= n <= 2048 or (n <= 4096 and n % 16 == 0)


def panels(n: int) -> list:
    """Column origins of the stage-1 panels of an n x n matrix."""
    return list(range(0, n - NB, NB))


def _check(X: Tensor) -> None:
    if X.dtype != torch.float32 or X.ndim != 3 or X.shape[1] != X.shape[2]:
        raise ValueError(f"eigen: expected (B, n, n) float32, got {tuple(X.shape)} {X.dtype}")
    if X.device.type != "cuda":
        raise RuntimeError("eigen: X must be on a ROCm device")
    if not X.is_contiguous():
        raise ValueError("eigen: X must be contiguous")
    if X.shape[1] > 4096 + NB:
        raise ValueError(f"eigen: n={X.shape[1]} above the supported {4096 + NB}")
    if X.shape[0] > MAX_BATCH:
        raise ValueError(f"eigen: batch {X.shape[0]} above {MAX_BATCH} (grid limit)")


def _reduce(X: Tensor):
    """Stages 1-2: returns (panel origins, T factors, band copy (B, n, b+1):
    lower diagonals 0..b of the band matrix, tridiagonal d, e)."""
    B, n, _ = X.shape
    dev = X.device
    f32 = torch.float32
    s = L.stream_ptr(dev)
    pcs = panels(n)
    Tall = torch.empty(max(len(pcs), 1), B, NB, NB, dtype=f32, device=dev)
    band = torch.zeros(B, n, BW, dtype=f32, device=dev)
    nn = n * n
    if pcs:
        _stage1_fused(X, pcs, Tall, band, s)
    orig = torch.empty(B, n, NB + 1, dtype=f32, device=dev)
    band64 = torch.empty(B, n, BW, dtype=torch.float64, device=dev)
    _call("scao_eig_band_finish", X.data_ptr(), nn, n, B, band.data_ptr(), n * BW,
           orig.data_ptr(), n * (NB + 1), band64.data_ptr(), s)
    del band
    d = torch.empty(B, n, dtype=torch.float64, device=dev)
    e = torch.zeros(B, n, dtype=torch.float64, device=dev)
    _call("scao_eig_sb2st", band64.data_ptr(), n, B, d.data_ptr(), e.data_ptr(), s)
    return pcs, Tall, orig, d, e


def _stage1_fused(X: Tensor, pcs: list, Tall: Tensor, band: Tensor, s: int) -> None:
    """Stage 1 on the lower triangle (module docstring, step 1).  Above the
    diagonal X holds stale values afterwards; nothing reads them."""
    B, n, _ = X.shape
    nn = n * n
    f32 = torch.float32
    base = X.data_ptr()
    _call("scao_eig_panel_qr", base, nn, n, 0, B, Tall[0].data_ptr(), band.data_ptr(), n * BW, s)
    Y = torch.bmm(X[:, NB:, NB:], X[:, NB:, 0:NB])      # X is whole and symmetric here
    work = torch.empty(max(L.lib().scao_eig_sy2sb_work(max(n - 2 * NB, 1), B), 8),
                       dtype=torch.uint8, device=X.device)
    for p, c0 in enumerate(pcs):
        r0 = c0 + NB
        last = p + 1 == len(pcs)
        # W = Y T - V (T^T V^T Y T) / 2 and, unless last, the next panel's
        # columns (rows r0..)
        W = torch.empty(B, n - r0, NB, dtype=f32, device=X.device)
        _call("scao_eig_sy2sb_panel_w", base, nn, n, c0, B, Y.data_ptr(), Tall[p].data_ptr(),
               W.data_ptr(), 0 if last else 1, s)
        if last:                                               # the last, in-band block
            V = X[:, r0:, c0:c0 + NB]
            A22 = X[:, r0:, r0:]
            A22.baddbmm_(torch.cat([V, W], 2), torch.cat([W, V], 2).transpose(1, 2), alpha=-1.0)
            break
        _call("scao_eig_panel_qr", base, nn, n, r0, B, Tall[p + 1].data_ptr(),
               band.data_ptr(), n * BW, s)
        # the rest of the trailing matrix (rows and columns r1..) and the next Y
        r1 = r0 + NB
        mr = n - r1
        Y = torch.empty(B, mr, NB, dtype=f32, device=X.device)
        _call("scao_eig_sy2sb_update", base + 4 * (r1 * n + r1), nn, n, mr, B,
               base + 4 * (r1 * n + c0), nn, n,
               W.data_ptr() + 4 * NB * NB, W.stride(0), NB,
               base + 4 * (r1 * n + r0), nn, n,
               Y.data_ptr(), mr * NB, work.data_ptr(), s)


def stages(X: Tensor):
    """Stages 1-2 alone (for tests): (band copy, d, e); X is overwritten."""
    _check(X)
    _, _, orig, d, e = _reduce(X)
    return orig, d, e


def topk_eigh(X: Tensor, kq: int):
    """The kq largest eigenpairs of each symmetric matrix of X (B, n, n).

    X must be a contiguous float32 device tensor; it is overwritten (its
    panels end up holding the stage-1 reflectors).  Returns (w, U, total):
    w (B, kq) float64 eigenvalues in descending order (Rayleigh quotients of
    the band matrix), U (B, n, kq) float32 orthonormal eigenvectors, total
    (B,) float64 = sum over all eigenvalues of max(lambda, 0)."""
    _check(X)
    B, n, _ = X.shape
    if not 1 <= kq <= n:
        raise ValueError(f"topk_eigh: kq={kq} outside [1, {n}]")
    want = kq
    kq = min(n, -(-kq // 16) * 16)   # whole 16-column slices: the exact back-transformation
    dev = X.device
    s = L.stream_ptr(dev)
    pcs, Tall, orig, d, e = _reduce(X)
    w = torch.empty(B, kq, dtype=torch.float64, device=dev)
    total = torch.empty(B, dtype=torch.float64, device=dev)
    work = torch.empty(max(L.lib().scao_eig_bisect_work(n, B), 8), dtype=torch.uint8, device=dev)
    _call("scao_eig_bisect", d.data_ptr(), e.data_ptr(), n, B, kq, w.data_ptr(),
           total.data_ptr(), work.data_ptr(), s)
    Z = torch.empty(B, n, kq, dtype=torch.float32, device=dev)
    work = torch.empty(max(L.lib().scao_eig_vectors_work(n, B, kq), 8), dtype=torch.uint8,
                       device=dev)
    _call("scao_eig_vectors", orig.data_ptr(), n * (NB + 1), n, B, kq, w.data_ptr(),
           Z.data_ptr(), n * kq, work.data_ptr(), s)
    del work
    if pcs:
        _call("scao_eig_back_transform", X.data_ptr(), n * n, n, B, Tall.data_ptr(),
               Z.data_ptr(), n * kq, kq, s)
    if kq != want:
        w, Z = w[:, :want].contiguous(), Z[:, :, :want].contiguous()
    return w, Z, total
