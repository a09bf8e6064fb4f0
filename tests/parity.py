"""Elementwise parity gates and shared-state plumbing for the GPU tests.

The north star's bar is stated per element: parameter updates within rtol
1e-4 in fp32.  An update element that is a small difference of larger terms
(an Adan step where m and the gradient delta nearly cancel) carries the
absolute rounding error of its terms, so every gate is |got - want| <=
atol + rtol * |want| with atol a stated fraction of the largest |want| of
the tensor.  ``ratio`` is the largest |got - want| / (atol + rtol * |want|)
over the tensor: <= 1 passes."""

from __future__ import annotations

import json
import os

import torch

UPDATE_RTOL = 1e-4      # north star: parameter updates within rtol 1e-4 (fp32)
UPDATE_ATOL = 1e-6      # x max |update| of the tensor
MOMENT_RTOL = 1e-4
MOMENT_ATOL = 1e-6      # x max |moment| of the tensor


def ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of the float32 grid at |x| (float64 result)."""
    a = x.detach().float().abs().cpu()
    return (torch.nextafter(a, torch.full_like(a, float("inf"))) - a).double()


def eig_input(leaf) -> torch.Tensor:
    """The eigh input of a CPU-reference block, in float64 from its own
    float32 arithmetic (scao/preconditioner.py:381-406): dequantised EMA
    over the bias factor plus the Tikhonov shift on the diagonal."""
    import oracle.scao_ref as R
    out = []
    bias = max(1.0 - leaf.rho ** leaf.precond_step, 1e-8)
    for side in ("L", "R"):
        if leaf.use_int8_ema:
            X = R.dequantize_sym_int8(getattr(leaf, f"{side}_ema_q"),
                                      getattr(leaf, f"{side}_ema_scale"))
        else:
            X = getattr(leaf, f"{side}_ema")
        X = X / bias
        tik = max(1e-8, 1e-4 * X.trace().item() / X.shape[0])
        X = X.clone()
        X.diagonal().add_(tik)
        out.append(X.double())
    return out


def ratio(got, want, rtol, atol_frac, extra=None) -> float:
    """max |got - want| / (atol_frac * max|want| + rtol * |want| + extra)."""
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    if want.numel() == 0:
        return 0.0
    atol = atol_frac * want.abs().max().item()
    bound = atol + rtol * want.abs()
    if extra is not None:
        bound = bound + extra
    err = (got - want).abs()
    bound = bound.clamp(min=1e-300)
    return (err / bound).max().item()


def assert_close(got, want, rtol, atol_frac, what, extra=None) -> float:
    r = ratio(got, want, rtol, atol_frac, extra)
    assert r <= 1.0, f"{what}: worst |err| / (atol + rtol|ref|) = {r:.3g} " \
                     f"(rtol {rtol:g}, atol {atol_frac:g} x max|ref|)"
    return r


def assert_update_close(p_new, p_new_ref, p_old, what, rtol=UPDATE_RTOL,
                        atol_frac=UPDATE_ATOL, extra_abs: float = 0.0) -> float:
    """The step's update p_new - p_old against the reference's, element by
    element.  An update is only observable through the stored parameter,
    which is rounded to float32 once: where the reference and the kernel
    round a new value to neighbouring floats, the two updates differ by one
    float32 spacing of the new parameter whatever their precision (with
    LARS the step lr * trust * u is often far below that spacing).  So the
    bound adds ulp(p_new_ref) to atol + rtol * |update|, and ``extra_abs``
    (an absolute allowance the caller states and justifies)."""
    p_old = p_old.detach().double().cpu()
    return assert_close(p_new.detach().double().cpu() - p_old,
                        p_new_ref.detach().double().cpu() - p_old, rtol, atol_frac, what,
                        extra=torch.maximum(ulp(p_new_ref), ulp(p_new)) + extra_abs)


def update_ratio(p_new, p_new_ref, p_old, rtol=UPDATE_RTOL, atol_frac=UPDATE_ATOL) -> float:
    """The ratio assert_update_close gates, without asserting."""
    p_old = p_old.detach().double().cpu()
    return ratio(p_new.detach().double().cpu() - p_old, p_new_ref.detach().double().cpu() - p_old,
                 rtol, atol_frac, extra=torch.maximum(ulp(p_new_ref), ulp(p_new)))


def eigh_error(a, b) -> float:
    """max |a - b| over a tensor pair (float64): the reference's own
    eigensolver error when a is its float32-eigh result and b the same step
    with a float64 eigh."""
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def report(test, case, data):
    """Append measured errors to $SCAO_REPORT (JSON lines) when set."""
    path = os.environ.get("SCAO_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"test": test, "case": case, "data": data}) + "\n")


def kron_leaves(pre, r0=0, c0=0):
    """Kronecker blocks of a CPU-reference preconditioner in block order
    (reference preconditioner.py:163-194), as (block, row, col)."""
    if pre.use_block_diagonal:
        off = 0
        for bs, blk in zip(pre._block_sizes, pre._blocks):
            if pre._block_dim == 0:
                yield from kron_leaves(blk, r0 + off, c0)
            else:
                yield from kron_leaves(blk, r0, c0 + off)
            off += bs
    elif pre.use_kronecker:
        yield pre, r0, c0


class IdenticalPostEma:
    """engine.AFTER_EMA_HOOK for one step: checks the GPU's new EMA of every
    refreshed block against the CPU reference's (int8 codes within 1 LSB,
    scales within 1e-6 relative; fp32 EMAs within 1e-5 relative), then
    replaces it by the reference's, so the eigen stage and the update that
    follow start from identical inputs.  ``pairs``: {id(gpu block): cpu block}."""

    def __init__(self, pairs: dict):
        self.pairs = pairs
        self.checked = 0
        self.max_lsb = 0
        self.max_scale_rel = 0.0

    def __call__(self, kron):
        for leaf, *_ in kron:
            ref = self.pairs[id(leaf)]
            dev = leaf.device
            if leaf.use_int8_ema:
                for side in ("L", "R"):
                    qg = getattr(leaf, f"{side}_ema_q").cpu().int()
                    qr = getattr(ref, f"{side}_ema_q").int()
                    lsb = (qg - qr).abs().max().item()
                    sg = getattr(leaf, f"{side}_ema_scale")
                    sr = getattr(ref, f"{side}_ema_scale")
                    rel = abs(sg - sr) / abs(sr)
                    self.max_lsb = max(self.max_lsb, lsb)
                    self.max_scale_rel = max(self.max_scale_rel, rel)
                    assert lsb <= 1, (side, lsb)
                    assert rel <= 1e-6, (side, sg, sr)
                leaf.L_ema_q = ref.L_ema_q.to(dev).contiguous()
                leaf.R_ema_q = ref.R_ema_q.to(dev).contiguous()
                leaf._scale = torch.tensor([ref.L_ema_scale, ref.R_ema_scale],
                                           dtype=torch.float64, device=dev)
            else:
                for side in ("L", "R"):
                    eg = getattr(leaf, f"{side}_ema").cpu().double()
                    er = getattr(ref, f"{side}_ema").double()
                    rel = ((eg - er).norm() / er.norm()).item()
                    assert rel < 1e-5, (side, rel)
                leaf.L_ema.copy_(ref.L_ema)
                leaf.R_ema.copy_(ref.R_ema)
            self.checked += 1


def lars_exact(rec: dict, wd: float, c: float):
    """The reference's LARS trust (scao/optimizer.py:371-377, float32 tensor
    arithmetic on the two norms) with correctly rounded float32 norms of the
    decayed parameter and the update recorded by the oracle (RECORD).
    Returns (trust, |p|, |u|)."""
    pn = rec["pdec"].double().norm().float()
    un = rec["upd"].double().norm().float()
    if float(pn) == 0.0 or float(un) == 0.0:
        return 1.0, float(pn), float(un)
    return float(c * pn / (un + wd * pn + 1e-8)), float(pn), float(un)


def norm_allowance(rec: dict, trust_exact: float, lr: float) -> float:
    """E_norm: how far the reference's own float32 norms move its update,
    max |lr * (trust - trust_exact) * u| over the tensor (the update is
    p_dec - lr * trust * u; only the trust depends on the norms)."""
    return lr * abs(rec["trust"] - trust_exact) * rec["upd"].double().abs().max().item()


def step_stats(opt) -> dict:
    """The kernels' per-parameter intermediates of opt's last step, keyed by
    id(parameter): the PARAM_STAT row (trust, clip, nu, unorm, pnorm, gnorm,
    alpha, ...) and, for parameters with LARS, the staged update u read from
    the step's workspace."""
    import numpy as np
    from scao_amd import _lib as L
    out = {}
    ws = opt._ws
    raw = ws._bufs["stat"].cpu().numpy().tobytes()
    rows = np.frombuffer(raw[:len(ws.last_items) * L.PARAM_STAT.itemsize], dtype=L.PARAM_STAT)
    for i, (p, row) in enumerate(zip(ws.last_items, rows)):
        d = {n: float(row[n]) for n in L.PARAM_STAT.names if n != "pad0"}
        off = ws.upd_offsets.get(i)
        if off is not None:
            flat = ws._bufs["upd"].view(torch.float32)
            d["upd"] = flat[off:off + p.numel()].view(p.shape).cpu()
        out[id(p)] = d
    return out


class ReferenceEigen:
    """engine.AFTER_EIGEN_HOOK for one step: for every refreshed block,
    checks the GPU's new eigenfactors against the CPU reference's from the
    same codes -- k and S (rtol 1e-4) and the spectral projector U S U^T,
    within max(1e-4, 3 E_ref) where E_ref is how far the reference's float32
    eigh is from float64 on the same input (computed only when needed) --
    then gives the GPU block the reference's U, S and k, so that the steps
    after a refresh are compared from identical factors.
    ``pairs``: {id(gpu block): cpu block}."""

    def __init__(self, pairs: dict):
        self.pairs = pairs
        self.worst = 0.0
        self.checked = 0

    @staticmethod
    def _proj(U, S):
        U = U.detach().double().cpu()
        return (U * S.detach().double().cpu()) @ U.T

    def __call__(self, kron):
        for leaf, *_ in kron:
            ref = self.pairs[id(leaf)]
            dev = leaf.U_l.device
            assert leaf.k == ref.k, (leaf.k, ref.k)
            for side, X in zip(("l", "r"), eig_input(ref)):
                Ug, Sg = getattr(leaf, f"U_{side}"), getattr(leaf, f"S_{side}")
                Ur, Sr = getattr(ref, f"U_{side}"), getattr(ref, f"S_{side}")
                torch.testing.assert_close(Sg.cpu(), Sr, rtol=1e-4, atol=0.0)
                pr = self._proj(Ur, Sr)
                e = ((self._proj(Ug, Sg) - pr).norm() / pr.norm()).item()
                bound = 1e-4
                if e > bound:   # the reference's own float32 eigh error on this input
                    w, V = torch.linalg.eigh(X)
                    w, V = w.flip(0)[:ref.k], V.flip(1)[:, :ref.k]
                    e_ref = (((V * w) @ V.T - pr).norm() / pr.norm()).item()
                    bound = max(bound, 3.0 * e_ref)
                assert e <= bound, (side, leaf.m, leaf.n, e, bound)
                self.worst = max(self.worst, e)
            leaf.U_l, leaf.S_l = ref.U_l.to(dev).contiguous(), ref.S_l.to(dev).contiguous()
            leaf.U_r, leaf.S_r = ref.U_r.to(dev).contiguous(), ref.S_r.to(dev).contiguous()
            leaf._touch()
            self.checked += 1
