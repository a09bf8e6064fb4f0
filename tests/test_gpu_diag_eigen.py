"""Exactly diagonal eigh inputs on the device against the CPU reference.

An int8 EMA of small gradients keeps only its diagonal codes, so the eigh
input of a refresh is a diagonal matrix with many tied values; the reference
(torch.linalg.eigh, LAPACK on the CPU) returns unit vectors in the order its
selection sort leaves the ties in (oracle.scao_ref.lapack_diagonal_order,
pinned on the CPU by tests/test_oracle_diag.py).  The refresh sends such
factors to scao_eig_diag, which reproduces that order.  These tests plant
diagonal EMAs with few distinct values at the configurations' block sizes
and require the eigen stage's U, S and k to equal the reference's exactly,
column for column; a factor with off-diagonal entries in the same batch
still goes through the solver."""

from __future__ import annotations

import pytest
import torch

from oracle import scao_ref as R
from parity import report

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _diag_codes(dim: int, levels: int, gen: torch.Generator):
    q = torch.zeros(dim, dim, dtype=torch.int8)
    q.diagonal().copy_(torch.randint(127 - levels + 1, 128, (dim,), generator=gen).to(torch.int8))
    return q


def _planted_dense(dim: int, k: int, gen: torch.Generator):
    """Codes of Q diag(lam) Q^T with lam_i = 1 - i/(2k) for the top k and at
    most 0.05 below: a well separated top-k eigenspace (for the solver side
    of a mixed batch)."""
    Q = torch.linalg.qr(torch.randn(dim, dim, generator=gen, dtype=torch.float64))[0]
    lam = 0.05 * torch.rand(dim, generator=gen, dtype=torch.float64)
    lam[:k] = 1.0 - torch.arange(k, dtype=torch.float64) / (2 * k)
    X = ((Q * lam) @ Q.T).float()
    return R.quantize_sym_int8(0.5 * (X + X.T))


def _count_diag_calls(monkeypatch):
    from scao_amd import engine
    calls = {"n": 0}
    orig = engine._diag_eigh

    def wrapped(part, *a):
        calls["n"] += len(part)
        return orig(part, *a)
    monkeypatch.setattr(engine, "_diag_eigh", wrapped)
    return calls


def _compare_exact(ra, gb, tag):
    assert gb.precond_step == ra.precond_step and gb.k == ra.k, tag
    for side, (U1, S1, U2, S2) in (("L", (ra.U_l, ra.S_l, gb.U_l, gb.S_l)),
                                  ("R", (ra.U_r, ra.S_r, gb.U_r, gb.S_r))):
        U2, S2 = U2.cpu(), S2.cpu()
        assert torch.equal(U2, U1), (tag, side, "U")
        assert torch.equal(S2, S1), (tag, side, "S")


# (m, n, k, distinct diagonal codes): C3 q and kv blocks, C5 q and kv blocks,
# C1's 768x1024 blocks, LAPACK's small-matrix path (<= 25 rows)
CASES = [(2048, 2048, 64, 2), (512, 2048, 64, 5), (4096, 4096, 256, 3), (1024, 4096, 256, 40),
         (768, 1024, 32, 1), (20, 30, 5, 2), (4112, 64, 16, 4)]


@pytest.mark.parametrize("m,n,k,levels", CASES)
def test_diag_eigen_stage_int8(m, n, k, levels, monkeypatch):
    from scao_amd import SparsePreconditioner, engine
    dev = _dev()
    kw = dict(k_min=k, k_max=k, max_precond_dim=max(m, n), use_int8_ema=True)
    ra = R.RefPreconditioner(torch.zeros(m, n), **kw)
    gb = SparsePreconditioner(torch.zeros(m, n, device=dev), **kw)
    gen = torch.Generator().manual_seed(m * 7 + n + levels)
    ra.L_ema_q, ra.L_ema_scale = _diag_codes(m, levels, gen), 8.04e-7
    ra.R_ema_q, ra.R_ema_scale = _diag_codes(n, levels, gen), 7.91e-7
    ra.precond_step, gb.precond_step = 5, 4
    gb.L_ema_q, gb.R_ema_q = ra.L_ema_q.to(dev), ra.R_ema_q.to(dev)
    gb._scale = torch.tensor([ra.L_ema_scale, ra.R_ema_scale], dtype=torch.float64, device=dev)
    calls = _count_diag_calls(monkeypatch)
    print(f"diag eigen stage {m}x{n} k={k} levels={levels}", flush=True)
    engine.refresh([(gb, torch.zeros(m, n, device=dev))], eigen_only=True)
    torch.cuda.synchronize()
    assert calls["n"] == 2
    ra._update_eigenfactors(1.0 - ra.rho ** ra.precond_step)
    _compare_exact(ra, gb, f"{m}x{n}")
    report("diag_eigen_stage", f"{m}x{n}/k{k}/levels{levels}", {"U": "equal", "S": "equal"})


def test_diag_eigen_stage_fp32_ema(monkeypatch):
    """The fp32 EMA (use_int8_ema=False) with a diagonal of tied values."""
    from scao_amd import SparsePreconditioner, engine
    dev = _dev()
    m, n, k = 300, 1000, 20
    kw = dict(k_min=k, k_max=k, max_precond_dim=1000, use_int8_ema=False)
    ra = R.RefPreconditioner(torch.zeros(m, n), **kw)
    gb = SparsePreconditioner(torch.zeros(m, n, device=dev), **kw)
    gen = torch.Generator().manual_seed(11)
    ra.L_ema = torch.diag(_diag_codes(m, 3, gen).diagonal().float() * 1e-6)
    ra.R_ema = torch.diag(_diag_codes(n, 2, gen).diagonal().float() * 3e-7)
    ra.precond_step, gb.precond_step = 2, 1
    gb.L_ema, gb.R_ema = ra.L_ema.to(dev), ra.R_ema.to(dev)
    calls = _count_diag_calls(monkeypatch)
    engine.refresh([(gb, torch.zeros(m, n, device=dev))], eigen_only=True)
    torch.cuda.synchronize()
    assert calls["n"] == 2
    ra._update_eigenfactors(1.0 - ra.rho ** ra.precond_step)
    _compare_exact(ra, gb, "fp32")


def test_mixed_batch(monkeypatch):
    """Two 1024x1024 blocks of one 1024x2048 weight: block 0 diagonal
    (closed form), block 1 dense (solver) in the same dimension's batch."""
    from scao_amd import SparsePreconditioner, engine
    dev = _dev()
    m, n, k, D = 1024, 2048, 32, 1024
    kw = dict(k_min=k, k_max=k, max_precond_dim=D, use_int8_ema=True)
    ra = R.RefPreconditioner(torch.zeros(m, n), **kw)
    gb = SparsePreconditioner(torch.zeros(m, n, device=dev), **kw)
    gen = torch.Generator().manual_seed(12)
    blocks_r = ra._blocks
    blocks_g = [lf for lf, *_ in gb.leaves()]
    assert len(blocks_r) == len(blocks_g) == 2
    codes = [(_diag_codes(D, 3, gen), 8e-7, _diag_codes(D, 2, gen), 7e-7),
             (*_planted_dense(D, k, gen), *_planted_dense(D, k, gen))]
    for la, lb, (ql, sl, qr, sr) in zip(blocks_r, blocks_g, codes):
        la.L_ema_q, la.L_ema_scale, la.R_ema_q, la.R_ema_scale = ql, sl, qr, sr
        la.precond_step, lb.precond_step = 3, 2
        lb.L_ema_q, lb.R_ema_q = ql.to(dev), qr.to(dev)
        lb._scale = torch.tensor([sl, sr], dtype=torch.float64, device=dev)
    ra.precond_step, gb.precond_step = 3, 2
    calls = _count_diag_calls(monkeypatch)
    engine.refresh([(gb, torch.zeros(m, n, device=dev))], eigen_only=True)
    torch.cuda.synchronize()
    assert calls["n"] == 2
    for la in blocks_r:
        la._update_eigenfactors(1.0 - la.rho ** la.precond_step)
    _compare_exact(blocks_r[0], blocks_g[0], "diagonal block")
    la, lb = blocks_r[1], blocks_g[1]
    assert lb.k == la.k
    for U1, S1, U2, S2 in ((la.U_l, la.S_l, lb.U_l, lb.S_l), (la.U_r, la.S_r, lb.U_r, lb.S_r)):
        a = (U1.double() * S1.double()) @ U1.double().T
        b = (U2.cpu().double() * S2.cpu().double()) @ U2.cpu().double().T
        assert ((a - b).norm() / a.norm()).item() < 1e-4
