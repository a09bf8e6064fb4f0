"""Exactly diagonal eigh inputs: the order LAPACK leaves tied eigenvalues in.

With the large configurations' gradients (N(0, 1e-3^2)) the reference's int8
EMAs keep only their diagonal codes (off-diagonal entries round to code 0 at
every refresh), so each eigh input is a diagonal matrix with a handful of
distinct values over thousands of rows.  torch.linalg.eigh (LAPACK ssyevd,
MKL on the CPU) then returns unit vectors, and which ones are the top k is
decided by the selection sort that ends divide and conquer.

These CPU tests pin oracle.scao_ref.lapack_diagonal_order, the restatement
the device kernel (scao_eig_diag) is built to, against
  * torch.linalg.eigh itself on diagonal inputs with ties, at sizes on both
    sides of LAPACK's small-matrix switch (25 rows) up to 4096;
  * the reference's own refreshes (golden diag_int8, written by
    tests/golden/make_goldens.py): rows, signs, S, codes, scales and k after
    three refreshes of a 2048x2048 and a 512x2048 block;
and show that a stable sort, the plausible mistake, fails them.
"""

from __future__ import annotations

import pytest
import torch

import parity as P
from oracle import scao_ref as R
from scao_inputs import load_golden


def _diag_values(n: int, ncodes: int, gen: torch.Generator) -> torch.Tensor:
    codes = torch.randint(127 - ncodes + 1, 128, (n,), generator=gen).float()
    return codes * (1e-3 / 127) / (1 - 0.999 ** 3) + 1e-7


def _eigh_perm(d: torch.Tensor):
    w, V = torch.linalg.eigh(torch.diag(d))
    rows = V.abs().argmax(0)
    return w, V, rows


@pytest.mark.parametrize("n", [1, 2, 3, 8, 25, 26, 27, 100, 512, 768, 1024, 2048, 4096])
def test_restatement_matches_eigh(n):
    gen = torch.Generator().manual_seed(n)
    for ncodes in (1, 2, 5, 40):
        d = _diag_values(n, ncodes, gen)
        w, V, rows = _eigh_perm(d)
        perm = R.lapack_diagonal_order(d)
        unit = torch.zeros_like(V)
        unit[torch.tensor(perm), torch.arange(n)] = 1.0
        assert torch.equal(V, unit), (n, ncodes)            # +e_perm[j], exactly
        assert torch.equal(w, d[torch.tensor(perm)]), (n, ncodes)   # the values themselves


def test_stable_order_is_not_lapacks():
    """A stable sort (ties in index order) is the obvious stand-in; on tied
    inputs it picks different unit vectors, so the tests above tell the two
    apart."""
    gen = torch.Generator().manual_seed(5)
    d = _diag_values(2048, 2, gen)
    _, _, rows = _eigh_perm(d)
    stable = torch.sort(d, stable=True).indices
    assert not torch.equal(rows, stable)
    assert torch.equal(rows, torch.tensor(R.lapack_diagonal_order(d)))


def _replay_diag():
    """Yields (name, refresh, preconditioner, golden tensors, golden record)
    right after each refresh of the golden's blocks, replayed by the oracle."""
    T, meta = load_golden("diag_int8")
    cfg = dict(meta["config"])
    for pi, (name, shape) in enumerate(meta["blocks"]):   # gradient seeds follow this order
        pre = R.RefPreconditioner(torch.zeros(tuple(shape)), **cfg)
        for r in range(meta["refreshes"]):
            g = torch.Generator().manual_seed(5000 + 10 * r + pi)
            pre.update_curvature(torch.randn(tuple(shape), generator=g) * 1e-3)
            yield name, r, pre, T, meta["rows"][f"{name}.r{r}"]


def test_oracle_matches_reference_diag_refreshes():
    for name, r, pre, T, rec in _replay_diag():
        assert pre.k == rec["k"] and pre.precond_step == rec["precond_step"]
        for side, U, S, q, sc in (("L", pre.U_l, pre.S_l, pre.L_ema_q, pre.L_ema_scale),
                                  ("R", pre.U_r, pre.S_r, pre.R_ema_q, pre.R_ema_scale)):
            key = f"{name}.r{r}.{side}"
            assert rec[side]["offdiag_nonzero"] == 0
            assert int((q != 0).sum() - (q.diagonal() != 0).sum()) == 0
            assert torch.equal(q.diagonal(), T[key + ".diag_codes"]), key
            assert sc == rec[side]["scale"], key
            cols = torch.arange(U.shape[1])
            want = torch.zeros_like(U)
            want[T[key + ".rows"].long(), cols] = T[key + ".sign"]
            assert torch.equal(U, want), key
            assert torch.equal(S, T[key + ".S"]), key


def test_restatement_reproduces_reference_diag_refreshes():
    """The golden's kept columns are the last k of the selection-sort order of
    the eigh input's diagonal, flipped.  (Here only 7-10 of 2048 diagonal
    codes are 126, none near the top, so a stable order would pick the same
    columns; test_stable_order_is_not_lapacks covers inputs where it does
    not.)"""
    for name, r, pre, T, rec in _replay_diag():
        for side, X in zip(("L", "R"), P.eig_input(pre)):
            key = f"{name}.r{r}.{side}"
            d = X.diagonal().float()
            assert torch.count_nonzero(X - torch.diag(X.diagonal())) == 0
            perm = R.lapack_diagonal_order(d)
            k = T[key + ".rows"].numel()
            top = list(reversed(perm))[:k]
            assert top == T[key + ".rows"].tolist(), key
            assert torch.equal(d[torch.tensor(top)], T[key + ".S"]), key
