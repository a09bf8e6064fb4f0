"""Preconditioner broadcast and averaging over a two-rank gloo group on the CPU
(reference scao/optimizer.py:686-710, scao/preconditioner.py:647-719,
scao/distributed.py:60-128)."""

from __future__ import annotations

import socket
import types

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from scao_amd import distributed as D
from scao_amd.preconditioner import SparsePreconditioner

SHAPES = [(24, 40), (24, 96), (16,)]   # Kronecker, block-diagonal (64 + 32), diagonal


def _nodes(pre):
    return D._nodes(pre)


def _fake_optimizer(rank: int, int8: bool, k: int = 8, k_other=None):
    """An optimizer-shaped object whose state is filled from a generator
    seeded by `rank`; `k_other` gives the Kronecker parameter another rank."""
    g = torch.Generator().manual_seed(100 + rank)
    params = [torch.nn.Parameter(torch.zeros(s)) for s in SHAPES]
    state = {}
    for i, p in enumerate(params):
        kk = k_other if (k_other is not None and i == 0) else k
        pre = SparsePreconditioner(p, k_min=kk, k_max=kk, max_precond_dim=64, use_int8_ema=int8)
        for node in _nodes(pre):
            node.precond_step = 3 + rank + i
            if node.use_block_diagonal:
                continue
            if node.use_kronecker:
                kn = node._k
                node.U_l = torch.randn(node.m, kn, generator=g)
                node.S_l = torch.rand(kn, generator=g)
                node.U_r = torch.randn(node.n, kn, generator=g)
                node.S_r = torch.rand(kn, generator=g)
                if int8:
                    node.L_ema_q = torch.randint(-127, 128, (node.m, node.m), generator=g,
                                                 dtype=torch.int8)
                    node.R_ema_q = torch.randint(-127, 128, (node.n, node.n), generator=g,
                                                 dtype=torch.int8)
                    node.L_ema_scale = 1e-4 * (1 + torch.rand(1, generator=g).item())
                    node.R_ema_scale = 1e-4 * (1 + torch.rand(1, generator=g).item())
                else:
                    node.L_ema = torch.rand(node.m, node.m, generator=g)
                    node.R_ema = torch.rand(node.n, node.n, generator=g)
            else:
                node.diag_ema = torch.rand(node.diag_ema.shape, generator=g)
        state[p] = {"step": 10 + rank, "scao_step": 2 + rank,
                    "exp_avg": torch.randn(p.shape, generator=g),
                    "exp_avg_sq": torch.rand(p.shape, generator=g),
                    "exp_avg_diff": torch.randn(p.shape, generator=g),
                    "prev_grad": torch.randn(p.shape, generator=g), "preconditioner": pre}
    return types.SimpleNamespace(param_groups=[{"params": params}], state=state)


def _check_broadcast(rank: int, int8: bool) -> None:
    mine = _fake_optimizer(rank, int8, k_other=6 if rank else None)
    src = _fake_optimizer(0, int8)
    D.broadcast_state(mine)
    own = D._states(_fake_optimizer(rank, int8, k_other=6 if rank else None))
    for i, (sm, ss) in enumerate(zip(D._states(mine), D._states(src))):
        for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff"):
            assert torch.equal(sm[key], ss[key]), key
        assert sm["step"] == ss["step"]
        assert sm["scao_step"] == 2 + rank           # not broadcast by the reference
        assert torch.equal(sm["prev_grad"], own[i]["prev_grad"])   # nor is prev_grad
        for a, b in zip(_nodes(sm["preconditioner"]), _nodes(ss["preconditioner"])):
            assert a.precond_step == b.precond_step and a._k == b._k
            if a.use_block_diagonal:
                continue
            if a.use_kronecker:
                for name in ("U_l", "S_l", "U_r", "S_r"):
                    assert torch.equal(getattr(a, name), getattr(b, name)), name
                if int8:
                    assert torch.equal(a.L_ema_q, b.L_ema_q) and torch.equal(a.R_ema_q, b.R_ema_q)
                    # scales travel as fp32 (default-dtype tensors in the reference)
                    f32 = torch.tensor([b.L_ema_scale, b.R_ema_scale], dtype=torch.float32)
                    assert [a.L_ema_scale, a.R_ema_scale] == f32.tolist()
                else:
                    assert torch.equal(a.L_ema, b.L_ema) and torch.equal(a.R_ema, b.R_ema)
            else:
                assert torch.equal(a.diag_ema, b.diag_ema)


def _check_mismatch(rank: int) -> None:
    # a rank that has not stepped: the broadcast refuses on every rank
    mine = _fake_optimizer(rank, False)
    if rank:
        mine.state = {}
    with pytest.raises(ValueError, match="different optimizer states"):
        D.broadcast_state(mine)


def _worker(rank: int, world: int, port: int, what: str) -> None:
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank,
                            world_size=world)
    try:
        if what == "broadcast":
            _check_broadcast(rank, int8=False)
            _check_broadcast(rank, int8=True)
        else:
            _check_mismatch(rank)
        dist.barrier()
    finally:
        dist.destroy_process_group()


def _port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


@pytest.mark.parametrize("what", ["broadcast", "mismatch"])
def test_two_rank_gloo(what):
    mp.spawn(_worker, args=(2, _port(), what), nprocs=2, join=True)


def test_without_a_process_group():
    """The optimizer's broadcast only warns when torch.distributed is not
    initialised (reference behaviour)."""
    assert not dist.is_initialized()
    opt = _fake_optimizer(0, True)
    from scao_amd.optimizer import SCAO
    with pytest.warns(RuntimeWarning, match="not initialised"):
        SCAO.sync_preconditioner(opt)
