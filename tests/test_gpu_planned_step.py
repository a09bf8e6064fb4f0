"""The planned-step fast path of SCAO.step against the full host path.

After a plain step (no refresh, filter, noise or host norms) SCAO.step keeps
the step's plan and, while only the step counters change, the next step
reuses its parameter table (engine.run_planned_step).  Two optimizers over
identical copies of a small model, one with the fast path switched off,
must stay bit-identical through Phase 1, refreshes (which fall back to the
full path), the blend and Phase 2, and the fast path must have run."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

PROFILE = dict(use_int8_ema=True, sparsity=0.0, noise_std_init=0.0, async_precond=False,
               lookahead_k=0)


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def test_planned_steps_match_full_steps(monkeypatch):
    import scao_amd
    from scao_amd import engine
    dev = _dev()
    shapes = [(96, 160), (64, 64), (200, 48), (160,), (3, 4, 5)]
    g = torch.Generator().manual_seed(0)
    init = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(x.clone().to(dev)) for x in init]
    pb = [torch.nn.Parameter(x.clone().to(dev)) for x in init]
    cfg = dict(k_min=4, k_max=8, max_precond_dim=64, warmup_steps=3, blend_steps=4,
               precond_freq=4, min_precond_updates=1, **PROFILE)
    fast = scao_amd.SCAO([{"params": pa[:3]}, {"params": pa[3:], "lr": 3e-3}], **cfg)
    full = scao_amd.SCAO([{"params": pb[:3]}, {"params": pb[3:], "lr": 3e-3}], **cfg)
    planned = []                     # the steps the fast path ran
    orig = engine.run_planned_step
    step_no = [0]

    def counted(*a, **kw):
        planned.append(step_no[0])
        return orig(*a, **kw)
    monkeypatch.setattr(engine, "run_planned_step", counted)
    monkeypatch.setattr(full, "_planned_step", lambda *a: False)
    for t in range(1, 23):
        gg = torch.Generator().manual_seed(100 + t)
        for a, b, s in zip(pa, pb, shapes):
            gr = torch.randn(s, generator=gg) * 0.02
            a.grad = gr.to(dev)
            b.grad = gr.to(dev)
        if t == 9:   # a learning-rate change between planned steps
            for opt in (fast, full):
                opt.param_groups[0]["lr"] = 5e-4
        if t == 13:  # a parameter without a gradient: the plan no longer fits
            pa[1].grad = None
            pb[1].grad = None
        if t == 15:  # new storage behind a parameter: the planned table's
            pa[0].data = pa[0].data.clone()   # pointer is stale, so the
            pb[0].data = pb[0].data.clone()   # full path must take it
        step_no[0] = t
        fast.step()
        full.step()
        torch.cuda.synchronize()
        for a, b in zip(pa, pb):
            assert torch.equal(a, b), t
            sa, sb = fast.state[a], full.state[b]
            for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
                assert torch.equal(sa[key], sb[key]), (t, key)
            assert sa["step"] == sb["step"] and sa["scao_step"] == sb["scao_step"], t
    # each plain step plans the next; steps 13-15 must fall back (a missing
    # gradient, then a parameter count and a storage that no longer match the
    # plan), and planning resumes after them
    assert not {13, 14, 15} & set(planned), planned
    assert any(t < 13 for t in planned) and any(t > 16 for t in planned), planned
