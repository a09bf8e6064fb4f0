"""Zero-size parameters beside ordinary ones.

The reference gives an empty parameter the diagonal mode (an empty matrix
never takes the Kronecker mode, scao/preconditioner.py:142-236) and steps it
with empty updates, so with sparsity 0 it changes nothing for the others and
only its step counters move.  With the sparse filter the reference raises
(torch.quantile refuses an empty input, scao/optimizer.py:56); this filter
skips an empty gradient, as it extends the quantile past torch's size limit.
Either way the ordinary parameters' trajectory with the empty ones present
must be bit-identical to the trajectory without them, through Phase 1,
refreshes, the blend and Phase 2, and the empty parameters' counters must
match the oracle's."""

from __future__ import annotations

import pytest
import torch

from oracle import scao_ref as R

pytestmark = pytest.mark.gpu

EMPTY = [(0, 8), (0,), (8, 0), (3, 0, 4)]
FULL = [(40, 24), (6, 5), (16,)]
MOMENTS = ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad")


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _groups(full, empty):
    """Empty parameters first in one group and last in the other, so the
    ordinary ones sit at shifted table positions."""
    return [{"params": empty[:2] + full[:2]}, {"params": full[2:] + empty[2:], "lr": 3e-3}]


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("sparsity", [0.0, 0.7])
def test_empty_params_change_nothing(sparsity, int8):
    import scao_amd
    dev = _dev()
    cfg = dict(lr=1e-3, weight_decay=0.01, k_min=2, k_max=4, max_precond_dim=32,
               warmup_steps=2, blend_steps=2, precond_freq=3, min_precond_updates=1,
               use_int8_ema=int8, sparsity=sparsity, noise_std_init=0.0, async_precond=False,
               lookahead_k=0)
    g = torch.Generator().manual_seed(0)
    init = [torch.randn(s, generator=g) * 0.02 for s in FULL]
    pa = [torch.nn.Parameter(x.clone().to(dev)) for x in init]
    pb = [torch.nn.Parameter(x.clone().to(dev)) for x in init]
    pe = [torch.nn.Parameter(torch.zeros(s, device=dev)) for s in EMPTY]
    with_empty = scao_amd.SCAO(_groups(pa, pe), **cfg)
    without = scao_amd.SCAO(_groups(pb, []), **cfg)
    ref = None
    if sparsity == 0.0:   # the reference runs this case; its empty parameters' counters
        rf = [torch.nn.Parameter(x.clone()) for x in init]
        re = [torch.nn.Parameter(torch.zeros(s)) for s in EMPTY]
        ref = R.RefSCAO(_groups(rf, re), **cfg)
    for t in range(1, 12):
        gg = torch.Generator().manual_seed(100 + t)
        grads = [torch.randn(s, generator=gg) * 0.02 for s in FULL]
        for a, b, gr in zip(pa, pb, grads):
            a.grad = gr.to(dev)
            b.grad = gr.to(dev)
        for e, s in zip(pe, EMPTY):
            e.grad = torch.zeros(s, device=dev)
        with_empty.step()
        without.step()
        torch.cuda.synchronize()
        for a, b in zip(pa, pb):
            assert torch.equal(a, b), t
            sa, sb = with_empty.state[a], without.state[b]
            for key in MOMENTS:
                assert torch.equal(sa[key], sb[key]), (t, key)
            assert sa["step"] == sb["step"] and sa["scao_step"] == sb["scao_step"], t
        for e, s in zip(pe, EMPTY):
            st = with_empty.state[e]
            assert tuple(e.shape) == s and st["step"] == t, (t, s)
            for key in MOMENTS:
                assert tuple(st[key].shape) == s and st[key].dtype == torch.float32, (t, s, key)
        if ref is not None:
            for p, gr in zip(rf, grads):
                p.grad = gr.clone()
            for e, s in zip(re, EMPTY):
                e.grad = torch.zeros(s)
            ref.step()
            for e, r in zip(pe, re):
                st, sr = with_empty.state[e], ref.state[r]
                assert (st["step"], st["scao_step"]) == (sr["step"], sr["scao_step"]), (t, r.shape)
    # the run reached Phase 2 on the ordinary parameters
    assert all(with_empty.state[a]["scao_step"] > 0 for a in pa[:2])


def test_noncontiguous_param_refused():
    """The kernels address every parameter as a dense row-major view, so a
    parameter whose storage is laid out otherwise (here a transposed view) is
    refused with a clear error at its first step; the reference accepts any
    layout."""
    import scao_amd
    dev = _dev()
    p = torch.nn.Parameter(torch.randn(8, 6, device=dev).t())
    q = torch.nn.Parameter(torch.randn(6, 5, device=dev))
    assert not p.is_contiguous()
    opt = scao_amd.SCAO([q, p], lr=1e-3, sparsity=0.0, noise_std_init=0.0, lookahead_k=0)
    p.grad = torch.randn_like(p)
    q.grad = torch.randn_like(q)
    with pytest.raises(RuntimeError, match="contiguous"):
        opt.step()


def test_param_above_2_31_elements():
    """A 1-D parameter of 2,147,484,000 elements (past 2**31) through Phase 1
    and the diagonal-mode Phase 2 (refreshes, LARS, the planned-step path).
    Parameters and gradients repeat with period 1000, and every update is
    elementwise apart from per-parameter scalars, so every output must repeat
    too, bit for bit: an offset that wrapped at 2**31, or a tail left
    unwritten, breaks the period past that point.  About 70 GB of device
    memory."""
    import scao_amd
    dev = _dev()
    P, K = 1000, 2147484
    assert P * K > 2 ** 31
    g = torch.Generator(device=dev).manual_seed(5)
    p = torch.nn.Parameter((torch.randn(P, generator=g, device=dev) * 0.02).repeat(K))
    opt = scao_amd.SCAO([p], lr=1e-3, weight_decay=0.01, warmup_steps=2, blend_steps=2,
                        precond_freq=2, min_precond_updates=1, sparsity=0.0, noise_std_init=0.0,
                        lookahead_k=0)

    def periodic(x):
        v = x.view(K, P)
        return torch.equal(v, v[:1].expand(K, P))

    for t in range(1, 6):
        p.grad = (torch.randn(P, generator=g, device=dev) * 0.02).repeat(K)
        opt.step()
        torch.cuda.synchronize()
        st = opt.state[p]
        assert st["step"] == t
        assert periodic(p.detach()), t
        for key in MOMENTS:
            assert periodic(st[key]), (t, key)
        p.grad = None
    assert opt.state[p]["scao_step"] > 0   # Phase 2 ran
    # the first period moved (a step that wrote nothing would pass the check)
    assert not torch.equal(p.detach()[:P], (torch.randn(P, generator=torch.Generator(
        device=dev).manual_seed(5), device=dev) * 0.02))
    # hand the memory back: later tests size their batches by the free memory
    del opt, p
    torch.cuda.empty_cache()
