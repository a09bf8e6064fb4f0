"""GPU parity of the sparse gradient filter (scao_sparse_filter) against the
oracle's restatement of scao/optimizer.py:42-57 on identical gradients:
magnitude EMA and filtered gradient bit-identical over successive calls.

Beyond torch.quantile's 2**24-element limit the reference raises; there the
threshold is checked against the order statistics of the EMA found by a full
partition (np.partition) and ATen's lerp, i.e. what torch.quantile computes
below the limit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import noise as NZ
from oracle import scao_ref as R

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.detach().cpu().float(), b.detach().cpu().float()
    return a.shape == b.shape and torch.equal(a.isnan(), b.isnan()) and \
        torch.equal(torch.nan_to_num(a), torch.nan_to_num(b)) and \
        torch.equal(torch.signbit(a), torch.signbit(b))


def _grads(n, calls, seed, kind="normal", dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(calls):
        if kind == "normal":
            x = torch.randn(n, generator=g) * 1e-3
        elif kind == "ties":          # few distinct magnitudes, many exact ties, zeros
            x = torch.randint(-2, 3, (n,), generator=g).float() * 1e-3
        else:                         # magnitudes within a few ulps of each other
            x = 0.5 * (1 + torch.randint(-3, 4, (n,), generator=g).float() * 2.0 ** -23)
        out.append(x.to(dtype))
    return out


@pytest.mark.parametrize("n,kind,q", [(1, "normal", 0.7), (37, "normal", 0.7),
                                      (4096, "normal", 0.7), (4097, "ties", 0.7),
                                      (100_003, "normal", 0.3), (100_003, "ulps", 0.7),
                                      (1 << 20, "normal", 0.9), (1 << 20, "ties", 0.5),
                                      (5000, "normal", 0.0), (5000, "normal", 1.0)])
def test_filter_matches_oracle(n, kind, q):
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    ref, gpu = R.RefSparseFilter(q), _SparseGradFilter(q)
    for t, g in enumerate(_grads(n, 3, n + 7, kind)):
        print(f"filter n={n} kind={kind} q={q} call={t}", flush=True)
        r = ref(g.clone())
        o = gpu(g.to(dev))
        torch.cuda.synchronize()
        assert _same(gpu.mag_ema, ref.mag_ema), (t, "mag_ema")
        assert _same(o, r), (t, "filtered gradient")


def test_filter_bf16_gradient():
    """The step filters p.grad.float(); the kernel converts bf16 on load."""
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    ref, gpu = R.RefSparseFilter(0.7), _SparseGradFilter(0.7)
    for g in _grads(70_000, 3, 5, dtype=torch.bfloat16):
        r = ref(g.float())
        o = gpu(g.to(dev))
        torch.cuda.synchronize()
        assert o.dtype == torch.float32
        assert _same(gpu.mag_ema, ref.mag_ema) and _same(o, r)


def test_filter_nan_gradient():
    """A NaN in the EMA makes torch.quantile return NaN: nothing passes the
    mask and NaN * 0 stays NaN."""
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    ref, gpu = R.RefSparseFilter(0.7), _SparseGradFilter(0.7)
    for t, g in enumerate(_grads(9000, 3, 11)):
        if t == 1:
            g[1234] = float("nan")
        r = ref(g.clone())
        o = gpu(g.to(dev))
        torch.cuda.synchronize()
        assert _same(gpu.mag_ema, ref.mag_ema) and _same(o, r), t


def test_filter_batched_launch_matches_single():
    """Several parameters in one launch sequence (as the step runs them)
    give what each filter gives on its own."""
    from scao_amd import engine
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    sizes = [(96, 160), (5000,), (3, 7, 11), (2048, 512)]
    qs = [0.7, 0.3, 0.9, 0.5]
    refs = [R.RefSparseFilter(q) for q in qs]
    gpus = [_SparseGradFilter(q) for q in qs]
    g = torch.Generator().manual_seed(3)
    for t in range(3):
        grads = [torch.randn(s, generator=g) * 1e-3 for s in sizes]
        outs = engine.sparse_filter([(f, x.to(dev)) for f, x in zip(gpus, grads)])
        torch.cuda.synchronize()
        for f, rf, x, o in zip(gpus, refs, grads, outs):
            r = rf(x.clone())
            assert _same(f.mag_ema, rf.mag_ema) and _same(o, r), (t, tuple(x.shape))


def _compact(f) -> int:
    """1 when the filter's last call histogrammed the candidate keys instead
    of the whole EMA in its refinement passes."""
    from scao_amd import _lib as L
    return int(f.work[L.FILTER_COMPACT_WORD].item())


@pytest.mark.parametrize("case", ["steady", "jump", "crowded", "q_change", "no_buffer",
                                  "long_segments"])
def test_filter_candidate_passes(case, monkeypatch):
    """The refinement passes read the candidates of the previous call's bin
    only when the threshold stays in that bin and every chunk's region held
    all of its keys of that bin ("crowded": over half of each chunk is in
    it); either way the EMA, threshold and mask match the oracle bit for
    bit."""
    from scao_amd import engine
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    # 300_007 elements give one chunk per block; 2**24 give segments of several
    # chunks whose candidates are streamed as one array
    n, calls = (1 << 24, 3) if case == "long_segments" else (300_007, 5)
    kind = "ulps" if case == "crowded" else "normal"
    grads = _grads(n, calls, 41, kind)
    qs = [0.7] * calls
    if case == "jump":
        grads[3] = grads[3] * 64.0          # the EMA moves up by more than a bin
    if case == "q_change":
        qs[2] = 0.2
    if case == "no_buffer":
        # the C ABI's optional candidate buffer left out (cand = NULL)
        orig = engine._filter_scratch

        def no_cand(f, numel, dev):
            orig(f, numel, dev)
            f.cand = None
        monkeypatch.setattr(engine, "_filter_scratch", no_cand)
    ref, gpu = R.RefSparseFilter(0.7), _SparseGradFilter(0.7)
    modes = []
    for t, g in enumerate(grads):
        print(f"filter candidates case={case} call={t}", flush=True)
        ref.sparsity = gpu.sparsity = qs[t]
        r = ref(g.clone())
        o = gpu(g.to(dev))
        torch.cuda.synchronize()
        modes.append(_compact(gpu))
        from scao_amd import _lib as L
        assert int(gpu.work[L.FILTER_COMPACT_WORD + 1].item()) == 3   # all digits selected
        assert _same(gpu.mag_ema, ref.mag_ema), (t, "mag_ema")
        assert _same(o, r), (t, "filtered gradient")
    assert modes[0] == 0                     # nothing predicted on the first call
    want = {"steady": [0, 1, 1, 1, 1], "jump": [0, 1, 1, 0, 1], "crowded": [0] * calls,
            "q_change": [0, 1, 0, 0, 1], "no_buffer": [0] * calls, "long_segments": [0, 1, 1]}
    assert modes == want[case], modes


def _aten_quantile(e: np.ndarray, q: float) -> np.float32:
    n = e.size
    ranks = np.float32(np.float32(q) * np.float32(n - 1))
    lo, hi = int(ranks), int(np.ceil(ranks))
    w = np.float32(ranks - np.float32(lo))
    part = np.partition(e, [lo, hi])
    a, b = part[lo], part[hi]
    d = np.float32(b - a)
    if abs(w) < 0.5:
        return np.float32(np.float64(w) * np.float64(d) + np.float64(a))
    return np.float32(-np.float64(d) * np.float64(np.float32(1 - w)) + np.float64(b))


@pytest.mark.parametrize("n", [1 << 24, (1 << 24) + 4100])
def test_filter_at_and_beyond_quantile_limit(n):
    """2**24 elements is the largest input torch.quantile takes: there the
    oracle runs whole.  Above it the oracle updates the EMA and then raises
    (as the reference does); the filter still computes the exact statistic,
    checked against a full partition of the same EMA."""
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    ref, gpu = R.RefSparseFilter(0.7), _SparseGradFilter(0.7)
    gen = torch.Generator().manual_seed(1)
    for t in range(2):
        g = torch.randn(n, generator=gen) * 1e-3
        print(f"filter n={n} call={t}", flush=True)
        o = gpu(g.to(dev)).cpu()
        if n <= 1 << 24:
            r = ref(g.clone())
            assert _same(gpu.mag_ema, ref.mag_ema) and _same(o, r), t
            continue
        with pytest.raises(RuntimeError, match="too large"):
            ref(g.clone())
        e = gpu.mag_ema.cpu()
        assert torch.equal(e, ref.mag_ema), t
        thr = _aten_quantile(e.numpy(), 0.7)
        assert torch.equal(o, g * (e >= float(thr)).float()), t


# ----------------------------------------------------------------- noise ---
# grad + randn_like(grad) * noise_std (scao/optimizer.py:544-545).  The
# reference's draws come from torch's generator and cannot be reproduced on
# another device, so the noise is checked for its distribution.

def _ks_normal(x: np.ndarray) -> float:
    from scipy import stats
    return stats.kstest(x, "norm").pvalue


def test_noise_distribution_and_independence():
    from scao_amd import engine
    dev = _dev()
    n, std = 1 << 22, 0.01
    g = torch.randn(n, generator=torch.Generator().manual_seed(2)) * 1e-3
    gd = g.to(dev)
    torch.manual_seed(123)
    a, b = engine.moment_grads([(None, gd), (None, gd)], std)
    c, = engine.moment_grads([(None, gd)], std)
    za = ((a.cpu().double() - g.double()) / std).numpy()
    zb = ((b.cpu().double() - g.double()) / std).numpy()
    zc = ((c.cpu().double() - g.double()) / std).numpy()
    for z in (za, zb, zc):
        assert abs(z.mean()) < 5.0 / np.sqrt(n)
        assert abs(z.std() - 1.0) < 5e-3
        assert _ks_normal(z) > 1e-4
    # separate parameters and separate calls draw separate streams
    assert abs(np.corrcoef(za, zb)[0, 1]) < 5.0 / np.sqrt(n)
    assert abs(np.corrcoef(za, zc)[0, 1]) < 5.0 / np.sqrt(n)
    # consecutive 4-element groups are not correlated either
    assert abs(np.corrcoef(za[:-4], za[4:])[0, 1]) < 5.0 / np.sqrt(n)
    # the same seed gives the same draws
    torch.manual_seed(123)
    a2, _ = engine.moment_grads([(None, gd), (None, gd)], std)
    assert torch.equal(a, a2)


# Box-Muller on the device uses the hardware log2, sqrt, sin and cos; the
# draws must match the float64 restatement to this absolute tolerance.  A
# mistake in the Philox stage (multiplier, key schedule, counter layout)
# changes the draws completely, so it shows at any tolerance.
NOISE_ATOL = 5e-5


@pytest.mark.parametrize("n", [1, 7, 4096 + 3, 1 << 20])
def test_noise_matches_philox_box_muller(n):
    """Noise on a zero gradient is fp32(z * std): z against the oracle's
    Philox4x32-10 + Box-Muller stream under the seed the call drew (torch's
    generator, randint(0, 2^62) per parameter)."""
    from scao_amd import engine
    dev = _dev()
    std = 0.25
    g = torch.zeros(n, device=dev)
    torch.manual_seed(77)
    o, = engine.moment_grads([(None, g)], std)
    torch.manual_seed(77)
    seed = int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64, device=dev).item())
    z = o.cpu().double().numpy() / np.float32(std)
    want = NZ.normals(seed, n)
    err = np.abs(z - want).max()
    assert err <= NOISE_ATOL, (n, err)


def test_filter_then_noise():
    """Noise goes on top of the filtered gradient, everywhere (masked-out
    elements included); the filter part is still bit-exact."""
    from scao_amd import engine
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    ref, gpu = R.RefSparseFilter(0.7), _SparseGradFilter(0.7)
    std = 0.005
    for t, g in enumerate(_grads(1 << 20, 2, 21)):
        r = ref(g.clone())
        o, = engine.moment_grads([(gpu, g.to(dev))], std)
        assert _same(gpu.mag_ema, ref.mag_ema), t
        z = ((o.cpu().double() - r.double()) / std).numpy()
        assert abs(z.mean()) < 5.0 / np.sqrt(z.size) and abs(z.std() - 1.0) < 1e-2
        assert _ks_normal(z) > 1e-4
        masked_out = (r == 0).numpy()
        assert masked_out.mean() > 0.6 and np.abs(z[masked_out]).max() > 0


def test_optimizer_noise_anneals_and_is_applied():
    """SCAO with noise only: the moment gradient differs from the raw one by
    noise of the current (annealed) scale."""
    import scao_amd
    dev = _dev()
    p = torch.nn.Parameter(torch.zeros(512, 256, device=dev))
    opt = scao_amd.SCAO([p], lr=1e-3, sparsity=0.0, noise_std_init=0.02, noise_anneal=0.5,
                        lookahead_k=0, async_precond=False)
    for step, std in enumerate([0.02, 0.01]):
        p.grad = torch.zeros_like(p)
        opt.step()
        # Phase 1 with g = noise only: m = (1 - beta1) * noise
        m = opt.state[p]["exp_avg"] if step == 0 else None
        if m is not None:
            z = (m.double().cpu() / (0.1 * std)).numpy().ravel()
            assert abs(z.std() - 1.0) < 2e-2 and _ks_normal(z) > 1e-4
    assert opt._noise_std == pytest.approx(0.005)


@pytest.mark.parametrize("phase2", [False, True])
def test_step_kernels_form_the_filter_output(phase2):
    """In a step the filter's output pass is skipped and the step kernels form
    fp32(g) * (ema >= t) + noise themselves.  The moment gradient they used
    (stored as prev_grad) equals, bit for bit, what the output pass writes for
    the same filter state and noise key: Phase 1 through the Adam kernel,
    Phase 2 through the wide, masked and diagonal apply paths."""
    import scao_amd
    from scao_amd import engine
    from scao_amd.optimizer import _SparseGradFilter
    dev = _dev()
    shapes = [(512, 512), (100, 37), (300,), (96, 160)]
    g = torch.Generator().manual_seed(17)
    params = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.02).to(dev)) for s in shapes]
    grads = [(torch.randn(s, generator=g) * 1e-3).to(dev) for s in shapes]
    sched = (dict(warmup_steps=0, min_precond_updates=0, precond_freq=10 ** 9) if phase2
             else dict(warmup_steps=10))
    opt = scao_amd.SCAO(params, lr=1e-3, sparsity=0.7, noise_std_init=0.01, lookahead_k=0,
                        async_precond=False, k_min=64, k_max=64, max_precond_dim=512, **sched)
    for p, gr in zip(params, grads):
        p.grad = gr.clone()
    torch.manual_seed(7)
    opt.step()
    filters = [_SparseGradFilter(0.7) for _ in shapes]
    torch.manual_seed(7)
    want = engine.moment_grads(list(zip(filters, grads)), 0.01)
    torch.cuda.synchronize()
    for p, w, f in zip(params, want, filters):
        st = opt.state[p]
        assert torch.equal(st["prev_grad"], w), tuple(p.shape)
        assert torch.equal(opt._sparse_filters[id(p)].mag_ema, f.mag_ema)
    if phase2:
        assert all(opt.state[p].get("scao_phase_started") for p in params)
