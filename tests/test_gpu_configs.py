"""GPU parity at every BASELINE configuration, against the CPU reference.

C1 (one 768x3072 weight, k=32, max_precond_dim=1024: three 768x1024 blocks)
runs all 100 steps of the reference's own run (scao/optimizer.py:452-503),
compared per step with the summary the reference itself wrote
(tests/golden/c1_summary.*) and with the oracle run beside it.

C2-C5 take one real layer of each model at its rank k and max_precond_dim D
(the shapes bench.py times, including the block-diagonal remainders
11008 = 5x2048 + 768 and 14336 = 3x4096 + 2048 and the 256x2048 / 1024x4096
kv blocks) plus its norm vectors on the Adam group, and check from shared
state:
  * one steady Phase-2 step through the fast kernels the bench times (wide
    16x256 apply tiles, pipelined apply at k >= 128, 128-row projection
    chunks), element by element at rtol 1e-4;
  * one Phase-1 (Adam) step;
  * the refresh's Gram -> EMA -> requantise, twice (from the identity
    initialisation and then from the reference's codes): codes within 1 LSB,
    scales within 1e-6 relative; C4's gradients carry the 1% x50 outliers
    that stress the int8 absmax scale (scao/utils.py:170-189);
  * for C3 and C5, the eigen stage of one 2048^2 / 4096^2 block from identical
    codes (scao/preconditioner.py:365-451).
The preconditioner state of the Phase-2 step (orthonormal U from QR of
random matrices, positive S, moments) is seeded, so no CPU eigh of a big
block sits in these tests except the one eigen-stage check.
"""

from __future__ import annotations

import copy
import math

import pytest
import torch

import bench
import parity as P
from oracle import scao_ref as R
from parity import report
from scao_inputs import load_golden

pytestmark = pytest.mark.gpu

PROFILE = dict(use_int8_ema=True, sparsity=0.0, noise_std_init=0.0, async_precond=False,
               lookahead_k=0)
# per config: bench.CONFIGS entry, gradient scale, outlier fraction, extra
# Adam-group matrices of one layer's sample
LAYERS = {
    "C2_gpt2s": ("gpt2s", 0.02, 0.0, {}),
    "C3_llama1b": ("llama1b", 1e-3, 0.0, {"embed_rows": (2048, 2048)}),
    "C4_qwen3b": ("qwen3b", 1e-3, 0.01, {}),
    "C5_llama8b": ("llama8b", 1e-3, 0.0, {}),
}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _layer(name):
    key, gscale, outl, extra = LAYERS[name]
    c = bench.CONFIGS[key]
    mats = {n: tuple(s) for n, s in c["mats"]}
    adam = {n: (d,) for n, d in c["vecs"]}
    adam.update(extra)
    return c, mats, adam, gscale, outl


def _params(shapes: dict, seed: int, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    return {k: torch.nn.Parameter(torch.randn(s, generator=g) * scale) for k, s in shapes.items()}


def _grads(shapes: dict, seed: int, scale: float, outliers: float):
    """N(0, scale^2) with a Bernoulli(outliers) mask of x50 entries (the
    C4 heavy tails), drawn from torch.Generator(seed) shape by shape."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for k, s in shapes.items():
        x = torch.randn(s, generator=g) * scale
        if outliers > 0:
            x = torch.where(torch.rand(s, generator=g) < outliers, x * 50.0, x)
        out[k] = x
    return out


def _groups(c, mats_p, adam_p, warmup):
    k, D = c["k"], c["D"]
    pre = dict(params=list(mats_p.values()), k_min=k, k_max=k, max_precond_dim=D,
               warmup_steps=warmup)
    ad = dict(params=list(adam_p.values()), k_min=k, k_max=k, max_precond_dim=D,
              warmup_steps=10 ** 9)
    return [pre, ad]


def _orth(m, k, g):
    return torch.linalg.qr(torch.randn(m, k, generator=g, dtype=torch.float64))[0].float()


def _seed_state(ref, t_next: int, phase2: bool, gen):
    """Fill the reference optimizer's state as if `t_next - 1` steps had run:
    moments of realistic size and, for the preconditioned group, Phase 2
    past the blend with seeded eigenfactors (orthonormal U, positive S in
    descending order) after three refreshes."""
    for gi, group in enumerate(ref.param_groups):
        for p in group["params"]:
            ref._init_state(p, group)
            st = ref.state[p]
            st["step"] = t_next - 1
            shp = p.shape
            st["exp_avg"].copy_(torch.randn(shp, generator=gen) * 3e-4)
            st["exp_avg_sq"].copy_(torch.randn(shp, generator=gen).square() * 1e-6 + 1e-9)
            st["exp_avg_diff"].copy_(torch.randn(shp, generator=gen) * 3e-5)
            st["prev_grad"].copy_(torch.randn(shp, generator=gen) * 1e-3)
            if gi == 0 and phase2:
                st["scao_phase_started"] = True
                st["phase2_start_step"] = t_next - 12
                st["scao_step"] = 11
                pre = st["preconditioner"]
                pre.precond_step = 3
                for leaf, *_ in P.kron_leaves(pre):
                    pre_k = leaf.k_max
                    leaf._k = pre_k
                    leaf.U_l = _orth(leaf.m, pre_k, gen)
                    leaf.U_r = _orth(leaf.n, pre_k, gen)
                    leaf.S_l = (torch.rand(pre_k, generator=gen) * 4e-3 + 1e-4).sort(
                        descending=True).values
                    leaf.S_r = (torch.rand(pre_k, generator=gen) * 4e-3 + 1e-4).sort(
                        descending=True).values
                    leaf.precond_step = 3
                if pre.use_block_diagonal:
                    for b in pre._blocks:
                        b.precond_step = 3
                    pre._k = sum(b._k for b in pre._blocks) // len(pre._blocks)


def _to_gpu(ref, params: dict, cfg_groups, dev):
    import scao_amd
    gp = {k: torch.nn.Parameter(v.detach().clone().to(dev)) for k, v in params.items()}
    names = list(params)
    groups = []
    for g in cfg_groups:
        ids = {id(p) for p in g["params"]}
        gg = dict(g)
        gg["params"] = [gp[n] for n in names if id(params[n]) in ids]
        groups.append(gg)
    opt = scao_amd.SCAO(groups, **PROFILE)
    opt.load_state_dict(copy.deepcopy(ref.state_dict()))
    return gp, opt


def _compare_step(name, phase, params, gp, ref, gopt, before, extra_abs=None):
    worst_u, worst_m = 0.0, 0.0
    for k in params:
        worst_u = max(worst_u, P.assert_update_close(
            gp[k], params[k], before[k], f"{name} {phase} {k} update",
            extra_abs=(extra_abs or {}).get(k, 0.0)))
        st_r, st_g = ref.state[params[k]], gopt.state[gp[k]]
        for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
            worst_m = max(worst_m, P.assert_close(st_g[key], st_r[key], P.MOMENT_RTOL,
                                                  P.MOMENT_ATOL, f"{name} {phase} {k} {key}"))
    report("config_step", f"{name}/{phase}", {"update_ratio": worst_u, "moment_ratio": worst_m,
                                             "gate": "elementwise ratio <= 1"})
    return worst_u


def _norm_ema_check(name, gopt, ref, ema_before, grads):
    """The grad-norm average (scao/optimizer.py:439-446): the kernels' norms
    are double; against the reference's formula with correctly rounded
    float32 norms at 1e-6, and against the reference as it runs within
    1e-6 plus twice its own float32-norm deviation."""
    norms = [float(g.double().norm().float()) for g in grads.values()]
    exact = 0.95 * ema_before + 0.05 * (sum(norms) / len(norms))
    dev32 = abs(ref._global_norm_ema - exact)
    got = gopt._global_norm_ema
    assert got == pytest.approx(exact, rel=1e-6)
    assert abs(got - ref._global_norm_ema) <= 1e-6 * abs(ref._global_norm_ema) + 2.0 * dev32
    return dev32 / abs(exact)


@pytest.mark.parametrize("p0", [False, True], ids=["params", "zero_params"])
@pytest.mark.parametrize("name", list(LAYERS))
def test_config_phase2_step(name, p0):
    """One steady Phase-2 step (blend done, no refresh) of one real layer from
    shared seeded state, through the kernels bench.py times, against the
    reference as it runs.

    The kernels take every norm in double; the reference takes them in
    float32 on the CPU, where they run low on tensors this size (0.45% at
    22.5M elements).  In this step only the LARS trust ratio depends on a
    norm (scao/optimizer.py:371-377), so the step is pinned in three parts:
      * the kernels' intermediates against the reference's (oracle RECORD):
        the staged update u elementwise at rtol 1e-4 (no norm enters it), the
        natural-gradient norm and clip factor at 1e-6, and the trust and both
        LARS norms at 1e-6 against the reference's formula with correctly
        rounded float32 norms;
      * the stored parameters against the unmodified reference, elementwise
        at rtol 1e-4 plus 2 E_norm, E_norm = max |lr (trust_f32 - trust_exact)
        u|: how far the reference's own float32 norms move its update (the
        rule the refresh steps use for the reference's eigensolver);
      * with ``zero_params`` the preconditioned matrices start at 0, so the
        stored parameter is the update itself, -lr * u (no decay; LARS trust 1
        for a zero norm in both), compared at rtol 1e-4 without the float32
        write resolution of a non-zero parameter."""
    from scao_amd import engine
    dev = _dev()
    c, mats, adam, gscale, outl = _layer(name)
    shapes = {**mats, **adam}
    params = _params(shapes, 0)
    if p0:
        for k in mats:
            params[k].data.zero_()
    groups = _groups(c, {k: params[k] for k in mats}, {k: params[k] for k in adam}, warmup=5)
    ref = R.RefSCAO(groups, precond_freq=10 ** 9, blend_steps=5, min_precond_updates=1,
                    **PROFILE)
    print(f"{name}: seeding state", flush=True)
    _seed_state(ref, 41, True, torch.Generator().manual_seed(7))
    gp, gopt = _to_gpu(ref, params, groups, dev)
    grads = _grads(shapes, 1041, gscale, outl)
    before = {k: v.detach().clone() for k, v in params.items()}
    for k in shapes:
        params[k].grad = grads[k]
        gp[k].grad = grads[k].to(dev)
    ema_before = ref._global_norm_ema
    print(f"{name}: reference step", flush=True)
    R.RECORD = {}
    try:
        ref.step()
    finally:
        rec, R.RECORD = R.RECORD, None
    print(f"{name}: GPU step", flush=True)
    gopt.step()
    torch.cuda.synchronize()
    # the launches are the bench's: wide tiles (variant bit 4) over whole
    # blocks, through a two-role kernel (pipelined bit 8, strip bit 16) at k >= 128
    ws = gopt._ws
    wide = sum(n for kind, n in ws.ntasks.items() if kind.startswith("apply") and int(kind[5:]) & 4)
    pipe = sum(n for kind, n in ws.ntasks.items() if kind.startswith("apply") and int(kind[5:]) & 24)
    assert wide > 0
    assert (pipe > 0) == (c["k"] >= engine.PIPE_MIN_RANK)
    grp = ref.param_groups[0]
    lr, wd, lc = grp["lr"], grp["weight_decay"], grp["lars_coeff"]
    stats = P.step_stats(gopt)
    extra, worst = {}, {"u": 0.0, "scalar_rel": 0.0, "e_norm_rel": 0.0}
    for k in mats:
        r, st = rec[id(params[k])], stats[id(gp[k])]
        worst["u"] = max(worst["u"], P.assert_close(st["upd"], r["upd"], P.UPDATE_RTOL,
                                                    P.UPDATE_ATOL, f"{name} {k} staged u"))
        trust_x, pn_x, un_x = P.lars_exact(r, wd, lc)
        for key, want in (("trust", trust_x), ("pnorm", pn_x), ("unorm", un_x),
                          ("nu", r["nu"]), ("clip", r["clip"])):
            rel = abs(st[key] - want) / max(abs(want), 1e-30)
            worst["scalar_rel"] = max(worst["scalar_rel"], rel)
            assert rel <= 1e-6, (name, k, key, st[key], want)
        e_norm = P.norm_allowance(r, trust_x, lr)
        extra[k] = 2.0 * e_norm
        umax = lr * r["trust"] * r["upd"].abs().max().item()
        worst["e_norm_rel"] = max(worst["e_norm_rel"], e_norm / umax if umax > 0 else 0.0)
        if p0:
            assert r["trust"] == 1.0 and e_norm == 0.0
    report("config_phase2_intermediates", f"{name}/{'p0' if p0 else 'params'}", worst)
    _compare_step(name, "phase2" + ("/p0" if p0 else ""), params, gp, ref, gopt, before,
                  extra_abs=extra)
    dev32 = _norm_ema_check(name, gopt, ref, ema_before, grads)
    report("config_reference_fp32_norm", name, {"grad_norm_avg_rel_deviation": dev32,
                                               "lars_update_deviation_rel": worst["e_norm_rel"]})


@pytest.mark.parametrize("name", ["C3_llama1b", "C4_qwen3b", "C5_llama8b"])
def test_projection_split_products(name):
    """The bench's projection of whole fp32 strips (64, 128 and 256 rows of T
    per task at k = 64, 128, 256) forms T = U_l^T G with each fp32 product as
    six bf16 MFMAs over exact three-way splits.  Every block's T, read from
    the step's workspace, is checked against float64 elementwise relative to
    (|U_l|^T |G|): fp32-grade accuracy (bf16 products alone would be ~1e-3
    off)."""
    import numpy as np
    from scao_amd import _lib as L
    dev = _dev()
    c, mats, adam, gscale, outl = _layer(name)
    shapes = {**mats, **adam}
    params = _params(shapes, 0)
    groups = _groups(c, {k: params[k] for k in mats}, {k: params[k] for k in adam}, warmup=5)
    ref = R.RefSCAO(groups, precond_freq=10 ** 9, blend_steps=5, min_precond_updates=1,
                    **PROFILE)
    _seed_state(ref, 41, True, torch.Generator().manual_seed(7))
    gp, gopt = _to_gpu(ref, params, groups, dev)
    grads = _grads(shapes, 1041, gscale, outl)
    for k in shapes:
        gp[k].grad = grads[k].to(dev)
    gopt.step()
    torch.cuda.synchronize()
    ws = gopt._ws
    scratch = ws._bufs["leaf_scratch"]
    tab = np.frombuffer(ws.leaf_dev.cpu().numpy().tobytes(), dtype=L.LEAF_DESC)
    owner = {}
    for nm in mats:
        for leaf, *_ in P.kron_leaves(gopt.state[gp[nm]]["preconditioner"]):
            owner[id(leaf)] = nm
    worst, nblk = 0.0, 0
    for (leaf, r0, c0, pi), e in zip(ws.leaves, tab):
        if not leaf.use_kronecker or id(leaf) not in owner:
            continue
        m, n, k = int(e["m"]), int(e["n"]), int(e["k"])
        off = (int(e["T"]) - scratch.data_ptr()) // 4
        T = scratch.view(torch.float32)[off:off + k * n].view(k, n).double().cpu()
        G = grads[owner[id(leaf)]]
        G = G.reshape(G.shape[0], -1)[r0:r0 + m, c0:c0 + n].double()
        U = leaf.U_l.double().cpu()
        exact = U.T @ G
        scale = U.abs().T @ G.abs()
        worst = max(worst, ((T - exact).abs() / scale.clamp_min(1e-30)).max().item())
        nblk += 1
    assert nblk > 0
    report("projection_split_products", name, {"blocks": nblk, "max_rel_to_abs_sum": worst})
    assert worst < 1e-5, worst


@pytest.mark.parametrize("name", ["C2_gpt2s", "C3_llama1b", "C4_qwen3b", "C5_llama8b"])
def test_config_phase1_step(name):
    """One Phase-1 (Adam(W)) step of the same layer from shared seeded moments."""
    dev = _dev()
    c, mats, adam, gscale, outl = _layer(name)
    shapes = {**mats, **adam}
    params = _params(shapes, 0)
    groups = _groups(c, {k: params[k] for k in mats}, {k: params[k] for k in adam},
                     warmup=10 ** 9)
    ref = R.RefSCAO(groups, precond_freq=10 ** 9, blend_steps=5, min_precond_updates=1,
                    **PROFILE)
    _seed_state(ref, 7, False, torch.Generator().manual_seed(9))
    gp, gopt = _to_gpu(ref, params, groups, dev)
    grads = _grads(shapes, 1007, gscale, outl)
    before = {k: v.detach().clone() for k, v in params.items()}
    for k in shapes:
        params[k].grad = grads[k]
        gp[k].grad = grads[k].to(dev)
    print(f"{name}: reference Adam step", flush=True)
    ema_before = ref._global_norm_ema
    ref.step()
    gopt.step()
    torch.cuda.synchronize()
    _compare_step(name, "phase1", params, gp, ref, gopt, before)
    _norm_ema_check(name, gopt, ref, ema_before, grads)


def _ema_pairs(ref_pre, gpu_pre):
    return list(zip(P.kron_leaves(ref_pre), gpu_pre.leaves()))


@pytest.mark.parametrize("name", list(LAYERS))
def test_config_refresh_ema(name):
    """Gram -> EMA -> requantise of every block of one layer, twice: the first
    refresh from the identity initialisation, the second from the reference's
    own codes.  Codes within 1 LSB, scales within 1e-6 relative."""
    from scao_amd import SparsePreconditioner, engine
    dev = _dev()
    c, mats, _, gscale, outl = _layer(name)
    kw = dict(k_min=c["k"], k_max=c["k"], max_precond_dim=c["D"], use_int8_ema=True)
    worst_lsb, worst_scale, nblk = 0, 0.0, 0
    lsb_hist = {}
    for mname, shape in mats.items():
        ra = R.RefPreconditioner(torch.zeros(shape), **kw)
        gb = SparsePreconditioner(torch.zeros(shape, device=dev), **kw)
        for r in range(2):
            g = _grads({mname: shape}, 2000 + 10 * r + len(mname), gscale, outl)[mname]
            print(f"{name} {mname} {shape}: refresh {r}", flush=True)
            if r == 1:   # continue from the reference's codes
                for (la, *_), (lb, *_) in _ema_pairs(ra, gb):
                    lb.L_ema_q = la.L_ema_q.to(dev)
                    lb.R_ema_q = la.R_ema_q.to(dev)
                    lb._scale = torch.tensor([la.L_ema_scale, la.R_ema_scale],
                                             dtype=torch.float64, device=dev)
            engine.refresh([(gb, g.to(dev))], ema_only=True)
            for (la, r0, c0), (lb, *_) in _ema_pairs(ra, gb):
                la._update_ema(g[r0:r0 + la.m, c0:c0 + la.n])
                for side in ("L", "R"):
                    qa = getattr(la, f"{side}_ema_q").int()
                    qb = getattr(lb, f"{side}_ema_q").cpu().int()
                    d = (qa - qb).abs()
                    lsb = d.max().item()
                    for v in range(lsb + 1):
                        lsb_hist[v] = lsb_hist.get(v, 0) + int((d == v).sum())
                    sa = getattr(la, f"{side}_ema_scale")
                    sb = getattr(lb, f"{side}_ema_scale")
                    rel = abs(sa - sb) / abs(sa)
                    worst_lsb, worst_scale = max(worst_lsb, lsb), max(worst_scale, rel)
                    assert lsb <= 1, (mname, r, side, lsb)
                    assert rel <= 1e-6, (mname, r, side, sa, sb)
                nblk += 1
    report("config_refresh_ema", name, {"max_code_lsb": worst_lsb, "max_scale_rel": worst_scale,
                                        "blocks": nblk, "code_diff_counts": lsb_hist})


def _planted_codes(dim, k, gen):
    """int8 codes and scale of Q diag(lam) Q^T, Q a random orthogonal matrix,
    lam_i = 1 - i/(2k) for the top k and at most 0.05 below: a spectrum whose
    top-k eigenspace is well defined (a gap of 10x at the cut) after int8
    quantisation, like a curvature EMA dominated by a few directions.  (From
    the identity initialisation the first EMA quantises to a diagonal matrix
    whose top-k eigenspace is not unique, so it cannot pin an eigensolver.)"""
    Q = torch.linalg.qr(torch.randn(dim, dim, generator=gen, dtype=torch.float64))[0]
    lam = torch.empty(dim, dtype=torch.float64)
    lam[:k] = 1.0 - torch.arange(k, dtype=torch.float64) / (2 * k)
    lam[k:] = 0.05 * torch.rand(dim - k, generator=gen, dtype=torch.float64)
    X = ((Q * lam) @ Q.T).float()
    X = 0.5 * (X + X.T)
    return R.quantize_sym_int8(X)


@pytest.mark.parametrize("name,mat", [("C3_llama1b", "q"), ("C5_llama8b", "q"),
                                      ("C4_qwen3b", "k")])
def test_config_eigen_stage(name, mat):
    """The eigen stage of one real block (2048^2 at C3, 4096^2 at C5, the
    256x2048 kv block at C4) from identical int8 codes: debias, Tikhonov,
    eigh, flip/clamp, adaptive rank, rank momentum
    (scao/preconditioner.py:365-451)."""
    from scao_amd import SparsePreconditioner, engine
    dev = _dev()
    c, mats, _, _, _ = _layer(name)
    shape = mats[mat]
    kw = dict(k_min=c["k"], k_max=c["k"], max_precond_dim=c["D"], use_int8_ema=True)
    ra = R.RefPreconditioner(torch.zeros(shape), **kw)
    gb = SparsePreconditioner(torch.zeros(shape, device=dev), **kw)
    gen = torch.Generator().manual_seed(3000)
    print(f"{name} {mat} {shape}: planting spectra", flush=True)
    ra.L_ema_q, ra.L_ema_scale = _planted_codes(shape[0], ra.k_max, gen)
    ra.R_ema_q, ra.R_ema_scale = _planted_codes(shape[1], ra.k_max, gen)
    ra.precond_step = 5
    gb.precond_step = 4
    gb.L_ema_q, gb.R_ema_q = ra.L_ema_q.to(dev), ra.R_ema_q.to(dev)
    gb._scale = torch.tensor([ra.L_ema_scale, ra.R_ema_scale], dtype=torch.float64, device=dev)
    print(f"{name} {mat} {shape}: GPU eigen stage", flush=True)
    engine.refresh([(gb, torch.zeros(shape, device=dev))], eigen_only=True)
    torch.cuda.synchronize()
    print(f"{name} {mat} {shape}: reference eigen stage (CPU eigh)", flush=True)
    ra._update_eigenfactors(1.0 - ra.rho ** ra.precond_step)
    assert gb.precond_step == ra.precond_step and gb.k == ra.k
    errs = {}
    for side, (U1, S1, U2, S2) in (("L", (ra.U_l, ra.S_l, gb.U_l, gb.S_l)),
                                  ("R", (ra.U_r, ra.S_r, gb.U_r, gb.S_r))):
        S2, U2 = S2.cpu(), U2.cpu()
        errs[side + "_S_rel"] = ((S2 - S1).abs() / S1.abs()).max().item()
        a = (U1.double() * S1.double()) @ U1.double().T
        b = (U2.double() * S2.double()) @ U2.double().T
        errs[side] = ((a - b).norm() / a.norm()).item()
        # orthonormal columns
        errs[side + "_orth"] = (U2.double().T @ U2.double() -
                                torch.eye(U2.shape[1], dtype=torch.float64)).abs().max().item()
    report("config_eigen_stage", f"{name}/{mat}", errs)
    for side in ("L", "R"):
        assert errs[side + "_S_rel"] < 1e-4, errs
        assert errs[side] < 1e-4, errs
        assert errs[side + "_orth"] < 1e-4, errs


def _from_reference_init(name, mats_sel, steps=8, exact_u=True):
    """Steps of one layer's weights from the reference's own initialisation
    (identity EMAs, U = eye, S = 1) at the configuration's gradient scale
    (with C4's outliers), a refresh every 2 steps (Adam at steps 1-2, blend
    over steps 3-4, Phase 2 after), against the CPU reference as it runs.

    At each refresh the GPU's new codes are checked against the reference's
    (1 LSB, scales 1e-6) and replaced by them (parity.IdenticalPostEma).
    With ``exact_u`` the new eigenfactors must then equal the reference's
    column for column (exactly diagonal inputs); otherwise they are checked
    by spectral projector and replaced by the reference's
    (parity.ReferenceEigen).  Every step's update (each side from its own
    previous parameters, as in the C1 run: an Adam step's rounding at 1e-3
    updates is far above a Phase-2 LARS step's size) must agree elementwise
    at rtol 1e-4 plus two float32 spacings of p (each side rounds its own
    decayed parameter and its own sum) plus 2 E_norm for the reference's
    float32 LARS norms, whose Phase-2 intermediates are checked as in
    test_config_phase2_step; the moments at rtol 1e-4; the whole trajectory
    at rtol 1e-4 of the cumulative update.  With dense factors (not
    ``exact_u``) a copy of the reference also takes each Phase-2 step with
    its preconditioned gradient in float64 (oracle EXACT_PRECOND): u and the
    moments are then allowed twice the largest difference between the two
    references (E_u, E_m), as the refresh steps of the shared-state tests are
    for the reference's float32 eigh -- at an element where the update is a
    small difference of larger terms the reference's own float32 GEMMs move
    it by more than rtol 1e-4."""
    import scao_amd
    from scao_amd import engine
    dev = _dev()
    c, mats, _, gscale, outl = _layer(name)
    shapes = {k: mats[k] for k in mats_sel}
    params = _params(shapes, 0)
    cfg = dict(precond_freq=2, warmup_steps=2, blend_steps=2, min_precond_updates=1)
    rgroups = [dict(params=list(params.values()), k_min=c["k"], k_max=c["k"],
                    max_precond_dim=c["D"])]
    ref = R.RefSCAO(rgroups, **cfg, **PROFILE)
    gp = {k: torch.nn.Parameter(v.detach().clone().to(dev)) for k, v in params.items()}
    gopt = scao_amd.SCAO([dict(rgroups[0], params=list(gp.values()))], **cfg, **PROFILE)
    worst = {"step_ratio": 0.0, "moment_ratio": 0.0, "traj_ratio": 0.0, "diag_calls": 0,
             "projector": 0.0}
    init = {k: v.detach().clone() for k, v in params.items()}
    prev_gpu = {k: v.detach().clone() for k, v in params.items()}
    cum_norm = {k: 0.0 for k in params}
    nblocks = sum(len(bench.leaves_of(s_, c["D"])) for s_ in shapes.values())
    orig = engine._diag_eigh

    def counted(part, *a):
        worst["diag_calls"] += len(part)
        return orig(part, *a)
    engine._diag_eigh = counted
    try:
        for t in range(1, steps + 1):
            grads = _grads(shapes, 3000 + t, gscale, outl)
            before = {k: v.detach().clone() for k, v in params.items()}
            for k in shapes:
                params[k].grad = grads[k]
                gp[k].grad = grads[k].to(dev)
            shadow = None
            if not exact_u and t > cfg["warmup_steps"]:
                # the reference with its preconditioned gradient in float64:
                # how far its own float32 GEMMs move u and the moments
                sp = {k: torch.nn.Parameter(v.detach().clone()) for k, v in params.items()}
                sr = R.RefSCAO([dict(rgroups[0], params=list(sp.values()))], **cfg, **PROFILE)
                sr.load_state_dict(copy.deepcopy(ref.state_dict()))
                for k in shapes:
                    sp[k].grad = grads[k].clone()
                shadow = (sr, sp)
            print(f"{name} from init: step {t} reference", flush=True)
            R.RECORD = {}
            try:
                ref.step()
            finally:
                rec, R.RECORD = R.RECORD, None
            e_u, e_mom = {}, {}
            if shadow is not None:
                R.RECORD, R.EXACT_PRECOND = {}, True
                try:
                    shadow[0].step()
                finally:
                    rec_x, R.RECORD, R.EXACT_PRECOND = R.RECORD, None, False
                for k in shapes:
                    px = shadow[1][k]
                    e_u[k] = (rec[id(params[k])]["upd"] - rec_x[id(px)]["upd"]).abs().max().item()
                    for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
                        e_mom[(k, key)] = (ref.state[params[k]][key] -
                                           shadow[0].state[px][key]).abs().max().item()
                    worst["e_u"] = max(worst.get("e_u", 0.0), e_u[k])
                del shadow, rec_x
            pairs = {}
            for k in shapes:
                if gp[k] in gopt.state:
                    for (la, *_), (lb, *_) in zip(P.kron_leaves(ref.state[params[k]]["preconditioner"]),
                                                  gopt.state[gp[k]]["preconditioner"].leaves()):
                        pairs[id(lb)] = la
            hook = P.IdenticalPostEma(pairs)
            eig_hook = None if exact_u else P.ReferenceEigen(pairs)
            engine.AFTER_EMA_HOOK, engine.AFTER_EIGEN_HOOK = hook, eig_hook
            try:
                print(f"{name} from init: step {t} GPU", flush=True)
                gopt.step()
            finally:
                engine.AFTER_EMA_HOOK = engine.AFTER_EIGEN_HOOK = None
            torch.cuda.synchronize()
            stats = P.step_stats(gopt) if rec else {}
            grp = ref.param_groups[0]
            for k in shapes:
                # a Phase-2 step: the staged u elementwise, the trust against
                # exact norms, E_norm for the reference's float32 norms
                e_norm = e_prec = 0.0
                if id(params[k]) in rec:
                    r_, st_ = rec[id(params[k])], stats[id(gp[k])]
                    P.assert_close(st_["upd"], r_["upd"], P.UPDATE_RTOL, P.UPDATE_ATOL,
                                   f"t{t} {k} staged u", extra=2.0 * e_u.get(k, 0.0))
                    trust_x = P.lars_exact(r_, grp["weight_decay"], grp["lars_coeff"])[0]
                    assert abs(st_["trust"] - trust_x) <= 1e-6 * trust_x, (t, k, st_["trust"], trust_x)
                    e_norm = P.norm_allowance(r_, trust_x, grp["lr"])
                    e_prec = grp["lr"] * r_["trust"] * e_u.get(k, 0.0)
                cum_norm[k] += 2.0 * (e_norm + e_prec)
                # each side rounds its own decayed parameter and its own sum
                # (its previous parameters differ by a few float32 spacings),
                # so the two step updates may differ by two spacings of p
                pg_new = gp[k].detach().cpu()
                r = P.ratio(pg_new - prev_gpu[k], params[k].detach() - before[k], P.UPDATE_RTOL,
                            P.UPDATE_ATOL,
                            extra=2.0 * torch.maximum(P.ulp(params[k]), P.ulp(pg_new)) +
                            2.0 * (e_norm + e_prec))
                assert r <= 1.0, (t, k, "step update", r)
                worst["step_ratio"] = max(worst["step_ratio"], r)
                worst["traj_ratio"] = max(worst["traj_ratio"], P.assert_close(
                    pg_new - init[k], params[k].detach() - init[k], 1e-4, 1e-5,
                    f"{name} from init t{t} {k} cumulative update", extra=cum_norm[k]))
                prev_gpu[k] = pg_new
                st_r, st_g = ref.state[params[k]], gopt.state[gp[k]]
                for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
                    worst["moment_ratio"] = max(worst["moment_ratio"], P.assert_close(
                        st_g[key], st_r[key], P.MOMENT_RTOL, P.MOMENT_ATOL, f"t{t} {k} {key}",
                        extra=2.0 * e_mom.get((k, key), 0.0)))
            if t % cfg["precond_freq"]:
                continue
            assert hook.checked == nblocks
            if eig_hook is not None:
                assert eig_hook.checked == nblocks
                worst["projector"] = max(worst["projector"], eig_hook.worst)
            for k in shapes:
                pr = ref.state[params[k]]["preconditioner"]
                pg = gopt.state[gp[k]]["preconditioner"]
                for (la, *_), (lb, *_) in zip(P.kron_leaves(pr), pg.leaves()):
                    if exact_u:
                        for q in (la.L_ema_q, la.R_ema_q):
                            assert int((q != 0).sum() - (q.diagonal() != 0).sum()) == 0
                    assert lb.k == la.k and lb.precond_step == la.precond_step, (t, k)
                    for U1, S1, U2, S2 in ((la.U_l, la.S_l, lb.U_l, lb.S_l),
                                           (la.U_r, la.S_r, lb.U_r, lb.S_r)):
                        assert torch.equal(U2.cpu(), U1), (t, k, "U")
                        assert torch.equal(S2.cpu(), S1), (t, k, "S")
    finally:
        engine._diag_eigh = orig
    return worst, nblocks


def test_c3_layer_from_reference_init():
    """C3 from the reference's own initialisation at N(0, 1e-3^2) gradients:
    the layer's q (2048^2), k (512x2048) and down (2048x8192: four strided
    2048^2 blocks) weights, 8 steps, four refreshes.  At this scale the int8
    EMAs keep only their diagonal codes (the CPU reference's off-diagonal
    codes are checked to be all zero), so every eigh input is exactly
    diagonal, the reference's eigenvectors are unit vectors in LAPACK's tie
    order, and the GPU's must equal them column for column
    (_from_reference_init)."""
    worst, nblocks = _from_reference_init("C3_llama1b", ("q", "k", "down"))
    assert worst["diag_calls"] == 4 * nblocks * 2
    report("c3_from_reference_init", "8 steps, 4 refreshes", worst)


def test_c4_layer_from_reference_init():
    """C4 from the reference's own initialisation: N(0, 1e-3^2) gradients
    with 1% x50 outliers, the layer's q (2048^2), k (256x2048) and gate
    (11008x2048: five 2048^2 blocks and a 768x2048 remainder) weights, 6
    steps, three refreshes.  The outliers give the EMAs off-diagonal codes
    (10-20% of them), a dense factor with distinct top-128 eigenvalues, so
    the solver runs on every factor; its eigenfactors are checked by
    spectral projector against the reference's (_from_reference_init)."""
    worst, nblocks = _from_reference_init("C4_qwen3b", ("q", "k", "gate"), steps=6,
                                          exact_u=False)
    assert worst["diag_calls"] == 0
    report("c4_from_reference_init", "6 steps, 3 refreshes", worst)


# ---------------------------------------------------------------- C1 ---

def _c1_quantities(p, st, pre):
    """The per-step quantities tests/golden/make_goldens.py records for C1."""
    pd = p.detach().cpu().double()
    q = {"p_norm": pd.norm().item(), "p_sum": pd.sum().item(),
         "p_head": pd.reshape(-1)[:16],
         "m_norm": st["exp_avg"].cpu().double().norm().item(),
         "v_sum": st["exp_avg_sq"].cpu().double().sum().item(), "blocks": []}
    for lb, *_ in P.kron_leaves(pre):
        q["blocks"].append({"L_scale": lb.L_ema_scale, "R_scale": lb.R_ema_scale, "k": lb.k,
                            "S_l_head": lb.S_l[:4].cpu().double()})
    return q


def _c1_diff(a, b, worst, tag):
    """Relative differences of two quantity records (b may be a golden row)."""
    def up(key, v):
        worst[f"{tag}:{key}"] = max(worst.get(f"{tag}:{key}", 0.0), v)
    up("p_norm", abs(a["p_norm"] - b["p_norm"]) / b["p_norm"])
    up("p_sum_abs", abs(a["p_sum"] - b["p_sum"]))
    hb = torch.as_tensor(b["p_head"], dtype=torch.float64)
    up("p_head", ((a["p_head"] - hb).abs().max() / hb.abs().max()).item())
    up("m_norm", abs(a["m_norm"] - b["m_norm"]) / b["m_norm"])
    up("v_sum", abs(a["v_sum"] - b["v_sum"]) / b["v_sum"])
    for x, y in zip(a["blocks"], b["blocks"]):
        assert x["k"] == y["k"]
        for side in ("L", "R"):
            up("scale", abs(x[f"{side}_scale"] - y[f"{side}_scale"]) / y[f"{side}_scale"])
        sh = torch.as_tensor(y["S_l_head"], dtype=torch.float64)
        up("S_l_head", ((x["S_l_head"] - sh).abs() / sh.abs()).max().item())


def test_c1_reference_run_100_steps():
    """The reference's own C1 run, all 100 steps (Phase 1 to step 20, blend to
    step 70, steady Phase 2 to 100; refresh every 10 steps), on the GPU.

    The oracle runs the same steps beside it.  At every refresh the GPU's new
    EMA codes are checked against the oracle's (1 LSB, scales 1e-6) and then
    replaced by them, so each step starts from the same EMA as the
    reference's run.  Against the oracle, every step's quantities (parameter
    norm, sum and first values, exp_avg norm, exp_avg_sq sum, per-block
    scales, ranks and leading eigenvalues) and the whole parameter trajectory,
    element by element, must agree tightly.  Against the summary the
    reference itself wrote (tests/golden/c1_summary.*, on the build
    container's CPU) the same quantities must agree to the variation the
    reference shows between two CPUs: the oracle on this machine is compared
    with the summary the same way and reported beside it (its GEMMs round
    differently, a few int8 codes flip, and the leading eigenvalues move by
    a few 1e-5)."""
    import scao_amd
    from scao_amd import engine
    dev = _dev()
    t_gold, meta = load_golden("c1_summary")
    cfg = dict(meta["config"])
    rows = meta["rows"]
    g0 = torch.Generator().manual_seed(0)
    w = torch.randn(768, 3072, generator=g0) * 0.02
    rp = torch.nn.Parameter(w.clone())
    gp = torch.nn.Parameter(w.clone().to(dev))
    ref = R.RefSCAO([rp], **cfg)
    gopt = scao_amd.SCAO([gp], **cfg)
    worst = {"traj_ratio": 0.0, "step_ratio": 0.0}
    prev_ref, prev_gpu = w.clone(), w.clone()
    for t in range(1, 101):
        gg = torch.Generator().manual_seed(1000 + t)
        gr = torch.randn(768, 3072, generator=gg) * 0.02
        rp.grad = gr.clone()
        gp.grad = gr.to(dev)
        ref.step()
        pairs = {}
        pa = ref.state[rp]["preconditioner"]
        if gp in gopt.state:
            for (la, *_), (lb, *_) in zip(P.kron_leaves(pa), gopt.state[gp]["preconditioner"].leaves()):
                pairs[id(lb)] = la
        engine.AFTER_EMA_HOOK = P.IdenticalPostEma(pairs)
        try:
            gopt.step()
        finally:
            engine.AFTER_EMA_HOOK = None
        torch.cuda.synchronize()
        row = rows[t - 1]
        assert row["t"] == t
        st = gopt.state[gp]
        pre = st["preconditioner"]
        assert pre.precond_step == row["precond_step"] and pre.k == row["k"], (t,)
        qg = _c1_quantities(gp, st, pre)
        qo = _c1_quantities(rp, ref.state[rp], pa)
        _c1_diff(qg, qo, worst, "gpu_vs_oracle")
        _c1_diff(qg, row, worst, "gpu_vs_reference_summary")
        _c1_diff(qo, row, worst, "oracle_vs_reference_summary")
        pg = gp.detach().cpu()
        worst["traj_ratio"] = max(worst["traj_ratio"], P.assert_close(
            pg - w, rp.detach() - w, 1e-4, 1e-5, f"C1 step {t} cumulative update"))
        worst["step_ratio"] = max(worst["step_ratio"], P.ratio(
            pg - prev_gpu, rp.detach() - prev_ref, P.UPDATE_RTOL, P.UPDATE_ATOL,
            extra=P.ulp(rp.detach())))
        prev_ref, prev_gpu = rp.detach().clone(), pg
        if t % cfg["precond_freq"] == 0:
            # attribute eigenvalue differences: each side against float64
            # eigenvalues of the identical eigh input
            for (la, *_), (lb, *_) in zip(P.kron_leaves(pa), pre.leaves()):
                for X, Sa, Sb in zip(P.eig_input(la), (la.S_l, la.S_r), (lb.S_l, lb.S_r)):
                    ev = torch.linalg.eigvalsh(X).flip(0)[:Sa.numel()]
                    for key, S in (("eig_cpu_vs_f64", Sa), ("eig_gpu_vs_f64", Sb.cpu())):
                        e = ((S.double() - ev).abs() / ev.abs()).max().item()
                        worst[key] = max(worst.get(key, 0.0), e)
            print(f"C1 t={t}: " + ", ".join(f"{k}={v:.2e}" for k, v in worst.items()), flush=True)
    final = t_gold["p_final_rows"].double()
    pg = gp.detach().cpu().double()
    worst["gpu_vs_reference_summary:p_final_rows"] = (
        (pg[:2] - final).abs().max() / final.abs().max()).item()   # rows 0 and 1
    report("c1_reference_run", "100 steps", worst)
    # against the oracle beside it
    for key, bar in (("p_norm", 1e-7), ("p_head", 1e-5), ("m_norm", 1e-5), ("v_sum", 1e-5),
                     ("scale", 1e-6), ("S_l_head", 1e-5)):
        assert worst[f"gpu_vs_oracle:{key}"] < bar, (key, worst)
    assert worst["step_ratio"] <= 1.0, worst
    # against the reference's own summary: within the reference's own
    # machine-to-machine variation (the oracle's here), or the oracle bar
    for key, bar in (("p_norm", 1e-7), ("p_head", 1e-5), ("m_norm", 1e-5), ("v_sum", 1e-5),
                     ("scale", 1e-6), ("S_l_head", 1e-5)):
        allowed = max(bar, 2.0 * worst[f"oracle_vs_reference_summary:{key}"])
        assert worst[f"gpu_vs_reference_summary:{key}"] < allowed, (key, worst)
    assert worst["gpu_vs_reference_summary:p_final_rows"] < 1e-5, worst
