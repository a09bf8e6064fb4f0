"""Host logic that needs no GPU: preconditioner construction and state layout
against the oracle, constructor validation, the no-CPU-path guard, task
and slot bookkeeping of the batched engine, and a planted-mistake check that
the golden fixtures would catch an oracle slip."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import scao_amd
from oracle import scao_ref as R
from scao_amd import SparsePreconditioner
from scao_amd import _lib as L
from scao_amd import engine as E

SHAPES = [(64, 64), (128, 16), (16, 128), (300, 64), (64, 300), (5000, 4100), (4, 3, 2, 2),
          (20,), (1, 50), (50, 1), (2049, 700), (3, 3)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("int8", [False, True])
def test_precond_construction_matches_oracle(shape, int8):
    kw = dict(k_min=8, k_max=128, max_precond_dim=64 if max(shape) < 1000 else 4096,
              use_int8_ema=int8)
    p = torch.zeros(shape)
    a, b = R.RefPreconditioner(p, **kw), SparsePreconditioner(p, **kw)
    _same_tree(a, b)


def _same_tree(a, b):
    for attr in ("m", "n", "k_min", "k_max", "use_block_diagonal", "use_kronecker",
                 "precond_step", "_k", "use_int8_ema"):
        assert getattr(a, attr) == getattr(b, attr), attr
    if a.use_block_diagonal:
        assert a._block_sizes == b._block_sizes and a._block_dim == b._block_dim
        for x, y in zip(a._blocks, b._blocks):
            _same_tree(x, y)
    elif a.use_kronecker:
        for t in ("U_l", "S_l", "U_r", "S_r"):
            assert torch.equal(getattr(a, t), getattr(b, t)), t
        if a.use_int8_ema:
            assert torch.equal(a.L_ema_q, b.L_ema_q) and torch.equal(a.R_ema_q, b.R_ema_q)
            assert a.L_ema_scale == b.L_ema_scale and a.R_ema_scale == b.R_ema_scale
        else:
            assert torch.equal(a.L_ema, b.L_ema) and torch.equal(a.R_ema, b.R_ema)
    else:
        assert torch.equal(a.diag_ema, b.diag_ema)
        assert a._diag_bias_factor == b._diag_bias_factor
    assert a.memory_bytes() == b.memory_bytes()
    sa, sb = a.state_dict(), b.state_dict()
    assert _skeleton(sa) == _skeleton(sb)


def _skeleton(d):
    return {k: ([_skeleton(x) for x in v] if k == "blocks" else
                (tuple(v.shape), str(v.dtype)) if isinstance(v, torch.Tensor) else v)
            for k, v in d.items()}


def test_leaves_tile_the_parameter():
    """Block-diagonal leaves cover the 2-D view exactly once (recursive split)."""
    for shape, D in [((5000, 4100), 4096), ((2048, 8192), 2048), ((128256, 2048), 2048),
                     ((11008, 2048), 2048), ((300, 64), 64)]:
        pre = SparsePreconditioner(torch.zeros(shape), max_precond_dim=D)
        cover = np.zeros(shape, dtype=np.int32)
        for leaf, r0, c0 in pre.leaves():
            assert leaf.use_kronecker and max(leaf.m, leaf.n) <= D
            cover[r0:r0 + leaf.m, c0:c0 + leaf.n] += 1
        assert (cover == 1).all(), shape


@pytest.mark.parametrize("shape,D", [((65, 40), 32), ((40, 65), 32), ((4097, 300), 2048),
                                     ((300, 2049), 2048), ((65, 65), 32)])
def test_step_leaves_cover_remainders_of_one(shape, D):
    """A 1-wide remainder of a block-diagonal split is a diagonal sub-block
    (reference preconditioner.py:142-153); with diag=True the leaves,
    Kronecker and diagonal, cover the 2-D view exactly once, and their modes
    match the oracle's blocks."""
    pre = SparsePreconditioner(torch.zeros(shape), max_precond_dim=D, use_int8_ema=True)
    ref = R.RefPreconditioner(torch.zeros(shape), max_precond_dim=D, use_int8_ema=True)
    cover = np.zeros(shape, dtype=np.int32)
    ndiag = 0
    for leaf, r0, c0 in pre.leaves(diag=True):
        if not leaf.use_kronecker:
            ndiag += 1
            assert min(leaf.m, leaf.n) == 1 and tuple(leaf.diag_ema.shape) == (leaf.m, leaf.n)
        cover[r0:r0 + leaf.m, c0:c0 + leaf.n] += 1
    assert (cover == 1).all(), shape
    assert ndiag >= 1
    assert pre.step_leaf_list() == list(pre.leaves(diag=True))
    _same_tree(ref, pre)


def test_diag_subblock_tasks():
    """A parameter with a diagonal sub-block: the sub-block takes no projection
    or lift task, its norm partials come from delta tasks with slots of their
    own, and masked apply tasks cover it once."""
    from scao_amd.engine import PItem
    p = torch.zeros(65, 40)
    pre = SparsePreconditioner(p, k_min=4, k_max=8, max_precond_dim=32, use_int8_ema=True)
    it = PItem(p=p, graw=p, gmom=None, st={}, group={}, pre=pre, phase2=True, step=3,
               lars=True, leaves=pre.step_leaf_list())
    arrays, ranges, nslots, leaves = E._build_structure([it])
    dl = [i for i, (lf, *_) in enumerate(leaves) if not lf.use_kronecker]
    assert len(dl) == 1
    d = dl[0]
    for kind in [f"proj{v}" for v in range(12)] + ["lift"]:
        assert not any(int(t["idx"]) == d for t in arrays[kind]), kind
    dtasks = [t for t in arrays["delta"] if int(t["idx"]) == d]
    assert len(dtasks) == 1 and dtasks[0]["slot"] >= 0
    assert ranges[0][0] <= dtasks[0]["slot"] < ranges[0][1]
    cover = np.zeros((1, 40), np.int32)
    for var in range(16):
        for t in arrays[f"apply{var}"]:
            if int(t["idx"]) == d:
                assert not var & 4
                cover[t["a"]:t["a"] + 64, t["b"]:t["b"] + 64] += 1
    assert (cover == 1).all()
    writes = np.zeros(nslots, int)
    for a in arrays.values():
        for t in a:
            if t["slot"] >= 0:
                writes[t["slot"]] += 1
    assert (writes == 1).all()
    tab = E._leaf_table(leaves, [it], E.Workspace(torch.device("cpu")))
    assert tab[d]["flags"] == L.LF_DIAG and tab[d]["k"] == 0
    assert tab[d]["Sl"] == leaves[d][0].diag_ema.data_ptr()
    assert tab[d]["off"] == 64 * 40 and tab[d]["ld"] == 40


def test_precond_k_setter_matches_oracle():
    p = torch.zeros(96, 80)
    a = R.RefPreconditioner(p, k_min=4, k_max=32, max_precond_dim=64)
    b = SparsePreconditioner(p, k_min=4, k_max=32, max_precond_dim=64)
    for k in (2, 40, 6, 3, 100):
        a.k, b.k = k, k
        _same_tree(a, b)


def test_constructor_validation_and_defaults():
    m = torch.nn.Linear(8, 4)
    with pytest.raises(ValueError):
        scao_amd.SCAO(m.parameters(), lr=-1e-3)
    with pytest.raises(ValueError):
        scao_amd.SCAO(m.parameters(), betas=(1.0, 0.999))
    with pytest.raises(ValueError):
        scao_amd.SCAO(m.parameters(), betas=(0.9, 1.0))
    with pytest.raises(ValueError):
        scao_amd.SCAO(m.parameters(), beta3=1.0)
    a = scao_amd.SCAO(m.parameters())
    b = R.RefSCAO(torch.nn.Linear(8, 4).parameters())
    assert a.defaults == b.defaults
    assert len(a.defaults) == 18
    assert a._callbacks == []


def test_step_on_cpu_raises():
    m = torch.nn.Linear(8, 4)
    opt = scao_amd.SCAO(m.parameters(), warmup_steps=0)
    m(torch.randn(2, 8)).sum().backward()
    with pytest.raises(RuntimeError, match="ROCm"):
        opt.step()


def test_load_state_dict_keeps_fp32_moments_for_bf16():
    """torch's Optimizer.load_state_dict casts state to the parameter dtype, so
    the reference (and the oracle, which inherits the same base) comes back
    from a checkpoint with bf16 moments.  This build restores them as
    bit-identical fp32 copies of the checkpoint's tensors."""
    g = torch.Generator().manual_seed(5)
    shapes = [(12, 20), (20,)]
    rp = [torch.nn.Parameter(torch.randn(s, generator=g).bfloat16()) for s in shapes]
    cfg = dict(lr=1e-2, warmup_steps=10, sparsity=0.0, noise_std_init=0.0,
               async_precond=False, lookahead_k=0)
    ref = R.RefSCAO(rp, **cfg)
    for _ in range(2):
        for p in rp:
            p.grad = torch.randn(p.shape, generator=g).bfloat16()
        ref.step()
    sd = ref.state_dict()
    assert sd["state"][0]["exp_avg"].dtype == torch.float32
    mp = [torch.nn.Parameter(p.detach().clone()) for p in rp]
    opt = scao_amd.SCAO(mp, **cfg)
    opt.load_state_dict(sd)
    for i, p in enumerate(mp):
        for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
            got = opt.state[p][key]
            assert got.dtype == torch.float32 and got.is_contiguous()
            assert torch.equal(got, sd["state"][i][key])
            assert got.data_ptr() != sd["state"][i][key].data_ptr()
    # what the inherited base does (the reference's behaviour after a resume)
    again = R.RefSCAO([torch.nn.Parameter(p.detach().clone()) for p in rp], **cfg)
    again.load_state_dict(sd)
    assert next(iter(again.state.values()))["exp_avg"].dtype == torch.bfloat16


def test_presets_construct():
    m = torch.nn.Linear(16, 8)
    for f in (scao_amd.scao_sub1b, scao_amd.scao_1b, scao_amd.scao_3b, scao_amd.scao_7b,
              scao_amd.scao_40b, scao_amd.scao_125b):
        opt = f(m)
        assert isinstance(opt, scao_amd.SCAO)
    assert scao_amd.scao_1b(m).defaults["k_max"] == 48
    assert scao_amd.scao_125b(m)._adaptive_rank


def test_engine_slots_cover_each_once():
    from scao_amd.engine import PItem
    items = []
    for i, shp in enumerate([(2048, 8192), (512, 2048), (2048,), (100, 37), (130, 70)]):
        p = torch.zeros(shp)
        pre = SparsePreconditioner(p, k_min=16, k_max=80, max_precond_dim=2048,
                                   use_int8_ema=True)
        diag = not (pre.use_block_diagonal or pre.use_kronecker)
        items.append(PItem(p=p, graw=p, gmom=None, st={}, group={}, pre=pre, phase2=i != 3,
                           step=3, lars=i % 2 == 0, diag=diag,
                           leaves=[] if diag else list(pre.leaves())))
    arrays, ranges, nslots, leaves = E._build_structure(items)
    writes = np.zeros(nslots, int)
    for a in arrays.values():
        for t in a:
            if t["slot"] >= 0:
                writes[t["slot"]] += 1
    assert (writes == 1).all()
    prev_end = 0
    for (pb, pe, qb, qe) in ranges:
        assert pb == prev_end and pb <= pe == qb <= qe
        prev_end = qe
    assert prev_end == nslots
    # every Phase-2 LARS param gets write-back tasks covering its numel
    for i, it in enumerate(items):
        n = sum(1 for t in arrays["lars"] if t["idx"] == i)
        assert n == (E._flat_chunks(it.p.numel()) if it.phase2 and it.lars else 0)


def test_param_table_fields_and_state_checks():
    """Per-step descriptors: group scalars at known steps, per-parameter
    pointers and flags, and the moment checks (again after a tensor is
    replaced)."""
    from scao_amd.engine import PItem
    g = {"lr": 0.1, "betas": (0.9, 0.999), "beta3": 0.99, "weight_decay": 0.01, "eps": 1e-8,
         "tau": 1.0, "lars_coeff": 1e-3, "blend_steps": 50}
    ws = E.Workspace(torch.device("cpu"))
    items = []
    for i, (shape, phase2) in enumerate([((8, 12), True), ((16,), False), ((4, 3, 5), True)]):
        p = torch.zeros(shape)
        st = {k: torch.zeros(shape) for k in E._MOMENTS}
        items.append(PItem(p=p, graw=torch.zeros(shape), gmom=None, st=st, group=g, pre=None,
                           phase2=phase2, step=1 if not phase2 else 30, scao_step=25,
                           lars=True))
    for it in items:
        it.ptrs = E._item_ptrs(it)
    ws.upd_offsets, ws.upd_total = {0: 0, 2: 96}, 156
    ranges = [(0, 1, 1, 2), (2, 2, 2, 2), (2, 3, 3, 4)]
    raw, classes = E._param_table(items, ranges, ws, None)
    tab = raw.view(L.PARAM_DESC).reshape(len(items))
    f4 = np.float32
    assert tab["bc1"][0] == f4(1 - 0.9 ** 30) and tab["bc1"][1] == 0.0
    assert tab["blend"][0] == f4(0.5) and tab["omblend"][2] == f4(0.5)
    assert tab["decay"][1] == f4(1 - 0.1 * 0.01)
    assert tab["adam_alpha"][1] == f4(-0.1 / (1 - 0.9)) and tab["adam_sqrt_bc2"][0] == 0.0
    assert list(tab["cols"]) == [12, 16, 15] and list(tab["numel"]) == [96, 16, 60]
    for i in (0, 2):
        assert tab["flags"][i] & L.PF_LARS and tab["flags"][i] & L.PF_CLIP
    assert not tab["flags"][1] & (L.PF_LARS | L.PF_CLIP)
    upd = ws.buf("upd", 4).data_ptr()
    assert list(tab["upd"]) == [upd, 0, upd + 4 * 96]
    assert tab["exp_avg_sq"][2] == items[2].st["exp_avg_sq"].data_ptr()
    assert [tuple(r) for r in tab[["pre_begin", "pre_end", "post_begin", "post_end"]]] == ranges
    assert list(tab["norm_index"]) == [0, 1, 2]
    items[1].st["exp_avg"] = torch.zeros(16, dtype=torch.bfloat16)   # replaced after a check
    with pytest.raises(ValueError, match="contiguous float32"):
        E._param_table(items, ranges, ws, None)
    items[1].st["exp_avg"] = torch.zeros(32)[::2]
    with pytest.raises(ValueError, match="contiguous float32"):
        E._param_table(items, ranges, ws, None)


def test_planned_step_table_matches_a_fresh_build():
    """A planned step (engine.run_planned_step) rewrites only the gradient
    addresses and each class's step scalars of the last table: after one
    step of every counter its table is byte for byte what _param_table
    builds from scratch at the next step (bias corrections, blend, Adam
    alpha, flags), for Phase-1 and Phase-2 rows of two groups, a
    diagonal-mode row's bias factor included."""
    from scao_amd.engine import PItem
    g1 = {"lr": 0.1, "betas": (0.9, 0.999), "beta3": 0.99, "weight_decay": 0.01, "eps": 1e-8,
          "tau": 1.0, "lars_coeff": 1e-3, "blend_steps": 50}
    g2 = dict(g1, lr=0.05, tau=None, lars_coeff=0.0, weight_decay=0.0, blend_steps=0)
    ws = E.Workspace(torch.device("cpu"))

    class Pre:
        diag_ema = torch.zeros(16)
        _diag_bias_factor = 0.25

    def build(step_shift, grads):
        items = []
        spec = [((8, 12), True, g1, False), ((16,), False, g1, False), ((4, 3, 5), True, g2, False),
                ((16,), True, g1, True)]
        for i, (shape, phase2, g, diag) in enumerate(spec):
            it = PItem(p=params[i], graw=grads[i], gmom=None, st=states[i], group=g,
                       pre=Pre() if diag else None, phase2=phase2,
                       step=(30 if phase2 else 3) + step_shift, scao_step=25 + step_shift,
                       lars=phase2 and g["lars_coeff"] > 0, diag=diag)
            it.ptrs = E._item_ptrs(it)
            items.append(it)
        return items

    shapes = [(8, 12), (16,), (4, 3, 5), (16,)]
    params = [torch.zeros(s) for s in shapes]
    states = [{k: torch.zeros(s) for k in E._MOMENTS} for s in shapes]
    ws.upd_offsets, ws.upd_total = {0: 0, 3: 96}, 112
    ranges = [(0, 1, 1, 2), (2, 2, 2, 2), (2, 3, 3, 4), (4, 5, 5, 6)]
    grads0 = [torch.zeros(s) for s in shapes]
    grads1 = [torch.zeros(s) for s in shapes]
    raw, classes = E._param_table(build(0, grads0), ranges, ws, 0.5)
    assert len(classes) == 3
    gptrs = np.array([g.data_ptr() for g in grads1], dtype=np.uint64)
    a, b, _ = E._BLOCKS["u8"]
    raw[:, a:b].view(np.uint64)[:, 1] = gptrs
    raw[:, a:b].view(np.uint64)[:, 2] = gptrs
    for cl in classes:
        cl.step += 1
        cl.scao_step += cl.phase2
        E._set_class_scalars(raw, cl, 0.5)
    fresh, _ = E._param_table(build(1, grads1), ranges, ws, 0.5)
    assert raw.tobytes() == fresh.tobytes()


def test_structure_cache_matches_fresh_builds():
    """Per-parameter shares cached across steps give the same task lists,
    slots and ranges as a fresh build, also when the set of parameters
    changes from step to step; the interleave keeps every task once."""
    from scao_amd.engine import PItem
    items = []
    for i, shp in enumerate([(512, 512), (256, 1024), (320, 448), (512,), (1024, 256),
                             (100, 37)]):
        p = torch.zeros(shp)
        pre = SparsePreconditioner(p, k_min=128 if i % 2 else 64, k_max=128 if i % 2 else 64,
                                   max_precond_dim=512, use_int8_ema=True)
        diag = not (pre.use_block_diagonal or pre.use_kronecker)
        items.append(PItem(p=p, graw=p, gmom=None, st={}, group={}, pre=pre, phase2=i != 4,
                           step=3, lars=i % 3 != 0, diag=diag,
                           leaves=[] if diag else list(pre.leaves())))
    cache = {}

    def same(a, b):
        assert set(a[0]) == set(b[0])
        for k in a[0]:
            assert a[0][k].tobytes() == b[0][k].tobytes(), k
        assert a[1:3] == b[1:3]
        assert [(id(x[0]),) + x[1:] for x in a[3]] == [(id(x[0]),) + x[1:] for x in b[3]]

    for sub in (items, items[1:], items[::2], items):
        same(E._build_structure(sub), E._build_structure(sub, cache))
        fresh = E._build_structure(sub)
        for k, arr in fresh[0].items():
            rows = sorted(map(tuple, arr.view(np.int32).reshape(-1, 4).tolist()))
            assert len(rows) == len(set(rows)), k
    assert cache


def _phase2_items(shapes, k):
    from scao_amd.engine import PItem
    items = []
    for shp in shapes:
        p = torch.zeros(shp)
        pre = SparsePreconditioner(p, k_min=k, k_max=k, max_precond_dim=2048)
        items.append(PItem(p=p, graw=p, gmom=None, st={}, group={}, pre=pre, phase2=True,
                           step=3, lars=True, leaves=list(pre.leaves())))
    return items


@pytest.mark.parametrize("k", [128, 256])
def test_strip_apply_tasks(k):
    """Blocks of rank 128 / 256 go to the strip kernel (variant bits 16, and
    32 for k = 128): each task a run of at most APPLY_GROUP tiles of TR rows
    down one SW-column strip; the runs tile every block interior once, their
    slot ranges are disjoint, and a block's runs stay on one die's queue
    (workgroup b takes queue b % XCDS)."""
    items = _phase2_items([(1024, 2048)] * 8 + [(640, 1536)], k)
    arrays, _, nslot, leaves = E._build_structure(items)
    sw, tr = (64, 128) if k == 256 else (128, 64)
    var = 2 | 4 | 16 | (32 if k == 128 else 0)
    runs = arrays[f"apply{var}"]
    assert all(len(arrays[f"apply{v}"]) == 0 for v in (14, 6) if v != var)
    cover = {}
    spans = []
    for t in runs:
        lf = leaves[int(t["idx"])][0]
        mw, nw = lf.m - lf.m % tr, lf.n - lf.n % sw
        a, b = int(t["a"]), int(t["b"])
        nt = min(L.APPLY_GROUP, (mw - a) // tr)
        assert nt >= 1 and a % tr == 0 and b % sw == 0 and b + sw <= nw
        for i in range(nt):
            key = (int(t["idx"]), a + i * tr, b)
            assert key not in cover
            cover[key] = 1
        spans.append((int(t["slot"]), nt))
    assert len(cover) == sum((lf.m // tr) * (lf.n // sw) for lf, *_ in leaves)
    spans.sort()
    for (s0, n0), (s1, _) in zip(spans, spans[1:]):
        assert s1 >= s0 + n0
    assert spans[-1][0] + spans[-1][1] <= nslot
    queue_of = {}
    for b, t in enumerate(runs[:E.XCDS * 16]):
        queue_of.setdefault(int(t["idx"]), b % E.XCDS)
        assert queue_of[int(t["idx"])] == b % E.XCDS


def test_pipelined_apply_tasks():
    """Wide tasks of blocks with another step width >= PIPE_MIN_RANK (here
    320) carry variant bit 8 and are ordered in runs of APPLY_GROUP tasks of
    one die's queue."""
    items = _phase2_items([(1024, 2048)] * 8 + [(512, 1536)], 320)
    arrays, _, _, leaves = E._build_structure(items)
    pipe = arrays["apply14"]
    assert len(pipe) == sum(lf.m // 16 * (lf.n // 256) for lf, *_ in leaves)
    assert len(arrays["apply6"]) == 0
    runs = [pipe[i:i + L.APPLY_GROUP] for i in range(0, len(pipe), L.APPLY_GROUP)]
    # eight equal blocks, one per die queue: workgroup b takes its run from
    # queue b % XCDS, and a block's tiles never change queue
    queue_of = {}
    for b, run in enumerate(runs[:E.XCDS * 32]):
        for t in run:
            queue_of.setdefault(int(t["idx"]), b % E.XCDS)
            assert queue_of[int(t["idx"])] == b % E.XCDS


@pytest.mark.parametrize("m,n,k,pipelined", [(4096, 4096, 256, True), (1024, 4096, 256, True),
                                             (2048, 2048, 128, False), (2048, 2048, 128, True),
                                             (2048, 2048, 64, False), (4096, 2048, 256, True)])
def test_wide_tile_order(m, n, k, pipelined):
    """Every wide tile once; leaves whose W and U_r exceed L2_OPERANDS, and
    every leaf of the pipelined kernel, go in super-tiles whose operands fit
    it, each run of APPLY_GROUP tiles inside one column strip (so the
    pipelined kernel can pair them); other leaves keep row-major order."""
    rows, cols = L.APPLY_WIDE_ROWS, L.APPLY_WIDE_COLS
    order = E._wide_tiles(m, n, k, pipelined)
    assert sorted(order) == [(i, j) for i in range(0, m, rows) for j in range(0, n, cols)]
    if (m + n) * k * 4 <= E.L2_OPERANDS and not pipelined:
        assert order == [(i, j) for i in range(0, m, rows) for j in range(0, n, cols)]
        return
    for b in range(0, len(order), L.APPLY_GROUP):
        assert len({j for _, j in order[b:b + L.APPLY_GROUP]}) == 1
    # a window of tiles the size of one super-tile touches at most
    # L2_OPERANDS of W rows and U_r rows
    half = E.L2_OPERANDS // 2
    s = max(1, half // (cols * k * 4))
    r = max(L.APPLY_GROUP, half // (rows * k * 4) // L.APPLY_GROUP * L.APPLY_GROUP)
    for b in range(0, len(order), r * s):
        win = order[b:b + r * s]
        strips = {j for _, j in win}
        bands = {i for i, _ in win}
        assert len(strips) * cols * k * 4 + len(bands) * rows * k * 4 <= E.L2_OPERANDS


@pytest.mark.parametrize("shape,fp32", [((2048, 8192), True), ((328, 264), True),
                                        ((320, 448), True), ((100, 37), True),
                                        ((300, 520), True), ((512, 512), False)])
def test_apply_tasks_tile_each_block_once(shape, fp32):
    """Wide 16x256 tasks (variant bit 4) over the exactly tiled interior and
    masked 64x64 tasks over the strips cover every element of every block
    once; wide tasks lie wholly inside their block."""
    from scao_amd.engine import PItem
    p = torch.zeros(shape)
    pre = SparsePreconditioner(p, k_min=16, k_max=64, max_precond_dim=2048, use_int8_ema=True)
    it = PItem(p=p, graw=p, gmom=None, st={}, group={}, pre=pre, phase2=True, step=3,
               lars=True, leaves=list(pre.leaves()), fp32=fp32)
    arrays, _, _, leaves = E._build_structure([it])
    seen_wide = False
    for li, (leaf, r0, c0, _) in enumerate(leaves):
        cover = np.zeros((leaf.m, leaf.n), np.int32)
        for var in range(16):
            for t in arrays[f"apply{var}"]:
                if t["idx"] != li:
                    continue
                i0, j0 = int(t["a"]), int(t["b"])
                if var & 4:
                    seen_wide = True
                    assert fp32
                    assert i0 + L.APPLY_WIDE_ROWS <= leaf.m and j0 + L.APPLY_WIDE_COLS <= leaf.n
                    cover[i0:i0 + L.APPLY_WIDE_ROWS, j0:j0 + L.APPLY_WIDE_COLS] += 1
                else:
                    cover[i0:i0 + L.APPLY_TILE, j0:j0 + L.APPLY_TILE] += 1
        assert (cover == 1).all(), (shape, leaf.m, leaf.n)
    assert seen_wide == (fp32 and shape[0] >= 16 and min(shape[1], 2048) >= 256)


def test_golden_catches_planted_oracle_mistake(monkeypatch):
    """Drop the '-1' of the projection correction in the oracle: the golden
    trajectory must then fail."""
    from scao_inputs import config_from_meta, grads_for_step, load_golden
    T, meta = load_golden("traj_int8")

    def wrong(U_l, s_l, U_r, s_r, G):
        P = (U_l.T @ G) @ U_r
        return G + U_l @ ((s_l[:, None] * s_r[None, :]) * P) @ U_r.T

    monkeypatch.setattr(R, "fused_kronecker_precond", wrong)
    names = meta["names"]
    shapes = {k: tuple(meta["shapes"][k]) for k in names}
    params = {k: torch.nn.Parameter(T[f"init.{k}"].clone()) for k in names}
    opt = R.RefSCAO(list(params.values()), **config_from_meta(meta))
    from test_oracle_golden import UPD_TOL, update_err
    worst = 0.0
    for t in range(1, meta["steps"] + 1):
        gr = grads_for_step(t, shapes)
        for k, p in params.items():
            p.grad = gr[k].clone()
        before = {k: p.detach().clone() for k, p in params.items()}
        opt.step()
        for k, p in params.items():
            prev = T[f"step{t - 1}.p.{k}"] if t > 1 else T[f"init.{k}"]
            ref = T[f"step{t}.p.{k}"] - prev
            worst = max(worst, update_err(p.detach() - before[k], ref))
        for k, p in params.items():   # replay from the golden state, as the gate does
            p.data.copy_(T[f"step{t}.p.{k}"])
    assert worst > 10 * UPD_TOL, worst


def test_reference_checkpoint_through_safe_torch_load():
    """A checkpoint file written by the reference's state_dict() (golden
    fixture) loads through scao_amd.checkpoint.load (torch.load with
    weights_only=True; plain weights_only refuses the reference's pickled
    preconditioner class) into scao_amd.SCAO with every tensor, counter and
    the diagonal bias factor intact, and this package's own checkpoints go
    through the same safe loader."""
    import io
    import json
    import os
    from safetensors.torch import load_file
    from scao_amd import checkpoint
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    meta = json.load(open(os.path.join(gdir, "ckpt_resume.json")))
    vals = load_file(os.path.join(gdir, "ckpt_resume.safetensors"))
    path = os.path.join(gdir, "ref_checkpoint.pt")
    with pytest.raises(Exception, match="scao.preconditioner.SparsePreconditioner"):
        torch.load(path, weights_only=True)
    sd = checkpoint.load(path)
    cfg = meta["config"]
    mp = [torch.nn.Parameter(vals[f"ckpt/{k}"].clone()) for k in meta["names"]]
    opt = scao_amd.SCAO(mp, **cfg)
    opt.load_state_dict(sd)
    assert opt._global_step == sd["_scao_runtime"]["global_step"] == 5
    assert opt._global_norm_ema == sd["_scao_runtime"]["global_norm_ema"]
    for i, (p, st) in enumerate(opt.state.items()):
        src = sd["state"][i]
        for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
            assert torch.equal(st[key], src[key])
        assert st["step"] == src["step"] and st["scao_step"] == src["scao_step"]
        pre = st["preconditioner"]
        assert isinstance(pre, SparsePreconditioner)
        assert pre.state_dict().keys() == sd["_scao_precond"][i].keys()
        for k, v in sd["_scao_precond"][i].items():
            if isinstance(v, torch.Tensor):
                assert torch.equal(pre.state_dict()[k], v), (i, k)
        bias = getattr(src["preconditioner"], "_diag_bias_factor", None)
        if bias is not None:
            assert pre._diag_bias_factor == bias
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    again = checkpoint.load(buf)
    assert again["_scao_runtime"] == sd["_scao_runtime"]
    assert isinstance(again["state"][0]["preconditioner"], SparsePreconditioner)


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N > 1 exits with a message, before touching a GPU."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_adaptive_rank_from_top_eigenvalues_matches_full_spectrum():
    """batched_adaptive_rank_topk (top kq values + the clamped total) picks the
    same rank as batched_adaptive_rank on the whole spectrum (and as the
    reference's utils.adaptive_rank restated in the oracle)."""
    from scao_amd.utils import batched_adaptive_rank, batched_adaptive_rank_topk
    g = torch.Generator().manual_seed(4)
    for dim, kq, eps in [(64, 16, 0.05), (64, 64, 0.05), (200, 24, 0.3), (200, 24, 0.001),
                         (32, 8, 0.5)]:
        for trial in range(20):
            lam = torch.rand(dim, generator=g) ** (1 + trial % 5) * (trial + 1)
            if trial % 7 == 0:
                lam[: dim // 2] = 0.0
            S = lam.sort(descending=True).values.clamp(min=0).unsqueeze(0)
            e = torch.tensor([eps], dtype=torch.float64)
            kmin = torch.tensor([min(4, kq)])
            kmax = torch.tensor([kq])
            want = batched_adaptive_rank(S, e, kmin, kmax)
            got = batched_adaptive_rank_topk(S[:, :kq], S.double().sum(dim=1), dim, e, kmin, kmax)
            ref = R.adaptive_rank(S[0], eps, int(kmin), int(kmax))
            assert int(got) == int(want) == ref, (dim, kq, eps, trial, int(got), int(want), ref)


def test_eigen_route_by_size_and_shape():
    """Which solver a refresh gives an n x n factor: the closed form for an
    exactly diagonal input up to 4096 + SCAO_EIG_BAND rows; the HIP solver
    for the sizes whose kernels need no scratch memory (up to 2048 rows, and
    multiples of 16 up to 4096); the library eigh for the rest."""
    from scao_amd import eigen, engine
    lim = engine.DIAG_MAX_DIM
    assert lim == 4096 + 16
    assert engine.eigen_route(2048, True) == "diag"
    assert engine.eigen_route(2048, False) == "hip"
    assert engine.eigen_route(lim, True) == "diag"
    assert engine.eigen_route(lim, False) == "library"
    assert engine.eigen_route(4096, False) == "hip"
    assert engine.eigen_route(4097, False) == "library"
    assert engine.eigen_route(lim + 1, True) == "library"
    assert engine.eigen_route(1, True) == "diag"
    # ragged sizes stay on the HIP solver up to 2048 rows, whole 16-row
    # multiples up to 4096
    for n, fits in ((1, True), (2047, True), (2048, True), (2049, False), (2064, True),
                    (3000, False), (3840, True), (4095, False), (4096, True), (4112, False)):
        assert eigen.solver_fits(n) == fits, n
        assert engine.eigen_route(n, False) == ("hip" if fits else "library"), n
    # a batch of one or two large factors goes to the library (latency floor)
    assert engine.batch_route("hip", 2048, 1) == "library"
    assert engine.batch_route("hip", 4096, 2) == "library"
    assert engine.batch_route("hip", 4096, 3) == "hip"
    assert engine.batch_route("hip", 1024, 1) == "hip"
    assert engine.batch_route("diag", 4096, 1) == "diag"


@pytest.mark.parametrize("k,width", [(1, 64), (8, 64), (50, 64), (64, 64), (65, 128), (127, 128),
                                     (128, 128), (129, 256), (192, 256), (256, 256), (300, 320)])
def test_step_width_pads_ranks(k, width):
    """A block's eigenfactors enter the step at width 64, 128 or 256 (beyond,
    a multiple of 64); a padded block gets zero-padded U copies and S copies
    padded with 1.0, and its projection and apply tasks are the whole-tile
    ones of that width."""
    items = _phase2_items([(512, 768)], k)   # whole 256-column projection tiles
    leaf = items[0].leaves[0][0]
    assert leaf.U_l.shape[1] == k and E._leaf_k(leaf) == width
    g = torch.Generator().manual_seed(k)
    leaf.U_l = torch.randn(leaf.m, k, generator=g)
    leaf.U_r = torch.randn(leaf.n, k, generator=g)
    leaf.S_l, leaf.S_r = torch.rand(k, generator=g), torch.rand(k, generator=g)
    ws = E.Workspace(torch.device("cpu"))
    pads = E._padded_factors([(leaf, 0, 0, 0)], ws)
    if width == k:
        assert pads == {}
    else:
        ul, ur, sl, sr = pads[0]
        assert ul.shape == (leaf.m, width) and ur.shape == (leaf.n, width)
        assert torch.equal(ul[:, :k], leaf.U_l) and not ul[:, k:].any()
        assert torch.equal(ur[:, :k], leaf.U_r) and not ur[:, k:].any()
        assert torch.equal(sl[:k], leaf.S_l) and bool((sl[k:] == 1.0).all())
        assert torch.equal(sr[:k], leaf.S_r) and bool((sr[k:] == 1.0).all())
    arrays, _, _, _ = E._build_structure(items)
    proj = [kind for kind, arr in arrays.items() if kind.startswith("proj") and len(arr)]
    assert proj and all(int(kind[4:]) & 1 for kind in proj)        # whole-tile (bf16) tiles
    wide = sum(len(arr) for kind, arr in arrays.items()
               if kind.startswith("apply") and int(kind[5:]) & 4)
    assert wide > 0
