"""Write the golden fixtures that pin the CPU oracle (oracle/scao_ref.py).

Run in the build container only:  python tests/golden/make_goldens.py
It imports the reference package from /root/reference (read-only), runs it
on the CPU on seeded inputs and stores inputs/outputs as data under
tests/golden/.  Nothing else in the repository imports this script or the
reference; the GPU box never sees either.

Cases (all grads for step t come from torch.Generator().manual_seed(1000+t),
drawn param by param in group order; params from manual_seed(0)):
  traj_int8     -- block-diagonal (row and column splits with remainders),
                   Kronecker, conv-shaped and 1-D params; int8 EMA; adaptive
                   rank; tau=1, LARS on; Phase 1 -> blend -> Phase 2.
  traj_fp32     -- fp32 EMA, tau=None, LARS off, fixed rank.
  traj_misc     -- lookahead, blend_steps=0, strong weight decay, int8.
  traj_bf16     -- bf16 params and grads.
  traj_sparse   -- default sparse filter (quantile mask) on, int8.
  traj_gsnr, traj_lazy, traj_awarmup, traj_dynsparse, traj_arank -- the
                   optional features (gSNR update mask, lazy refresh trigger,
                   adaptive warm-up, dynamic sparsity, adaptive rank), each on
                   the fp32 or int8 small configuration the GPU feature tests
                   use; the warm-up flag is recorded per step.
  diag_int8     -- the reference's refreshes from its initialisation at the
                   large configurations' gradient scale (2048x2048 and
                   512x2048, k=64, N(0,1e-3^2)): exactly diagonal int8 EMAs,
                   unit-vector eigenfactors in LAPACK's tie order.
  ops           -- operator-level vectors (projection, int8 EMA update,
                   low-rank mm, quantise, adaptive rank, natural norm).
  c1_summary    -- the 768x3072 parity config, 100 steps: per-step norms,
                   leading values, int8 code digests, scales and ranks.
  ref_checkpoint.pt + ckpt_resume -- a checkpoint file written by the
                   reference's state_dict() after 5 steps, and the parameters
                   of a fresh reference optimizer resumed from it for 2 steps.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import warnings

import torch
from safetensors.torch import save_file

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))

PARITY = dict(sparsity=0.0, noise_std_init=0.0, async_precond=False, lookahead_k=0)

SMALL_SHAPES = {
    "w_col": (20, 80),      # D=32 -> column blocks 32, 32, 16
    "w_row": (70, 12),      # D=32 -> row blocks 32, 32, 6
    "w_kron": (12, 20),     # Kronecker
    "w_conv": (4, 3, 2, 2),  # to_2d -> (4, 12), Kronecker
    "b": (20,),             # diagonal
}


def make_params(shapes, dtype=torch.float32, scale=0.02):
    g = torch.Generator().manual_seed(0)
    return {k: torch.nn.Parameter((torch.randn(s, generator=g) * scale).to(dtype))
            for k, s in shapes.items()}


def grads_for_step(t, params, scale=0.02, outliers=0.0):
    g = torch.Generator().manual_seed(1000 + t)
    out = {}
    for k, p in params.items():
        x = torch.randn(p.shape, generator=g) * scale
        if outliers > 0:
            mask = torch.rand(p.shape, generator=g) < outliers
            x = torch.where(mask, x * 50.0, x)
        out[k] = x.to(p.dtype)
    return out


def flatten_precond(prefix, d, tensors, meta):
    for key, val in d.items():
        name = f"{prefix}.{key}"
        if key == "blocks":
            meta[name] = len(val)
            for i, b in enumerate(val):
                flatten_precond(f"{name}.{i}", b, tensors, meta)
        elif isinstance(val, torch.Tensor):
            tensors[name] = val.detach().clone().contiguous()
        else:
            meta[name] = val


def run_traj(scao, name, cfg, steps, snap_steps, dtype=torch.float32, outliers=0.0):
    params = make_params(SMALL_SHAPES, dtype)
    opt = scao.SCAO(list(params.values()), **cfg)
    tensors, meta = {}, {"config": {k: (list(v) if isinstance(v, tuple) else v)
                                    for k, v in cfg.items()},
                         "steps": steps, "dtype": str(dtype), "names": list(params),
                         "shapes": {k: list(v) for k, v in SMALL_SHAPES.items()},
                         "outliers": outliers}
    for k, p in params.items():
        tensors[f"init.{k}"] = p.detach().clone()
    per_step = []
    for t in range(1, steps + 1):
        gr = grads_for_step(t, params, outliers=outliers)
        for k, p in params.items():
            p.grad = gr[k].clone()
        opt.step()
        rec = {"global_step": opt._global_step, "global_norm_ema": opt._global_norm_ema,
               "ranks": {str(i): k for i, k in opt.current_ranks().items()},
               "in_warmup": bool(opt._in_warmup_global)}
        for i, (k, p) in enumerate(params.items()):
            st = opt.state[p]
            tensors[f"step{t}.p.{k}"] = p.detach().clone()
            rec[k] = {"step": st["step"], "scao_step": st["scao_step"],
                      "phase2": bool(st.get("scao_phase_started", False)),
                      "precond_step": st["preconditioner"].precond_step}
        per_step.append(rec)
        if t in snap_steps:
            sd = opt.state_dict()
            for i, (k, p) in enumerate(params.items()):
                st = opt.state[p]
                for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
                    tensors[f"snap{t}.{k}.{key}"] = st[key].detach().clone()
            for idx, d in sd["_scao_precond"].items():
                flatten_precond(f"snap{t}.precond{idx}", d, tensors, meta)
            meta[f"snap{t}.runtime"] = sd["_scao_runtime"]
            meta[f"snap{t}.state_keys"] = {str(i): sorted(v.keys()) for i, v in sd["state"].items()}
            meta[f"snap{t}.group_keys"] = sorted(k for k in sd["param_groups"][0] if k != "params")
    meta["per_step"] = per_step
    meta["snap_steps"] = list(snap_steps)
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"))
    with open(os.path.join(HERE, f"{name}.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True, default=str)
    print(f"{name}: {len(tensors)} tensors")


def run_ops(scao):
    from scao import utils as U
    from scao.cuda import _fused_kronecker_precond_pytorch, _low_rank_precond_mm_pytorch, \
        _int8_ema_update_pytorch
    from scao.preconditioner import SparsePreconditioner
    g = torch.Generator().manual_seed(7)
    T, M = {}, {}
    for i, (m, n, k) in enumerate([(48, 64, 8), (33, 70, 5), (64, 40, 16)]):
        G = torch.randn(m, n, generator=g)
        Ul, _ = torch.linalg.qr(torch.randn(m, k, generator=g))
        Ur, _ = torch.linalg.qr(torch.randn(n, k, generator=g))
        sl = torch.rand(k, generator=g) + 0.2
        sr = torch.rand(k, generator=g) + 0.2
        T.update({f"fkp{i}.G": G, f"fkp{i}.Ul": Ul.contiguous(), f"fkp{i}.Ur": Ur.contiguous(),
                  f"fkp{i}.sl": sl, f"fkp{i}.sr": sr,
                  f"fkp{i}.out": _fused_kronecker_precond_pytorch(Ul, sl, Ur, sr, G)})
        T[f"lrmm{i}.left"] = _low_rank_precond_mm_pytorch(Ul, sl, G, True)
        T[f"lrmm{i}.right"] = _low_rank_precond_mm_pytorch(Ur, sr, G, False)
    for i, (nel, sc) in enumerate([(4096, 1e-3), (1000, 3.0), (257, 1e-20)]):
        x = torch.randn(nel, generator=g) * sc
        q, s = U.quantize_sym_int8(x)
        T[f"quant{i}.x"], T[f"quant{i}.q"] = x, q
        M[f"quant{i}.scale"] = s
        T[f"quant{i}.deq"] = U.dequantize_sym_int8(q, s)
        nv = torch.randn(nel, generator=g) * sc * 0.1
        q2, s2 = _int8_ema_update_pytorch(q.clone(), s, nv, 0.99)
        T[f"ema{i}.new"], T[f"ema{i}.q"] = nv, q2
        M[f"ema{i}.scale"] = s2
    x = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -126.5, 127.0]) * (1.0 / 127.0)
    q, s = U.quantize_sym_int8(x)
    T["ties.x"], T["ties.q"] = x, q
    M["ties.scale"] = s
    eye = torch.eye(16) * 1e-4
    q, s = U.quantize_sym_int8(eye)
    T["eye.q"] = q
    M["eye.scale"] = s
    spectra = [torch.linspace(10, 0, 50), torch.logspace(0, -6, 64), torch.zeros(10),
               torch.ones(32), torch.tensor([5.0, 1e-9, 1e-9, 0.0])]
    for i, sp in enumerate(spectra):
        T[f"rank{i}.s"] = sp
        M[f"rank{i}.k"] = [U.adaptive_rank(sp, e, kmin, kmax)
                           for e, kmin, kmax in [(0.05, 4, 128), (0.2, 1, 8), (0.0, 2, 1000)]]
    # standalone preconditioner: precondition + natural norm after refreshes
    for i, (shape, D, int8) in enumerate([((40, 24), 64, True), ((96, 20), 32, True),
                                          ((18, 50), 32, False), ((30,), 64, True)]):
        p = torch.zeros(shape)
        pre = SparsePreconditioner(p, k_min=3, k_max=12, rho=0.9, max_precond_dim=D,
                                   use_int8_ema=int8)
        for r in range(3):
            gr = torch.randn(shape, generator=g)
            T[f"pre{i}.g{r}"] = gr
            pre.update_curvature(gr)
        gq = torch.randn(shape, generator=g)
        T[f"pre{i}.gq"] = gq
        T[f"pre{i}.out"] = pre.precondition(gq)
        T[f"pre{i}.nat"] = pre.natural_grad_norm(gq, eps=1e-8).reshape(1)
        M[f"pre{i}"] = {"shape": list(shape), "D": D, "int8": int8, "k": pre.k,
                        "memory_bytes": pre.memory_bytes()}
    save_file({k: v.contiguous() for k, v in T.items()}, os.path.join(HERE, "ops.safetensors"))
    with open(os.path.join(HERE, "ops.json"), "w") as f:
        json.dump(M, f, indent=1, sort_keys=True)
    print(f"ops: {len(T)} tensors")


def run_c1(scao, steps=100):
    """The 768x3072 parity configuration: one fp32 Linear weight."""
    g0 = torch.Generator().manual_seed(0)
    p = torch.nn.Parameter(torch.randn(768, 3072, generator=g0) * 0.02)
    cfg = dict(lr=1e-3, use_int8_ema=True, k_min=32, k_max=32, max_precond_dim=1024,
               warmup_steps=20, blend_steps=50, precond_freq=10, min_precond_updates=2,
               **PARITY)
    opt = scao.SCAO([p], **cfg)
    rows = []
    for t in range(1, steps + 1):
        gg = torch.Generator().manual_seed(1000 + t)
        p.grad = torch.randn(p.shape, generator=gg) * 0.02
        opt.step()
        st = opt.state[p]
        pre = st["preconditioner"]
        rec = {"t": t, "p_norm": float(p.detach().double().norm()),
               "p_sum": float(p.detach().double().sum()),
               "p_head": [float(v) for v in p.detach().flatten()[:16]],
               "m_norm": float(st["exp_avg"].double().norm()),
               "v_sum": float(st["exp_avg_sq"].double().sum()),
               "precond_step": pre.precond_step, "k": pre.k, "blocks": []}
        for b in pre._blocks:
            rec["blocks"].append({
                "L_scale": b.L_ema_scale, "R_scale": b.R_ema_scale, "k": b.k,
                "L_sha": hashlib.sha256(b.L_ema_q.numpy().tobytes()).hexdigest()[:16],
                "R_sha": hashlib.sha256(b.R_ema_q.numpy().tobytes()).hexdigest()[:16],
                "L_code_sum": int(b.L_ema_q.to(torch.int64).sum()),
                "S_l_head": [float(v) for v in b.S_l[:4]]})
        rows.append(rec)
    # full end state of block 0 for tolerance checks
    b0 = pre._blocks[0]
    save_file({"L_q": b0.L_ema_q[:32].clone(), "R_q": b0.R_ema_q[:32].clone(),
               "p_final_rows": p.detach()[:2].clone()},
              os.path.join(HERE, "c1_summary.safetensors"))
    with open(os.path.join(HERE, "c1_summary.json"), "w") as f:
        json.dump({"config": cfg, "rows": rows}, f, indent=0, sort_keys=True)
    print("c1_summary done")


def run_ckpt(scao):
    """A reference checkpoint file and what the reference does after resuming
    from it: 5 steps (Phase 1, a refresh, Phase 2), torch.save of
    state_dict(); a fresh reference optimizer loads the file and takes two
    more Phase-2 steps.  Stored: the file, the parameters at the save and
    after each resumed step."""
    import io
    cfg = dict(lr=1e-2, weight_decay=0.01, max_precond_dim=32, rho=0.99, use_int8_ema=True,
               k_min=2, k_max=6, warmup_steps=2, blend_steps=3, precond_freq=4,
               min_precond_updates=1, tau=1.0, lars_coeff=1e-3, **PARITY)
    params = make_params(SMALL_SHAPES)
    opt = scao.SCAO(list(params.values()), **cfg)
    for t in range(1, 6):
        grads = grads_for_step(t, params)
        for k, p in params.items():
            p.grad = grads[k]
        opt.step()
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    with open(os.path.join(HERE, "ref_checkpoint.pt"), "wb") as f:
        f.write(buf.getvalue())
    out = {f"ckpt/{k}": p.detach().clone() for k, p in params.items()}
    resumed = {k: torch.nn.Parameter(p.detach().clone()) for k, p in params.items()}
    opt2 = scao.SCAO(list(resumed.values()), **cfg)
    buf.seek(0)
    opt2.load_state_dict(torch.load(buf, weights_only=False))   # written above
    for t in (6, 7):
        grads = grads_for_step(t, resumed)
        for k, p in resumed.items():
            p.grad = grads[k]
        opt2.step()
        for k, p in resumed.items():
            out[f"step{t}/{k}"] = p.detach().clone()
    save_file({k: v.contiguous() for k, v in out.items()},
              os.path.join(HERE, "ckpt_resume.safetensors"))
    meta = {"config": cfg, "names": list(SMALL_SHAPES), "saved_after_step": 5,
            "resumed_steps": [6, 7]}
    with open(os.path.join(HERE, "ckpt_resume.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


DIAG_SHAPES = {"q": (2048, 2048), "kv": (512, 2048)}
DIAG_CFG = dict(k_min=64, k_max=64, rho=0.999, max_precond_dim=2048, use_int8_ema=True)


def diag_grad(shape, r: int, pi: int):
    """Refresh r's gradient of the pi-th diag_int8 weight: N(0, 1e-3^2)."""
    g = torch.Generator().manual_seed(5000 + 10 * r + pi)
    return torch.randn(shape, generator=g) * 1e-3


def run_diag(scao):
    """The reference's own refreshes from its initialisation at the gradient
    scale of the Llama/Qwen configurations: an int8 SparsePreconditioner on a
    2048x2048 and a 512x2048 weight (k = 64, max_precond_dim 2048, rho
    0.999), three update_curvature calls with N(0, 1e-3^2) gradients.  The
    requantised EMAs keep only their diagonal codes, so every eigh input is
    exactly diagonal and its eigenvectors are unit vectors, in the order
    LAPACK's selection sort leaves tied values.  Stored per refresh and side:
    each kept column's row and sign, S, the diagonal codes, the scale, the
    count of non-zero off-diagonal codes and k."""
    from scao.preconditioner import SparsePreconditioner
    out, meta = {}, {"config": DIAG_CFG, "blocks": [[k, list(v)] for k, v in DIAG_SHAPES.items()],
                     "refreshes": 3, "rows": {}}
    for pi, (name, shape) in enumerate(DIAG_SHAPES.items()):
        pre = SparsePreconditioner(torch.zeros(shape), **DIAG_CFG)
        for r in range(3):
            pre.update_curvature(diag_grad(shape, r, pi))
            rec = {"k": pre.k, "precond_step": pre.precond_step}
            for side, U, S, q, sc in (("L", pre.U_l, pre.S_l, pre.L_ema_q, pre.L_ema_scale),
                                      ("R", pre.U_r, pre.S_r, pre.R_ema_q, pre.R_ema_scale)):
                cols = torch.arange(U.shape[1])
                rows = U.abs().argmax(0)
                sign = U[rows, cols]
                unit = torch.zeros_like(U)
                unit[rows, cols] = sign
                assert torch.equal(unit, U), "eigenvectors are not unit vectors"
                off = int((q != 0).sum()) - int((q.diagonal() != 0).sum())
                key = f"{name}.r{r}.{side}"
                out[key + ".rows"] = rows.to(torch.int32)
                out[key + ".sign"] = sign.clone()
                out[key + ".S"] = S.clone()
                out[key + ".diag_codes"] = q.diagonal().clone()
                rec[side] = {"scale": sc, "offdiag_nonzero": off,
                             "sha": hashlib.sha256(q.numpy().tobytes()).hexdigest()[:16]}
            meta["rows"][f"{name}.r{r}"] = rec
    save_file(out, os.path.join(HERE, "diag_int8.safetensors"))
    with open(os.path.join(HERE, "diag_int8.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print("diag_int8 done")


def main(only=None):
    """Write every fixture, or only those named on the command line."""
    sys.path.insert(0, REF)
    warnings.simplefilter("ignore")
    torch.set_num_threads(8)
    import scao  # the reference package

    def want(name):
        return not only or name in only

    base = dict(lr=1e-2, weight_decay=0.01, max_precond_dim=32, rho=0.99, **PARITY)
    fp32_small = dict(base, use_int8_ema=False, k_min=4, k_max=4, warmup_steps=4,
                      blend_steps=4, precond_freq=2, min_precond_updates=1, tau=None,
                      lars_coeff=0.0)
    int8_small = dict(base, use_int8_ema=True, k_min=2, k_max=8, warmup_steps=6,
                      blend_steps=5, precond_freq=3, min_precond_updates=2, tau=1.0,
                      lars_coeff=1e-3)
    features = {
        # gSNR mask on the update (scao/optimizer.py:160-181)
        "traj_gsnr": (dict(fp32_small, use_gsnr_clip=True, gsnr_threshold=0.5), 12),
        # refresh triggered by the gradient-norm change (:187-214)
        "traj_lazy": (dict(int8_small, lazy_precond=True, lazy_delta_threshold=0.05,
                           lazy_max_skip=3), 14),
        # warm-up that ends when the gradient norm settles (:106-154)
        "traj_awarmup": (dict(fp32_small, adaptive_warmup=True, warmup_steps=30,
                              warmup_stability_threshold=0.5, warmup_patience=2), 26),
        # sparsity from the layer's norm against the global EMA (:60-99)
        "traj_dynsparse": (dict(int8_small, sparsity=0.7, dynamic_sparsity=True), 12),
        # rank moved by the gradient-norm ratio (:383-401)
        "traj_arank": (dict(fp32_small, adaptive_rank=True, k_min=2, k_max=8), 12),
    }
    for name, (cfg, steps) in features.items():
        if want(name):
            run_traj(scao, name, cfg, steps=steps, snap_steps=(steps,))
    if want("diag_int8"):
        run_diag(scao)
    if not want("traj_int8"):
        return
    run_traj(scao, "traj_int8", dict(base, use_int8_ema=True, k_min=2, k_max=8,
                                     warmup_steps=6, blend_steps=5, precond_freq=3,
                                     min_precond_updates=2, tau=1.0, lars_coeff=1e-3),
             steps=24, snap_steps=(6, 9, 24))
    run_traj(scao, "traj_fp32", dict(base, use_int8_ema=False, k_min=4, k_max=4,
                                     warmup_steps=4, blend_steps=4, precond_freq=2,
                                     min_precond_updates=1, tau=None, lars_coeff=0.0),
             steps=16, snap_steps=(16,))
    run_traj(scao, "traj_misc", dict(base, use_int8_ema=True, k_min=3, k_max=6,
                                     warmup_steps=3, blend_steps=0, precond_freq=2,
                                     min_precond_updates=1, tau=0.05, lars_coeff=1e-3,
                                     weight_decay=0.1, lookahead_k=3, lookahead_alpha=0.5),
             steps=14, snap_steps=(14,))
    run_traj(scao, "traj_bf16", dict(base, use_int8_ema=True, k_min=2, k_max=4,
                                     warmup_steps=3, blend_steps=3, precond_freq=2,
                                     min_precond_updates=1),
             steps=10, snap_steps=(10,), dtype=torch.bfloat16)
    run_traj(scao, "traj_sparse", dict(base, use_int8_ema=True, k_min=2, k_max=6,
                                       warmup_steps=3, blend_steps=3, precond_freq=2,
                                       min_precond_updates=1, sparsity=0.7),
             steps=10, snap_steps=(10,), outliers=0.01)
    run_ops(scao)
    run_c1(scao)
    run_ckpt(scao)


if __name__ == "__main__":
    main(set(sys.argv[1:]) or None)
