"""Drop-in ``SCAO`` optimizer (reference: scao/optimizer.py:221-1002).

Constructor arguments, the 18 per-group ``defaults`` keys, per-parameter
state keys, the Phase 1 (Adam(W)) -> Phase 2 (blended, preconditioned Adan)
state machine, the refresh schedule, ``state_dict`` layout, callbacks and
presets follow the reference.  The per-parameter Python loop survives only
as host bookkeeping (integer counters and phase flags); every tensor update
of a step is launched by ``scao_amd.engine`` as a few batched HIP kernels
on the current stream, with no host synchronisation in a non-refresh step.

Differences a caller can observe:
  * parameters must be on a ROCm device (``step`` raises otherwise);
  * ``async_precond`` is accepted and ignored: the refresh runs in stream
    order on the current stream, before the update that uses it (the
    reference's side stream has no synchronisation, scao/optimizer.py:651-665);
  * ``_global_norm_ema`` is kept on the device and read back on access.
"""

from __future__ import annotations

import warnings
from typing import Callable, Iterable, Optional

import numpy as np
import torch
from torch import Tensor
from torch.optim import Optimizer

from . import engine
from .engine import PItem, Workspace, require_hip
from .preconditioner import SparsePreconditioner


# --------------------------------------------------------------------------
# v3 helpers (reference scao/optimizer.py:42-214), device tensors
# --------------------------------------------------------------------------

def _carry_diag_bias(src, dst) -> None:
    """A diagonal preconditioner's bias factor is not part of the portable
    ``_scao_precond`` state (scao/preconditioner.py:570-600); the object in
    the per-parameter state carries it.  Take it over when a preconditioner
    is rebuilt from another object (the reference's, a checkpoint record or
    one on another device)."""
    bias = getattr(src, "_diag_bias_factor", None)
    if bias is not None and hasattr(dst, "_diag_bias_factor"):
        dst._diag_bias_factor = float(bias)
    for a, b in zip(getattr(src, "_blocks", None) or [], getattr(dst, "_blocks", None) or []):
        _carry_diag_bias(a, b)


class _SparseGradFilter:
    """reference :42-57: EMA of |g| and the mask ``ema >= quantile(ema, q)``.
    The work runs in ``scao_sparse_filter`` (one batched launch sequence per
    step, exact order statistics by radix select); ``__call__`` filters one
    gradient through the same entry point.  torch.quantile refuses more than
    2**24 elements, so the reference raises for such a parameter; this filter
    computes the same statistic for any size.  It refuses an empty input too
    (reference :56); here an empty gradient is skipped and stays empty."""

    def __init__(self, sparsity: float = 0.7, ema: float = 0.99):
        self.sparsity, self.ema, self.mag_ema = sparsity, ema, None
        self.work = None          # device scratch of the batched kernel: selection
        self.cand = None          # state, and the candidate keys of one bin

    def prepare(self, grad: Tensor) -> None:
        """Host-side update before the batched launch (dynamic sparsity)."""

    def __call__(self, grad: Tensor) -> Tensor:
        self.prepare(grad)
        return engine.moment_grads([(self, grad.contiguous())])[0]


class _DynamicSparseFilter(_SparseGradFilter):
    """reference :60-99."""

    def __init__(self, base_sparsity=0.7, min_sparsity=0.3, max_sparsity=0.9, ema=0.99,
                 norm_ema=0.95):
        super().__init__(sparsity=base_sparsity, ema=ema)
        self.base_sparsity, self.min_sparsity, self.max_sparsity = base_sparsity, min_sparsity, max_sparsity
        self.norm_ema_coeff = norm_ema
        self._norm_ema = 1.0
        self._global_norm_ema = 1.0

    def set_global_norm_ref(self, v: float) -> None:
        self._global_norm_ema = max(v, 1e-8)

    def prepare(self, grad: Tensor) -> None:
        """reference :88-99: the sparsity for this call from the layer norm."""
        ln = float(grad.float().norm())
        self._norm_ema = self.norm_ema_coeff * self._norm_ema + (1.0 - self.norm_ema_coeff) * ln
        ratio = self._norm_ema / self._global_norm_ema
        margin = 0.2 * (1.0 - min(ratio, 2.0) / 2.0)
        self.sparsity = float(max(self.min_sparsity, min(self.max_sparsity, self.base_sparsity + margin)))


class _AdaptiveWarmupScheduler:
    """reference :106-154."""

    def __init__(self, warmup_steps=100, stability_threshold=0.05, patience=5, min_warmup=20):
        self.warmup_steps, self.stability_threshold = warmup_steps, stability_threshold
        self.patience, self.min_warmup = patience, min_warmup
        self._prev_norm = float("inf")
        self._stable_count = 0
        self._early_exit_step: Optional[int] = None

    def update(self, step: int, avg_grad_norm: float) -> bool:
        if step < self.min_warmup:
            return True
        if self._prev_norm > 0:
            rel = abs(avg_grad_norm - self._prev_norm) / (self._prev_norm + 1e-8)
            self._stable_count = self._stable_count + 1 if rel < self.stability_threshold else 0
        self._prev_norm = avg_grad_norm
        if self._stable_count >= self.patience:
            self._early_exit_step = self._early_exit_step or step
            return False
        return step < self.warmup_steps

    @property
    def exited_early(self) -> bool:
        return self._early_exit_step is not None

    @property
    def actual_warmup_steps(self) -> int:
        return self._early_exit_step or self.warmup_steps


class _LazyPrecondTrigger:
    """reference :182-214."""

    def __init__(self, delta_threshold: float = 0.1, max_skip: int = 50):
        self.delta_threshold, self.max_skip = delta_threshold, max_skip
        self._prev_grad_norm = 0.0
        self._steps_since_update = 0

    def should_update(self, grad_norm: float) -> bool:
        self._steps_since_update += 1
        if self._steps_since_update >= self.max_skip:
            self._steps_since_update = 0
            self._prev_grad_norm = grad_norm
            return True
        if self._prev_grad_norm > 0:
            rel = abs(grad_norm - self._prev_grad_norm) / (self._prev_grad_norm + 1e-8)
            if rel > self.delta_threshold:
                self._steps_since_update = 0
                self._prev_grad_norm = grad_norm
                return True
        self._prev_grad_norm = grad_norm
        return False


# --------------------------------------------------------------------------
# SCAO
# --------------------------------------------------------------------------

class SCAO(Optimizer):
    """Sparse Curvature-Aware Adaptive Optimizer on MI355X (drop-in for scao.SCAO)."""

    def __init__(self, params: Iterable, lr: float = 1e-3, betas: tuple = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.01, precond_freq: int = 20,
                 epsilon_sparse: float = 0.05, k_min: int = 8, k_max: int = 128,
                 rho: float = 0.999, tau: float | None = 1.0, warmup_steps: int = 100,
                 blend_steps: int = 50, min_precond_updates: int = 10,
                 max_precond_dim: int = 4096, use_newton_schulz: bool = False,
                 use_int8_ema: bool = False, async_precond: bool = True, beta3: float = 0.99,
                 sparsity: float = 0.7, noise_std_init: float = 0.01,
                 noise_anneal: float = 0.998, lars_coeff: float = 1e-3, lookahead_k: int = 5,
                 lookahead_alpha: float = 0.5, dynamic_sparsity: bool = False,
                 adaptive_warmup: bool = False, warmup_stability_threshold: float = 0.05,
                 warmup_patience: int = 5, lazy_precond: bool = False,
                 lazy_delta_threshold: float = 0.1, lazy_max_skip: int = 50,
                 use_gsnr_clip: bool = False, gsnr_threshold: float = 0.5,
                 adaptive_rank: bool = False) -> None:
        # reference :297-304
        if lr < 0:
            raise ValueError(f"Invalid lr: {lr}")
        if not (0.0 <= betas[0] < 1.0):
            raise ValueError(f"Invalid beta1: {betas[0]}")
        if not (0.0 <= betas[1] < 1.0):
            raise ValueError(f"Invalid beta2: {betas[1]}")
        if not (0.0 <= beta3 < 1.0):
            raise ValueError(f"Invalid beta3: {beta3}")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                        precond_freq=precond_freq, epsilon_sparse=epsilon_sparse,
                        k_min=k_min, k_max=k_max, rho=rho, tau=tau,
                        warmup_steps=warmup_steps, blend_steps=blend_steps,
                        min_precond_updates=min_precond_updates,
                        max_precond_dim=max_precond_dim, use_newton_schulz=use_newton_schulz,
                        use_int8_ema=use_int8_ema, beta3=beta3, lars_coeff=lars_coeff)
        super().__init__(params, defaults)
        self._precond_stream = None
        self._async_precond = async_precond
        self._callbacks: list = []
        self._global_step = 0
        self._noise_std = noise_std_init
        self._noise_anneal = noise_anneal
        self._lookahead_k = lookahead_k
        self._lookahead_alpha = lookahead_alpha
        self._slow_weights: dict = {}
        self._sparsity = sparsity
        self._dynamic_sparsity = dynamic_sparsity
        self._sparse_filters: dict = {}
        self._norm_ema_host = 1.0
        self._adaptive_warmup = adaptive_warmup
        self._warmup_scheduler = _AdaptiveWarmupScheduler(
            warmup_steps=warmup_steps, stability_threshold=warmup_stability_threshold,
            patience=warmup_patience, min_warmup=max(20, warmup_steps // 5))
        self._lazy_precond = lazy_precond
        self._lazy_triggers: dict = {}
        self._lazy_delta_threshold = lazy_delta_threshold
        self._lazy_max_skip = lazy_max_skip
        self._use_gsnr_clip = use_gsnr_clip
        self._gsnr_threshold = gsnr_threshold
        self._adaptive_rank = adaptive_rank
        self._in_warmup_global = True
        self._ws: Optional[Workspace] = None
        self._plan = None   # engine.StepPlan of the last plain step, or None

    # ---------------------------------------------------------- runtime --
    @property
    def _global_norm_ema(self) -> float:
        if self._ws is not None:
            return float(self._ws.runtime[0])
        return self._norm_ema_host

    @_global_norm_ema.setter
    def _global_norm_ema(self, v: float) -> None:
        self._norm_ema_host = float(v)
        if self._ws is not None:
            self._ws.runtime[0] = float(v)

    def _active(self) -> list:
        """(group, parameter) for every parameter with a gradient, each
        checked to live on a ROCm device."""
        active = [(g, p) for g in self.param_groups for p in g["params"] if p.grad is not None]
        for _, p in active:
            require_hip(p, "parameter")
        return active

    def _workspace(self, device: torch.device) -> Workspace:
        if self._ws is None:
            self._ws = Workspace(device)
            self._ws.runtime[0] = self._norm_ema_host
        elif self._ws.device != device:
            raise RuntimeError("scao_amd.SCAO: all parameters must be on one device "
                               f"({self._ws.device} vs {device})")
        return self._ws

    # ------------------------------------------------------- lookahead ---
    @torch.no_grad()
    def _lookahead_sync(self) -> None:
        """reference :356-365, every parameter in one batched launch
        (``scao_lookahead``): slow += alpha * (p - slow); p = slow."""
        pairs = []
        for g in self.param_groups:
            for p in g["params"]:
                pid = id(p)
                if pid not in self._slow_weights:
                    self._slow_weights[pid] = p.data.clone(memory_format=torch.contiguous_format)
                pairs.append((p.data, self._slow_weights[pid]))
        engine.lookahead(pairs, self._lookahead_alpha)

    # ------------------------------------------------------------ rank ---
    def _maybe_adjust_rank(self, pre: SparsePreconditioner, grad_norm: float, group: dict) -> None:
        """reference :383-401."""
        if not self._adaptive_rank:
            return
        ratio = grad_norm / (self._global_norm_ema + 1e-8)
        cur = pre.k
        if ratio > 2.0:
            nk = min(group["k_max"], int(cur * 1.25))
        elif ratio < 0.5:
            nk = max(group["k_min"], int(cur * 0.8))
        else:
            return
        if nk != cur:
            pre.k = nk

    # ------------------------------------------------------------ state --
    def _init_state(self, p: Tensor, group: dict) -> None:
        """reference :407-433."""
        st = self.state[p]
        if len(st) > 0:
            return
        st["step"] = 0
        st["scao_step"] = 0
        for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
            st[key] = torch.zeros_like(p, dtype=torch.float32, memory_format=torch.contiguous_format)
        st["preconditioner"] = self._make_precond(p, group)

    @staticmethod
    def _make_precond(p: Tensor, group: dict) -> SparsePreconditioner:
        return SparsePreconditioner(
            param=p, epsilon_sparse=group["epsilon_sparse"], k_min=group["k_min"],
            k_max=group["k_max"], rho=group["rho"], max_precond_dim=group["max_precond_dim"],
            use_newton_schulz=group["use_newton_schulz"], use_int8_ema=group["use_int8_ema"])

    # ------------------------------------------------------------- step --
    @torch.no_grad()
    def step(self, closure: Callable | None = None) -> Tensor | None:
        """reference :452-503 (host bookkeeping) + one batched engine launch."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._global_step += 1
        host_norms = (self._dynamic_sparsity or self._adaptive_warmup or self._adaptive_rank
                      or self._lazy_precond)
        active = self._active() if host_norms else None
        avg = 0.0
        if host_norms and active:
            norms = [float(p.grad.norm()) for _, p in active]
            avg = sum(norms) / len(norms)
            self._global_norm_ema = 0.95 * self._global_norm_ema + 0.05 * avg
        if self._dynamic_sparsity:
            ref = self._global_norm_ema
            for f in self._sparse_filters.values():
                if isinstance(f, _DynamicSparseFilter):
                    f.set_global_norm_ref(ref)
        if self._adaptive_warmup:
            self._in_warmup_global = self._warmup_scheduler.update(self._global_step, avg)
        else:
            wmax = max((g.get("warmup_steps", 100) for g in self.param_groups), default=100)
            self._in_warmup_global = self._global_step <= wmax

        gsnr = self._gsnr_threshold if self._use_gsnr_clip else None
        # a plain step of the planned parameters checks each of them itself
        # (_planned_step); any other step checks and plans every parameter
        # that has a gradient
        if not self._planned_step(self._ws, host_norms, gsnr):
            if active is None:
                active = self._active()
            ws = self._workspace(active[0][1].device) if active else self._ws
            self._plan = None
            items, refresh, filtered = [], [], []
            for group, p in active:
                it = self._plan_param(group, p, refresh, filtered)
                items.append(it)
            self._filter_and_noise(items, filtered)
            engine.refresh(refresh)
            if ws is not None:
                plan = engine.run_step(items, ws, update_norm_ema=not host_norms, gsnr=gsnr)
                if (plan is not None and not host_norms and not refresh and not filtered
                        and self._noise_std <= 1e-9
                        and all(it.graw is it.p.grad and it.msrc is None and it.gmom is None
                                for it in items)):
                    self._plan = plan

        self._noise_std *= self._noise_anneal
        if self._lookahead_k > 0 and self._global_step % self._lookahead_k == 0:
            self._lookahead_sync()
        if self._callbacks:
            from .logging import collect_metrics
            metrics = collect_metrics(self)
            metrics["noise_std"] = self._noise_std
            metrics["global_norm_ema"] = self._global_norm_ema
            metrics["warmup_active"] = self._in_warmup_global
            for cb in self._callbacks:
                cb(metrics)
        return loss

    def _planned_step(self, ws, host_norms: bool, gsnr) -> bool:
        """The next step of the last plain step's parameters, when nothing
        but the step counters changes: the same parameters (same groups, same
        order) have gradients, contiguous and with the planned alignment; the
        moment tensors and the parameters' storage are the planned ones; no
        refresh is due and no phase changes (a Phase-1 class stays inside its
        warm-up, a Phase-2 class keeps its LARS setting); no filter, noise or
        host norms.  Then the host bookkeeping of _plan_param reduces to the
        counters (every planned item had step t, now t + 1) and the launch
        reuses the planned parameter table (engine.run_planned_step).
        Returns False, changing nothing, when any of this does not hold."""
        plan = self._plan
        if (plan is None or ws is None or host_norms or self._sparsity > 0.0
                or self._noise_std > 1e-9 or plan.gsnr != gsnr
                or plan.epoch != engine.leaf_epoch()):
            return False
        items = plan.items
        n = len(items)
        ptrs = []
        grads = []
        i = 0
        for g in self.param_groups:
            for p in g["params"]:
                gr = p.grad
                if gr is None:
                    continue
                if i >= n:
                    return False
                it = items[i]
                if it.p is not p or it.group is not g or gr.is_sparse or not gr.is_contiguous():
                    return False
                ptr = gr.data_ptr()
                if (it.aligned and ptr & 15) or it.ptrs[0] != p.data_ptr():
                    return False
                ptrs.append(ptr)
                grads.append(gr)
                i += 1
        if i != n:
            return False
        gptrs = np.array(ptrs, dtype=np.uint64)
        for it, moms in zip(items, plan.moments):
            st = it.st
            if (st["step"] != it.step or st["exp_avg"] is not moms[0]
                    or st["exp_avg_sq"] is not moms[1] or st["exp_avg_diff"] is not moms[2]
                    or st["prev_grad"] is not moms[3]):
                return False
        if plan.min_pre is None:   # precond_step only moves with a refresh
            plan.min_pre = [min(items[r].pre.precond_step for r in cl.rows)
                            for cl in plan.classes]
        for cl, min_pre in zip(plan.classes, plan.min_pre):
            g, t = cl.group, cl.step + 1
            if t % g["precond_freq"] == 0:
                return False
            if cl.phase2:
                if (t <= g["warmup_steps"] or cl.lars != (g["lars_coeff"] > 0)
                        or min_pre < g["min_precond_updates"]):
                    return False
            elif t > g["warmup_steps"]:
                return False
        # the launch needs only the class counters (advanced inside); the
        # per-parameter host counters follow once the kernels are queued
        engine.run_planned_step(plan, gptrs, ws, update_norm_ema=True)
        for it, gr in zip(items, grads):
            st = it.st
            st["step"] += 1
            it.step += 1
            if it.phase2:
                st["scao_step"] += 1
                it.scao_step += 1
            it.graw = gr
        return True

    def _filter_and_noise(self, items: list, filtered: list) -> None:
        """The gradient the moments see (reference :533-545): the filtered
        parameters go through one batched launch (scao_sparse_filter: EMA and
        threshold); the step kernels then form fp32(g) * mask + noise_std *
        N(0, 1) themselves (counter-based generator keyed per parameter and
        step), so the moment gradient is never written out."""
        noise = self._noise_std if self._noise_std > 1e-9 else 0.0
        filt = {id(it): f for it, f, _ in filtered}
        todo = [it for it in items if id(it) in filt or noise > 0.0]
        if not todo:
            return
        srcs = engine.moment_sources([(filt.get(id(it)), it.graw) for it in todo], noise)
        for it, src in zip(todo, srcs):
            it.msrc = src

    def _plan_param(self, group: dict, p: Tensor, refresh: list, filtered: list) -> PItem:
        """Host half of reference _step_group (:521-605) for one parameter."""
        grad = p.grad
        if grad.is_sparse:
            raise RuntimeError("SCAO does not support sparse gradients.")
        if not p.is_contiguous():
            raise RuntimeError("scao_amd.SCAO needs contiguous parameters")
        st = self.state[p]
        if not st:
            self._init_state(p, group)
        st["step"] += 1
        t = st["step"]
        pid = id(p)
        graw = grad if grad.is_contiguous() else grad.contiguous()
        need_gnorm = self._lazy_precond or self._adaptive_rank
        gnorm = float(graw.float().norm()) if need_gnorm else 0.0
        gmom = None   # set by _filter_and_noise when filtered or noised
        filt = None
        if self._sparsity > 0.0:
            if pid not in self._sparse_filters:
                self._sparse_filters[pid] = (_DynamicSparseFilter(base_sparsity=self._sparsity)
                                             if self._dynamic_sparsity
                                             else _SparseGradFilter(self._sparsity))
            filt = self._sparse_filters[pid]
            filt.prepare(graw)
        pre: SparsePreconditioner = st["preconditioner"]
        self._maybe_adjust_rank(pre, gnorm, group)
        in_warmup = (self._in_warmup_global if self._adaptive_warmup
                     else (t <= group["warmup_steps"])) or \
            (pre.precond_step < group["min_precond_updates"])
        if in_warmup:
            if t % group["precond_freq"] == 0:
                refresh.append((pre, grad))
            it = PItem(p=p, graw=graw, gmom=gmom, st=st, group=group, pre=pre,
                       phase2=False, step=t)
            if filt is not None:
                filtered.append((it, filt, graw))
            return it
        if not st.get("scao_phase_started", False):
            st["scao_phase_started"] = True
            st["phase2_start_step"] = t
            st["scao_step"] = 0
        st["scao_step"] += 1
        if self._lazy_precond:
            if pid not in self._lazy_triggers:
                self._lazy_triggers[pid] = _LazyPrecondTrigger(self._lazy_delta_threshold,
                                                               self._lazy_max_skip)
            should = self._lazy_triggers[pid].should_update(gnorm)
        else:
            should = t % group["precond_freq"] == 0
        if should:
            refresh.append((pre, grad))
        diag = not (pre.use_block_diagonal or pre.use_kronecker)
        it = PItem(p=p, graw=graw, gmom=gmom, st=st, group=group, pre=pre, phase2=True,
                   step=t, scao_step=st["scao_step"], lars=group["lars_coeff"] > 0,
                   diag=diag, leaves=[] if diag else pre.step_leaf_list())
        if filt is not None:
            filtered.append((it, filt, graw))
        return it

    # ------------------------------------------------------------ misc ---
    def synchronize_precond(self) -> None:
        """reference :680-684.  The refresh runs on the current stream, in
        order; there is no side stream to wait for."""

    def sync_preconditioner(self, process_group=None) -> None:
        """reference :686-710: rank 0's moments, step counters and
        preconditioner state on every rank (``distributed.broadcast_state``);
        a warning and nothing else when torch.distributed is not initialised."""
        import torch.distributed as dist
        if not dist.is_available() or not dist.is_initialized():
            warnings.warn("sync_preconditioner() called but distributed is not initialised.",
                          RuntimeWarning, stacklevel=2)
            return
        from .distributed import broadcast_state
        broadcast_state(self, process_group)

    def add_callback(self, callback) -> None:
        self._callbacks.append(callback)

    def remove_callback(self, callback) -> None:
        try:
            self._callbacks.remove(callback)
        except ValueError:
            pass

    def clear_callbacks(self) -> None:
        self._callbacks.clear()

    def state_dict(self) -> dict:
        """reference :732-756."""
        self.synchronize_precond()
        base = super().state_dict()
        base["_scao_precond"] = {idx: st["preconditioner"].state_dict()
                                 for idx, st in enumerate(self.state.values())
                                 if "preconditioner" in st}
        ws = self._warmup_scheduler
        base["_scao_runtime"] = {
            "global_step": self._global_step, "noise_std": self._noise_std,
            "global_norm_ema": self._global_norm_ema, "warmup_prev_norm": ws._prev_norm,
            "warmup_stable_count": ws._stable_count,
            "warmup_early_exit_step": ws._early_exit_step}
        return base

    def load_state_dict(self, state_dict: dict) -> None:
        """reference :758-776.  Preconditioner objects of another type (the
        reference's, or the CPU oracle's) are rebuilt from the parameter and
        its group before the portable ``_scao_precond`` entry is loaded."""
        self._plan = None
        sd = dict(state_dict)
        extra = sd.pop("_scao_precond", {})
        rt = sd.pop("_scao_runtime", {})
        super().load_state_dict(sd)
        self._restore_fp32_moments(sd)
        owner = {id(p): g for g in self.param_groups for p in g["params"]}
        for idx, (p, st) in enumerate(self.state.items()):
            old = st.get("preconditioner")
            if old is not None and (not isinstance(old, SparsePreconditioner)
                                    or old.device != p.device):
                st["preconditioner"] = self._make_precond(p, owner[id(p)])
                _carry_diag_bias(old, st["preconditioner"])
            if idx in extra and "preconditioner" in st:
                st["preconditioner"].load_state_dict(extra[idx])
        if rt:
            self._global_step = int(rt.get("global_step", self._global_step))
            self._noise_std = float(rt.get("noise_std", self._noise_std))
            self._global_norm_ema = float(rt.get("global_norm_ema", self._global_norm_ema))
            ws = self._warmup_scheduler
            ws._prev_norm = float(rt.get("warmup_prev_norm", ws._prev_norm))
            ws._stable_count = int(rt.get("warmup_stable_count", ws._stable_count))
            ws._early_exit_step = rt.get("warmup_early_exit_step", ws._early_exit_step)
        if self._ws is not None:
            self._ws.invalidate()

    def _restore_fp32_moments(self, sd: dict) -> None:
        """``torch.optim.Optimizer.load_state_dict`` casts every floating state
        tensor to its parameter's dtype.  The reference inherits that, so after
        a resume its bf16/fp16 parameters carry reduced-precision moments,
        although it creates them in fp32 (scao/optimizer.py:407-433).  The
        step kernels keep fp32 statistics, so the moments are taken again from
        the checkpoint at full precision, contiguous, on the parameter's
        device."""
        saved = [i for g in sd.get("param_groups", []) for i in g["params"]]
        current = [p for g in self.param_groups for p in g["params"]]
        for i, p in zip(saved, current):
            src = sd.get("state", {}).get(i)
            if not src or p not in self.state:
                continue
            st = self.state[p]
            for key in ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad"):
                v, cur = src.get(key), st.get(key)
                if not isinstance(v, Tensor) or not isinstance(cur, Tensor):
                    continue
                if cur.dtype != torch.float32:
                    cur = v.to(device=p.device, dtype=torch.float32, copy=True)
                st[key] = cur.contiguous()

    def current_ranks(self) -> dict:
        """reference :782-787."""
        return {idx: st["preconditioner"].k for idx, st in enumerate(self.state.values())
                if "preconditioner" in st}

    def precond_stats(self) -> dict:
        """reference :789-801."""
        ks = list(self.current_ranks().values())
        if not ks:
            return {}
        return {"num_precond_layers": len(ks), "rank_min": min(ks), "rank_max": max(ks),
                "rank_mean": sum(ks) / len(ks), "global_norm_ema": self._global_norm_ema,
                "warmup_exited_early": self._warmup_scheduler.exited_early,
                "actual_warmup_steps": self._warmup_scheduler.actual_warmup_steps}


# --------------------------------------------------------------------------
# presets (the definitions in effect in the reference, scao/optimizer.py:958-1002)
# --------------------------------------------------------------------------

def _params_of(x):
    return x.parameters() if hasattr(x, "parameters") else x


def scao_sub1b(model_or_params, lr=1e-3, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=64, use_int8_ema=False, **kwargs)


def scao_1b(model_or_params, lr=1e-3, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=48, use_int8_ema=True,
                async_precond=True, **kwargs)


def scao_3b(model_or_params, lr=3e-4, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=32, use_int8_ema=True,
                async_precond=True, warmup_steps=20, blend_steps=10, **kwargs)


def scao_7b(model_or_params, lr=1e-4, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=24, use_int8_ema=True,
                async_precond=False, dynamic_sparsity=False, **kwargs)


def scao_40b(model_or_params, lr=1e-4, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=16, use_int8_ema=True,
                async_precond=True, lazy_precond=True, use_gsnr_clip=True, **kwargs)


def scao_125b(model_or_params, lr=5e-5, **kwargs):
    return SCAO(_params_of(model_or_params), lr=lr, k_max=8, use_int8_ema=True,
                async_precond=True, lazy_precond=True, lazy_max_skip=100, use_gsnr_clip=True,
                adaptive_rank=True, **kwargs)
