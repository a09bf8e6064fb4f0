"""Callback metrics (reference: scao/logging.py:151-219).

Computed only when a callback is registered; a callback is any callable
taking the metrics dict.  ``scao/L_norm_mean`` for int8
EMAs uses ``scale * 127`` as the reference does; the per-block values are
gathered on the device and read back in one transfer.
"""

from __future__ import annotations

from typing import Callable

import torch

MetricsDict = dict
Callback = Callable[[MetricsDict], None]


def _l_norm_device(pre):
    """max|L_ema| (int8: scale * 127, in double as the reference's Python
    float) or ||L_ema||_F, as a device scalar."""
    scale = getattr(pre, "_scale", None)
    if getattr(pre, "use_int8_ema", False) and isinstance(scale, torch.Tensor):
        return scale[0] * 127.0
    if getattr(pre, "use_int8_ema", False):
        return torch.tensor(pre.L_ema_scale * 127.0, dtype=torch.float64)
    return pre.L_ema.norm(p="fro").double()


def collect_metrics(optimizer) -> MetricsDict:
    """reference :151-219.  The per-block EMA norms are gathered on the
    device and read back in one transfer (the reference reads one Python
    scalar per block)."""
    step = 0
    ranks, groups, vals = [], [], []
    for st in optimizer.state.values():
        if "step" in st:
            step = max(step, st["step"])
        if "preconditioner" in st:
            pre = st["preconditioner"]
            ranks.append(pre.k)
            if getattr(pre, "use_block_diagonal", False):
                bl = [b for b in pre._blocks if b.use_kronecker]
                if bl:
                    groups.append(len(bl))
                    vals += [_l_norm_device(b) for b in bl]
            elif getattr(pre, "use_kronecker", False):
                groups.append(1)
                vals.append(_l_norm_device(pre))
    host = []
    if vals:
        dev = next((v.device for v in vals if v.device.type != "cpu"), torch.device("cpu"))
        host = torch.stack([v.to(dev) for v in vals]).cpu().tolist()
    lnorms, i = [], 0
    for n in groups:
        bn = host[i:i + n]
        i += n
        lnorms.append(bn[0] if n == 1 else sum(bn) / len(bn))
    metrics: MetricsDict = {"step": step}
    if ranks:
        metrics["scao/rank_mean"] = sum(ranks) / len(ranks)
        metrics["scao/rank_min"] = min(ranks)
        metrics["scao/rank_max"] = max(ranks)
        metrics["scao/layers"] = len(ranks)
    if lnorms:
        metrics["scao/L_norm_mean"] = sum(lnorms) / len(lnorms)
    metrics["scao/precond_freq"] = optimizer.param_groups[0].get("precond_freq", -1)
    ws = getattr(optimizer, "_warmup_scheduler", None)
    if ws is not None:
        metrics["scao/warmup_exited_early"] = ws.exited_early
        metrics["scao/actual_warmup_steps"] = ws.actual_warmup_steps
    return metrics
