"""Distributed helpers (reference: scao/distributed.py:60-160).

This build targets one GPU.  The functions keep the reference's names and
single-process behaviour (silent no-op when torch.distributed is not
initialised or the world has one rank) and refuse multi-rank use.
"""

from __future__ import annotations

import warnings


def sync_preconditioners(optimizer, process_group=None) -> None:
    """reference :60-128."""
    import torch.distributed as dist
    if not dist.is_available() or not dist.is_initialized():
        return
    if dist.get_world_size(group=process_group) == 1:
        return
    raise NotImplementedError("scao_amd is a single-GPU build: multi-rank preconditioner "
                              "averaging is not provided")


def wrap_scao_for_fsdp(optimizer):
    """reference :131-160: patch ``step`` to sync preconditioners on refresh steps."""
    try:
        from torch.distributed.fsdp import FullyShardedDataParallel  # noqa: F401
    except ImportError:
        warnings.warn("torch.distributed.fsdp not available; FSDP wrapping skipped.")
        return optimizer
    original_step = optimizer.step

    def patched_step(closure=None):
        result = original_step(closure)
        step = next((s.get("step", 0) for s in optimizer.state.values() if "step" in s), 0)
        if step % optimizer.defaults["precond_freq"] == 0:
            optimizer.synchronize_precond()
            sync_preconditioners(optimizer)
        return result

    optimizer.step = patched_step
    return optimizer
