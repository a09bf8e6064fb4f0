"""The preconditioner broadcast over torch.distributed (reference:
scao/optimizer.py:686-710 and scao/preconditioner.py:647-719).

The measured path runs on one GPU; the broadcast runs over any initialised
torch.distributed group.  Instead of one collective per tensor they move
flat buckets, one per dtype: first the integer metadata (step counters,
adaptive ranks) so that every rank can size its buffers, then the payload.
With the gloo backend the buckets are host tensors (gloo is given CPU
tensors only, and device tensors are copied through them); with nccl (RCCL)
they stay on the device.
"""

from __future__ import annotations

import torch

from .preconditioner import PRECOND_DTYPE

_MOMENTS = ("exp_avg", "exp_avg_sq", "exp_avg_diff")   # the keys the reference broadcasts


def _states(optimizer):
    """Per-parameter states in parameter-group order (the same on every rank,
    unlike the insertion order of ``optimizer.state``)."""
    out = []
    for group in optimizer.param_groups:
        for p in group["params"]:
            st = optimizer.state.get(p)
            if st:
                out.append(st)
    return out


def _nodes(pre):
    """Every preconditioner of a parameter: block-diagonal parents first, then
    their blocks, recursively (the reference's broadcast order)."""
    out = [pre]
    if getattr(pre, "use_block_diagonal", False):
        for blk in pre._blocks:
            out += _nodes(blk)
    return out


def _bucket_device(tensors, group):
    """The device collectives on `group` run on: the CPU for gloo."""
    import torch.distributed as dist
    if dist.get_backend(group) == "gloo":
        return torch.device("cpu")
    return next((t.device for t in tensors if t.device.type != "cpu"),
                torch.device("cuda", torch.cuda.current_device()))


def _flat(tensors, dtype, device):
    if not tensors:
        return None
    return torch.cat([t.detach().reshape(-1).to(device=device, dtype=dtype) for t in tensors])


def _unflat(buf, tensors) -> None:
    off = 0
    for t in tensors:
        n = t.numel()
        t.copy_(buf[off:off + n].view(t.shape).to(device=t.device, dtype=t.dtype))
        off += n


def _touch_all(optimizer, pres) -> None:
    for pre in pres:
        for node in _nodes(pre):
            if hasattr(node, "_touch"):
                node._touch()
    ws = getattr(optimizer, "_ws", None)
    if ws is not None and hasattr(ws, "invalidate"):
        ws.invalidate()


# --------------------------------------------------------------------------
# broadcast from rank 0 (SCAO.sync_preconditioner)
# --------------------------------------------------------------------------

def broadcast_state(optimizer, process_group=None) -> None:
    """scao/optimizer.py:686-710 with scao/preconditioner.py:647-719: rank 0's
    moments (``exp_avg``, ``exp_avg_sq``, ``exp_avg_diff``), step counters and
    preconditioner state on every rank.  A Kronecker preconditioner whose
    rank differs from rank 0's is resized first; int8 EMA scales travel as
    fp32, as in the reference (which wraps the Python floats in default-dtype
    tensors), so every rank, rank 0 included, ends with fp32-rounded scales;
    a block-diagonal parent's rank is then the mean of its blocks'."""
    import torch.distributed as dist
    states = _states(optimizer)
    pres = [st["preconditioner"] for st in states if st.get("preconditioner") is not None]
    probe = [t for st in states for t in (st.get(k) for k in _MOMENTS) if t is not None]
    dev = _bucket_device(probe, process_group)

    # 1) metadata: step per state, then precond_step (and k for Kronecker
    #    leaves) per preconditioner node
    meta = []
    for st in states:
        if "step" in st:
            meta.append(int(st["step"]))
    for pre in pres:
        for node in _nodes(pre):
            meta.append(int(node.precond_step))
            if node.use_kronecker and not node.use_block_diagonal:
                meta.append(int(node._k))
    n = torch.tensor([len(meta), -len(meta)], dtype=torch.int64, device=dev)
    dist.all_reduce(n, op=dist.ReduceOp.MIN, group=process_group)
    if n[0].item() != -n[1].item():
        raise ValueError("sync_preconditioner: ranks hold different optimizer states "
                         f"({n[0].item()} to {-n[1].item()} entries); every rank must have "
                         "stepped (or loaded a checkpoint) before the broadcast")
    mt = torch.tensor(meta, dtype=torch.int64, device=dev)
    if mt.numel():
        dist.broadcast(mt, src=0, group=process_group)
    vals = iter(mt.tolist())
    for st in states:
        if "step" in st:
            st["step"] = next(vals)
    for pre in pres:
        for node in _nodes(pre):
            node.precond_step = next(vals)
            if node.use_kronecker and not node.use_block_diagonal:
                k = next(vals)
                if k != node._k:
                    node._k = k
                    d = node.device
                    node.U_l = torch.empty(node.m, k, dtype=PRECOND_DTYPE, device=d)
                    node.S_l = torch.empty(k, dtype=PRECOND_DTYPE, device=d)
                    node.U_r = torch.empty(node.n, k, dtype=PRECOND_DTYPE, device=d)
                    node.S_r = torch.empty(k, dtype=PRECOND_DTYPE, device=d)

    # 2) payload: fp32 moments and preconditioner tensors, int8 codes, scales
    f32, i8, scales = [], [], []
    for st in states:
        f32 += [st[k] for k in _MOMENTS if k in st]
    for pre in pres:
        for node in _nodes(pre):
            if node.use_block_diagonal:
                continue
            if node.use_kronecker:
                if node.use_int8_ema:
                    i8 += [node.L_ema_q, node.R_ema_q]
                    scales.append(node)
                else:
                    f32 += [node.L_ema, node.R_ema]
                f32 += [node.U_l, node.S_l, node.U_r, node.S_r]
            else:
                f32.append(node.diag_ema)
    for tensors, dtype in ((f32, torch.float32), (i8, torch.int8)):
        buf = _flat(tensors, dtype, dev)
        if buf is not None:
            dist.broadcast(buf, src=0, group=process_group)
            _unflat(buf, tensors)
    if scales:
        sc = torch.tensor([[n.L_ema_scale, n.R_ema_scale] for n in scales], dtype=torch.float32,
                          device=dev)
        dist.broadcast(sc, src=0, group=process_group)
        for n, (sl, sr) in zip(scales, sc.tolist()):
            n.L_ema_scale, n.R_ema_scale = sl, sr
    # 3) a block-diagonal parent's rank from its (now synced) blocks
    for pre in pres:
        for node in reversed(_nodes(pre)):
            if node.use_block_diagonal:
                node._k = sum(b._k for b in node._blocks) // max(len(node._blocks), 1)
    _touch_all(optimizer, pres)
