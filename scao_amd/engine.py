"""Batched execution of the SCAO step on one ROCm device.

The reference walks parameters and Kronecker blocks one at a time in Python
(scao/optimizer.py:509-645 -> scao/preconditioner.py:457-564), issuing ~10
small ATen calls per block and ~20 full-size elementwise passes per
parameter with several host synchronisations.  Here one step is a fixed
sequence of launches over *all* parameters and blocks at once:

    adam_step          Phase-1 parameters                      (flat chunks)
    kron_project       T = U_l^T G       for every Phase-2 block (256-col strips)
    kron_delta         P = T U_r -> Delta, nu^2                  (k x k tiles)
    kron_lift          W = U_l Delta                             (64-row strips)
    diag_reduce        diagonal-mode Phase-2 parameters
    step_finalize(0)   per-param norms, clip factor, global grad-norm EMA
    kron_apply         G + W U_r^T -> clip -> blend -> Adan -> update
    diag_apply
    step_finalize(1)   LARS trust ratio
    lars_write         p = fma(u, -(lr*trust), p*decay)

No host synchronisation happens inside a non-refresh step.  Descriptor
tables are numpy record arrays uploaded through pinned memory; the task
lists (which depend only on shapes and phases) are cached on the device.

The curvature refresh (``refresh``) batches every block due for an update:
Gram -> EMA -> requantise on the GPU (no host round trip for the int8
scale), then the eigen stage on stacked equal-size matrices
(``scao_amd.eigen.topk_eigh``: the k_max largest eigenpairs and the sum of
the clamped spectrum) and the adaptive-rank choice with one host read of all
ranks.
"""

from __future__ import annotations

import math
import weakref
from dataclasses import dataclass, field
from typing import NamedTuple

import numpy as np
import torch
from torch import Tensor

from . import _lib as L
from . import eigen
from .preconditioner import SparsePreconditioner, leaf_epoch
from .utils import batched_adaptive_rank_topk, to_2d



def _align4(n: int) -> int:
    return (n + 3) & ~3


def _aligned16(*ptrs) -> bool:
    x = 0
    for p in ptrs:
        x |= p
    return x & 15 == 0


def _item_ptrs(it: "PItem") -> tuple:
    """PItem.ptrs: the device addresses a step reads, once per step."""
    st, ms = it.st, it.msrc
    return (it.p.data_ptr(), it.graw.data_ptr(),
            it.gmom.data_ptr() if it.gmom is not None else 0,
            ms.ema.data_ptr() if ms is not None and ms.ema is not None else 0,
            st["exp_avg"].data_ptr(), st["exp_avg_sq"].data_ptr(),
            st["exp_avg_diff"].data_ptr(), st["prev_grad"].data_ptr())


def require_hip(t: Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"scao_amd runs on ROCm devices only: {what} is on '{t.device}'. "
            "Move the model to the GPU (there is no CPU path).")


# --------------------------------------------------------------------------
# per-step parameter record
# --------------------------------------------------------------------------

@dataclass(slots=True)
class PItem:
    """One parameter taking part in a step (host-side bookkeeping)."""
    p: Tensor
    graw: Tensor                 # p.grad (contiguous view)
    gmom: Tensor | None          # filtered/noised fp32 grad for the moments, or None
    st: dict
    group: dict
    pre: SparsePreconditioner
    phase2: bool
    step: int
    scao_step: int = 0
    lars: bool = False
    diag: bool = False           # diagonal-mode preconditioner in Phase 2
    leaves: list = field(default_factory=list)  # [(leaf, r0, c0)]
    fp32: bool = True            # param and gradient are float32
    aligned: bool = True         # every pointer of the param is 16-byte aligned
    msrc: "MomentSource | None" = None   # filter/noise formed inside the step kernels
    # device addresses, read once per step: p, graw, gmom, filter EMA (0 when
    # absent) and the four moments in _MOMENTS order
    ptrs: tuple = ()

    @property
    def mgrad(self) -> bool:
        """The moments see another gradient than p.grad."""
        return self.gmom is not None or self.msrc is not None


PARAM_RING = 4   # parameter-table staging slots (steps the host may run ahead)


class Workspace:
    """Device buffers reused across steps (one per optimizer)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.runtime = torch.tensor([1.0, 0.0], dtype=torch.float64, device=device)
        self._bufs: dict[str, Tensor] = {}
        # moment tensors already checked (contiguous fp32 on the device), per
        # parameter state: weak references, so a replaced tensor is checked again
        self.checked: dict = {}
        # per-parameter shares of the step structure (engine._build_structure)
        self.structures: dict = {}
        # the last RECENT_STRUCTURES whole structures, most recent last
        self.recent: dict = {}
        self.struct_key = None
        self.cheap_key = None
        self.leaf_epoch = -1
        self.tasks: dict[str, Tensor] = {}
        self.ntasks: dict[str, int] = {}
        self.slot_ranges = None
        self.nslots = 0
        self.leaf_dev = None
        self.leaf_index = {}
        self.upd_offsets = {}
        # parameter-table staging: PARAM_RING slots of (pinned host buffer,
        # device buffer, event recorded after the step that last used them)
        self._ring: list = [None] * PARAM_RING
        self._ring_next = 0

    def stage_params(self, raw: np.ndarray) -> Tensor:
        """The step's parameter table on the device, through the next slot of
        the staging ring.  The slot's event was recorded after the kernels of
        the step that last used it (finish_params), so once it has completed
        neither its host buffer (still being copied) nor its device buffer
        (still being read) is in use; in a steady loop that step is
        PARAM_RING steps back and the wait returns at once."""
        nbytes = raw.nbytes
        i = self._ring_next
        self._ring_next = (i + 1) % PARAM_RING
        ent = self._ring[i]
        if ent is None or ent[0].numel() < nbytes:
            cap = max(nbytes, 4096)
            ent = [torch.empty(cap, dtype=torch.uint8, pin_memory=True),
                   torch.empty(cap, dtype=torch.uint8, device=self.device), None]
            self._ring[i] = ent
        elif ent[2] is not None:
            ent[2].synchronize()
        host, dev = ent[0][:nbytes], ent[1][:nbytes]
        host.numpy()[:] = raw.reshape(-1).view(np.uint8)
        dev.copy_(host, non_blocking=True)
        self._ring_slot = ent
        return dev

    def finish_params(self) -> None:
        """Mark the staged table's slot busy until the work enqueued so far
        (the step's kernels) has run."""
        ent = self._ring_slot
        if ent[2] is None:
            ent[2] = torch.cuda.Event()
        ent[2].record()

    def invalidate(self) -> None:
        """Forget the cached step structures (rebuilt on the next step)."""
        self.struct_key = None
        self.cheap_key = None
        self.recent.clear()
        self.structures.clear()

    def buf(self, name: str, nbytes: int) -> Tensor:
        b = self._bufs.get(name)
        if b is None or b.numel() < nbytes:
            b = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self._bufs[name] = b
        return b


# --------------------------------------------------------------------------
# task lists
# --------------------------------------------------------------------------

# Optional per-launch timing: when ``TIMING`` is a dict, every launch of the
# step and of the refresh is bracketed by a pair of events on the launch
# stream and appended under its entry-point name (used by bench.py).
TIMING = None
TIMING_ONLY = None   # optional set of entry-point names to time (None: all)


def _call(name: str, *args) -> None:
    if TIMING is None or (TIMING_ONLY is not None and name not in TIMING_ONLY):
        L.call(name, *args)
        return
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    L.call(name, *args)
    b.record()
    TIMING.setdefault(name, []).append((a, b))


def _mark(name: str):
    """Context manager timing a host-driven stage (e.g. torch eigh) on the stream."""
    class _M:
        def __enter__(self):
            if TIMING is not None:
                self.a = torch.cuda.Event(enable_timing=True)
                self.a.record()

        def __exit__(self, *exc):
            if TIMING is not None:
                b = torch.cuda.Event(enable_timing=True)
                b.record()
                TIMING.setdefault(name, []).append((self.a, b))
    return _M()


def timing_summary() -> dict:
    """{name: (count, mean ms, total ms)} of the recorded events (synchronises)."""
    torch.cuda.synchronize()
    out = {}
    for name, ev in (TIMING or {}).items():
        ms = [a.elapsed_time(b) for a, b in ev]
        out[name] = (len(ms), sum(ms) / len(ms), sum(ms))
    return out


def _flat_chunks(numel: int) -> int:
    return (numel + L.FLAT_CHUNK - 1) // L.FLAT_CHUNK


_LEAF_TASKS = ("delta", "lift")   # with proj* and apply*: idx is a block index
_TASK_TYPES = (["adam", "delta", "lift", "dred", "dapply", "lars"] +
               [f"proj{v}" for v in range(12)] + [f"apply{v}" for v in range(64)])


STEP_WIDTHS = (64, 128, 256)   # eigenfactor widths the step kernels are built for


def _leaf_k(leaf) -> int:
    """Width of a step leaf's eigenfactors in the step: its rank rounded up to
    64, 128 or 256 (beyond 256, to a multiple of 64); 0 for a diagonal
    sub-block.  The reference's adaptive rank moves k by -1..+4 per refresh,
    so most ranks are no multiple of 16; a padded leaf runs the whole-tile
    kernels on zero-padded copies of U_l and U_r (_leaf_table).  The padded
    rows of T and P are zero, so Delta, W and nu^2 are the unpadded ones."""
    if not leaf.use_kronecker:
        return 0
    k = leaf.U_l.shape[1]
    for w in STEP_WIDTHS:
        if k <= w:
            return w
    return -(-k // 64) * 64


def _param_tasks(it: PItem):
    """One parameter's share of a step structure, with local indices: block
    indices from 0 (first block of the parameter), parameter index 0, slots
    from 0.  Returns ({type: int32 array (n, 4)}, local slot ranges, slot
    count, [(leaf, r0, c0)])."""
    tasks = {}

    def add(kind, t):
        tasks.setdefault(kind, []).append(t)

    slot = 0
    leaves = list(it.leaves) if it.phase2 and not it.diag else []
    if not it.phase2:
        for c in range(_flat_chunks(it.p.numel())):
            add("adam", (0, c, 0, slot))
            slot += 1
        rng = (0, slot, slot, slot)
    elif it.diag:
        for c in range(_flat_chunks(it.p.numel())):
            add("dred", (0, c, 0, slot))
            slot += 1
        pre_end = slot
        for c in range(_flat_chunks(it.p.numel())):
            add("dapply", (0, c, 0, slot))
            slot += 1
        rng = (0, pre_end, pre_end, slot)
    else:
        # projection (chunk 0 owns the norm slots)
        for li, (leaf, r0, c0l) in enumerate(leaves):
            if not leaf.use_kronecker:
                continue
            m, n = leaf.m, leaf.n
            k = _leaf_k(leaf)
            vec = _leaf_vec(it, leaf, r0, c0l)
            # the bf16-split tiles address a lane's rows with a 32-bit byte
            # offset: 24 row strides + a strip, below 2^32 for rows under 2^25
            short_rows = _cols(it.p) < (1 << 25)
            for j0 in range(0, n, L.PROJ_COLS):
                whole = (vec and it.fp32 and j0 + L.PROJ_COLS <= n and m % 32 == 0
                         and short_rows)
                # 128 or 256 rows of T per task where k allows (variant bits 4, 8)
                cr = 64
                if whole and k % 128 == 0:
                    cr = 256 if k % 256 == 0 else 128
                for c0 in range(0, k, cr):
                    fast = whole and c0 + 64 <= k
                    do_p = c0 == 0 and it.lars
                    var = ((1 if fast else 0) | (2 if do_p else 0) | (4 if cr == 128 else 0)
                           | (8 if cr == 256 else 0))
                    if c0 == 0:
                        add(f"proj{var}", (li, j0, c0, slot))
                        slot += 1
                    else:
                        add(f"proj{var}", (li, j0, c0, -1))
        for li, (leaf, _, _) in enumerate(leaves):
            if not leaf.use_kronecker:
                # a diagonal sub-block: its norm partials, 64x64 tiles
                for a in range(0, leaf.m, 64):
                    for b in range(0, leaf.n, 64):
                        add("delta", (li, a, b, slot))
                        slot += 1
                continue
            k = _leaf_k(leaf)
            for a in range(0, k, 64):
                for b in range(0, k, 64):
                    add("delta", (li, a, b, slot))
                    slot += 1
        pre_end = slot
        for li, (leaf, r0, c0l) in enumerate(leaves):
            k = _leaf_k(leaf)
            for i0 in range(0, leaf.m, 64):
                for d0 in range(0, k, 64):
                    add("lift", (li, i0, d0, -1))
            var = (1 if it.mgrad else 0) | (2 if it.lars else 0)
            ok = (leaf.use_kronecker and _leaf_vec(it, leaf, r0, c0l) and it.fp32 and it.aligned
                  and k % 16 == 0)
            m, n, T = leaf.m, leaf.n, L.APPLY_TILE
            if ok and k in STRIP_RANKS:
                # runs of strip tiles over the interior they tile exactly
                sw, tr = (64, 128) if k == 256 else (128, 64)   # the kernel's strip_shape
                mw, nw = m - m % tr, n - n % sw
                if not (mw and nw):
                    mw = nw = 0
                wide = var | 4 | 16 | (32 if k == 128 else 0)
                for i0, j0 in _strip_runs(mw, nw, tr, sw):
                    add(f"apply{wide}", (li, i0, j0, slot))
                    slot += min(L.APPLY_GROUP, (mw - i0) // tr)
            else:
                # wide 16x256 tiles over the interior that they tile exactly,
                # masked 64x64 tiles over the right column strip and the
                # bottom row strip
                mw = m - m % L.APPLY_WIDE_ROWS if ok else 0
                nw = n - n % L.APPLY_WIDE_COLS if ok else 0
                if not (mw and nw):
                    mw = nw = 0
                wide = var | 4 | (8 if k >= PIPE_MIN_RANK else 0)
                for i0, j0 in _wide_tiles(mw, nw, k, k >= PIPE_MIN_RANK):
                    add(f"apply{wide}", (li, i0, j0, slot))
                    slot += 1
            for i0 in range(0, m, T):
                for j0 in range(nw, n, T):
                    add(f"apply{var}", (li, i0, j0, slot))
                    slot += 1
            for i0 in range(mw, m, T):
                for j0 in range(0, nw, T):
                    add(f"apply{var}", (li, i0, j0, slot))
                    slot += 1
        rng = (0, pre_end, pre_end, slot)
    if it.phase2 and it.lars:
        for c in range(_flat_chunks(it.p.numel())):
            add("lars", (0, c, 0, -1))
    arrays = {k: np.array(v, dtype=np.int32).reshape(-1, 4) for k, v in tasks.items()}
    return arrays, rng, slot, leaves


def _item_key(it: PItem) -> tuple:
    """Everything _param_tasks reads from an item."""
    return (id(it.p), it.phase2, it.diag, it.lars, it.mgrad, it.p.numel(), it.fp32, it.aligned,
            _cols(it.p), tuple((id(lf), r0, c0, _leaf_k(lf)) for lf, r0, c0 in it.leaves)
            if it.phase2 and not it.diag else ())


def _build_structure(items: list[PItem], cache: dict | None = None):
    """Slots, task lists and the Phase-2 leaf list for a step structure.

    Every reduction slot is written by exactly one task; each parameter's
    pre-finalize slots and post-finalize slots are contiguous ranges.  Each
    parameter's share is built once per configuration (``cache``, keyed by
    the item and the module's tiling settings) and placed by offsets, so a
    step whose set of parameters changes (a parameter without a gradient,
    a rank change) costs array arithmetic, not a rebuild of every tile."""
    knobs = (PIPE_MIN_RANK, L2_OPERANDS, L.APPLY_GROUP)
    if cache is not None and len(cache) > 4 * len(items) + 64:
        cache.clear()
    parts = {k: [] for k in _TASK_TYPES}
    offs = {k: [] for k in _TASK_TYPES}    # (index offset, slot offset, rows) per part
    ranges, leaves = [], []
    slot = 0
    for pi, it in enumerate(items):
        key = (_item_key(it), knobs)
        frag = cache.get(key) if cache is not None else None
        if frag is None:
            frag = _param_tasks(it)
            if cache is not None:
                cache[key] = frag
        arrays, rng, nslot, lvs = frag
        base = len(leaves)
        for kind, arr in arrays.items():
            parts[kind].append(arr)
            offs[kind].append((base if (kind in _LEAF_TASKS or kind.startswith(("proj", "apply")))
                               else pi, slot, len(arr)))
        ranges.append(tuple(x + slot for x in rng))
        leaves.extend((lf, r0, c0, pi) for lf, r0, c0 in lvs)
        slot += nslot
    arrays = {}
    for kind in _TASK_TYPES:
        if parts[kind]:
            a = np.concatenate(parts[kind])
            o = np.array(offs[kind], dtype=np.int64)
            a[:, 0] += np.repeat(o[:, 0], o[:, 2]).astype(np.int32)
            a[:, 3] += np.where(a[:, 3] >= 0, np.repeat(o[:, 1], o[:, 2]), 0).astype(np.int32)
        else:
            a = np.zeros((0, 4), np.int32)
        if kind.startswith("apply") or kind.startswith("proj"):
            grp = L.APPLY_GROUP if kind.startswith("apply") and int(kind[5:]) & 8 else 1
            a = _xcd_interleave(a, grp)
        arrays[kind] = np.ascontiguousarray(a, dtype=np.int32).view(L.TASK).reshape(-1)
    return arrays, ranges, slot, leaves


XCDS = 8   # MI355X: 8 accelerator dies, workgroup i is dispatched to die i % 8
PIPE_MIN_RANK = 128   # wide apply tiles of blocks with k >= this use the pipelined kernel
RECENT_STRUCTURES = 4   # whole step structures kept on the device (run_step)
L2_OPERANDS = 2 << 20   # bytes of W / U_r rows a die's L2 (4 MB) keeps beside the streams


def _wide_tiles(mw: int, nw: int, k: int, pipelined: bool = False) -> list:
    """(i0, j0) of a leaf's wide apply tiles in the order their blocks run.

    A tile reads the W rows of its row band (16 x k) and the U_r rows of its
    column strip (256 x k) from L2.  While a leaf's whole W and U_r fit in
    L2_OPERANDS the tiles go row by row (a block's run of APPLY_GROUP tiles
    crosses the strips of one band, which streams best).  Beyond that (k=256
    at 4096 x 4096: 4 MB each) row-major order makes a die's resident blocks
    cycle through every strip's U_r, and the misses refetch it from HBM.
    Then the tiles go in super-tiles of R bands x S strips, strip by strip,
    with R and S sized so that one super-tile's operands take L2_OPERANDS:
    a block's run stays in one strip and the die shares a few strips.  The
    pipelined kernel's leaves always take that order: it computes two tiles
    of one strip per pass over their U_r rows."""
    rows, cols = L.APPLY_WIDE_ROWS, L.APPLY_WIDE_COLS
    if (mw + nw) * k * 4 <= L2_OPERANDS and not pipelined:
        return [(i0, j0) for i0 in range(0, mw, rows) for j0 in range(0, nw, cols)]
    half = L2_OPERANDS // 2
    s = max(1, half // (cols * k * 4))
    r = max(L.APPLY_GROUP, half // (rows * k * 4) // L.APPLY_GROUP * L.APPLY_GROUP)
    out = []
    for ib in range(0, mw, r * rows):
        for jb in range(0, nw, s * cols):
            for j0 in range(jb, min(nw, jb + s * cols), cols):
                for i0 in range(ib, min(mw, ib + r * rows), rows):
                    out.append((i0, j0))
    return out


STRIP_RANKS = (128, 256)   # ranks of the strip apply kernel (others >= PIPE_MIN_RANK: pipelined)


def _strip_runs(mw: int, nw: int, tr: int, sw: int) -> list:
    """(i0, j0) of a leaf's strip-apply runs: APPLY_GROUP tiles of tr rows
    down one strip of sw columns each, band group by band group and, within
    one, strip by strip, so the workgroups a die runs together share the
    band group's W rows in L2 while each keeps its strip's U_r in LDS."""
    step = L.APPLY_GROUP * tr
    return [(i0, j0) for i0 in range(0, mw, step) for j0 in range(0, nw, sw)]


def _xcd_interleave(tasks: np.ndarray, group: int = 1) -> np.ndarray:
    """Order a launch's tasks (int32 rows: idx, a, b, slot) so that every tile
    of one block runs on the same die: the blocks are dealt to XCDS queues
    (largest first, ties in order of appearance, each to the first
    least-loaded queue), each queue is cut into runs of `group` tasks (the
    tasks one workgroup takes) and the runs are interleaved, so workgroup i
    takes its run from queue i % XCDS while all queues last.  Each die's L2
    then fetches a block's shared operands (U_l; W and U_r) once instead of
    every die doing so.  Only the order changes: tasks, slots and sums are
    the same."""
    n = len(tasks)
    if n <= XCDS * group:
        return tasks
    u, first, inv, cnt = np.unique(tasks[:, 0], return_index=True, return_inverse=True,
                                   return_counts=True)
    app = np.argsort(first, kind="stable")                 # blocks in order of appearance
    srt = app[np.argsort(-cnt[app], kind="stable")]        # largest first
    queue = np.empty(len(u), dtype=np.int64)
    rank = np.empty(len(u), dtype=np.int64)
    qlen = [0] * XCDS
    for r, j in enumerate(srt.tolist()):
        q = min(range(XCDS), key=qlen.__getitem__)
        queue[j], rank[j] = q, r
        qlen[q] += int(cnt[j])
    tq, tr = queue[inv], rank[inv]
    o1 = np.lexsort((np.arange(n), tr, tq))               # each queue's tasks in order
    q1 = tq[o1]
    starts = np.concatenate(([0], np.cumsum(np.bincount(q1, minlength=XCDS))[:-1]))
    pos = np.arange(n) - starts[q1]                       # position inside its queue
    o2 = np.lexsort((pos, q1, pos // group))              # run by run, queue by queue
    return tasks[o1][o2]


def _cols(t: Tensor) -> int:
    """Columns of to_2d(t) (1-D: n; N-D: prod(shape[1:])), without a view."""
    shape = t.shape
    if len(shape) == 1:
        return shape[0]
    if len(shape) == 2 or shape[0] == 0:
        return shape[1] if len(shape) == 2 else to_2d(t)[0].shape[1]
    return math.prod(shape[1:])


def _leaf_vec(it: PItem, leaf, r0: int, c0: int) -> bool:
    """float4 access is legal for the block: 4-aligned origin, row stride and width."""
    cols = _cols(it.p)
    return ((r0 * cols + c0) % 4 == 0 and cols % 4 == 0 and leaf.n % 4 == 0
            and it.aligned)


def _padded_factors(leaves, ws: Workspace) -> dict:
    """{leaf index: (U_l, U_r, S_l, S_r)} padded to _leaf_k columns for the
    leaves whose rank is below it: U's extra columns zero, S's extra entries
    1.0 (finite, so (s_l s_r - 1) * 0 stays 0).  Written on the current
    stream, ahead of the step's kernels, each time the block table is built
    (any change to the factors moves leaf_epoch, which rebuilds it)."""
    need = []
    for i, (leaf, *_r) in enumerate(leaves):
        if leaf.use_kronecker and _leaf_k(leaf) != leaf.U_l.shape[1]:
            need.append(i)
    if not need:
        return {}
    sizes = []
    for i in need:
        leaf, kp = leaves[i][0], _leaf_k(leaves[i][0])
        sizes.append((_align4(leaf.m * kp), _align4(leaf.n * kp), _align4(kp), _align4(kp)))
    buf = ws.buf("leaf_pad", sum(map(sum, sizes)) * 4).view(torch.float32)
    out, off = {}, 0
    for i, sz in zip(need, sizes):
        leaf, kp = leaves[i][0], _leaf_k(leaves[i][0])
        k = leaf.U_l.shape[1]
        views = []
        for (src, rows), n in zip(((leaf.U_l, leaf.m), (leaf.U_r, leaf.n), (leaf.S_l, 1),
                                   (leaf.S_r, 1)), sz):
            v = buf[off:off + rows * kp].view(rows, kp) if src.ndim == 2 else buf[off:off + kp]
            if src.ndim == 2:
                v.zero_()
                v[:, :k].copy_(src)
            else:
                v.fill_(1.0)
                v[:k].copy_(src)
            views.append(v)
            off += n
        out[i] = tuple(views)
    return out


def _leaf_table(leaves, items: list[PItem], ws: Workspace):
    """Block descriptors plus T/Delta/W scratch for every Phase-2 block."""
    sizes = []
    for (leaf, r0, c0, pi) in leaves:
        k = _leaf_k(leaf)
        # W, then (strip-apply ranks) its three bf16 planes: 1.5 floats per element
        wsz = _align4(leaf.m * k) + (_align4((3 * leaf.m * k + 1) // 2) if k in STRIP_RANKS else 0)
        sizes.append((_align4(k * leaf.n), _align4(k * k), wsz))
    total = sum(a + b + c for a, b, c in sizes)
    scratch = ws.buf("leaf_scratch", max(total, 1) * 4)
    base = scratch.data_ptr()
    pads = _padded_factors(leaves, ws)
    tab = np.zeros(len(leaves), dtype=L.LEAF_DESC)
    off = 0
    for i, ((leaf, r0, c0, pi), (st, sd, sw)) in enumerate(zip(leaves, sizes)):
        it = items[pi]
        cols = it.graw.shape[-1] if it.graw.ndim == 2 else to_2d(it.graw)[0].shape[1]
        e = tab[i]
        e["off"] = r0 * cols + c0
        e["ld"] = cols
        e["param"] = pi
        if not leaf.use_kronecker:
            # diagonal sub-block: its EMA in Sl, the bias factor in dbias
            e["Sl"] = leaf.diag_ema.data_ptr()
            e["m"], e["n"], e["k"] = leaf.m, leaf.n, 0
            e["flags"] = L.LF_DIAG
            e["dbias"] = getattr(leaf, "_diag_bias_factor", 1.0)
            continue
        k = _leaf_k(leaf)
        if k == leaf.U_l.shape[1]:
            e["Ul"], e["Ur"] = leaf.U_l.data_ptr(), leaf.U_r.data_ptr()
            e["Sl"], e["Sr"] = leaf.S_l.data_ptr(), leaf.S_r.data_ptr()
        else:
            ul, ur, sl, sr = pads[i]
            e["Ul"], e["Ur"], e["Sl"], e["Sr"] = (ul.data_ptr(), ur.data_ptr(), sl.data_ptr(),
                                                  sr.data_ptr())
        e["T"] = base + 4 * off
        e["Delta"] = base + 4 * (off + st)
        e["W"] = base + 4 * (off + st + sd)
        e["Wb"] = base + 4 * (off + st + sd + _align4(leaf.m * k)) if k in STRIP_RANKS else 0
        off += st + sd + sw
        e["m"], e["n"], e["k"] = leaf.m, leaf.n, k
        vec = _leaf_vec(it, leaf, r0, c0) and _aligned16(int(e["T"]))
        e["flags"] = L.LF_VEC4 if vec else 0
    return tab


# --------------------------------------------------------------------------
# the step
# --------------------------------------------------------------------------

_MOMENTS = ("exp_avg", "exp_avg_sq", "exp_avg_diff", "prev_grad")


def _group_scalars(g: dict, t: int, phase2: bool, scao_step: int, lars: bool,
                   gsnr: float | None) -> tuple:
    """The descriptor fields every parameter of a group shares at one step:
    (lr .. gsnr), (adam_sqrt_bc2, adam_alpha) and the group's flags."""
    lr = g["lr"]
    beta1, beta2 = g["betas"]
    beta3 = g["beta3"]
    wd = g["weight_decay"]
    flags = L.PF_NORM
    decay = 1.0
    if wd != 0.0:
        flags |= L.PF_DECAY
        decay = 1.0 - lr * wd
    bc1 = bc2 = bc3 = blend = omb = tau = lv = wdv = gs = sq = alpha = 0.0
    if not phase2:
        sq, alpha = math.sqrt(1.0 - beta2 ** t), -(lr / (1.0 - beta1 ** t))
    else:
        bc1, bc2, bc3 = 1.0 - beta1 ** t, 1.0 - beta2 ** t, 1.0 - beta3 ** t
        bsteps = g.get("blend_steps", 50)
        blend = min(1.0, scao_step / bsteps) if bsteps > 0 else 1.0
        omb = 1.0 - blend
        if g["tau"] is not None:
            flags |= L.PF_CLIP
            tau = g["tau"]
        if lars:
            flags |= L.PF_LARS
            lv, wdv = g["lars_coeff"], wd
        if gsnr is not None:
            flags |= L.PF_GSNR
            gs = gsnr
    head = (lr, decay, beta1, 1.0 - beta1, beta2, 1.0 - beta2, beta3, 1.0 - beta3, bc1, bc2,
            bc3, blend, omb, g["eps"], tau, lv, wdv, gs)
    return head, (sq, alpha), flags


def _desc_blocks():
    """Byte ranges of scao_param_desc's runs of same-typed fields: 64-bit
    addresses and sizes (p .. cols), lr (double), the fp32 scalars (decay ..
    adam_alpha), the int32 fields (dtype .. norm_index) and fnoise."""
    f = L.PARAM_DESC.fields
    names = list(L.PARAM_DESC.names)

    def run(first, last, size):
        i, j = names.index(first), names.index(last)
        for a, b in zip(names[i:j], names[i + 1:j + 1]):
            assert f[b][1] == f[a][1] + size, (a, b)
        return f[first][1], f[last][1] + size, j - i + 1

    blocks = {"u8": run("p", "cols", 8), "f8": run("lr", "lr", 8),
              "f4": run("decay", "adam_alpha", 4), "i4": run("dtype", "norm_index", 4),
              "fnoise": run("fnoise", "fnoise", 4)}
    assert names[-1] == "fnoise" and blocks["fnoise"][1] <= L.PARAM_DESC.itemsize
    assert names.index("decay") == names.index("lr") + 1
    assert names.index("dtype") == names.index("adam_alpha") + 1
    return blocks


_BLOCKS = _desc_blocks()
_DBIAS = list(L.PARAM_DESC.names).index("diag_bias") - list(L.PARAM_DESC.names).index("decay")


def _param_table(items: list[PItem], ranges, ws: Workspace, gsnr: float | None):
    """The per-step parameter descriptors (scao_param_desc records).  The
    device addresses come from ``it.ptrs``; scalars shared by a group at one
    step are computed once and written to all its rows together.

    Scalars are Python floats rounded to fp32 by the float32 columns (the
    same round-to-nearest ATen applies to a scalar operand of an fp32 op)."""
    n = len(items)
    upd_base = ws.buf("upd", 4).data_ptr() if ws.upd_total else 0
    f32 = torch.float32
    shared: dict = {}
    u8rows, i4rows, fnoise, dbias = [], [], [], []
    for i, it in enumerate(items):
        st, p = it.st, it.p
        pp, graw, gmom, fema, m0, m1, m2, m3 = it.ptrs
        # per parameter, kept while the parameter and its moment tensors are
        # the same objects: the moments' check, numel, columns, dtype code
        seen = ws.checked.get(id(st))
        if (seen is None or seen[0]() is not st["exp_avg"] or seen[1]() is not st["exp_avg_sq"]
                or seen[2]() is not st["exp_avg_diff"] or seen[3]() is not st["prev_grad"]
                or seen[4]() is not p):
            dev = p.device
            moms = [st[key] for key in _MOMENTS]
            for key, m in zip(_MOMENTS, moms):
                if m.dtype != f32 or not m.is_contiguous() or m.device != dev:
                    raise ValueError(f"state[{key!r}] must be a contiguous float32 tensor on "
                                     f"{dev}; got {m.dtype} on {m.device}")
            seen = ws.checked[id(st)] = (*(weakref.ref(m) for m in moms), weakref.ref(p),
                                         p.numel(), _cols(p), L.DTYPE_CODE[p.dtype])
        lars = it.phase2 and it.lars
        skey = (id(it.group), it.step, it.phase2, it.scao_step if it.phase2 else 0, lars)
        sc = shared.get(skey)
        if sc is None:
            sc = shared[skey] = list(_group_scalars(it.group, it.step, it.phase2, it.scao_step,
                                                    lars, gsnr)) + [[]]
        sc[3].append(i)
        flags = sc[2]
        if gmom:
            flags |= L.PF_GF32
        fthr = fseed = 0
        fn = 0.0
        ms = it.msrc
        if ms is not None:
            flags |= L.PF_GF32
            if ms.ema is not None:
                flags |= L.PF_FMASK
                fthr = ms.thr
            if ms.noise > 0.0:
                flags |= L.PF_FNOISE
                fseed, fn = ms.seed, ms.noise
        upd = diag = 0
        if lars:
            upd = upd_base + 4 * ws.upd_offsets[i]
        if it.phase2 and it.diag:
            flags |= L.PF_DIAG
            diag = it.pre.diag_ema.data_ptr()
            dbias.append((i, getattr(it.pre, "_diag_bias_factor", 1.0)))
        if it.aligned:
            flags |= L.PF_ALIGNED
        u8rows.append((pp, gmom or graw, graw, m0, m1, m2, m3, upd, diag, fema, fthr, fseed,
                       seen[5], seen[6]))
        r = ranges[i]
        i4rows.append((seen[7], flags, r[0], r[1], r[2], r[3], i))
        fnoise.append(fn)
    raw = np.zeros((n, L.PARAM_DESC.itemsize), dtype=np.uint8)

    def cols(block, dt):
        a, b, _ = _BLOCKS[block]
        return raw[:, a:b].view(dt)

    cols("u8", np.uint64)[:] = np.array(u8rows, dtype=np.uint64)
    cols("i4", np.int32)[:] = np.array(i4rows, dtype=np.int32)
    cols("fnoise", np.float32)[:, 0] = np.array(fnoise, dtype=np.float32)
    f8, f4 = cols("f8", np.float64), cols("f4", np.float32)
    for head, tail, _, rows in shared.values():
        f8[rows, 0] = head[0]
        f4[rows] = np.array(head[1:] + (0.0,) + tail, dtype=np.float32)
    for i, v in dbias:
        f4[i, _DBIAS] = v
    # rows sharing a group's step scalars: (group, step, phase2, scao_step,
    # lars, rows, flags of each row beyond the group's)
    classes = []
    for (gid, t, ph2, ss, lars), (_, _, gflags, rows) in shared.items():
        rows = np.array(rows, dtype=np.int64)
        extra = cols("i4", np.int32)[rows, 1] & ~np.int32(gflags)
        classes.append(StepClass(items[int(rows[0])].group, t, ph2, ss, lars, rows, extra))
    return raw, classes


@dataclass(slots=True)
class StepClass:
    """Rows of a step's parameter table that share a group's step scalars."""
    group: dict
    step: int
    phase2: bool
    scao_step: int
    lars: bool
    rows: np.ndarray
    extra_flags: np.ndarray   # per-row flags beyond the group's (alignment, diagonal mode)


@dataclass(slots=True)
class StepPlan:
    """What a plain step (no refresh, no filter or noise, no host norms)
    leaves for the next one: its items, its parameter table and the rows'
    classes.  While the same parameters step again with gradients of the
    same layout, the next step only rewrites the gradient addresses and each
    class's step scalars (run_planned_step)."""
    items: list
    raw: np.ndarray
    classes: list
    gsnr: float | None
    epoch: int
    moments: list   # per item: the four moment tensors the table points at
    min_pre: list | None = None   # per class: the smallest precond_step of its rows


def _set_class_scalars(raw: np.ndarray, cl: StepClass, gsnr) -> None:
    head, tail, gflags = _group_scalars(cl.group, cl.step, cl.phase2, cl.scao_step, cl.lars,
                                        gsnr)
    a8, b8, _ = _BLOCKS["f8"]
    a4, b4, _ = _BLOCKS["f4"]
    ai, bi, _ = _BLOCKS["i4"]
    raw[cl.rows, a8:b8].view(np.float64)[:, 0] = head[0]
    f4 = raw[:, a4:b4].view(np.float32)
    dbias = f4[cl.rows, _DBIAS].copy()
    f4[cl.rows] = np.array(head[1:] + (0.0,) + tail, dtype=np.float32)
    f4[cl.rows, _DBIAS] = dbias
    raw[:, ai:bi].view(np.int32)[cl.rows, 1] = cl.extra_flags | np.int32(gflags)


def run_step(items: list[PItem], ws: Workspace, update_norm_ema: bool,
             gsnr: float | None = None) -> "StepPlan | None":
    """Launch one optimizer step for ``items`` (all on ws.device); returns
    the step's plan (see StepPlan)."""
    if not items:
        return None
    dev = ws.device
    f32 = torch.float32
    for it in items:
        it.fp32 = it.p.dtype == f32 and it.graw.dtype == f32
        it.ptrs = _item_ptrs(it)
        it.aligned = _aligned16(*it.ptrs)
    # the full structure key (with every block's rank) is only rebuilt when
    # the cheap one or the global factor epoch says something may have changed
    ckey = (tuple((id(it.p), it.phase2, it.diag, it.lars, it.mgrad, it.p.numel(),
                   it.fp32, it.aligned, len(it.leaves)) for it in items), leaf_epoch())
    skey = ws.struct_key
    if ckey != ws.cheap_key:
        skey = tuple((id(it.p), it.phase2, it.diag, it.lars, it.mgrad, it.p.numel(),
                      it.fp32, it.aligned,
                      tuple((id(lf), r0, c0, _leaf_k(lf)) for lf, r0, c0 in it.leaves))
                     for it in items)
        ws.cheap_key = ckey
    if skey != ws.struct_key:
        # the last few structures stay on the device (their task lists hold
        # indices only, and their leaf lists keep the blocks alive, so a key
        # cannot be reused by other blocks); the block table, which holds
        # addresses, is rebuilt on every switch
        ent = ws.recent.pop(skey, None)
        if ent is None:
            arrays, ranges, nslots, leaves = _build_structure(items, ws.structures)
            upd_offsets, off = {}, 0
            for i, it in enumerate(items):
                if it.phase2 and it.lars:
                    upd_offsets[i] = off
                    off += _align4(it.p.numel())
            ent = ({k: (L.upload(v, dev) if len(v) else None) for k, v in arrays.items()},
                   {k: len(v) for k, v in arrays.items()}, ranges, nslots, leaves, upd_offsets,
                   off)
        ws.recent[skey] = ent
        while len(ws.recent) > RECENT_STRUCTURES:
            ws.recent.pop(next(iter(ws.recent)))
        (ws.tasks, ws.ntasks, ws.slot_ranges, ws.nslots, ws.leaves, ws.upd_offsets,
         ws.upd_total) = ent
        ws.struct_key = skey
        ws.leaf_epoch = -1
    if ws.upd_total:
        ws.buf("upd", ws.upd_total * 4)
    # the block table holds no gradient pointer: a gradient that moves keeps
    # it valid (its alignment is part of the structure key)
    if ws.leaf_epoch != leaf_epoch() or ws.leaf_dev is None:
        tab = _leaf_table(ws.leaves, items, ws)
        ws.leaf_dev = L.upload(tab, dev) if len(tab) else None
        ws.leaf_epoch = leaf_epoch()
    raw, classes = _param_table(items, ws.slot_ranges, ws, gsnr)
    _launch_step(ws, raw, len(items), update_norm_ema)
    ws.last_items = [it.p for it in items]   # row i of the "stat" buffer is items[i]
    return StepPlan(items, raw, classes, gsnr, leaf_epoch(),
                    [tuple(it.st[key] for key in _MOMENTS) for it in items])


def run_planned_step(plan: StepPlan, gptrs: np.ndarray, ws: Workspace,
                     update_norm_ema: bool) -> None:
    """The next plain step of ``plan``'s parameters: every step counter has
    advanced by one (the caller checked that no refresh or phase change is
    due and that the gradients have the planned layout), the gradients are
    at ``gptrs``.  Rewrites those addresses and the classes' step scalars in
    the table and launches the same kernels as run_step."""
    raw = plan.raw
    a, b, _ = _BLOCKS["u8"]
    u8 = raw[:, a:b].view(np.uint64)
    u8[:, 1] = gptrs   # gradient the moments see (no filter or noise)
    u8[:, 2] = gptrs   # raw gradient
    for cl in plan.classes:
        cl.step += 1
        if cl.phase2:
            cl.scao_step += 1
        _set_class_scalars(raw, cl, plan.gsnr)
    _launch_step(ws, raw, len(plan.items), update_norm_ema)


def _launch_step(ws: Workspace, raw: np.ndarray, n: int, update_norm_ema: bool) -> None:
    """Upload the parameter table and launch one step's kernels."""
    dev = ws.device
    params = ws.stage_params(raw)
    slots = ws.buf("slots", max(ws.nslots, 1) * 8 * L.SLOT_WIDTH)
    stat = ws.buf("stat", n * L.PARAM_STAT.itemsize)
    s = L.stream_ptr(dev)
    T, N = ws.tasks, ws.ntasks
    P, S, SL = params.data_ptr(), stat.data_ptr(), slots.data_ptr()
    LF = ws.leaf_dev.data_ptr() if ws.leaf_dev is not None else 0

    def tp(name):
        return T[name].data_ptr() if T[name] is not None else 0

    if N["adam"]:
        _call("scao_adam_step", tp("adam"), N["adam"], P, SL, s)
    for var in range(12):
        if N[f"proj{var}"]:
            _call("scao_kron_project", tp(f"proj{var}"), N[f"proj{var}"], LF, P, SL, var, s)
    if N["delta"]:
        _call("scao_kron_delta", tp("delta"), N["delta"], LF, P, SL, s)
        _call("scao_kron_lift", tp("lift"), N["lift"], LF, s)
    if N["dred"]:
        _call("scao_diag_reduce", tp("dred"), N["dred"], P, SL, s)
    _call("scao_step_finalize", P, n, SL, S, ws.runtime.data_ptr(), 0,
           1 if update_norm_ema else 0, n, s)
    for var in range(64):
        if N[f"apply{var}"]:
            _call("scao_kron_apply", tp(f"apply{var}"), N[f"apply{var}"], LF, P, S, SL, var, s)
    if N["dapply"]:
        _call("scao_diag_apply", tp("dapply"), N["dapply"], P, S, SL, s)
    if N["lars"]:
        _call("scao_step_finalize", P, n, SL, S, 0, 1, 0, n, s)
        _call("scao_lars_write", tp("lars"), N["lars"], P, S, s)
    ws.finish_params()


# --------------------------------------------------------------------------
# sparse gradient filter (reference scao/optimizer.py:42-57)
# --------------------------------------------------------------------------

_FILTER_TASKS: dict = {}


def _filter_tasks(numels: tuple, dev) -> Tensor:
    """Device task list (desc, chunk) for a tuple of element counts, cached."""
    key = (numels, str(dev))
    t = _FILTER_TASKS.get(key)
    if t is None:
        counts = np.array([_flat_chunks(n) for n in numels], dtype=np.int64)
        arr = np.zeros((int(counts.sum()), 4), dtype=np.int32)
        arr[:, 0] = np.repeat(np.arange(len(numels), dtype=np.int32), counts)
        starts = np.repeat(np.cumsum(counts) - counts, counts)
        arr[:, 1] = np.arange(int(counts.sum()), dtype=np.int64) - starts
        arr[:, 3] = -1
        t = L.upload(arr.view(L.TASK).reshape(-1), dev)
        if len(_FILTER_TASKS) > 16:
            _FILTER_TASKS.clear()
        _FILTER_TASKS[key] = t
    return t


def _filter_scratch(f, numel: int, dev) -> None:
    """The filter's device scratch on ``dev``: ``work`` (selection state,
    zero before the first call) and ``cand``, the candidate buffer (half a
    float per element, plus four counts per chunk): it holds the keys of the
    top-digit bin (a quarter octave) the previous threshold fell in, so the
    last refinement pass of a steady filter reads about a tenth of the EMA."""
    if getattr(f, "work", None) is None or f.work.device != dev:
        f.work = torch.zeros(L.FILTER_WORK_WORDS, dtype=torch.int32, device=dev)
        f.cand = None
    cap = _flat_chunks(numel) * (L.FILTER_REGION + 4)
    if getattr(f, "cand", None) is None or f.cand.numel() != cap:
        f.cand = torch.empty(cap, dtype=torch.float32, device=dev)


def moment_grads(entries, noise_std: float = 0.0) -> list:
    """The gradient the moments see, for [(filter or None, grad)], in one
    batched launch sequence (reference scao/optimizer.py:533-545): the sparse
    filter where a filter is given, then ``noise_std * N(0, 1)`` when
    noise_std > 0.  A filter carries ``mag_ema`` (None before its first call),
    ``work`` (zeroed device scratch, allocated here), ``ema`` and
    ``sparsity``.  Gradients must be contiguous and on one ROCm device; each
    result is a new fp32 tensor of the gradient's shape."""
    keep = [(f, g) for f, g in entries if g.numel() > 0]
    if not keep:
        return [torch.empty(g.shape, dtype=torch.float32, device=g.device) for _, g in entries]
    dev = keep[0][1].device
    n = len(keep)
    outs = []
    cols = {k: [] for k in ("g", "ema", "out", "work", "seed", "numel", "decay", "omd", "q",
                            "dtype", "flags", "cand", "cap")}
    noisy = noise_std > 0.0
    seeds = (torch.randint(0, 2 ** 62, (n,), dtype=torch.int64, device=dev) if noisy else None)
    for i, (f, g) in enumerate(keep):
        require_hip(g, "moment gradient")
        out = torch.empty(g.shape, dtype=torch.float32, device=dev)
        outs.append(out)
        flags, ema, work, decay, omd, q = 0, 0, 0, 0.0, 0.0, 0.0
        if f is not None:
            flags = L.FILTER_MASK
            if f.mag_ema is None:
                f.mag_ema = torch.empty(g.shape, dtype=torch.float32, device=dev)
                flags |= L.FILTER_FIRST
            _filter_scratch(f, g.numel(), dev)
            ema, work = f.mag_ema.data_ptr(), f.work.data_ptr()
            decay, omd, q = f.ema, 1.0 - f.ema, f.sparsity
        cols["g"].append(g.data_ptr())
        cols["ema"].append(ema)
        cols["out"].append(out.data_ptr())
        cols["work"].append(work)
        cols["seed"].append(seeds.data_ptr() + 8 * i if noisy else 0)
        cols["numel"].append(g.numel())
        cols["decay"].append(decay)
        cols["omd"].append(omd)
        cols["q"].append(q)
        cols["dtype"].append(L.DTYPE_CODE[g.dtype])
        cols["flags"].append(flags)
        cand = f.cand if f is not None else None
        cols["cand"].append(cand.data_ptr() if cand is not None else 0)
        cols["cap"].append(cand.numel() if cand is not None else 0)
    descs = np.zeros(n, dtype=L.FILTER_DESC)
    for k, v in cols.items():
        descs[k] = np.asarray(v, dtype=descs.dtype.fields[k][0])
    descs["noise"] = noise_std if noisy else 0.0
    tasks = _filter_tasks(tuple(int(g.numel()) for _, g in keep), dev)
    dd = L.upload(descs, dev)
    _call("scao_sparse_filter", tasks.data_ptr(), tasks.numel() // L.TASK.itemsize,
          dd.data_ptr(), n, L.stream_ptr(dev))
    it = iter(outs)
    return [next(it) if g.numel() > 0 else torch.empty(g.shape, dtype=torch.float32, device=g.device)
            for _, g in entries]


def lookahead(pairs, alpha: float) -> None:
    """slow = slow + alpha * (p - slow); p = slow for [(p, slow)] in one launch
    (reference scao/optimizer.py:356-365).  Tensors contiguous, same dtype,
    on one ROCm device."""
    pairs = [(p, w) for p, w in pairs if p.numel() > 0]
    if not pairs:
        return
    dev = pairs[0][0].device
    descs = np.zeros(len(pairs), dtype=L.LOOKAHEAD_DESC)
    for i, (p, w) in enumerate(pairs):
        require_hip(p, "lookahead parameter")
        if w.dtype != p.dtype or w.shape != p.shape or not (p.is_contiguous() and w.is_contiguous()):
            raise ValueError("lookahead: slow weights must match the parameter")
        descs[i]["p"], descs[i]["slow"] = p.data_ptr(), w.data_ptr()
        descs[i]["numel"], descs[i]["dtype"] = p.numel(), L.DTYPE_CODE[p.dtype]
    tasks = _filter_tasks(tuple(int(p.numel()) for p, _ in pairs), dev)
    dd = L.upload(descs, dev)
    _call("scao_lookahead", tasks.data_ptr(), tasks.numel() // L.TASK.itemsize, dd.data_ptr(),
          alpha, L.stream_ptr(dev))


class MomentSource(NamedTuple):
    """Where the step kernels find the moment gradient's ingredients: the
    filter's EMA (or None) and the device addresses of its threshold and of
    the noise key.  ``keep`` holds the tensors those addresses point into."""
    ema: Tensor | None
    thr: int
    seed: int
    noise: float
    keep: tuple


def moment_sources(entries, noise_std: float = 0.0) -> list:
    """Like ``moment_grads`` but without writing the moment gradients: the
    filter's EMA and threshold are computed (one batched launch, output pass
    skipped) and the step kernels form fp32(g) * (ema >= t) + noise
    themselves from them (SCAO_PF_FMASK / SCAO_PF_FNOISE).  Returns one
    MomentSource per entry."""
    entries = list(entries)
    if not entries:
        return []
    dev = entries[0][1].device
    noisy = noise_std > 0.0
    seeds = (torch.randint(0, 2 ** 62, (len(entries),), dtype=torch.int64, device=dev)
             if noisy else None)
    launch = [(i, f, g) for i, (f, g) in enumerate(entries) if f is not None and g.numel() > 0]
    if launch:
        n = len(launch)
        descs = np.zeros(n, dtype=L.FILTER_DESC)
        for j, (_, f, g) in enumerate(launch):
            require_hip(g, "moment gradient")
            flags = L.FILTER_MASK
            if f.mag_ema is None:
                f.mag_ema = torch.empty(g.shape, dtype=torch.float32, device=dev)
                flags |= L.FILTER_FIRST
            _filter_scratch(f, g.numel(), dev)
            e = descs[j]
            e["g"], e["ema"], e["out"] = g.data_ptr(), f.mag_ema.data_ptr(), 0
            e["work"] = f.work.data_ptr()
            e["numel"] = g.numel()
            e["decay"], e["omd"], e["q"] = f.ema, 1.0 - f.ema, f.sparsity
            e["dtype"] = L.DTYPE_CODE[g.dtype]
            e["flags"] = flags
            if f.cand is not None:
                e["cand"], e["cap"] = f.cand.data_ptr(), f.cand.numel()
        tasks = _filter_tasks(tuple(int(g.numel()) for _, _, g in launch), dev)
        dd = L.upload(descs, dev)
        _call("scao_sparse_filter", tasks.data_ptr(), tasks.numel() // L.TASK.itemsize,
              dd.data_ptr(), n, L.stream_ptr(dev))
    out = []
    for i, (f, g) in enumerate(entries):
        ema = f.mag_ema if f is not None and g.numel() > 0 else None
        thr = f.work.data_ptr() + 4 * L.FILTER_THR_WORD if ema is not None else 0
        seed = seeds.data_ptr() + 8 * i if noisy else 0
        keep = tuple(x for x in (ema, f.work if ema is not None else None, seeds)
                     if x is not None)
        out.append(MomentSource(ema, thr, seed, noise_std if noisy else 0.0, keep))
    return out


def sparse_filter(entries) -> list:
    """The sparse filter alone for [(filter, grad)] (no noise)."""
    return moment_grads(entries, 0.0)


# --------------------------------------------------------------------------
# curvature refresh
# --------------------------------------------------------------------------

REFRESH_SCRATCH_BYTES = 2 << 30   # fp32 EMA staging per refresh chunk (int8 mode)
# The eigen stage runs scao_amd.eigen.topk_eigh (two-stage reduction,
# bisection, inverse iteration: only the k_max vectors a factor can keep) for
# the sizes eigen.solver_fits accepts (up to 4096 rows), and
# torch.linalg.eigh on the device (rocSOLVER syevd) for the others.  Factors
# whose eigh input is exactly diagonal, up to DIAG_MAX_DIM rows, take the
# closed form of scao_eig_diag instead.
DIAG_MAX_DIM = 4096 + L.EIG_BAND
EIGEN_BATCH_BYTES = 8 << 30       # stacked eigen-stage inputs per launch (HIP solver), at most
EIGEN_BATCH_FREE_FRACTION = 4     # ... and at most 1/4 of the device memory free at the refresh
EIGH_BATCH_BYTES = 1 << 30        # stacked eigh inputs per launch (library solver)
# Optional callable run between a refresh's EMA update and its eigen stage,
# with the list of (block, gradient, offset, row stride) being refreshed.  Used
# by the parity tests to check the new EMA and then continue from the CPU
# reference's own post-EMA state, so the eigen stage and the step that follows
# are compared from identical inputs.
AFTER_EMA_HOOK = None
# Optional callable run after a refresh's eigen stage, rank selection and
# truncation, with the same list: the parity tests check the new eigenfactors
# against the CPU reference's and continue from the reference's, where a
# solver's freedom (the basis of a cluster, float32 rounding of eigenvectors)
# would otherwise carry into the steps that follow.
AFTER_EIGEN_HOOK = None
# factors per eigen-stage route in the last refresh (reported by bench.py)
LAST_REFRESH_ROUTES: dict = {}


def eigen_route(dim: int, diagonal: bool) -> str:
    """Which solver takes an n x n factor: "diag" (exactly diagonal input up
    to DIAG_MAX_DIM rows, closed form), "hip" (the batched HIP solver, sizes
    eigen.solver_fits accepts) or "library" (torch.linalg.eigh on the
    device)."""
    if diagonal and dim <= DIAG_MAX_DIM:
        return "diag"
    return "hip" if eigen.solver_fits(dim) else "library"


# The batched solver has a latency floor (its panel loop and bulge chasing
# run the same number of steps for one matrix as for hundreds: 61 ms at
# 2048^2, 205 ms at 4096^2); the library eigh takes 42 / 109 ms for one
# matrix and about as long as the batched solver for four.  A batch of at
# most this many matrices of at least 2048 rows goes to the library.
LIBRARY_SMALL_BATCH = 2


def batch_route(route: str, dim: int, count: int) -> str:
    """The route of a dimension's batch of ``count`` factors that
    eigen_route sent to ``route``."""
    if route == "hip" and count <= LIBRARY_SMALL_BATCH and dim >= 2048:
        return "library"
    return route


def refresh(entries, eigen_only: bool = False, ema_only: bool = False) -> None:
    """update_curvature for several preconditioners at once.

    ``entries``: list of (SparsePreconditioner, grad tensor).  Follows
    scao/preconditioner.py:297-451: precond_step bookkeeping, the EMA update
    (Gram on MFMA, int8 requantisation on the device), bias correction,
    Tikhonov shift, eigh, flip/clamp, adaptive rank with rank momentum.
    ``eigen_only`` skips the EMA update (the curvature factors are taken as
    they are) and ``ema_only`` the eigen stage -- used to check each stage in
    isolation."""
    if not entries:
        return
    dev = entries[0][1].device
    kron, diag = [], []
    for pre, grad in entries:
        require_hip(grad, "gradient")
        if grad.is_sparse:
            raise RuntimeError("SCAO does not support sparse gradients.")
        g = grad.detach()
        if not g.is_contiguous():
            g = g.contiguous()
        pre._bump_steps()
        if pre.use_block_diagonal or pre.use_kronecker:
            g2 = to_2d(g)[0]
            cols = g2.shape[1]
            for leaf, r0, c0 in pre.leaves(diag=True):
                if leaf.use_kronecker:
                    kron.append((leaf, g, r0 * cols + c0, cols))
                else:
                    # a diagonal sub-block (1-wide remainder): its slice of the
                    # gradient, gathered contiguous (reference :316-339)
                    diag.append((leaf, g2[r0:r0 + leaf.m, c0:c0 + leaf.n].contiguous()))
        else:
            diag.append((pre, g))
    s = L.stream_ptr(dev)
    if diag and not eigen_only:
        _refresh_diag(diag, dev, s)
    if kron:
        _refresh_kron(kron, dev, s, eigen_only, ema_only)
    for pre, _ in entries:
        pre._sync_k()


def _refresh_diag(diag, dev, s):
    tab = np.zeros(len(diag), dtype=L.PARAM_DESC)
    ra = np.zeros(2 * len(diag), dtype=np.float32)
    tasks = []
    for i, (pre, g) in enumerate(diag):
        e = tab[i]
        e["graw"] = e["g"] = g.data_ptr()
        e["diag_ema"] = pre.diag_ema.data_ptr()
        e["numel"] = g.numel()
        e["dtype"] = L.DTYPE_CODE[g.dtype]
        ra[2 * i], ra[2 * i + 1] = pre.rho, 1.0 - pre.rho
        tasks += [(i, c, 0, -1) for c in range(_flat_chunks(g.numel()))]
    tt = np.array(tasks, dtype=np.int32).reshape(-1, 4).copy().view(L.TASK).reshape(-1)
    td, pd = L.upload(tt, dev), L.upload(tab, dev)
    rd = L.upload(ra, dev)
    _call("scao_diag_ema", td.data_ptr(), len(tt), pd.data_ptr(), rd.data_ptr(), s)
    for pre, _ in diag:
        pre._diag_bias_factor = max(1.0 - pre.rho ** pre.precond_step, 1e-8)
        pre._touch()   # a diagonal sub-block's bias factor sits in the block table


_SIDE_STREAMS: dict = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """A second stream on dev (default priority), made once per device."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _SIDE_STREAMS[key]


def _refresh_kron(kron, dev, s, eigen_only=False, ema_only=False):
    # 1) Gram -> EMA (-> requantise), chunked by staging memory
    todo = [] if eigen_only else list(kron)
    while todo:
        chunk, used = [], 0
        while todo:
            leaf = todo[0][0]
            need = 4 * (leaf.m * leaf.m + leaf.n * leaf.n) if leaf.use_int8_ema else 0
            if chunk and used + need > REFRESH_SCRATCH_BYTES:
                break
            chunk.append(todo.pop(0))
            used += need
        _gram_chunk(chunk, dev, s)
    if AFTER_EMA_HOOK is not None and not eigen_only:
        AFTER_EMA_HOOK(kron)
    if ema_only:
        for leaf, *_ in kron:
            leaf._touch()
        return
    # 2) eigendecomposition, batched by dimension.  Factors whose eigh input
    # is exactly diagonal (an int8 EMA of small gradients keeps only its
    # diagonal codes) take scao_eig_diag, which reproduces LAPACK's order of
    # tied eigenvalues; the others go to the solver their size selects.
    jobs = {}   # dim -> list of (leaf, side)
    for leaf, *_ in kron:
        jobs.setdefault(leaf.m, []).append((leaf, 0))
        jobs.setdefault(leaf.n, []).append((leaf, 1))
    spectra = {}   # (id(leaf), side) -> (S_desc, U_desc, total)
    LAST_REFRESH_ROUTES.clear()
    eig_timer = _mark("refresh:eigh+rank")
    eig_timer.__enter__()
    diagonal = _diagonal_factors(jobs, dev, s)
    # With several dimensions, every batch but the largest runs on a second
    # stream beside it (enqueued first, so it starts at once): a batch of a
    # few small factors leaves most of the GPU idle, and its latency-bound
    # kernels fit beside the large batch's.
    main = torch.cuda.current_stream(dev)
    # a batch's transient buffers (the stacked inputs, the band copies, the
    # eigenvector workspace) come to about twice its inputs: keep the inputs
    # to a quarter of what is free (the caching allocator's idle blocks count)
    free = torch.cuda.mem_get_info(dev)[0] + (torch.cuda.memory_reserved(dev) -
                                               torch.cuda.memory_allocated(dev))
    hip_budget = min(EIGEN_BATCH_BYTES, free // EIGEN_BATCH_FREE_FRACTION)
    order = sorted(jobs.items(), key=lambda kv: len(kv[1]) * kv[0] ** 2)
    side = _side_stream(dev) if len(order) > 1 else None
    if side is not None:
        side.wait_stream(main)   # the EMA codes
    for bi, (dim, lst) in enumerate(order):
        strm = side if side is not None and bi + 1 < len(order) else main
        with torch.cuda.stream(strm):
            s_b = L.stream_ptr(dev)
            # vectors a factor can keep: k <= k_max (rank momentum and clamps)
            kq = min(dim, max(leaf.k_max for leaf, _ in lst))
            routes = {}
            for key in lst:
                r = eigen_route(dim, (id(key[0]), key[1]) in diagonal)
                routes.setdefault(r, []).append(key)
            if "hip" in routes and batch_route("hip", dim, len(routes["hip"])) == "library":
                routes.setdefault("library", []).extend(routes.pop("hip"))
            for r, keys in routes.items():
                LAST_REFRESH_ROUTES[r] = LAST_REFRESH_ROUTES.get(r, 0) + len(keys)
            for route, keys in routes.items():
                budget = EIGH_BATCH_BYTES if route == "library" else hip_budget
                per = len(keys) if route == "diag" else \
                    min(max(1, budget // (4 * dim * dim)), eigen.MAX_BATCH)
                for b0 in range(0, len(keys), per):
                    part = keys[b0:b0 + per]
                    if route == "diag":
                        w, U_desc, total = _diag_eigh(part, dim, kq, dev, s_b)
                        S_desc = w.clamp(min=0.0).float()
                    elif route == "hip":
                        X = _eig_inputs(part, dim, dev, s_b)
                        w, U_desc, total = eigen.topk_eigh(X, kq)
                        S_desc = w.clamp(min=0.0).float()
                        del X
                    else:
                        X = _eig_inputs(part, dim, dev, s_b)
                        w, V = _eigh_batched(X)
                        S_desc = w.flip(-1).clamp(min=0.0)[:, :kq].contiguous()
                        U_desc = V.flip(-1)[:, :, :kq].contiguous()
                        total = w.clamp(min=0.0).sum(dim=1).double()
                        del X, V
                    if strm is not main:   # used on the current stream from here on
                        for t in (S_desc, U_desc, total):
                            t.record_stream(main)
                    for (leaf, side_), Sd, Ud, tot in zip(part, S_desc, U_desc, total):
                        spectra[(id(leaf), side_)] = (Sd, Ud, tot)
    if side is not None:
        main.wait_stream(side)
    # 3) adaptive rank for every (leaf, side) in one device pass + one read
    keys = [(leaf, side) for leaf, *_ in kron for side in (0, 1)]
    ranks = {}
    by_dim = {}
    for leaf, side in keys:
        dim = leaf.m if side == 0 else leaf.n
        by_dim.setdefault(dim, []).append((leaf, side))
    dev_ranks = []
    for dim, lst in by_dim.items():
        S = torch.stack([spectra[(id(lf), sd)][0] for lf, sd in lst])
        eps = torch.tensor([lf.epsilon_sparse for lf, _ in lst], device=dev, dtype=torch.float64)
        kmin = torch.tensor([lf.k_min for lf, _ in lst], device=dev, dtype=torch.int64)
        kmax = torch.tensor([lf.k_max for lf, _ in lst], device=dev, dtype=torch.int64)
        tot = torch.stack([spectra[(id(lf), sd)][2] for lf, sd in lst])
        dev_ranks.append((lst, batched_adaptive_rank_topk(S, tot, dim, eps, kmin, kmax)))
    host = torch.cat([r for _, r in dev_ranks]).cpu().tolist() if dev_ranks else []
    i = 0
    for lst, _ in dev_ranks:
        for key in lst:
            ranks[(id(key[0]), key[1])] = int(host[i])
            i += 1
    eig_timer.__exit__(None, None, None)
    # 4) rank momentum and truncation (reference :437-451)
    for leaf, *_ in kron:
        k = min(ranks[(id(leaf), 0)], ranks[(id(leaf), 1)])
        k = max(k, leaf._k - 1)
        k = min(k, leaf._k + 4)
        k = int(min(leaf.k_max, max(leaf.k_min, k)))
        leaf._k = k
        Sl, Ul, _ = spectra[(id(leaf), 0)]
        Sr, Ur, _ = spectra[(id(leaf), 1)]
        leaf.U_l = Ul[:, :k].contiguous()
        leaf.S_l = Sl[:k].contiguous()
        leaf.U_r = Ur[:, :k].contiguous()
        leaf.S_r = Sr[:k].contiguous()
        leaf._touch()
    if AFTER_EIGEN_HOOK is not None:
        AFTER_EIGEN_HOOK(kron)


def _task_rows(idx, a, b, slot) -> np.ndarray:
    """TASK rows from equal-length integer arrays (or scalars)."""
    n = max(np.size(x) for x in (idx, a, b, slot))
    t = np.empty((n, 4), dtype=np.int32)
    t[:, 0], t[:, 1], t[:, 2], t[:, 3] = idx, a, b, slot
    return t


_GRAM_TILE_IDX: dict = {}


def _gram_tile_idx(nt: int):
    """(a, b, slot) of a factor's Gram tasks for nt x nt tiles: the lower
    tiles, each also writing its transpose (GRAM_SYM), cached per size."""
    v = _GRAM_TILE_IDX.get(nt)
    if v is None:
        a, b = np.tril_indices(nt)
        v = (a.astype(np.int32), b.astype(np.int32), (a * nt + b).astype(np.int32))
        _GRAM_TILE_IDX[nt] = v
    return v


def _gram_chunk(chunk, dev, s):
    """Gram/EMA (and requantisation) launches for a chunk of (leaf, grad,
    offset, ld): the descriptor table is filled column by column and the int8
    staging buffers come from one allocation (per-record host work was most
    of the refresh's idle GPU time before its first kernel)."""
    recs = [(leaf, g, off, ld, side) for leaf, g, off, ld in chunk for side in (0, 1)]
    n = len(recs)
    dtab = np.zeros(n, dtype=L.GRAM_DESC)
    dims = np.array([lf.m if sd == 0 else lf.n for lf, _, _, _, sd in recs], dtype=np.int64)
    nts = (dims + L.GRAM_TILE - 1) // L.GRAM_TILE
    int8 = np.array([lf.use_int8_ema for lf, *_ in recs], dtype=bool)
    dtab["g"] = [g.data_ptr() for _, g, _, _, _ in recs]
    dtab["off"] = [off for _, _, off, _, _ in recs]
    dtab["ld"] = [ld for _, _, _, ld, _ in recs]
    dtab["rows"] = [lf.m for lf, *_ in recs]
    dtab["cols"] = [lf.n for lf, *_ in recs]
    dtab["side"] = [sd for *_, sd in recs]
    dtab["dtype"] = [L.DTYPE_CODE[g.dtype] for _, g, _, _, _ in recs]
    dtab["ntiles"] = nts * nts
    rho = np.array([lf.rho for lf, *_ in recs], dtype=np.float64)
    dtab["rho"], dtab["alpha"] = rho, 1.0 - rho
    dtab["flags"] = L.GRAM_SYM
    # int8 sides: fp32 EMA staging (dim^2) and tile maxima (nt^2), one buffer
    sizes = np.where(int8, dims * dims + nts * nts, 0)
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    staging = torch.empty(max(int(sizes.sum()), 1), dtype=torch.float32, device=dev)
    base = staging.data_ptr()
    q_ptr = np.array([(lf.L_ema_q if sd == 0 else lf.R_ema_q).data_ptr() if q8 else 0
                      for (lf, *_, sd), q8 in zip(recs, int8)], dtype=np.uint64)
    scale_ptrs = np.array([lf._scale.data_ptr() + 8 * sd if q8 else 0
                           for (lf, *_, sd), q8 in zip(recs, int8)], dtype=np.uint64)
    ema_fp32 = np.array([0 if q8 else (lf.L_ema if sd == 0 else lf.R_ema).data_ptr()
                         for (lf, *_, sd), q8 in zip(recs, int8)], dtype=np.uint64)
    off8 = (base + 4 * starts).astype(np.uint64)
    dtab["q"], dtab["scale"] = q_ptr, scale_ptrs
    dtab["ema"] = np.where(int8, off8, ema_fp32)
    dtab["amax"] = np.where(int8, off8 + (4 * dims * dims).astype(np.uint64), 0)
    # tasks, in record order
    parts = [_gram_tile_idx(int(nt)) for nt in nts]
    cnt = np.array([len(p[0]) for p in parts], dtype=np.int64)
    tt = np.empty((int(cnt.sum()), 4), dtype=np.int32)
    tt[:, 0] = np.repeat(np.arange(n, dtype=np.int32), cnt)
    tt[:, 1] = np.concatenate([p[0] for p in parts])
    tt[:, 2] = np.concatenate([p[1] for p in parts])
    tt[:, 3] = np.concatenate([p[2] for p in parts])
    dd = L.upload(dtab, dev)
    tt = tt.view(L.TASK).reshape(-1)
    td = L.upload(tt, dev)
    _call("scao_gram_ema", td.data_ptr(), len(tt), dd.data_ptr(), s)
    if int8.any():
        nch = np.array([_flat_chunks(int(d * d)) if q8 else 0 for d, q8 in zip(dims, int8)],
                       dtype=np.int64)
        rt = np.empty((int(nch.sum()), 4), dtype=np.int32)
        rt[:, 0] = np.repeat(np.arange(n, dtype=np.int32), nch)
        rt[:, 1] = np.arange(len(rt), dtype=np.int64) - np.repeat(np.cumsum(nch) - nch, nch)
        rt[:, 2], rt[:, 3] = 0, -1
        rt = rt.view(L.TASK).reshape(-1)
        rd = L.upload(rt, dev)
        sp = L.upload(scale_ptrs, dev)
        _call("scao_requant", rd.data_ptr(), len(rt), dd.data_ptr(), sp.data_ptr(), s)
    del staging   # stream-ordered reuse by the caching allocator is safe


def _prep_descs(part, dim, out: Tensor | None, shift: Tensor) -> np.ndarray:
    """PREP_DESC rows for (leaf, side) factors of one dimension: the EMA
    source (codes and scale, or the fp32 EMA), the bias factor, a shift slot
    and, when given, the output matrix out[i]."""
    tab = np.zeros(len(part), dtype=L.PREP_DESC)
    for i, (leaf, side) in enumerate(part):
        e = tab[i]
        e["bias"] = max(1.0 - leaf.rho ** leaf.precond_step, 1e-8)
        e["dim"] = dim
        if out is not None:
            e["out"] = out[i].data_ptr()
        e["shift"] = shift.data_ptr() + 4 * i
        if leaf.use_int8_ema:
            e["q"] = (leaf.L_ema_q if side == 0 else leaf.R_ema_q).data_ptr()
            e["scale"] = leaf._scale.data_ptr() + 8 * side
        else:
            e["ema"] = (leaf.L_ema if side == 0 else leaf.R_ema).data_ptr()
    return tab


def _eig_inputs(part, dim, dev, s) -> Tensor:
    X = torch.empty(len(part), dim, dim, dtype=torch.float32, device=dev)
    shift = torch.empty(len(part), dtype=torch.float32, device=dev)
    dd = L.upload(_prep_descs(part, dim, X, shift), dev)
    n = len(part)
    nchunk = _flat_chunks(dim * dim)
    tt = _task_rows(np.repeat(np.arange(n), nchunk), np.tile(np.arange(nchunk), n), 0,
                    -1).view(L.TASK).reshape(-1)
    td = L.upload(tt, dev)
    _call("scao_eig_prep", td.data_ptr(), len(tt), dd.data_ptr(), n, s)
    return X


def _diagonal_factors(jobs: dict, dev, s) -> set:
    """(id(leaf), side) of every factor up to DIAG_MAX_DIM rows whose EMA
    has no non-zero off-diagonal entry: one scan of the codes on the device
    and one read of the flags."""
    keys = [key for dim, lst in jobs.items() if dim <= DIAG_MAX_DIM for key in lst]
    if not keys:
        return set()
    dims = [key[0].m if key[1] == 0 else key[0].n for key in keys]
    shift = torch.empty(1, dtype=torch.float32, device=dev)   # not written by the scan
    tab = np.concatenate([_prep_descs([key], d, None, shift) for key, d in zip(keys, dims)])
    flags = torch.empty(len(keys), dtype=torch.int32, device=dev)
    codes = int(all(key[0].use_int8_ema for key in keys))
    dd = L.upload(tab, dev)
    for c0 in range(0, len(keys), 65535):
        c1 = min(c0 + 65535, len(keys))
        _call("scao_eig_offdiag", dd.data_ptr() + c0 * L.PREP_DESC.itemsize, c1 - c0,
              max(dims[c0:c1]), codes, flags.data_ptr() + 4 * c0, s)
    host = flags.cpu().tolist()
    return {(id(key[0]), key[1]) for key, f in zip(keys, host) if f == 0}


def _diag_eigh(part, dim, kq, dev, s):
    """topk_eigh's (w, U, total) for exactly diagonal factors of one dimension
    (scao_eig_diag)."""
    n = len(part)
    shift = torch.empty(n, dtype=torch.float32, device=dev)
    w = torch.empty(n, kq, dtype=torch.float64, device=dev)
    U = torch.empty(n, dim, kq, dtype=torch.float32, device=dev)
    total = torch.empty(n, dtype=torch.float64, device=dev)
    dd = L.upload(_prep_descs(part, dim, None, shift), dev)
    for c0 in range(0, n, 65535):
        c1 = min(c0 + 65535, n)
        _call("scao_eig_diag", dd.data_ptr() + c0 * L.PREP_DESC.itemsize, c1 - c0, dim, kq,
              w[c0].data_ptr(), U[c0].data_ptr(), dim * kq, total[c0].data_ptr(), s)
    return w, U, total


def _eigh_batched(X: Tensor):
    """torch.linalg.eigh on a stack; on LinAlgError retry each matrix, adding
    1e-8 to its diagonal when it fails again (reference :413-428)."""
    try:
        return torch.linalg.eigh(X)
    except torch.linalg.LinAlgError:
        ws, vs = [], []
        for A in X:
            try:
                w, V = torch.linalg.eigh(A)
            except torch.linalg.LinAlgError:
                A = A.clone()
                A.diagonal().add_(1e-8)
                w, V = torch.linalg.eigh(A)
            ws.append(w)
            vs.append(V)
        return torch.stack(ws), torch.stack(vs)


# --------------------------------------------------------------------------
# standalone preconditioner methods
# --------------------------------------------------------------------------

def precondition_one(pre: SparsePreconditioner, grad: Tensor) -> Tensor:
    """SparsePreconditioner.precondition through the HIP fused operator."""
    require_hip(grad, "gradient")
    dt = grad.dtype
    g2, shape = to_2d(grad.to(torch.float32))
    g2 = g2.contiguous()
    if pre.use_block_diagonal or pre.use_kronecker:
        out = torch.zeros_like(g2) if pre.use_block_diagonal else None
        for leaf, r0, c0 in pre.leaves(diag=True):
            gb = g2[r0:r0 + leaf.m, c0:c0 + leaf.n]
            if not leaf.use_kronecker:
                out[r0:r0 + leaf.m, c0:c0 + leaf.n] = precondition_one(leaf, gb)
                continue
            from .hip import fused_kronecker_precond
            _, sl = leaf.U_l, leaf.S_l.clamp(min=1e-8).pow(-0.25)
            sr = leaf.S_r.clamp(min=1e-8).pow(-0.25)
            res = fused_kronecker_precond(leaf.U_l, sl, leaf.U_r, sr, gb)
            if out is None:
                out = res
            else:
                out[r0:r0 + leaf.m, c0:c0 + leaf.n] = res
        return out.reshape(shape).to(dt)
    bias = getattr(pre, "_diag_bias_factor", 1.0)
    den = (pre.diag_ema / bias).reshape_as(g2).pow(0.25).add_(1e-8)
    return (g2 / den).reshape(shape).to(dt)


def natural_norm_one(pre: SparsePreconditioner, grad: Tensor, eps: float) -> Tensor:
    """SparsePreconditioner.natural_grad_norm (small-matrix torch ops on device)."""
    require_hip(grad, "gradient")
    g2, _ = to_2d(grad.to(torch.float32))
    if pre.use_block_diagonal:
        parts = []
        for leaf, r0, c0 in pre.leaves(diag=True):
            parts.append(natural_norm_one(leaf, g2[r0:r0 + leaf.m, c0:c0 + leaf.n], eps).pow(2))
        return torch.stack(parts).sum().sqrt()
    if not pre.use_kronecker:
        den = pre.diag_ema.reshape_as(g2).pow(0.5).add_(eps)
        return (g2.pow(2) / den).sum().sqrt()
    il = pre.S_l.clamp(min=eps).pow(-0.5)
    ir = pre.S_r.clamp(min=eps).pow(-0.5)
    proj = (pre.U_l.T @ g2) @ pre.U_r
    return (il.unsqueeze(1) * proj * ir.unsqueeze(0)).norm(p="fro")
