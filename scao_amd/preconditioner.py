"""Drop-in ``SparsePreconditioner`` (reference: scao/preconditioner.py:72-719).

Same constructor, mode selection (Kronecker / recursive block-diagonal /
diagonal), rank clamping, ``k`` property, attributes and ``state_dict``
layout as the reference.  What differs is where the work runs:

* the optimizer never calls ``precondition`` / ``natural_grad_norm`` /
  ``update_curvature`` per block; ``scao_amd.engine`` batches every block
  of every parameter into a handful of HIP launches;
* int8 EMA scales live on the device as float64 (exactly the reference's
  Python-float value), so a refresh needs no host round trip;
  ``L_ema_scale``/``R_ema_scale`` read them back on access;
* every change to U/S/k bumps ``_version`` (and a global epoch) so the
  engine knows when to re-upload its block descriptors.

The standalone methods (``update_curvature``, ``precondition``,
``natural_grad_norm``) exist for API compatibility and go through the same
HIP library; parameters must live on a ROCm device for them.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from .utils import to_2d, from_2d

PRECOND_DTYPE = torch.float32
_EPOCH = [0]


def leaf_epoch() -> int:
    """Monotone counter of eigenfactor/EMA changes across all preconditioners."""
    return _EPOCH[0]


def _init_int8_identity(dim: int, device) -> tuple[Tensor, float]:
    """quantize_sym_int8(eye(dim) * 1e-4) in closed form (scao/utils.py:170-189):
    absmax = fp32(1e-4), scale = absmax/127 (double), diagonal code
    clamp(rint(fp32(1e-4) / fp32(scale)), +-127)."""
    amax = float(np.float32(1e-4))
    scale = amax / 127.0
    code = float(np.clip(np.rint(np.float32(amax) / np.float32(scale)), -127, 127))
    q = torch.zeros(dim, dim, dtype=torch.int8, device=device)
    q.diagonal().fill_(int(code))
    return q, scale


class SparsePreconditioner:
    """Per-parameter Kronecker / block-diagonal / diagonal preconditioner state."""

    def __init__(self, param: Tensor, epsilon_sparse: float = 0.05, k_min: int = 8,
                 k_max: int = 128, rho: float = 0.999, max_precond_dim: int = 4096,
                 use_newton_schulz: bool = False, use_int8_ema: bool = False) -> None:
        p2, _ = to_2d(param)
        m, n = p2.shape
        self.original_shape = param.shape
        self.m, self.n = m, n
        self.epsilon_sparse = epsilon_sparse
        dmin = min(m, n)
        self.k_min = min(k_min, dmin)
        self.k_max = min(k_max, dmin // 2) if dmin > 2 * self.k_min else self.k_min
        self.rho = rho
        self.use_newton_schulz = use_newton_schulz
        self.use_int8_ema = use_int8_ema
        self.device = param.device
        self.param_dtype = param.dtype
        self._version = 0
        two_d = param.ndim >= 2 and m > 1 and n > 1
        self.use_block_diagonal = two_d and max(m, n) > max_precond_dim
        self.use_kronecker = two_d and max(m, n) <= max_precond_dim
        if self.use_kronecker and not use_newton_schulz:
            use_newton_schulz = min(m, n) > 512   # reference :160-161 (read nowhere)
        if self.use_block_diagonal:
            rows_split = m >= n
            big, small = (m, n) if rows_split else (n, m)
            self._block_dim = 0 if rows_split else 1
            sizes = [max_precond_dim] * (big // max_precond_dim)
            if big % max_precond_dim:
                sizes.append(big % max_precond_dim)
            self._block_sizes = sizes
            self._blocks = []
            for bs in sizes:
                shp = (bs, small) if rows_split else (small, bs)
                self._blocks.append(SparsePreconditioner(
                    _Shape(shp, param.dtype, self.device),
                    epsilon_sparse=epsilon_sparse, k_min=k_min, k_max=k_max, rho=rho,
                    max_precond_dim=max_precond_dim, use_newton_schulz=use_newton_schulz,
                    use_int8_ema=use_int8_ema))
            self._k = self._blocks[0]._k if self._blocks else k_min
        elif self.use_kronecker:
            k0 = min(k_min, min(m, n))
            self._k = k0
            dev = self.device
            if use_int8_ema:
                self.L_ema_q, sl = _init_int8_identity(m, dev)
                self.R_ema_q, sr = _init_int8_identity(n, dev)
                self._scale = torch.tensor([sl, sr], dtype=torch.float64, device=dev)
            else:
                self.L_ema = torch.eye(m, device=dev, dtype=PRECOND_DTYPE) * 1e-4
                self.R_ema = torch.eye(n, device=dev, dtype=PRECOND_DTYPE) * 1e-4
            self.U_l = torch.eye(m, k0, device=dev, dtype=PRECOND_DTYPE)
            self.S_l = torch.ones(k0, device=dev, dtype=PRECOND_DTYPE)
            self.U_r = torch.eye(n, k0, device=dev, dtype=PRECOND_DTYPE)
            self.S_r = torch.ones(k0, device=dev, dtype=PRECOND_DTYPE)
        else:
            self.diag_ema = torch.zeros(param.shape, device=self.device, dtype=PRECOND_DTYPE)
            self._diag_bias_factor = 1e-8
            self._k = 1
        self.precond_step = 0

    # ------------------------------------------------------------ scales --
    @property
    def L_ema_scale(self) -> float:
        return float(self._scale[0])

    @L_ema_scale.setter
    def L_ema_scale(self, v: float) -> None:
        self._scale[0] = float(v)

    @property
    def R_ema_scale(self) -> float:
        return float(self._scale[1])

    @R_ema_scale.setter
    def R_ema_scale(self, v: float) -> None:
        self._scale[1] = float(v)

    def _touch(self) -> None:
        self._version += 1
        _EPOCH[0] += 1

    # ------------------------------------------------------------- rank ---
    @property
    def k(self) -> int:
        return self._k

    @k.setter
    def k(self, new_k: int) -> None:
        """reference :250-291 -- clamp, truncate U/S when the rank drops."""
        new_k = int(min(self.k_max, max(self.k_min, new_k)))
        if self.use_block_diagonal:
            for b in self._blocks:
                b.k = new_k
            self._k = sum(b._k for b in self._blocks) // max(len(self._blocks), 1)
            return
        if self.use_kronecker:
            if new_k < self._k:
                self.U_l = self.U_l[:, :new_k].contiguous()
                self.S_l = self.S_l[:new_k].contiguous()
                self.U_r = self.U_r[:, :new_k].contiguous()
                self.S_r = self.S_r[:new_k].contiguous()
                self._touch()
            elif new_k > self._k:
                cols = self.U_l.shape[1]
                new_k = min(new_k, cols) if new_k > cols else new_k
        self._k = new_k

    # ------------------------------------------------------------ leaves --
    def leaf_list(self) -> list:
        """``list(self.leaves())``, kept: the block split is fixed at
        construction (rank changes do not alter it)."""
        cached = self.__dict__.get("_leaves_cache")
        if cached is None:
            cached = self.__dict__["_leaves_cache"] = list(self.leaves())
        return cached

    def step_leaf_list(self) -> list:
        """``list(self.leaves(diag=True))``, kept like ``leaf_list``."""
        cached = self.__dict__.get("_step_leaves_cache")
        if cached is None:
            cached = self.__dict__["_step_leaves_cache"] = list(self.leaves(diag=True))
        return cached

    def __getstate__(self) -> dict:
        state = dict(self.__dict__)
        state.pop("_leaves_cache", None)
        state.pop("_step_leaves_cache", None)
        return state

    def leaves(self, r0: int = 0, c0: int = 0, diag: bool = False):
        """Kronecker blocks as (block, row offset, col offset) in the 2-D view.
        With ``diag``, also the diagonal sub-blocks of a block-diagonal split
        (a remainder one row or one column wide: reference
        preconditioner.py:142-153 gives it the diagonal mode), in block order."""
        if self.use_block_diagonal:
            off = 0
            for bs, b in zip(self._block_sizes, self._blocks):
                r, c = (r0 + off, c0) if self._block_dim == 0 else (r0, c0 + off)
                if b.use_block_diagonal or b.use_kronecker:
                    yield from b.leaves(r, c, diag)
                elif diag:
                    yield b, r, c
                off += bs
        elif self.use_kronecker:
            yield self, r0, c0

    def _bump_steps(self) -> None:
        """precond_step sequencing of update_curvature (reference :312, :319-330)."""
        self.precond_step += 1
        if self.use_block_diagonal:
            for b in self._blocks:
                b._bump_steps()

    def _sync_k(self) -> None:
        if self.use_block_diagonal:
            for b in self._blocks:
                b._sync_k()
            self._k = sum(b._k for b in self._blocks) // max(len(self._blocks), 1)

    # ----------------------------------------------------- standalone API --
    @torch.no_grad()
    def update_curvature(self, grad: Tensor) -> None:
        """reference :297-361, run through the batched HIP refresh."""
        from . import engine
        engine.refresh([(self, grad)])

    @torch.no_grad()
    def precondition(self, grad: Tensor) -> Tensor:
        """reference :457-521; Kronecker blocks use the HIP fused operator."""
        from . import engine
        return engine.precondition_one(self, grad)

    @torch.no_grad()
    def natural_grad_norm(self, grad: Tensor, eps: float = 1e-8) -> Tensor:
        """reference :527-564."""
        from . import engine
        return engine.natural_norm_one(self, grad, eps)

    # -------------------------------------------------------- checkpoint --
    def state_dict(self) -> dict:
        """reference :570-600 (same keys; scales as Python floats)."""
        d = {"precond_step": self.precond_step, "k": self._k,
             "use_kronecker": self.use_kronecker,
             "use_block_diagonal": self.use_block_diagonal}
        if self.use_block_diagonal:
            d["blocks"] = [b.state_dict() for b in self._blocks]
        elif self.use_kronecker:
            if self.use_int8_ema:
                sl, sr = (float(x) for x in self._scale.tolist())
                d.update({"L_ema_q": self.L_ema_q, "L_ema_scale": sl,
                          "R_ema_q": self.R_ema_q, "R_ema_scale": sr})
            else:
                d.update({"L_ema": self.L_ema, "R_ema": self.R_ema})
            d.update({"U_l": self.U_l, "S_l": self.S_l, "U_r": self.U_r, "S_r": self.S_r})
        else:
            d["diag_ema"] = self.diag_ema
        return d

    def memory_bytes(self) -> int:
        """reference :602-619."""
        if self.use_block_diagonal:
            return sum(b.memory_bytes() for b in self._blocks)
        tot = 0
        if self.use_kronecker:
            if self.use_int8_ema:
                tot += self.L_ema_q.numel() + 8 + self.R_ema_q.numel() + 8
            else:
                tot += self.L_ema.numel() * self.L_ema.element_size()
                tot += self.R_ema.numel() * self.R_ema.element_size()
            for t in (self.U_l, self.S_l, self.U_r, self.S_r):
                tot += t.numel() * t.element_size()
        else:
            tot += self.diag_ema.numel() * self.diag_ema.element_size()
        return tot

    def load_state_dict(self, st: dict) -> None:
        """reference :621-644."""
        self.precond_step = st["precond_step"]
        self._k = st["k"]
        if self.use_block_diagonal:
            for b, bs in zip(self._blocks, st["blocks"]):
                b.load_state_dict(bs)
        elif self.use_kronecker:
            if self.use_int8_ema:
                self.L_ema_q = st["L_ema_q"].to(device=self.device, dtype=torch.int8).contiguous()
                self.R_ema_q = st["R_ema_q"].to(device=self.device, dtype=torch.int8).contiguous()
                self._scale = torch.tensor([float(st["L_ema_scale"]), float(st["R_ema_scale"])],
                                           dtype=torch.float64, device=self.device)
            else:
                self.L_ema.copy_(st["L_ema"])
                self.R_ema.copy_(st["R_ema"])
            for name in ("U_l", "S_l", "U_r", "S_r"):
                setattr(self, name, st[name].to(device=self.device,
                                                dtype=PRECOND_DTYPE).contiguous())
            self._touch()
        else:
            self.diag_ema.copy_(st["diag_ema"])


class _Shape:
    """Shape/dtype/device stand-in for building sub-block preconditioners
    without allocating a fake parameter."""

    def __init__(self, shape, dtype, device):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.device = device
        self.ndim = len(shape)

    def unsqueeze(self, d):
        return _Shape((1, *self.shape), self.dtype, self.device)

    def reshape(self, *s):
        return self
