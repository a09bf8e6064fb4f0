"""The no-allocation operator entry point against the workspace one.

scao_fused_kronecker_precond_noalloc runs the same kernels as
scao_fused_kronecker_precond with its scratch in a static device array, so
the two outputs must be bit-identical.  Two calls in a row (the second one
smaller) check that the shared array's leftover contents never leak into a
later call."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(m, n, k, ldg, seed, dev):
    g = torch.Generator().manual_seed(seed)
    Ul = torch.linalg.qr(torch.randn(m, k, generator=g, dtype=torch.float64))[0].float()
    Ur = torch.linalg.qr(torch.randn(n, k, generator=g, dtype=torch.float64))[0].float()
    sl = torch.rand(k, generator=g) * 3 + 0.1
    sr = torch.rand(k, generator=g) * 3 + 0.1
    Gbig = torch.randn(m, ldg, generator=g) * 1e-3
    return [t.to(dev) for t in (Ul, sl, Ur, sr, Gbig)]


def _run(name, Ul, sl, Ur, sr, G, m, n, k, ws=None):
    from scao_amd import _lib as L
    out = torch.full((m, n), float("nan"), device=G.device)
    args = [Ul.data_ptr(), sl.data_ptr(), Ur.data_ptr(), sr.data_ptr(), G.data_ptr(),
            G.stride(0), out.data_ptr(), m, n, k]
    if ws is not None:
        args.append(ws.data_ptr())
    L.call(name, *args, L.stream_ptr(G.device))
    return out


def test_noalloc_matches_workspace_entry_point(hip_device):
    from scao_amd import _lib as L
    lib = L.lib()
    dev = hip_device
    # (m, n, k, ldG): the largest block of the benchmark configurations first
    # (4096 x 4096 at k = 256 fills 8.25 MiB of the array), then a smaller,
    # ragged one read through a strided column slice.
    for i, (m, n, k, ldg) in enumerate(((4096, 4096, 256, 4096), (200, 150, 24, 301))):
        print(f"noalloc case {i}: m={m} n={n} k={k} ldG={ldg}", flush=True)
        Ul, sl, Ur, sr, Gbig = _operands(m, n, k, ldg, 100 + i, dev)
        G = Gbig[:, :n]
        ws = torch.empty(lib.scao_fused_kronecker_workspace(m, n, k) // 4, device=dev)
        want = _run("scao_fused_kronecker_precond", Ul, sl, Ur, sr, G, m, n, k, ws)
        got = _run("scao_fused_kronecker_precond_noalloc", Ul, sl, Ur, sr, G, m, n, k)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), (m, n, k, (got - want).abs().max().item())


def test_noalloc_rejects_sizes_above_its_scratch(hip_device):
    from scao_amd import _lib as L
    lib = L.lib()
    dev = hip_device
    x = torch.zeros(16, device=dev)
    p = x.data_ptr()
    rc = lib.scao_fused_kronecker_precond_noalloc(p, p, p, p, p, 8192, p, 8192, 8192, 256,
                                                  L.stream_ptr(dev))
    assert rc == 1
    assert b"maximum" in lib.scao_last_error()
    torch.cuda.synchronize()
