"""Counter-based normal draws of the noise injection -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module; the product never does.

The reference adds ``torch.randn_like(grad) * noise_std`` to the gradient
(scao/optimizer.py:544-545).  Those draws come from torch's generator and
cannot be reproduced bit for bit on another device, so the product defines
its own counter-based stream, restated here in numpy:

  * Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
    easy as 1, 2, 3", SC'11): round multipliers 0xD2511F53 / 0xCD9E8D57,
    Weyl key increments 0x9E3779B9 / 0xBB67AE85, ten rounds.  Counter of
    element e: (e >> 2) as a 64-bit value in words 0 and 1, words 2 and 3
    zero; key: the parameter's 64-bit seed, low word first.
  * Box-Muller on the four output words w0..w3: u = (w >> 8 + 0.5) * 2^-24
    in float32 (the sum rounded to float32 as the kernels do),
    z[4q + 2j] = r cos(2 pi u'), z[4q + 2j + 1] = r sin(2 pi u') with
    r = sqrt(-2 ln u) for (u, u') = (u(w_2j), u(w_2j+1)).

Pinned by the published Philox4x32-10 known-answer vectors (Random123's
kat_vectors) in tests/test_oracle_noise.py, and the transform by the moments
and the Kolmogorov-Smirnov statistic of a large sample.  The device draws are
compared with this restatement to a stated absolute tolerance (the kernels
use the hardware transcendentals); a mistake in the Philox stage changes the
draws completely, so it shows at any tolerance.
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_LO = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 of counters ``ctr`` (uint32, shape (..., 4)) under the
    two-word ``key``; returns uint32 of the same shape."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0, k1 = np.uint32(key[0] & 0xFFFFFFFF), np.uint32(key[1] & 0xFFFFFFFF)
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = M0 * c[0]
            p1 = M1 * c[2]
            hi0, lo0 = p0 >> np.uint64(32), p0 & _LO
            hi1, lo1 = p1 >> np.uint64(32), p1 & _LO
            c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
            k0 = np.uint32(k0 + W0)
            k1 = np.uint32(k1 + W1)
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def words(seed: int, n: int) -> np.ndarray:
    """The Philox words behind elements 0 .. n-1 (shape (ceil(n/4), 4))."""
    q = np.arange((n + 3) // 4, dtype=np.uint64)
    ctr = np.zeros(q.shape + (4,), dtype=np.uint32)
    ctr[:, 0] = (q & _LO).astype(np.uint32)
    ctr[:, 1] = (q >> np.uint64(32)).astype(np.uint32)
    seed &= (1 << 64) - 1
    return philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))


def uniforms(w: np.ndarray) -> np.ndarray:
    """u = fp32(fp32(w >> 8) + 0.5) * 2^-24, in (0, 1]."""
    v = (w >> np.uint32(8)).astype(np.float32) + np.float32(0.5)
    return v.astype(np.float64) * 2.0 ** -24


def normals(seed: int, n: int) -> np.ndarray:
    """N(0, 1) draws of elements 0 .. n-1 under ``seed`` (float64)."""
    u = uniforms(words(seed, n))
    z = np.empty(u.shape, dtype=np.float64)
    for j in range(2):
        r = np.sqrt(-2.0 * np.log(u[:, 2 * j]))
        a = 2.0 * np.pi * u[:, 2 * j + 1]
        z[:, 2 * j] = r * np.cos(a)
        z[:, 2 * j + 1] = r * np.sin(a)
    return z.reshape(-1)[:n]
