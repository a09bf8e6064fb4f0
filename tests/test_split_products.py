"""The three-way bf16 split behind the fp32 products that the projection and
Gram kernels run on the bf16 matrix cores (scao_common.hpp split_bf3 /
mfma_x6), restated in numpy: x = h + m + l exactly, and the six kept
products of two split values are within 2^-23 |x y| of x y."""

from __future__ import annotations

import numpy as np


def bf16_rn(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even, as v_cvt_pk_bf16_f32), as fp32."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def split3(x: np.ndarray):
    h = bf16_rn(x)
    r = (x - h).astype(np.float32)
    m = bf16_rn(r)
    lo = bf16_rn((r - m).astype(np.float32))
    return h, m, lo


def _values(n, seed):
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(n) * 10.0 ** rng.uniform(-30, 30, n)).astype(np.float32)
    b = rng.integers(0x00800000, 0x7F000000, n, dtype=np.int64).astype(np.uint32).view(np.float32)
    x = np.concatenate([a, b, -b])
    return x[np.isfinite(x) & (np.abs(x) > 1e-30)]


def test_split_is_exact():
    x = _values(400_000, 1)
    h, m, lo = split3(x)
    assert np.array_equal(h.astype(np.float64) + m + lo, x.astype(np.float64))
    # each part is a bf16 value (low 16 bits zero)
    for part in (h, m, lo):
        assert not np.any(part.view(np.uint32) & 0xFFFF)


def test_six_products_within_fp32_rounding():
    x, y = _values(200_000, 2), _values(200_000, 3)
    n = min(len(x), len(y))
    x, y = x[:n], y[:n]
    keep = (np.abs(x.astype(np.float64) * y) > 1e-280) & (np.abs(x.astype(np.float64) * y) < 1e280)
    x, y = x[keep], y[keep]
    (xh, xm, xl), (yh, ym, yl) = split3(x), split3(y)
    d = lambda a: a.astype(np.float64)
    six = (d(xh) * d(yh) + d(xh) * d(ym) + d(xm) * d(yh) + d(xh) * d(yl) + d(xl) * d(yh)
           + d(xm) * d(ym))
    exact = d(x) * d(y)
    rel = np.abs(six - exact) / np.abs(exact)
    assert rel.max() <= 2.0 ** -23, rel.max()
