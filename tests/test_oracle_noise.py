"""The noise oracle against published known answers (CPU only)."""

import numpy as np
import pytest

from oracle import noise as N

# Random123 kat_vectors, philox4x32 with 10 rounds: counter words, key words,
# expected output words
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = N.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
    assert [int(x) for x in got] == list(want)


def test_counter_and_key_layout():
    """Element e uses counter (e >> 2) split low word first; the seed is the
    key, low word first."""
    seed = 0x0123456789ABCDEF
    w = N.words(seed, 4 * 5 + 3)
    assert w.shape == (6, 4)
    for q in (0, 3, 5):
        ctr = np.array([[q & 0xFFFFFFFF, q >> 32, 0, 0]], dtype=np.uint32)
        assert np.array_equal(w[q], N.philox4x32_10(ctr, (0x89ABCDEF, 0x01234567))[0])


def test_uniform_range_and_rounding():
    w = np.array([0, 0xFF, 0x100, 0x7FFFFFFF, 0xFFFFFFFF], dtype=np.uint32)
    u = N.uniforms(w)
    assert u[0] == u[1] == 0.5 * 2.0 ** -24          # the smallest value, never 0
    assert u[2] == 1.5 * 2.0 ** -24
    # (2^24 - 1) + 0.5 does not fit 24 bits: float32 rounds it to 2^24, u = 1
    assert u[4] == 1.0
    assert 0.0 < u.min() and u.max() <= 1.0


def test_normal_sample_moments_and_ks():
    from scipy import stats
    n = 1 << 20
    z = N.normals(12345, n)
    assert abs(z.mean()) < 5.0 / np.sqrt(n)
    assert abs(z.var() - 1.0) < 5.0 * np.sqrt(2.0 / n)
    assert stats.kstest(z, "norm").pvalue > 1e-4
    # separate seeds and neighbouring groups are uncorrelated
    z2 = N.normals(12346, n)
    assert abs(np.corrcoef(z, z2)[0, 1]) < 5.0 / np.sqrt(n)
    assert abs(np.corrcoef(z[:-4], z[4:])[0, 1]) < 5.0 / np.sqrt(n)
