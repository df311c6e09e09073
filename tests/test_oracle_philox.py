"""Philox4x32-10 of the oracle against the published known-answer vectors.

The vectors are the Philox4x32 (10 rounds) known answers published with the
generator (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as
1, 2, 3", SC'11; the Random123 distribution's kat_vectors).  The HIP kernels
run the same generator with the same counter layout, which the GPU parity
tests check through every Philox-drawn uniform (crates, resets, sampling).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import philox

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
    got = philox.philox4x32(*ctr, *key)
    assert tuple(int(v) for v in got) == want


def test_philox_round_count_matters():
    """A planted mistake (9 rounds) must fail the known answers."""
    ctr, key, want = KAT[2]
    got = philox.philox4x32(*ctr, *key, rounds=9)
    assert tuple(int(v) for v in got) != want


def test_philox_vectorises_like_scalar_calls():
    c0 = np.arange(5, dtype=np.uint32)
    vec = philox.philox4x32(c0, 7, 3, 1, 11, 12)
    for i in range(5):
        one = philox.philox4x32(i, 7, 3, 1, 11, 12)
        assert all(int(v[i]) == int(o) for v, o in zip(vec, one))


def test_unit_conversion_is_exact_24_bit():
    x = np.array([0, 0xFF, 0x100, 0xFFFFFFFF, 0x80000000], dtype=np.uint32)
    u = philox.to_unit(x)
    assert u.dtype == np.float32
    np.testing.assert_array_equal(u, np.float32([0.0, 0.0, 2.0 ** -24, 1.0 - 2.0 ** -24, 0.5]))


def test_uniform_layout_blocks_and_words():
    """Value j of env e is word j % 4 of block j // 4 of
    Philox(key=seed, ctr=(e, epoch, stream, j // 4))."""
    seed, epoch, stream = 0x1234_5678_9ABC_DEF0, 17, philox.STREAM_CRATE
    envs = np.array([0, 3, 1000])
    u = philox.uniforms(seed, envs, epoch, stream, 6)
    k0, k1 = seed & 0xFFFFFFFF, seed >> 32
    for i, e in enumerate(envs):
        for j in range(6):
            words = philox.philox4x32(int(e), epoch, stream, j // 4, k0, k1)
            assert u[i, j] == philox.to_unit(words[j % 4])


def test_uniforms_are_uniform():
    u = philox.uniforms(7, np.arange(20000), 3, philox.STREAM_POLICY, 4).ravel()
    assert 0.0 <= u.min() and u.max() < 1.0
    assert abs(float(u.mean()) - 0.5) < 0.005
    assert abs(float(u.var()) - 1.0 / 12.0) < 0.002
    hist = np.histogram(u, bins=16, range=(0.0, 1.0))[0]
    exp = u.size / 16
    assert float(((hist - exp) ** 2 / exp).sum()) < 50.0
