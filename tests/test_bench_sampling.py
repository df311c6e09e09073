"""Which timed steps of `bench.py` carry the kernel-duration events (CPU only).

The bench times K steps and arms HIP event pairs on the launches of every
EVERY-th step to measure each kernel's duration inside the timed region.
The first timed step is left out whenever there is another to sample (events
on the first launches after the synchronised, idle queue cost wall time that
later steps do not), and every K >= 1 yields at least one sampled step, so
the per-kernel averages always exist.
"""

from __future__ import annotations

import bench


def _steps(k_total):
    return [k for k in range(k_total) if bench.sampled(k, k_total)]


def test_driver_and_default_step_counts():
    assert _steps(20) == [4, 12]
    assert _steps(256) == list(range(4, 256, bench.EVERY))
    assert len(_steps(256)) == 256 // bench.EVERY


def test_every_step_count_samples_at_least_once_and_skips_step_zero():
    for k_total in range(1, 300):
        got = _steps(k_total)
        assert got, k_total
        if k_total > 1:
            assert 0 not in got, k_total
        # one sample per EVERY steps at most, spaced EVERY apart
        assert all(b - a == bench.EVERY for a, b in zip(got, got[1:])), k_total
