"""`make_sim` with the reference factory's signature (sim/factory.py:11-35).

The reference picks between its torch and CUDA backends; this package adds
the HIP backend.  `backend` "hip" (or "auto") returns a `HipBatchedSim`;
any other name raises `ValueError`, as the reference does for unknown
backends.  There is no fallback: the HIP library must be built.
"""

from __future__ import annotations

from .config import SimConfig
from .maps import MapSpec
from .sim import HipBatchedSim


def make_sim(cfg: SimConfig, num_envs: int, backend: str = "auto", device: str | None = None,
             seed: int = 0, map_spec: MapSpec | None = None):
    if backend not in ("auto", "hip"):
        raise ValueError(f"unknown backend: {backend!r} (this package provides 'hip')")
    return HipBatchedSim(cfg, num_envs, device=device or "cuda", seed=seed, map_spec=map_spec)
