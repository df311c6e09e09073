"""Philox4x32-10 counter-based generator in numpy (uint32 arithmetic).

Follows the published algorithm of Salmon, Moraes, Dror and Shaw, "Parallel
Random Numbers: As Easy as 1, 2, 3" (SC'11): ten rounds of two 32x32->64
multiplies with the key bumped by the Weyl constants between rounds.  The HIP
kernels use the same generator and the same stream layout, so every injected
uniform is reproducible on the host.  Pinned by the paper's known-answer
vectors in tests/test_oracle_philox.py.
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
_MASK = np.uint64(0xFFFFFFFF)

# Stream ids (third counter word) shared with the HIP kernels.
STREAM_CRATE = 1      # per tick: (u_hit, u_grow) per player
STREAM_RESET_CELL = 2  # per reset: one uniform per cell (brick draw)
STREAM_RESET_MISC = 3  # per reset: spawn swap + per-player cap draws
STREAM_POLICY = 4     # per tick: (u_move, u_bomb) per player for sampling
STREAM_RANDOM_ACT = 5  # per tick: uniform-legal random actions
STREAM_INJECT_ACT = 6  # per tick: unmasked injected actions
STREAM_BOT = 7        # per tick: rule-bot noise
STREAM_RECYCLE = 8    # per flush: one key per (player, cell) for recycle crates
STREAM_BOT_MODE = 9   # per switch of the astar bot's mode: (u_mode, u_timer) per env


def philox4x32(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Vectorised Philox4x32: all arguments broadcast uint32 arrays."""
    c0, c1, c2, c3 = (np.asarray(v, dtype=np.uint32) for v in (c0, c1, c2, c3))
    c0, c1, c2, c3 = np.broadcast_arrays(c0, c1, c2, c3)
    c0, c1, c2, c3 = (v.copy() for v in (c0, c1, c2, c3))
    k0 = np.asarray(k0, dtype=np.uint32).copy()
    k1 = np.asarray(k1, dtype=np.uint32).copy()
    for r in range(rounds):
        p0 = M0 * c0.astype(np.uint64)
        p1 = M1 * c2.astype(np.uint64)
        hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
        lo0 = (p0 & _MASK).astype(np.uint32)
        hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
        lo1 = (p1 & _MASK).astype(np.uint32)
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        if r != rounds - 1:
            k0 = ((k0.astype(np.uint64) + np.uint64(W0)) & _MASK).astype(np.uint32)
            k1 = ((k1.astype(np.uint64) + np.uint64(W1)) & _MASK).astype(np.uint32)
    return c0, c1, c2, c3


def to_unit(x) -> np.ndarray:
    """uint32 -> float32 in [0, 1) with 24 random bits (exact in float32)."""
    return (np.asarray(x, dtype=np.uint32) >> np.uint32(8)).astype(np.float32) \
        * np.float32(1.0 / 16777216.0)


def uniforms(seed: int, env, epoch: int, stream: int, count: int) -> np.ndarray:
    """(len(env), count) float32 uniforms: value j of env e comes from block
    j // 4, word j % 4 of Philox(key=seed, ctr=(e, epoch, stream, j // 4))."""
    env = np.asarray(env, dtype=np.uint32).reshape(-1, 1)
    nb = (count + 3) // 4
    blk = np.arange(nb, dtype=np.uint32).reshape(1, -1)
    k0 = np.uint32(seed & 0xFFFFFFFF)
    k1 = np.uint32((seed >> 32) & 0xFFFFFFFF)
    o = philox4x32(env, np.uint32(epoch & 0xFFFFFFFF), np.uint32(stream), blk, k0, k1)
    words = np.stack(o, axis=-1).reshape(env.shape[0], nb * 4)[:, :count]
    return to_unit(words)
