"""The template maps every benchmark workload resets to (`oracle.sim.
template_maps`, which the HIP reset kernel reproduces bit for bit), checked
against the workload text itself rather than against a restatement of the
generator:

* 13 x 13 with border walls and indestructible pillars at the interior
  even/even cells (rows and columns 2, 4, ..., 10: exactly 25), nothing
  else a wall;
* players in opposite corners, cell centres (1.5, 1.5) and (11.5, 11.5),
  each with a clear 3-cell L (the spawn cell and its two neighbours toward
  the interior) that never holds a brick;
* every other free cell a brick with probability p, independently: each
  cell's frequency over 4096 envs within 5 sigma of p, the total within 4
  sigma, p = 0 and p = 1 exact;
* the optional side swap at rate 1/2 (4 sigma);
* per-player caps uniform over the inclusive ranges (bombs 1-4 and blast
  2-5 for the bomb-stress workload): every value drawn, frequencies within
  4 sigma, nothing outside.

Planted misreadings (pillars on odd cells, a spawn L on the wrong cells, a
brick law that skips a cell, an exclusive upper cap bound) are applied to
real draws and must be caught by the same checks."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.sim import template_maps
from qqtsim import corridor_training_config
from qqtsim.maps import BOMB_STRESS_40, CORRIDOR_70, OPEN_PILLARS, MapSpec

H = W = 13
N = 4096
PILLARS = {(r, c) for r in range(2, 11, 2) for c in range(2, 11, 2)}
BORDER = {(r, c) for r in range(H) for c in range(W) if r in (0, H - 1) or c in (0, W - 1)}
SPAWN_L = [{(1, 1), (1, 2), (2, 1)}, {(11, 11), (11, 10), (10, 11)}]
SPAWN_POS = [(1.5, 1.5), (11.5, 11.5)]


def _draw(spec, seed=3, epoch=0):
    cfg = corridor_training_config()
    return template_maps(cfg, spec, np.arange(N), seed, epoch)


def _violations(wall, brick, pos, bombs, blast, spec) -> list[str]:
    bad = []
    walls = {(r, c) for r in range(H) for c in range(W) if wall[0, r, c]}
    if walls != BORDER | PILLARS:
        bad.append("walls are not the border plus the 25 interior even/even pillars")
    if not (wall == wall[:1]).all():
        bad.append("walls differ between envs")
    if len(PILLARS) != 25:
        bad.append("pillar count")
    if (brick & wall).any():
        bad.append("brick on a wall")
    for i, cells in enumerate(SPAWN_L):
        for r, c in cells:
            if brick[:, r, c].any():
                bad.append(f"brick in player {i}'s spawn L at {(r, c)}")
    free = [(r, c) for r in range(H) for c in range(W)
            if (r, c) not in BORDER | PILLARS | SPAWN_L[0] | SPAWN_L[1]]
    if len(free) != 169 - 48 - 25 - 6:
        bad.append("free cell count")
    p = spec.brick_p
    freq = np.array([brick[:, r, c].mean() for r, c in free])
    if p in (0.0, 1.0):
        if not np.all(freq == p):
            bad.append("brick law not exact at p in {0, 1}")
    else:
        sig = math.sqrt(p * (1 - p) / N)
        if np.abs(freq - p).max() > 5 * sig:
            bad.append("a cell's brick frequency is off p")
        tot = brick[:, [r for r, _ in free], [c for _, c in free]].mean()
        if abs(tot - p) > 4 * sig / math.sqrt(len(free)):
            bad.append("overall brick fraction is off p")
        # independence between envs: no two envs share a brick pattern
        pats = {brick[e].tobytes() for e in range(N)}
        if len(pats) < N:
            bad.append("identical brick patterns in different envs")
    spawns = {tuple(map(float, pos[e, i])) for e in range(N) for i in range(2)}
    if spawns != set(SPAWN_POS):
        bad.append("spawn positions are not the two corner cell centres")
    swapped = pos[:, 0, 0] > 6.0
    if not ((pos[:, 0] != pos[:, 1]).any(axis=1)).all():
        bad.append("both players on one spawn")
    if spec.swap_spawns:
        if abs(swapped.mean() - 0.5) > 4 * math.sqrt(0.25 / N):
            bad.append("swap rate is off 1/2")
    elif swapped.any():
        bad.append("swapped spawns without swap_spawns")
    for name, arr, (lo, hi) in (("bombs", bombs, spec.bombs_cap), ("blast", blast, spec.blast_cap)):
        vals = np.asarray(arr).reshape(-1)
        if vals.min() < lo or vals.max() > hi:
            bad.append(f"{name} cap outside [{lo}, {hi}]")
        k = hi - lo + 1
        counts = np.array([(vals == v).sum() for v in range(lo, hi + 1)])
        if (counts == 0).any():
            bad.append(f"{name} cap value never drawn")
        if k > 1:
            q = 1.0 / k
            if np.abs(counts / vals.size - q).max() > 4 * math.sqrt(q * (1 - q) / vals.size):
                bad.append(f"{name} cap is not uniform")
    return bad


SPECS = [OPEN_PILLARS, CORRIDOR_70, BOMB_STRESS_40,
         MapSpec(kind="pillars", brick_p=1.0, swap_spawns=True, bombs_cap=(0, 10),
                 blast_cap=(7, 7)),
         MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)]


@pytest.mark.parametrize("spec", SPECS, ids=["open_pillars", "corridor70", "stress40", "full",
                                             "corridor70_swap"])
def test_template_matches_workload_text(spec):
    wall, brick, pos, bombs, blast, spd = _draw(spec)
    assert _violations(wall, brick, pos, bombs, blast, spec) == []
    assert np.all(spd == np.float32(spec.speed))


def test_template_draws_differ_by_epoch_and_seed():
    a = _draw(CORRIDOR_70, seed=3, epoch=0)[1]
    b = _draw(CORRIDOR_70, seed=3, epoch=1)[1]
    c = _draw(CORRIDOR_70, seed=4, epoch=0)[1]
    assert not np.array_equal(a, b) and not np.array_equal(a, c)
    assert np.array_equal(a, _draw(CORRIDOR_70, seed=3, epoch=0)[1])


def _mutated(kind):
    spec = BOMB_STRESS_40
    wall, brick, pos, bombs, blast, spd = _draw(spec)
    wall, brick, bombs = wall.copy(), brick.copy(), np.asarray(bombs).copy()
    rng = np.random.default_rng(0)
    if kind == "odd_pillars":
        wall[:] = False
        for r, c in BORDER | {(r, c) for r in range(1, 12, 2) for c in range(1, 12, 2)}:
            wall[:, r, c] = True
        brick &= ~wall
    elif kind == "wrong_l":                 # (1, 2) drawn, (1, 3) kept clear instead
        brick[:, 1, 2] = rng.random(N) < spec.brick_p
        brick[:, 1, 3] = False
    elif kind == "skipped_cell":
        brick[:, 5, 7] = False
    elif kind == "exclusive_hi":
        lo, hi = spec.bombs_cap
        u = rng.random(bombs.shape)
        bombs = lo + np.floor(u * (hi - lo)).astype(np.int64)
    return _violations(wall, brick, pos, bombs, blast, spec)


@pytest.mark.parametrize("kind", ["odd_pillars", "wrong_l", "skipped_cell", "exclusive_hi"])
def test_planted_misreadings_are_caught(kind):
    assert _mutated(kind) != []
