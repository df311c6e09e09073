"""Synthetic map templates for resets (the rollout workloads' maps).

The reference generates maps on the host with its own CPU generator
(sim/mapgen.py, sim/torch_sim.py:178-420).  The rollout workloads instead use
synthetic templates drawn on the device from counter-based uniforms, so a
reset needs no host round trip and is reproducible on the host:

* `pillars`: border walls plus indestructible pillars at even/even interior
  cells; with `brick_p > 0` every free cell outside the spawn L (the spawn
  cell and its two in-map neighbours) is a brick with that probability.
* `open`: no walls and no bricks.
* `reference`: the reference's own map modes, configured by the SimConfig
  (`map_mode`, `pure_open_fraction` / `open_fraction` / `ring_fraction`,
  `random_wall_rows`, `top_wall_rows`, `corridor_width`, `wall_density`,
  `open_obstacle_max`, the ring and start-cap fields) and the sim's
  `set_opp_boost` tier: corridor maps with random top/bottom wall rows and
  side bricks, open maps with the centre cross crates, ring maps
  (sim/torch_sim.py:178-420, sim/mapgen.py), drawn from Philox uniforms
  on the device.  The MapSpec's other fields are unused for this kind.

Template spawns sit in opposite corners ((1.5, 1.5) and (h-1.5, w-1.5) for
two players; the other two corners for players 3 and 4).  Per-player starting
caps are drawn uniformly from the inclusive ranges `bombs_cap` and
`blast_cap`; the hit-penalty floors (`_lo_*`) are set to the drawn starts,
matching the reference's rule that a player is clamped back to its own
starting values (sim/torch_sim.py:1083-1102).
"""

from __future__ import annotations

from dataclasses import dataclass

KIND_CODES = {"pillars": 0, "open": 1, "reference": 2}


@dataclass(frozen=True)
class MapSpec:
    kind: str = "pillars"
    brick_p: float = 0.0
    swap_spawns: bool = False
    bombs_cap: tuple[int, int] = (2, 2)
    blast_cap: tuple[int, int] = (2, 2)
    speed: float = 1.0

    def __post_init__(self) -> None:
        if self.kind not in KIND_CODES:
            raise ValueError(f"unknown map kind {self.kind!r}")
        if not 0.0 <= self.brick_p <= 1.0:
            raise ValueError("brick_p must be in [0, 1]")
        for lo, hi in (self.bombs_cap, self.blast_cap):
            if not 0 <= lo <= hi <= 255:
                raise ValueError("cap ranges must satisfy 0 <= lo <= hi <= 255")


def spawn_cells(h: int, w: int, p: int) -> list[tuple[int, int]]:
    corners = [(1, 1), (h - 2, w - 2), (1, w - 2), (h - 2, 1)]
    return corners[:p]


def spawn_l_cells(h: int, w: int, p: int) -> set[tuple[int, int]]:
    """Each spawn cell plus its neighbours toward the map interior."""
    out = set()
    for r, c in spawn_cells(h, w, p):
        dr = 1 if r < h // 2 else -1
        dc = 1 if c < w // 2 else -1
        out |= {(r, c), (r, c + dc), (r + dr, c)}
    return out


# Workload presets (named by what they are).
OPEN_PILLARS = MapSpec(kind="pillars", brick_p=0.0)
CORRIDOR_70 = MapSpec(kind="pillars", brick_p=0.7)
BOMB_STRESS_40 = MapSpec(kind="pillars", brick_p=0.4, bombs_cap=(1, 4), blast_cap=(2, 5))


def recycle_exclusion(cfg) -> list[int]:
    """Flat cells a recycle crate never lands on (sim/torch_sim.py:455-533,
    `_recycle_excl`): each spawn cell and its 4-neighbours for the open-mode
    spawns (middle row, columns split evenly), `cfg.spawn_cells()` and the
    ring-mode corners, plus the open-mode centre cross (rows and columns
    (n-1)//2 - 1 and (n-1)//2), sorted."""
    h, w, p = cfg.height, cfg.width, cfg.n_players
    row = (h - 1) / 2.0 + 0.5
    spawns = [(row, (w - 1) * (i + 1) / (p + 1) + 0.5) for i in range(p)]
    spawns += [(float(r), float(c)) for r, c in cfg.spawn_cells()]
    spawns += [(float(r), float(c)) for r, c in cfg.ring_spawn_cells()]
    cells = set()
    for sy, sx in spawns:
        r0, c0 = int(sy), int(sx)
        for r, c in ((r0, c0), (r0 - 1, c0), (r0 + 1, c0), (r0, c0 - 1), (r0, c0 + 1)):
            if 0 <= r < h and 0 <= c < w:
                cells.add(r * w + c)
    cy, cx = (h - 1) // 2, (w - 1) // 2
    cells |= {r * w + c for r in (cy - 1, cy) for c in range(w)}
    cells |= {r * w + c for r in range(h) for c in (cx - 1, cx)}
    return sorted(cells)
