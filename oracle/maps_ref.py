"""The reference's own reset map modes, restated with injected uniforms.

Test infrastructure: the CPU restatement the HIP reset kernel is checked
against; nothing in the product imports it.

Follows `BatchedSim.reset_` (sim/torch_sim.py:178-420) and the generators
it calls (sim/mapgen.py:15-242, `_opp_start` :433-453, `_open_spawns`
:455-463, `_open_geometry` :465-499, `_place_open_cross_crates` :535-547,
`_ring_spawns` :598-600, `SimConfig.spawn_pos` / `ring_spawns`
sim/config.py:561-603).  The reference draws from a host `torch.Generator`;
here every draw is a Philox uniform keyed by (seed, env, reset epoch), the
same law:

* STREAM_RESET_MISC, value j of the env:
    0 map type (pure open / open / ring / corridor by the cumulative
      fractions), 1 corridor top wall rows U{0..top_wall_rows},
    2 spawn swap (< 0.5), 3 open obstacle count U{0..open_obstacle_max},
    4 + 3i + (0, 1, 2) start, length and on/off of the vertical brick
      segment on edge column i (wall_density > 0),
    16 + (0, 1, 2) the same for the horizontal segment;
* STREAM_RESET_CELL, value c: the ring band's brick draw of cell c;
  value H*W + c: the open obstacles' key of cell c (the obstacles are the n
  cells with the smallest (key, cell), a uniform n-subset like the
  reference's first n of a random permutation).

Pinned against the reference's own generators on the same draws in
tests/test_oracle_maps_ref.py (fixtures from
tests/golden/gen_reference_maps.py).

Reference behaviour kept on purpose: the open obstacles clear the
neighbourhoods of `cfg.spawn_cells()` (the corridor spawns in corridor
mode), not of the open spawns; corridor bricks are laid in the bottom wall
rows too (wall and brick both set; a blast never reaches a wall cell);
only players 0 and 1 get new caps, speeds and hit-penalty floors (players
2 and 3 keep theirs across episodes).
"""

from __future__ import annotations

import numpy as np

from . import philox

MISC_TYPE, MISC_TOP, MISC_SWAP, MISC_NOBST, MISC_VSEG, MISC_HSEG = 0, 1, 2, 3, 4, 16
N_MISC = 19
KIND_CORRIDOR, KIND_OPEN, KIND_RING = 0, 1, 2
DIRS = ((-1, 0), (1, 0), (0, -1), (0, 1))
F32 = np.float32


def _clear_around(grid, cells, h, w):
    """grid (k, h, w): clear each cell and its in-map 4-neighbours."""
    for r, c in cells:
        grid[:, r, c] = False
        for dr, dc in DIRS:
            if 0 <= r + dr < h and 0 <= c + dc < w:
                grid[:, r + dr, c + dc] = False


def corridor_spawns(cfg):
    """SimConfig.spawn_pos in corridor mode (sim/config.py:573-580)."""
    w = float(cfg.width)
    row = (cfg.top_wall_rows + (cfg.height - 1)) / 2.0 + 0.5
    c0 = (w - cfg.corridor_width) / 2.0 + 0.5
    step = (cfg.corridor_width - 2) / max(1, cfg.n_players - 1)
    return [(row, c0 + 1.0 + i * step) for i in range(cfg.n_players)]


def open_spawns(cfg):
    """Middle row, columns split evenly (sim/torch_sim.py:455-463; also
    SimConfig.spawn_pos outside corridor mode)."""
    h, w = float(cfg.height), float(cfg.width)
    row = (h - 1) / 2.0 + 0.5
    return [(row, (w - 1) * (i + 1) / (cfg.n_players + 1) + 0.5) for i in range(cfg.n_players)]


def ring_spawns(cfg):
    """Corners (sim/config.py:590-599)."""
    h, w = float(cfg.height), float(cfg.width)
    return [(1.5, 1.5), (1.5, w - 0.5), (h - 0.5, w - 0.5), (h - 0.5, 1.5)][: cfg.n_players]


def mode_spawns(cfg):
    """cfg.spawn_pos() for the config's map mode."""
    return corridor_spawns(cfg) if cfg.map_mode == "corridor" else open_spawns(cfg)


def cells_of(spawns):
    return [(int(y), int(x)) for y, x in spawns]


def corridor_walls(cfg, top):
    """make_walls in corridor mode (sim/mapgen.py:36-52,61-67): `top` (k,)
    int rows of wall at the top and top_wall_rows - top at the bottom, or
    None for the fixed top_wall_rows rows; spawn neighbourhoods cleared."""
    h, w = cfg.height, cfg.width
    rows = np.arange(h)[None, :]
    if top is None:
        wall = np.zeros((1, h, w), dtype=bool)
        wall[:, : cfg.top_wall_rows, :] = True
    else:
        top = np.asarray(top)[:, None]
        bot = cfg.top_wall_rows - top
        wall = ((rows < top) | (rows >= h - bot))[:, :, None].repeat(w, 2)
    _clear_around(wall, cells_of(mode_spawns(cfg)), h, w)
    return wall


def corridor_bricks(cfg, top, useg=None):
    """make_bricks in corridor mode (sim/mapgen.py:101-199).  `useg` (k, 15)
    float32: (start, length, on) for the four edge columns, then for the
    horizontal segment; needed when wall_density > 0."""
    h, w = cfg.height, cfg.width
    c0 = (w - cfg.corridor_width) // 2
    c1 = c0 + cfg.corridor_width
    rows = np.arange(h)[:, None]
    cols = np.arange(w)[None, :]
    side = (cols < c0) | (cols >= c1)
    if top is None:
        out = (side & ~(rows < cfg.top_wall_rows))[None].copy()
        k = 1 if useg is None else useg.shape[0]
        out = out.repeat(k, 0)
    else:
        top = np.asarray(top)
        k = top.shape[0]
        in_top = np.arange(h)[None, :] < top[:, None]
        out = side[None] & ~in_top[:, :, None]
    if cfg.wall_density > 0:
        useg = np.asarray(useg, dtype=F32)
        dens = F32(cfg.wall_density)
        edge = [c for c in (c0, c0 + 1, c1 - 2, c1 - 1) if c0 <= c < c1]
        for ci, col in enumerate(edge):
            us, ul, ua = useg[:, 3 * ci], useg[:, 3 * ci + 1], useg[:, 3 * ci + 2]
            if top is None:
                start = (us * F32(h - cfg.top_wall_rows - 4) + F32(cfg.top_wall_rows)).astype(np.int64)
            else:
                bot = cfg.top_wall_rows - top
                span = np.maximum(h - bot - 4 - top, 1)
                start = (us * span.astype(F32) + top.astype(F32)).astype(np.int64)
            length = 2 + (ul * F32(3.0)).astype(np.int64)
            act = ua < dens
            r = np.arange(h)[None, :]
            seg = act[:, None] & (r >= start[:, None]) & (r < (start + length)[:, None])
            out[:, :, col] |= seg
        if c1 - c0 > 4:
            us, ul, ua = useg[:, 12], useg[:, 13], useg[:, 14]
            hs = (us * F32(c1 - c0 - 4) + F32(c0)).astype(np.int64)
            hl = 2 + (ul * F32(3.0)).astype(np.int64)
            act = ua < dens
            cc = np.arange(c0, c1)[None, :]
            hseg = act[:, None] & (cc >= hs[:, None]) & (cc < (hs + hl)[:, None])
            for e in range(out.shape[0]):
                if top is None:
                    band = range(cfg.top_wall_rows, cfg.top_wall_rows + min(2, h - cfg.top_wall_rows))
                else:
                    band = (int(top[e]), int(top[e]) + 1)
                for r in band:
                    out[e, r, c0:c1] |= hseg[e]
    _clear_around(out, cells_of(mode_spawns(cfg)), h, w)
    return out


def ring_block(cfg):
    r0 = (cfg.height - cfg.ring_center_h) // 2
    c0 = (cfg.width - cfg.ring_center_w) // 2
    return r0, c0, r0 + cfg.ring_center_h, c0 + cfg.ring_center_w


def ring_walls(cfg, k):
    """make_ring_walls (sim/mapgen.py:227-242)."""
    r0, c0, r1, c1 = ring_block(cfg)
    wall = np.zeros((k, cfg.height, cfg.width), dtype=bool)
    wall[:, r0:r1, c0:c1] = True
    return wall


def ring_bricks(cfg, ucell):
    """make_ring_bricks (sim/mapgen.py:202-224): the one-cell band around
    the centre block, brick where ucell (k, H, W) < ring_brick_density,
    corner spawn neighbourhoods cleared."""
    h, w = cfg.height, cfg.width
    r0, c0, r1, c1 = ring_block(cfg)
    band = np.zeros((h, w), dtype=bool)
    band[r0 - 1:r1 + 1, c0 - 1:c1 + 1] = True
    band[r0:r1, c0:c1] = False
    brick = band[None] & (np.asarray(ucell, dtype=F32) < F32(cfg.ring_brick_density))
    _clear_around(brick, cells_of(ring_spawns(cfg)), h, w)
    return brick


def open_obstacles(cfg, n, ukey):
    """make_open_obstacles (sim/mapgen.py:70-98): per env the n cells with
    the smallest (key, cell) of ukey (k, H*W) become walls, then the
    neighbourhoods of cfg.spawn_cells() are cleared."""
    h, w = cfg.height, cfg.width
    n = np.asarray(n)
    k = n.shape[0]
    wall = np.zeros((k, h * w), dtype=bool)
    if cfg.open_obstacle_max > 0:
        cells = np.arange(h * w)
        for e in range(k):
            order = np.lexsort((cells, ukey[e]))
            wall[e, order[: int(n[e])]] = True
    wall = wall.reshape(k, h, w)
    _clear_around(wall, cells_of(mode_spawns(cfg)), h, w)
    return wall


def cross_cells(cfg):
    """The open-mode start crates (sim/torch_sim.py:465-499): rows
    (h-1)//2 - 1 and (h-1)//2, columns (w-1)//2 - 1 and (w-1)//2, minus the
    open spawns and their 4-neighbours."""
    h, w = cfg.height, cfg.width
    excl = set()
    for r, c in cells_of(open_spawns(cfg)):
        excl.add((r, c))
        for dr, dc in DIRS:
            if 0 <= r + dr < h and 0 <= c + dc < w:
                excl.add((r + dr, c + dc))
    cy, cx = (h - 1) // 2, (w - 1) // 2
    cross = {(r, c) for c in range(w) for r in (cy - 1, cy)} | \
            {(r, c) for r in range(h) for c in (cx - 1, cx)}
    return sorted(cross - excl)


def opp_start(cfg, boost, b0, z0, s0):
    """_opp_start (sim/torch_sim.py:433-453): player 1's starting caps and
    speed for opponent boost 0 (same as player 0), 1 (x opp_hist_mult,
    rounded half to even, capped) or 2 (opp_growth_*).  float32 math."""
    b0, z0, s0 = F32(b0), F32(z0), F32(s0)
    m = F32(cfg.opp_hist_mult)
    if boost == 2:
        return int(cfg.opp_growth_bombs), int(cfg.opp_growth_blast), F32(cfg.opp_growth_speed)
    if boost == 1:
        b = min(np.rint(b0 * m), F32(cfg.growth_bombs_max))
        z = min(np.rint(z0 * m), F32(cfg.growth_blast_max))
        s = min(s0 * m, F32(cfg.growth_speed_max))
        return int(b), int(z), F32(s)
    return int(b0), int(z0), s0


def reference_maps(cfg, env_ids, seed, epoch, opp_boost=0):
    """Per-env reset draws of the reference map modes for the envs env_ids.

    Returns a dict of numpy arrays: wall, brick, crate (k, H, W) bool; pos
    (k, P, 2) f32; caps01 (k, 2, 3) = (bombs, blast, speed) of players 0
    and 1; crate_prob (k,) f32 with NaN where the reference leaves it
    unchanged; map_kind (k,) int64.
    """
    h, w, p = cfg.height, cfg.width, cfg.n_players
    hw = h * w
    ids = np.asarray(env_ids)
    k = ids.shape[0]
    um = philox.uniforms(seed, ids, epoch, philox.STREAM_RESET_MISC, N_MISC)
    uc = philox.uniforms(seed, ids, epoch, philox.STREAM_RESET_CELL, 2 * hw)
    wall = np.zeros((k, h, w), dtype=bool)
    brick = np.zeros((k, h, w), dtype=bool)
    crate = np.zeros((k, h, w), dtype=bool)
    pos = np.zeros((k, p, 2), dtype=F32)
    caps = np.zeros((k, 2, 3), dtype=F32)
    crate_prob = np.full(k, np.nan, dtype=F32)
    kind = np.zeros(k, dtype=np.int64)
    nmax = cfg.open_obstacle_max
    nobst = np.minimum(np.floor(um[:, MISC_NOBST] * F32(nmax + 1)).astype(np.int64), nmax)
    obst = open_obstacles(cfg, nobst, uc[:, hw:])
    cross = cross_cells(cfg)
    for e in range(k):
        if cfg.map_mode != "corridor":
            wall[e] = obst[e]
            b0, z0, s0 = cfg.max_bombs, cfg.blast, 1.0
            kind[e] = KIND_OPEN
            spawns = open_spawns(cfg)
        else:
            r = um[e, MISC_TYPE]
            pf = F32(cfg.pure_open_fraction)
            of = F32(cfg.pure_open_fraction + cfg.open_fraction)
            rf = F32(cfg.pure_open_fraction + cfg.open_fraction + cfg.ring_fraction)
            if r < of:                                   # pure open or open
                wall[e] = False if r < pf else obst[e]
                b0, z0, s0 = cfg.open_growth_bombs, cfg.open_growth_blast, cfg.open_growth_speed
                crate_prob[e] = 1.0
                kind[e] = KIND_OPEN
                spawns = open_spawns(cfg)
                if cfg.open_crate_cross:
                    for (y, x) in cross:
                        crate[e, y, x] = True
            elif r < rf:                                 # ring
                wall[e] = ring_walls(cfg, 1)[0]
                brick[e] = ring_bricks(cfg, uc[e, :hw].reshape(1, h, w))[0]
                b0, z0, s0 = cfg.growth_bombs_start, cfg.growth_blast_start, cfg.growth_speed_start
                crate_prob[e] = cfg.ring_crate_prob
                kind[e] = KIND_RING
                spawns = ring_spawns(cfg)
            else:                                        # corridor
                T = cfg.top_wall_rows
                top = None
                if cfg.random_wall_rows:
                    top = np.array([min(int(np.floor(um[e, MISC_TOP] * F32(T + 1))), T)])
                wall[e] = corridor_walls(cfg, top)[0]
                brick[e] = corridor_bricks(cfg, top, um[e:e + 1, MISC_VSEG:MISC_VSEG + 15])[0]
                b0, z0, s0 = cfg.growth_bombs_start, cfg.growth_blast_start, cfg.growth_speed_start
                crate_prob[e] = cfg.growth_crate_prob
                kind[e] = KIND_CORRIDOR
                spawns = corridor_spawns(cfg)
        ob, oz, os_ = opp_start(cfg, opp_boost, float(b0), float(z0), float(s0))
        caps[e, 0] = (b0, z0, F32(s0))
        caps[e, 1] = (ob, oz, os_)
        for i, (y, x) in enumerate(spawns):
            pos[e, i] = (F32(y), F32(x))
        if um[e, MISC_SWAP] < F32(0.5):
            pos[e, [0, 1]] = pos[e, [1, 0]]
    return dict(wall=wall, brick=brick, crate=crate, pos=pos, caps01=caps,
                crate_prob=crate_prob, map_kind=kind)
