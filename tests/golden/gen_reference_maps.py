#!/usr/bin/env python3
"""Write ref_maps.npz by running the reference's map generators.

Run in the build container, where the reference checkout sits at
/root/reference:

    python tests/golden/gen_reference_maps.py

It imports the reference's `sim.mapgen`, `sim.config` and `sim.torch_sim`
and writes input/output vectors of its reset map modes (only vectors; no
reference source is copied):

* corridor walls and bricks for every top-row count (random wall rows) and
  for the fixed top rows, for 2, 3 and 4 players;
* corridor bricks with edge segments (wall_density 0.45), random and fixed
  top rows, with the uniforms the generator drew, replayed from a clone of
  its seeded generator;
* ring walls and ring bricks (with the drawn uniform field), 2 and 4
  players;
* open obstacles (open_obstacle_max 6) with the drawn counts and keys, in
  corridor and open map mode;
* `BatchedSim.reset_all` outcomes for all-open, all-ring, all-corridor and
  open-map-mode configs at opponent boosts 0, 1 and 2: start crates, caps,
  speeds, hit-penalty floors, crate probability, map kind, spawn positions.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
sys.path.insert(0, REF)

import sim.torch_sim as ref_torch_sim  # noqa: E402
from sim import mapgen  # noqa: E402
from sim.config import SimConfig as RefConfig  # noqa: E402

ref_torch_sim._HAS_TRITON = False
ref_torch_sim._move_triton = None

BASE = dict(map_mode="corridor", speed=3.0, tick_hz=10, max_steps=1800, obs_fp16=True)


def cfg_of(**kw):
    if kw.get("n_players", 2) == 4:           # corridor_width >= 2P - 1
        kw.setdefault("corridor_width", 7)
    return RefConfig(**dict(BASE, **kw))


def main():
    out = {}
    # ---- corridor walls/bricks, no segments
    for p in (2, 3, 4):
        cfg = cfg_of(n_players=p)
        top = torch.arange(cfg.top_wall_rows + 1)
        g = torch.Generator().manual_seed(0)
        out[f"corr_walls_rand_p{p}"] = mapgen.make_walls(cfg, len(top), g, "cpu", top_rows=top).numpy()
        out[f"corr_bricks_rand_p{p}"] = mapgen.make_bricks(cfg, len(top), g, "cpu", top_rows=top).numpy()
        cfgf = cfg_of(n_players=p, random_wall_rows=False)
        out[f"corr_walls_fixed_p{p}"] = mapgen.make_walls(cfgf, 1, g, "cpu").numpy()
        out[f"corr_bricks_fixed_p{p}"] = mapgen.make_bricks(cfgf, 1, g, "cpu").numpy()
    # ---- corridor bricks with segments: the draws replayed from a clone
    n = 64
    for tag, rand_rows in (("rand", True), ("fixed", False)):
        cfg = cfg_of(wall_density=0.45, random_wall_rows=rand_rows)
        g = torch.Generator().manual_seed(11)
        top = torch.randint(0, cfg.top_wall_rows + 1, (n,), generator=g) if rand_rows else None
        g2 = torch.Generator().manual_seed(0)
        g2.set_state(g.get_state())
        bricks = mapgen.make_bricks(cfg, n, g, "cpu", top_rows=top)
        st = torch.rand((n, 4), generator=g2)
        ln = torch.rand((n, 4), generator=g2)
        ac = torch.rand((n, 4), generator=g2)
        hs = torch.rand((n,), generator=g2)
        hl = torch.rand((n,), generator=g2)
        ha = torch.rand((n,), generator=g2)
        useg = np.zeros((n, 15), dtype=np.float32)
        for ci in range(4):
            useg[:, 3 * ci] = st[:, ci].numpy()
            useg[:, 3 * ci + 1] = ln[:, ci].numpy()
            useg[:, 3 * ci + 2] = ac[:, ci].numpy()
        useg[:, 12], useg[:, 13], useg[:, 14] = hs.numpy(), hl.numpy(), ha.numpy()
        assert torch.equal(torch.rand(3, generator=g), torch.rand(3, generator=g2)), "replay drift"
        out[f"seg_{tag}_useg"] = useg
        out[f"seg_{tag}_top"] = (top.numpy() if top is not None else np.zeros(0, np.int64))
        out[f"seg_{tag}_bricks"] = bricks.numpy()
        if rand_rows:
            out["seg_rand_walls"] = mapgen.make_walls(cfg, n, g, "cpu", top_rows=top).numpy()
    # ---- ring
    for p in (2, 4):
        cfg = cfg_of(n_players=p, ring_fraction=1.0)
        g = torch.Generator().manual_seed(5)
        g2 = torch.Generator().manual_seed(0)
        g2.set_state(g.get_state())
        out[f"ring_bricks_p{p}"] = mapgen.make_ring_bricks(cfg, 16, g, "cpu").numpy()
        out[f"ring_u_p{p}"] = torch.rand((16, cfg.height, cfg.width), generator=g2).numpy()
        out[f"ring_walls_p{p}"] = mapgen.make_ring_walls(cfg, 1, "cpu").numpy()
    # ---- open obstacles (corridor mode clears the corridor spawns; open mode its own)
    for tag, mode in (("corr", "corridor"), ("open", "open")):
        cfg = cfg_of(map_mode=mode, open_obstacle_max=6)
        g = torch.Generator().manual_seed(9)
        g2 = torch.Generator().manual_seed(0)
        g2.set_state(g.get_state())
        out[f"obst_{tag}_walls"] = mapgen.make_open_obstacles(cfg, 32, g, "cpu").numpy()
        out[f"obst_{tag}_n"] = torch.randint(0, 7, (32,), generator=g2).numpy()
        out[f"obst_{tag}_u"] = torch.rand((32, cfg.height * cfg.width), generator=g2).numpy()
    # ---- whole resets, one map kind at a time
    kinds = {"open": dict(open_fraction=1.0), "ring": dict(ring_fraction=1.0),
             "corr": dict(), "mode_open": dict(map_mode="open")}
    for p in (2, 4):
        for tag, kw in kinds.items():
            cfg = cfg_of(n_players=p, **kw)
            s = ref_torch_sim.BatchedSim(cfg, 8, device="cpu", seed=3)
            for boost in (0, 1, 2):
                s.set_opp_boost(boost)
                s.reset_all()
                key = f"reset_{tag}_p{p}_b{boost}"
                out[key + "_crate"] = s.crate.numpy().copy()
                out[key + "_wall"] = s.wall.numpy().copy()
                out[key + "_caps"] = np.stack([s.bombs_cap.numpy().astype(np.float64),
                                               s.blast_cap.numpy().astype(np.float64),
                                               s.spd_g.numpy().astype(np.float64)], -1)
                out[key + "_lo"] = np.stack([s._lo_bombs.numpy().astype(np.float64),
                                             s._lo_blast.numpy().astype(np.float64),
                                             s._lo_spd.numpy().astype(np.float64)], -1)
                out[key + "_crate_prob"] = s.crate_prob.numpy().copy()
                out[key + "_map_kind"] = s._map_kind.numpy().copy()
                out[key + "_pos"] = s.pos.numpy().copy()
    np.savez_compressed(os.path.join(HERE, "ref_maps.npz"), **out)
    print("wrote ref_maps.npz:", len(out), "arrays")


if __name__ == "__main__":
    main()
