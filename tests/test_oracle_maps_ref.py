"""The oracle's restatement of the reference's reset map modes
(oracle/maps_ref.py) against vectors written by the reference's own
generators (tests/golden/gen_reference_maps.py -> ref_maps.npz): corridor
walls and bricks (random and fixed top rows, with and without edge
segments), ring walls and bricks, open obstacles, and whole resets (start
crates, caps, speeds, hit-penalty floors, crate probability, map kind,
spawns) at opponent boosts 0, 1 and 2.  Plus the draw laws the Philox
restatement adds (map-type shares, uniform top rows)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import maps_ref as mr
from oracle.sim import OracleSim
from qqtsim.config import corridor_training_config
from qqtsim.maps import MapSpec

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_maps.npz")


@pytest.fixture(scope="module")
def z():
    return np.load(GOLD)


def cfg_of(**kw):
    if kw.get("n_players", 2) == 4:
        kw.setdefault("corridor_width", 7)
    return corridor_training_config(**kw)


@pytest.mark.parametrize("p", [2, 3, 4])
def test_corridor_walls_and_bricks(z, p):
    cfg = cfg_of(n_players=p)
    top = np.arange(cfg.top_wall_rows + 1)
    np.testing.assert_array_equal(mr.corridor_walls(cfg, top), z[f"corr_walls_rand_p{p}"])
    np.testing.assert_array_equal(mr.corridor_bricks(cfg, top), z[f"corr_bricks_rand_p{p}"])
    cfgf = cfg_of(n_players=p, random_wall_rows=False)
    np.testing.assert_array_equal(mr.corridor_walls(cfgf, None), z[f"corr_walls_fixed_p{p}"])
    np.testing.assert_array_equal(mr.corridor_bricks(cfgf, None), z[f"corr_bricks_fixed_p{p}"])


def test_corridor_bricks_in_bottom_wall_rows(z):
    """The reference lays side bricks in the bottom wall rows too."""
    b, w = z["corr_bricks_rand_p2"], z["corr_walls_rand_p2"]
    assert (b & w).any()


@pytest.mark.parametrize("tag", ["rand", "fixed"])
def test_corridor_edge_segments(z, tag):
    cfg = cfg_of(wall_density=0.45, random_wall_rows=(tag == "rand"))
    top = z[f"seg_{tag}_top"] if tag == "rand" else None
    got = mr.corridor_bricks(cfg, top, z[f"seg_{tag}_useg"])
    want = z[f"seg_{tag}_bricks"]
    np.testing.assert_array_equal(got, want)
    base = mr.corridor_bricks(cfg_of(random_wall_rows=(tag == "rand")), top,
                              z[f"seg_{tag}_useg"])
    assert (want & ~base).any(), "the draws switch some segments on"
    if tag == "rand":
        np.testing.assert_array_equal(mr.corridor_walls(cfg, top), z["seg_rand_walls"])


@pytest.mark.parametrize("p", [2, 4])
def test_ring(z, p):
    cfg = cfg_of(n_players=p, ring_fraction=1.0)
    np.testing.assert_array_equal(mr.ring_walls(cfg, 1), z[f"ring_walls_p{p}"])
    np.testing.assert_array_equal(mr.ring_bricks(cfg, z[f"ring_u_p{p}"]), z[f"ring_bricks_p{p}"])


@pytest.mark.parametrize("tag,mode", [("corr", "corridor"), ("open", "open")])
def test_open_obstacles(z, tag, mode):
    cfg = cfg_of(map_mode=mode, open_obstacle_max=6)
    got = mr.open_obstacles(cfg, z[f"obst_{tag}_n"], z[f"obst_{tag}_u"])
    np.testing.assert_array_equal(got, z[f"obst_{tag}_walls"])


KINDS = {"open": dict(open_fraction=1.0), "ring": dict(ring_fraction=1.0), "corr": dict(),
         "mode_open": dict(map_mode="open")}


@pytest.mark.parametrize("p", [2, 4])
@pytest.mark.parametrize("tag", list(KINDS))
def test_whole_reset_matches_reference(z, p, tag):
    """Everything a reset fixes without a random draw: start crates, the
    deterministic walls (ring, open), caps/speeds/floors of players 0 and 1
    per boost, crate probability, map kind, the spawn set (up to the swap)."""
    cfg = cfg_of(n_players=p, **KINDS[tag])
    o = OracleSim(cfg, 8, MapSpec(kind="reference"), seed=3)
    for boost in (0, 1, 2):
        o.set_opp_boost(boost)
        o.reset_all()
        key = f"reset_{tag}_p{p}_b{boost}"
        np.testing.assert_array_equal(o.crate.numpy(), z[key + "_crate"], err_msg=key)
        if tag in ("ring", "mode_open"):
            np.testing.assert_array_equal(o.wall.numpy(), z[key + "_wall"], err_msg=key)
        caps = np.stack([o.bombs_cap.numpy(), o.blast_cap.numpy(), o.spd_g.numpy()], -1)
        lo = np.stack([o.lo_bombs.numpy(), o.lo_blast.numpy(), o.lo_spd.numpy()], -1)
        np.testing.assert_array_equal(caps.astype(np.float64), z[key + "_caps"], err_msg=key)
        np.testing.assert_array_equal(lo.astype(np.float64), z[key + "_lo"], err_msg=key)
        np.testing.assert_array_equal(o.crate_prob.numpy(), z[key + "_crate_prob"], err_msg=key)
        np.testing.assert_array_equal(o.map_kind.numpy(), z[key + "_map_kind"], err_msg=key)
        want = z[key + "_pos"]
        got = o.pos.numpy()
        for e in range(8):           # same spawns, players 0 and 1 possibly swapped
            same = np.array_equal(got[e], want[e])
            sw = got[e].copy()
            sw[[0, 1]] = sw[[1, 0]]
            assert same or np.array_equal(sw, want[e]), (key, e)


def test_boost_one_rounds_half_to_even():
    """opp_hist_mult 1.5 on a start of 3 bombs: 4.5 rounds to 4 (torch.round)."""
    cfg = cfg_of(opp_hist_mult=1.5)
    assert mr.opp_start(cfg, 1, 3.0, 3.0, 1.0)[:2] == (4, 4)
    assert mr.opp_start(cfg, 1, 5.0, 1.0, 1.0)[:2] == (8, 2)   # 7.5 -> 8, 1.5 -> 2
    assert mr.opp_start(cfg, 1, 5.0, 5.0, 1.0)[1] == cfg.growth_blast_max   # 8 capped


def test_map_type_shares_and_uniform_top_rows():
    cfg = cfg_of(pure_open_fraction=0.1, open_fraction=0.2, ring_fraction=0.3)
    ids = np.arange(20000)
    d = mr.reference_maps(cfg, ids[:4000], 5, 0)
    kind = d["map_kind"]
    n = len(kind)
    frac_open, frac_ring = (kind == 1).mean(), (kind == 2).mean()
    tol = 4 * np.sqrt(0.25 / n)
    assert abs(frac_open - 0.3) < tol and abs(frac_ring - 0.3) < tol
    pure = (kind == 1) & ~d["wall"].reshape(n, -1).any(1)
    assert pure.sum() > 0
    corr = kind == 0
    tops = d["wall"][corr][:, :, 6].sum(1)           # wall rows of a middle column
    assert set(np.unique(tops)) == {cfg.top_wall_rows}
    first = d["wall"][corr][:, 0, 6]                 # row 0 is wall iff top >= 1
    assert abs(first.mean() - 0.8) < 4 * np.sqrt(0.16 / corr.sum())


def test_planted_wrong_corridor_spawn_fails(z):
    """A corridor spawn one column off no longer reproduces the reference's
    cleared neighbourhoods."""
    cfg = cfg_of()
    saved = mr.corridor_spawns
    try:
        mr.corridor_spawns = lambda c: [(y, x + 1.0) for y, x in saved(c)]
        got = mr.corridor_walls(cfg, np.arange(cfg.top_wall_rows + 1))
        assert not np.array_equal(got, z["corr_walls_rand_p2"])
    finally:
        mr.corridor_spawns = saved


def test_reference_kind_resets_keep_players_beyond_two():
    """Players 2 and 3 keep caps, speed and floors across resets."""
    cfg = cfg_of(n_players=4)
    o = OracleSim(cfg, 4, MapSpec(kind="reference"), seed=1)
    o.bombs_cap[:, 2] = 7
    o.spd_g[:, 3] = 1.5
    o.reset_all()
    assert (o.bombs_cap[:, 2] == 7).all() and (o.spd_g[:, 3] == 1.5).all()
    assert torch.equal(o.bombs_cap[:, 0], torch.full((4,), cfg.growth_bombs_start))
