"""Recycle flush (BatchedSim.flush_recycle, sim/torch_sim.py:549-596) in the
oracle: the exclusion set against the reference's geometry worked out by
hand, and the flush's laws (conservation, placement, reset of the counts,
uniform choice among the free cells)."""

from __future__ import annotations

import numpy as np
import torch

from oracle.sim import OracleSim, recycle_exclusion
from qqtsim.config import corridor_training_config
from qqtsim.maps import MapSpec
from qqtsim.maps import recycle_exclusion as product_exclusion


def _expected_exclusion_13x13_p2():
    """From sim/torch_sim.py:455-533 and sim/config.py:561-605 for 13x13, two
    players, corridor_width 5, top_wall_rows 4: open spawns (6.5, 4.5) and
    (6.5, 8.5); corridor spawns (8.5, 5.5) and (8.5, 8.5); ring corners
    (1.5, 1.5) and (1.5, 12.5); each cell with its 4-neighbours; the cross
    rows 5, 6 and columns 5, 6."""
    cells = set()
    for r, c in ((6, 4), (6, 8), (8, 5), (8, 8), (1, 1), (1, 12)):
        for dr, dc in ((0, 0), (-1, 0), (1, 0), (0, -1), (0, 1)):
            if 0 <= r + dr < 13 and 0 <= c + dc < 13:
                cells.add((r + dr) * 13 + c + dc)
    for i in range(13):
        for j in (5, 6):
            cells.add(j * 13 + i)
            cells.add(i * 13 + j)
    return sorted(cells)


def test_exclusion_matches_the_reference_geometry():
    cfg = corridor_training_config()
    want = _expected_exclusion_13x13_p2()
    assert list(np.flatnonzero(recycle_exclusion(cfg))) == want
    assert product_exclusion(cfg) == want


def test_planted_missing_cross_fails():
    want = set(_expected_exclusion_13x13_p2())
    no_cross = {c for c in want if not (c // 13 in (5, 6) or c % 13 in (5, 6))}
    assert no_cross != want


def _sim(n=64, seed=3):
    cfg = corridor_training_config()
    sim = OracleSim(cfg, n, MapSpec(kind="pillars", brick_p=0.4), seed=seed)
    return cfg, sim


def test_flush_places_pending_crates_on_free_cells_and_resets_counts():
    cfg, sim = _sim()
    n, hw = sim.num_envs, cfg.n_cells
    g = torch.Generator().manual_seed(0)
    pend = torch.randint(0, 4, (n, 2), generator=g)
    pend[:, 1] = 0                               # one player: exact conservation
    sim.pending_lost.copy_(pend)
    free = (~sim.wall.view(n, hw) & ~sim.brick.view(n, hw)).numpy() & ~recycle_exclusion(cfg)
    sim.flush_recycle(0)
    rec = sim.recycle.view(n, hw).numpy()
    assert not (rec & ~free).any()
    assert np.array_equal(sim.crate.view(n, hw).numpy(), rec)   # started with no crates
    want = np.minimum(pend[:, 0].numpy(), free.sum(1))
    np.testing.assert_array_equal(rec.sum(1), want)
    assert int(sim.pending_lost.abs().sum()) == 0


def test_two_players_draw_independently():
    cfg, sim = _sim(n=256)
    n, hw = sim.num_envs, cfg.n_cells
    sim.pending_lost.fill_(3)
    sim.flush_recycle(5)
    got = sim.recycle.view(n, hw).numpy().sum(1)
    assert (got >= 3).all() and (got <= 6).all()
    assert (got < 6).any(), "two independent 3-subsets of ~60 cells overlap sometimes"


def test_flush_choice_is_uniform_over_free_cells():
    cfg, sim = _sim(n=1)
    hw = cfg.n_cells
    base = sim.state_dict()
    free = (~sim.wall.view(hw) & ~sim.brick.view(hw)).numpy() & ~recycle_exclusion(cfg)
    counts = np.zeros(hw)
    draws = 3000
    for epoch in range(draws):
        sim.load_state_dict(base)
        sim.pending_lost[0, 0] = 1
        sim.flush_recycle(epoch)
        counts += sim.recycle.view(hw).numpy()
    assert counts[~free].sum() == 0
    f = counts[free]
    expect = draws / free.sum()
    chi2 = float(((f - expect) ** 2 / expect).sum())
    dof = int(free.sum()) - 1
    assert chi2 < dof + 5 * np.sqrt(2 * dof), (chi2, dof)


def test_flush_epochs_draw_differently():
    cfg, sim = _sim(n=32)
    base = sim.state_dict()
    picks = []
    for epoch in (0, 1):
        sim.load_state_dict(base)
        sim.pending_lost.fill_(2)
        sim.flush_recycle(epoch)
        picks.append(sim.recycle.clone())
    assert not torch.equal(picks[0], picks[1])
