"""The oracle's astar bot against the reference's astar_attack vectors, and
its cost field against a textbook Dijkstra (heap) on small grids."""

from __future__ import annotations

import heapq

import numpy as np
import pytest
import torch

from golden_io import GOLDEN
from oracle.bots import astar_act, cost_field
from qqtsim.config import corridor_training_config

NAMES = ["p70", "p30", "open"]


def _load(name):
    return np.load(f"{GOLDEN}/astar_{name}.npz")


def _state(z, t):
    return {k: torch.from_numpy(np.ascontiguousarray(z[k][t]))
            for k in ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")}


@pytest.mark.parametrize("name", NAMES + ["chain"])
def test_bot_actions_match_reference(name):
    z = _load(name)
    cfg = corridor_training_config()
    for t in range(z["bot"].shape[0]):
        got = astar_act(cfg, _state(z, t), torch.from_numpy(z["obs"][t]),
                        torch.from_numpy(z["mm1"][t]), torch.from_numpy(z["bm1"][t]), 1,
                        torch.from_numpy(z["u"][t]), reach=int(z["reach"][t]))
        np.testing.assert_array_equal(got.numpy(), z["bot"][t], err_msg=f"{name} tick {t}")


def test_default_reach_is_the_batch_max():
    z = _load("open")
    cfg = corridor_training_config()
    t = 10
    args = (cfg, _state(z, t), torch.from_numpy(z["obs"][t]), torch.from_numpy(z["mm1"][t]),
            torch.from_numpy(z["bm1"][t]), 1, torch.from_numpy(z["u"][t]))
    assert int(z["reach"][t]) == int(z["blast_cap"][t][:, 1].max())
    assert torch.equal(astar_act(*args), astar_act(*args, reach=int(z["reach"][t])))


def test_fixtures_exercise_the_bot():
    bots = np.concatenate([_load(n)["bot"].reshape(-1, 2) for n in NAMES])
    assert np.bincount(bots[:, 0], minlength=5).min() > 100
    assert bots[:, 1].sum() > 50


@pytest.mark.parametrize("name", NAMES)
def test_cost_fields_match_reference(name):
    z = _load(name)
    for j, t in enumerate(z["field_tick"]):
        st = _state(z, t)
        obs = torch.from_numpy(z["obs"][t])
        danger = obs.float()[:, 5]
        block = st["wall"] | st["brick"] | (st["fuse"] > 0)
        vs = cost_field(danger < 0.35, danger, block)
        np.testing.assert_array_equal(vs.numpy(), z["v_safe"][j], err_msg=f"V_safe tick {t}")
        n, h, w = danger.shape
        r0 = st["pos"][:, 0, 0].floor().long().clamp(0, h - 1)
        c0 = st["pos"][:, 0, 1].floor().long().clamp(0, w - 1)
        src = torch.zeros(n, h * w, dtype=torch.bool)
        src[torch.arange(n), r0 * w + c0] = st["alive"][:, 0]
        vo = cost_field(src.view(n, h, w), danger, block)
        np.testing.assert_array_equal(vo.numpy(), z["v_opp"][j], err_msg=f"V_opp tick {t}")


def _dijkstra(src, cost, blocked, h, w):
    """Textbook Dijkstra with the relaxation d(v) = d(u) + cost(v) in float32;
    sources start at 0 (even on blocked cells), blocked cells are never
    entered."""
    dist = np.full(h * w, np.inf, dtype=np.float32)
    heap = []
    for v in np.flatnonzero(src):
        dist[v] = np.float32(0.0)
        heapq.heappush(heap, (0.0, int(v)))
    while heap:
        d, u = heapq.heappop(heap)
        if d > dist[u]:
            continue
        r, c = divmod(u, w)
        for dr, dc in ((-1, 0), (1, 0), (0, -1), (0, 1)):
            rr, cc = r + dr, c + dc
            if 0 <= rr < h and 0 <= cc < w:
                v = rr * w + cc
                if blocked[v]:
                    continue
                nd = np.float32(dist[u] + cost[v])
                if nd < dist[v]:
                    dist[v] = nd
                    heapq.heappush(heap, (float(nd), v))
    return dist


def test_cost_field_equals_textbook_dijkstra():
    rng = np.random.default_rng(0)
    for trial in range(200):
        h, w = int(rng.integers(2, 8)), int(rng.integers(2, 8))
        danger = (rng.random((1, h, w)) * (rng.random((1, h, w)) < 0.4)).astype(np.float32)
        blocked = rng.random((1, h, w)) < 0.25
        src = rng.random((1, h, w)) < 0.15
        got = cost_field(torch.from_numpy(src), torch.from_numpy(danger),
                         torch.from_numpy(blocked))[0].numpy()
        cost = (np.float32(1.0) + np.float32(2.0) * danger.reshape(-1)).astype(np.float32)
        want = _dijkstra(src.reshape(-1), cost, blocked.reshape(-1), h, w)
        np.testing.assert_array_equal(got, want, err_msg=f"trial {trial}")


def test_planted_cost_weight_fails():
    z = _load("open")
    dsum = [float(z["obs"][t][:, 5].astype(np.float32).sum()) for t in z["field_tick"]]
    j = int(np.argmax(dsum))
    t = int(z["field_tick"][j])
    st = _state(z, t)
    danger = torch.from_numpy(z["obs"][t]).float()[:, 5]
    block = st["wall"] | st["brick"] | (st["fuse"] > 0)
    vs = cost_field(danger < 0.35, danger, block, lam=3.0)
    assert not np.array_equal(vs.numpy(), z["v_safe"][j])


def test_planted_own_cap_reach_fails():
    """The reference walks the chain check out to the batch-max blast cap
    (hand-built states: own cap 2, batch max 5, a short-fuse bomb 1..5 cells
    out); a bot limited to its own cap places differently."""
    z = _load("chain")
    cfg = corridor_training_config()
    base = (cfg, _state(z, 0), torch.from_numpy(z["obs"][0]), torch.from_numpy(z["mm1"][0]),
            torch.from_numpy(z["bm1"][0]), 1, torch.from_numpy(z["u"][0]))
    assert int(z["reach"][0]) == 5
    assert z["bot"][0][:, 1].sum() > 0
    own = astar_act(*base, reach=2)
    assert not np.array_equal(own.numpy(), z["bot"][0])


def test_flee_mode_actions_match_reference():
    """Behaviour modes (sim/bots.py:433-443, 496-503): with the fixture's
    per-env approach / flee modes the oracle reproduces the reference's
    decisions; ignoring the modes does not (the fixture discriminates), and
    it holds placements of both modes."""
    z = np.load(f"{GOLDEN}/astar_flee.npz")
    cfg = corridor_training_config()
    assert 0 < int(z["mode"].sum()) < z["mode"].size
    differs = 0
    for t in range(z["bot"].shape[0]):
        args = (cfg, _state(z, t), torch.from_numpy(z["obs"][t]), torch.from_numpy(z["mm1"][t]),
                torch.from_numpy(z["bm1"][t]), 1, torch.from_numpy(z["u"][t]))
        got = astar_act(*args, mode=torch.from_numpy(z["mode"][t]).long())
        np.testing.assert_array_equal(got.numpy(), z["bot"][t], err_msg=f"tick {t}")
        differs += int((astar_act(*args).numpy() != z["bot"][t]).any(axis=1).sum())
    assert differs > 100
    places = z["bot"][..., 1]
    assert places[z["mode"] == 0].sum() > 0 and places[z["mode"] == 1].sum() > 0


def test_mode_ticker_laws():
    """The mode ticker (sim/bots.py:241-264): timers count down by one per
    call; only on calls that are multiples of 16, and only for envs at or
    below 0, does a switch happen, to a timer on 60 .. 239 and a mode that is
    1 about half the time."""
    from oracle.bots import mode_tick

    n = 4096
    g = torch.Generator().manual_seed(5)
    mode = torch.randint(0, 2, (n,), generator=g, dtype=torch.int8)
    timer = torch.randint(-20, 40, (n,), generator=g, dtype=torch.int32)
    new_modes = []
    for count in range(1, 65):
        m2, t2 = mode_tick(mode, timer, count, seed=9)
        due = (timer - 1 <= 0) & (count % 16 == 0)
        assert torch.equal(t2[~due], timer[~due] - 1)
        assert torch.equal(m2[~due], mode[~due])
        if due.any():
            assert int(t2[due].min()) >= 60 and int(t2[due].max()) <= 239
            new_modes.append(m2[due])
        mode, timer = m2, t2
    drawn = torch.cat(new_modes).float()
    assert drawn.numel() > 1000 and abs(float(drawn.mean()) - 0.5) < 0.05
