"""The reference's reset map modes on the device (needs an MI355X): resets
with MapSpec(kind="reference") against the oracle's restatement
(oracle/maps_ref.py, pinned to the reference's generators) on the same
Philox draws, bit-exact: every state tensor, the observation and the masks
after reset_all, after a partial reset_, and through rollouts whose short
episodes auto-reset into all three map kinds."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = {
    # mixed kinds, obstacles, edge segments, opponent x opp_hist_mult
    "mixed_p2": dict(cfg=dict(pure_open_fraction=0.1, open_fraction=0.3, ring_fraction=0.3,
                              open_obstacle_max=4, wall_density=0.45), boost=1),
    # four players (players 2 and 3 keep their caps), fixed top rows, opponent tier 2
    "mixed_p4": dict(cfg=dict(n_players=4, corridor_width=7, random_wall_rows=False,
                              open_fraction=0.4, ring_fraction=0.3, open_obstacle_max=3),
                     boost=2),
    # open map mode (no corridor rules), three players
    "mode_open_p3": dict(cfg=dict(n_players=3, map_mode="open", open_obstacle_max=5), boost=0),
}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _pair(dev, name, n, seed, **over):
    from oracle.sim import OracleSim
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.sim import HipBatchedSim

    c = CASES[name]
    cfg = corridor_training_config(**dict(c["cfg"], **over))
    spec = MapSpec(kind="reference")
    ora = OracleSim(cfg, n, spec, seed=seed)
    ora.set_opp_boost(c["boost"])
    ora.reset_all()
    hip = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    hip.set_opp_boost(c["boost"])
    hip.reset_all()
    return cfg, hip, ora


def _same_state(hip, ora, msg):
    got, want = hip.state_dict(), ora.state_dict()
    for k in sorted(set(got) & set(want)):
        g = got[k].cpu().numpy()
        np.testing.assert_array_equal(g, want[k].numpy().astype(g.dtype), err_msg=f"{k} {msg}")


def _same_views(hip, ora, msg):
    np.testing.assert_array_equal(hip.observe().cpu().numpy().view(np.uint16),
                                  ora.observe().numpy().view(np.uint16), err_msg=f"obs {msg}")
    hm, hb = hip.legal_mask()
    om, ob = ora.legal_mask()
    np.testing.assert_array_equal(hm.cpu().numpy(), om.numpy(), err_msg=f"mm {msg}")
    np.testing.assert_array_equal(hb.cpu().numpy(), ob.numpy(), err_msg=f"bm {msg}")


@pytest.mark.parametrize("name", list(CASES))
def test_reset_all_and_partial_reset_match_oracle(dev, name):
    cfg, hip, ora = _pair(dev, name, 257, seed=4)
    _same_state(hip, ora, "reset_all")
    _same_views(hip, ora, "reset_all")
    kinds = ora.map_kind.numpy()
    if cfg.map_mode == "corridor":
        assert set(np.unique(kinds)) == {0, 1, 2}, "all three map kinds drawn"
    mask = torch.zeros(257, dtype=torch.bool)
    mask[::3] = True
    ora.reset_(mask)
    hip.reset_(mask.to(dev))
    _same_state(hip, ora, "reset_")
    _same_views(hip, ora, "reset_")


@pytest.mark.parametrize("name", ["mixed_p2", "mixed_p4"])
def test_rollout_with_auto_resets_matches_oracle(dev, name):
    """Random legal actions, 24-tick episodes: every auto-reset draws a new
    reference map; state, rewards, done, observation and masks every tick."""
    from oracle import philox
    from oracle.policy import sample_masked

    n, seed = 96, 9
    cfg, hip, ora = _pair(dev, name, n, seed, max_steps=24, max_hp=2, invuln_ticks=3)
    p = cfg.n_players
    resets = 0
    for t in range(60):
        mm, bm = ora.legal_mask()
        u = philox.uniforms(seed, np.arange(n), t, philox.STREAM_RANDOM_ACT, 2 * p)
        a = np.zeros((n, p, 2), dtype=np.int64)
        for i in range(p):
            a[:, i, 0] = sample_masked(mm[:, i].numpy().astype(np.float32), mm[:, i].numpy(),
                                       u[:, 2 * i])[0]
            a[:, i, 1] = sample_masked(bm[:, i].numpy().astype(np.float32), bm[:, i].numpy(),
                                       u[:, 2 * i + 1])[0]
        act = torch.from_numpy(a)
        r1, d1, _ = ora.step(act, auto_reset=True)
        r2, d2, _ = hip.step(act, auto_reset=True)
        resets += int(d1.sum())
        np.testing.assert_array_equal(d2.cpu().numpy(), d1.numpy(), err_msg=f"done {t}")
        assert float((r2.cpu() - r1).abs().max()) <= 1e-5, f"reward {t}"
        _same_state(hip, ora, f"tick {t}")
        _same_views(hip, ora, f"tick {t}")
    assert resets >= n, "every env went through at least one auto-reset"


def test_opp_boost_is_validated(dev):
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.sim import HipBatchedSim

    hip = HipBatchedSim(corridor_training_config(), 4, device=dev, map_spec=MapSpec(kind="reference"))
    with pytest.raises(ValueError):
        hip.set_opp_boost(3)
