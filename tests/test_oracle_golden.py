"""Pin the CPU oracle to the reference's own vectors.

* The reference's single-state fixtures (deploy/ref_state.json, 60 states of
  deploy/sweep_states.json; checked by web/parity.js:29-95 at 1e-4 float /
  exact int): danger, 14-channel fp32 observation, masks, explosion cover.
* Multi-tick trajectories written from the reference implementation
  (tests/golden/gen_reference_vectors.py): full state, reward, done, info,
  masks and observations after every tick must be bit-exact.
* The MLP actor/critic forward and evaluate outputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import TRAJ_CFG, json_state_tensors, json_states, mlp_params, state_at, traj
from oracle.grid import danger_map, resolve_explosions
from oracle.obs import encode_obs, legal_mask
from oracle.policy import exp_f32, log_f32, mlp_forward
from oracle.sim import OracleSim
from qqtsim.config import SimConfig, corridor_training_config
from qqtsim.maps import MapSpec

FIXTURE_CFG = SimConfig(height=13, width=13, n_players=2, map_mode="corridor",
                        speed=3.0, max_steps=1800, obs_extra_enabled=True, obs_fp16=False)


def _fixture_outputs(st):
    s = json_state_tensors(st)
    cfg = FIXTURE_CFG
    bmap = torch.where(s["bomb_blast"] > 0, s["bomb_blast"].long(),
                       torch.full_like(s["bomb_blast"].long(), cfg.blast))
    dng = danger_map(s["fuse"], s["wall"], bmap, cfg.fuse, s["brick"], cfg.max_chain)
    obs = encode_obs(cfg, s["wall"], s["fuse"], s["owner"], s["pos"], s["alive"], s["t"],
                     s["brick"], s["bomb_blast"], s["crate"], s["invuln"], s["bombs_cap"],
                     danger=dng)
    mm, bm = legal_mask(cfg, s["wall"], s["fuse"], s["owner"], s["pos"], s["alive"],
                        s["brick"], s["bombs_cap"])
    cov, trig = resolve_explosions(s["fuse"], s["owner"], s["wall"], bmap, cfg.max_chain,
                                   s["brick"])
    return dng, obs, mm, bm, cov, trig


@pytest.mark.parametrize("name", ["ref_state.json", "sweep_states.json"])
def test_oracle_matches_reference_json_fixtures(name):
    for st in json_states(name):
        dng, obs, mm, bm, cov, trig = _fixture_outputs(st)
        np.testing.assert_array_equal(dng.flatten().numpy(), np.float32(st["danger"]))
        np.testing.assert_array_equal(obs.flatten().numpy(), np.float32(st["obs"]))
        np.testing.assert_array_equal(mm[0].int().numpy(), np.array(st["mm"]))
        np.testing.assert_array_equal(bm[0].int().numpy(), np.array(st["bm"]))
        np.testing.assert_array_equal(cov.flatten().int().numpy(), np.array(st["covered"]))
        np.testing.assert_array_equal(trig.flatten().int().numpy(), np.array(st["triggered"]))


def test_ref_state_fixture_has_a_real_chain():
    """ref_state.json is the only reference fixture with in-play bombs: its
    fuse-0 bomb at (5,5) ignites (5,7), the (8,9) bomb stays live."""
    st = json_states("ref_state.json")[0]
    trig = np.array(st["triggered"]).reshape(13, 13)
    assert trig[5, 5] and trig[5, 7] and not trig[8, 9]


def oracle_for(z, name):
    cfg = corridor_training_config(**TRAJ_CFG[name])
    n = z["init_fuse"].shape[0]
    s = OracleSim(cfg, n, MapSpec(), seed=0)
    init = state_at(z, 0)
    s.load_state_dict(init)
    s.lo_bombs.copy_(init["bombs_cap"])
    s.lo_blast.copy_(init["blast_cap"])
    s.lo_spd.copy_(init["spd_g"])
    s.resolve_tiers = int(z["resolve_hint"])
    return s


@pytest.mark.parametrize("name", list(TRAJ_CFG))
def test_oracle_replays_reference_trajectory_bit_exact(name):
    z = traj(name)
    s = oracle_for(z, name)
    ticks = z["actions"].shape[0]
    for t in range(ticks):
        mm, bm = s.legal_mask()
        np.testing.assert_array_equal(mm.numpy(), z["mm"][t], err_msg=f"move mask tick {t}")
        np.testing.assert_array_equal(bm.numpy(), z["bm"][t], err_msg=f"bomb mask tick {t}")
        obs = s.observe()[:4].numpy()
        np.testing.assert_array_equal(obs.view(np.uint16), z["obs"][t].view(np.uint16),
                                      err_msg=f"obs tick {t}")
        r, d, info = s.step(torch.from_numpy(z["actions"][t]), auto_reset=False,
                            crate_u=torch.from_numpy(z["crate_u"][t]))
        for k in ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast", "pos",
                  "alive", "hp", "since_bomb", "t", "bombs_cap", "blast_cap", "spd_g",
                  "invuln", "combo", "last_hit", "pending_lost"):
            np.testing.assert_array_equal(getattr(s, k).numpy(), z["state_" + k][t],
                                          err_msg=f"{k} tick {t}")
        np.testing.assert_array_equal(r.numpy(), z["reward"][t], err_msg=f"reward tick {t}")
        np.testing.assert_array_equal(d.numpy(), z["done"][t])
        np.testing.assert_array_equal(info["blast"].numpy(), z["covered"][t])
        np.testing.assert_array_equal(info["trig"].numpy(), z["trig"][t])
        np.testing.assert_array_equal(info["died"].numpy(), z["died"][t])
        np.testing.assert_array_equal(info["winner"].numpy(), z["winner"][t])
        np.testing.assert_array_equal(info["n_alive"].numpy(), z["n_alive"][t])
        np.testing.assert_array_equal(s.danger().numpy(), z["danger"][t])


def test_trajectories_exercise_the_rules():
    """The golden set must actually contain the events it is meant to pin."""
    dm = traj("deathmatch")
    assert dm["died"].sum() > 20 and dm["done"].any()
    assert (dm["winner"].sum() > 0)
    p70 = traj("pillars70")
    assert (p70["state_blast_cap"][-1] > 2).any(), "crate growth"
    assert (p70["state_pending_lost"][-1] > 0).any() or (p70["state_crate"].any())
    st = traj("stress40")
    assert int(st["resolve_hint"]) == 5
    assert st["trig"].sum() > 100


def test_oracle_deep_chain_truncates_like_reference():
    """Chains needing more than 8 relay rounds stop at 1 + 8 bombs in the
    tick (sim/torch_sim.py:825-830) while danger still marks the tail."""
    z = np.load(__import__("golden_io").GOLDEN + "/deep_chain.npz")
    cfg = corridor_training_config()
    s = OracleSim(cfg, 4, MapSpec(kind="open"), seed=1)
    init = {k: torch.from_numpy(np.ascontiguousarray(z["init_" + k]))
            for k in ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast",
                      "pos", "alive", "hp", "since_bomb", "t", "bombs_cap", "blast_cap",
                      "spd_g", "invuln", "combo", "last_hit", "pending_lost")}
    s.load_state_dict(init)
    s.lo_bombs.copy_(init["bombs_cap"])
    s.lo_blast.copy_(init["blast_cap"])
    s.lo_spd.copy_(init["spd_g"])
    s.resolve_tiers = int(z["resolve_hint"])
    np.testing.assert_array_equal(s.danger().numpy(), z["danger_init"])
    r, d, info = s.step(torch.from_numpy(z["actions"]), auto_reset=False,
                        crate_u=torch.zeros(2, 2, 4))
    np.testing.assert_array_equal(info["trig"].numpy(), z["trig"])
    np.testing.assert_array_equal(info["blast"].numpy(), z["covered"])
    np.testing.assert_array_equal(r.numpy(), z["reward"])
    np.testing.assert_array_equal(s.fuse.numpy(), z["state_fuse"])
    np.testing.assert_array_equal(s.danger().numpy(), z["danger"])
    assert int(z["trig"][0].sum()) == 9


def test_oracle_mlp_matches_reference_forward():
    z = np.load(__import__("golden_io").GOLDEN + "/mlp.npz")
    params = mlp_params(z)
    assert sum(v.numel() for v in params.values()) == 345288 == int(z["param_count"])
    obs = torch.from_numpy(z["obs"])
    for pid in range(2):
        ml, bl, v = mlp_forward(params, obs, pid)
        np.testing.assert_array_equal(ml.numpy(), z[f"move_logits_{pid}"])
        np.testing.assert_array_equal(bl.numpy(), z[f"bomb_logits_{pid}"])
        np.testing.assert_array_equal(v.numpy(), z[f"value_{pid}"])


def test_oracle_logp_matches_reference_evaluate():
    """logp of the recorded actions under the masked Categorical
    (train/model.py:215-256) from the oracle's own exp/log."""
    z = np.load(__import__("golden_io").GOLDEN + "/mlp.npz")
    params = mlp_params(z)
    obs = torch.from_numpy(z["obs"])
    neg = np.float32(-3.4028235e38)
    for pid in range(2):
        ml, bl, _ = mlp_forward(params, obs, pid)
        total = np.zeros(obs.shape[0], dtype=np.float32)
        for logits, mask, act in ((ml.numpy(), z["mm"][:, pid], z["actions"][:, pid, 0]),
                                  (bl.numpy(), z["bm"][:, pid], z["actions"][:, pid, 1])):
            lg = np.where(mask, logits, neg).astype(np.float32)
            m = lg.max(1)
            s = exp_f32(lg - m[:, None]).sum(1).astype(np.float32)
            total += (lg[np.arange(len(act)), act] - m) - log_f32(s)
        np.testing.assert_allclose(total, z[f"logp_{pid}"], atol=2e-6)


def test_oracle_cnn_matches_reference_forward():
    """ActorCritic(arch="cnn") (train/model.py:79-96, 186-190): the oracle's
    restatement equals the reference module's forward on 96 recorded
    observations for both players (view permutation on conv0's inputs)."""
    from golden_io import cnn_params
    from oracle.policy import cnn_forward

    z = np.load(__import__("golden_io").GOLDEN + "/cnn.npz")
    params = cnn_params(z)
    assert sum(v.numel() for v in params.values()) == 281744 == int(z["param_count"])
    obs = torch.from_numpy(z["obs"])
    for pid in range(2):
        ml, bl, v = cnn_forward(params, obs, pid)
        np.testing.assert_allclose(ml.numpy(), z[f"move_logits_{pid}"], rtol=0, atol=1e-5)
        np.testing.assert_allclose(bl.numpy(), z[f"bomb_logits_{pid}"], rtol=0, atol=1e-5)
        np.testing.assert_allclose(v.numpy(), z[f"value_{pid}"], rtol=0, atol=1e-5)
    ml0 = cnn_forward(params, obs, 0)[0]
    ml1 = cnn_forward(params, obs, 1)[0]
    assert float((ml0 - ml1).abs().max()) > 1e-3, "the two views differ"
