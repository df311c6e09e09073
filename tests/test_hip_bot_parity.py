"""HIP astar bot vs the reference's astar_attack vectors and the oracle
(needs an MI355X).  Bar: actions bit-exact given the same state,
observation, masks and noise uniforms."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import GOLDEN

pytestmark = pytest.mark.gpu

NAMES = ["p70", "p30", "open", "chain"]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("name", NAMES)
def test_hip_bot_matches_reference_vectors(dev, name):
    from qqtsim import HipAstarBot, HipBatchedSim, MapSpec, corridor_training_config

    z = np.load(f"{GOLDEN}/astar_{name}.npz")
    n = z["bot"].shape[1]
    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=0, map_spec=MapSpec(kind="open"))
    bot = HipAstarBot(sim, pid=1)
    for t in range(z["bot"].shape[0]):
        snap = {k: torch.from_numpy(np.ascontiguousarray(z[k][t]))
                for k in ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")}
        sim.load_state_dict(snap)
        got = bot.act(torch.from_numpy(z["obs"][t]), torch.from_numpy(z["mm1"][t]),
                      torch.from_numpy(z["bm1"][t]), 1, uniforms=torch.from_numpy(z["u"][t]))
        np.testing.assert_array_equal(got.cpu().numpy(), z["bot"][t], err_msg=f"{name} tick {t}")


def test_learner_vs_bot_rollout_matches_oracle(dev):
    """Rollout(policy pid 0, astar bot pid 1): MLP actions, bot actions (Philox
    noise) and the stepped state agree with the oracle tick after tick."""
    from oracle import philox
    from oracle.bots import astar_act
    from oracle.policy import mlp_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim import (HipActorCritic, HipAstarBot, HipBatchedSim, MapSpec, Rollout,
                        corridor_training_config)
    from qqtsim.policy import default_init

    n, seed, ticks = 128, 9, 24
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.3, bombs_cap=(2, 3), blast_cap=(2, 4))
    params = default_init(cfg.obs_shape)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipActorCritic(params, device=dev, seed=seed)
    bot = HipAstarBot(sim, pid=1)
    roll = Rollout(sim, net, opponent=bot)
    ora = OracleSim(cfg, n, spec, seed=seed)
    rows = np.arange(n)
    moved = placed = 0
    for t in range(ticks):
        o_obs = ora.observe()
        mm, bm = ora.legal_mask()
        u_pol = philox.uniforms(seed, rows, net.tick, philox.STREAM_POLICY, 4)
        u_bot = torch.from_numpy(philox.uniforms(seed, rows, bot.tick, philox.STREAM_BOT, 5))
        lg = torch.stack([torch.cat([a, b, c[:, None]], 1)
                          for a, b, c in [net.forward(sim.observe(), 0)]], 1).cpu()
        roll.launch_act()
        acts = roll.actions.long().cpu()
        ml, bl, v = mlp_forward(params, o_obs, 0)
        ref = torch.cat([ml, bl, v[:, None]], 1)
        assert float((lg[:, 0] - ref).abs().max()) <= 1e-3
        want = torch.zeros((n, 2, 2), dtype=torch.int64)
        want[:, 0, 0] = torch.from_numpy(sample_masked(lg[:, 0, :5].numpy(), mm[:, 0].numpy(),
                                                       u_pol[:, 0])[0])
        want[:, 0, 1] = torch.from_numpy(sample_masked(lg[:, 0, 5:7].numpy(), bm[:, 0].numpy(),
                                                       u_pol[:, 1])[0])
        st = ora.state_dict()
        want[:, 1] = astar_act(cfg, st, o_obs, mm[:, 1], bm[:, 1], 1, u_bot)
        np.testing.assert_array_equal(acts.numpy(), want.numpy(), err_msg=f"actions tick {t}")
        moved += int((want[:, 1, 0] != 4).sum())
        placed += int(want[:, 1, 1].sum())
        roll.launch_tick()
        ora.step(acts, auto_reset=True)
        got, ref_sd = sim.state_dict(), ora.state_dict()
        for k in sorted(set(got) & set(ref_sd)):
            a = got[k].cpu().numpy()
            np.testing.assert_array_equal(a, ref_sd[k].numpy().astype(a.dtype),
                                          err_msg=f"{k} tick {t}")
    assert moved > 0
    print(f"learner vs bot: {ticks} ticks x {n} envs, bot moves {moved}, placements {placed}")


def test_hip_bot_reach_follows_the_batch_from_call_to_call(dev):
    """The batch-max reach is recomputed on every call (two alternating
    reduction slots): on the hand-built chain states (batch max 5) the bot
    places as the reference does, after lowering every cap to 2 it acts as
    the oracle with reach 2 (which differs), and back at 5 it matches again."""
    from oracle.bots import astar_act
    from qqtsim import HipAstarBot, HipBatchedSim, MapSpec, corridor_training_config

    z = np.load(f"{GOLDEN}/astar_chain.npz")
    n = z["bot"].shape[1]
    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=0, map_spec=MapSpec(kind="open"))
    bot = HipAstarBot(sim, pid=1)
    base = {k: torch.from_numpy(np.ascontiguousarray(z[k][0]))
            for k in ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")}
    low = dict(base)
    low["blast_cap"] = base["blast_cap"].clone()
    low["blast_cap"][:, 1] = 2
    inputs = (torch.from_numpy(z["obs"][0]), torch.from_numpy(z["mm1"][0]),
              torch.from_numpy(z["bm1"][0]))
    u = torch.from_numpy(z["u"][0])
    want_low = astar_act(cfg, low, *inputs, 1, u, reach=2)
    assert not np.array_equal(want_low.numpy(), z["bot"][0])
    for rep in range(2):
        for state, want in ((base, z["bot"][0]), (low, want_low.numpy())):
            sim.load_state_dict(state)
            got = bot.act(*inputs, 1, uniforms=u)
            np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=f"rep {rep}")


@pytest.mark.parametrize("n", [301, 8200])
def test_tick_written_reach_equals_the_batch_max(dev, n):
    """A Rollout's STEP ticks leave the bot's chain-check reach source (the
    batch max of its blast cap, sim/bots.py:477): the largest cap among each
    tick wavefront's envs (groups of 2 up to 8192 envs, 301 -> 151 entries;
    groups of 4 above, 8200 -> 2050), padding zero; the bot's next call reads
    them (reach mode 3) and draws the same actions as a twin bot reducing
    the batch itself (mode 1), and a state change after the tick sends the
    bot back to the reduction."""
    from qqtsim.bots import HipAstarBot
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import BOMB_STRESS_40
    from qqtsim.policy import HipActorCritic, default_init
    from qqtsim.rollout import Rollout
    from qqtsim.sim import HipBatchedSim

    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=3, map_spec=BOMB_STRESS_40)
    net = HipActorCritic(default_init(cfg.obs_shape), device=dev, seed=3)
    bot = HipAstarBot(sim, pid=1)
    roll = Rollout(sim, net, opponent=bot)
    group = 2 if n <= 8192 else 4
    ng = -(-n // group)
    for _ in range(6):
        roll.step()
        torch.cuda.synchronize()
        cap = sim.state_dict()["blast_cap"][:, 1].cpu().numpy()
        pad = np.zeros(ng * group, dtype=cap.dtype)
        pad[:n] = cap
        want = pad.reshape(ng, group).max(axis=1)
        caps = bot._caps.cpu().numpy()
        np.testing.assert_array_equal(caps[:ng], want)
        assert int(np.abs(caps[ng:]).sum()) == 0
        assert int(caps.max()) == int(cap.max())
    assert len(set(sim.state_dict()["blast_cap"][:, 1].tolist())) > 1
    twin = HipAstarBot(sim, pid=1)
    twin.tick = bot.tick
    a3 = torch.zeros_like(roll.actions)
    a1 = torch.zeros_like(roll.actions)
    bot.launch(a3)
    twin.launch(a1)
    assert bot._args.reach_mode == 3 and twin._args.reach_mode == 1
    assert torch.equal(a3[:, 1], a1[:, 1])
    sim.load_state_dict(sim.state_dict())
    bot.launch(a3)
    assert bot._args.reach_mode == 1
