"""HIP kernels at the measured launch shapes against the oracle (needs an
MI355X).

The tick and act kernels deal 64-env row blocks to the XCDs
(row block = (seq / workgroups per block) * 8 + xcd); above 512 envs the
first term is non-zero, so these tests run the benchmark sizes themselves:

* the self-play MLP rollout at 5632 envs (the headline workload's map law:
  70% bricks, spawn swap), short episodes so auto-reset runs, once with the
  training corridor rules and once with a 5-tick fuse so bombs explode,
  chain and damage within the run: observation, masks, sampled actions
  (the host sampler on the kernel's logits with the same Philox uniforms),
  logits against the oracle's forward, every state field, done and reward;
* the learner (MLP, player 0) vs astar bot (player 1) rollout at 5632 envs:
  the bot kernel over every row block, the batch-max reach and the
  single-player act kernel at their measured launch shapes;
* the bomb-stress tick at 16384 envs (injected unmasked actions, 40%
  bricks, caps 1-4 / 2-5, 5-tick fuse), bit-exact state tick after tick;
* the reference-written deep-chain fixture (`tests/golden/deep_chain.npz`:
  a 13-bomb row, a snake and a cross with ranges 2-7, chains deeper than
  the 8 relay rounds) through `HipBatchedSim`: the float32 danger map
  before and after the tick, the exploded bombs, the flame cover, fuses and
  rewards, exactly as the reference computed them.

Bar: integer state, observation bits, masks, actions exact; positions exact;
rewards within 1e-5; logits within 1e-3 (north star)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import GOLDEN

pytestmark = pytest.mark.gpu

REWARD_ATOL = 1e-5
LOGIT_ATOL = 1e-3
STATE_KEYS = ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast", "alive",
              "hp", "since_bomb", "t", "bombs_cap", "blast_cap", "invuln", "combo",
              "last_hit", "pending_lost", "pos", "spd_g", "lo_bombs", "lo_blast", "lo_spd",
              "crate_prob")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.set_num_threads(16)
    return torch.device("cuda:0")


def _same_state(hip, ora, tick):
    got, ref = hip.state_dict(), ora.state_dict()
    for k in STATE_KEYS:
        a = got[k].cpu().numpy()
        b = ref[k].cpu().numpy() if torch.is_tensor(ref[k]) else np.asarray(ref[k])
        np.testing.assert_array_equal(a, b.astype(a.dtype), err_msg=f"{k} after tick {tick}")


@pytest.mark.parametrize("rules", ["training", "short_fuse"])
def test_mlp_rollout_5632_matches_oracle(dev, rules):
    from oracle import philox
    from oracle.policy import mlp_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim import HipActorCritic, HipBatchedSim, MapSpec, Rollout, corridor_training_config
    from qqtsim.policy import default_init

    n, seed = 5632, 21
    cfg = (corridor_training_config(max_steps=6) if rules == "training" else
           corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=12))
    ticks = 16
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    params = default_init(cfg.obs_shape)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipActorCritic(params, device=dev, seed=seed)
    roll = Rollout(sim, net)
    ora = OracleSim(cfg, n, spec, seed=seed)
    rows = np.arange(n)
    resets = exploded = 0
    for t in range(ticks):
        print(f"[large] rollout {rules} n={n} tick {t}", flush=True)
        o_obs = ora.observe()
        obs = sim.observe()
        np.testing.assert_array_equal(obs.cpu().numpy().view(np.uint16),
                                      o_obs.numpy().view(np.uint16), err_msg=f"obs {t}")
        mm, bm = ora.legal_mask()
        hm, hb = sim.legal_mask()
        assert torch.equal(hm.cpu(), mm) and torch.equal(hb.cpu(), bm), t
        lg = torch.stack([torch.cat([ml, bl, v[:, None]], 1)
                          for ml, bl, v in (net.forward(obs, pid) for pid in range(2))], 1).cpu()
        u = philox.uniforms(seed, rows, net.tick, philox.STREAM_POLICY, 4)
        roll.launch_act()
        acts = roll.actions.long().cpu()
        want = torch.zeros((n, 2, 2), dtype=torch.int64)
        for pid in range(2):
            if t % 4 == 0:
                ml, bl, v = mlp_forward(params, o_obs, pid)
                ref = torch.cat([ml, bl, v[:, None]], 1)
                err = float((lg[:, pid] - ref).abs().max())
                assert err <= LOGIT_ATOL, f"tick {t} pid {pid}: logit error {err:.2e}"
            want[:, pid, 0] = torch.from_numpy(sample_masked(
                lg[:, pid, :5].numpy(), mm[:, pid].numpy(), u[:, 2 * pid])[0])
            want[:, pid, 1] = torch.from_numpy(sample_masked(
                lg[:, pid, 5:7].numpy(), bm[:, pid].numpy(), u[:, 2 * pid + 1])[0])
        assert torch.equal(acts, want), f"tick {t}: sampled actions differ"
        roll.launch_tick()
        o_rew, o_done, o_info = ora.step(acts, auto_reset=True)
        resets += int(o_done.sum())
        exploded += int(o_info["trig"].sum())
        _same_state(sim, ora, t)
        np.testing.assert_array_equal(roll.done.cpu().numpy(), o_done.numpy(), err_msg=f"done {t}")
        r_err = float((roll.reward.cpu() - o_rew).abs().max())
        assert r_err <= REWARD_ATOL, f"tick {t}: reward error {r_err:.2e}"
    assert resets > 0
    if rules == "short_fuse":
        assert exploded > 0
    print(f"rollout {rules}: {ticks} ticks x {n} envs exact, {resets} resets, "
          f"{exploded} bombs exploded")


def test_learner_vs_astar_5632_matches_oracle(dev):
    """The learner-vs-astar rollout at its measured size (5632 envs, 70%
    bricks, spawn swap): the MLP plays player 0 and the astar bot player 1
    (`HipAstarBot`: bot_kernel over every 44-env row block, the batch-max
    reach of reach_kernel, and the single-player act kernel at 5632 rows).
    A 5-tick fuse and 10-tick episodes make bombs explode and every env
    auto-reset within the run.  Every tick: the learner's logits (every
    fourth tick) against the oracle forward, its sampled actions against the
    host sampler on the kernel's logits, the bot's actions against the
    oracle bot with the same Philox noise, then every state field, done and
    reward after the tick."""
    from oracle import philox
    from oracle.bots import astar_act
    from oracle.policy import mlp_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim import (HipActorCritic, HipAstarBot, HipBatchedSim, MapSpec, Rollout,
                        corridor_training_config)
    from qqtsim.policy import default_init

    n, seed, ticks = 5632, 31, 12
    cfg = corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=10)
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    params = default_init(cfg.obs_shape)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipActorCritic(params, device=dev, seed=seed)
    bot = HipAstarBot(sim, pid=1)
    roll = Rollout(sim, net, opponent=bot)
    ora = OracleSim(cfg, n, spec, seed=seed)
    rows = np.arange(n)
    resets = exploded = bot_moves = bot_bombs = 0
    for t in range(ticks):
        print(f"[large] learner vs astar n={n} tick {t}", flush=True)
        o_obs = ora.observe()
        mm, bm = ora.legal_mask()
        u_pol = philox.uniforms(seed, rows, net.tick, philox.STREAM_POLICY, 4)
        u_bot = torch.from_numpy(philox.uniforms(seed, rows, bot.tick, philox.STREAM_BOT, 5))
        ml, bl, v = net.forward(sim.observe(), 0)
        lg = torch.cat([ml, bl, v[:, None]], 1).cpu()
        if t % 4 == 0:
            rml, rbl, rv = mlp_forward(params, o_obs, 0)
            err = float((lg - torch.cat([rml, rbl, rv[:, None]], 1)).abs().max())
            assert err <= LOGIT_ATOL, f"tick {t}: logit error {err:.2e}"
        roll.launch_act()
        acts = roll.actions.long().cpu()
        want = torch.zeros((n, 2, 2), dtype=torch.int64)
        want[:, 0, 0] = torch.from_numpy(sample_masked(lg[:, :5].numpy(), mm[:, 0].numpy(),
                                                       u_pol[:, 0])[0])
        want[:, 0, 1] = torch.from_numpy(sample_masked(lg[:, 5:7].numpy(), bm[:, 0].numpy(),
                                                       u_pol[:, 1])[0])
        want[:, 1] = astar_act(cfg, ora.state_dict(), o_obs, mm[:, 1], bm[:, 1], 1, u_bot)
        np.testing.assert_array_equal(acts[:, 0].numpy(), want[:, 0].numpy(),
                                      err_msg=f"learner actions tick {t}")
        np.testing.assert_array_equal(acts[:, 1].numpy(), want[:, 1].numpy(),
                                      err_msg=f"bot actions tick {t}")
        bot_moves += int((want[:, 1, 0] != 4).sum())
        bot_bombs += int(want[:, 1, 1].sum())
        roll.launch_tick()
        o_rew, o_done, o_info = ora.step(acts, auto_reset=True)
        resets += int(o_done.sum())
        exploded += int(o_info["trig"].sum())
        _same_state(sim, ora, t)
        np.testing.assert_array_equal(roll.done.cpu().numpy(), o_done.numpy(), err_msg=f"done {t}")
        r_err = float((roll.reward.cpu() - o_rew).abs().max())
        assert r_err <= REWARD_ATOL, f"tick {t}: reward error {r_err:.2e}"
    # (the bot's placements are pinned by the reference's astar fixtures;
    # in these short episodes it may place none)
    assert resets > 0 and exploded > 0 and bot_moves > 0
    print(f"learner vs astar: {ticks} ticks x {n} envs exact, {resets} resets, {exploded} "
          f"bombs exploded, bot moves {bot_moves}, bot bombs {bot_bombs}")


def test_bomb_stress_16384_matches_oracle(dev):
    from oracle.sim import OracleSim
    from qqtsim import BOMB_STRESS_40, HipBatchedSim, corridor_training_config
    from qqtsim.rollout import TickLoop

    n, ticks, seed = 16384, 16, 8
    cfg = corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=12)
    hip = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=BOMB_STRESS_40)
    ora = OracleSim(cfg, n, BOMB_STRESS_40, seed=seed)
    loop = TickLoop(hip)
    g = torch.Generator().manual_seed(seed)
    _same_state(hip, ora, -1)
    resets = exploded = 0
    for t in range(ticks):
        print(f"[large] stress n={n} tick {t}", flush=True)
        mv = torch.randint(0, 5, (n, 2), generator=g)
        bb = (torch.rand((n, 2), generator=g) < 0.5).long()
        act = torch.stack([mv, bb], -1)
        r1, d1, info = ora.step(act, auto_reset=True)
        loop.launch_tick(act.to(torch.int8).to(dev).contiguous())
        resets += int(d1.sum())
        exploded += int(info["trig"].sum())
        np.testing.assert_array_equal(hip._done.cpu().numpy().astype(bool), d1.numpy(),
                                      err_msg=f"done {t}")
        assert float((hip._reward.cpu() - r1).abs().max()) <= REWARD_ATOL, f"reward {t}"
        _same_state(hip, ora, t)
    np.testing.assert_array_equal(hip.observe().cpu().numpy().view(np.uint16),
                                  ora.observe().numpy().view(np.uint16))
    assert resets > 0 and exploded > 0
    print(f"stress: {ticks} ticks x {n} envs exact, {resets} resets, {exploded} bombs exploded")


def test_deep_chain_fixture_through_hip(dev):
    from qqtsim import HipBatchedSim, MapSpec, corridor_training_config

    z = np.load(GOLDEN + "/deep_chain.npz")
    cfg = corridor_training_config()
    n = z["init_fuse"].shape[0]
    sim = HipBatchedSim(cfg, n, device=dev, seed=1, map_spec=MapSpec(kind="open"))
    init = {k: torch.from_numpy(np.ascontiguousarray(z["init_" + k]))
            for k in ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast",
                      "pos", "alive", "hp", "since_bomb", "t", "bombs_cap", "blast_cap",
                      "spd_g", "invuln", "combo", "last_hit", "pending_lost")}
    init.update(lo_bombs=init["bombs_cap"], lo_blast=init["blast_cap"], lo_spd=init["spd_g"],
                crate_prob=torch.full((n,), cfg.growth_crate_prob), map_kind=torch.zeros(n))
    sim.load_state_dict(init)
    sim.resolve_tiers = int(z["resolve_hint"])
    d0 = sim.danger().cpu().numpy()
    np.testing.assert_array_equal(d0, z["danger_init"])
    # the observation's danger channel (2P + 1) is the float16 of that map
    obs = sim.observe().cpu().numpy()
    np.testing.assert_array_equal(obs[:, 5].view(np.uint16),
                                  z["danger_init"].astype(np.float16).view(np.uint16))
    r, d, info = sim.step(torch.from_numpy(z["actions"]), auto_reset=False,
                          crate_u=torch.zeros(2, 2, n))
    np.testing.assert_array_equal(info["trig"].cpu().numpy(), z["trig"])
    np.testing.assert_array_equal(info["blast"].cpu().numpy(), z["covered"])
    assert float(np.abs(r.cpu().numpy() - z["reward"]).max()) <= REWARD_ATOL
    sd = sim.state_dict()
    for k in ("fuse", "owner", "bomb_blast", "brick", "crate", "hp", "alive"):
        np.testing.assert_array_equal(sd[k].cpu().numpy(),
                                      z["state_" + k].astype(sd[k].cpu().numpy().dtype),
                                      err_msg=k)
    np.testing.assert_array_equal(sim.danger().cpu().numpy(), z["danger"])
    assert int(z["trig"][0].sum()) == 9       # 1 + 8 relay rounds, the rest of the row waits
