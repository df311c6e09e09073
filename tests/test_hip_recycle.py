"""Recycle flush on the device (needs an MI355X): HIP against the oracle
bit for bit on states with pending lost growth, and inside the collect loop
at the reference's cadence (train/ppo.py:263-264, :292)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def test_flush_matches_oracle(dev):
    from oracle.sim import OracleSim
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import BOMB_STRESS_40
    from qqtsim.sim import HipBatchedSim

    cfg = corridor_training_config()
    n, seed = 131, 4
    hip = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=BOMB_STRESS_40)
    ora = OracleSim(cfg, n, BOMB_STRESS_40, seed=seed)
    g = torch.Generator().manual_seed(seed)
    for flush in range(3):
        for _ in range(12):       # some bombs, crates and burnt bricks in the state
            mv = torch.randint(0, 5, (n, 2), generator=g)
            bb = (torch.rand((n, 2), generator=g) < 0.3).long()
            act = torch.stack([mv, bb], -1)
            ora.step(act, auto_reset=True)
            hip.step(act, auto_reset=True)
        pend = torch.randint(0, 5, (n, 2), generator=g)
        pend[torch.rand(n, generator=g) < 0.3] = 0
        snap = ora.state_dict()
        snap["pending_lost"] = pend
        ora.load_state_dict(snap)
        hip.load_state_dict(snap)
        assert hip.flushes == flush
        ora.flush_recycle(flush)
        hip.flush_recycle()
        got, want = hip.state_dict(), ora.state_dict()
        for k in sorted(set(got) & set(want)):
            a = got[k].cpu().numpy()
            np.testing.assert_array_equal(a, want[k].numpy().astype(a.dtype),
                                          err_msg=f"{k} flush {flush}")
        np.testing.assert_array_equal(hip.observe().cpu().numpy().view(np.uint16),
                                      ora.observe().numpy().view(np.uint16))
        mm, bm = ora.legal_mask()
        hm, hb = hip.legal_mask()
        np.testing.assert_array_equal(hm.cpu().numpy(), mm.numpy())
        np.testing.assert_array_equal(hb.cpu().numpy(), bm.numpy())
        assert int(want["recycle"].sum()) > 0


def test_collect_flushes_like_the_reference_loop(dev):
    """collect(flush_every=4) equals a step loop that flushes after every
    4th step and once at the end, field by field."""
    from qqtsim import (HipActorCritic, HipBatchedSim, HipRolloutBuffer, MapSpec, Rollout,
                        corridor_training_config)
    from qqtsim.policy import default_init

    n, T, seed, every = 128, 14, 6, 4
    cfg = corridor_training_config(max_steps=60)
    spec = MapSpec(kind="pillars", brick_p=0.4, bombs_cap=(1, 4), blast_cap=(2, 5))

    def make():
        sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
        net = HipActorCritic(default_init(cfg.obs_shape), device=dev, seed=seed)
        return sim, Rollout(sim, net)

    sim_a, roll_a = make()
    sim_b, roll_b = make()
    for sim, roll in ((sim_a, roll_a), (sim_b, roll_b)):
        for _ in range(3):
            roll.step()
        snap = sim.state_dict()
        snap["pending_lost"] = torch.full((n, 2), 2, dtype=snap["pending_lost"].dtype)
        sim.load_state_dict(snap)          # pending growth for the flushes to place
    buf = HipRolloutBuffer(T, n, cfg.obs_shape, dev)
    roll_a.collect(buf, flush_every=every)
    obs, rew = [], []
    for k in range(T):
        obs.append(sim_b.observe().clone())
        roll_b.step()
        rew.append(roll_b.reward[:, 0].clone())
        if k % every == every - 1 and k + 1 < T:
            sim_b.flush_recycle()
    sim_b.flush_recycle()
    assert torch.equal(buf.obs.cpu(), torch.stack(obs).cpu())
    assert torch.equal(buf.rew.cpu(), torch.stack(rew).cpu())
    assert sim_a.flushes == sim_b.flushes == (T - 1) // every + 1
    for k, v in sim_a.state_dict().items():
        assert torch.equal(v.cpu(), sim_b.state_dict()[k].cpu()), k
    assert torch.equal(sim_a.observe().cpu(), sim_b.observe().cpu())
    assert int(sim_a.state_dict()["recycle"].sum()) > 0
