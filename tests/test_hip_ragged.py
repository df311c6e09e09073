"""Ragged batch sizes (needs an MI355X): env and row counts that leave the
last workgroup partly empty (the tick and bot kernels run two envs per
workgroup, the MLP 64-row blocks dealt over 8 XCDs, GAE 256 envs per
workgroup), against the oracle on the same inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 65, 131]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.mark.parametrize("n", SIZES)
def test_tick_ragged_envs_match_oracle(dev, n):
    """Random legal actions with auto-reset for 44 ticks (40-tick episodes):
    state, done and rewards as the oracle's, every tick."""
    from oracle import philox
    from oracle.policy import sample_masked
    from oracle.sim import OracleSim
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.sim import HipBatchedSim

    spec = MapSpec(kind="pillars", brick_p=0.4, bombs_cap=(1, 4), blast_cap=(2, 5))
    cfg = corridor_training_config(max_hp=2, invuln_ticks=3, max_steps=40)
    seed = 7
    hip = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    ora = OracleSim(cfg, n, spec, seed=seed)
    resets = 0
    for t in range(44):
        mm, bm = ora.legal_mask()
        hm, hb = hip.legal_mask()
        np.testing.assert_array_equal(hm.cpu().numpy(), mm.numpy(), err_msg=f"mm {t}")
        np.testing.assert_array_equal(hb.cpu().numpy(), bm.numpy(), err_msg=f"bm {t}")
        np.testing.assert_array_equal(hip.observe().cpu().numpy().view(np.uint16),
                                      ora.observe().numpy().view(np.uint16), err_msg=f"obs {t}")
        u = philox.uniforms(seed, np.arange(n), t, philox.STREAM_RANDOM_ACT, 4)
        a = np.zeros((n, 2, 2), dtype=np.int64)
        for i in range(2):
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
        got, want = hip.state_dict(), ora.state_dict()
        for k in sorted(set(got) & set(want)):
            g = got[k].cpu().numpy()
            np.testing.assert_array_equal(g, want[k].numpy().astype(g.dtype), err_msg=f"{k} {t}")
    assert resets > 0


@pytest.mark.parametrize("b", [1, 63, 65, 130, 515])
def test_mlp_ragged_rows_match_oracle(dev, b):
    """Forward of both players over b rows within the logit tolerance, and
    sampled actions equal to the host sampler's on the kernel's logits."""
    from oracle.policy import mlp_forward, sample_masked
    from qqtsim.policy import HipActorCritic, default_init

    params = default_init()
    net = HipActorCritic(params, device=dev)
    g = torch.Generator().manual_seed(b)
    obs = (torch.rand((b, 14, 13, 13), generator=g) < 0.3).half()
    mm = torch.rand((b, 2, 5), generator=g) < 0.7
    mm[:, :, 4] = True
    bm = torch.ones((b, 2, 2), dtype=torch.bool)
    bm[:, :, 1] = torch.rand((b, 2), generator=g) < 0.5
    u = torch.rand((b, 2, 2), generator=g)
    acts, logp, val, lg = net.act_pair(obs.to(dev), mm.to(dev), bm.to(dev),
                                       uniforms=u.to(dev), logits=True)
    lg = lg.cpu().numpy()
    for pid in range(2):
        ml, bl, v = mlp_forward(params, obs, pid)
        ref = np.concatenate([ml.numpy(), bl.numpy(), v.numpy()[:, None]], 1)
        assert float(np.abs(lg[:, pid] - ref).max()) <= 1e-3
        am = sample_masked(lg[:, pid, :5], mm[:, pid].numpy(), u[:, pid, 0].numpy())[0]
        ab = sample_masked(lg[:, pid, 5:7], bm[:, pid].numpy(), u[:, pid, 1].numpy())[0]
        np.testing.assert_array_equal(acts[:, pid, 0].cpu().numpy(), am)
        np.testing.assert_array_equal(acts[:, pid, 1].cpu().numpy(), ab)


@pytest.mark.parametrize("n", SIZES)
def test_bot_ragged_envs_match_oracle(dev, n):
    """The astar bot on n envs drawn (cyclically) from a reference astar
    fixture of 64 envs."""
    from golden_io import GOLDEN
    from oracle.bots import astar_act
    from qqtsim import HipAstarBot, HipBatchedSim, MapSpec, corridor_training_config

    z = np.load(f"{GOLDEN}/astar_p30.npz")
    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=0, map_spec=MapSpec(kind="open"))
    bot = HipAstarBot(sim, pid=1)
    idx = np.arange(n) % z["bot"].shape[1]
    for t in (3, 17):
        snap = {k: torch.from_numpy(np.ascontiguousarray(z[k][t][idx]))
                for k in ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")}
        sim.load_state_dict(snap)
        args = (torch.from_numpy(z["obs"][t][idx]), torch.from_numpy(z["mm1"][t][idx]),
                torch.from_numpy(z["bm1"][t][idx]))
        u = torch.from_numpy(z["u"][t][idx])
        got = bot.act(*args, 1, uniforms=u)
        want = astar_act(cfg, snap, *args, 1, u)          # reach = this batch's max cap
        np.testing.assert_array_equal(got.cpu().numpy(), want.numpy(), err_msg=f"tick {t}")


@pytest.mark.parametrize("b", [65536, 70001])
def test_large_forward_matches_oracle(dev, b):
    """Forward batches from 65536 rows take two 64-row blocks per workgroup;
    a ragged one (70001 rows) ends in a half-filled workgroup."""
    from oracle.policy import mlp_forward
    from qqtsim.policy import HipActorCritic, default_init

    params = default_init()
    net = HipActorCritic(params, device=dev)
    g = torch.Generator().manual_seed(b)
    obs = (torch.rand((b, 14, 13, 13), generator=g) < 0.3).half()
    sel = torch.cat([torch.arange(0, 300), torch.arange(b - 300, b)])
    for pid in range(2):
        ml, bl, v = net.forward(obs.to(dev), pid)
        got = torch.cat([ml, bl, v[:, None]], 1).cpu()[sel].numpy()
        rml, rbl, rv = mlp_forward(params, obs[sel], pid)
        ref = np.concatenate([rml.numpy(), rbl.numpy(), rv.numpy()[:, None]], 1)
        assert float(np.abs(got - ref).max()) <= 1e-3
