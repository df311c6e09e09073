"""Device rollout buffer and GAE (needs an MI355X): qqt_gae bit-exact against
the oracle's compute_gae restatement, and Rollout.collect filling the
buffer exactly as a step-by-step collect loop over the same kernels does
(RolloutBuffer.add semantics of train/ppo.py:213-276, dmg included)."""

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


@pytest.mark.parametrize("t,n,gamma,lam", [(128, 5632, 0.995, 0.95), (37, 1000, 0.9973, 0.8117),
                                           (1, 7, 0.99, 0.9)])
def test_gae_kernel_matches_oracle(dev, t, n, gamma, lam):
    from oracle.ppo import gae
    from qqtsim import HipRolloutBuffer, compute_gae

    g = torch.Generator().manual_seed(t * 1000 + n)
    buf = HipRolloutBuffer(t, n, (14, 13, 13), dev)
    buf._rew.copy_(torch.randn((t, n, 2), generator=g) * 0.5)
    buf._val.copy_(torch.randn((t, n, 2), generator=g))
    buf._done.copy_((torch.rand((t, n), generator=g) < 0.05).to(torch.uint8))
    last = torch.randn(n, generator=g)
    adv, ret = compute_gae(buf, last.to(dev), gamma, lam)
    wa, wr = gae(buf.rew.cpu().numpy(), buf.val.cpu().numpy(), buf.done.cpu().numpy(),
                 last.numpy(), gamma, lam)
    np.testing.assert_array_equal(adv.cpu().numpy(), wa)
    np.testing.assert_array_equal(ret.cpu().numpy(), wr)


def _make(dev, n, seed, bot, max_steps=1800):
    from qqtsim import HipActorCritic, HipAstarBot, HipBatchedSim, MapSpec, Rollout
    from qqtsim import corridor_training_config
    from qqtsim.policy import default_init

    cfg = corridor_training_config(max_steps=max_steps)
    spec = MapSpec(kind="pillars", brick_p=0.3, bombs_cap=(2, 4), blast_cap=(2, 4))
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipActorCritic(default_init(cfg.obs_shape), device=dev, seed=seed)
    opp = HipAstarBot(sim, pid=1) if bot else None
    return sim, net, Rollout(sim, net, opponent=opp)


@pytest.mark.parametrize("bot", [False, True])
def test_collect_fills_the_buffer_like_the_step_loop(dev, bot):
    from qqtsim import HipRolloutBuffer

    n, T, seed = 256, 48, 5
    # 45-tick episodes: bombs (30-tick fuse) go off and timeouts with
    # auto-resets land inside the buffer (3 + 48 ticks)
    sim_a, net_a, roll_a = _make(dev, n, seed, bot, max_steps=45)
    sim_b, net_b, roll_b = _make(dev, n, seed, bot, max_steps=45)
    for _ in range(3):          # leave the first-tick path behind on both
        roll_a.step()
        roll_b.step()
    buf = HipRolloutBuffer(T, n, sim_a.cfg.obs_shape, dev)
    roll_a.collect(buf, flush_every=0)     # the flush cadence is tested on its own
    assert buf.ptr == T

    want = {k: [] for k in ("obs", "mm", "bm", "act", "logp", "val", "rew", "done", "dmg")}
    for _ in range(T):
        want["obs"].append(sim_b.observe().clone())
        mm, bm = sim_b.legal_mask()
        want["mm"].append(mm[:, 0].clone())
        want["bm"].append(bm[:, 0].clone())
        hp0 = sim_b.state_dict()["hp"][:, 0].clone()
        roll_b.step()
        want["act"].append(roll_b.actions[:, 0].long().clone())
        want["logp"].append(roll_b.logp[:, 0].clone())
        want["val"].append(roll_b.value[:, 0].clone())
        want["rew"].append(roll_b.reward[:, 0].clone())
        want["done"].append(roll_b.done.float().clone())
        hp1 = sim_b.state_dict()["hp"][:, 0]
        want["dmg"].append((hp0.long() - hp1.long()).clamp(min=0) > 0)
    got = {"obs": buf.obs, "mm": buf.mmask, "bm": buf.bmask, "act": buf.act, "logp": buf.logp,
           "val": buf.val, "rew": buf.rew, "done": buf.done, "dmg": buf.dmg}
    for k, w in want.items():
        w = torch.stack(w).cpu()
        assert torch.equal(got[k].cpu(), w), k
    assert bool(buf.dmg.any()), "the rollout should contain damage"
    assert bool(buf.done.any()), "the rollout should contain finished episodes"
    # both sims end in the same state, and the rollout's outputs describe the last step
    for k, v in sim_a.state_dict().items():
        assert torch.equal(v.cpu(), sim_b.state_dict()[k].cpu()), k
    assert torch.equal(roll_a.actions.cpu(), roll_b.actions.cpu())
    assert torch.equal(sim_a.observe().cpu(), sim_b.observe().cpu())


def test_collect_then_gae_matches_oracle(dev):
    from oracle.ppo import gae
    from qqtsim import HipRolloutBuffer, compute_gae

    n, T = 512, 64
    sim, net, roll = _make(dev, n, 11, False)
    buf = HipRolloutBuffer(T, n, sim.cfg.obs_shape, dev)
    roll.collect(buf)
    last_val = net.forward(sim.observe(), 0)[2]
    adv, ret = compute_gae(buf, last_val, 0.995, 0.95)
    wa, wr = gae(buf.rew.cpu().numpy(), buf.val.cpu().numpy(), buf.done.cpu().numpy(),
                 last_val.cpu().numpy(), 0.995, 0.95)
    np.testing.assert_array_equal(adv.cpu().numpy(), wa)
    np.testing.assert_array_equal(ret.cpu().numpy(), wr)
