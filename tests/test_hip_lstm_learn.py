"""The lstm arch's training path on the GPU: an LstmRollout collect into the
lstm rollout buffer, the truncated-BPTT PPO update (qqtsim.ppo_update with
an LstmLearner) and the weight sync back to the acting kernel.

The update is checked against a restatement of the reference's
_ppo_update_lstm (train/ppo.py:440-537) written here step by step: the
per-frame heads and torch.distributions.Categorical, the host-side
`if done.any()` reset, the oracle's GAE.  With plain SGD the weights after
a whole update (2 epochs x 3 minibatches, with a bptt window) must agree
within 2e-6 absolute; the statistics within 1e-5 relative.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _collect(dev, n, T, seed):
    from qqtsim import (HipAstarBot, HipBatchedSim, HipLstmActorCritic, HipRolloutBuffer,
                        LstmRollout, MapSpec, corridor_training_config)

    cfg = corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=9)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed,
                        map_spec=MapSpec(kind="pillars", brick_p=0.5, swap_spawns=True))
    net = HipLstmActorCritic(device=dev, seed=seed)
    roll = LstmRollout(sim, net, HipAstarBot(sim, pid=1))
    buf = HipRolloutBuffer(T, n, cfg.obs_shape, dev, arch="lstm")
    roll.collect(buf)
    return sim, net, roll, buf


def _reference_update(learner, opt, buf, last_val, cfg, entropy_coef):
    """train/ppo.py:440-537 restated for the check."""
    from oracle.ppo import gae

    T, N = buf.rew.shape
    dev = buf.rew.device
    a, r = gae(buf.rew.cpu(), buf.val.cpu(), buf.done.cpu(), last_val.cpu(), cfg.gamma,
               cfg.gae_lambda)
    adv, ret = torch.from_numpy(a).to(dev), torch.from_numpy(r).to(dev)
    adv = (adv - adv.mean()) / (adv.std() + 1e-8)
    old_logp, old_val = buf.logp, buf.val
    stats = {"pg": 0.0, "vf": 0.0, "ent": 0.0, "kl": 0.0, "clipfrac": 0.0}
    n_updates = 0
    mb_n = max(1, N // cfg.minibatches)
    for _ in range(cfg.epochs):
        env_perm = torch.randperm(N, device=dev)
        for start in range(0, N, mb_n):
            sel = env_perm[start:start + mb_n]
            ns = sel.numel()
            logp = torch.empty((T, ns), device=dev)
            ent = torch.empty((T, ns), device=dev)
            value = torch.empty((T, ns), device=dev)
            fused_all = learner.extract_fused(buf.local[:, sel].reshape(T * ns, -1, 7, 7),
                                              buf.rel[:, sel].reshape(T * ns, -1, 6),
                                              buf.glob[:, sel].reshape(T * ns, -1)).view(T, ns, -1)
            hidden = None
            for t in range(T):
                if cfg.bptt_window > 0 and t % cfg.bptt_window == 0 and hidden is not None:
                    hidden = (hidden[0].detach(), hidden[1].detach())
                lo, hidden = learner.lstm(fused_all[t].unsqueeze(1), hidden)
                lo = lo.squeeze(1)
                ml, bl = learner.move_head(lo), learner.bomb_head(lo)
                v = learner.critic(lo).squeeze(-1)
                neg = torch.finfo(ml.dtype).min
                dm = torch.distributions.Categorical(
                    logits=torch.where(buf.mmask[t][sel], ml, torch.full_like(ml, neg)))
                db = torch.distributions.Categorical(
                    logits=torch.where(buf.bmask[t][sel], bl, torch.full_like(bl, neg)))
                am, ab = buf.act[t][sel, 0], buf.act[t][sel, 1]
                logp[t] = dm.log_prob(am) + db.log_prob(ab)
                ent[t] = dm.entropy() + db.entropy()
                value[t] = v
                if bool(buf.done[t][sel].any()):
                    dk = buf.done[t][sel].to(hidden[0].dtype).view(1, -1, 1)
                    hidden = (hidden[0] * (1 - dk), hidden[1] * (1 - dk))
            ratio = (logp - old_logp[:, sel]).exp()
            pg = -torch.min(ratio * adv[:, sel],
                            ratio.clamp(1 - cfg.clip_eps, 1 + cfg.clip_eps) * adv[:, sel]).mean()
            v_clipped = old_val[:, sel] + (value - old_val[:, sel]).clamp(-cfg.clip_eps,
                                                                           cfg.clip_eps)
            vf = 0.5 * torch.max((value - ret[:, sel]) ** 2, (v_clipped - ret[:, sel]) ** 2).mean()
            loss = pg + cfg.value_coef * vf - entropy_coef * ent.mean()
            opt.zero_grad(set_to_none=True)
            loss.backward()
            torch.nn.utils.clip_grad_norm_(learner.parameters(), cfg.max_grad_norm)
            opt.step()
            with torch.no_grad():
                stats["pg"] += float(pg)
                stats["vf"] += float(vf)
                stats["ent"] += float(ent.mean())
                stats["kl"] += float((old_logp[:, sel] - logp).mean())
                stats["clipfrac"] += float(((ratio - 1).abs() > cfg.clip_eps).float().mean())
            n_updates += 1
    return {k: v / max(1, n_updates) for k, v in stats.items()}


def test_lstm_update_matches_the_reference_restatement(dev):
    from qqtsim import LstmLearner, PPOConfig, ppo_update

    n, T, seed = 48, 14, 6
    sim, net, roll, buf = _collect(dev, n, T, seed)
    assert float(buf.done.sum()) > 0
    last_val = roll.last_value()
    cfg = PPOConfig(epochs=2, minibatches=3, bptt_window=5)
    a = LstmLearner().to(dev)
    b = copy.deepcopy(a)
    oa = torch.optim.SGD(a.parameters(), lr=0.05)
    ob = torch.optim.SGD(b.parameters(), lr=0.05)
    torch.manual_seed(3)
    got = ppo_update(a, oa, buf, last_val, cfg, 0.05)
    torch.manual_seed(3)
    want = _reference_update(b, ob, buf, last_val, cfg, 0.05)
    print("stats", got, want)
    for k in want:
        assert np.isfinite(got[k])
        assert abs(got[k] - want[k]) <= 1e-5 * max(1.0, abs(want[k])), k
    worst = 0.0
    for (name, pa), (_, pb) in zip(a.named_parameters(), b.named_parameters()):
        worst = max(worst, float((pa - pb).detach().abs().max()))
    moved = max(float((pa - p0).detach().abs().max()) for pa, p0 in
                zip(a.parameters(), LstmLearner().to(dev).parameters()))
    print(f"weights: max |diff| {worst:.2e}, max move {moved:.2e}")
    assert moved > 1e-4 and worst <= 2e-6


def test_lstm_training_iterations_stay_finite_and_sync(dev):
    """Two collect + update iterations with Adam and the weight sync to the
    acting network; after the sync the acting kernel reproduces the
    learner's forward on the buffer's first frame."""
    from qqtsim import HipRolloutBuffer, LstmLearner, PPOConfig, ppo_update

    n, T, seed = 512, 32, 2
    sim, net, roll, buf = _collect(dev, n, T, seed)
    learner = LstmLearner().to(dev)
    opt = torch.optim.Adam(learner.parameters(), lr=3e-4)
    cfg = PPOConfig()
    for it in range(2):
        print(f"[lstm learn] iteration {it}", flush=True)
        if it:
            roll.collect(buf)
        stats = ppo_update(learner, opt, buf, roll.last_value(), cfg, 0.05)
        assert all(np.isfinite(v) for v in stats.values()), stats
        assert all(bool(torch.isfinite(p).all()) for p in learner.parameters())
        net.load_state_dict(learner.state_dict())
    f = (buf.local[0], buf.rel[0], buf.glob[0])
    with torch.no_grad():
        ml, bl, v, (h, c) = learner(f, 0, None)
    hml, hbl, hv, (hh, hc) = net.forward(f, 0, None)
    for x, y in ((ml, hml), (bl, hbl), (v, hv), (h, hh), (c, hc)):
        assert float((x - y).abs().max()) <= 1e-4
    assert isinstance(buf, HipRolloutBuffer)
