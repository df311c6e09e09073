"""Training iterations at the benchmark's shape (needs an MI355X): collect
5632 envs x 128 steps into the device rollout buffer, one PPO update
(train/ppo.py:364-437) with the fused loss + backward, and the copy of the
updated weights into the acting network, three times in a row.

Checks per iteration: the update's statistics and every learner weight are
finite, and the acting network's outputs after the weight copy equal the
learner's own forward on the same observation (a rollout whose argument
block still pointed at the weights it was built with would act with stale
or freed weights).  The log-probabilities and values the acting network recorded in
the buffer equal the learner's evaluation of the same actions before its
update (ratio 1).  Separately, one minibatch of
a collected buffer at its full size (180,224 rows) gets its gradients from
`ppo_grads` and from `loss.backward()` through `evaluate()` on the same
module, compared parameter by parameter."""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

N_ENVS, STEPS = 5632, 128


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _workload(dev, sd, seed):
    from qqtsim import CORRIDOR_70, HipActorCritic, HipBatchedSim, Rollout, corridor_training_config

    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, N_ENVS, device=dev, seed=seed, map_spec=CORRIDOR_70)
    actor = HipActorCritic(sd, device=dev, seed=seed)
    return cfg, Rollout(sim, actor)


def _finite_weights(module) -> bool:
    return all(bool(torch.isfinite(p).all()) for p in module.parameters())


@pytest.mark.parametrize("init", ["reference", "pytorch_default"])
def test_training_iterations_stay_finite_and_sync(dev, init):
    from qqtsim import HipMlpActorCritic, HipRolloutBuffer, PPOConfig, ppo_update
    from qqtsim.policy import default_init, reference_init

    sd = reference_init() if init == "reference" else default_init()
    cfg, roll = _workload(dev, sd, seed=11)
    learner = HipMlpActorCritic(device=dev, state_dict=sd)
    pcfg = PPOConfig()
    opt = torch.optim.Adam(learner.parameters(), lr=pcfg.lr)
    buf = HipRolloutBuffer(STEPS, N_ENVS, cfg.obs_shape, dev)
    actor = roll.policy
    torch.manual_seed(0)
    for it in range(3):
        print(f"[train] init={init} iteration {it}: collect", flush=True)
        roll.collect(buf)
        # the buffer was acted by the learner's current weights (the initial
        # ones, then the synced ones): its log-probabilities of the recorded
        # actions equal the recorded ones (both use the float16-rounded first
        # layer)
        rows = slice(0, 4096)
        for t in (0, STEPS - 1):
            with torch.no_grad():
                lp, _, val = learner.evaluate(buf.obs[t, rows], buf.mmask[t, rows],
                                              buf.bmask[t, rows], buf.act[t, rows])
            assert float((lp - buf.logp[t, rows]).abs().max()) <= 2e-3, (it, t)
            assert float((val - buf.val[t, rows]).abs().max()) <= 2e-3, (it, t)
        last_val = actor.forward(roll.sim.observe(), 0)[2]
        stats = ppo_update(learner, opt, buf, last_val, pcfg, pcfg.entropy_coef)
        print(f"[train] iteration {it}: {stats}", flush=True)
        assert all(math.isfinite(v) for v in stats.values()), (it, stats)
        assert abs(stats["kl"]) < 0.5 and stats["clipfrac"] < 0.9, (it, stats)
        assert _finite_weights(learner), it
        actor.load_state_dict(learner.state_dict())
        obs = roll.sim.observe()
        with torch.no_grad():
            for pid in range(2):
                want = learner(obs, pid)
                got = actor.forward(obs, pid)
                for w, g in zip(want, got):
                    assert float((w - g).abs().max()) <= 2e-3, (it, pid)


def test_full_minibatch_gradients_match_autograd(dev):
    """ppo_grads against loss.backward() through evaluate() on one real
    minibatch of a collected 5632 x 128 buffer (reference init)."""
    from qqtsim import HipMlpActorCritic, HipRolloutBuffer, PPOConfig, compute_gae
    from qqtsim.learn import _Transitions
    from qqtsim.policy import reference_init

    sd = reference_init(seed=5)
    cfg, roll = _workload(dev, sd, seed=12)
    buf = HipRolloutBuffer(STEPS, N_ENVS, cfg.obs_shape, dev)
    roll.collect(buf)
    pcfg = PPOConfig()
    last_val = roll.policy.forward(roll.sim.observe(), 0)[2]
    adv, ret = compute_gae(buf, last_val, pcfg.gamma, pcfg.gae_lambda)
    data = _Transitions(buf, adv, ret)
    g = torch.Generator(device=dev).manual_seed(3)
    idx = torch.randperm(data.count, device=dev, generator=g)[:data.count // pcfg.minibatches]
    mb = data.select(idx)
    net = HipMlpActorCritic(device=dev, state_dict=sd)

    logp, ent, value = net.evaluate(mb["obs"], mb["mmask"], mb["bmask"], mb["act"])
    ratio = torch.exp(logp - mb["old_logp"])
    adv_, ov, rt = mb["adv"], mb["old_val"], mb["ret"]
    pg = -torch.min(ratio * adv_, ratio.clamp(0.8, 1.2) * adv_).mean()
    vc = ov + (value - ov).clamp(-0.2, 0.2)
    vf = 0.5 * torch.max((value - rt) ** 2, (vc - rt) ** 2).mean()
    loss = pg + pcfg.value_coef * vf - pcfg.entropy_coef * ent.mean()
    loss.backward()
    want = {k: p.grad.detach().clone() for k, p in net.named_parameters()}
    want_st = torch.stack([pg, vf, ent.mean(), (mb["old_logp"] - logp).mean(),
                           ((ratio - 1).abs() > 0.2).float().mean()]).detach()
    net.zero_grad(set_to_none=True)
    st = net.ppo_grads(mb["obs"], mb["mmask"], mb["bmask"], mb["act"], mb["old_logp"],
                       mb["adv"], mb["ret"], mb["old_val"], pcfg, pcfg.entropy_coef)
    for k, p in net.named_parameters():
        assert torch.isfinite(p.grad).all(), k
        err = float((p.grad - want[k]).norm() / want[k].norm().clamp_min(1e-12))
        assert err <= 1e-3, (k, err)
    assert float((st - want_st).abs().max()) <= 1e-4 * max(1.0, float(want_st.abs().max()))
