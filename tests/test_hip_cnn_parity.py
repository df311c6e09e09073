"""cnn actor/critic kernel (qqt_cnn_act) vs the reference forward and the host sampler.

Bars: logits and value within 1e-4 absolute of the float32 forward (the
kernel computes every layer in float32 on MFMA, in another summation order;
observed errors are below 2e-6); sampled actions bit-exact against the host
sampler given the kernel's own logits and the same uniforms, with logp within
1e-6; Philox-drawn actions bit-exact against the host sampler on the
oracle's Philox uniforms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import GOLDEN, cnn_params, traj

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 1e-4


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _logits(net, obs, pid):
    ml, bl, v = net.forward(obs, pid)
    return torch.cat([ml, bl, v[:, None]], 1).cpu()


def test_cnn_forward_matches_reference_golden(dev):
    """Weights and outputs recorded from the reference's ActorCritic(arch="cnn"),
    and evaluate()'s log-probabilities and entropies of the recorded actions."""
    from qqtsim.policy import HipCnnActorCritic

    z = np.load(GOLDEN + "/cnn.npz")
    net = HipCnnActorCritic(cnn_params(z), device=dev)
    assert net.n_params() == int(z["param_count"]) == 281744
    obs = torch.from_numpy(z["obs"]).to(dev)
    mm = torch.from_numpy(z["mm"]).to(dev)
    bm = torch.from_numpy(z["bm"]).to(dev)
    acts = torch.from_numpy(z["actions"]).to(dev)
    for pid in range(2):
        ml, bl, v = net.forward(obs, pid)
        for got, key in ((ml, "move_logits"), (bl, "bomb_logits"), (v, "value")):
            err = float(np.abs(got.cpu().numpy() - z[f"{key}_{pid}"]).max())
            print(f"pid {pid} {key}: max |err| {err:.2e}")
            assert err <= LOGIT_ATOL
        lp, ent, _ = net.evaluate(obs, mm[:, pid], bm[:, pid], acts[:, pid], pid)
        np.testing.assert_allclose(lp.cpu().numpy(), z[f"logp_{pid}"], atol=2e-4, rtol=0)
        np.testing.assert_allclose(ent.cpu().numpy(), z[f"entropy_{pid}"], atol=2e-4, rtol=0)


@pytest.mark.parametrize("name", ["pillars70", "stress40"])
def test_cnn_forward_matches_oracle_default_init(dev, name):
    """PyTorch default init on observations from reference trajectories, both
    players from one pass, against the oracle in float64."""
    from oracle.policy import cnn_forward
    from qqtsim.policy import HipCnnActorCritic, default_init_cnn

    params = default_init_cnn(seed=1)
    net = HipCnnActorCritic(params, device=dev)
    z = traj(name)
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13)[:600].copy())
    b = obs.shape[0]
    mm = torch.ones((b, 2, 5), dtype=torch.bool)
    bm = torch.ones((b, 2, 2), dtype=torch.bool)
    _, _, val, lg = net.act_pair(obs.to(dev), mm.to(dev), bm.to(dev), logits=True)
    lg = lg.cpu().numpy()
    worst = 0.0
    for pid in range(2):
        ml, bl, v = cnn_forward(params, obs, pid, dtype=torch.float64)
        ref = np.concatenate([ml.numpy(), bl.numpy(), v.numpy()[:, None]], 1)
        worst = max(worst, float(np.abs(lg[:, pid] - ref).max()))
        np.testing.assert_array_equal(val.cpu().numpy()[:, pid], lg[:, pid, 7])
        np.testing.assert_array_equal(lg[:, pid], _logits(net, obs.to(dev), pid).numpy())
    print(f"{name}: {b} rows x 2 players, max |logit err| {worst:.2e}")
    assert worst <= LOGIT_ATOL


def test_cnn_sampling_bit_exact_given_logits(dev):
    """Same logits, masks and uniforms -> same actions as the host sampler,
    including all-masked rows and the uniforms' end points."""
    from oracle.policy import sample_masked
    from qqtsim.policy import HipCnnActorCritic

    net = HipCnnActorCritic(device=dev, seed=3)
    z = traj("deathmatch")
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13)[:800].copy())
    b = obs.shape[0]
    g = torch.Generator().manual_seed(0)
    mm = torch.rand((b, 2, 5), generator=g) < 0.6
    bm = torch.rand((b, 2, 2), generator=g) < 0.6
    mm[..., 4] |= torch.rand((b, 2), generator=g) < 0.5
    u = torch.rand((b, 2, 2), generator=g)
    u[:7] = torch.tensor([0.0, 1.0 - 2 ** -24]).repeat(7, 2, 1)
    acts, logp, val, lg = net.act_pair(obs.to(dev), mm.to(dev), bm.to(dev), uniforms=u.to(dev),
                                       logits=True)
    acts, logp, lg = acts.cpu().numpy(), logp.cpu().numpy(), lg.cpu().numpy()
    for pid in range(2):
        am, lpm = sample_masked(lg[:, pid, :5], mm[:, pid].numpy(), u[:, pid, 0].numpy())
        ab, lpb = sample_masked(lg[:, pid, 5:7], bm[:, pid].numpy(), u[:, pid, 1].numpy())
        np.testing.assert_array_equal(acts[:, pid, 0], am)
        np.testing.assert_array_equal(acts[:, pid, 1], ab)
        np.testing.assert_allclose(logp[:, pid], lpm + lpb, atol=1e-6, rtol=0)


def test_cnn_philox_draws_match_oracle_uniforms(dev):
    """Without injected uniforms the kernel draws Philox(seed, row, tick,
    policy stream): the actions equal the host sampler's on the oracle's
    Philox uniforms, tick after tick."""
    from oracle import philox
    from oracle.policy import sample_masked
    from qqtsim.policy import HipCnnActorCritic

    seed = 11
    net = HipCnnActorCritic(device=dev, seed=seed)
    z = traj("pillars70")
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13)[:512].copy()).to(dev)
    b = obs.shape[0]
    g = torch.Generator().manual_seed(2)
    mm = (torch.rand((b, 2, 5), generator=g) < 0.7).to(dev)
    bm = (torch.rand((b, 2, 2), generator=g) < 0.7).to(dev)
    rows = np.arange(b)
    for _ in range(3):
        u = philox.uniforms(seed, rows, net.tick, philox.STREAM_POLICY, 4)
        acts, _, _, lg = net.act_pair(obs, mm, bm, logits=True)
        lg = lg.cpu().numpy()
        for pid in range(2):
            am, _ = sample_masked(lg[:, pid, :5], mm[:, pid].cpu().numpy(), u[:, 2 * pid])
            ab, _ = sample_masked(lg[:, pid, 5:7], bm[:, pid].cpu().numpy(), u[:, 2 * pid + 1])
            np.testing.assert_array_equal(acts[:, pid, 0].cpu().numpy(), am)
            np.testing.assert_array_equal(acts[:, pid, 1].cpu().numpy(), ab)


def test_cnn_single_player_act_matches_pair(dev):
    """act(pid) on one player equals that player's slot of act_pair."""
    from qqtsim.policy import HipCnnActorCritic

    net = HipCnnActorCritic(device=dev, seed=5)
    z = traj("pillars70")
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13)[:300].copy()).to(dev)
    b = obs.shape[0]
    mm = torch.from_numpy(np.ascontiguousarray(z["mm"][:75, :4].reshape(-1, 2, 5)[:b])).to(dev)
    bm = torch.from_numpy(np.ascontiguousarray(z["bm"][:75, :4].reshape(-1, 2, 2)[:b])).to(dev)
    u = torch.rand((b, 2, 2), generator=torch.Generator().manual_seed(1)).to(dev)
    pa, pl, pv = net.act_pair(obs, mm, bm, uniforms=u)
    for pid in range(2):
        a, lp, v = net.act(obs, mm[:, pid], bm[:, pid], pid, uniforms=u[:, pid])
        torch.testing.assert_close(a, pa[:, pid], rtol=0, atol=0)
        torch.testing.assert_close(lp, pl[:, pid], rtol=0, atol=0)
        torch.testing.assert_close(v, pv[:, pid], rtol=0, atol=0)


def test_cnn_rollout_self_play(dev):
    """The collect loop with the cnn policy: Rollout's per-tick actions equal
    act_pair on the same observation, masks and Philox tick, and the sim
    state equals a second sim stepped with those actions."""
    from qqtsim import HipBatchedSim, MapSpec, Rollout, corridor_training_config
    from qqtsim.policy import HipCnnActorCritic, default_init_cnn

    n, T, seed = 128, 6, 9
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    params = default_init_cnn(cfg.obs_shape, seed=2)
    a_sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    a = Rollout(a_sim, HipCnnActorCritic(params, device=dev, seed=seed))
    b_sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    b_net = HipCnnActorCritic(params, device=dev, seed=seed)
    for t in range(T):
        obs = b_sim.observe()
        mm, bm = b_sim.legal_mask()
        want, lp, v = b_net.act_pair(obs, mm, bm)
        a.step()
        assert torch.equal(a.actions.long(), want), t
        assert torch.equal(a.logp, lp) and torch.equal(a.value, v), t
        b_sim.step(want)
        assert torch.equal(a_sim.observe(), b_sim.observe()), t


def test_cnn_ragged_batches_are_row_independent(dev):
    """The persistent kernel splits items over workgroups and batches of 16 by
    the launch size; each item's outputs must not depend on that split.
    Forwards over ragged slices (1 to 4099 rows, both players and one) equal
    the same rows of one large launch bit for bit, and the small ones match
    the oracle."""
    from oracle.policy import cnn_forward
    from qqtsim.policy import HipCnnActorCritic, default_init_cnn

    params = default_init_cnn(seed=4)
    net = HipCnnActorCritic(params, device=dev)
    z = traj("pillars70")
    base = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13).copy())
    obs = base.repeat((5000 + base.shape[0] - 1) // base.shape[0], 1, 1, 1)[:5000].to(dev)
    b = obs.shape[0]
    ones_m = torch.ones((b, 2, 5), dtype=torch.bool, device=dev)
    ones_b = torch.ones((b, 2, 2), dtype=torch.bool, device=dev)
    _, _, _, full = net.act_pair(obs, ones_m, ones_b, logits=True)
    start = 0
    for n in (1, 5, 17, 33, 100, 255, 4099):
        sl = slice(start, start + n)
        _, _, _, lg = net.act_pair(obs[sl], ones_m[sl], ones_b[sl], logits=True)
        assert torch.equal(lg, full[sl]), n
        for pid in range(2):
            ml, bl, v = net.forward(obs[sl], pid)
            assert torch.equal(torch.cat([ml, bl, v[:, None]], 1), full[sl, pid]), (n, pid)
        if n <= 33:
            for pid in range(2):
                ml, bl, v = cnn_forward(params, obs[sl].cpu(), pid, dtype=torch.float64)
                ref = torch.cat([ml, bl, v[:, None]], 1)
                assert float((full[sl, pid].cpu().double() - ref).abs().max()) <= LOGIT_ATOL
        start = (start + n) % (b - 4100)


def test_cnn_learner_vs_astar_rollout(dev):
    """The cnn policy as the learner (player 0) against the astar bot: the
    rollout's player-0 actions equal act(pid=0) on the same observation,
    masks and Philox tick, and player 1's slot is the bot's."""
    from qqtsim import HipAstarBot, HipBatchedSim, MapSpec, Rollout, corridor_training_config
    from qqtsim.policy import HipCnnActorCritic, default_init_cnn

    n, T, seed = 96, 5, 13
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.5, swap_spawns=True)
    params = default_init_cnn(cfg.obs_shape, seed=5)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipCnnActorCritic(params, device=dev, seed=seed)
    bot = HipAstarBot(sim, pid=1)
    roll = Rollout(sim, net, opponent=bot)
    ref_net = HipCnnActorCritic(params, device=dev, seed=seed)
    for t in range(T):
        obs = sim.observe().clone()
        mm, bm = (m.clone() for m in sim.legal_mask())
        want, lp, v = ref_net.act(obs, mm[:, 0], bm[:, 0], 0)
        roll.launch_act()
        assert torch.equal(roll.actions[:, 0].long(), want), t
        assert torch.equal(roll.logp[:, 0], lp) and torch.equal(roll.value[:, 0], v), t
        roll.launch_tick()


def test_cnn_strided_observation_rows(dev):
    """Observation rows inside a wider buffer (obs_stride > 14 * 169, as a
    slab with padding would hand them over) give the same outputs as the
    contiguous rows, through the C ABI directly."""
    from qqtsim import _capi
    from qqtsim.policy import HipCnnActorCritic

    net = HipCnnActorCritic(device=dev, seed=2)
    z = traj("stress40")
    obs = torch.from_numpy(z["obs"].reshape(-1, 14 * 169)[:200].copy()).half().to(dev)
    b = obs.shape[0]
    wide = torch.zeros((b, 14 * 169 + 40), dtype=torch.float16, device=dev)
    wide[:, :14 * 169] = obs
    outs = []
    for src, stride in ((obs, 14 * 169), (wide, 14 * 169 + 40)):
        lg = torch.full((b, 2, 8), float("nan"), device=dev)
        a = net._args(b, 2, 0, 0, src.data_ptr(), stride)
        a.logits_out = lg.data_ptr()
        net._launch(a, _capi.stream_handle(dev))
        outs.append(lg)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])


def _torch_cnn_learner(sd, dev):
    """The reference's cnn ActorCritic as float32 torch modules with its
    evaluate() for player 0 (train/model.py:79-96, 186-196, 215-256): the
    autograd learner of a cnn training iteration."""
    import torch.nn as nn
    import torch.nn.functional as F

    from qqtsim.config import view_perm

    class Cnn(nn.Module):
        def __init__(self):
            super().__init__()
            self.conv0 = nn.Conv2d(14, 16, 3, padding=1)
            self.conv = nn.Sequential(
                nn.LayerNorm([16, 13, 13]), nn.ReLU(), nn.Conv2d(16, 32, 3, padding=1),
                nn.LayerNorm([32, 13, 13]), nn.ReLU(), nn.Conv2d(32, 64, 3, padding=1),
                nn.LayerNorm([64, 13, 13]), nn.ReLU(), nn.Conv2d(64, 8, 1),
                nn.LayerNorm([8, 13, 13]), nn.ReLU())
            self.shared = nn.Sequential(nn.Linear(1352, 128), nn.LayerNorm(128), nn.ReLU(),
                                        nn.Linear(128, 128), nn.LayerNorm(128), nn.ReLU())
            self.move_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 5))
            self.bomb_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 2))
            self.critic = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 1))
            self.inv = torch.argsort(torch.tensor(view_perm(0, 2, 14))).to(dev)

        def forward(self, obs):
            x = F.conv2d(obs.float(), self.conv0.weight[:, self.inv], self.conv0.bias, padding=1)
            x = self.shared(self.conv(x).flatten(1))
            return self.move_head(x), self.bomb_head(x), self.critic(x).squeeze(-1)

        def evaluate(self, obs, mm, bm, act):
            ml, bl, v = self(obs)
            neg = torch.finfo(ml.dtype).min
            dm = torch.distributions.Categorical(logits=torch.where(mm.bool(), ml, torch.full_like(ml, neg)))
            db = torch.distributions.Categorical(logits=torch.where(bm.bool(), bl, torch.full_like(bl, neg)))
            return (dm.log_prob(act[..., 0]) + db.log_prob(act[..., 1]),
                    dm.entropy() + db.entropy(), v)

    m = Cnn()
    m.load_state_dict(sd)
    return m.to(dev)


def test_cnn_training_iteration(dev):
    """A cnn training iteration of the reference's loop: collect 32 steps of
    64 envs with HipCnnActorCritic into the device buffer (arch "cnn"),
    ppo_update on the reference network as an autograd learner, and the
    updated weights loaded back into the acting network, whose forward then
    matches the learner's (1e-4)."""
    from qqtsim import (HipBatchedSim, HipCnnActorCritic, HipRolloutBuffer, MapSpec, PPOConfig,
                        Rollout, corridor_training_config, ppo_update)
    from qqtsim.policy import default_init_cnn

    cfg = corridor_training_config(max_steps=40)
    n, t = 64, 32
    sd = default_init_cnn(cfg.obs_shape, seed=6)
    sim = HipBatchedSim(cfg, n, device=dev, seed=3,
                        map_spec=MapSpec(kind="pillars", brick_p=0.5, bombs_cap=(2, 3)))
    actor = HipCnnActorCritic(sd, device=dev, seed=3)
    roll = Rollout(sim, actor)
    buf = HipRolloutBuffer(t, n, cfg.obs_shape, dev, arch="cnn")
    roll.collect(buf)
    learner = _torch_cnn_learner(sd, dev)
    with torch.no_grad():                      # the buffer's log-probs are the acting network's
        lp, _, v = learner.evaluate(buf.obs[:4].reshape(-1, 14, 13, 13), buf.mmask[:4].reshape(-1, 5),
                                    buf.bmask[:4].reshape(-1, 2), buf.act[:4].reshape(-1, 2))
    assert float((lp - buf.logp[:4].reshape(-1)).abs().max()) <= 2e-4
    assert float((v - buf.val[:4].reshape(-1)).abs().max()) <= 1e-4
    before = {k: v.detach().clone() for k, v in learner.state_dict().items()}
    opt = torch.optim.Adam(learner.parameters(), lr=3e-4)
    last_val = actor.forward(sim.observe(), 0)[2]
    torch.manual_seed(0)
    stats = ppo_update(learner, opt, buf, last_val, PPOConfig(minibatches=2, epochs=2), 0.05)
    assert all(np.isfinite(x) for x in stats.values()), stats
    after = {k: v.detach().cpu() for k, v in learner.state_dict().items()}
    assert any(not torch.equal(before[k].cpu(), after[k]) for k in after)
    actor.load_state_dict(after)
    obs = sim.observe()
    ml, bl, v = actor.forward(obs, 0)
    with torch.no_grad():
        rml, rbl, rv = learner(obs)
    got = torch.cat([ml, bl, v[:, None]], 1)
    ref = torch.cat([rml, rbl, rv[:, None]], 1)
    assert float((got - ref).abs().max()) <= 1e-4
