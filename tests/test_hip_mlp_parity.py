"""MFMA actor/critic kernel vs the reference forward and the host sampler.

Bars: logits and value within 1e-3 absolute of the float32 forward (the
kernel computes in float16 MFMA with float32 accumulation, the layers after
the first as float16 hi/lo pairs); sampled actions
bit-exact against the host sampler given the kernel's own logits and the same
uniforms, with logp within 1e-6.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import GOLDEN, mlp_params, traj

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def test_forward_matches_reference_golden(dev):
    """Weights and outputs recorded from the reference's ActorCritic."""
    from qqtsim.policy import HipActorCritic

    z = np.load(GOLDEN + "/mlp.npz")
    net = HipActorCritic(mlp_params(z), device=dev)
    assert net.n_params() == 345288
    obs = torch.from_numpy(z["obs"]).to(dev)
    for pid in range(2):
        ml, bl, v = net.forward(obs, pid)
        for got, key in ((ml, "move_logits"), (bl, "bomb_logits"), (v, "value")):
            err = float(np.abs(got.cpu().numpy() - z[f"{key}_{pid}"]).max())
            print(f"pid {pid} {key}: max |err| {err:.2e}")
            assert err <= LOGIT_ATOL


@pytest.mark.parametrize("name", ["pillars70", "stress40"])
def test_forward_matches_oracle_default_init(dev, name):
    """PyTorch default init (the rollout workloads' weights) on observations
    from reference trajectories, both players from one pass."""
    from oracle.policy import mlp_forward
    from qqtsim.policy import HipActorCritic, default_init

    params = default_init()
    net = HipActorCritic(params, device=dev)
    z = traj(name)
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13)[:1000].copy())
    b = obs.shape[0]
    mm = torch.ones((b, 2, 5), dtype=torch.bool)
    bm = torch.ones((b, 2, 2), dtype=torch.bool)
    _, _, val, lg = net.act_pair(obs.to(dev), mm.to(dev), bm.to(dev), logits=True)
    lg = lg.cpu().numpy()
    worst = 0.0
    for pid in range(2):
        ml, bl, v = mlp_forward(params, obs, pid)
        ref = np.concatenate([ml.numpy(), bl.numpy(), v.numpy()[:, None]], 1)
        worst = max(worst, float(np.abs(lg[:, pid] - ref).max()))
        np.testing.assert_array_equal(val.cpu().numpy()[:, pid], lg[:, pid, 7])
    print(f"{name}: {b} rows x 2 players, max |logit err| {worst:.2e}")
    assert worst <= LOGIT_ATOL


def test_sampling_bit_exact_given_logits(dev):
    """Same logits, masks and uniforms -> same actions as the host sampler."""
    from oracle.policy import sample_masked
    from qqtsim.policy import HipActorCritic

    net = HipActorCritic(device=dev, seed=3)
    z = traj("deathmatch")
    obs = torch.from_numpy(z["obs"].reshape(-1, 14, 13, 13).copy())
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
        legal_m = mm[:, pid].numpy()[np.arange(b), acts[:, pid, 0]]
        legal_b = bm[:, pid].numpy()[np.arange(b), acts[:, pid, 1]]
        all_masked = ~mm[:, pid].numpy().any(1)
        assert np.all(legal_m | all_masked)
        assert np.all(legal_b | ~bm[:, pid].numpy().any(1))


def test_single_player_act_matches_pair(dev):
    """act(pid) on one player equals that player's slot of act_pair."""
    from qqtsim.policy import HipActorCritic

    net = HipActorCritic(device=dev, seed=5)
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


def test_sampling_frequencies_follow_softmax(dev):
    """Many draws of one state: frequencies match the masked softmax."""
    from qqtsim.policy import HipActorCritic

    net = HipActorCritic(device=dev, seed=7)
    z = traj("pillars70")
    one = torch.from_numpy(z["obs"][10, 0].copy())
    b = 40000
    obs = one.unsqueeze(0).expand(b, -1, -1, -1).contiguous().to(dev)
    mm = torch.tensor([True, False, True, True, True]).view(1, 1, 5).expand(b, 2, 5).contiguous().to(dev)
    bm = torch.ones((b, 2, 2), dtype=torch.bool, device=dev)
    acts, _, _, lg = net.act_pair(obs, mm, bm, logits=True)
    lm = lg[0, 0, :5].double().cpu()
    lm[1] = -float("inf")
    p = torch.softmax(lm, 0).numpy()
    cnt = np.bincount(acts[:, 0, 0].cpu().numpy(), minlength=5)
    assert cnt[1] == 0
    exp = p * b
    chi2 = float(((cnt - exp) ** 2 / np.maximum(exp, 1e-9))[[0, 2, 3, 4]].sum())
    assert chi2 < 25.0, (cnt, exp)


def test_rollout_into_buffer_and_batched_forward(dev):
    """Rollout.run_into writes the observation each step acted on into a
    (T, N, C, H, W) slab (identical to stepping and copying observe()), and
    the batched evaluation forward over all T*N rows matches the oracle
    forward on sampled rows."""
    from oracle.policy import mlp_forward
    from qqtsim import HipActorCritic, HipBatchedSim, MapSpec, Rollout, corridor_training_config
    from qqtsim.policy import default_init

    n, T, seed = 256, 12, 4
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    params = default_init(cfg.obs_shape)
    a_sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    a = Rollout(a_sim, HipActorCritic(params, device=dev, seed=seed))
    buf = torch.empty((T, n) + tuple(cfg.obs_shape), dtype=torch.float16, device=dev)
    a.run_into(buf)
    b_sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    b = Rollout(b_sim, HipActorCritic(params, device=dev, seed=seed))
    for t in range(T):
        assert torch.equal(b_sim.observe(), buf[t]), t
        b.step()
    assert torch.equal(a_sim.observe(), b_sim.observe())
    for k, v in a_sim.state_dict().items():
        assert torch.equal(v, b_sim.state_dict()[k]), k

    net = HipActorCritic(params, device=dev)
    flat = buf.view(T * n, *cfg.obs_shape)
    ml, bl, v = net.forward(flat, 0)
    idx = torch.randperm(T * n, generator=torch.Generator().manual_seed(0))[:512]
    rml, rbl, rv = mlp_forward(params, flat[idx.to(dev)].cpu(), 0)
    got = torch.cat([ml[idx.to(dev)], bl[idx.to(dev)], v[idx.to(dev)][:, None]], 1).cpu()
    ref = torch.cat([rml, rbl, rv[:, None]], 1)
    assert float((got - ref).abs().max()) <= LOGIT_ATOL
