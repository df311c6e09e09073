"""The lstm arch's training path on the GPU: an LstmRollout collect into the
lstm rollout buffer, the truncated-BPTT PPO update (qqtsim.ppo_update with
an LstmLearner) and the weight sync back to the acting kernel.

The update is checked against the oracle's restatement of the reference's
_ppo_update_lstm (train/ppo.py:440-537, `oracle.ppo_lstm.lstm_update`): the
same randperm consumption, per-frame torch.distributions.Categorical, the
host-side `if done.any()` reset and the oracle's GAE.  With plain SGD the
weights after a whole update (2 epochs x 3 minibatches, with a bptt window)
must agree within 2e-6 absolute; the statistics within 1e-5 relative.
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


def test_lstm_update_matches_the_reference_restatement(dev):
    from oracle.ppo_lstm import lstm_update
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
    want = lstm_update(b, ob, buf, last_val, cfg, 0.05)
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
