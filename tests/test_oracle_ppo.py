"""The oracle's advantage estimation (compute_gae, train/ppo.py:101-110)
against closed forms, a float64 recurrence and torch's own evaluation of the
reference expression (the scalar handling is the part a restatement gets
wrong most easily)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ppo import gae

GAMMA, LAM = 0.995, 0.95     # PPOConfig defaults (train/ppo.py:42-43)


def _inputs(t=64, n=257, p_done=0.05, seed=0):
    rng = np.random.default_rng(seed)
    rew = (rng.standard_normal((t, n)) * 0.5).astype(np.float32)
    val = rng.standard_normal((t, n)).astype(np.float32)
    done = (rng.random((t, n)) < p_done).astype(np.float32)
    last = rng.standard_normal(n).astype(np.float32)
    return rew, val, done, last


def _torch_reference_expression(rew, val, done, last, gamma, lam):
    """The reference's loop as written, on float32 torch tensors (torch
    applies the Python-float scalars the reference multiplies by)."""
    rew, val, done, last = (torch.from_numpy(x) for x in (rew, val, done, last))
    adv = torch.zeros_like(rew)
    run = torch.zeros_like(last)
    steps = rew.shape[0]
    for t in reversed(range(steps)):
        nonterminal = 1.0 - done[t]
        next_val = last if t == steps - 1 else val[t + 1]
        delta = rew[t] + gamma * next_val * nonterminal - val[t]
        run = delta + gamma * lam * nonterminal * run
        adv[t] = run
    return adv.numpy(), (adv + val).numpy()


@pytest.mark.parametrize("gamma,lam", [(GAMMA, LAM), (0.99, 0.9), (0.9973, 0.8117)])
def test_gae_matches_torch_evaluation_bit_for_bit(gamma, lam):
    rew, val, done, last = _inputs()
    adv, ret = gae(rew, val, done, last, gamma, lam)
    ta, tr = _torch_reference_expression(rew, val, done, last, gamma, lam)
    np.testing.assert_array_equal(adv, ta)
    np.testing.assert_array_equal(ret, tr)


def test_all_terminal_is_reward_minus_value_exactly():
    rew, val, _, last = _inputs()
    adv, ret = gae(rew, val, np.ones_like(rew), last, GAMMA, LAM)
    np.testing.assert_array_equal(adv, rew - val)
    np.testing.assert_array_equal(ret, (rew - val) + val)


def test_lambda_zero_is_the_one_step_td_error():
    rew, val, done, last = _inputs(seed=1)
    adv, _ = gae(rew, val, done, last, GAMMA, 0.0)
    nxt = np.concatenate([val[1:], last[None]], 0).astype(np.float64)
    want = rew + GAMMA * nxt * (1.0 - done) - val
    np.testing.assert_allclose(adv, want, rtol=1e-6, atol=1e-6)


def test_undiscounted_without_terminals_telescopes():
    """gamma = lam = 1, no done: adv[t] = sum_{k>=t} rew[k] + last - val[t]."""
    rew, val, _, last = _inputs(t=40, seed=2)
    adv, _ = gae(rew, val, np.zeros_like(rew), last, 1.0, 1.0)
    want = np.cumsum(rew[::-1].astype(np.float64), 0)[::-1] + last - val
    np.testing.assert_allclose(adv, want, rtol=0, atol=2e-4)


def test_float64_recurrence():
    rew, val, done, last = _inputs(t=128, seed=3)
    adv, _ = gae(rew, val, done, last, GAMMA, LAM)
    r, v, d = (x.astype(np.float64) for x in (rew, val, done))
    run = np.zeros(rew.shape[1])
    want = np.zeros_like(r)
    for t in reversed(range(r.shape[0])):
        nv = last.astype(np.float64) if t == r.shape[0] - 1 else v[t + 1]
        run = r[t] + GAMMA * nv * (1 - d[t]) - v[t] + GAMMA * LAM * (1 - d[t]) * run
        want[t] = run
    np.testing.assert_allclose(adv, want, rtol=1e-4, atol=1e-4)


def test_planted_mistakes_fail():
    """Two plausible slips in a restatement: rounding gamma and lam to
    float32 separately, and dropping the terminal mask on the bootstrap."""
    rew, val, done, last = _inputs(seed=4)
    gamma, lam = 0.9973, 0.8117
    assert np.float32(gamma * lam) != np.float32(gamma) * np.float32(lam)
    ta, _ = _torch_reference_expression(rew, val, done, last, gamma, lam)
    # separately rounded gamma * lam
    adv = np.zeros_like(rew)
    run = np.zeros_like(last)
    gl = np.float32(gamma) * np.float32(lam)
    for t in reversed(range(rew.shape[0])):
        nt = np.float32(1.0) - done[t]
        nv = last if t == rew.shape[0] - 1 else val[t + 1]
        run = ((rew[t] + (np.float32(gamma) * nv) * nt) - val[t]) + (gl * nt) * run
        adv[t] = run
    assert not np.array_equal(adv, ta)
    # bootstrap without the terminal mask
    adv2 = np.zeros_like(rew)
    run = np.zeros_like(last)
    for t in reversed(range(rew.shape[0])):
        nt = np.float32(1.0) - done[t]
        nv = last if t == rew.shape[0] - 1 else val[t + 1]
        run = ((rew[t] + np.float32(gamma) * nv) - val[t]) + (np.float32(gamma * lam) * nt) * run
        adv2[t] = run
    assert not np.array_equal(adv2, ta)


def _lstm_buffer(steps=5, n=6, seed=0):
    """A synthetic lstm rollout buffer on the CPU with the reference
    RolloutBuffer's (T, N, ...) fields."""
    from types import SimpleNamespace

    g = torch.Generator().manual_seed(seed)
    done = torch.zeros((steps, n), dtype=torch.bool)
    done[2, 1] = done[3, 4] = True
    return SimpleNamespace(
        local=torch.rand((steps, n, 14, 7, 7), generator=g).half(),
        rel=torch.rand((steps, n, 10, 6), generator=g).half(),
        glob=torch.rand((steps, n, 5), generator=g).half(),
        act=torch.stack([torch.randint(0, 5, (steps, n), generator=g),
                         torch.randint(0, 2, (steps, n), generator=g)], -1),
        mmask=torch.ones((steps, n, 5), dtype=torch.bool),
        bmask=torch.ones((steps, n, 2), dtype=torch.bool),
        rew=torch.randn((steps, n), generator=g), val=torch.randn((steps, n), generator=g),
        logp=-torch.rand((steps, n), generator=g) * 2, done=done)


def test_lstm_update_minibatches_consume_the_random_stream_like_the_reference():
    """One randperm of the envs per epoch, cut into slices of N // minibatches
    (train/ppo.py:460-465): replaying the same seed by hand gives the same
    slices in the same order."""
    from oracle.ppo_lstm import env_minibatches
    from qqtsim.learn import PPOConfig

    cfg = PPOConfig(epochs=3, minibatches=4)
    torch.manual_seed(11)
    got = [s.tolist() for s in env_minibatches(10, cfg, torch.device("cpu"))]
    torch.manual_seed(11)
    want = []
    for _ in range(3):
        perm = torch.randperm(10).tolist()
        want += [perm[i:i + 2] for i in range(0, 10, 2)]
    assert got == want


def test_lstm_update_losses_reduce_to_closed_forms():
    """At ratio 1 (new log-probs equal the old) the clipped surrogate is
    -mean(adv) and the value loss is 0.5 mean((v - ret)^2) when v equals
    the old value (no clipping in play); the entropy bonus enters with its
    coefficient."""
    from oracle.ppo_lstm import clipped_losses
    from qqtsim.learn import PPOConfig

    cfg = PPOConfig()
    g = torch.Generator().manual_seed(2)
    logp = -torch.rand((4, 3), generator=g)
    ent = torch.rand((4, 3), generator=g)
    val = torch.randn((4, 3), generator=g)
    adv, ret = torch.randn((4, 3), generator=g), torch.randn((4, 3), generator=g)
    loss, st = clipped_losses(logp, ent, val, logp.clone(), val.clone(), adv, ret, cfg, 0.07)
    pg = -float(adv.mean())
    vf = 0.5 * float(((val - ret) ** 2).mean())
    assert abs(st["pg"] - pg) <= 1e-6 and abs(st["vf"] - vf) <= 1e-6
    assert st["kl"] == 0.0 and st["clipfrac"] == 0.0
    assert abs(float(loss) - (pg + cfg.value_coef * vf - 0.07 * float(ent.mean()))) <= 1e-6


def test_lstm_replay_resets_the_state_where_an_episode_ended():
    """The frame after a done frame starts from a zero LSTM state: replaying
    env 1 of the buffer from frame 3 alone (a fresh zero state) gives the same
    log-probs, entropies and values as frames 3.. of the full replay."""
    from oracle.ppo_lstm import replay_sequence
    from qqtsim.learn import LstmLearner

    torch.manual_seed(0)
    learner = LstmLearner()
    buf = _lstm_buffer()
    full = replay_sequence(learner, buf, torch.tensor([1]), window=0)
    tail = type(buf)(**{k: v[3:] for k, v in vars(buf).items()})
    part = replay_sequence(learner, tail, torch.tensor([1]), window=0)
    for a, b in zip(full, part):
        assert torch.allclose(a[3:], b, atol=1e-6), (a[3:], b)
    # without the reset (an env that never ended) the replays differ
    ref = replay_sequence(learner, buf, torch.tensor([0]), window=0)
    tail0 = replay_sequence(learner, tail, torch.tensor([0]), window=0)
    assert not torch.allclose(ref[2][3:], tail0[2], atol=1e-6)
