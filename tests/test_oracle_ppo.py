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
