"""Pins of the oracle beyond the reference's vectors, and planted mistakes.

* exp_f32 / log_f32 against float64 libm (error bounds), the masked sampler
  against a float64 brute-force inverse CDF, masked-softmax log-probabilities
  and its boundary rules (the reference samples with torch.multinomial, which
  takes no injected uniforms, so the rule itself is this build's and is pinned
  by these properties: never illegal, logp = log softmax, frequencies).
* Planted mistakes in the oracle (movement stop margin, bomb danger weight,
  view permutation, explosion tier hint) must make the reference's golden
  vectors fail - so those vectors really constrain the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.grid
import oracle.move
import oracle.policy
from golden_io import TRAJ_CFG, json_states, mlp_params, traj
from oracle.policy import exp_f32, log_f32, mlp_forward, sample_masked

F32 = np.float32


def test_exp_f32_error_bound():
    x = np.concatenate([np.linspace(-80.0, 0.0, 200001, dtype=F32),
                        F32([0.0, -1e-7, -0.34657359, -0.6931472, -79.99])])
    got = exp_f32(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    rel = np.abs(got - want) / want
    assert rel.max() < 4 * 2.0 ** -23
    assert exp_f32(F32([-80.5, -1000.0, -3.4e38])).tolist() == [0.0, 0.0, 0.0]
    assert float(exp_f32(F32(0.0))) == 1.0


def test_log_f32_error_bound():
    x = np.concatenate([np.logspace(-30, 30, 200001).astype(F32),
                        F32([1.0, 2.0, 0.5, 1.4142135, 0.70710677, 1.0000001])])
    got = log_f32(x).astype(np.float64)
    want = np.log(x.astype(np.float64))
    err = np.abs(got - want)
    assert (err <= 4 * 2.0 ** -23 * np.maximum(np.abs(want), 1.0)).all()
    assert float(log_f32(F32(1.0))) == 0.0


def _brute_force(logits, mask, u):
    """float64 inverse CDF over the masked softmax: first k with cdf_k > u."""
    lg = np.where(mask, logits.astype(np.float64), -np.inf)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    cdf = np.cumsum(p)
    return int(np.searchsorted(cdf, u, side="right").clip(0, len(p) - 1)), cdf


def test_sampler_matches_float64_inverse_cdf_away_from_boundaries():
    rng = np.random.default_rng(0)
    n, k = 20000, 5
    logits = (rng.standard_normal((n, k)) * 3).astype(F32)
    mask = rng.random((n, k)) < 0.7
    mask[np.arange(n), rng.integers(0, k, n)] = True
    u = rng.random(n).astype(F32)
    a, logp = sample_masked(logits, mask, u)
    checked = 0
    for i in range(n):
        b, cdf = _brute_force(logits[i], mask[i], float(u[i]))
        if np.min(np.abs(cdf - float(u[i]))) > 1e-5:
            assert a[i] == b, i
            checked += 1
        assert mask[i, a[i]]
    assert checked > 0.99 * n
    lg = np.where(mask, logits.astype(np.float64), -np.inf)
    lsm = lg - lg.max(1, keepdims=True)
    lsm = lsm - np.log(np.exp(lsm).sum(1, keepdims=True))
    np.testing.assert_allclose(logp, lsm[np.arange(n), a], atol=2e-6, rtol=0)


def test_sampler_boundaries():
    logits = F32([[0.3, -1.0, 2.0, 0.0, 5.0]])
    mask = np.array([[False, True, True, False, False]])
    assert int(sample_masked(logits, mask, F32([0.0]))[0][0]) == 1
    assert int(sample_masked(logits, mask, F32([1.0 - 2.0 ** -24]))[0][0]) == 2
    # equal logits, u exactly at the CDF step: cdf_0 <= u counts (rule "<=")
    assert int(sample_masked(F32([[0.0, 0.0]]), np.ones((1, 2), bool), F32([0.5]))[0][0]) == 1
    # a single legal action is always taken, with logp 0
    a, lp = sample_masked(F32([[9.0, 1.0, 1.0]]), np.array([[False, True, False]]),
                          F32([0.999]))
    assert int(a[0]) == 1 and float(lp[0]) == 0.0


def test_sampler_frequencies_follow_softmax():
    rng = np.random.default_rng(1)
    logits = np.tile(F32([0.5, -1.0, 1.5, 0.0, 0.2]), (200000, 1))
    mask = np.tile(np.array([True, True, True, False, True]), (200000, 1))
    a, _ = sample_masked(logits, mask, rng.random(200000).astype(F32))
    cnt = np.bincount(a, minlength=5)
    p = np.exp(np.where(mask[0], logits[0], -np.inf))
    p /= p.sum()
    assert cnt[3] == 0
    exp = p * 200000
    keep = exp > 0
    assert float(((cnt[keep] - exp[keep]) ** 2 / exp[keep]).sum()) < 20.0


# ------------------------------------------------------------------ planted mistakes
def _replay_matches(name, ticks):
    from test_oracle_golden import oracle_for

    z = traj(name)
    s = oracle_for(z, name)
    for t in range(ticks):
        s.step(torch.from_numpy(z["actions"][t]), auto_reset=False,
               crate_u=torch.from_numpy(z["crate_u"][t]))
        for k in ("pos", "fuse", "brick", "hp", "alive"):
            if not np.array_equal(getattr(s, k).numpy(), z["state_" + k][t]):
                return False
        if not np.array_equal(s.danger().numpy(), z["danger"][t]):
            return False
    return True


def test_unplanted_short_replays_match():
    assert _replay_matches("pillars0", 40)
    assert _replay_matches("stress40", 40)


def test_planted_stop_margin_fails(monkeypatch):
    monkeypatch.setattr(oracle.move, "EPS", 0.0)
    assert not _replay_matches("pillars0", 40)


def test_planted_danger_weight_fails(monkeypatch):
    orig = oracle.grid.bomb_weight
    monkeypatch.setattr(oracle.grid, "bomb_weight", lambda f, m, exp=2.0: orig(f, m, 1.0))
    assert not _replay_matches("stress40", 40)


def test_planted_resolve_hint_fails():
    """Resolving every bomb with its own range (no frozen first-tick hint)
    diverges from the reference once crate growth lifts a blast range above
    the first tick's hint (pillars70)."""
    from test_oracle_golden import oracle_for

    z = traj("pillars70")
    s = oracle_for(z, "pillars70")
    s.resolve_tiers = 255
    diverged = False
    for t in range(z["actions"].shape[0]):
        _, _, info = s.step(torch.from_numpy(z["actions"][t]), auto_reset=False,
                            crate_u=torch.from_numpy(z["crate_u"][t]))
        if not np.array_equal(info["blast"].numpy(), z["covered"][t]):
            diverged = True
            break
    assert int(z["resolve_hint"]) < int(z["state_blast_cap"][-1].max()) and diverged


def test_planted_view_permutation_fails(monkeypatch):
    z = np.load(__import__("golden_io").GOLDEN + "/mlp.npz")
    params = mlp_params(z)
    obs = torch.from_numpy(z["obs"])
    monkeypatch.setattr(oracle.policy, "view_perm", lambda me, p, c: list(range(c)))
    ml, _, _ = mlp_forward(params, obs, 1)
    assert not np.array_equal(ml.numpy(), z["move_logits_1"])


def test_planted_fixture_danger_fails(monkeypatch):
    from test_oracle_golden import _fixture_outputs

    st = json_states("ref_state.json")[0]
    orig = oracle.grid.bomb_weight
    monkeypatch.setattr(oracle.grid, "bomb_weight", lambda f, m, exp=2.0: orig(f, m, 3.0))
    dng = _fixture_outputs(st)[0]
    assert not np.array_equal(dng.flatten().numpy(), np.float32(st["danger"]))


def test_trajectory_configs_cover_reference_rules():
    assert set(TRAJ_CFG) == {"pillars0", "pillars70", "stress40", "deathmatch"}
