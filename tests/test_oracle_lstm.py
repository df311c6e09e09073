"""The lstm arch's oracle (CPU only): local_view_features (oracle/obs.py)
and the lstm ActorCritic forward (oracle/policy.py) against vectors the
reference wrote (tests/golden/lstm.npz: sim/obs.py local_view_features on
bomb-rich states, train/model.py ActorCritic(arch="lstm") over those frames
as sequences with resets), plus the tie rule and planted mistakes."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from golden_io import check_features, lstm_params
from oracle.obs import local_view_features
from oracle.policy import lstm_cell, lstm_forward
from qqtsim.config import corridor_training_config

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def z():
    return np.load(os.path.join(HERE, "golden", "lstm.npz"))


def _inputs(z, i):
    return [torch.from_numpy(z[k][i]) for k in ("obs", "pos", "alive", "t", "fuse", "hp")]


def test_features_match_reference(z):
    cfg = corridor_training_config()
    frames = z["obs"].shape[0]
    for i in range(frames):
        args = _inputs(z, i)
        for only, sfx in ((False, ""), (True, "0")):
            got = [t.numpy() for t in local_view_features(cfg, *args, only_p0=only)]
            check_features([z[k + sfx][i] for k in ("local", "rel", "glob")], got)
    # the fixture exercises what it should: bombs, ties, empty slots, both players
    assert (z["fuse"] > 0).sum() > 100
    assert (z["rel"][..., 3] == 0).any() and (z["rel"][..., 3] == 1).any()


def test_tie_rule_ascending_cell_index():
    """Bombs at equal distance come in ascending cell index; empty slots
    take the lowest-index remaining cells."""
    cfg = corridor_training_config()
    n, h, w = 1, 13, 13
    fuse = torch.zeros((n, h, w), dtype=torch.int16)
    for y, x in ((5, 7), (7, 5), (6, 8), (4, 6)):      # all at L1 distance 2 from (6, 6)
        fuse[0, y, x] = 10
    fuse[0, 6, 7] = 3                                   # distance 1
    pos = torch.tensor([[[6.5, 6.5], [1.5, 1.5]]])
    obs = torch.zeros((n, 14, h, w), dtype=torch.float16)
    _, rel, _ = local_view_features(cfg, obs, pos, torch.ones((n, 2), dtype=torch.bool),
                                    torch.zeros(n, dtype=torch.long), fuse,
                                    torch.full((n, 2), 5, dtype=torch.uint8), only_p0=True)
    r = rel[0, 0].float().numpy()
    # (column offset, row offset) per slot
    want = [(1, 0), (0, -2), (1, -1), (2, 0), (-1, 1)]   # cells 85 | 58, 72, 86, 96
    assert [tuple(r[1 + j, :2]) for j in range(5)] == want
    assert list(r[1:6, 3]) == [1] * 5 and list(r[6:, 3]) == [0] * 4
    # empty slots: cells 0, 1, 2, 3 (row 0) relative to (6, 6)
    assert [tuple(r[6 + j, :2]) for j in range(4)] == [(-6 + j, -6) for j in range(4)]


def test_planted_feature_mistakes_fail(z):
    cfg = corridor_training_config()
    args = _inputs(z, z["obs"].shape[0] - 1)
    ref = [z[k][-1] for k in ("local", "rel", "glob")]
    l, r, g = (t.numpy().copy() for t in local_view_features(cfg, *args))
    swapped = r.copy()
    swapped[:, :, 0, [0, 1]] = r[:, :, 0, [1, 0]]      # opponent axes in the bomb order
    with pytest.raises(AssertionError):
        check_features(ref, (l, swapped, g))
    shifted = np.roll(l, 1, axis=-1)                     # window off by one column
    with pytest.raises(AssertionError):
        check_features(ref, (shifted, r, g))
    danger = g.copy()
    danger[..., 2] = 0                                   # danger read from the wrong place
    with pytest.raises(AssertionError):
        check_features(ref, (l, r, danger))


def _sequence(z, params, cell=lstm_cell, dtype=torch.float32):
    import oracle.policy as op

    saved = op.lstm_cell
    op.lstm_cell = cell
    try:
        hidden, worst = None, 0.0
        for i in range(z["local0"].shape[0]):
            f = [torch.from_numpy(z[k][i][:, 0]) for k in ("local0", "rel0", "glob0")]
            ml, bl, v, hidden = lstm_forward(params, *f, hidden, dtype=dtype)
            for a, k in ((ml, "move_logits"), (bl, "bomb_logits"), (v, "value"),
                         (hidden[0], "h"), (hidden[1], "c")):
                worst = max(worst, float((a.double() - torch.from_numpy(z[k][i]).double())
                                         .abs().max()))
            keep = (~torch.from_numpy(z["reset"][i])).to(dtype).view(-1, 1)
            hidden = (hidden[0] * keep, hidden[1] * keep)
        return worst
    finally:
        op.lstm_cell = saved


def test_lstm_forward_matches_reference(z):
    params = lstm_params(z)
    assert sum(v.numel() for v in params.values()) == int(z["param_count"]) == 368816
    assert _sequence(z, params) <= 1e-5
    assert _sequence(z, params, dtype=torch.float64) <= 1e-5
    assert z["reset"].any()


def test_planted_lstm_gate_order_fails(z):
    import torch.nn.functional as F

    def swapped(x, h, c, w_ih, w_hh, b_ih, b_hh):      # forget and input gates exchanged
        g = F.linear(x, w_ih, b_ih) + F.linear(h, w_hh, b_hh)
        f, i, gg, o = g.chunk(4, dim=1)
        c2 = torch.sigmoid(f) * c + torch.sigmoid(i) * torch.tanh(gg)
        return torch.sigmoid(o) * torch.tanh(c2), c2

    assert _sequence(z, lstm_params(z), cell=swapped) > 1e-3
