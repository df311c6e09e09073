"""The packed parameter block of the lstm kernel (qqtsim.policy.pack_lstm),
read the way qqt-gpu-sim_amd/csrc/lstm.hip reads it, on the CPU.

`_emulate` restates the kernel's indexing in float64 numpy: the 7x7 windows
in zero-bordered 9x9 grids with 16 channel slots, tap-major K for both
convolutions (k = tap * slots + channel, tap offset (tap / 3) * 9 + tap % 3),
conv1's output written back into a bordered grid, conv2 evaluated only at
the 36 positions the 2x2 pool reads, ordered by pooling window, and pooled
as relu(max + bias), the k-major blocks and the float16 hi / lo MFMA
fragments (read back as hi + lo) with their padding, the stacked LSTM
block and the block-diagonal output layer.  Run over the reference's frames
(tests/golden/lstm.npz, train/model.py:176-185 with the hidden state carried
and reset) it must reproduce the reference's logits, values and (h, c);
packings with a planted mistake (a transposed 3x3 kernel, the gates of W_hh
in another order, the move and bomb output columns swapped) must not.  The
trainable `LstmLearner` (the lstm PPO update's module) is pinned to the same
frames.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from golden_io import lstm_params
from qqtsim.policy import _LSTM_BLOCKS, LSTM_PARAMS, lstm_block_offsets, pack_lstm

HERE = os.path.dirname(os.path.abspath(__file__))
_LOGICAL_ROWS = {"g1w": 8, "g2w": 16, "fuw": 168}      # rows past these are K padding


@pytest.fixture(scope="module")
def z():
    return np.load(os.path.join(HERE, "golden", "lstm.npz"))


def _tapoff(t):
    return (t // 3) * 9 + t % 3


def _poff(p):
    return (p // 7) * 9 + p % 7


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _emulate(block, local, rel, glob, h, c):
    P = block.double().numpy()
    off = lstm_block_offsets()
    shapes = {k: (r, c, lay) for k, r, c, lay in _LSTM_BLOCKS}

    def W(k):
        r, cc, lay = shapes[k]
        flat = P[off[k]:off[k] + r * cc]
        if lay == "v":
            return flat
        if lay == "k":
            return flat.reshape(r, cc)
        # float16 hi / lo planes of MFMA fragments [t][s][q][r][i] ->
        # W[32 s + 8 q + i][16 t + r] = hi + lo
        halves = block[off[k]:off[k] + r * cc].contiguous().view(torch.float16).double().numpy()
        planes = halves.reshape(2, cc // 16, r // 32, 4, 16, 8).transpose(0, 2, 3, 5, 1, 4)
        m = planes.reshape(2, r, cc).sum(axis=0)
        return m[:_LOGICAL_ROWS.get(k, r)]

    relu = lambda x: np.maximum(x, 0.0)  # noqa: E731
    b, ch = local.shape[0], local.shape[1]
    pos = np.arange(49)
    grid = np.zeros((b, 16 * 81))
    for ci in range(ch):
        for p in pos:
            grid[:, ci * 81 + (p // 7 + 1) * 9 + p % 7 + 1] = local[:, ci, p // 7, p % 7]
    k1 = np.arange(144)
    idx1 = (k1 % 16)[None, :] * 81 + _poff(pos)[:, None] + _tapoff(k1 // 16)[None, :]
    a1 = relu(grid[:, idx1] @ W("c1w") + W("c1b")[:32])            # (B, 49, 32)
    grid2 = np.zeros((b, 32 * 81))
    for co in range(32):
        grid2[:, co * 81 + (pos // 7 + 1) * 9 + pos % 7 + 1] = a1[:, :, co]
    m = np.arange(36)
    wi, s4 = m // 4, m % 4
    top = (2 * (wi // 3) + s4 // 2) * 9 + 2 * (wi % 3) + s4 % 2     # window position (y, x)
    k2 = np.arange(288)
    idx2 = (k2 % 32)[None, :] * 81 + top[:, None] + _tapoff(k2 // 32)[None, :]
    v = (grid2[:, idx2] @ W("c2w")).reshape(b, 9, 4, 64).max(axis=2)      # (B, 9, 64)
    pooled = relu(v + W("c2b")).transpose(0, 2, 1).reshape(b, 576)     # channel-major
    fc = relu(pooled @ W("fcw") + W("fcb"))
    rin = np.zeros((b, 64))
    rin[:, :60] = rel.reshape(b, 60)
    r2 = relu(relu(rin @ W("r1w") + W("r1b")) @ W("r2w") + W("r2b")[:32])
    gin = np.zeros((b, 8))
    gin[:, :5] = glob
    g2 = relu(relu(gin @ W("g1w") + W("g1b")[:16]) @ W("g2w") + W("g2b")[:16])[:, :8]
    fu = relu(np.concatenate([fc, r2, g2], 1) @ W("fuw") + W("fub"))
    g = np.concatenate([fu, h], 1) @ W("lw") + W("lb")
    gi, gf, gg, go = (g[:, 128 * j:128 * (j + 1)] for j in range(4))
    c2 = _sig(gf) * c + _sig(gi) * np.tanh(gg)
    h2 = _sig(go) * np.tanh(c2)
    lg = relu(h2 @ W("hw") + W("hb")) @ W("ow") + W("ob")[:16]
    return lg, h2, c2


def _worst(z, block):
    n = z["local0"].shape[1]
    h = np.zeros((n, 128))
    c = np.zeros((n, 128))
    worst = 0.0
    for i in range(z["local0"].shape[0]):
        f = [z[k][i][:, 0].astype(np.float64) for k in ("local0", "rel0", "glob0")]
        lg, h, c = _emulate(block, *f, h, c)
        assert np.all(lg[:, 8:] == 0.0)
        for got, key in ((lg[:, :5], "move_logits"), (lg[:, 5:7], "bomb_logits"),
                         (lg[:, 7], "value"), (h, "h"), (c, "c")):
            worst = max(worst, float(np.abs(got - z[key][i]).max()))
        keep = ~z["reset"][i]
        h, c = h * keep[:, None], c * keep[:, None]
    return worst


def test_packed_block_reproduces_the_reference_sequence(z):
    params = lstm_params(z)
    block = pack_lstm(params)
    assert block.shape == (LSTM_PARAMS,) and block.dtype == torch.float32
    assert _worst(z, block) <= 1e-5


@pytest.mark.parametrize("kind", ["conv_kernel_transposed", "hh_gates_rolled", "heads_swapped"])
def test_planted_packing_mistakes_fail(z, kind):
    params = {k: v.clone() for k, v in lstm_params(z).items()}
    if kind == "conv_kernel_transposed":
        params["l_conv2.weight"] = params["l_conv2.weight"].transpose(2, 3).contiguous()
    elif kind == "hh_gates_rolled":
        params["lstm.weight_hh_l0"] = params["lstm.weight_hh_l0"].roll(128, 0)
    else:
        m, bo = params["move_head.2.weight"], params["bomb_head.2.weight"]
        params["move_head.2.weight"] = torch.cat([bo, m[2:]])
        params["bomb_head.2.weight"] = m[:2].clone()
    assert _worst(z, pack_lstm(params)) > 1e-3


def test_pack_rejects_wrong_shapes(z):
    params = lstm_params(z)
    bad = dict(params)
    bad["l_rel_fc1.weight"] = torch.zeros(64, 54)
    with pytest.raises(ValueError, match="l_rel_fc1.weight"):
        pack_lstm(bad)
    with pytest.raises(ValueError, match="14"):
        pack_lstm(params, obs_channels=15)


def test_lstm_learner_matches_the_reference_sequence(z):
    """The trainable LstmLearner (torch ops, CPU here) over the reference's
    frames: logits, values and state, and evaluate()'s log-probabilities and
    entropies of the recorded actions (the masked-logit distribution)."""
    from qqtsim.learn import LstmLearner

    net = LstmLearner(state_dict=lstm_params(z))
    assert net.n_params() == int(z["param_count"])
    hidden, worst = None, 0.0
    with torch.no_grad():
        for i in range(z["local0"].shape[0]):
            f = tuple(torch.from_numpy(z[k][i][:, 0]) for k in ("local0", "rel0", "glob0"))
            mm = torch.from_numpy(z["mm"][i][:, 0])
            bm = torch.from_numpy(z["bm"][i][:, 0])
            lp, ent, _ = net.evaluate(f, mm, bm, torch.from_numpy(z["actions"][i]), 0, hidden)
            ml, bl, v, hidden = net(f, 0, hidden)
            for got, key in ((ml, "move_logits"), (bl, "bomb_logits"), (v, "value"),
                             (hidden[0][0], "h"), (hidden[1][0], "c"), (lp, "logp"),
                             (ent, "entropy")):
                worst = max(worst, float(np.abs(got.numpy() - z[key][i]).max()))
            keep = (~torch.from_numpy(z["reset"][i])).float().view(1, -1, 1)
            hidden = (hidden[0] * keep, hidden[1] * keep)
    assert worst <= 1e-5
