"""MLP actor/critic forward and masked factored sampling (restates
train/model.py:121-196 and :215-245).

The forward runs in float32 (or float64) torch ops on an `ActorCritic`
mlp state_dict (keys `shared.0.weight`, ..., `critic.2.bias`).  The sampler is
the build's injected-uniform rule, written in float32 numpy arithmetic that
the HIP kernel reproduces operation for operation:

    ml_k = mask_k ? logit_k : -FLT_MAX          (train/model.py:215-220)
    m = max_k ml_k,  e_k = exp(ml_k - m),  S = sum_k e_k (in k order)
    a = #{k : e_0 + ... + e_k <= u * S}, clamped to the last k with e_k > 0
    logp = (ml_a - m) - log(S)

`exp` and `log` are this module's own float32 routines (Cody-Waite range
reduction with a degree-6 Taylor polynomial; an atanh series for log), so
host and device agree bit for bit given identical logits and uniforms.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

F32 = np.float32
NEG_MAX = F32(-3.4028234663852886e38)           # torch.finfo(float32).min
LOG2E = F32(1.4426950408889634)
LN2_HI = F32(0.693145751953125)                 # 0x3f317200, exact in 16 bits
LN2_LO = F32(1.428606765330187e-06)             # ln2 - LN2_HI
LN2 = F32(0.6931471805599453)
EXP_CUTOFF = F32(-80.0)
_EXP_C = [F32(1.0 / 720.0), F32(1.0 / 120.0), F32(1.0 / 24.0), F32(1.0 / 6.0),
          F32(0.5), F32(1.0), F32(1.0)]
_LOG_C = [F32(1.0 / 9.0), F32(1.0 / 7.0), F32(1.0 / 5.0), F32(1.0 / 3.0), F32(1.0)]
SQRT_HALF = F32(0.70710678118654752)


def exp_f32(x) -> np.ndarray:
    """exp for x <= 0 in float32: x = n ln2 + r, |r| <= ln2/2; exp(r) by Horner
    on the Taylor coefficients; times 2^n; 0 below EXP_CUTOFF."""
    x = np.asarray(x, dtype=F32)
    xc = np.maximum(x, EXP_CUTOFF)
    n = np.rint(xc * LOG2E).astype(F32)
    r = (xc - n * LN2_HI) - n * LN2_LO
    p = _EXP_C[0]
    for c in _EXP_C[1:]:
        p = p * r + c
    scale = ((n.astype(np.int32) + 127) << 23).astype(np.uint32).view(F32)
    out = (p * scale).astype(F32)
    return np.where(x < EXP_CUTOFF, F32(0.0), out).astype(F32)


def log_f32(x) -> np.ndarray:
    """log for normal x > 0 in float32: x = 2^k m with m in [sqrt(1/2), sqrt(2));
    log m = 2 atanh(s), s = (m-1)/(m+1), odd series to s^9."""
    x = np.asarray(x, dtype=F32)
    bits = x.view(np.uint32).astype(np.int64)
    k = ((bits >> 23) & 0xFF) - 127
    m = ((bits & 0x7FFFFF) | (127 << 23)).astype(np.uint32).view(F32)
    big = m >= F32(1.4142135623730951)
    m = np.where(big, m * F32(0.5), m).astype(F32)
    k = np.where(big, k + 1, k)
    s = ((m - F32(1.0)) / (m + F32(1.0))).astype(F32)
    s2 = (s * s).astype(F32)
    q = _LOG_C[0]
    for c in _LOG_C[1:]:
        q = q * s2 + c
    lm = F32(2.0) * (s * q)
    return (k.astype(F32) * LN2 + lm).astype(F32)


def sample_masked(logits, mask, u):
    """(a int64 (B,), logp float32 (B,)) for (B, K) logits/mask and (B,) u."""
    logits = np.asarray(logits, dtype=F32)
    mask = np.asarray(mask, dtype=bool)
    u = np.asarray(u, dtype=F32)
    b, k = logits.shape
    ml = np.where(mask, logits, NEG_MAX).astype(F32)
    m = ml[:, 0].copy()
    for j in range(1, k):
        m = np.maximum(m, ml[:, j])
    e = np.stack([exp_f32(ml[:, j] - m) for j in range(k)], 1)
    s = e[:, 0].copy()
    for j in range(1, k):
        s = (s + e[:, j]).astype(F32)
    t = (u * s).astype(F32)
    run = F32(0.0) * s
    count = np.zeros(b, dtype=np.int64)
    last = np.zeros(b, dtype=np.int64)
    for j in range(k):
        run = (run + e[:, j]).astype(F32)
        count += (run <= t)
        last = np.where(e[:, j] > 0, j, last)
    a = np.where(count >= k, last, count)
    picked = ml[np.arange(b), a]
    logp = ((picked - m).astype(F32) - log_f32(s)).astype(F32)
    return a.astype(np.int64), logp


def view_perm(me: int, p: int, c: int) -> list[int]:
    opp = [i for i in range(p) if i != me]
    head = [me, p + me] + opp + [p + o for o in opp] + [2 * p, 2 * p + 1, 2 * p + 2]
    return head + list(range(2 * p + 3, c))


def column_permutation(pid: int, p: int, c: int, hw: int) -> torch.Tensor:
    """Column index map folding player `pid`'s view permutation into the
    first layer: block k of the permuted weight is block inv[k] of the
    original, inv = argsort(view_perm) (train/model.py:121-139)."""
    perm = torch.tensor(view_perm(pid, p, c))
    inv = torch.argsort(perm)
    cols = torch.empty(c * hw, dtype=torch.long)
    for k in range(c):
        cols[k * hw:(k + 1) * hw] = torch.arange(hw) + int(inv[k]) * hw
    return cols


def mlp_forward(params: dict, obs: torch.Tensor, pid: int, n_players: int = 2,
                dtype=torch.float32):
    """(move_logits, bomb_logits, value) of the mlp ActorCritic for player
    `pid` (train/model.py:192-196); `params` is its state_dict."""
    P = {k: v.to(dtype) for k, v in params.items()}
    b = obs.shape[0]
    c, h, w = obs.shape[1:]
    x = obs.to(dtype).reshape(b, -1)
    cols = column_permutation(pid, n_players, c, h * w)
    x = F.linear(x, P["shared.0.weight"][:, cols], P["shared.0.bias"])
    x = F.relu(F.layer_norm(x, (x.shape[-1],), P["shared.1.weight"], P["shared.1.bias"]))
    x = F.linear(x, P["shared.3.weight"], P["shared.3.bias"])
    x = F.relu(F.layer_norm(x, (x.shape[-1],), P["shared.4.weight"], P["shared.4.bias"]))

    def head(name):
        y = F.relu(F.linear(x, P[f"{name}.0.weight"], P[f"{name}.0.bias"]))
        return F.linear(y, P[f"{name}.2.weight"], P[f"{name}.2.bias"])

    return head("move_head"), head("bomb_head"), head("critic").squeeze(-1)


def cnn_forward(params: dict, obs: torch.Tensor, pid: int, n_players: int = 2,
                dtype=torch.float32):
    """(move_logits, bomb_logits, value) of the cnn ActorCritic for player
    `pid` (train/model.py:79-96, 186-190): conv0 reads the observation
    through the view permutation of its input channels, then 3x3 convs
    16 -> 32 -> 64 and a 1x1 conv to 8 channels, each followed by a
    per-sample LayerNorm over [C, H, W] and ReLU, then the shared MLP
    (1352 -> 128 -> 128) and the heads."""
    P = {k: v.to(dtype) for k, v in params.items()}
    c, h, w = obs.shape[1:]
    inv = torch.argsort(torch.tensor(view_perm(pid, n_players, c)))
    x = F.conv2d(obs.to(dtype), P["conv0.weight"][:, inv], P["conv0.bias"], padding=1)
    for ln, conv in (("conv.0", "conv.2"), ("conv.3", "conv.5"), ("conv.6", "conv.8"),
                     ("conv.9", None)):
        x = F.relu(F.layer_norm(x, tuple(x.shape[1:]), P[f"{ln}.weight"], P[f"{ln}.bias"]))
        if conv is not None:
            k = P[f"{conv}.weight"].shape[-1]
            x = F.conv2d(x, P[f"{conv}.weight"], P[f"{conv}.bias"], padding=k // 2)
    x = x.flatten(1)
    x = F.linear(x, P["shared.0.weight"], P["shared.0.bias"])
    x = F.relu(F.layer_norm(x, (x.shape[-1],), P["shared.1.weight"], P["shared.1.bias"]))
    x = F.linear(x, P["shared.3.weight"], P["shared.3.bias"])
    x = F.relu(F.layer_norm(x, (x.shape[-1],), P["shared.4.weight"], P["shared.4.bias"]))

    def head(name):
        y = F.relu(F.linear(x, P[f"{name}.0.weight"], P[f"{name}.0.bias"]))
        return F.linear(y, P[f"{name}.2.weight"], P[f"{name}.2.bias"])

    return head("move_head"), head("bomb_head"), head("critic").squeeze(-1)


LSTM_HIDDEN = 128


def lstm_cell(x, h, c, w_ih, w_hh, b_ih, b_hh):
    """One step of a single-layer LSTM (gate order input, forget, cell,
    output, as torch.nn.LSTM stores them): returns (h', c')."""
    g = F.linear(x, w_ih, b_ih) + F.linear(h, w_hh, b_hh)
    i, f, gg, o = g.chunk(4, dim=1)
    c2 = torch.sigmoid(f) * c + torch.sigmoid(i) * torch.tanh(gg)
    return torch.sigmoid(o) * torch.tanh(c2), c2


def lstm_fused(params: dict, local, rel, glob, dtype=torch.float32):
    """The lstm arch's per-frame features (train/model.py:198-214,
    extract_fused): conv 3x3 C->32, ReLU, conv 3x3 32->64, ReLU, 2x2 max
    pool (7 -> 3), Linear(576,128) ReLU; rel Linear(60,64) ReLU Linear(64,32)
    ReLU; glob Linear(5,16) ReLU Linear(16,8) ReLU; Linear(168,256) ReLU."""
    P = {k: v.to(dtype) for k, v in params.items()}
    b = local.shape[0]
    x = F.relu(F.conv2d(local.to(dtype), P["l_conv1.weight"], P["l_conv1.bias"], padding=1))
    x = F.max_pool2d(F.relu(F.conv2d(x, P["l_conv2.weight"], P["l_conv2.bias"], padding=1)), 2)
    x = F.relu(F.linear(x.reshape(b, -1), P["l_cnn_fc.weight"], P["l_cnn_fc.bias"]))
    r = F.relu(F.linear(rel.to(dtype).reshape(b, -1), P["l_rel_fc1.weight"], P["l_rel_fc1.bias"]))
    r = F.relu(F.linear(r, P["l_rel_fc2.weight"], P["l_rel_fc2.bias"]))
    g = F.relu(F.linear(glob.to(dtype), P["l_glob_fc1.weight"], P["l_glob_fc1.bias"]))
    g = F.relu(F.linear(g, P["l_glob_fc2.weight"], P["l_glob_fc2.bias"]))
    return F.relu(F.linear(torch.cat([x, r, g], 1), P["l_fusion.weight"], P["l_fusion.bias"]))


def lstm_forward(params: dict, local, rel, glob, hidden=None, dtype=torch.float32):
    """(move_logits, bomb_logits, value, (h', c')) of the lstm ActorCritic
    for one frame (train/model.py:176-185); hidden = (h, c), each (B, 128),
    or None for the zero state."""
    P = {k: v.to(dtype) for k, v in params.items()}
    x = lstm_fused(params, local, rel, glob, dtype)
    b = x.shape[0]
    if hidden is None:
        h = torch.zeros((b, LSTM_HIDDEN), dtype=dtype)
        c = torch.zeros_like(h)
    else:
        h, c = (t.to(dtype) for t in hidden)
    h, c = lstm_cell(x, h, c, P["lstm.weight_ih_l0"], P["lstm.weight_hh_l0"],
                     P["lstm.bias_ih_l0"], P["lstm.bias_hh_l0"])

    def head(name):
        y = F.relu(F.linear(h, P[f"{name}.0.weight"], P[f"{name}.0.bias"]))
        return F.linear(y, P[f"{name}.2.weight"], P[f"{name}.2.bias"])

    return head("move_head"), head("bomb_head"), head("critic").squeeze(-1), (h, c)
