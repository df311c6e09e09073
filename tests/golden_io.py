"""Loaders for the committed golden fixtures (test helper, not a test module).

* ref_state.json / sweep_states.json: the reference's own single-state
  fixtures (deploy/parity_ref.py, deploy/parity_sweep.py) - danger map,
  14-channel fp32 observation, legality masks and explosion cover.
* traj_*.npz, deep_chain.npz, mlp.npz: vectors written by
  tests/golden/gen_reference_vectors.py from the reference implementation.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

STATE_KEYS = ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast",
              "pos", "alive", "hp", "since_bomb", "t", "bombs_cap", "blast_cap",
              "spd_g", "invuln", "combo", "last_hit", "pending_lost")

TRAJ_CFG = {
    "pillars0": {},
    "pillars70": {},
    "stress40": {},
    "deathmatch": dict(max_hp=2, invuln_ticks=4, max_steps=70),
}


def json_states(name):
    """List of fixture dicts (the 60 sweep states, or the single ref state)."""
    with open(os.path.join(GOLDEN, name)) as f:
        d = json.load(f)
    return d["states"] if "states" in d else [d]


def json_state_tensors(st, h=13, w=13):
    s = st["state"]
    grid = lambda k, dt: torch.tensor(s[k], dtype=dt).view(1, h, w)  # noqa: E731
    return dict(
        wall=grid("wall", torch.bool), brick=grid("brick", torch.bool),
        fuse=grid("fuse", torch.int16), owner=grid("owner", torch.int8),
        bomb_blast=grid("bomb_blast", torch.int16), crate=grid("crate", torch.bool),
        pos=torch.tensor(s["pos"], dtype=torch.float32).view(1, 2, 2),
        alive=torch.tensor([s["alive"]], dtype=torch.bool),
        t=torch.tensor([s["t"]], dtype=torch.long),
        invuln=torch.tensor([s["invuln"]], dtype=torch.long),
        bombs_cap=torch.tensor([s["bombs_cap"]], dtype=torch.long),
        blast_cap=torch.tensor([s["blast_cap"]], dtype=torch.long),
    )


def traj(name):
    return np.load(os.path.join(GOLDEN, f"traj_{name}.npz"))


def state_at(z, tick):
    """Full state after `tick` steps (tick 0 = the initial state)."""
    pre = "init_" if tick == 0 else "state_"
    out = {}
    for k in STATE_KEYS:
        v = z[pre + k] if tick == 0 else z[pre + k][tick - 1]
        out[k] = torch.from_numpy(np.ascontiguousarray(v))
    return out


def mlp_params(z):
    out = {}
    for k in z.files:
        if not k.startswith("w_"):
            continue
        name = k[2:]
        for pre in ("move_head", "bomb_head", "critic", "shared"):
            if name.startswith(pre):
                out[pre + "." + name[len(pre) + 1:].replace("_", ".")] = torch.from_numpy(z[k])
    return out


def cnn_params(z):
    """state_dict of the cnn ActorCritic from cnn.npz's w_* arrays."""
    out = mlp_params(z)
    for k in z.files:
        if k.startswith("w_conv0_"):
            out["conv0." + k[len("w_conv0_"):]] = torch.from_numpy(z[k])
        elif k.startswith("w_conv_"):
            out["conv." + k[len("w_conv_"):].replace("_", ".")] = torch.from_numpy(z[k])
    return out


LSTM_KEYS = ("l_conv1.weight", "l_conv1.bias", "l_conv2.weight", "l_conv2.bias",
             "l_cnn_fc.weight", "l_cnn_fc.bias", "l_rel_fc1.weight", "l_rel_fc1.bias",
             "l_rel_fc2.weight", "l_rel_fc2.bias", "l_glob_fc1.weight", "l_glob_fc1.bias",
             "l_glob_fc2.weight", "l_glob_fc2.bias", "l_fusion.weight", "l_fusion.bias",
             "lstm.weight_ih_l0", "lstm.weight_hh_l0", "lstm.bias_ih_l0", "lstm.bias_hh_l0")


def lstm_params(z):
    """state_dict of the lstm ActorCritic from lstm.npz's w_* arrays."""
    out = mlp_params(z)
    for k in LSTM_KEYS:
        out[k] = torch.from_numpy(z["w_" + k.replace(".", "_")])
    return out


def _bits(a):
    return np.asarray(a).view(np.uint16)


def check_features(ref, got):
    """local and glob bit for bit; rel: opponent slots bit for bit, bomb
    slots' flags and L1 distances exact and their offsets equal as a set
    within each distance (the reference's order among equal distances is
    torch.topk's), empty slots' type entries 0."""
    (L, R, G), (l, r, g) = ref, got
    assert np.array_equal(_bits(l), _bits(L)), "local window"
    assert np.array_equal(_bits(g), _bits(G)), "global scalars"
    n_opp = 1
    assert np.array_equal(_bits(r[:, :, :n_opp]), _bits(R[:, :, :n_opp])), "opponent slots"
    assert np.array_equal(r[..., 3], R[..., 3]), "bomb flags"
    assert not np.any(r[..., n_opp:, 2]) and not np.any(r[..., n_opp:, 4:]), "bomb slot types"
    f32 = lambda x: np.asarray(x, dtype=np.float32)  # noqa: E731
    d_ref = np.abs(f32(R[..., 0])) + np.abs(f32(R[..., 1]))
    d_got = np.abs(f32(r[..., 0])) + np.abs(f32(r[..., 1]))
    ok = R[..., 3] > 0
    assert np.array_equal(d_ref[ok], d_got[ok]), "bomb distances"
    for e, me in zip(*np.nonzero(ok.any(-1))):
        m = ok[e, me]
        for d in np.unique(d_ref[e, me][m]):
            sel = m & (d_ref[e, me] == d)
            a = sorted(map(tuple, f32(R[e, me][sel][:, :2])))
            b = sorted(map(tuple, f32(r[e, me][sel][:, :2])))
            assert a == b, f"bomb offsets at distance {d}"
