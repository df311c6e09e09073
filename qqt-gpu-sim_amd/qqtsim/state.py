"""Conversion between the reference's (N,H,W)/(N,P) state tensors and the
packed device state of the HIP kernels (cell words, player records, env
records; layout in include/qqt_hip.h).  Torch ops on the state's device;
used by state_dict/load_state_dict and the attribute views, never per tick.
"""

from __future__ import annotations

import torch

P_Y, P_X, P_ALIVE, P_HP, P_SINCE, P_BOMBS, P_BLAST, P_SPD, P_INV, P_COMBO, P_LAST, \
    P_PEND, P_LOB, P_LOZ, P_LOS = range(15)
P_SLOTS = 16
E_T, E_CRATE_PROB, E_KIND = 0, 1, 2
E_SLOTS = 4

F_WALL, F_BRICK, F_CRATE, F_REC = 24, 25, 26, 27

GRID_KEYS = ("wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast")
PLAYER_INT = {"alive": (P_ALIVE, torch.bool), "hp": (P_HP, torch.uint8),
              "since_bomb": (P_SINCE, torch.int32), "bombs_cap": (P_BOMBS, torch.long),
              "blast_cap": (P_BLAST, torch.long), "invuln": (P_INV, torch.long),
              "combo": (P_COMBO, torch.long), "last_hit": (P_LAST, torch.long),
              "pending_lost": (P_PEND, torch.long), "lo_bombs": (P_LOB, torch.long),
              "lo_blast": (P_LOZ, torch.long)}
PLAYER_FLOAT = {"spd_g": P_SPD, "lo_spd": P_LOS}
ENV_KEYS = ("t", "crate_prob", "map_kind")
ALL_KEYS = GRID_KEYS + ("pos",) + tuple(PLAYER_INT) + tuple(PLAYER_FLOAT) + ENV_KEYS


def _bits(x, shift):
    return (x >> shift) & 1


def unpack_key(cells, players, envs, h, w, key):
    """One state tensor in the reference's layout and dtype."""
    n = cells.shape[0]
    if key in GRID_KEYS:
        cw = cells.view(n, h, w)
        if key == "fuse":
            return (cw & 0xFF).to(torch.int16)
        if key == "owner":
            return ((((cw >> 8) & 0xFF) ^ 0x80) - 0x80).to(torch.int8)
        if key == "bomb_blast":
            return ((cw >> 16) & 0xFF).to(torch.int16)
        shift = {"wall": F_WALL, "brick": F_BRICK, "crate": F_CRATE, "recycle": F_REC}[key]
        return _bits(cw, shift).bool()
    if key == "pos":
        return players[..., P_Y:P_X + 1].contiguous().view(torch.float32).clone()
    if key in PLAYER_INT:
        slot, dt = PLAYER_INT[key]
        return players[..., slot].to(dt)
    if key in PLAYER_FLOAT:
        return players[..., PLAYER_FLOAT[key]].contiguous().view(torch.float32).clone()
    if key == "t":
        return envs[:, E_T].long()
    if key == "crate_prob":
        return envs[:, E_CRATE_PROB].contiguous().view(torch.float32).clone()
    if key == "map_kind":
        return envs[:, E_KIND].long()
    raise KeyError(key)


def unpack(cells, players, envs, h, w):
    """Reference-layout dict of every state tensor."""
    return {k: unpack_key(cells, players, envs, h, w, k) for k in ALL_KEYS}


def _check_range(name, v, lo, hi):
    if v.numel() and (int(v.min()) < lo or int(v.max()) > hi):
        raise ValueError(f"{name} must lie in [{lo}, {hi}] for the packed device state")


def pack_into(cells, players, envs, snap, h, w):
    """Write the tensors of `snap` (any subset of ALL_KEYS, reference layout)
    into the packed state."""
    unknown = set(snap) - set(ALL_KEYS)
    if unknown:
        raise KeyError(f"unknown state keys {sorted(unknown)}")
    n = cells.shape[0]
    dev = cells.device
    if any(k in snap for k in GRID_KEYS):
        cur = unpack(cells, players, envs, h, w)
        g = {k: snap[k].to(dev) if k in snap else cur[k] for k in GRID_KEYS}
        _check_range("fuse", g["fuse"], 0, 255)
        _check_range("bomb_blast", g["bomb_blast"], 0, 255)
        _check_range("owner", g["owner"], -128, 127)
        cw = (g["fuse"].to(torch.int32) & 0xFF) \
            | ((g["owner"].to(torch.int32) & 0xFF) << 8) \
            | ((g["bomb_blast"].to(torch.int32) & 0xFF) << 16) \
            | (g["wall"].to(torch.int32) << F_WALL) | (g["brick"].to(torch.int32) << F_BRICK) \
            | (g["crate"].to(torch.int32) << F_CRATE) | (g["recycle"].to(torch.int32) << F_REC)
        cells.copy_(cw.view(n, h * w))
    if "pos" in snap:
        players[..., P_Y:P_X + 1] = snap["pos"].to(dev, torch.float32).contiguous().view(torch.int32)
    for k, (slot, _) in PLAYER_INT.items():
        if k in snap:
            v = snap[k].to(dev)
            if k in ("last_hit", "bombs_cap", "blast_cap", "invuln", "combo", "pending_lost",
                     "lo_bombs", "lo_blast"):
                _check_range(k, v.long(), -2 ** 31, 2 ** 31 - 1)
            players[..., slot] = v.to(torch.int32)
    for k, slot in PLAYER_FLOAT.items():
        if k in snap:
            players[..., slot] = snap[k].to(dev, torch.float32).contiguous().view(torch.int32)
    if "t" in snap:
        _check_range("t", snap["t"].long(), 0, 2 ** 31 - 1)
        envs[:, E_T] = snap["t"].to(dev).to(torch.int32)
    if "crate_prob" in snap:
        envs[:, E_CRATE_PROB] = snap["crate_prob"].to(dev, torch.float32).contiguous().view(torch.int32)
    if "map_kind" in snap:
        envs[:, E_KIND] = snap["map_kind"].to(dev).to(torch.int32)


def unpack_bits(words, h, w):
    """(N, 8) int32 bitsets -> (N, H, W) bool."""
    n = words.shape[0]
    c = h * w
    idx = torch.arange(c, device=words.device)
    wsel = words[:, idx // 32]
    return ((wsel >> (idx % 32)) & 1).bool().view(n, h, w)
