"""Flame rays, fixed-round chain explosion and the chain-corrected danger map.

Restates sim/blast.py.  Everything is a synchronous, fixed-round sweep over
(..., H, W) tensors: each round reads only the previous round's result.
"""

from __future__ import annotations

import torch

# Unit steps (drow, dcol): up, down, left, right (sim/blast.py:32).
_STEPS = ((-1, 0), (1, 0), (0, -1), (0, 1))


def shifted(x: torch.Tensor, drow: int, dcol: int, fill=0) -> torch.Tensor:
    """out[i, j] = x[i - drow, j - dcol]; cells shifted in from outside get
    `fill` (sim/blast.py:13-29)."""
    h, w = x.shape[-2], x.shape[-1]
    out = torch.full_like(x, fill)
    rs_dst = slice(max(drow, 0), h + min(drow, 0))
    cs_dst = slice(max(dcol, 0), w + min(dcol, 0))
    rs_src = slice(max(-drow, 0), h + min(-drow, 0))
    cs_src = slice(max(-dcol, 0), w + min(-dcol, 0))
    out[..., rs_dst, cs_dst] = x[..., rs_src, cs_src]
    return out


def rays(sources, wall, bombed, blast, brick=None, blast_max_hint=None):
    """Cross-shaped flame cover from `sources` (sim/blast.py:43-98).

    Walls stop flame and are never covered.  Bombs and bricks are covered but
    stop the flame.  Sources on a wall or a brick do not fire.  `blast` is an
    int or a per-cell int tensor (each bomb's own range).
    """
    if isinstance(blast, int):
        per_cell = torch.full(sources.shape, blast, dtype=torch.int32,
                              device=sources.device)
        b_top = blast
    else:
        per_cell = blast
        b_top = int(per_cell.max()) if per_cell.numel() else 0
        if blast_max_hint is not None:
            # tiers above the largest range present have no sources
            b_top = min(b_top, int(blast_max_hint))
    brk = brick if brick is not None else torch.zeros_like(sources)
    open_cell = ~wall
    passes = ~(bombed | brk)
    seed = sources & open_cell & ~brk
    cover = seed.clone()
    for b in range(1, b_top + 1):
        tier = seed & (per_cell == b)
        for dr, dc in _STEPS:
            front = tier
            for _ in range(b):
                front = shifted(front, dr, dc, False) & open_cell
                cover = cover | front
                front = front & passes
    return cover


def resolve_explosions(fuse, owner, wall, blast, max_chain, brick=None,
                       rounds=None, blast_max_hint=None):
    """(covered, triggered) of this tick's explosions (sim/blast.py:101-155).

    Sources are bombs whose fuse reached 0 (`fuse == 0 & owner >= 0`); live
    bombs (`fuse > 0`) absorb flame and are ignited by it.  The chain runs a
    fixed number of rounds: `min(max_chain - 1, rounds)` when `rounds` is
    given (the sync-free mode the tick uses, sim/torch_sim.py:809-833), else
    `max_chain - 1`.  Empty trailing rounds do not change the result.
    """
    trig = (fuse == 0) & (owner >= 0)
    live = fuse > 0
    cover = rays(trig, wall, live, blast, brick, blast_max_hint)
    n_rounds = max_chain - 1 if rounds is None else min(max_chain - 1, rounds)
    for _ in range(n_rounds):
        newly = live & cover & ~trig
        if not bool(newly.any()):
            break
        cover = cover | rays(newly, wall, live, blast, brick, blast_max_hint)
        trig = trig | newly
    return cover, trig


def bomb_weight(fuse: torch.Tensor, fuse_max: int, exp: float = 2.0) -> torch.Tensor:
    """(1 - (fuse-1)/FUSE)^2 clamped at 0 for live bombs, else 0
    (sim/blast.py:218-220)."""
    raw = 1.0 - (fuse.float() - 1.0) / float(fuse_max)
    if exp == 2.0:
        val = raw.clamp_min(0.0)
        val = val * val
    else:
        val = raw.clamp_min(0.0).pow(exp)
    return torch.where(fuse > 0, val, torch.zeros_like(raw))


def _sweep(front_w, front_d, passable, not_solid, steps, record):
    """Push (weight, remaining range) pairs `steps` cells along each of the
    four directions; each reached cell is recorded (max) before a bomb or a
    brick stops the wave (sim/blast.py:264-280, 305-316)."""
    one = torch.ones_like(passable)
    for dr, dc in _STEPS:
        fw, fd = front_w, front_d
        for _ in range(steps):
            nw = shifted(fw, dr, dc, 0.0) * passable
            nd = shifted(fd, dr, dc, 0.0) * passable
            nd = nd - one
            nw = nw * (nd >= 0)
            torch.maximum(record, nw, out=record)
            fw = nw * not_solid
            fd = nd * not_solid
    return record


def danger_map(fuse, wall, blast, fuse_max, brick=None, max_chain=1,
               rounds=None, blast_max_hint=None):
    """Chain-corrected danger in [0, 1] (sim/blast.py:158-317).

    Stage A relays bomb weights between bombs for `min(max_chain, rounds)`
    rounds (each round only the bombs whose weight rose send again), so a
    bomb that an earlier one will ignite inherits the earlier one's weight.
    Stage B spreads each bomb's corrected weight along its flame cross.
    Stage-A sources are not masked by `passable` at the origin; stage B's are.
    """
    bombed = fuse > 0
    weight = bomb_weight(fuse, fuse_max)
    brk = brick if brick is not None else torch.zeros_like(bombed)
    not_solid = (~(bombed | brk)).float()
    passable = (~wall).float()
    if isinstance(blast, int):
        blast_f = torch.full_like(weight, float(blast))
    else:
        blast_f = blast.float()
    if blast_max_hint is not None:
        steps = int(blast_max_hint)
    else:
        steps = int(blast_f.max()) if blast_f.numel() else 0
    zero = torch.zeros_like(weight)
    if max_chain > 1:
        n_rounds = max_chain if rounds is None else min(max_chain, rounds)
        w = weight.clone()
        front_w = torch.where(bombed, w, zero)
        front_d = torch.where(bombed, blast_f, zero)
        bombed_f = bombed.float()
        for _ in range(n_rounds):
            spread = _sweep(front_w, front_d, passable, not_solid, steps,
                            torch.zeros_like(weight))
            spread = spread * bombed_f
            newly = (spread > w) & bombed
            w = torch.maximum(w, spread)
            front_w = torch.where(newly, spread, zero)
            front_d = torch.where(newly, blast_f, zero)
            if not bool(newly.any()):
                break
        weight = w
    seed = weight * passable
    danger = seed.clone()
    front_d = torch.where(bombed, blast_f, zero)
    return _sweep(seed.clone(), front_d, passable, not_solid, steps, danger)
