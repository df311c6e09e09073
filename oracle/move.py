"""Continuous-coordinate AABB movement with slide-stop (restates sim/move.py).

All arithmetic is float32 in the reference's operation order, so the HIP
kernel can be compared bit for bit.
"""

from __future__ import annotations

import torch

EPS = 1e-4  # sim/move.py:33


def step_table(step: float, device, dtype=torch.float32) -> torch.Tensor:
    """(5, 2) table: move code -> (dy, dx); IDLE is (0, 0) (sim/move.py:39-48)."""
    rows = [[-step, 0.0], [step, 0.0], [0.0, -step], [0.0, step], [0.0, 0.0]]
    return torch.tensor(rows, dtype=dtype, device=device)


def _blocked_pair(r0, c0, r1, c1, yb, xb, blocked_flat, rad, h, w):
    """(N, K) bool: either cell (r0,c0) or (r1,c1) stops this box
    (sim/move.py:154-181).  Out of bounds stops; a blocked cell that the box
    currently overlaps does not (a bomb just placed under the player)."""
    n, k = r0.shape
    oob = ((r0 < 0) | (r0 >= h) | (c0 < 0) | (c0 >= w)
           | (r1 < 0) | (r1 >= h) | (c1 < 0) | (c1 >= w))
    i0 = r0.clamp(0, h - 1) * w + c0.clamp(0, w - 1)
    i1 = r1.clamp(0, h - 1) * w + c1.clamp(0, w - 1)
    s0 = blocked_flat.gather(1, i0.reshape(n, -1)).reshape(n, k)
    s1 = blocked_flat.gather(1, i1.reshape(n, -1)).reshape(n, k)
    top = (yb - rad).floor().long()
    bot = (yb + rad).floor().long()
    lef = (xb - rad).floor().long()
    rig = (xb + rad).floor().long()
    in0 = (r0 >= top) & (r0 <= bot) & (c0 >= lef) & (c0 <= rig)
    in1 = (r1 >= top) & (r1 <= bot) & (c1 >= lef) & (c1 <= rig)
    return oob | (s0 & ~in0) | (s1 & ~in1)


def resolve_axis(coord, delta, other, y, x, blocked_flat, rad, h, w, vertical):
    """Resolve one axis of a move (sim/move.py:184-231).

    The leading edge sweeps from its old cell to its new cell (at most two
    cells); the nearest stopping cell along the move wins: the new lead cell
    first, then the old one.  The box stops `EPS` short of that cell.
    """
    sgn = torch.sign(delta)
    old_lead = (coord - delta + sgn * rad).floor().long()
    new_lead = (coord + sgn * rad).floor().long()
    lo = torch.minimum(old_lead, new_lead)
    hi = torch.maximum(old_lead, new_lead)
    a0 = (other - rad).floor().long()
    a1 = (other + rad).floor().long()
    if vertical:
        hit_lo = _blocked_pair(lo, a0, lo, a1, y, x, blocked_flat, rad, h, w)
        hit_hi = _blocked_pair(hi, a0, hi, a1, y, x, blocked_flat, rad, h, w)
    else:
        hit_lo = _blocked_pair(a0, lo, a1, lo, y, x, blocked_flat, rad, h, w)
        hit_hi = _blocked_pair(a0, hi, a1, hi, y, x, blocked_flat, rad, h, w)
    fwd = sgn > 0
    first_lead = torch.where(fwd, hi, lo)
    second_lead = torch.where(fwd, lo, hi)
    first_hit = torch.where(fwd, hit_hi, hit_lo)
    second_hit = torch.where(fwd, hit_lo, hit_hi)
    stop_cell = torch.where(first_hit, first_lead,
                            torch.where(second_hit, second_lead,
                                        torch.zeros_like(lo)))
    sc = stop_cell.to(coord.dtype)
    stop = torch.where(fwd, sc - rad - EPS, sc + 1.0 + rad + EPS)
    return torch.where(first_hit | second_hit, stop, coord)


def move_players(cfg, pos, move, alive, blocked, speed_mult=None):
    """New (N, P, 2) positions; players pass through each other
    (sim/move.py:234-279).  Displacement = table[move] * speed multiplier,
    zero for IDLE or dead players; the result is clamped to [r, h - r]."""
    n, p, _ = pos.shape
    h, w, rad = cfg.height, cfg.width, cfg.radius
    if speed_mult is None:
        speed_mult = torch.ones((n, p), dtype=pos.dtype, device=pos.device)
    flat = blocked.reshape(n, -1)
    tbl = step_table(cfg.step_len, pos.device, pos.dtype)
    delta = tbl[move.clamp(0, 4)] * speed_mult.unsqueeze(-1)
    go = alive & (move != 4)
    delta = torch.where(go.unsqueeze(-1), delta, torch.zeros_like(delta))
    dy, dx = delta[..., 0], delta[..., 1]
    y, x = pos[..., 0], pos[..., 1]
    ny = resolve_axis(y + dy, dy, x, y, x, flat, rad, h, w, True)
    nx = resolve_axis(x + dx, dx, y, y, x, flat, rad, h, w, False)
    out = pos.clone()
    out[..., 0] = torch.where(dy != 0, ny, y).clamp(rad, h - rad)
    out[..., 1] = torch.where(dx != 0, nx, x).clamp(rad, w - rad)
    return out


def center_cell(pos: torch.Tensor) -> torch.Tensor:
    """Cell under the player's centre (sim/move.py:282-288)."""
    return pos.floor().long()
