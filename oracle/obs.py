"""Shared observation encoding and legality masks (restates sim/obs.py)."""

from __future__ import annotations

import torch

from .grid import danger_map
from .move import EPS, center_cell, resolve_axis


def splat(pos_me, gate, h, w):
    """Bilinear splat of a continuous position, total mass 1 (0 when `gate` is
    False).  The four corner terms are accumulated in the fixed order
    (y0,x0), (y0,x1), (y1,x0), (y1,x1) (sim/obs.py:25-45)."""
    n = pos_me.shape[0]
    fy = (pos_me[:, 0] - 0.5).clamp(0.0, h - 1.0)
    fx = (pos_me[:, 1] - 0.5).clamp(0.0, w - 1.0)
    y0 = fy.floor().long().clamp(0, h - 1)
    x0 = fx.floor().long().clamp(0, w - 1)
    y1 = (y0 + 1).clamp(0, h - 1)
    x1 = (x0 + 1).clamp(0, w - 1)
    wy = (fy - y0.to(fy.dtype)).clamp(0.0, 1.0)
    wx = (fx - x0.to(fx.dtype)).clamp(0.0, 1.0)
    g = gate.to(fy.dtype)
    out = torch.zeros((n, h * w), dtype=fy.dtype, device=pos_me.device)
    for yy, ky in ((y0, 1.0 - wy), (y1, wy)):
        for xx, kx in ((x0, 1.0 - wx), (x1, wx)):
            out.scatter_add_(1, (yy * w + xx).unsqueeze(1), (ky * kx * g).unsqueeze(1))
    return out.view(n, h, w)


def live_counts(owner, fuse, p):
    """(N, P) live bombs per owner."""
    return torch.stack([((owner == i) & (fuse > 0)).flatten(1).sum(1)
                        for i in range(p)], dim=1)


def encode_obs(cfg, wall, fuse, owner, pos, alive, t, brick=None,
               bomb_blast=None, crate=None, invuln=None, bombs_p=None,
               danger=None, rounds=None):
    """(N, C, H, W) shared observation, computed in float32 and cast once
    (sim/obs.py:48-136)."""
    n, p = alive.shape
    h, w = cfg.height, cfg.width
    fnorm = fuse.float() / float(cfg.fuse)
    zero = torch.zeros_like(fnorm)
    obs = torch.zeros((n, cfg.n_channels, h, w), dtype=torch.float32,
                      device=wall.device)
    for i in range(p):
        obs[:, i] = splat(pos[:, i], alive[:, i], h, w)
        obs[:, p + i] = torch.where((owner == i) & (fuse > 0), fnorm, zero)
    brk = brick if brick is not None else torch.zeros_like(wall)
    obs[:, 2 * p] = (wall | brk).float()
    if danger is None:
        if bomb_blast is not None:
            bmap = torch.where(bomb_blast > 0, bomb_blast.long(),
                               torch.full_like(bomb_blast.long(), cfg.blast))
        else:
            bmap = cfg.blast
        danger = danger_map(fuse, wall, bmap, cfg.fuse, brick, cfg.max_chain,
                            rounds=rounds)
    obs[:, 2 * p + 1] = danger
    obs[:, 2 * p + 2] = (t.float() / float(cfg.max_steps)).view(n, 1, 1)
    if not cfg.obs_extra_enabled:
        return obs.half() if cfg.obs_fp16 else obs
    if crate is not None:
        obs[:, 2 * p + 3] = crate.float()
    cell = center_cell(pos)
    flat = cell[..., 0] * w + cell[..., 1]
    if invuln is not None:
        for i in range(p):
            on = ((invuln[:, i] > 0) & alive[:, i]).float()
            obs[:, 2 * p + 4 + i].view(n, -1).scatter_(1, flat[:, i:i + 1],
                                                       on.unsqueeze(1))
    if bombs_p is not None:
        cap = bombs_p.float().clamp(min=1)
        avail = (bombs_p - live_counts(owner, fuse, p)).float().clamp(min=0)
        base = 3 * p + 4
        for i in range(p):
            a = alive[:, i].float()
            obs[:, base + i].view(n, -1).scatter_(
                1, flat[:, i:i + 1], ((avail[:, i] / cap[:, i]) * a).unsqueeze(1))
            obs[:, base + p + i].view(n, -1).scatter_(
                1, flat[:, i:i + 1],
                ((cap[:, i] / cfg.growth_bombs_max) * a).unsqueeze(1))
    return obs.half() if cfg.obs_fp16 else obs


def can_place(cfg, fuse, owner, pos, brick=None, bombs_p=None):
    """(N, P): the centre cell holds no bomb and no brick and the player is
    under its live-bomb cap (sim/obs.py:139-167)."""
    n, p, _ = pos.shape
    w = cfg.width
    cell = center_cell(pos)
    flat = cell[..., 0] * w + cell[..., 1]
    ffl = fuse.reshape(n, -1)
    brk = brick if brick is not None else torch.zeros_like(fuse, dtype=torch.bool)
    occupied = ((fuse > 0) | brk).reshape(n, -1)
    live = live_counts(owner, fuse, p)
    ok = torch.zeros((n, p), dtype=torch.bool, device=pos.device)
    for me in range(p):
        idx = flat[:, me:me + 1]
        bomb_under = ffl.gather(1, idx).squeeze(1) > 0
        blocked_under = occupied.gather(1, idx).squeeze(1)
        cap = bombs_p[:, me] if bombs_p is not None else cfg.max_bombs
        ok[:, me] = ~bomb_under & ~blocked_under & (live[:, me] < cap)
    return ok


def legal_mask(cfg, wall, fuse, owner, pos, alive, brick=None, bombs_p=None):
    """(move_mask (N,P,5), bomb_mask (N,P,2)) (sim/obs.py:170-229).

    A direction is legal when a base-speed probe (`step_len`, not scaled by
    growth) moves the player by more than 2*EPS.  IDLE and "no bomb" are
    always legal; a dead player's rows are all True.
    """
    n, p, _ = pos.shape
    h, w, rad = cfg.height, cfg.width, cfg.radius
    brk = brick if brick is not None else torch.zeros_like(wall)
    flat = (wall | (fuse > 0) | brk).reshape(n, -1)
    step = cfg.step_len
    y, x = pos[..., 0], pos[..., 1]
    yk = y.unsqueeze(-1).expand(n, p, 2).reshape(n, -1)
    xk = x.unsqueeze(-1).expand(n, p, 2).reshape(n, -1)
    d = torch.full_like(yk, step)
    d[:, 0::2] = -step
    ny = resolve_axis(yk + d, d, xk, yk, xk, flat, rad, h, w, True)
    mv_v = (ny - yk).abs() > EPS * 2
    nx = resolve_axis(xk + d, d, yk, yk, xk, flat, rad, h, w, False)
    mv_h = (nx - xk).abs() > EPS * 2
    mm = torch.ones((n, p, 5), dtype=torch.bool, device=pos.device)
    mm[..., 0] = mv_v[:, 0::2]
    mm[..., 1] = mv_v[:, 1::2]
    mm[..., 2] = mv_h[:, 0::2]
    mm[..., 3] = mv_h[:, 1::2]
    mm = (mm & alive.unsqueeze(-1)) | (~alive).unsqueeze(-1)
    place = can_place(cfg, fuse, owner, pos, brick, bombs_p) & alive
    bm = torch.ones((n, p, 2), dtype=torch.bool, device=pos.device)
    bm[..., 1] = place | ~alive
    return mm, bm


# ---------------------------------------------------------------- lstm arch
MAX_T = 10          # target slots of the relative-coordinate block
GLOB_FEAT = 5       # global scalars
LOCAL_K = 7         # side of the local window


def local_view_features(cfg, obs, pos, alive, t, fuse, hp, only_p0: bool = False):
    """Per-player features of the lstm arch (sim/obs.py:243-340):
    local (N, P', C, 7, 7), rel (N, P', MAX_T, 6), glob (N, P', 5), in obs's
    dtype, P' = 1 when only_p0 else P.

    * local: the 7x7 window of every observation channel centred on the
      player's centre cell (zero outside the grid).
    * rel: slots 0..P-2 are the opponents (me + i + 1) % P: (pos diff axis 0,
      pos diff axis 1, alive); the rest are the bombs (fuse > 0) nearest to
      the centre cell in L1 distance: (column offset, row offset, 0, 1).
      Slots past the last bomb carry the offsets of the remaining cells with
      their third/fourth entries 0.  Bombs at equal distance, and the cells
      of empty slots, are taken in ascending cell index (the reference takes
      them in whatever order torch.topk returns among equal keys, which
      differs between its CPU and GPU implementations).
    * glob: t / max_steps, hp / max_hp, the danger channel at the centre
      cell, bombs on the map / max_bombs, fuse total / (max_bombs * fuse).
    """
    n, p_full, _ = pos.shape
    c, h, w = obs.shape[1], cfg.height, cfg.width
    dt = obs.dtype
    k, half = LOCAL_K, LOCAL_K // 2
    p_out = 1 if only_p0 else p_full
    cell = center_cell(pos)                                   # (N, P, 2)
    pad = torch.nn.functional.pad(obs, (half, half, half, half))
    local = torch.empty((n, p_out, c, k, k), dtype=dt)
    rows = torch.arange(n)
    for me in range(p_out):
        for dy in range(k):
            for dx in range(k):
                local[:, me, :, dy, dx] = pad[rows, :, cell[:, me, 0] + dy, cell[:, me, 1] + dx]
    rel = torch.zeros((n, p_out, MAX_T, 6), dtype=dt)
    n_opp = p_full - 1
    for me in range(p_out):
        for i in range(n_opp):
            opp = (me + i + 1) % p_full
            rel[:, me, i, 0] = (pos[:, opp, 0] - pos[:, me, 0]).to(dt)
            rel[:, me, i, 1] = (pos[:, opp, 1] - pos[:, me, 1]).to(dt)
            rel[:, me, i, 2] = alive[:, opp].to(dt)
    slots = min(MAX_T - n_opp, h * w)
    gy = torch.arange(h).view(1, h, 1)
    gx = torch.arange(w).view(1, 1, w)
    has = (fuse > 0).reshape(n, -1)
    idx = torch.arange(h * w)
    for me in range(p_out):
        cy, cx = cell[:, me, 0], cell[:, me, 1]
        dist = ((gy - cy.view(n, 1, 1)).abs() + (gx - cx.view(n, 1, 1)).abs()).reshape(n, -1)
        # (distance, cell) ascending; cells without a bomb after every bomb
        key = torch.where(has, dist, torch.full_like(dist, 1 << 20)) * (h * w) + idx
        order = key.argsort(dim=1)[:, :slots]
        for j in range(slots):
            gi = order[:, j]
            rel[:, me, n_opp + j, 0] = ((gi % w).float() - cx.float()).to(dt)
            rel[:, me, n_opp + j, 1] = ((gi // w).float() - cy.float()).to(dt)
            rel[:, me, n_opp + j, 3] = has[rows, gi].to(dt)
    glob = torch.zeros((n, p_out, GLOB_FEAT), dtype=dt)
    glob[..., 0] = (t.to(dt) / cfg.max_steps).unsqueeze(-1)
    glob[..., 1] = hp[:, :p_out].to(dt) / cfg.max_hp
    dflat = obs[:, 2 * p_full + 1].reshape(n, -1)
    glob[..., 2] = dflat.gather(1, (cell[:, :p_out, 0] * w + cell[:, :p_out, 1]).reshape(n, -1))
    glob[..., 3] = (has.float().sum(1) / cfg.max_bombs).to(dt).unsqueeze(-1)
    glob[..., 4] = (fuse.float().reshape(n, -1).sum(1) / (cfg.max_bombs * cfg.fuse)).to(dt).unsqueeze(-1)
    return local, rel, glob
