"""The astar bot (restates sim/bots.py:179-238 and :267-508).  TEST
INFRASTRUCTURE ONLY (see the package docstring).

`astar_act` is `astar_attack(sim, obs, mmask, bmask, pid)` with
`eat_crates=False`, behaviour modes off (no `_bmode` on the sim, the
configuration the learner-vs-bot workload uses) or given per env (`mode`,
the flee branch of sim/bots.py:433-443 and :496-503); `mode_tick` is the
mode ticker (:241-264).  Differences, shared with the HIP kernel:

* the 0.05-scaled noise comes in as injected uniforms `u` (N, 5) instead of
  `torch.rand(n, 5)` (sim/bots.py:355): noise = 0.05 * u;
* the chain check walks k = 1..reach cells out from the bot; the reference
  uses reach = max over the batch of the bot's blast_cap
  (`int(cap.max().item())`, sim/bots.py:477), which is the default here.

The cost fields are the reference's Bellman-Ford relaxation run to its fixed
point: dist = min(dist, min_4nbr(dist) + cost), cost = 1 + 2 * danger
(inf on blocked cells), sources at 0 even when blocked.  float32 addition is
monotone, so the fixed point does not depend on the update order or on how
often convergence is checked.
"""

from __future__ import annotations

import torch

DIRS = ((-1, 0), (1, 0), (0, -1), (0, 1))     # sim/bots.py:25 (up, down, left, right)
INF = float("inf")


def cost_field(sources, danger, blocked, lam: float = 2.0, max_passes=None):
    """(N, H*W) float32 multi-source shortest cost (sim/bots.py:179-238)."""
    n, h, w = sources.shape
    v = h * w
    rc = torch.arange(v)
    rr, cc = rc // w, rc % w
    idx, oob = [], []
    for dr, dc in DIRS:
        nr, nc = rr + dr, cc + dc
        oob.append((nr < 0) | (nr >= h) | (nc < 0) | (nc >= w))
        idx.append(nr.clamp(0, h - 1) * w + nc.clamp(0, w - 1))
    cost = 1.0 + lam * danger.reshape(n, v).float()
    cost = torch.where(blocked.reshape(n, v), torch.full_like(cost, INF), cost)
    dist = torch.where(sources.reshape(n, v), torch.zeros_like(cost), torch.full_like(cost, INF))
    for _ in range(max_passes or v):
        nd = torch.full_like(dist, INF)
        for k in range(4):
            nb = dist[:, idx[k]]
            nd = torch.minimum(nd, torch.where(oob[k], torch.full_like(nb, INF), nb))
        new = torch.minimum(dist, nd + cost)
        if torch.equal(new, dist):
            break
        dist = new
    return dist


def mode_tick(mode, timer, count: int, seed: int):
    """One step of the astar bot's approach / flee mode ticker (sim/bots.py:
    241-264, `_mode_ticker`) for its call number `count` (1, 2, ...): every
    env's timer counts down by one, and on calls with count % 16 == 0 the
    envs whose timer is at or below 0 draw a new mode (0 approach, 1 flee,
    probability 1/2 each) and a new timer uniform on 60 .. 239.  The draws are
    Philox stream 9 (key seed, counter (env, count)): the reference's laws,
    not its torch draws.  Returns the new (mode, timer)."""
    from .philox import STREAM_BOT_MODE, uniforms

    timer = timer - 1
    if count % 16 == 0:
        sw = timer <= 0
        u = torch.from_numpy(uniforms(seed, range(mode.shape[0]), count, STREAM_BOT_MODE, 2))
        new_mode = (u[:, 0] >= 0.5).to(mode.dtype)
        new_timer = (60 + (u[:, 1] * 180.0).long().clamp(max=179)).to(timer.dtype)
        mode = torch.where(sw, new_mode, mode)
        timer = torch.where(sw, new_timer, timer)
    return mode, timer


def astar_act(cfg, st, obs, mmask, bmask, pid: int, u, reach=None, mode=None):
    """(N, 2) int64 [move, place] of the astar bot for player `pid`.

    st: dict of reference-layout state tensors (wall, brick, fuse, owner, pos,
    alive, blast_cap); obs: (N, C, H, W) observation (danger is channel
    2P+1, read back from float16); mmask/bmask: (N, 5)/(N, 2) bool legality of
    `pid`; u: (N, 5) float32 uniforms; mode: (N,) behaviour mode per env (0
    approach, 1 flee; None = always approach, `make_bot(..., mode=False)`)."""
    n = obs.shape[0]
    p, h, w = cfg.n_players, cfg.height, cfg.width
    wall, brick = st["wall"].bool(), st["brick"].bool()
    fuse, owner = st["fuse"].long(), st["owner"].long()
    pos, alive = st["pos"].float(), st["alive"].bool()
    danger = obs.float()[:, 2 * p + 1]
    r = pos[:, pid, 0].floor().long().clamp(0, h - 1)
    c = pos[:, pid, 1].floor().long().clamp(0, w - 1)
    own = r * w + c
    own_dng = danger.flatten(1).gather(1, own.unsqueeze(1)).squeeze(1)

    # the bot's own live bombs, dilated growth_blast_max times (sim/bots.py:320-333)
    threat = (owner == pid) & (fuse > 0)
    for _ in range(int(cfg.growth_blast_max)):
        nb = threat.clone()
        nb[:, 1:, :] |= threat[:, :-1, :]
        nb[:, :-1, :] |= threat[:, 1:, :]
        nb[:, :, 1:] |= threat[:, :, :-1]
        nb[:, :, :-1] |= threat[:, :, 1:]
        threat = nb

    block_all = wall | brick | (fuse > 0)
    v_safe = cost_field(danger < 0.35, danger, block_all)
    opp_src = torch.zeros(n, h * w, dtype=torch.bool)
    rows = torch.arange(n)
    for o in range(p):
        if o == pid:
            continue
        ro = pos[:, o, 0].floor().long().clamp(0, h - 1)
        co = pos[:, o, 1].floor().long().clamp(0, w - 1)
        opp_src[rows, ro * w + co] = alive[:, o]
    v_opp = cost_field(opp_src.view(n, h, w), danger, block_all)

    cr = torch.stack([(r - 1).clamp(0, h - 1), (r + 1).clamp(0, h - 1), r, r, r], 1)
    cc = torch.stack([c, c, (c - 1).clamp(0, w - 1), (c + 1).clamp(0, w - 1), c], 1)
    cflat = cr * w + cc
    vopp_c = v_opp.gather(1, cflat)
    vsafe_c = v_safe.gather(1, cflat)
    dng_c = danger.flatten(1).gather(1, cflat)
    thr_c = threat.flatten(1).gather(1, cflat).float()
    blk_c = (wall | brick).flatten(1).gather(1, cflat)
    legal = mmask.bool() & ~blk_c
    noise = 0.05 * u.float()
    inf = torch.full_like(dng_c, INF)
    k5 = torch.arange(5)

    app = vopp_c + 2.0 * dng_c + 2.0 * thr_c + noise
    app = torch.where(dng_c >= 0.5, inf, app)
    app = torch.where(legal, app, inf)
    app_ok = app.min(dim=1).values.isfinite()
    use_esc = (own_dng >= 0.35) | ~app_ok
    esc = vsafe_c * 100.0 + 2.0 * thr_c + noise
    esc = torch.where(use_esc.unsqueeze(1) & (k5 == 4), inf, esc)
    esc = torch.where(legal, esc, inf)
    score = torch.where(use_esc.unsqueeze(1), esc, app)
    if mode is not None:
        # flee (sim/bots.py:433-443): away from the opponent (V_opp clamped
        # at 1e3), avoiding danger; escape first when escaping
        flee = -vopp_c.clamp(max=1e3) + 2.0 * dng_c + 2.0 * thr_c + noise
        flee = torch.where(dng_c >= 0.5, inf, flee)
        flee = torch.where(legal, flee, inf)
        flee = torch.where(use_esc.unsqueeze(1), esc, flee)
        score = torch.where((mode == 1).unsqueeze(1), flee, score)
    move = score.argmin(dim=1).long()

    any_legal = legal.any(dim=1)
    no_path = ~score.isfinite().any(dim=1)
    dng_legal = torch.where(legal, dng_c, inf)
    dng_move = torch.where(k5 < 4, dng_legal, inf)
    fallback = torch.where(dng_move.min(dim=1).values.isfinite(), dng_move.argmin(dim=1),
                           dng_legal.argmin(dim=1))
    move = torch.where(no_path & any_legal, fallback, move)

    cap = st["blast_cap"][:, pid].long()
    big = torch.full((n,), 10 ** 9, dtype=torch.long)
    dr_o, dc_o = big.clone(), big.clone()
    for o in range(p):
        if o == pid:
            continue
        ro = pos[:, o, 0].floor().long().clamp(0, h - 1)
        co = pos[:, o, 1].floor().long().clamp(0, w - 1)
        dr_o = torch.where(alive[:, o], (r - ro).abs(), dr_o)
        dc_o = torch.where(alive[:, o], (c - co).abs(), dc_o)
    aligned = ((dr_o == 0) & (dc_o <= cap)) | ((dc_o == 0) & (dr_o <= cap))
    near = (dr_o + dc_o).clamp(max=10 ** 8) <= (cap + 1).clamp(min=1)
    chain = torch.zeros(n, dtype=torch.bool)
    kmax = int(cap.max()) if reach is None else int(reach)
    for k in range(1, kmax + 1):
        for dr, dc in DIRS:
            rr_, cc_ = r + dr * k, c + dc * k
            inb = (rr_ >= 0) & (rr_ < h) & (cc_ >= 0) & (cc_ < w)
            f = fuse[rows, rr_.clamp(0, h - 1), cc_.clamp(0, w - 1)]
            chain |= inb & (f > 0) & (f <= 10)
    can_escape = (legal & (dng_c < 0.35) & ~thr_c.bool()).any(dim=1)
    place = (bmask[:, 1].bool() & (aligned | near | chain) & (own_dng < 0.2)
             & can_escape).long()
    if mode is not None:
        # flee places only on an opponent in reach, never for a chain (:496-503)
        flee_place = (bmask[:, 1].bool() & (aligned | near) & (own_dng < 0.2)
                      & can_escape).long()
        place = torch.where(mode == 1, flee_place, place)

    dead = ~alive[:, pid]
    move = torch.where(dead, torch.full_like(move, 4), move)
    place = torch.where(dead, torch.zeros_like(place), place)
    return torch.stack([move, place], dim=-1)
