"""`OracleSim`: the reference's `BatchedSim` tick restated in PyTorch ops.

Follows sim/torch_sim.py:895-1402 stage by stage (the tick), :178-420 for the
per-env re-initialisation done by a reset, :605-645 for observe/legal_mask.
Differences from the reference, all on purpose and all shared with the HIP
path:

* Randomness is injected: crate-hit / growth uniforms arrive as a (P, 2, N)
  float32 tensor, the layout the reference draws with `torch.rand(2PN)`
  (sim/torch_sim.py:1135-1138); when none is given they come from Philox
  stream `STREAM_CRATE` keyed by (seed, env, tick).
* Resets draw synthetic template maps (`qqtsim.maps.MapSpec`) from Philox
  uniforms, or with `MapSpec(kind="reference")` the reference's own map
  modes (oracle/maps_ref.py) from Philox uniforms instead of the
  reference's host generator.
* The chain explosion and danger stage A run exactly `chain_cap_rounds`
  rounds (the sync-free mode the reference's tick uses,
  sim/torch_sim.py:732-833), with empty trailing rounds skipped.
* Hazard waves and the reference's CUDA-graph mode are not modelled
  (`hazard_fraction` must be 0).
* `flush_recycle` takes each player's recycle cells as the k free cells with
  the smallest Philox keys (stream `STREAM_RECYCLE`, keyed by a flush
  counter) where the reference takes the first k of `torch.randperm`: the
  same uniform law over k-subsets, from injectable draws.

Explosion tiers.  The reference resolves explosions through a function it
builds once per sim with the first tick's blast hint bound as a default
argument (sim/torch_sim.py:809-833, `_h=hint`).  Every later tick resolves
blast tiers 1..H0 only, H0 = max(cfg.blast, largest bomb_blast after the
first tick's placement): a bomb whose own range exceeds H0 covers its cell
but sends no flame.  `resolve_tiers` holds H0 (None until the first step);
`exact_reference_resolve=False` resolves every bomb with its own range.
"""

from __future__ import annotations

import numpy as np
import torch

from . import philox
from .grid import danger_map, rays, resolve_explosions
from .maps_ref import reference_maps
from .move import center_cell, move_players
from .obs import encode_obs, legal_mask

def recycle_exclusion(cfg) -> np.ndarray:
    """(H*W,) bool: cells a recycle crate never lands on
    (sim/torch_sim.py:455-533, `_recycle_excl`): the cell and 4-neighbours
    of the open-mode spawns (the row through the middle, columns split
    evenly), of `cfg.spawn_cells()` and of the ring-mode corner spawns, plus
    the open-mode centre cross (rows and columns (n-1)//2 - 1 and (n-1)//2)."""
    h, w, p = cfg.height, cfg.width, cfg.n_players
    excl = set()
    open_row = (h - 1) / 2.0 + 0.5
    open_spawns = [(open_row, (w - 1) * (i + 1) / (p + 1) + 0.5) for i in range(p)]
    spawn_sets = [open_spawns, [(float(r), float(c)) for r, c in cfg.spawn_cells()],
                  [(float(r), float(c)) for r, c in cfg.ring_spawn_cells()]]
    for spawns in spawn_sets:
        for sy, sx in spawns:
            r, c = int(sy), int(sx)
            for dr, dc in ((0, 0), (-1, 0), (1, 0), (0, -1), (0, 1)):
                if 0 <= r + dr < h and 0 <= c + dc < w:
                    excl.add((r + dr) * w + (c + dc))
    cy, cx = (h - 1) // 2, (w - 1) // 2
    for r in range(h):
        for c in range(w):
            if r in (cy - 1, cy) or c in (cx - 1, cx):
                excl.add(r * w + c)
    m = np.zeros(h * w, dtype=bool)
    m[sorted(excl)] = True
    return m


STATE_KEYS = (
    "wall", "brick", "crate", "recycle", "fuse", "owner", "bomb_blast",
    "pos", "alive", "hp", "since_bomb", "t", "bombs_cap", "blast_cap",
    "spd_g", "invuln", "combo", "last_hit", "pending_lost", "crate_prob",
    "lo_bombs", "lo_blast", "lo_spd", "map_kind",
)


def template_maps(cfg, spec, env_ids, seed, epoch):
    """Per-env template draws shared with the HIP reset kernel.

    Returns numpy arrays: wall, brick (k, H, W) bool; pos (k, P, 2) f32;
    bombs_cap, blast_cap (k, P) int64; spd (k, P) f32.
    """
    h, w, p = cfg.height, cfg.width, cfg.n_players
    k = len(env_ids)
    if spec.kind == "pillars":
        rr, cc = np.meshgrid(np.arange(h), np.arange(w), indexing="ij")
        base = (rr == 0) | (rr == h - 1) | (cc == 0) | (cc == w - 1) \
            | ((rr % 2 == 0) & (cc % 2 == 0))
    else:
        base = np.zeros((h, w), dtype=bool)
    corners = [(1, 1), (h - 2, w - 2), (1, w - 2), (h - 2, 1)][:p]
    keep_free = np.zeros((h, w), dtype=bool)
    for r, c in corners:
        dr = 1 if r < h // 2 else -1
        dc = 1 if c < w // 2 else -1
        for (y, x) in ((r, c), (r, c + dc), (r + dr, c)):
            keep_free[y, x] = True
    wall = np.broadcast_to(base, (k, h, w)).copy()
    u_cell = philox.uniforms(seed, env_ids, epoch, philox.STREAM_RESET_CELL, h * w)
    u_cell = u_cell.reshape(k, h, w)
    brick = (~base & ~keep_free)[None] & (u_cell < np.float32(spec.brick_p))
    u_misc = philox.uniforms(seed, env_ids, epoch, philox.STREAM_RESET_MISC, 1 + 2 * p)
    pos = np.zeros((k, p, 2), dtype=np.float32)
    for i, (r, c) in enumerate(corners):
        pos[:, i, 0] = r + 0.5
        pos[:, i, 1] = c + 0.5
    if spec.swap_spawns:
        sw = u_misc[:, 0] < np.float32(0.5)
        tmp = pos[sw, 0].copy()
        pos[sw, 0] = pos[sw, 1]
        pos[sw, 1] = tmp

    def draw(u, lo, hi):
        span = hi - lo + 1
        v = np.floor(u * np.float32(span)).astype(np.int64)
        return lo + np.minimum(v, span - 1)

    bombs = np.stack([draw(u_misc[:, 1 + 2 * i], *spec.bombs_cap) for i in range(p)], 1)
    blast = np.stack([draw(u_misc[:, 2 + 2 * i], *spec.blast_cap) for i in range(p)], 1)
    spd = np.full((k, p), spec.speed, dtype=np.float32)
    return wall, brick, pos, bombs, blast, spd


class OracleSim:
    """Reference-semantics batched sim on any torch device (CPU for tests)."""

    def __init__(self, cfg, num_envs, map_spec, device="cpu", seed=0,
                 exact_reference_resolve=True):
        if cfg.hazard_fraction > 0:
            raise ValueError("hazard waves are not on the modelled path")
        self.cfg = cfg
        self.spec = map_spec
        self.num_envs = num_envs
        self.device = torch.device(device)
        self.seed = int(seed)
        self.tick = 0           # steps taken (keys the per-tick uniforms)
        self.epoch = 0          # reset calls made (keys the template draws)
        self.explore_coef = 1.0
        self.opp_boost = 0      # set_opp_boost (reference map modes only)
        self.exact_reference_resolve = exact_reference_resolve
        self.resolve_tiers = None
        n, h, w, p = num_envs, cfg.height, cfg.width, cfg.n_players
        d = self.device
        z = lambda shape, dt: torch.zeros(shape, dtype=dt, device=d)  # noqa: E731
        self.wall = z((n, h, w), torch.bool)
        self.brick = z((n, h, w), torch.bool)
        self.crate = z((n, h, w), torch.bool)
        self.recycle = z((n, h, w), torch.bool)
        self.fuse = z((n, h, w), torch.int16)
        self.owner = torch.full((n, h, w), -1, dtype=torch.int8, device=d)
        self.bomb_blast = z((n, h, w), torch.int16)
        self.pos = z((n, p, 2), torch.float32)
        self.alive = torch.ones((n, p), dtype=torch.bool, device=d)
        self.hp = torch.full((n, p), cfg.max_hp, dtype=torch.uint8, device=d)
        self.since_bomb = z((n, p), torch.int32)
        self.t = z((n,), torch.long)
        self.bombs_cap = z((n, p), torch.long)
        self.blast_cap = z((n, p), torch.long)
        self.spd_g = torch.ones((n, p), dtype=torch.float32, device=d)
        self.invuln = z((n, p), torch.long)
        self.combo = z((n, p), torch.long)
        self.last_hit = torch.full((n, p), -10 ** 9, dtype=torch.long, device=d)
        self.pending_lost = z((n, p), torch.long)
        self.crate_prob = torch.full((n,), cfg.growth_crate_prob, device=d)
        self.lo_bombs = torch.full((n, p), cfg.growth_bombs_start, dtype=torch.long, device=d)
        self.lo_blast = torch.full((n, p), cfg.growth_blast_start, dtype=torch.long, device=d)
        self.lo_spd = torch.full((n, p), cfg.growth_speed_start, dtype=torch.float32, device=d)
        self.map_kind = z((n,), torch.long)
        self.reset_all()

    # ------------------------------------------------------------ reset
    def reset_all(self) -> None:
        self.reset_(torch.ones(self.num_envs, dtype=torch.bool, device=self.device))

    def reset_(self, mask: torch.Tensor) -> None:
        """Re-initialise the envs where `mask` is True (sim/torch_sim.py:178-420
        re-init values, template maps instead of the host generators)."""
        epoch = self.epoch
        self.epoch += 1
        idx = mask.nonzero(as_tuple=True)[0]
        if idx.numel() == 0:
            return
        cfg = self.cfg
        ids = idx.cpu().numpy()
        dev = self.device
        ref = None
        if self.spec.kind == "reference":
            ref = reference_maps(cfg, ids, self.seed, epoch, self.opp_boost)
            self.wall[idx] = torch.from_numpy(ref["wall"]).to(dev)
            self.brick[idx] = torch.from_numpy(ref["brick"]).to(dev)
            self.pos[idx] = torch.from_numpy(ref["pos"]).to(dev)
            c = ref["caps01"]
            for i in range(2):          # players 2 and 3 keep theirs
                bi = torch.from_numpy(c[:, i, 0].astype(np.int64)).to(dev)
                zi = torch.from_numpy(c[:, i, 1].astype(np.int64)).to(dev)
                si = torch.from_numpy(c[:, i, 2].copy()).to(dev)
                self.bombs_cap[idx, i] = bi
                self.blast_cap[idx, i] = zi
                self.spd_g[idx, i] = si
                self.lo_bombs[idx, i] = bi
                self.lo_blast[idx, i] = zi
                self.lo_spd[idx, i] = si
            cp = torch.from_numpy(ref["crate_prob"]).to(dev)
            keep = torch.isnan(cp)
            self.crate_prob[idx] = torch.where(keep, self.crate_prob[idx], cp)
            self.map_kind[idx] = torch.from_numpy(ref["map_kind"]).to(dev)
        else:
            wall, brick, pos, bombs, blast, spd = template_maps(
                cfg, self.spec, ids, self.seed, epoch)
            self.wall[idx] = torch.from_numpy(wall).to(dev)
            self.brick[idx] = torch.from_numpy(brick).to(dev)
            self.pos[idx] = torch.from_numpy(pos).to(dev)
            self.bombs_cap[idx] = torch.from_numpy(bombs).to(dev)
            self.blast_cap[idx] = torch.from_numpy(blast).to(dev)
            self.spd_g[idx] = torch.from_numpy(spd).to(dev)
            self.lo_bombs[idx] = torch.from_numpy(bombs).to(dev)
            self.lo_blast[idx] = torch.from_numpy(blast).to(dev)
            self.lo_spd[idx] = torch.from_numpy(spd).to(dev)
            self.crate_prob[idx] = cfg.growth_crate_prob
            self.map_kind[idx] = 0
        self.crate[idx] = False
        if ref is not None:             # the open-mode start crates, after the clear
            self.crate[idx] = torch.from_numpy(ref["crate"]).to(dev)
        self.recycle[idx] = False
        self.pending_lost[idx] = 0
        self.combo[idx] = 0
        self.last_hit[idx] = -10 ** 9
        self.fuse[idx] = 0
        self.owner[idx] = -1
        self.bomb_blast[idx] = 0
        self.alive[idx] = True
        self.hp[idx] = cfg.max_hp
        self.since_bomb[idx] = cfg.place_dist_cooldown
        self.invuln[idx] = 0
        self.t[idx] = 0

    def set_opp_boost(self, v: int) -> None:
        """sim/torch_sim.py:422-426: player 1's starting caps tier (0, 1, 2)
        for the reference map modes."""
        self.opp_boost = int(v)

    # ------------------------------------------------------------ recycle flush
    def flush_recycle(self, flush_epoch: int) -> None:
        """sim/torch_sim.py:549-596: for each env and each player in id order
        with pending lost growth k > 0, min(k, free) distinct free cells (no
        wall, no brick, not excluded) become recycle crates; then every
        pending count resets.  The cells are the k free ones with the
        smallest (key, cell) of Philox stream STREAM_RECYCLE, value p*C + c,
        keyed by (seed, env, flush_epoch)."""
        cfg = self.cfg
        n, p, hw = self.num_envs, cfg.n_players, cfg.n_cells
        excl = recycle_exclusion(cfg)
        pend = self.pending_lost.numpy()
        todo = np.flatnonzero(pend.sum(1) > 0)
        if todo.size:
            u = philox.uniforms(self.seed, todo, flush_epoch, philox.STREAM_RECYCLE, p * hw)
            free = (~self.wall.view(n, hw) & ~self.brick.view(n, hw)).numpy()[todo] & ~excl
            crate, rec = self.crate.view(n, hw), self.recycle.view(n, hw)
            for row, e in enumerate(todo):
                for i in range(p):
                    k = int(pend[e, i])
                    if k <= 0:
                        continue
                    cells = np.flatnonzero(free[row])
                    keys = u[row, i * hw + cells]
                    order = np.lexsort((cells, keys))        # by key, then cell
                    pick = cells[order[:k]]
                    crate[e, pick] = True
                    rec[e, pick] = True
        self.pending_lost.zero_()

    # ------------------------------------------------------------ state I/O
    def state_dict(self) -> dict:
        return {k: getattr(self, k).clone() for k in STATE_KEYS}

    def load_state_dict(self, snap: dict) -> None:
        for k, v in snap.items():
            getattr(self, k).copy_(v)

    # ------------------------------------------------------------ views
    def blast_map(self) -> torch.Tensor:
        """Per-cell blast: the bomb's own range, cfg.blast where unset
        (sim/torch_sim.py:727-730)."""
        return torch.where(self.bomb_blast > 0, self.bomb_blast.long(),
                           torch.full_like(self.bomb_blast.long(), self.cfg.blast))

    def danger(self) -> torch.Tensor:
        cfg = self.cfg
        return danger_map(self.fuse, self.wall, self.blast_map(), cfg.fuse,
                          self.brick, cfg.max_chain, rounds=cfg.chain_cap_rounds)

    def observe(self) -> torch.Tensor:
        """(N, C, H, W) observation of the current state (sim/torch_sim.py:605-627)."""
        return encode_obs(self.cfg, self.wall, self.fuse, self.owner, self.pos,
                          self.alive, self.t, self.brick, self.bomb_blast,
                          crate=self.crate, invuln=self.invuln,
                          bombs_p=self.bombs_cap, danger=self.danger())

    def legal_mask(self):
        return legal_mask(self.cfg, self.wall, self.fuse, self.owner, self.pos,
                          self.alive, self.brick, self.bombs_cap)

    def crate_uniforms(self) -> torch.Tensor:
        """(P, 2, N) uniforms of Philox stream STREAM_CRATE for this tick."""
        n, p = self.num_envs, self.cfg.n_players
        u = philox.uniforms(self.seed, np.arange(n), self.tick, philox.STREAM_CRATE, 2 * p)
        return torch.from_numpy(u.reshape(n, p, 2).transpose(1, 2, 0).copy()).to(self.device)

    # ------------------------------------------------------------ the tick
    def _place_bombs(self, bomb, alive0):
        """Players place in id order at their pre-move centre cell
        (sim/torch_sim.py:1357-1402)."""
        cfg = self.cfg
        n, w = self.num_envs, cfg.width
        ff = self.fuse.view(n, -1)
        fo = self.owner.view(n, -1)
        fb = self.bomb_blast.view(n, -1)
        fr = self.brick.view(n, -1)
        cell = center_cell(self.pos)
        placed = torch.zeros((n, cfg.n_players), dtype=torch.bool, device=self.device)
        for me in range(cfg.n_players):
            idx = (cell[:, me, 0] * w + cell[:, me, 1]).clamp(0, cfg.n_cells - 1).unsqueeze(1)
            live = ((self.owner == me) & (self.fuse > 0)).flatten(1).sum(1)
            cur_f = ff.gather(1, idx).squeeze(1)
            on_brick = fr.gather(1, idx).squeeze(1)
            ok = (alive0[:, me] & (bomb[:, me] == 1) & (cur_f <= 0) & ~on_brick
                  & (live < self.bombs_cap[:, me]))
            placed[:, me] = ok
            ff.scatter_(1, idx, torch.where(ok, torch.full_like(cur_f, cfg.fuse),
                                            cur_f).unsqueeze(1))
            cur_o = fo.gather(1, idx).squeeze(1)
            fo.scatter_(1, idx, torch.where(ok, torch.full_like(cur_o, me),
                                            cur_o).unsqueeze(1))
            cur_b = fb.gather(1, idx).squeeze(1)
            fb.scatter_(1, idx, torch.where(ok, self.blast_cap[:, me].to(cur_b.dtype),
                                            cur_b).unsqueeze(1))
        return placed

    def _place_bonus(self, placed, alive0):
        """Placement reward from this tick's new bombs (sim/torch_sim.py:1263-1355):
        0.05 per alive enemy whose centre cell the new bomb's flame covers, plus
        0.20 x (0.15 + 0.85 (1 - fuse/FUSE)) per live older bomb it would ignite."""
        cfg = self.cfg
        n, p, w, hw = self.num_envs, cfg.n_players, cfg.width, cfg.n_cells
        if not (cfg.place_cover_reward or cfg.place_chain_reward or cfg.place_dist_reward):
            return torch.zeros(n, p, device=self.device)
        live = self.fuse > 0
        bmap = self.blast_map()
        frac = (self.fuse.float() / float(cfg.fuse)).clamp(0.0, 1.0)
        weight = cfg.chain_time_factor + (1.0 - cfg.chain_time_factor) * (1.0 - frac)
        cell = center_cell(self.pos)
        flat = (cell[..., 0] * w + cell[..., 1]).clamp(0, hw - 1)
        placed_map = torch.zeros(n, hw, dtype=torch.bool, device=self.device)
        for me in range(p):                      # later players overwrite
            placed_map.scatter_(1, flat[:, me:me + 1], placed[:, me:me + 1])
        placed_map = placed_map.view(n, cfg.height, w)
        cover = torch.zeros(n, p, device=self.device)
        chain = torch.zeros(n, p, device=self.device)
        dist = torch.zeros(n, p, device=self.device)
        cooldown_ok = self.since_bomb >= cfg.place_dist_cooldown
        cell_f = cell.float()
        for me in range(p):
            seed = torch.zeros(n, hw, dtype=torch.bool, device=self.device)
            seed.scatter_(1, flat[:, me:me + 1], placed[:, me:me + 1])
            cov = rays(seed.view(n, cfg.height, w), self.wall, live, bmap, self.brick)
            cf = cov.view(n, -1)
            for o in range(p):
                if o == me:
                    continue
                under = cf.gather(1, flat[:, o:o + 1]).squeeze(1)
                cover[:, me] += (under & alive0[:, o]).float()
                if cfg.place_dist_reward > 0:
                    dd = (cell_f[:, me] - cell_f[:, o]).norm(dim=-1)
                    ok = placed[:, me] & ~under & (dd < cfg.place_dist_radius) \
                        & cooldown_ok[:, me] & alive0[:, o]
                    gain = 1.0 - dd / cfg.place_dist_radius
                    dist[:, me] += (ok * gain.clamp(min=0.0)).float()
            chained = cov & live & (self.owner >= 0) & ~placed_map
            chain[:, me] = (weight * chained.float()).flatten(1).sum(1)
        bonus = (cfg.place_cover_reward * cover + cfg.place_dist_reward * dist
                 + cfg.place_chain_reward * chain)
        return bonus * alive0.float()

    def _grow(self, hits, alive0, u_grow):
        """Crate growth: attribute floor(3u) -> +1 bomb / +1 blast / +speed step,
        each clamped to its cap (sim/torch_sim.py:862-893)."""
        cfg = self.cfg
        hits = hits.long() * alive0.long()
        attr = (u_grow * 3).floor().long()
        self.bombs_cap = torch.clamp(self.bombs_cap + (attr == 0).long() * hits,
                                     max=cfg.growth_bombs_max)
        self.blast_cap = torch.clamp(self.blast_cap + (attr == 1).long() * hits,
                                     max=cfg.growth_blast_max)
        self.spd_g = torch.min(self.spd_g + ((attr == 2).long() * hits).float()
                               * cfg.growth_speed_step,
                               torch.full_like(self.spd_g, cfg.growth_speed_max))

    def step(self, actions, auto_reset=True, crate_u=None):
        """One tick (sim/torch_sim.py:895-1261).  `actions` (N, P, 2) int."""
        cfg = self.cfg
        n, p, w, hw = self.num_envs, cfg.n_players, cfg.width, cfg.n_cells
        if crate_u is None:
            crate_u = self.crate_uniforms()
        self.tick += 1
        alpha = self.explore_coef
        alive0 = self.alive.clone()
        hp_before = self.hp.clone()
        move, bomb = actions[..., 0].long(), actions[..., 1].long()
        # 1. fuse countdown
        self.fuse.copy_(torch.where(self.fuse > 0, self.fuse - 1, self.fuse))
        # 2. placement + its reward
        placed = self._place_bombs(bomb, alive0)
        hint = max(int(self.bomb_blast.max()), int(cfg.blast))
        if self.resolve_tiers is None:
            self.resolve_tiers = hint
        tiers = self.resolve_tiers if self.exact_reference_resolve else hint
        if bool(placed.any()):
            place_bonus = self._place_bonus(placed, alive0)
        else:
            place_bonus = torch.zeros(n, p, device=self.device)
        self.since_bomb.add_(1)
        self.since_bomb.masked_fill_(placed, 0)
        # 3. movement (blocked after placement)
        blocked = self.wall | self.brick | (self.fuse > 0)
        self.pos.copy_(move_players(cfg, self.pos, move, alive0, blocked, self.spd_g))
        # 4. explosions
        covered, trig = resolve_explosions(self.fuse, self.owner, self.wall,
                                           self.blast_map(), cfg.max_chain, self.brick,
                                           rounds=cfg.chain_cap_rounds, blast_max_hint=tiers)
        if cfg.map_mode == "corridor":
            self.crate |= self.brick & covered
        self.brick &= ~covered
        # 5. damage at the post-move centre cell
        cell = center_cell(self.pos)
        flat = (cell[..., 0] * w + cell[..., 1]).clamp(0, hw - 1)
        hit = alive0 & covered.view(n, -1).gather(1, flat)
        hit_eff = hit & (self.invuln <= 0)
        hp_new = (self.hp.to(torch.int32) - hit_eff.to(torch.int32)).clamp(min=0)
        died = hit_eff & (hp_new == 0)
        self.hp.copy_(hp_new.to(torch.uint8))
        self.alive.copy_(alive0 & ~died)
        self.invuln.sub_(1).clamp_(min=0)
        self.invuln.masked_fill_(hit_eff, cfg.invuln_ticks)
        # 6. clear exploded cells
        self.fuse.masked_fill_(trig, 0)
        self.owner.masked_fill_(trig, -1)
        self.bomb_blast.masked_fill_(trig, 0)
        # 7. time and termination
        self.t.add_(1)
        n_alive = self.alive.sum(dim=1)
        done = (n_alive <= 1) | (self.t >= cfg.max_steps)
        dmg = (hp_before.to(torch.int32) - self.hp.to(torch.int32)).clamp(min=0).float()
        dealt = dmg.sum(dim=1, keepdim=True) - dmg
        a0 = alive0.float()
        reward = (-torch.full_like(a0, cfg.step_penalty) * a0
                  + torch.full_like(a0, cfg.hit_reward) * dealt
                  - torch.full_like(a0, cfg.hit_reward) * dmg
                  + torch.full_like(a0, alpha) * place_bonus * a0)
        if cfg.hit_attr_penalty > 0:
            hit_any = (dmg > 0) & alive0
            pen = cfg.hit_attr_penalty
            nb = torch.clamp(self.bombs_cap - pen, min=self.lo_bombs)
            nz = torch.clamp(self.blast_cap - pen, min=self.lo_blast)
            ns = torch.max(self.spd_g - torch.full_like(self.spd_g, pen * cfg.growth_speed_step),
                           self.lo_spd)
            lost = ((self.bombs_cap - nb) + (self.blast_cap - nz)
                    + torch.round((self.spd_g - ns) / cfg.growth_speed_step)).long()
            self.bombs_cap = torch.where(hit_any, nb, self.bombs_cap)
            self.blast_cap = torch.where(hit_any, nz, self.blast_cap)
            self.spd_g = torch.where(hit_any, ns, self.spd_g)
            self.pending_lost.add_(lost * hit_any.long())
        # chain_blast_bonus is 0 in every modelled config; its term adds 0
        reward = reward + torch.full_like(a0, alpha) * torch.zeros_like(a0) * a0
        if cfg.map_mode == "corridor":
            stood = self.crate.view(n, -1).gather(1, flat)
            reward = reward + torch.full_like(a0, cfg.brick_reward) * stood.float() * a0
            u_hit = crate_u[:, 0, :].transpose(0, 1)
            u_grow = crate_u[:, 1, :].transpose(0, 1)
            rec = self.recycle.view(n, -1).gather(1, flat)
            prob = torch.where(rec, torch.full_like(u_hit, cfg.recycle_crate_prob),
                               self.crate_prob.unsqueeze(1).expand(n, p))
            hits = stood & (u_hit < prob) & alive0
            self._grow(hits, alive0, u_grow)
            self.crate.view(n, -1).scatter_(1, flat, False)
            self.recycle.view(n, -1).scatter_(1, flat, False)
        # danger on the post-clear state (cached for observe by the reference)
        dng = danger_map(self.fuse, self.wall, self.blast_map(), cfg.fuse, self.brick,
                         cfg.max_chain, rounds=cfg.chain_cap_rounds, blast_max_hint=hint)
        standing = dng.view(n, -1).gather(1, flat)
        reward = reward - torch.full_like(a0, alpha * cfg.danger_penalty) * standing * a0
        if cfg.combo_reward > 0:
            hit_this = dmg > 0
            for me in range(p):
                dealt_me = dealt[:, me]
                c = self.combo[:, me].clone()
                gap = self.t - self.last_hit[:, me]
                factor = cfg.combo_gap_factor ** gap.clamp(min=0).float()
                inc = (dealt_me > 0).long()
                combo_now = (c + inc) * inc
                pts = (combo_now.float() * torch.full_like(dealt_me, cfg.combo_reward)
                       * factor * dealt_me.clamp(max=1).float())
                reward[:, me] += pts * a0[:, me]
                self.combo[:, me] = torch.where(inc.bool(), combo_now, c)
                self.last_hit[:, me] = torch.where(inc.bool(), self.t, self.last_hit[:, me])
                self.combo[:, me] = torch.where(hit_this[:, me], torch.zeros_like(c),
                                                self.combo[:, me])
        death_done = done & (n_alive == 1)
        one_left = (n_alive == 1).unsqueeze(1)
        winner = death_done.unsqueeze(1) & self.alive & one_left
        loser = death_done.unsqueeze(1) & ~self.alive & one_left
        hpf = self.hp.float()
        all_alive = done & (n_alive == p)
        if cfg.timeout_draw:
            tscale = alpha
        else:
            for me in range(p):
                others = [o for o in range(p) if o != me]
                winner[:, me] |= all_alive & (hpf[:, me:me + 1] > hpf[:, others]).all(dim=1)
                loser[:, me] |= all_alive & (hpf[:, me:me + 1] < hpf[:, others]).any(dim=1)
            tscale = 1.0
        if cfg.win_hp_scaled:
            for me in range(p):
                diff = hpf[:, me] - (hpf.sum(dim=1) - hpf[:, me]) / (p - 1)
                base = (cfg.win_bonus / cfg.max_hp) * diff
                reward[:, me] += base * death_done.float() + base * all_alive.float() * tscale
        else:
            reward = reward + torch.full_like(a0, cfg.win_bonus) * (winner.float() - loser.float())
            if cfg.timeout_draw:
                for me in range(p):
                    diff = hpf[:, me] - (hpf.sum(dim=1) - hpf[:, me]) / (p - 1)
                    reward[:, me] += (torch.full_like(diff, cfg.win_bonus / cfg.max_hp)
                                      * diff * all_alive.float() * tscale)
        info = {"n_alive": n_alive, "blast": covered, "trig": trig, "died": died,
                "winner": winner.clone()}
        if auto_reset:
            self.reset_(done)
        return reward, done, info
