"""`HipBatchedSim`: the reference's `BatchedSim` API on the MI355X HIP kernels.

Drop-in for `sim.torch_sim.BatchedSim` (sim/torch_sim.py:53-1466) on the
rollout path: `reset_all()`, `reset_(mask)`, `step(actions, auto_reset)`,
`observe()`, `legal_mask()`, `state_dict()` / `load_state_dict()`,
`set_explore_coef`, plus read-only reference-layout views of the state
attributes callers read (`pos`, `alive`, `hp`, `fuse`, `owner`, `t`, ...).

Each `step` is ONE kernel launch: the tick, the auto-reset of finished envs,
and the observation + legality masks of the resulting state, which
`observe()` / `legal_mask()` then return without another launch (the
reference recomputes them, sim/torch_sim.py:605-645).  `observe()` returns a
persistent buffer, as the reference's CUDA backend does
(sim/cuda/wrapper.py:140-147); callers that keep it across ticks copy it.

Randomness is injected (see `oracle/philox.py` for the shared layout):
crate-hit / growth uniforms per tick come from Philox(seed, env, tick) unless
`step(..., crate_u=(P,2,N) float32)` passes them, as the reference's
`torch.rand(2PN).view(P,2,N)` would (sim/torch_sim.py:1135-1138).  Resets
draw template maps (`MapSpec`), or with `MapSpec(kind="reference")` the
reference's own corridor / open / ring map modes, from Philox(seed, env,
epoch).

Explosion tiers: the reference binds the first tick's blast hint into its
explosion resolver (sim/torch_sim.py:809-833, `_h=hint`), so later ticks
only resolve blast tiers up to that first hint.  `resolve_tiers` reproduces
that (it is measured at the first `step`); pass
`exact_reference_resolve=False` to resolve each bomb with its own range.
"""

from __future__ import annotations

import torch

from . import _capi, state as st
from .config import N_BOMB, N_MOVES, SimConfig
from .maps import KIND_CODES, MapSpec, recycle_exclusion

SUPPORTED = {(13, 13, 2), (7, 7, 2), (9, 9, 2), (13, 13, 3), (13, 13, 4)}


def config_struct(cfg: SimConfig, spec: MapSpec) -> _capi.SimConfigC:
    """float32 constants exactly as the reference's tensor ops round them."""
    c = _capi.SimConfigC()
    ints = dict(height=cfg.height, width=cfg.width, n_players=cfg.n_players, fuse=cfg.fuse,
                blast=cfg.blast, max_steps=cfg.max_steps, max_chain=cfg.max_chain,
                chain_cap_rounds=cfg.chain_cap_rounds, max_hp=cfg.max_hp,
                invuln_ticks=cfg.invuln_ticks, hit_attr_penalty=cfg.hit_attr_penalty,
                place_dist_cooldown=cfg.place_dist_cooldown,
                growth_bombs_max=cfg.growth_bombs_max, growth_blast_max=cfg.growth_blast_max,
                corridor=int(cfg.map_mode == "corridor"), timeout_draw=int(cfg.timeout_draw),
                win_hp_scaled=int(cfg.win_hp_scaled),
                map_kind=KIND_CODES[spec.kind], swap_spawns=int(spec.swap_spawns),
                bombs_lo=spec.bombs_cap[0], bombs_hi=spec.bombs_cap[1],
                blast_lo=spec.blast_cap[0], blast_hi=spec.blast_cap[1],
                spawn_cooldown=cfg.place_dist_cooldown)
    floats = dict(radius=cfg.radius, step_len=cfg.step_len,
                  pos_hi_y=cfg.height - cfg.radius, pos_hi_x=cfg.width - cfg.radius,
                  step_penalty=cfg.step_penalty, hit_reward=cfg.hit_reward,
                  win_bonus=cfg.win_bonus, win_per_hp=cfg.win_bonus / cfg.max_hp,
                  danger_penalty=cfg.danger_penalty, brick_reward=cfg.brick_reward,
                  place_cover_reward=cfg.place_cover_reward,
                  place_chain_reward=cfg.place_chain_reward,
                  place_dist_reward=cfg.place_dist_reward,
                  place_dist_radius=cfg.place_dist_radius,
                  chain_time_factor=cfg.chain_time_factor,
                  chain_time_rest=1.0 - cfg.chain_time_factor,
                  combo_reward=cfg.combo_reward, combo_gap_factor=cfg.combo_gap_factor,
                  growth_speed_step=cfg.growth_speed_step,
                  growth_speed_max=cfg.growth_speed_max,
                  hit_speed_drop=cfg.hit_attr_penalty * cfg.growth_speed_step,
                  recycle_crate_prob=cfg.recycle_crate_prob,
                  growth_crate_prob=cfg.growth_crate_prob,
                  brick_p=spec.brick_p, spawn_speed=spec.speed)
    for k, v in ints.items():
        setattr(c, k, int(v))
    for k, v in floats.items():
        setattr(c, k, float(v))
    _reference_map_fields(c, cfg)
    return c


def _reference_map_fields(c, cfg: SimConfig) -> None:
    """Fields of the reference map modes (sim/torch_sim.py:178-420): the
    cumulative map-type thresholds as the reference's Python sums, and the
    corridor / open / ring spawn tables with their cells taken from the
    double values (cfg.spawn_cells())."""
    h, w, p = cfg.height, cfg.width, cfg.n_players
    for k in ("top_wall_rows", "corridor_width", "open_obstacle_max", "ring_center_h",
              "ring_center_w", "max_bombs", "growth_bombs_start", "growth_blast_start",
              "open_growth_bombs", "open_growth_blast", "opp_growth_bombs", "opp_growth_blast"):
        setattr(c, k, int(getattr(cfg, k)))
    c.random_wall_rows = int(bool(cfg.random_wall_rows))
    c.open_crate_cross = int(bool(cfg.open_crate_cross))
    for k in ("wall_density", "ring_brick_density", "ring_crate_prob", "growth_speed_start",
              "open_growth_speed", "opp_growth_speed", "opp_hist_mult"):
        setattr(c, k, float(getattr(cfg, k)))
    pf = cfg.pure_open_fraction
    c.thr_pure = pf
    c.thr_open = pf + cfg.open_fraction
    c.thr_ring = pf + cfg.open_fraction + cfg.ring_fraction
    row_c = (cfg.top_wall_rows + (h - 1)) / 2.0 + 0.5
    c0 = (w - cfg.corridor_width) / 2.0 + 0.5
    step = (cfg.corridor_width - 2) / max(1, p - 1)
    row_o = (h - 1) / 2.0 + 0.5
    tables = ([(row_c, c0 + 1.0 + i * step) for i in range(p)],
              [(row_o, (w - 1) * (i + 1) / (p + 1) + 0.5) for i in range(p)],
              [(1.5, 1.5), (1.5, w - 0.5), (h - 0.5, w - 0.5), (h - 0.5, 1.5)][:p])
    for k, spawns in enumerate(tables):
        for i, (y, x) in enumerate(spawns):
            c.ref_spawn_y[k][i] = y
            c.ref_spawn_x[k][i] = x
            c.ref_spawn_cell[k][i] = int(y) * w + int(x)


class _Info(dict):
    """The step's info dict; the (N,H,W) cover/trigger maps are unpacked from
    bitsets on first access."""

    def __init__(self, base, cov_bits, trg_bits, h, w):
        super().__init__(base)
        self._lazy = {"blast": cov_bits, "trig": trg_bits}
        self._hw = (h, w)

    def __missing__(self, key):
        if key in self._lazy:
            v = st.unpack_bits(self._lazy[key], *self._hw)
            self[key] = v
            return v
        raise KeyError(key)

    def __contains__(self, key):
        return key in self._lazy or dict.__contains__(self, key)


class HipBatchedSim:
    def __init__(self, cfg: SimConfig, num_envs: int, device="cuda", seed: int = 0,
                 map_spec: MapSpec | None = None, exact_reference_resolve: bool = True):
        key = (cfg.height, cfg.width, cfg.n_players)
        if key not in SUPPORTED:
            raise ValueError(f"HIP kernels are compiled for (H, W, P) in {sorted(SUPPORTED)}")
        if cfg.hazard_fraction > 0:
            raise ValueError("hazard waves are not on the HIP rollout path")
        if not (cfg.obs_fp16 and cfg.obs_extra_enabled):
            raise ValueError("the HIP path writes the 5P+4-channel float16 observation")
        if cfg.fuse > 255:
            raise ValueError("fuse must be <= 255 for the packed cell word")
        if cfg.chain_blast_bonus != 0:
            raise ValueError("chain_blast_bonus (sim/torch_sim.py:981-1005) is not on the HIP "
                             "rollout path; it must be 0")
        self.cfg = cfg
        self.spec = map_spec or MapSpec()
        self.num_envs = int(num_envs)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HipBatchedSim runs on a ROCm device")
        self.seed = int(seed)
        self.tick = 0
        self.epoch = 0
        self.flushes = 0          # recycle flushes so far (keys their cell draws)
        self._excl = None
        self.explore_coef = 1.0
        self.exact_reference_resolve = exact_reference_resolve
        self.resolve_tiers: int | None = None
        self._lib = _capi.lib()
        self._cfg_c = config_struct(cfg, self.spec)
        n, h, w, p = self.num_envs, cfg.height, cfg.width, cfg.n_players
        d = self.device
        i32 = dict(dtype=torch.int32, device=d)
        self._cells = torch.zeros((n, h * w), **i32)
        self._players = torch.zeros((n, p, st.P_SLOTS), **i32)
        self._envs = torch.zeros((n, st.E_SLOTS), **i32)
        # the reference's initial values where no reset writes (sim/torch_sim.py:
        # 80-87, 105, 147-149): speed 1, penalty floors at the growth starts,
        # crate probability growth_crate_prob
        f32bits = lambda v: torch.tensor([v], dtype=torch.float32).view(torch.int32).item()  # noqa: E731
        self._players[..., st.P_SPD] = f32bits(1.0)
        self._players[..., st.P_LOB] = cfg.growth_bombs_start
        self._players[..., st.P_LOZ] = cfg.growth_blast_start
        self._players[..., st.P_LOS] = f32bits(cfg.growth_speed_start)
        self._envs[:, st.E_CRATE_PROB] = f32bits(cfg.growth_crate_prob)
        self._opp_boost = 0
        self._obs = torch.zeros((n, cfg.n_channels, h, w), dtype=torch.float16, device=d)
        self._mm = torch.zeros((n, p, N_MOVES), dtype=torch.uint8, device=d)
        self._bm = torch.zeros((n, p, N_BOMB), dtype=torch.uint8, device=d)
        self._reward = torch.zeros((n, p), dtype=torch.float32, device=d)
        self._done = torch.zeros((n,), dtype=torch.uint8, device=d)
        self._n_alive = torch.zeros((n,), **i32)
        self._died = torch.zeros((n, p), dtype=torch.uint8, device=d)
        self._winner = torch.zeros((n, p), dtype=torch.uint8, device=d)
        self._cov = torch.zeros((n, 8), **i32)
        self._trg = torch.zeros((n, 8), **i32)
        self._probe = torch.zeros((n,), **i32)
        self._fresh = False   # obs/mask buffers describe the current state
        self.reset_all()

    # ---------------------------------------------------------------- launch
    def _launch(self, mode, actions=None, crate_u=None, reset_mask=None, auto_reset=True,
                outputs=True, epoch=None, danger_out=None):
        a = _capi.TickArgsC()
        a.n_envs = self.num_envs
        a.mode = mode
        a.auto_reset = int(bool(auto_reset))
        a.resolve_tiers = int(self.resolve_tiers if self.resolve_tiers is not None else 255)
        a.explore_coef = float(self.explore_coef)
        a.danger_coef = float(self.explore_coef * self.cfg.danger_penalty)
        a.seed = self.seed & 0xFFFFFFFFFFFFFFFF
        a.opp_boost = self._opp_boost
        a.tick = self.tick & 0xFFFFFFFF
        a.epoch = (self.epoch if epoch is None else epoch) & 0xFFFFFFFF
        a.cells = self._cells.data_ptr()
        a.players = self._players.data_ptr()
        a.envs = self._envs.data_ptr()
        if actions is not None:
            if actions.dtype == torch.int8:
                a.actions_i8 = actions.data_ptr()
            else:
                a.actions = actions.data_ptr()
        a.crate_u = _capi.ptr(crate_u)
        a.reset_mask = _capi.ptr(reset_mask)
        if mode == _capi.MODE_STEP:
            a.reward = self._reward.data_ptr()
            a.done = self._done.data_ptr()
            a.n_alive = self._n_alive.data_ptr()
            a.died = self._died.data_ptr()
            a.winner = self._winner.data_ptr()
            a.covered = self._cov.data_ptr()
            a.triggered = self._trg.data_ptr()
        if outputs:
            a.obs = self._obs.data_ptr()
            a.move_mask = self._mm.data_ptr()
            a.bomb_mask = self._bm.data_ptr()
        if mode == _capi.MODE_PROBE:
            a.probe_out = self._probe.data_ptr()
        if mode == _capi.MODE_FLUSH:
            a.recycle_excl = self.recycle_excl().data_ptr()
        a.danger_out = _capi.ptr(danger_out)
        _capi.check(self._lib.qqt_tick(self._cfg_c, a, _capi.stream_handle(self.device)))

    def _as_device(self, t, dtype, shape):
        t = torch.as_tensor(t)
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"expected shape {tuple(shape)}, got {tuple(t.shape)}")
        return t.to(self.device, dtype).contiguous()

    # ---------------------------------------------------------------- reset
    def reset_all(self) -> None:
        self.reset_(torch.ones(self.num_envs, dtype=torch.bool, device=self.device))

    def reset_(self, mask: torch.Tensor) -> None:
        """Reset of the envs where `mask` is True (sim/torch_sim.py:178-420):
        template maps, or the reference's map modes for MapSpec("reference")."""
        m = self._as_device(mask, torch.uint8, (self.num_envs,))
        self._launch(_capi.MODE_RESET, reset_mask=m)
        self.epoch += 1
        self._fresh = True

    # ---------------------------------------------------------------- tick
    def _first_tick_tiers(self, acts) -> int:
        """Largest bomb_blast after this tick's placement, at least cfg.blast:
        the hint the reference binds into its resolver at its first tick."""
        self._launch(_capi.MODE_PROBE, actions=acts, outputs=False)
        return max(int(self._probe.max()), int(self.cfg.blast))

    def step(self, actions: torch.Tensor, auto_reset: bool = True, crate_u=None):
        """actions (N, P, 2) int: [..., 0] move, [..., 1] bomb.  Returns
        (reward (N,P) f32, done (N,) bool, info) like sim/torch_sim.py:895-1261."""
        n, p = self.num_envs, self.cfg.n_players
        acts = actions if (torch.is_tensor(actions) and actions.dtype == torch.int8
                           and actions.is_cuda and actions.is_contiguous()) \
            else self._as_device(actions, torch.int64, (n, p, 2))
        if crate_u is not None:
            crate_u = self._as_device(crate_u, torch.float32, (p, 2, n))
        if self.resolve_tiers is None:
            self.resolve_tiers = self._first_tick_tiers(acts) \
                if self.exact_reference_resolve else 255
        self._launch(_capi.MODE_STEP, actions=acts, crate_u=crate_u, auto_reset=auto_reset)
        self.tick += 1
        if auto_reset:
            self.epoch += 1
        self._fresh = True
        info = _Info({"n_alive": self._n_alive.long(), "died": self._died.clone().view(torch.bool),
                      "winner": self._winner.clone().view(torch.bool)},
                     self._cov.clone(), self._trg.clone(), self.cfg.height, self.cfg.width)
        return self._reward.clone(), self._done.clone().view(torch.bool), info

    def _refresh(self) -> None:
        if not self._fresh:
            self._launch(_capi.MODE_OBSERVE)
            self._fresh = True

    def observe(self) -> torch.Tensor:
        """(N, C, H, W) float16 observation of the current state (persistent buffer)."""
        self._refresh()
        return self._obs

    def legal_mask(self):
        """(move_mask (N,P,5) bool, bomb_mask (N,P,2) bool) of the current state."""
        self._refresh()
        return self._mm.view(torch.bool), self._bm.view(torch.bool)

    def local_view_features(self, only_p0: bool = False, out=None):
        """The lstm arch's per-player features of the current state
        (sim/obs.py:243-340 local_view_features(cfg, obs, pos, alive, t,
        fuse, hp, only_p0)) in one launch: (local (N,P',C,7,7), rel
        (N,P',10,6), glob (N,P',5)) float16, P' = 1 when only_p0.  Bombs at
        equal L1 distance, and the cells of the slots past the last bomb, are
        taken in ascending cell index (the reference leaves that order to
        torch.topk).  `out` = three tensors of those shapes to write into
        (rows may be strided, e.g. one tick of a rollout buffer)."""
        self._refresh()
        n, p, c = self.num_envs, self.cfg.n_players, self.cfg.n_channels
        po = 1 if only_p0 else p
        shapes = ((n, po, c, 7, 7), (n, po, 10, 6), (n, po, 5))
        if out is None:
            out = tuple(torch.empty(s, dtype=torch.float16, device=self.device) for s in shapes)
        for t, s in zip(out, shapes):
            if tuple(t.shape) != s or t.dtype != torch.float16 or t.device != self.device \
                    or not t[0].is_contiguous():
                raise ValueError(f"feature output must be float16 {s} with contiguous rows")
        a = _capi.LstmFeatArgsC()
        a.n_envs, a.p_out = n, po
        a.cells, a.players, a.envs = (self._cells.data_ptr(), self._players.data_ptr(),
                                      self._envs.data_ptr())
        a.obs = self._obs.data_ptr()
        a.local, a.rel, a.glob = (t.data_ptr() for t in out)
        a.local_stride, a.rel_stride, a.glob_stride = (t.stride(0) for t in out)
        _capi.check(self._lib.qqt_lstm_features(self._cfg_c, a, _capi.stream_handle(self.device)))
        return out

    def danger(self) -> torch.Tensor:
        """(N, H, W) float32 danger map of the current state, as the
        reference's `_danger_c()` / `blast.danger_map` gives it
        (sim/torch_sim.py:732-762, sim/blast.py:158-317); the observation's
        danger channel is its float16 rounding.  One OBSERVE launch, which
        also refreshes the observation and masks."""
        out = torch.empty((self.num_envs, self.cfg.height, self.cfg.width),
                          dtype=torch.float32, device=self.device)
        self._launch(_capi.MODE_OBSERVE, danger_out=out)
        self._fresh = True
        return out

    # ---------------------------------------------------------------- state
    def state_dict(self) -> dict:
        """Every state tensor in the reference's layout and dtypes (the
        reference's 11 keys, sim/torch_sim.py:705-723, plus the per-player
        growth/penalty/combo state it keeps outside state_dict)."""
        return st.unpack(self._cells, self._players, self._envs, self.cfg.height, self.cfg.width)

    def load_state_dict(self, snap: dict) -> None:
        st.pack_into(self._cells, self._players, self._envs, snap, self.cfg.height,
                     self.cfg.width)
        self._fresh = False

    def set_explore_coef(self, v: float) -> None:
        self.explore_coef = float(v)

    def set_opp_boost(self, v: int) -> None:
        """Player 1's starting tier for the reference map modes
        (sim/torch_sim.py:422-426; 0, 1 or 2).  Template resets draw caps
        from the MapSpec instead."""
        if int(v) not in (0, 1, 2):
            raise ValueError("opp boost must be 0, 1 or 2")
        self._opp_boost = int(v)

    def recycle_excl(self) -> torch.Tensor:
        """(H*W,) uint8 device mask of the cells recycle crates avoid."""
        if self._excl is None:
            m = torch.zeros(self.cfg.height * self.cfg.width, dtype=torch.uint8)
            m[recycle_exclusion(self.cfg)] = 1
            self._excl = m.to(self.device)
        return self._excl

    def flush_recycle(self) -> None:
        """BatchedSim.flush_recycle (sim/torch_sim.py:549-596) as one launch:
        every player's pending lost growth becomes that many recycle crates on
        distinct free cells (the k smallest Philox keys among them, the
        uniform k-subset law of the reference's randperm), the counts reset,
        and the observation and masks are refreshed.  No host sync: envs with
        nothing pending are left as they are."""
        self._launch(_capi.MODE_FLUSH, epoch=self.flushes)
        self.flushes += 1
        self._fresh = True

    # Every launch and load_state_dict assigns `_fresh`, so an assignment
    # marks the packed state as possibly changed: it drops the converted
    # attribute views and counts a state version (a bot reading a batch
    # statistic that a tick wrote checks that nothing changed since).
    @property
    def _fresh(self) -> bool:
        return self.__dict__["_fresh_flag"]

    @_fresh.setter
    def _fresh(self, v: bool) -> None:
        self.__dict__["_fresh_flag"] = bool(v)
        self.__dict__["_views"] = {}
        self.__dict__["_state_version"] = self.__dict__.get("_state_version", 0) + 1

    def __getattr__(self, name):
        """Reference attribute reads (`sim.hp`, `sim.pos`, `sim.fuse`, ...): the
        one tensor asked for, in the reference's layout, converted once per
        state change and cached until the next launch (read-only copies)."""
        if name in st.ALL_KEYS:
            views = self.__dict__.setdefault("_views", {})
            if name not in views:
                views[name] = st.unpack_key(self._cells, self._players, self._envs,
                                            self.cfg.height, self.cfg.width, name)
            return views[name]
        raise AttributeError(name)
