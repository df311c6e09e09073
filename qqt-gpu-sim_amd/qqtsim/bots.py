"""`HipAstarBot`: the reference's astar rule bot on the MI355X kernel.

Drop-in for `make_bot(sim, "astar", mode=...)` (sim/bots.py:538-560: the
`astar_attack` policy of :267-508 in a `BotWrapper`, :511-535) for the
learner-vs-bot rollout: `act(obs, mmask, bmask, pid)` returns (N, 2) int64
actions like the reference bot, computed by one `qqt_bot_act` call that reads
the sim's device state directly.  `mode=True` attaches the approach / flee
mode ticker (`_mode_ticker`, :241-264): per env a mode and a countdown
drawn at construction (torch generator seeded by the bot's seed), advanced
by every call on the device (new draws from Philox stream 9); `mode=False`
(the default here, as in the learner-vs-bot benchmark) always approaches.
The crate-eating layer (`eat_crates=True`, the "hunter" bot) is not on this
path.

The noise uniforms come from Philox (stream 7, keyed by env and this bot's
call counter) unless `uniforms=(N, 5)` is passed.  The chain check reaches
out to the batch maximum of the bot's blast cap, as in the reference
(`int(cap.max().item())`, sim/bots.py:477), computed on the device without a
host round trip: from the per-row-block maxima the last STEP tick wrote
when a `Rollout` drives this bot and nothing changed the state since that
tick, else by a reduction launched by `qqt_bot_act`; `own_cap_reach=True`
uses each bot's own cap instead.
"""

from __future__ import annotations

import torch

from . import _capi
from .sim import HipBatchedSim


class HipAstarBot:
    is_bot = True

    def __init__(self, sim: HipBatchedSim, pid: int = 1, seed: int | None = None,
                 own_cap_reach: bool = False, mode: bool = False):
        if not 0 <= pid < sim.cfg.n_players:
            raise ValueError("pid out of range")
        self.sim, self.pid = sim, int(pid)
        self.seed = sim.seed if seed is None else int(seed)
        self.own_cap_reach = own_cap_reach
        self.tick = 0
        self._lib = _capi.lib()
        self._stream = _capi.stream_handle(sim.device)
        # two reach slots (the batch-max reduction alternates between them)
        self._reach = torch.full((2,), -2 ** 31, dtype=torch.int32, device=sim.device)
        # the per-env caps a Rollout's STEP ticks write (padding 0) and the
        # state version right after the last such tick
        self._caps = torch.zeros((-(-sim.num_envs // 16) * 16,), dtype=torch.int8, device=sim.device)
        self._tick_version = None
        self._calls = 0
        self._out = torch.zeros((sim.num_envs, sim.cfg.n_players, 2), dtype=torch.int64,
                                device=sim.device)
        b = _capi.BotArgsC()
        b.n_envs, b.pid = sim.num_envs, self.pid
        b.seed = self.seed & 0xFFFFFFFFFFFFFFFF
        b.cells, b.players = sim._cells.data_ptr(), sim._players.data_ptr()
        b.obs = sim._obs.data_ptr()
        b.move_mask, b.bomb_mask = sim._mm.data_ptr(), sim._bm.data_ptr()
        b.reach_mode = 0 if own_cap_reach else 1
        b.reach = self._reach.data_ptr()
        self.mode_count = 0
        if mode:
            # the ticker's initial draws (sim/bots.py:248-250): mode 0 / 1,
            # countdown 60 .. 239
            g = torch.Generator().manual_seed(self.seed)
            n = sim.num_envs
            self.modes = torch.randint(0, 2, (n,), generator=g, dtype=torch.int8).to(sim.device)
            self.mode_timers = torch.randint(60, 240, (n,), generator=g,
                                             dtype=torch.int32).to(sim.device)
            b.mode, b.mode_timer = self.modes.data_ptr(), self.mode_timers.data_ptr()
        else:
            self.modes = self.mode_timers = None
        self._args = b

    def _step_modes(self, b) -> None:
        """This call's ticker count (the reference steps its ticker on every
        act call, sim/bots.py:529-531)."""
        if self.modes is not None:
            self.mode_count += 1
            b.mode_tick = self.mode_count & 0xFFFFFFFF or 1

    def _set_reach(self, b) -> None:
        """The chain check's reach source for this call: the caps the last STEP
        tick wrote when the sim's state is still that tick's (mode 3), else a
        reduction of the batch (mode 1), or the own cap (mode 0)."""
        if self.own_cap_reach:
            b.reach_mode = 0
        elif self._tick_version is not None and self._tick_version == self.sim._state_version:
            b.reach_mode, b.reach_caps = 3, self._caps.data_ptr()
        else:
            b.reach_mode, b.reach, b.reach_slot = 1, self._reach.data_ptr(), self._calls & 1
            self._calls += 1

    def tick_writes_reach(self, tick_args) -> None:
        """Point a STEP tick's argument block at this bot's cap array, before
        the launch."""
        tick_args.reach_caps = 0 if self.own_cap_reach else self._caps.data_ptr()
        tick_args.reach_pid = self.pid

    def tick_wrote_reach(self) -> None:
        """Record that the STEP tick just launched wrote the caps (after the
        sim marked its state changed by that tick)."""
        if not self.own_cap_reach:
            self._tick_version = self.sim._state_version

    def launch(self, actions: torch.Tensor) -> None:
        """Write this bot's [move, place] into slot `pid` of an (N, P, 2)
        int8 or int64 device action buffer (observation and masks are the
        sim's current ones)."""
        n, p = self.sim.num_envs, self.sim.cfg.n_players
        if tuple(actions.shape) != (n, p, 2) or not actions.is_contiguous():
            raise ValueError("actions must be a contiguous (N, P, 2) tensor")
        self.sim._refresh()
        b = self._args
        b.tick = self.tick & 0xFFFFFFFF
        self._set_reach(b)
        self._step_modes(b)
        b.uniforms = None
        b.actions = actions.data_ptr() if actions.dtype == torch.int64 else None
        b.actions_i8 = actions.data_ptr() if actions.dtype == torch.int8 else None
        if b.actions is None and b.actions_i8 is None:
            raise ValueError("actions must be int8 or int64")
        _capi.check(self._lib.qqt_bot_act(self.sim._cfg_c, b, self._stream))
        self.tick += 1

    def act(self, obs, mmask, bmask, pid: int | None = None, uniforms=None):
        """(N, 2) int64 [move, place] (BotWrapper.act, sim/bots.py:511-545).
        `obs`/`mmask`/`bmask` are the observation and this player's masks;
        the sim's own buffers are used when they are the ones passed."""
        if pid is not None and int(pid) != self.pid:
            raise ValueError("this bot plays pid %d" % self.pid)
        sim, n, p = self.sim, self.sim.num_envs, self.sim.cfg.n_players
        sim._refresh()
        b = self._args
        obs_t = obs.to(sim.device, torch.float16).contiguous()
        if tuple(obs_t.shape) != tuple(sim._obs.shape):
            raise ValueError("observation shape differs from the sim's")
        mm = torch.zeros((n, p, 5), dtype=torch.uint8, device=sim.device)
        bm = torch.zeros((n, p, 2), dtype=torch.uint8, device=sim.device)
        mm[:, self.pid] = mmask.to(sim.device).to(torch.uint8)
        bm[:, self.pid] = bmask.to(sim.device).to(torch.uint8)
        u = None if uniforms is None else uniforms.to(sim.device, torch.float32).contiguous()
        b.obs, b.move_mask, b.bomb_mask = obs_t.data_ptr(), mm.data_ptr(), bm.data_ptr()
        b.tick = self.tick & 0xFFFFFFFF
        self._set_reach(b)
        self._step_modes(b)
        b.uniforms = _capi.ptr(u)
        b.actions, b.actions_i8 = self._out.data_ptr(), None
        try:
            _capi.check(self._lib.qqt_bot_act(sim._cfg_c, b, self._stream))
        finally:
            b.obs, b.move_mask, b.bomb_mask = sim._obs.data_ptr(), sim._mm.data_ptr(), \
                sim._bm.data_ptr()
        if uniforms is None:
            self.tick += 1
        return self._out[:, self.pid].clone()
