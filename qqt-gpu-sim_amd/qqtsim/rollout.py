"""`Rollout`: one env-step of the self-play collect loop in two launches.

The reference's collect loop (train/ppo.py:213-249) does, per tick,
`observe()` -> `legal_mask()` -> `act(obs, mm, bm, pid=0)` -> `act(..., pid=1)`
-> `step(actions)` with auto-reset.  On the HIP path the observation and masks
of the current state are already in the sim's persistent buffers (the tick
kernel writes them after stepping and auto-resetting), so an env-step is

    qqt_mlp_act  (both players, masked sampling, int8 actions; qqt_cnn_act
                  for the cnn policy)
    qqt_tick     (step + auto-reset + observe + legal masks)

with both argument blocks built once: a tick only updates the Philox counter
words.  Rewards, done flags, log-probabilities and values land in persistent
device buffers (`reward`, `done`, `logp`, `value`, `actions`), which callers
that keep them across ticks copy.  Nothing here synchronises with the host
except the sim's first tick (it measures the reference's explosion tier
hint, see `HipBatchedSim`).
"""

from __future__ import annotations

import math

import torch

from . import _capi
from .policy import HipActorCritic
from .sim import HipBatchedSim


class Rollout:
    """Self-play (both players from `policy`) or learner vs `opponent`: the
    policy plays player 0 and an opponent with a `launch(actions)` method
    (`qqtsim.bots.HipAstarBot`) writes player 1's slot of the same int8
    action buffer before the tick."""

    def __init__(self, sim: HipBatchedSim, policy: HipActorCritic, opponent=None):
        p = sim.cfg.n_players
        if p != 2 or policy.n_players != 2:
            raise ValueError("the self-play rollout serves two players")
        if opponent is not None and (getattr(opponent, "pid", None) != 1
                                     or getattr(opponent, "sim", None) is not sim):
            raise ValueError("the opponent must play pid 1 on this sim")
        self.opponent = opponent
        if tuple(sim.cfg.obs_shape) != tuple(policy.obs_shape):
            raise ValueError("sim observation and policy input shapes differ")
        if sim.device != policy.device:
            raise ValueError("sim and policy live on different devices")
        self.sim, self.policy = sim, policy
        n, d = sim.num_envs, sim.device
        self.actions = torch.zeros((n, p, 2), dtype=torch.int8, device=d)
        self.logp = torch.zeros((n, p), dtype=torch.float32, device=d)
        self.value = torch.zeros((n, p), dtype=torch.float32, device=d)
        self._stream = _capi.stream_handle(d)
        self._lib = _capi.lib()

        m = policy._args(n, 2 if opponent is None else 1, 0, 1, sim._obs.data_ptr(),
                         math.prod(policy.obs_shape))
        m.out_slots, m.out_slot = 2, 0
        m.mm_row_stride, m.mm_pid_stride = 5 * p, 5
        m.bm_row_stride, m.bm_pid_stride = 2 * p, 2
        m.move_mask, m.bomb_mask = sim._mm.data_ptr(), sim._bm.data_ptr()
        m.actions_i8 = self.actions.data_ptr()
        m.logp_out, m.value_out = self.logp.data_ptr(), self.value.data_ptr()
        self._act = m

        t = _capi.TickArgsC()
        t.n_envs, t.mode, t.auto_reset = n, _capi.MODE_STEP, 1
        t.seed = sim.seed & 0xFFFFFFFFFFFFFFFF
        t.cells, t.players, t.envs = (sim._cells.data_ptr(), sim._players.data_ptr(),
                                      sim._envs.data_ptr())
        t.actions_i8 = self.actions.data_ptr()
        for k, buf in (("reward", sim._reward), ("done", sim._done), ("n_alive", sim._n_alive),
                       ("died", sim._died), ("winner", sim._winner), ("covered", sim._cov),
                       ("triggered", sim._trg), ("obs", sim._obs), ("move_mask", sim._mm),
                       ("bomb_mask", sim._bm)):
            setattr(t, k, buf.data_ptr())
        self._tick = t

        f = _capi.TickArgsC()
        f.n_envs, f.mode = n, _capi.MODE_FLUSH
        f.seed = sim.seed & 0xFFFFFFFFFFFFFFFF
        f.cells, f.players, f.envs = t.cells, t.players, t.envs
        f.recycle_excl = sim.recycle_excl().data_ptr()
        self._flush = f

    @property
    def reward(self) -> torch.Tensor:
        return self.sim._reward

    @property
    def done(self) -> torch.Tensor:
        return self.sim._done.view(torch.bool)

    def launch_policy(self) -> None:
        """The policy's actions (both players in self-play, player 0 against an
        opponent) for the current observation (train/model.py:230-245)."""
        self.sim._refresh()
        self._act.tick = self.policy.tick & 0xFFFFFFFF
        self.policy._launch(self._act, self._stream)
        self.policy.tick += 1

    def launch_opponent(self) -> None:
        """The opponent bot's actions (sim/bots.py:267-508), if there is one."""
        if self.opponent is not None:
            self.opponent.launch(self.actions)

    def launch_act(self) -> None:
        """Both players' actions for the current observation."""
        self.launch_policy()
        self.launch_opponent()

    def launch_tick(self, actions: torch.Tensor | None = None) -> None:
        """Step with the sampled actions (`self.actions`, or the int8 buffer
        the tick arguments point at), auto-reset, observe, masks
        (sim/torch_sim.py:895-1261, :605-645)."""
        sim = self.sim
        if sim.resolve_tiers is None:
            acts = self.actions if actions is None else actions
            sim.resolve_tiers = sim._first_tick_tiers(acts) \
                if sim.exact_reference_resolve else 255
        t = self._tick
        t.resolve_tiers = sim.resolve_tiers
        t.explore_coef = float(sim.explore_coef)
        t.danger_coef = float(sim.explore_coef * sim.cfg.danger_penalty)
        t.tick = sim.tick & 0xFFFFFFFF
        t.epoch = sim.epoch & 0xFFFFFFFF
        bot = self.opponent if hasattr(self.opponent, "tick_writes_reach") else None
        if bot is not None:          # the tick leaves the bot's reach for its next call
            bot.tick_writes_reach(t)
        _capi.check(self._lib.qqt_tick(sim._cfg_c, t, self._stream))
        sim.tick += 1
        sim.epoch += 1
        sim._fresh = True
        if bot is not None:
            bot.tick_wrote_reach()

    def step(self) -> None:
        """One env-step for every env."""
        self.launch_act()
        self.launch_tick()

    def run_into(self, buf: torch.Tensor) -> None:
        """T env-steps writing the observation each step acts on straight into
        `buf` (T, N, C, H, W) float16, the rollout buffer's observation
        slab (train/ppo.py:54-110): buf[0] is the current observation, the
        tick of step t writes buf[t + 1] (the last one lands in the sim's own
        buffer), and the policy of step t reads buf[t].  No copies besides
        buf[0]."""
        sim = self.sim
        n = sim.num_envs
        if buf.dtype != torch.float16 or not buf.is_contiguous() or buf.device != sim.device \
                or tuple(buf.shape[1:]) != (n,) + tuple(sim.cfg.obs_shape):
            raise ValueError("buf must be a contiguous (T, N, C, H, W) float16 device tensor")
        if (n * buf[0, 0].numel() * 2) % 16:
            raise ValueError("the number of envs must be a multiple of 4 (16-byte aligned slabs)")
        T = buf.shape[0]
        bot = self.opponent
        buf[0].copy_(sim.observe())
        try:
            for t in range(T):
                cur = buf[t].data_ptr()
                self._act.obs = cur
                if bot is not None:
                    bot._args.obs = cur
                self.launch_act()
                self._tick.obs = buf[t + 1].data_ptr() if t + 1 < T else sim._obs.data_ptr()
                self.launch_tick()
        finally:
            self._act.obs = sim._obs.data_ptr()
            self._tick.obs = sim._obs.data_ptr()
            if bot is not None:
                bot._args.obs = sim._obs.data_ptr()

    def collect(self, buf, flush_every: int = 16) -> None:
        """`buf.steps` env-steps filling a `qqtsim.ppo.HipRolloutBuffer` in
        place: the collect loop of train/ppo.py:213-276 with RolloutBuffer.add
        fused into the launches.  Step t's policy (and opponent) read slot
        t's observation and masks and write slot t's actions, log-probs and
        values; its tick writes slot t's rewards, done and damage flags and
        the next observation and masks into slot t + 1 (the sim's own
        buffers after the last step).  Slot 0 is copied from the sim.  Like
        the reference loop (train/ppo.py:263-264, :292) the recycle flush
        runs after every `flush_every`-th step and once after the last one
        (0 = never); a flush rewrites the next slot's observation and
        masks."""
        sim = self.sim
        n, p, T = sim.num_envs, sim.cfg.n_players, buf.steps
        if buf.arch == "lstm" or buf.num_envs != n or buf.n_players != p \
                or buf.device != sim.device or tuple(buf.obs.shape[2:]) != tuple(sim.cfg.obs_shape):
            raise ValueError("buffer shape or device differs from the sim's")
        if (n * buf.obs[0, 0].numel() * 2) % 16:
            raise ValueError("the number of envs must be a multiple of 4 (16-byte aligned slabs)")
        m, tk, bot = self._act, self._tick, self.opponent
        saved_m = (m.obs, m.move_mask, m.bomb_mask, m.actions_i8, m.logp_out, m.value_out)
        saved_t = (tk.actions_i8, tk.reward, tk.done, tk.damaged, tk.obs, tk.move_mask,
                   tk.bomb_mask)
        saved_b = None if bot is None else (bot._args.obs, bot._args.move_mask,
                                            bot._args.bomb_mask)
        sim._refresh()
        buf.obs[0].copy_(sim._obs.view(buf.obs[0].shape))
        buf._mm[0].copy_(sim._mm)
        buf._bm[0].copy_(sim._bm)
        try:
            for k in range(T):
                obs, mm, bm = buf.obs[k].data_ptr(), buf._mm[k].data_ptr(), buf._bm[k].data_ptr()
                m.obs, m.move_mask, m.bomb_mask = obs, mm, bm
                m.actions_i8, m.logp_out = buf._act[k].data_ptr(), buf._logp[k].data_ptr()
                m.value_out = buf._val[k].data_ptr()
                self.launch_policy()
                if bot is not None:
                    bot._args.obs, bot._args.move_mask, bot._args.bomb_mask = obs, mm, bm
                    bot.launch(buf._act[k])
                last = k + 1 == T
                tk.actions_i8 = buf._act[k].data_ptr()
                tk.reward, tk.done = buf._rew[k].data_ptr(), buf._done[k].data_ptr()
                tk.damaged = buf._dmg[k].data_ptr()
                tk.obs = (sim._obs if last else buf.obs[k + 1]).data_ptr()
                tk.move_mask = (sim._mm if last else buf._mm[k + 1]).data_ptr()
                tk.bomb_mask = (sim._bm if last else buf._bm[k + 1]).data_ptr()
                self.launch_tick(buf._act[k])
                if flush_every > 0 and k % flush_every == flush_every - 1 and not last:
                    self._launch_flush(tk.obs, tk.move_mask, tk.bomb_mask)
            if flush_every > 0:
                self._launch_flush(sim._obs.data_ptr(), sim._mm.data_ptr(), sim._bm.data_ptr())
        finally:
            (m.obs, m.move_mask, m.bomb_mask, m.actions_i8, m.logp_out, m.value_out) = saved_m
            (tk.actions_i8, tk.reward, tk.done, tk.damaged, tk.obs, tk.move_mask,
             tk.bomb_mask) = saved_t
            if bot is not None:
                bot._args.obs, bot._args.move_mask, bot._args.bomb_mask = saved_b
        buf.ptr = T
        # the sim's own outputs describe the last step, as after step()
        sim._reward.copy_(buf._rew[T - 1])
        sim._done.copy_(buf._done[T - 1])
        self.actions.copy_(buf._act[T - 1])
        self.logp.copy_(buf._logp[T - 1])
        self.value.copy_(buf._val[T - 1])

    def _launch_flush(self, obs: int, mm: int, bm: int) -> None:
        """The sim's recycle flush, writing observation and masks to the given
        device addresses (sim/torch_sim.py:549-596)."""
        sim = self.sim
        f = self._flush
        f.epoch = sim.flushes & 0xFFFFFFFF
        f.obs, f.move_mask, f.bomb_mask = obs, mm, bm
        _capi.check(self._lib.qqt_tick(sim._cfg_c, f, self._stream))
        sim.flushes += 1

    def run(self, ticks: int) -> None:
        for _ in range(int(ticks)):
            self.launch_act()
            self.launch_tick()


class TickLoop:
    """Ticks driven by injected actions (the bomb-stress workload): one
    `qqt_tick` launch per step with a prebuilt argument block; `actions` is
    any (N, P, 2) int8 device tensor (a slice of a pre-generated batch)."""

    def __init__(self, sim: HipBatchedSim):
        self.sim = sim
        self._stream = _capi.stream_handle(sim.device)
        self._lib = _capi.lib()
        t = _capi.TickArgsC()
        t.n_envs, t.mode, t.auto_reset = sim.num_envs, _capi.MODE_STEP, 1
        t.seed = sim.seed & 0xFFFFFFFFFFFFFFFF
        t.cells, t.players, t.envs = (sim._cells.data_ptr(), sim._players.data_ptr(),
                                      sim._envs.data_ptr())
        for k, buf in (("reward", sim._reward), ("done", sim._done), ("n_alive", sim._n_alive),
                       ("died", sim._died), ("winner", sim._winner), ("covered", sim._cov),
                       ("triggered", sim._trg), ("obs", sim._obs), ("move_mask", sim._mm),
                       ("bomb_mask", sim._bm)):
            setattr(t, k, buf.data_ptr())
        self._tick = t

    def launch_tick(self, actions: torch.Tensor) -> None:
        sim = self.sim
        if actions.dtype != torch.int8 or not actions.is_contiguous() or \
                tuple(actions.shape) != (sim.num_envs, sim.cfg.n_players, 2):
            raise ValueError("actions must be a contiguous (N, P, 2) int8 tensor")
        if sim.resolve_tiers is None:
            sim.resolve_tiers = sim._first_tick_tiers(actions) \
                if sim.exact_reference_resolve else 255
        t = self._tick
        t.actions_i8 = actions.data_ptr()
        t.resolve_tiers = sim.resolve_tiers
        t.explore_coef = float(sim.explore_coef)
        t.danger_coef = float(sim.explore_coef * sim.cfg.danger_penalty)
        t.tick = sim.tick & 0xFFFFFFFF
        t.epoch = sim.epoch & 0xFFFFFFFF
        _capi.check(self._lib.qqt_tick(sim._cfg_c, t, self._stream))
        sim.tick += 1
        sim.epoch += 1
        sim._fresh = True


class LstmRollout:
    """The collect loop of the lstm arch (train/ppo.py:204-276, lstm
    branch): player 0 acts from its own local features with the LSTM state
    carried across ticks, player 1 is an opponent with a `launch(actions)`
    method (`qqtsim.bots.HipAstarBot`).  One env-step is

        qqt_lstm_features  (player 0's local window, rel targets, scalars)
        qqt_lstm_act       (network, state update, masked sampling)
        qqt_bot_act        (player 1)
        qqt_tick           (step + auto-reset + observe + legal masks)

    The state `h`, `c` ((N, 128) float32) is updated in place by the act
    kernel, which zeroes the rows of envs whose episode ended at the previous
    tick before reading them: the reference's hidden * (1 - done) after each
    step (:261-264).  `reset_hidden()` is the reference's hidden = None."""

    def __init__(self, sim: HipBatchedSim, policy, opponent):
        if sim.cfg.n_players != 2:
            raise ValueError("the lstm rollout serves two players")
        if getattr(policy, "arch", None) != "lstm":
            raise ValueError("policy must be a HipLstmActorCritic")
        if getattr(opponent, "pid", None) != 1 or getattr(opponent, "sim", None) is not sim:
            raise ValueError("the opponent must play pid 1 on this sim")
        if sim.device != policy.device or sim.cfg.n_channels != policy.obs_shape[0]:
            raise ValueError("sim and policy differ in device or observation channels")
        self.sim, self.policy, self.opponent = sim, policy, opponent
        n, p, c, d = sim.num_envs, sim.cfg.n_players, sim.cfg.n_channels, sim.device
        self.actions = torch.zeros((n, p, 2), dtype=torch.int8, device=d)
        self.logp = torch.zeros((n, p), dtype=torch.float32, device=d)
        self.value = torch.zeros((n, p), dtype=torch.float32, device=d)
        self.h = torch.zeros((n, 128), dtype=torch.float32, device=d)
        self.c = torch.zeros((n, 128), dtype=torch.float32, device=d)
        self.local = torch.zeros((n, 1, c, 7, 7), dtype=torch.float16, device=d)
        self.rel = torch.zeros((n, 1, 10, 6), dtype=torch.float16, device=d)
        self.glob = torch.zeros((n, 1, 5), dtype=torch.float16, device=d)
        self._fresh_state = True      # h, c are zero: no reset flags to apply
        self._stream = _capi.stream_handle(d)
        self._lib = _capi.lib()

        f = _capi.LstmFeatArgsC()
        f.n_envs, f.p_out = n, 1
        f.cells, f.players, f.envs = (sim._cells.data_ptr(), sim._players.data_ptr(),
                                      sim._envs.data_ptr())
        f.obs = sim._obs.data_ptr()
        self._feat = f
        self._point_features(self.local, self.rel, self.glob)

        a = policy.args(self.local.view(n, -1), self.rel.view(n, -1), self.glob.view(n, -1),
                        self.h, self.c, rows_per_env=1, pid0=0)
        a.sample = 1
        a.move_mask, a.bomb_mask = sim._mm.data_ptr(), sim._bm.data_ptr()
        a.mm_row_stride, a.bm_row_stride = 5 * p, 2 * p
        a.out_stride, a.out_slot = p, 0
        a.actions_i8 = self.actions.data_ptr()
        a.logp_out, a.value_out = self.logp.data_ptr(), self.value.data_ptr()
        self._act = a

        t = _capi.TickArgsC()
        t.n_envs, t.mode, t.auto_reset = n, _capi.MODE_STEP, 1
        t.seed = sim.seed & 0xFFFFFFFFFFFFFFFF
        t.cells, t.players, t.envs = f.cells, f.players, f.envs
        t.actions_i8 = self.actions.data_ptr()
        for k, buf in (("reward", sim._reward), ("done", sim._done), ("n_alive", sim._n_alive),
                       ("died", sim._died), ("winner", sim._winner), ("covered", sim._cov),
                       ("triggered", sim._trg), ("obs", sim._obs), ("move_mask", sim._mm),
                       ("bomb_mask", sim._bm)):
            setattr(t, k, buf.data_ptr())
        self._tick = t

        fl = _capi.TickArgsC()
        fl.n_envs, fl.mode = n, _capi.MODE_FLUSH
        fl.seed = t.seed
        fl.cells, fl.players, fl.envs = t.cells, t.players, t.envs
        fl.recycle_excl = sim.recycle_excl().data_ptr()
        fl.obs, fl.move_mask, fl.bomb_mask = t.obs, sim._mm.data_ptr(), sim._bm.data_ptr()
        self._flush = fl

    def _point_features(self, local, rel, glob) -> None:
        f = self._feat
        f.local, f.rel, f.glob = local.data_ptr(), rel.data_ptr(), glob.data_ptr()
        f.local_stride, f.rel_stride, f.glob_stride = local.stride(0), rel.stride(0), glob.stride(0)

    @property
    def reward(self) -> torch.Tensor:
        return self.sim._reward

    @property
    def done(self) -> torch.Tensor:
        return self.sim._done.view(torch.bool)

    def reset_hidden(self) -> None:
        """Zero LSTM state for every env (the reference's hidden = None)."""
        self.h.zero_()
        self.c.zero_()
        self._fresh_state = True

    def launch_features(self) -> None:
        self.sim._refresh()
        _capi.check(self._lib.qqt_lstm_features(self.sim._cfg_c, self._feat, self._stream))

    def launch_policy(self, reset=None) -> None:
        """Player 0's actions from the features in the argument block; the
        state rows of envs flagged in `reset` (uint8 (N,) device tensor,
        default: the sim's done flags of the last tick) start from zero."""
        a = self._act
        if reset is None and not self._fresh_state:
            reset = self.sim._done
        a.reset = _capi.ptr(reset)
        a.tick = self.policy.tick & 0xFFFFFFFF
        self.policy.launch(a)
        self.policy.tick += 1
        self._fresh_state = False

    def launch_tick(self, actions: torch.Tensor | None = None) -> None:
        sim = self.sim
        if sim.resolve_tiers is None:
            acts = self.actions if actions is None else actions
            sim.resolve_tiers = sim._first_tick_tiers(acts) \
                if sim.exact_reference_resolve else 255
        t = self._tick
        t.resolve_tiers = sim.resolve_tiers
        t.explore_coef = float(sim.explore_coef)
        t.danger_coef = float(sim.explore_coef * sim.cfg.danger_penalty)
        t.tick = sim.tick & 0xFFFFFFFF
        t.epoch = sim.epoch & 0xFFFFFFFF
        bot = self.opponent if hasattr(self.opponent, "tick_writes_reach") else None
        if bot is not None:          # the tick leaves the bot's reach for its next call
            bot.tick_writes_reach(t)
        _capi.check(self._lib.qqt_tick(sim._cfg_c, t, self._stream))
        sim.tick += 1
        sim.epoch += 1
        sim._fresh = True
        if bot is not None:
            bot.tick_wrote_reach()

    def step(self) -> None:
        """One env-step for every env."""
        self.launch_features()
        self.launch_policy()
        self.opponent.launch(self.actions)
        self.launch_tick()

    def run(self, ticks: int) -> None:
        for _ in range(int(ticks)):
            self.step()

    def collect(self, buf, flush_every: int = 16) -> None:
        """`buf.steps` env-steps into a `HipRolloutBuffer(..., arch="lstm")`:
        the reference's collect (train/ppo.py:197-276) from hidden = None.
        Step t writes slot t's features, masks, actions, log-probabilities,
        values, rewards, done and damage flags (the tick writes the next
        masks straight into slot t + 1); the recycle flush runs after every
        `flush_every`-th step and once after the last (0 = never)."""
        sim = self.sim
        n, p, T = sim.num_envs, sim.cfg.n_players, buf.steps
        if getattr(buf, "arch", None) != "lstm" or buf.num_envs != n or buf.n_players != p \
                or buf.device != sim.device or buf.local.shape[2] != sim.cfg.n_channels:
            raise ValueError("buffer must be an lstm HipRolloutBuffer of this sim's shape")
        a, tk, bot = self._act, self._tick, self.opponent
        fl = self._flush
        saved_a = (a.local, a.rel, a.glob, a.move_mask, a.bomb_mask, a.actions_i8, a.logp_out,
                   a.value_out)
        saved_t = (tk.actions_i8, tk.reward, tk.done, tk.damaged, tk.move_mask, tk.bomb_mask)
        saved_b = (bot._args.move_mask, bot._args.bomb_mask)
        saved_f = (fl.move_mask, fl.bomb_mask)
        sim._refresh()
        buf._mm[0].copy_(sim._mm)
        buf._bm[0].copy_(sim._bm)
        self.reset_hidden()
        try:
            for k in range(T):
                loc, rel, glb = buf.local[k], buf.rel[k], buf.glob[k]
                self._point_features(loc, rel, glb)
                _capi.check(self._lib.qqt_lstm_features(sim._cfg_c, self._feat, self._stream))
                mm, bm = buf._mm[k].data_ptr(), buf._bm[k].data_ptr()
                a.local, a.rel, a.glob = loc.data_ptr(), rel.data_ptr(), glb.data_ptr()
                a.move_mask, a.bomb_mask = mm, bm
                a.actions_i8, a.logp_out = buf._act[k].data_ptr(), buf._logp[k].data_ptr()
                a.value_out = buf._val[k].data_ptr()
                self.launch_policy(None if k == 0 else buf._done[k - 1])
                bot._args.move_mask, bot._args.bomb_mask = mm, bm
                bot.launch(buf._act[k])
                last = k + 1 == T
                tk.actions_i8 = buf._act[k].data_ptr()
                tk.reward, tk.done = buf._rew[k].data_ptr(), buf._done[k].data_ptr()
                tk.damaged = buf._dmg[k].data_ptr()
                tk.move_mask = (sim._mm if last else buf._mm[k + 1]).data_ptr()
                tk.bomb_mask = (sim._bm if last else buf._bm[k + 1]).data_ptr()
                self.launch_tick(buf._act[k])
                if flush_every > 0 and k % flush_every == flush_every - 1 and not last:
                    fl.move_mask, fl.bomb_mask = tk.move_mask, tk.bomb_mask
                    self._launch_flush()
            if flush_every > 0:
                fl.move_mask, fl.bomb_mask = sim._mm.data_ptr(), sim._bm.data_ptr()
                self._launch_flush()
        finally:
            (a.local, a.rel, a.glob, a.move_mask, a.bomb_mask, a.actions_i8, a.logp_out,
             a.value_out) = saved_a
            (tk.actions_i8, tk.reward, tk.done, tk.damaged, tk.move_mask, tk.bomb_mask) = saved_t
            bot._args.move_mask, bot._args.bomb_mask = saved_b
            fl.move_mask, fl.bomb_mask = saved_f
            self._point_features(self.local, self.rel, self.glob)
        buf.ptr = T
        sim._reward.copy_(buf._rew[T - 1])
        sim._done.copy_(buf._done[T - 1])
        self.actions.copy_(buf._act[T - 1])
        self.logp.copy_(buf._logp[T - 1])
        self.value.copy_(buf._val[T - 1])

    def _launch_flush(self) -> None:
        sim = self.sim
        fl = self._flush
        fl.epoch = sim.flushes & 0xFFFFFFFF
        _capi.check(self._lib.qqt_tick(sim._cfg_c, fl, self._stream))
        sim.flushes += 1

    def last_value(self) -> torch.Tensor:
        """Player 0's value of the current state under the carried state,
        the state zeroed for envs done at the last tick (the reference's
        next_val, train/ppo.py:296-304); `h`, `c` are left as they are."""
        sim, n = self.sim, self.sim.num_envs
        loc, rel, glb = sim.local_view_features(only_p0=True)
        h, c = self.h.clone(), self.c.clone()
        a = self.policy.args(loc.view(n, -1), rel.view(n, -1), glb.view(n, -1), h, c)
        a.reset = None if self._fresh_state else sim._done.data_ptr()
        out = torch.empty((n,), dtype=torch.float32, device=sim.device)
        a.value_out = out.data_ptr()
        self.policy.launch(a)
        return out
