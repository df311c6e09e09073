"""The reference's rollout buffer and advantage estimation on the device.

`HipRolloutBuffer` mirrors `RolloutBuffer` (train/ppo.py:54-99): the same
attribute names, shapes and dtypes (`obs`, `mmask`, `bmask`, `act`, `logp`,
`val`, `rew`, `done`, `dmg`, `steps`, `ptr`, `add`, `reset`; for the lstm
arch also `local` (T,N,C,7,7), `rel` (T,N,10,6), `glob` (T,N,5), the
learner's per-player features, with `obs` an all-zero view that the lstm
path never fills, as in the reference).
Underneath, every per-step field is a slab in the layout the kernels write
(`[T][N][P]` for per-player values, int8 actions, uint8 flags), so
`Rollout.collect` fills a whole buffer with no per-step copies: the MLP
writes slot t's actions, log-probabilities and values, the tick writes slot
t's rewards, done and damage flags and slot t+1's observation and masks.
The reference's fields (player 0, the learner) are views of those slabs;
`act` and `done` convert to int64 / float32 when read.

`compute_gae` is the reference's compute_gae (train/ppo.py:101-110) as one
`qqt_gae` launch.
"""

from __future__ import annotations

import torch

from . import _capi


class HipRolloutBuffer:
    """Fixed-length buffer of T x N learner (player 0) transitions."""

    def __init__(self, steps: int, num_envs: int, obs_shape, device,
                 obs_dtype=torch.float16, arch: str = "mlp", n_players: int = 2) -> None:
        if arch not in ("mlp", "cnn", "lstm"):
            raise ValueError(f"unknown arch {arch!r}")
        if obs_dtype != torch.float16:
            raise ValueError("the device rollout keeps float16 observations")
        c, h, w = obs_shape
        t, n, p = int(steps), int(num_envs), int(n_players)
        if t <= 0 or n <= 0:
            raise ValueError("steps and num_envs must be positive")
        dev = torch.device(device)
        self.arch, self.steps, self.num_envs, self.n_players, self.ptr = arch, t, n, p, 0
        if arch == "lstm":
            self.obs = torch.zeros((), dtype=torch.float16, device=dev).expand(t, n, c, h, w)
            self.local = torch.zeros((t, n, c, 7, 7), dtype=torch.float16, device=dev)
            self.rel = torch.zeros((t, n, 10, 6), dtype=torch.float16, device=dev)
            self.glob = torch.zeros((t, n, 5), dtype=torch.float16, device=dev)
        else:
            self.obs = torch.zeros((t, n, c, h, w), dtype=torch.float16, device=dev)
        self._mm = torch.zeros((t, n, p, 5), dtype=torch.uint8, device=dev)
        self._bm = torch.zeros((t, n, p, 2), dtype=torch.uint8, device=dev)
        self._act = torch.zeros((t, n, p, 2), dtype=torch.int8, device=dev)
        self._logp = torch.zeros((t, n, p), dtype=torch.float32, device=dev)
        self._val = torch.zeros((t, n, p), dtype=torch.float32, device=dev)
        self._rew = torch.zeros((t, n, p), dtype=torch.float32, device=dev)
        self._done = torch.zeros((t, n), dtype=torch.uint8, device=dev)
        self._dmg = torch.zeros((t, n, p), dtype=torch.uint8, device=dev)

    # -- the reference's fields (player 0)
    @property
    def mmask(self) -> torch.Tensor:
        return self._mm[:, :, 0].view(torch.bool)

    @property
    def bmask(self) -> torch.Tensor:
        return self._bm[:, :, 0].view(torch.bool)

    @property
    def act(self) -> torch.Tensor:
        return self._act[:, :, 0].long()

    @property
    def logp(self) -> torch.Tensor:
        return self._logp[:, :, 0]

    @property
    def val(self) -> torch.Tensor:
        return self._val[:, :, 0]

    @property
    def rew(self) -> torch.Tensor:
        return self._rew[:, :, 0]

    @property
    def done(self) -> torch.Tensor:
        return self._done.float()

    @property
    def dmg(self) -> torch.Tensor:
        return self._dmg[:, :, 0].view(torch.bool)

    @property
    def device(self) -> torch.device:
        return self._rew.device

    def add(self, obs, mmask, bmask, act, logp, val, rew, done, dmg) -> None:
        """RolloutBuffer.add (train/ppo.py:84-95): one step of player-0 data
        from host or device tensors, copied into slot `ptr`; for the lstm arch
        `obs` is the feature triple (local, rel, glob)."""
        i = self.ptr
        if i >= self.steps:
            raise IndexError("rollout buffer is full")
        d = self.device
        if self.arch == "lstm":
            local, rel, glob = obs
            self.local[i], self.rel[i], self.glob[i] = local.to(d), rel.to(d), glob.to(d)
        else:
            self.obs[i] = obs.to(d)
        self._mm[i, :, 0] = mmask.to(d).to(torch.uint8)
        self._bm[i, :, 0] = bmask.to(d).to(torch.uint8)
        self._act[i, :, 0] = act.to(d).to(torch.int8)
        self._logp[i, :, 0] = logp.to(d)
        self._val[i, :, 0] = val.to(d)
        self._rew[i, :, 0] = rew.to(d)
        self._done[i] = done.to(d).to(torch.uint8)
        self._dmg[i, :, 0] = dmg.to(d).to(torch.uint8)
        self.ptr += 1

    def reset(self) -> None:
        self.ptr = 0


def compute_gae(buf: HipRolloutBuffer, last_val: torch.Tensor, gamma: float, lam: float):
    """(adv, ret) float32 (T, N): compute_gae (train/ppo.py:101-110) over the
    buffer's player-0 rewards and values, one `qqt_gae` launch on the current
    stream."""
    t, n, p = buf.steps, buf.num_envs, buf.n_players
    last_val = last_val.to(buf.device, torch.float32).contiguous()
    if tuple(last_val.shape) != (n,):
        raise ValueError("last_val must have shape (num_envs,)")
    adv = torch.empty((t, n), dtype=torch.float32, device=buf.device)
    ret = torch.empty_like(adv)
    a = _capi.GaeArgsC()
    a.steps, a.n_envs = t, n
    a.gamma, a.gamma_lam = float(gamma), float(gamma * lam)   # rounded to float32 by ctypes
    a.step_stride, a.env_stride = n * p, p
    a.rew, a.val = buf._rew.data_ptr(), buf._val.data_ptr()
    a.done, a.last_val = buf._done.data_ptr(), last_val.data_ptr()
    a.adv, a.ret = adv.data_ptr(), ret.data_ptr()
    _capi.check(_capi.lib().qqt_gae(a, _capi.stream_handle(buf.device)))
    return adv, ret
