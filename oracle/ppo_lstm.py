"""CPU-side restatement of the reference's truncated-BPTT PPO update for the
lstm arch (test infrastructure only: imported by tests/).

Follows `_ppo_update_lstm` (train/ppo.py:440-537).  What the check of the
build's `ppo_update(LstmLearner, ...)` depends on is kept in the reference's
semantics; the code is organised around this module's own helpers:

* advantages: compute_gae (oracle.ppo.gae, train/ppo.py:101-110) normalised
  over the whole (T, N) buffer with the unbiased std + 1e-8 (ppo.py:451-452);
* minibatches: env-sliced, one device `torch.randperm(N)` per epoch and
  consecutive slices of max(1, N // minibatches) envs (ppo.py:460-465), so
  the random stream is consumed exactly as the reference consumes it;
* the sequence replay of a minibatch: the frame-independent trunk over all
  T x n frames at once, then the LSTM frame by frame with the hidden state
  detached every `bptt_window` frames and zeroed for the envs whose frame
  ended an episode (ppo.py:470-508); per frame, torch.distributions.
  Categorical on the masked logits (masked entries at the float minimum);
* losses: clipped policy surrogate, clipped value loss, entropy bonus
  (ppo.py:509-517); gradient clipping by global norm, one optimizer step
  per minibatch; statistics averaged over the minibatch updates.

The learner is any module with the reference lstm ActorCritic's members
(`extract_fused`, `lstm`, `move_head`, `bomb_head`, `critic`); the buffer
any object with the reference RolloutBuffer's (T, N, ...) tensors
(`rew`, `val`, `done`, `logp`, `act`, `mmask`, `bmask`, `local`, `rel`,
`glob`).  Pins (tests/test_oracle_ppo.py): the minibatch plan replays the
random stream as a hand-written randperm sequence; the losses reduce to
their closed forms at ratio 1; the state reset at a done frame equals a
replay restarted from a zero state; advantages are oracle.ppo.gae's.  The
composition as a whole has no reference-written vectors (train/ppo.py does
not import in this build's environment: sim/dev.py lacks `synchronize`), so
beyond those pins it is parity unpinned; tests/test_hip_lstm_learn.py checks
the build's update against it.
"""

from __future__ import annotations

import torch

from .ppo import gae

STAT_KEYS = ("pg", "vf", "ent", "kl", "clipfrac")


def advantages(buf, last_val, cfg):
    """(normalised advantages, returns) (T, N) on the buffer's device."""
    dev = buf.rew.device
    a, r = gae(buf.rew.cpu(), buf.val.cpu(), buf.done.cpu(), last_val.cpu(), cfg.gamma,
               cfg.gae_lambda)
    adv = torch.from_numpy(a).to(dev)
    ret = torch.from_numpy(r).to(dev)
    return (adv - adv.mean()) / (adv.std() + 1e-8), ret


def env_minibatches(n_envs, cfg, device):
    """Per epoch one randperm of the envs, cut into consecutive slices."""
    size = max(1, n_envs // cfg.minibatches)
    for _ in range(cfg.epochs):
        order = torch.randperm(n_envs, device=device)
        for start in range(0, n_envs, size):
            yield order[start:start + size]


def _frame_terms(learner, out, mmask, bmask, acts):
    """log-prob of the taken (move, bomb) pair, summed entropy and value of
    one frame from the LSTM output `out` (n, hidden)."""
    move_logits, bomb_logits = learner.move_head(out), learner.bomb_head(out)
    floor = torch.finfo(move_logits.dtype).min
    move = torch.distributions.Categorical(
        logits=torch.where(mmask, move_logits, torch.full_like(move_logits, floor)))
    bomb = torch.distributions.Categorical(
        logits=torch.where(bmask, bomb_logits, torch.full_like(bomb_logits, floor)))
    logp = move.log_prob(acts[:, 0]) + bomb.log_prob(acts[:, 1])
    return logp, move.entropy() + bomb.entropy(), learner.critic(out).squeeze(-1)


def replay_sequence(learner, buf, envs, window):
    """(logp, entropy, value) (T, n) of the selected envs, the LSTM run
    frame by frame from a zero state (truncated every `window` frames,
    reset where an episode ended)."""
    steps = buf.rew.shape[0]
    n = envs.numel()
    dev = buf.rew.device
    trunk = learner.extract_fused(buf.local[:, envs].reshape(steps * n, -1, 7, 7),
                                  buf.rel[:, envs].reshape(steps * n, -1, 6),
                                  buf.glob[:, envs].reshape(steps * n, -1)).view(steps, n, -1)
    logp = torch.empty((steps, n), device=dev)
    ent = torch.empty((steps, n), device=dev)
    value = torch.empty((steps, n), device=dev)
    state = None
    for t in range(steps):
        if window > 0 and t % window == 0 and state is not None:
            state = tuple(s.detach() for s in state)
        out, state = learner.lstm(trunk[t].unsqueeze(1), state)
        logp[t], ent[t], value[t] = _frame_terms(learner, out.squeeze(1), buf.mmask[t][envs],
                                                 buf.bmask[t][envs], buf.act[t][envs])
        ended = buf.done[t][envs]
        if bool(ended.any()):
            keep = 1 - ended.to(state[0].dtype).view(1, -1, 1)
            state = (state[0] * keep, state[1] * keep)
    return logp, ent, value


def clipped_losses(logp, ent, value, old_logp, old_val, adv, ret, cfg, entropy_coef):
    """(loss, statistics) of one minibatch."""
    ratio = (logp - old_logp).exp()
    surrogate = torch.min(ratio * adv, ratio.clamp(1 - cfg.clip_eps, 1 + cfg.clip_eps) * adv)
    pg = -surrogate.mean()
    v_clip = old_val + (value - old_val).clamp(-cfg.clip_eps, cfg.clip_eps)
    vf = 0.5 * torch.max((value - ret) ** 2, (v_clip - ret) ** 2).mean()
    loss = pg + cfg.value_coef * vf - entropy_coef * ent.mean()
    with torch.no_grad():
        stats = {"pg": float(pg), "vf": float(vf), "ent": float(ent.mean()),
                 "kl": float((old_logp - logp).mean()),
                 "clipfrac": float(((ratio - 1).abs() > cfg.clip_eps).float().mean())}
    return loss, stats


def lstm_update(learner, opt, buf, last_val, cfg, entropy_coef):
    """One update of the lstm learner (train/ppo.py:440-537); returns the
    statistics averaged over the minibatch steps."""
    adv, ret = advantages(buf, last_val, cfg)
    totals = dict.fromkeys(STAT_KEYS, 0.0)
    updates = 0
    window = getattr(cfg, "bptt_window", 0)
    for envs in env_minibatches(buf.rew.shape[1], cfg, buf.rew.device):
        logp, ent, value = replay_sequence(learner, buf, envs, window)
        loss, stats = clipped_losses(logp, ent, value, buf.logp[:, envs], buf.val[:, envs],
                                     adv[:, envs], ret[:, envs], cfg, entropy_coef)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(learner.parameters(), cfg.max_grad_norm)
        opt.step()
        for k in STAT_KEYS:
            totals[k] += stats[k]
        updates += 1
    return {k: v / max(1, updates) for k, v in totals.items()}
