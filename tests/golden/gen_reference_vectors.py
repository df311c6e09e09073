#!/usr/bin/env python3
"""Write golden input/output vectors by running the reference implementation.

Run in the build container, where the reference checkout sits at
/root/reference:

    python tests/golden/gen_reference_vectors.py

It imports the reference's `sim` and `train.model` packages (their Triton move
kernel is switched off, so `BatchedSim.step` takes the eager `move_players`,
which the reference keeps bit-identical to it) and writes `.npz` fixtures next
to this script.  Only vectors are written; no reference source is copied.

Fixtures (the functions they pin are the ones the JSON fixtures under the
reference's deploy/ leave open: multi-tick `BatchedSim.step` including
placement reward, hit-attribute penalty, combo, crate growth, auto-free chain
truncation at 8 rounds, and the MLP forward with its per-player column
permutation):

* traj_<name>.npz - a 64-env rollout of T ticks with `auto_reset=False`.
  The initial state comes from the oracle's template maps; actions and crate
  uniforms are injected and recorded; after every tick the full state,
  reward, done, info and the next tick's masks are stored, plus the
  observation of envs 0..3.
* deep_chain.npz - single-tick states with chains longer than 8 rounds.
* mlp.npz - MLP ActorCritic weights, inputs and forward/evaluate outputs.
* cnn.npz - the same for ActorCritic(arch="cnn") (conv trunk with the view
  permutation on conv0's input channels, per-sample LayerNorms).
* lstm.npz - the lstm arch's per-player features (sim/obs.py
  local_view_features) on bomb-rich states, and ActorCritic(arch="lstm") run
  over those frames as sequences (hidden state carried, zeroed on reset).
* astar_<name>.npz - the reference astar bot (sim/bots.py astar_attack, no
  behaviour modes, no crate eating) as player 1 against random legal moves
  for player 0: per tick the bot's inputs (state, observation, masks, the
  noise uniforms its torch.rand(n, 5) draws, seeded per tick), its output,
  and on every 4th tick its two cost fields (V_safe, V_opp).
* astar_flee.npz - the same with behaviour modes: a seeded approach / flee
  mode per env, from tick 32 on flipped every 4 ticks (so that bots that
  approached flee from close by), set as the sim's `_bmode` before each astar_attack call
  (the flee branch of sim/bots.py:433-443, 496-503) and recorded per tick
  with the bot's inputs and outputs.

Run a subset by name: `python tests/golden/gen_reference_vectors.py astar`.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"
sys.path.insert(0, os.path.join(REPO, "qqt-gpu-sim_amd"))
sys.path.insert(0, REPO)
sys.path.insert(0, REF)

import sim.torch_sim as ref_torch_sim  # noqa: E402
from sim.config import SimConfig as RefConfig  # noqa: E402
from train.model import ActorCritic  # noqa: E402

from oracle import philox  # noqa: E402
from oracle.policy import sample_masked  # noqa: E402
from oracle.sim import template_maps  # noqa: E402
from qqtsim.maps import MapSpec  # noqa: E402

ref_torch_sim._HAS_TRITON = False
ref_torch_sim._move_triton = None

CFG_KW = dict(map_mode="corridor", speed=3.0, tick_hz=10, max_steps=1800,
              open_fraction=0.0, n_players=2, obs_fp16=True)


def ref_sim(n, spec, seed, cfg_kw=None):
    cfg = RefConfig(**dict(CFG_KW, **(cfg_kw or {})))
    s = ref_torch_sim.BatchedSim(cfg, n, device="cpu", seed=seed)
    wall, brick, pos, bombs, blast, spd = template_maps(cfg, spec, np.arange(n), seed, 0)
    s.wall.copy_(torch.from_numpy(wall))
    s.brick.copy_(torch.from_numpy(brick))
    s.crate.zero_()
    s._recycle_crate.zero_()
    s.fuse.zero_()
    s.owner.fill_(-1)
    s.bomb_blast.zero_()
    s.pos.copy_(torch.from_numpy(pos))
    s.alive.fill_(True)
    s.hp.fill_(cfg.max_hp)
    s.since_bomb.fill_(cfg.place_dist_cooldown)
    s.t.zero_()
    s.bombs_cap = torch.from_numpy(bombs).clone()
    s.blast_cap = torch.from_numpy(blast).clone()
    s.spd_g = torch.from_numpy(spd).clone()
    s.invuln.zero_()
    s._combo.zero_()
    s._last_hit.fill_(-10 ** 9)
    s._pending_lost.zero_()
    s.crate_prob.fill_(cfg.growth_crate_prob)
    s._lo_bombs = torch.from_numpy(bombs).clone()
    s._lo_blast = torch.from_numpy(blast).clone()
    s._lo_spd = torch.from_numpy(spd).clone()
    s._map_kind.zero_()
    s._is_open.zero_()
    s._hazard.zero_()
    return s


def snapshot(s):
    return dict(
        wall=s.wall.numpy().copy(), brick=s.brick.numpy().copy(),
        crate=s.crate.numpy().copy(), recycle=s._recycle_crate.numpy().copy(),
        fuse=s.fuse.numpy().copy(), owner=s.owner.numpy().copy(),
        bomb_blast=s.bomb_blast.numpy().copy(), pos=s.pos.numpy().copy(),
        alive=s.alive.numpy().copy(), hp=s.hp.numpy().copy(),
        since_bomb=s.since_bomb.numpy().copy(), t=s.t.numpy().copy(),
        bombs_cap=s.bombs_cap.numpy().copy(), blast_cap=s.blast_cap.numpy().copy(),
        spd_g=s.spd_g.numpy().copy(), invuln=s.invuln.numpy().copy(),
        combo=s._combo.numpy().copy(), last_hit=s._last_hit.numpy().copy(),
        pending_lost=s._pending_lost.numpy().copy(),
    )


def actions_for(kind, mm, bm, n, seed, tick):
    p = mm.shape[1]
    if kind == "legal":
        u = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_RANDOM_ACT, 2 * p)
        out = np.zeros((n, p, 2), dtype=np.int64)
        for i in range(p):
            out[:, i, 0] = sample_masked(mm[:, i].astype(np.float32), mm[:, i], u[:, 2 * i])[0]
            out[:, i, 1] = sample_masked(bm[:, i].astype(np.float32), bm[:, i], u[:, 2 * i + 1])[0]
        return out
    u = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_INJECT_ACT, 2 * p)
    out = np.zeros((n, p, 2), dtype=np.int64)
    for i in range(p):
        out[:, i, 0] = np.minimum(np.floor(u[:, 2 * i] * np.float32(5)).astype(np.int64), 4)
        out[:, i, 1] = (u[:, 2 * i + 1] < np.float32(0.5)).astype(np.int64)
    return out


def rollout(name, spec, kind, n=64, ticks=128, seed=0, obs_envs=4, cfg_kw=None):
    s = ref_sim(n, spec, seed, cfg_kw)
    p = s.cfg.n_players
    rec = {k: [] for k in ("actions", "crate_u", "reward", "done", "n_alive", "covered",
                           "trig", "died", "winner", "mm", "bm", "obs", "danger")}
    states = []
    init = snapshot(s)
    mm, bm = (m.numpy().copy() for m in s.legal_mask())
    rec["mm"].append(mm)
    rec["bm"].append(bm)
    rec["obs"].append(s.observe()[:obs_envs].numpy().copy())
    for tick in range(ticks):
        a = actions_for(kind, mm, bm, n, seed, tick)
        cu = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_CRATE, 2 * p)
        cu = cu.reshape(n, p, 2).transpose(1, 2, 0).copy()          # (P, 2, N)
        s._rand_buf = torch.from_numpy(np.concatenate(
            [cu[:, 0, :].T.reshape(-1), cu[:, 1, :].T.reshape(-1)]))
        r, d, info = s.step(torch.from_numpy(a), auto_reset=False)
        rec["actions"].append(a)
        rec["crate_u"].append(cu)
        rec["reward"].append(r.numpy().copy())
        rec["done"].append(d.numpy().copy())
        rec["n_alive"].append(info["n_alive"].numpy().copy())
        rec["covered"].append(info["blast"].numpy().copy())
        rec["trig"].append(info["trig"].numpy().copy())
        rec["died"].append(info["died"].numpy().copy())
        rec["winner"].append(info["winner"].numpy().copy())
        rec["danger"].append(s._dng_cache.numpy().copy())
        states.append(snapshot(s))
        mm, bm = (m.numpy().copy() for m in s.legal_mask())
        rec["mm"].append(mm)
        rec["bm"].append(bm)
        rec["obs"].append(s.observe()[:obs_envs].numpy().copy())
    out = {f"init_{k}": v for k, v in init.items()}
    for k in states[0]:
        out[f"state_{k}"] = np.stack([st[k] for st in states])
    for k, v in rec.items():
        out[k] = np.stack(v)
    out["seed"] = np.int64(seed)
    out["resolve_hint"] = np.int64(s._res_cached.__defaults__[0])
    out["map_spec"] = np.array([spec.kind, str(spec.brick_p), str(int(spec.swap_spawns)),
                                str(spec.bombs_cap[0]), str(spec.bombs_cap[1]),
                                str(spec.blast_cap[0]), str(spec.blast_cap[1]),
                                str(spec.speed)])
    np.savez_compressed(os.path.join(HERE, f"traj_{name}.npz"), **out)
    placed = int((np.stack([st["fuse"] for st in states]) == 30).sum())
    print(f"{name}: ticks={ticks} placed~{placed} deaths={int(out['died'].sum())} "
          f"done_ticks={int(out['done'].sum())} resolve_hint={int(out['resolve_hint'])}")


def lstm(n=64, ticks=48, seed=23, every=4):
    """lstm.npz: the reference's per-player features for the lstm arch
    (sim/obs.py local_view_features, full P and only_p0) on states of a
    bomb-rich rollout, and the lstm ActorCritic (train/model.py, arch "lstm")
    run over those frames as a sequence with its hidden state carried."""
    from sim.obs import local_view_features

    spec = MapSpec(kind="pillars", brick_p=0.4, bombs_cap=(2, 4), blast_cap=(2, 5))
    s = ref_sim(n, spec, seed)
    p = s.cfg.n_players
    rec = {k: [] for k in ("obs", "pos", "alive", "t", "fuse", "hp", "local", "rel", "glob",
                           "local0", "rel0", "glob0", "mm", "bm")}
    mm, bm = (m.numpy().copy() for m in s.legal_mask())
    for tick in range(ticks):
        if tick % every == every - 1:
            obs = s.observe()
            args = (s.cfg, obs, s.pos, s.alive, s.t, s.fuse, s.hp)
            lf = local_view_features(*args, only_p0=False)
            l0 = local_view_features(*args, only_p0=True)
            for k, v in (("obs", obs), ("pos", s.pos), ("alive", s.alive), ("t", s.t),
                         ("fuse", s.fuse), ("hp", s.hp), ("local", lf[0]), ("rel", lf[1]),
                         ("glob", lf[2]), ("local0", l0[0]), ("rel0", l0[1]), ("glob0", l0[2])):
                rec[k].append(v.numpy().copy())
            rec["mm"].append(mm)
            rec["bm"].append(bm)
        a = actions_for("inject", mm, bm, n, seed, tick)
        cu = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_CRATE, 2 * p)
        cu = cu.reshape(n, p, 2).transpose(1, 2, 0).copy()
        s._rand_buf = torch.from_numpy(np.concatenate(
            [cu[:, 0, :].T.reshape(-1), cu[:, 1, :].T.reshape(-1)]))
        s.step(torch.from_numpy(a), auto_reset=False)
        mm, bm = (m.numpy().copy() for m in s.legal_mask())
    out = {k: np.stack(v) for k, v in rec.items()}

    torch.manual_seed(0)
    net = ActorCritic((14, 13, 13), arch="lstm", n_players=2)
    g = torch.Generator().manual_seed(2)
    with torch.no_grad():
        for name, prm in net.named_parameters():
            if "bias" in name:
                prm.add_(0.1 * torch.randn(prm.shape, generator=g))
    out.update({"w_" + k.replace(".", "_"): v.numpy().copy() for k, v in net.state_dict().items()})
    # player 0's frames as one sequence per env; hidden carried from zero,
    # zeroed for envs flagged in `reset` after a frame (as collect does on done)
    steps = out["local0"].shape[0]
    reset = np.zeros((steps, n), dtype=bool)
    reset[steps // 2, ::5] = True
    hidden = None
    acts = np.stack([actions_for("legal", out["mm"][i], out["bm"][i], n, seed, 1000 + i)[:, 0]
                     for i in range(steps)])
    res = {k: [] for k in ("move_logits", "bomb_logits", "value", "h", "c", "logp", "entropy")}
    with torch.no_grad():
        for i in range(steps):
            f = (torch.from_numpy(out["local0"][i][:, 0]), torch.from_numpy(out["rel0"][i][:, 0]),
                 torch.from_numpy(out["glob0"][i][:, 0]))
            lp, ent, _ = net.evaluate(f, torch.from_numpy(out["mm"][i][:, 0]),
                                      torch.from_numpy(out["bm"][i][:, 0]),
                                      torch.from_numpy(acts[i]), 0, hidden)
            ml, bl, v, hidden = net(f, 0, hidden)
            for k, x in (("move_logits", ml), ("bomb_logits", bl), ("value", v),
                         ("h", hidden[0][0]), ("c", hidden[1][0]), ("logp", lp), ("entropy", ent)):
                res[k].append(x.numpy().copy())
            if reset[i].any():
                dk = torch.from_numpy(reset[i]).float().view(1, -1, 1)
                hidden = (hidden[0] * (1 - dk), hidden[1] * (1 - dk))
    out.update({k: np.stack(v) for k, v in res.items()})
    out["actions"] = acts
    out["reset"] = reset
    out["param_count"] = np.int64(sum(q.numel() for q in net.parameters()))
    np.savez_compressed(os.path.join(HERE, "lstm.npz"), **out)
    print("lstm: frames", steps, "envs", n, "bombs/frame",
          float((out["fuse"] > 0).sum(axis=(1, 2, 3)).mean()), "params", int(out["param_count"]))


def deep_chain():
    """States whose chain needs more than 8 relay rounds."""
    cfg = RefConfig(**CFG_KW)
    n = 4
    s = ref_sim(n, MapSpec(kind="open"), 1)
    s.wall.zero_()
    s.brick.zero_()
    # env 0: 13 bombs in row 6, blast 1, leftmost due now
    for i in range(13):
        s.fuse[0, 6, i] = 1 if i == 0 else cfg.fuse
        s.owner[0, 6, i] = 0
        s.bomb_blast[0, 6, i] = 1
    # env 1: snake of blast-2 bombs alternating rows, mixed fuses
    cells = [(2, 1), (2, 3), (4, 3), (4, 5), (6, 5), (6, 7), (8, 7), (8, 9), (10, 9),
             (10, 11), (12, 11), (12, 9)]
    for k, (r, c) in enumerate(cells):
        s.fuse[1, r, c] = 1 if k == 0 else 5 + 2 * k
        s.owner[1, r, c] = k % 2
        s.bomb_blast[1, r, c] = 2
    # env 2: a column chain with a brick gap and a wall stop
    s.brick[2, 5, 4] = True
    s.wall[2, 9, 4] = True
    for r in range(0, 13):
        if r in (5, 9):
            continue
        s.fuse[2, r, 4] = 1 if r == 0 else 3 + r
        s.owner[2, r, 4] = r % 2
        s.bomb_blast[2, r, 4] = 3 if r % 3 == 0 else 1
    # env 3: a cross of bombs, blasts 2..7
    for k, (r, c) in enumerate([(6, 6), (6, 8), (6, 11), (3, 6), (1, 6), (9, 6), (12, 6),
                                (6, 3), (6, 1)]):
        s.fuse[3, r, c] = 1 if k == 0 else 20 - k
        s.owner[3, r, c] = k % 2
        s.bomb_blast[3, r, c] = 2 + (k % 6)
    s.pos[:, 0] = torch.tensor([6.5, 2.5])
    s.pos[:, 1] = torch.tensor([3.5, 10.5])
    init = snapshot(s)
    danger0 = ref_torch_sim.danger_map(
        s.fuse, s.wall, s._blast_map(), cfg.fuse, s.brick, cfg.max_chain,
        early_exit=False, blast_max_hint=7, chain_cap=cfg.chain_cap_rounds).numpy().copy()
    a = np.full((n, 2, 2), 0, dtype=np.int64)
    a[..., 0] = 4
    s._rand_buf = torch.zeros(2 * n * 2)
    r, d, info = s.step(torch.from_numpy(a), auto_reset=False)
    out = {f"init_{k}": v for k, v in init.items()}
    out.update({f"state_{k}": v for k, v in snapshot(s).items()})
    out.update(resolve_hint=np.int64(s._res_cached.__defaults__[0]))
    out.update(actions=a, reward=r.numpy(), covered=info["blast"].numpy(),
               trig=info["trig"].numpy(), danger_init=danger0,
               danger=s._dng_cache.numpy())
    np.savez_compressed(os.path.join(HERE, "deep_chain.npz"), **out)
    print("deep_chain: trig per env", info["trig"].flatten(1).sum(1).tolist())


def mlp(traj_name="pillars70", arch="mlp"):
    torch.manual_seed(0)
    net = ActorCritic((14, 13, 13), arch=arch, n_players=2)
    # Perturb biases and LayerNorm affine terms so every parameter matters.
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for name, prm in net.named_parameters():
            if name.endswith("bias") or ".1." in name or ".4." in name or (
                    arch == "cnn" and name.startswith("conv.")):
                prm.add_(0.1 * torch.randn(prm.shape, generator=g))
    z = np.load(os.path.join(HERE, f"traj_{traj_name}.npz"))
    obs = torch.from_numpy(z["obs"][::4].reshape(-1, 14, 13, 13)[:96].copy())
    b = obs.shape[0]
    mm = torch.from_numpy(z["mm"][::4, :4].reshape(-1, 2, 5)[:b].copy())
    bm = torch.from_numpy(z["bm"][::4, :4].reshape(-1, 2, 2)[:b].copy())
    acts = torch.from_numpy(z["actions"][::4, :4].reshape(-1, 2, 2)[:b].copy())
    out = {k: v.numpy().copy() for k, v in net.state_dict().items()}
    out = {"w_" + k.replace(".", "_"): v for k, v in out.items()}
    out["obs"] = obs.numpy()
    out["mm"] = mm.numpy()
    out["bm"] = bm.numpy()
    out["actions"] = acts.numpy()
    with torch.no_grad():
        for pid in range(2):
            ml, bl, v = net(obs, pid)
            lp, ent, v2 = net.evaluate(obs, mm[:, pid], bm[:, pid], acts[:, pid], pid)
            out[f"move_logits_{pid}"] = ml.numpy()
            out[f"bomb_logits_{pid}"] = bl.numpy()
            out[f"value_{pid}"] = v.numpy()
            out[f"logp_{pid}"] = lp.numpy()
            out[f"entropy_{pid}"] = ent.numpy()
    out["param_count"] = np.int64(sum(p.numel() for p in net.parameters()))
    np.savez_compressed(os.path.join(HERE, f"{arch}.npz"), **out)
    print(f"{arch}: batch", b, "params", int(out["param_count"]))


def astar(name, spec, n=64, ticks=64, seed=11):
    import sim.bots as ref_bots

    s = ref_sim(n, spec, seed)
    p = s.cfg.n_players
    keys = ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")
    rec = {k: [] for k in keys + ("obs", "mm1", "bm1", "u", "reach", "bot", "field_tick",
                                  "v_safe", "v_opp")}
    for tick in range(ticks):
        snap = snapshot(s)
        obs = s.observe()
        mm, bm = s.legal_mask()
        seed_t = seed * 100003 + tick
        torch.manual_seed(seed_t)
        u = torch.rand(n, 5)
        torch.manual_seed(seed_t)
        bot = ref_bots.astar_attack(s, obs, mm[:, 1], bm[:, 1], 1)
        for k in keys:
            rec[k].append(snap[k])
        rec["obs"].append(obs.numpy().copy())
        rec["mm1"].append(mm[:, 1].numpy().copy())
        rec["bm1"].append(bm[:, 1].numpy().copy())
        rec["u"].append(u.numpy().copy())
        rec["reach"].append(np.int64(s.blast_cap[:, 1].max()))
        rec["bot"].append(bot.numpy().copy())
        if tick % 4 == 0:
            danger = obs.float()[:, 2 * p + 1]
            block_all = s.wall | s.brick | (s.fuse > 0)
            rec["v_safe"].append(ref_bots._dijkstra_field(
                s, danger < 0.35, danger, blocked=block_all).numpy().copy())
            r0 = s.pos[:, 0, 0].floor().long().clamp(0, s.cfg.height - 1)
            c0 = s.pos[:, 0, 1].floor().long().clamp(0, s.cfg.width - 1)
            src = torch.zeros(n, s.cfg.height * s.cfg.width, dtype=torch.bool)
            src[torch.arange(n), r0 * s.cfg.width + c0] = s.alive[:, 0]
            rec["v_opp"].append(ref_bots._dijkstra_field(
                s, src.view(n, s.cfg.height, s.cfg.width), danger,
                blocked=block_all).numpy().copy())
            rec["field_tick"].append(np.int64(tick))
        a = actions_for("legal", mm.numpy(), bm.numpy(), n, seed, tick)
        a[:, 1] = bot.numpy()
        cu = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_CRATE, 2 * p)
        cu = cu.reshape(n, p, 2).transpose(1, 2, 0).copy()
        s._rand_buf = torch.from_numpy(np.concatenate(
            [cu[:, 0, :].T.reshape(-1), cu[:, 1, :].T.reshape(-1)]))
        s.step(torch.from_numpy(a), auto_reset=False)
    out = {k: np.stack(v) for k, v in rec.items()}
    np.savez_compressed(os.path.join(HERE, f"astar_{name}.npz"), **out)
    bots = out["bot"]
    print(f"astar_{name}: ticks={ticks} moves={np.bincount(bots[..., 0].ravel(), minlength=5)} "
          f"places={int(bots[..., 1].sum())} reach={sorted(set(out['reach'].tolist()))} "
          f"alive1={int(out['alive'][-1][:, 1].sum())}")


def astar_flee(spec, n=64, ticks=96, seed=29):
    import sim.bots as ref_bots

    s = ref_sim(n, spec, seed)
    g = torch.Generator().manual_seed(seed)
    mode = torch.randint(0, 2, (n,), generator=g)
    keys = ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")
    rec = {k: [] for k in keys + ("obs", "mm1", "bm1", "u", "bot", "mode")}
    for tick in range(ticks):
        if tick >= 32 and tick % 4 == 0:
            mode = 1 - mode
        snap = snapshot(s)
        obs = s.observe()
        mm, bm = s.legal_mask()
        seed_t = seed * 100003 + tick
        torch.manual_seed(seed_t)
        u = torch.rand(n, 5)
        torch.manual_seed(seed_t)
        s._bmode = mode
        bot = ref_bots.astar_attack(s, obs, mm[:, 1], bm[:, 1], 1)
        for k in keys:
            rec[k].append(snap[k])
        rec["obs"].append(obs.numpy().copy())
        rec["mm1"].append(mm[:, 1].numpy().copy())
        rec["bm1"].append(bm[:, 1].numpy().copy())
        rec["u"].append(u.numpy().copy())
        rec["bot"].append(bot.numpy().copy())
        rec["mode"].append(mode.numpy().astype(np.int8))
        a = actions_for("legal", mm.numpy(), bm.numpy(), n, seed, tick)
        a[:, 1] = bot.numpy()
        cu = philox.uniforms(seed, np.arange(n), tick, philox.STREAM_CRATE, 2 * s.cfg.n_players)
        cu = cu.reshape(n, s.cfg.n_players, 2).transpose(1, 2, 0).copy()
        s._rand_buf = torch.from_numpy(np.concatenate(
            [cu[:, 0, :].T.reshape(-1), cu[:, 1, :].T.reshape(-1)]))
        s.step(torch.from_numpy(a), auto_reset=False)
    out = {k: np.stack(v) for k, v in rec.items()}
    np.savez_compressed(os.path.join(HERE, "astar_flee.npz"), **out)
    bots, md = out["bot"], out["mode"]
    print(f"astar_flee: ticks={ticks} moves={np.bincount(bots[..., 0].ravel(), minlength=5)} "
          f"places approach={int(bots[..., 1][md == 0].sum())} flee={int(bots[..., 1][md == 1].sum())}")


def astar_chain(seed=19):
    """Hand-built states where the bot's chain check matters: the bot stands
    in the open with a short-fuse bomb k cells away in a straight line; env 0's
    bot has blast cap 5 (the batch max), the others cap 2, so bombs 3..5 cells
    out are in reach only through the batch-max loop bound."""
    import sim.bots as ref_bots

    n = 16
    s = ref_sim(n, MapSpec(kind="open"), seed)
    s.pos[:, 1, 0] = 6.5
    s.pos[:, 1, 1] = 6.5
    s.pos[:, 0, 0] = 1.5            # opponent far away, not aligned
    s.pos[:, 0, 1] = 11.5
    s.blast_cap[:, 1] = 2
    s.blast_cap[0, 1] = 5
    for e in range(n):
        k = 1 + e % 5                # bomb distance 1..5
        d = (e // 5) % 4            # direction
        dr, dc = ((-1, 0), (1, 0), (0, -1), (0, 1))[d]
        s.fuse[e, 6 + dr * k, 6 + dc * k] = 3 + (e % 9)      # fuse 3..11
        s.owner[e, 6 + dr * k, 6 + dc * k] = 0
        s.bomb_blast[e, 6 + dr * k, 6 + dc * k] = 2
    obs = s.observe()
    mm, bm = s.legal_mask()
    torch.manual_seed(seed)
    u = torch.rand(n, 5)
    torch.manual_seed(seed)
    bot = ref_bots.astar_attack(s, obs, mm[:, 1], bm[:, 1], 1)
    snap = snapshot(s)
    out = {k: snap[k][None] for k in ("wall", "brick", "fuse", "owner", "pos", "alive",
                                       "blast_cap")}
    out.update(obs=obs.numpy()[None], mm1=mm[:, 1].numpy()[None], bm1=bm[:, 1].numpy()[None],
               u=u.numpy()[None], reach=np.array([int(s.blast_cap[:, 1].max())]),
               bot=bot.numpy()[None])
    np.savez_compressed(os.path.join(HERE, "astar_chain.npz"), **out)
    print("astar_chain: places", bot[:, 1].tolist())


if __name__ == "__main__" and len(sys.argv) > 1:
    for what in sys.argv[1:]:
        if what == "astar":
            astar("p70", MapSpec(kind="pillars", brick_p=0.7))
            astar("p30", MapSpec(kind="pillars", brick_p=0.3, bombs_cap=(2, 4), blast_cap=(2, 5)),
                  seed=13)
            astar("open", MapSpec(kind="open", bombs_cap=(2, 3), blast_cap=(2, 4)), ticks=96,
                  seed=17)
            astar_chain()
        elif what == "astar_flee":
            astar_flee(MapSpec(kind="open", bombs_cap=(2, 3), blast_cap=(2, 4)))
        elif what == "cnn":
            mlp(arch="cnn")
        elif what == "lstm":
            lstm()
        else:
            raise SystemExit(f"unknown fixture group {what!r}")
elif __name__ == "__main__":
    rollout("pillars0", MapSpec(kind="pillars", brick_p=0.0), "legal", ticks=128, seed=0)
    rollout("pillars70", MapSpec(kind="pillars", brick_p=0.7), "legal", ticks=128, seed=3)
    rollout("stress40", MapSpec(kind="pillars", brick_p=0.4, bombs_cap=(1, 4),
                                blast_cap=(2, 5)), "inject", ticks=128, seed=5)
    rollout("deathmatch", MapSpec(kind="pillars", brick_p=0.3, bombs_cap=(2, 4),
                                  blast_cap=(2, 3)), "inject", ticks=96, seed=7,
            cfg_kw=dict(max_hp=2, invuln_ticks=4, max_steps=70))
    deep_chain()
    mlp()
    mlp(arch="cnn")
    astar("p70", MapSpec(kind="pillars", brick_p=0.7))
    astar("p30", MapSpec(kind="pillars", brick_p=0.3, bombs_cap=(2, 4), blast_cap=(2, 5)),
          seed=13)
    astar("open", MapSpec(kind="open", bombs_cap=(2, 3), blast_cap=(2, 4)), ticks=96, seed=17)
    astar_chain()
    astar_flee(MapSpec(kind="open", bombs_cap=(2, 3), blast_cap=(2, 4)))
    lstm()
