#!/usr/bin/env python3
"""Self-play rollout throughput on one MI355X: env-steps/s at 5632 envs.

One step = one env-step of the collect loop for every env (train/ppo.py:213-249):
both players' MLP actor/critic forward with masked factored sampling, then
the tick (movement, bombs, chain explosion, danger map, rewards, auto-reset,
14-channel float16 observation, legality masks).  On this path that is two
kernel launches per step, `mlp_act_kernel` and `tick_kernel`, on torch's
current stream.

Workload: 5632 envs, 13x13 map with border walls, pillars at even/even
cells and a brick on every other free cell outside the spawn L with p 0.7,
two players spawning in opposite corners (random side swap), training corridor
rules (0.3 cell/tick, 1800-tick episodes), MLP 2366->128->LN->ReLU->128->LN->
ReLU->heads with PyTorch default init (manual_seed 0), auto-reset on done.
Maps and weights are synthetic; everything is resident in HBM before timing.

Prints ONE JSON line (rank 0).  `roofline` prices the dominant kernel against
its bound: the tick kernel against HBM (algorithmic bytes per env-step below),
the MLP kernel against dense float16 MFMA (algorithmic FLOP per env-step).
Kernel durations come from HIP event pairs that the library records on the
dispatch packets of both launches of every 8th step inside the timed region
(hipExtLaunchKernel on the launch stream), i.e. kernel begin to kernel end.  `traffic` is read from the committed
rocprofv3 FETCH_SIZE/WRITE_SIZE summary when one exists.  `cpu_baseline`
times the oracle (the CPU restatement of the reference path) on the host
cores over a bounded sample of the same workload.  `torch_gpu_bound` bounds
the reference's own PyTorch-on-GPU step from above: its launch count per tick
times the eager launch cost measured on this GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qqt-gpu-sim_amd"))

METRIC = "env-steps/s at 5632 envs (step+obs+MLP act), 1 MI355X; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

# Algorithmic bytes of one env-step of the tick kernel: packed state read +
# write (169 cells x 4 B + 2 players x 48 B + 16 B, twice), the float16
# observation (14 x 169 x 2 B), actions (4 B), masks (14 B), reward (8 B),
# done (1 B).
TICK_BYTES_PER_ENV = 2 * (169 * 4 + 2 * 48 + 16) + 14 * 169 * 2 + 4 + 14 + 8 + 1
# Algorithmic bytes of one env-step of the MLP kernel: observation read once
# for both players, masks, int8 actions, logp and value.
MLP_BYTES_PER_ENV = 14 * 169 * 2 + 14 + 4 + 16
# Algorithmic FLOP of one env-step of the MLP: two players x 2 x MACs of
# 2366x128 + 128x128 + 3 x 128x64 + 64x(5+2+1).
MLP_FLOP_PER_ENV = 2 * 2 * (2366 * 128 + 128 * 128 + 3 * 128 * 64 + 64 * 8)

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_rollout_5632.json")
STRESS_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_bomb_stress_16384.json")
EVAL_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_eval_forward_4M.json")
EVERY = 8   # kernel durations are sampled on every 8th timed step


def sampled(k, steps):
    """Whether timed step k of `steps` carries the kernel-duration events:
    every EVERY-th step from step EVERY // 2 (the last step when there are
    fewer).  Step 0 is left out: event pairs on the first launches after
    the synchronised, idle queue cost about 50 us of wall time (2.5 us per
    step over 20 timed steps on MI355X), on later steps nothing measurable."""
    return k % EVERY == min(EVERY // 2, steps - 1)

from qqtsim import _capi  # noqa: E402  (C ABI loader; loads the library lazily)


def kernel_ms():
    """{kernel: mean ms per timed dispatch} of the launches armed since the
    last call (each timed by an event pair on its own dispatch packet)."""
    return {k: ms / c for k, (ms, c) in _capi.timing_collect().items()}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--envs", type=int, default=5632)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU work budget of the cpu_baseline sample (0 = skip)")
    ap.add_argument("--workload", choices=("rollout", "stress", "astar", "evalfwd", "collect",
                                           "ppo", "train", "cnn", "lstm"),
                    default="rollout",
                    help="rollout: the headline self-play rollout (default); stress: "
                         "16384-env bomb-stress ticks with injected actions; astar: "
                         "learner (MLP) vs the astar bot, 5632 envs; evalfwd: 32768-env x "
                         "128-tick rollout into the observation slab, then the batched "
                         "evaluation forward over all 4.19M observations; collect: "
                         "128-step self-play collects into the device rollout buffer "
                         "(5632 envs) + last-value forward + GAE; ppo: one PPO update "
                         "(4 epochs x 4 minibatches) over a 5632 x 128 collected buffer; "
                         "train: whole training iterations (collect 128 steps + PPO update "
                         "+ weight sync to the acting network); cnn: the self-play rollout "
                         "with the reference's cnn actor/critic, 5632 envs; lstm: the lstm "
                         "learner (local features + LSTM) vs the astar bot, 5632 envs")
    ap.add_argument("--copy-calibrate", action="store_true",
                    help="after timing, run a 512 MiB device copy (HBM counter calibration)")
    ap.add_argument("--no-torch-baseline", action="store_true",
                    help="ppo: skip the eager-torch update on the GPU (kernel traces of the "
                         "library's update alone)")
    return ap.parse_args()


def build_workload(n, seed, device):
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.policy import HipActorCritic, default_init
    from qqtsim.rollout import Rollout
    from qqtsim.sim import HipBatchedSim

    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    sim = HipBatchedSim(cfg, n, device=device, seed=seed, map_spec=spec)
    net = HipActorCritic(default_init(cfg.obs_shape), device=device, seed=seed)
    return cfg, spec, Rollout(sim, net)


STRESS_ENVS = 16384


def stress_actions(n, steps, seed, device):
    """(steps, N, 2, 2) int8 injected actions: move ~ U{0..4} (unmasked), bomb ~
    Bernoulli(0.5), generated on the device before timing."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    mv = torch.randint(0, 5, (steps, n, 2), generator=g, device=device, dtype=torch.int8)
    bb = (torch.rand((steps, n, 2), generator=g, device=device) < 0.5).to(torch.int8)
    return torch.stack([mv, bb], dim=-1).contiguous()


def cpu_baseline_stress(cfg, spec, n, seed, budget_s):
    """The oracle's tick on the host cores with the same injected-action rule."""
    import torch

    from oracle.sim import OracleSim

    cores = _cores(torch)
    sim = OracleSim(cfg, n, spec, seed=seed)
    g = torch.Generator().manual_seed(seed)

    def tick():
        mv = torch.randint(0, 5, (n, 2), generator=g)
        bb = (torch.rand((n, 2), generator=g) < 0.5).long()
        sim.step(torch.stack([mv, bb], -1), auto_reset=True)

    tick()
    ticks, t0 = 0, time.perf_counter()
    while True:
        tick()
        ticks += 1
        el = time.perf_counter() - t0
        if el >= budget_s or ticks >= 256:
            break
    return {"value": n * ticks / el, "unit": "env-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle (torch CPU restatement) tick with injected actions, {n} envs x "
                      f"{ticks} timed ticks after 1 warm-up tick, {el:.1f} s"}


def _cpu_model():
    """lscpu's model name with its family / model / stepping ids and the
    logical CPU count of the host (the name alone can be generic in a VM)."""
    info = {}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if not info.get("Model name"):
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    info["Model name"] = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    name = info.get("Model name", "unknown")
    ids = ", ".join(f"{k.lower()} {info[k]}" for k in ("CPU family", "Model", "Stepping")
                    if info.get(k))
    cpus = info.get("CPU(s)")
    return f"{name} ({ids}; {cpus} logical CPUs on the host)" if ids or cpus else name


def _cores(torch):
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(max(1, cores))
    return torch.get_num_threads()


def cpu_baseline(cfg, spec, n, seed, budget_s, arch="mlp"):
    """The oracle's env-step on the host cores: observe, legal_mask, both
    players' forward (mlp or cnn network) + masked sampling, step with
    auto-reset."""
    import numpy as np
    import torch

    from oracle import philox
    from oracle.policy import cnn_forward, mlp_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim.policy import default_init, default_init_cnn

    cores = _cores(torch)
    if arch == "cnn":
        params, forward = default_init_cnn(cfg.obs_shape), cnn_forward
    else:
        params, forward = default_init(cfg.obs_shape), mlp_forward
    sim = OracleSim(cfg, n, spec, seed=seed)
    envs = np.arange(n)

    def env_step(t):
        obs = sim.observe()
        mm, bm = sim.legal_mask()
        u = philox.uniforms(seed, envs, t, philox.STREAM_POLICY, 4)
        acts = torch.zeros((n, 2, 2), dtype=torch.int64)
        for pid in range(2):
            ml, bl, _ = forward(params, obs, pid)
            acts[:, pid, 0] = torch.from_numpy(
                sample_masked(ml.numpy(), mm[:, pid].numpy(), u[:, 2 * pid])[0])
            acts[:, pid, 1] = torch.from_numpy(
                sample_masked(bl.numpy(), bm[:, pid].numpy(), u[:, 2 * pid + 1])[0])
        sim.step(acts, auto_reset=True)

    for t in range(2):
        env_step(t)
    ticks, t0 = 0, time.perf_counter()
    while True:
        env_step(2 + ticks)
        ticks += 1
        el = time.perf_counter() - t0
        if el >= budget_s or ticks >= 256:
            break
    # the same env-step on one thread, over a quarter of the budget
    torch.set_num_threads(1)
    ticks1, t1 = 0, time.perf_counter()
    while True:
        env_step(2 + ticks + ticks1)
        ticks1 += 1
        el1 = time.perf_counter() - t1
        if el1 >= budget_s / 4 or ticks1 >= 64:
            break
    torch.set_num_threads(cores)
    return {"value": n * ticks / el, "unit": "env-steps/s", "cores": cores,
            "kind": "port", "cpu_model": _cpu_model(),
            "value_1thread": n * ticks1 / el1,
            "sample": f"oracle (torch CPU restatement, {arch} network) on the same workload, "
                      f"{n} envs x {ticks} timed ticks after 2 warm-up ticks, {el:.1f} s; one thread: "
                      f"{ticks1} ticks, {el1:.1f} s"}


def read_traffic(kernel, path=TRAFFIC_FILE):
    """HBM bytes per dispatch of `kernel` (FETCH + WRITE, copy-calibrated) from
    a committed rocprofv3 traffic summary, or None."""
    try:
        with open(path) as f:
            d = json.load(f)
        k = d["kernels"][kernel]
        return int(round(k["fetch_bytes"] + k["write_bytes"]))
    except (OSError, KeyError, ValueError, TypeError):
        return None


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        sys.exit("bench.py measures one GPU: the rollout has no cross-GPU step and this "
                 "build runs on a single MI355X (envs shard by index across GPUs with "
                 "replicated weights; see the sharding notes). Run with --gpus 1.")
    import torch

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a ROCm GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "stress":
        return main_stress(args, torch, dev)
    if args.workload == "astar":
        return main_astar(args, torch, dev)
    if args.workload == "evalfwd":
        return main_evalfwd(args, torch, dev)
    if args.workload == "collect":
        return main_collect(args, torch, dev)
    if args.workload == "ppo":
        return main_ppo(args, torch, dev)
    if args.workload == "train":
        return main_train(args, torch, dev)
    if args.workload == "lstm":
        return main_lstm(args, torch, dev)
    if args.workload == "cnn":
        return main_cnn(args, torch, dev)
    n, K, W = args.envs, args.steps, args.warmup
    cfg, spec, roll = build_workload(n, args.seed, dev)
    # The timed window must see the whole tick: bombs placed from the first
    # tick explode at tick cfg.fuse, so at least cfg.fuse + 2 untimed ticks
    # run before the warm-up, whatever --warmup is.
    preroll = cfg.fuse + 2
    for _ in range(preroll + W):
        roll.step()
    stats = torch.zeros((n, 4), dtype=torch.int32, device=dev)
    roll._tick.tick_stats = stats.data_ptr()   # the tick counts what the timed steps did
    torch.cuda.synchronize()

    # Both launches of every EVERY-th timed step (`sampled`) carry a HIP event pair on
    # their own dispatch packet (the stream they run on); sampling keeps the
    # cost out of `value`.
    _capi.timing_arm(0)          # creates the event pool outside the timed region
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        if sampled(k, K):
            _capi.timing_arm(2)
        roll.launch_act()
        roll.launch_tick()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    roll._tick.tick_stats = 0
    kms = kernel_ms()
    act_ms, tick_ms = kms["mlp_act_kernel"], kms["tick_kernel"]
    done_frac = float(roll.done.float().mean())
    window = timed_window(stats, preroll + W, K, n)

    if args.copy_calibrate:
        _calibration_copy(torch, dev)

    kernels = {
        "tick_kernel": {"us": tick_ms * 1e3, "bound": "hbm",
                        "achieved": TICK_BYTES_PER_ENV * n / (tick_ms * 1e-3) / 1e9,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "bytes_per_env": TICK_BYTES_PER_ENV},
        "mlp_act_kernel": {"us": act_ms * 1e3, "bound": "mfma",
                           "achieved": MLP_FLOP_PER_ENV * n / (act_ms * 1e-3) / 1e12,
                           "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "flop_per_env": MLP_FLOP_PER_ENV,
                           "hbm_gbs": MLP_BYTES_PER_ENV * n / (act_ms * 1e-3) / 1e9},
    }
    for v in kernels.values():
        v["frac"] = v["achieved"] / v["peak"]
    dom = max(kernels, key=lambda k: kernels[k]["us"])
    d = kernels[dom]
    roofline = {"kernel": dom, "bound": d["bound"], "achieved": round(d["achieved"], 3),
                "peak": d["peak"], "unit": d["unit"], "frac": round(d["frac"], 5),
                "traffic": read_traffic(dom)}

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(cfg, spec, n, args.seed, args.cpu_seconds)
    value = n * K / el
    tgb = torch_gpu_bound(torch, dev, n, value)

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": el / K * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 sim / f16 MFMA (f32 accumulate)",
        "data": "synthetic: template maps from Philox draws, PyTorch default-init MLP weights",
        "config": {"workload": "self-play rollout, 5632 envs, 13x13 pillars + 70% bricks, "
                               "P=2, 14-ch f16 obs, MLP act both players + masked sampling, "
                               "auto-reset",
                   "envs": n, "grid": [cfg.height, cfg.width], "players": cfg.n_players,
                   "brick_p": spec.brick_p, "step_len": cfg.step_len,
                   "max_steps": cfg.max_steps, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "torch_gpu_bound": tgb,
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in kernels.items()},
        "done_fraction_last_tick": done_frac,
        "timed_window": window,
    }
    print(json.dumps(out), flush=True)


def timed_window(stats, untimed, steps, n):
    """What the timed ticks did, from the tick kernel's own per-env counters
    (summed over envs after timing): bombs exploded, players died and envs
    auto-reset over the timed steps."""
    ex, dead, resets = (int(v) for v in stats[:, :3].long().sum(0).tolist())
    return {"ticks_before_timing": untimed, "timed_ticks": steps, "exploded_bombs": ex,
            "deaths": dead, "auto_resets": resets,
            "exploded_bombs_per_env_tick": round(ex / (n * steps), 5)}


# Kernel launches of one eager BatchedSim.step of the reference on a GPU, as
# its authors counted them (HANDOFF_20260810.md:209, n = 20000; observe,
# legal_mask and both act() calls come on top and are left out here).
REF_LAUNCHES_PER_TICK = 5145


def torch_gpu_bound(torch, dev, n, value, reps=4):
    """Upper bound on the reference PyTorch-on-GPU path at n envs: its step
    issues REF_LAUNCHES_PER_TICK eager kernel launches, so one tick takes at
    least that many times the cost of one eager elementwise op on (n,13,13)
    tensors, measured here on the same GPU and host.  The reference itself
    does not run here; this is a floor on its tick time (an upper bound on
    its env-steps/s), so value / bound is a lower bound on the speedup."""
    f = torch.rand((n, 13, 13), device=dev)
    g = torch.rand((n, 13, 13), device=dev)
    m = f > 0.5
    b = torch.zeros_like(m)

    def cycle():                      # eight ops, one kernel launch each
        nonlocal f, m, b
        f = f * 0.9
        m = f > 0.3
        f = torch.where(m, f, g)
        b = b | m
        f = f + g
        f = f.clamp(0.0, 4.0)
        f = torch.maximum(f, g)
        f = f * 0.5
    for _ in range(64):
        cycle()
    torch.cuda.synchronize()
    ops = 8 * (REF_LAUNCHES_PER_TICK // 8)
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(ops // 8):
            cycle()
        torch.cuda.synchronize()
        best = min(best, (time.perf_counter() - t0) / ops)
    upper = n / (REF_LAUNCHES_PER_TICK * best)
    return {"us_per_eager_launch": round(best * 1e6, 3),
            "ref_launches_per_tick": REF_LAUNCHES_PER_TICK,
            "ref_env_steps_per_s_upper": round(upper, 1),
            "speedup_lower": round(value / upper, 1),
            "note": "floor of the reference eager step on this GPU: launch count x measured "
                    "eager launch cost (observe/legal_mask/act launches not counted)"}


def _calibration_copy(torch, dev):
    src = torch.empty(256 << 20, dtype=torch.int16, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def main_stress(args, torch, dev):
    """Bomb-stress ticks: 16384 envs, corridor map with 40% bricks, per-player
    bombs 1-4 and blast 2-5, injected unmasked actions (bomb w.p. 0.5)."""
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import BOMB_STRESS_40
    from qqtsim.rollout import TickLoop
    from qqtsim.sim import HipBatchedSim

    n = STRESS_ENVS if args.envs == 5632 else args.envs
    K, W = args.steps, args.warmup
    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=args.seed, map_spec=BOMB_STRESS_40)
    U = cfg.fuse + 2 + W      # untimed ticks: the timed window sees the whole tick
    acts = stress_actions(n, K + U, args.seed, dev)
    loop = TickLoop(sim)
    for k in range(U):
        loop.launch_tick(acts[k])
    stats = torch.zeros((n, 4), dtype=torch.int32, device=dev)
    loop._tick.tick_stats = stats.data_ptr()
    torch.cuda.synchronize()
    _capi.timing_arm(0)          # creates the event pool outside the timed region
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        if sampled(k, K):
            _capi.timing_arm(1)
        loop.launch_tick(acts[U + k])
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    loop._tick.tick_stats = 0
    tick_ms = kernel_ms()["tick_kernel"]
    if args.copy_calibrate:
        _calibration_copy(torch, dev)
    achieved = TICK_BYTES_PER_ENV * n / (tick_ms * 1e-3) / 1e9
    cpu = cpu_baseline_stress(cfg, BOMB_STRESS_40, n, args.seed, args.cpu_seconds) \
        if args.cpu_seconds > 0 else None
    out = {
        "metric": "env-steps/s at 16384 envs, bomb-stress tick (injected actions), 1 MI355X",
        "value": n * K / el, "unit": "env-steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": el / K * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 sim",
        "data": "synthetic: template maps from Philox draws, actions from a seeded device generator",
        "config": {"workload": "bomb-stress ticks, 16384 envs, 13x13 pillars + 40% bricks, "
                               "bombs 1-4, blast 2-5, injected actions (bomb w.p. 0.5), auto-reset",
                   "envs": n, "parallelism": "single GPU"},
        "roofline": {"kernel": "tick_kernel", "bound": "hbm", "achieved": round(achieved, 3),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5),
                     "traffic": read_traffic("tick_kernel", STRESS_TRAFFIC_FILE)},
        "cpu_baseline": cpu,
        "kernels": {"tick_kernel": {"us": round(tick_ms * 1e3, 4),
                                    "bytes_per_env": TICK_BYTES_PER_ENV}},
        "timed_window": timed_window(stats, U, K, n),
    }
    print(json.dumps(out), flush=True)


# Algorithmic bytes of one env-step of the bot kernel: cell words (169 x 4 B),
# the danger channel of the observation (169 x 2 B), the player records
# (2 x 64 B), the bot's masks (7 B) and its action (2 B).
BOT_BYTES_PER_ENV = 169 * 4 + 169 * 2 + 2 * 64 + 7 + 2


def cpu_baseline_astar(cfg, spec, n, seed, budget_s):
    """The oracle's learner-vs-bot env-step on the host cores."""
    import numpy as np
    import torch

    from oracle import philox
    from oracle.bots import astar_act
    from oracle.policy import mlp_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim.policy import default_init

    cores = _cores(torch)
    params = default_init(cfg.obs_shape)
    sim = OracleSim(cfg, n, spec, seed=seed)
    envs = np.arange(n)

    def env_step(t):
        obs = sim.observe()
        mm, bm = sim.legal_mask()
        u = philox.uniforms(seed, envs, t, philox.STREAM_POLICY, 2)
        ub = torch.from_numpy(philox.uniforms(seed, envs, t, philox.STREAM_BOT, 5))
        acts = torch.zeros((n, 2, 2), dtype=torch.int64)
        ml, bl, _ = mlp_forward(params, obs, 0)
        acts[:, 0, 0] = torch.from_numpy(sample_masked(ml.numpy(), mm[:, 0].numpy(), u[:, 0])[0])
        acts[:, 0, 1] = torch.from_numpy(sample_masked(bl.numpy(), bm[:, 0].numpy(), u[:, 1])[0])
        acts[:, 1] = astar_act(cfg, sim.state_dict(), obs, mm[:, 1], bm[:, 1], 1, ub)
        sim.step(acts, auto_reset=True)

    env_step(0)
    ticks, t0 = 0, time.perf_counter()
    while True:
        env_step(1 + ticks)
        ticks += 1
        el = time.perf_counter() - t0
        if el >= budget_s or ticks >= 128:
            break
    return {"value": n * ticks / el, "unit": "env-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle (torch CPU restatement) learner-vs-astar env-step, {n} envs x "
                      f"{ticks} timed ticks after 1 warm-up tick, {el:.1f} s"}


def main_astar(args, torch, dev):
    """Learner vs astar bot: 5632 envs, 13x13 pillars + 70% bricks; player 0
    = the MLP (masked sampling), player 1 = the astar bot (two cost fields per
    env per tick); tick with auto-reset."""
    from qqtsim.bots import HipAstarBot
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.policy import HipActorCritic, default_init
    from qqtsim.rollout import Rollout
    from qqtsim.sim import HipBatchedSim

    n, K, W = args.envs, args.steps, args.warmup
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    sim = HipBatchedSim(cfg, n, device=dev, seed=args.seed, map_spec=spec)
    net = HipActorCritic(default_init(cfg.obs_shape), device=dev, seed=args.seed)
    bot = HipAstarBot(sim, pid=1)
    roll = Rollout(sim, net, opponent=bot)
    for _ in range(W):
        roll.step()
    torch.cuda.synchronize()
    _capi.timing_arm(0)          # creates the event pool outside the timed region
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        if sampled(k, K):
            _capi.timing_arm(4)          # policy, bot reach, bot, tick
        roll.step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    kms = kernel_ms()
    # the bot's share is its two launches (batch-max reach, then the bot)
    us = [kms["mlp_act_kernel"] * 1e3, (kms["bot_kernel"] + kms.get("reach_kernel", 0.0)) * 1e3,
          kms["tick_kernel"] * 1e3]
    kernels = {
        "mlp_act_kernel": {"us": us[0], "bound": "mfma",
                           "achieved": MLP_FLOP_PER_ENV / 2 * n / (us[0] * 1e-6) / 1e12,
                           "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s"},
        "bot_kernel": {"us": us[1], "bound": "hbm",
                       "achieved": BOT_BYTES_PER_ENV * n / (us[1] * 1e-6) / 1e9,
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "bytes_per_env": BOT_BYTES_PER_ENV},
        "tick_kernel": {"us": us[2], "bound": "hbm",
                        "achieved": TICK_BYTES_PER_ENV * n / (us[2] * 1e-6) / 1e9,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "bytes_per_env": TICK_BYTES_PER_ENV},
    }
    for v in kernels.values():
        v["frac"] = v["achieved"] / v["peak"]
    dom = max(kernels, key=lambda k: kernels[k]["us"])
    d = kernels[dom]
    cpu = cpu_baseline_astar(cfg, spec, n, args.seed, args.cpu_seconds) \
        if args.cpu_seconds > 0 else None
    out = {
        "metric": "env-steps/s at 5632 envs, learner MLP vs astar bot (step+obs+act+bot), 1 MI355X",
        "value": n * K / el, "unit": "env-steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": el / K * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 sim and bot / f16 MFMA (f32 accumulate)",
        "data": "synthetic: template maps from Philox draws, PyTorch default-init MLP weights",
        "config": {"workload": "learner MLP (player 0) vs astar bot (player 1), 5632 envs, "
                               "13x13 pillars + 70% bricks, auto-reset",
                   "envs": n, "parallelism": "single GPU"},
        "roofline": {"kernel": dom, "bound": d["bound"], "achieved": round(d["achieved"], 3),
                     "peak": d["peak"], "unit": d["unit"], "frac": round(d["frac"], 5),
                     "traffic": None},
        "cpu_baseline": cpu,
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in kernels.items()},
    }
    print(json.dumps(out), flush=True)


EVAL_ENVS, EVAL_TICKS = 32768, 128
EVAL_FLOP_PER_ROW = MLP_FLOP_PER_ENV // 2          # one player per row
EVAL_BYTES_PER_ROW = 14 * 169 * 2 + 8 * 4          # observation in, 8 float32 logits out


def cpu_baseline_forward(cfg, rows, seed, budget_s):
    """The oracle's float32 forward (one player) on the host cores."""
    import torch

    from oracle.policy import mlp_forward
    from qqtsim.policy import default_init

    cores = _cores(torch)
    params = default_init(cfg.obs_shape)
    g = torch.Generator().manual_seed(seed)
    obs = (torch.rand((rows,) + tuple(cfg.obs_shape), generator=g) < 0.3).half()
    mlp_forward(params, obs[:1024], 0)
    done, t0 = 0, time.perf_counter()
    while True:
        mlp_forward(params, obs, 0)
        done += rows
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 64 * rows:
            break
    return {"value": done / el, "unit": "obs/s", "cores": cores, "kind": "port",
            "sample": f"oracle float32 forward, {done // rows} passes over {rows} synthetic "
                      f"observations, {el:.1f} s"}


def main_evalfwd(args, torch, dev):
    """32768 envs x 128 ticks of self-play rollout writing the observation
    slab (128, 32768, 14, 13, 13) float16 (19.85 GB) directly, then one
    batched actor/critic forward (player 0: logits + value) over all
    4,194,304 observations, as the PPO evaluation pass does."""
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.policy import HipActorCritic, default_init
    from qqtsim.rollout import Rollout
    from qqtsim.sim import HipBatchedSim

    n = EVAL_ENVS if args.envs == 5632 else args.envs
    T = EVAL_TICKS
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    params = default_init(cfg.obs_shape)
    sim = HipBatchedSim(cfg, n, device=dev, seed=args.seed, map_spec=spec)
    net = HipActorCritic(params, device=dev, seed=args.seed)
    roll = Rollout(sim, net)
    for _ in range(4):
        roll.step()
    buf = torch.empty((T, n) + tuple(cfg.obs_shape), dtype=torch.float16, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    roll.run_into(buf)
    torch.cuda.synchronize()
    el_roll = time.perf_counter() - t0

    rows = T * n
    flat = buf.view(rows, -1)
    out = torch.empty((rows, 1, 8), dtype=torch.float32, device=dev)
    net._run(flat, 1, 0, False, logits=out)          # warm-up
    torch.cuda.synchronize()
    reps = max(1, args.steps // 64)
    _capi.timing_arm(0)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _capi.timing_arm(reps)
    for _ in range(reps):
        net._run(flat, 1, 0, False, logits=out)
    torch.cuda.synchronize()
    el_fwd = (time.perf_counter() - t1) / reps
    fwd_ms = kernel_ms()["mlp_act_kernel"]     # the policy launches' timing slot (mlp_fwd_kernel here)
    if args.copy_calibrate:
        _calibration_copy(torch, dev)
    gbs = EVAL_BYTES_PER_ROW * rows / (fwd_ms * 1e-3) / 1e9
    tflops = EVAL_FLOP_PER_ROW * rows / (fwd_ms * 1e-3) / 1e12
    cpu = cpu_baseline_forward(cfg, 32768, args.seed, args.cpu_seconds) \
        if args.cpu_seconds > 0 else None
    res = {
        "metric": "obs/s of the batched actor/critic evaluation forward over a 128 x 32768 "
                  "rollout slab (4.19M observations), 1 MI355X",
        "value": rows / el_fwd, "unit": "obs/s", "n_gpus": 1, "steps": reps, "warmup": 1,
        "ms_per_step": el_fwd * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 MFMA (f32 accumulate; hi/lo f16 after layer 1)",
        "data": "synthetic: observations from a self-play rollout on template maps, "
                "PyTorch default-init MLP weights",
        "config": {"workload": "rollout 32768 envs x 128 ticks into the float16 observation "
                               "slab, then one forward (player 0) over all 4,194,304 rows",
                   "envs": n, "ticks": T, "rows": rows, "parallelism": "single GPU"},
        "roofline": {"kernel": "mlp_fwd_kernel (forward, 4.19M rows)", "bound": "hbm",
                     "achieved": round(gbs, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 5),
                     "traffic": read_traffic("mlp_fwd_kernel", EVAL_TRAFFIC_FILE)},
        "mfma": {"achieved_tflops": round(tflops, 3), "peak_tflops": MFMA_F16_PEAK_TFLOPS,
                 "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 5),
                 "flop_per_row": EVAL_FLOP_PER_ROW},
        "rollout": {"env_steps_per_s": n * T / el_roll, "ms": el_roll * 1e3,
                    "slab_gb": buf.numel() * 2 / 1e9},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)



# Algorithmic bytes of the GAE scan per (step, env): reward, value, done read,
# advantage and return written.
GAE_BYTES = 4 + 4 + 1 + 4 + 4
COLLECT_T = 128


def cpu_baseline_collect(cfg, spec, n, seed, budget_s):
    """The oracle's collect loop on the host cores: env-steps (observe,
    masks, both players' forward + sampling, step) appended to host lists,
    then the oracle's GAE over the sampled steps."""
    import numpy as np
    import torch

    from oracle import philox
    from oracle.policy import mlp_forward, sample_masked
    from oracle.ppo import gae
    from oracle.sim import OracleSim
    from qqtsim.policy import default_init

    cores = _cores(torch)
    params = default_init(cfg.obs_shape)
    sim = OracleSim(cfg, n, spec, seed=seed)
    envs = np.arange(n)
    rec = {k: [] for k in ("obs", "mm", "bm", "act", "val", "rew", "done")}

    def env_step(t):
        obs = sim.observe()
        mm, bm = sim.legal_mask()
        u = philox.uniforms(seed, envs, t, philox.STREAM_POLICY, 4)
        acts = torch.zeros((n, 2, 2), dtype=torch.int64)
        v0 = None
        for pid in range(2):
            ml, bl, v = mlp_forward(params, obs, pid)
            v0 = v if pid == 0 else v0
            acts[:, pid, 0] = torch.from_numpy(
                sample_masked(ml.numpy(), mm[:, pid].numpy(), u[:, 2 * pid])[0])
            acts[:, pid, 1] = torch.from_numpy(
                sample_masked(bl.numpy(), bm[:, pid].numpy(), u[:, 2 * pid + 1])[0])
        rew, done, _ = sim.step(acts, auto_reset=True)
        for k, x in (("obs", obs), ("mm", mm[:, 0]), ("bm", bm[:, 0]), ("act", acts[:, 0]),
                     ("val", v0), ("rew", rew[:, 0]), ("done", done)):
            rec[k].append(np.array(x))

    env_step(0)
    for k in rec:
        rec[k].clear()
    ticks, t0 = 0, time.perf_counter()
    while True:
        env_step(1 + ticks)
        ticks += 1
        if time.perf_counter() - t0 >= budget_s or ticks >= COLLECT_T:
            break
    last = mlp_forward(params, sim.observe(), 0)[2].numpy()
    gae(np.stack(rec["rew"]), np.stack(rec["val"]), np.stack(rec["done"]).astype(np.float32),
        last, 0.995, 0.95)
    el = time.perf_counter() - t0
    return {"value": n * ticks / el, "unit": "env-steps/s", "cores": cores, "kind": "port",
            "sample": f"oracle (torch CPU restatement) collect loop, {n} envs x {ticks} "
                      f"steps into host buffers + GAE, after 1 warm-up step, {el:.1f} s"}


def main_collect(args, torch, dev):
    """Self-play collects into the device rollout buffer: 5632 envs x 128
    steps per collect (observation slab, masks, actions, log-probs, values,
    rewards, done and damage flags written by the kernels in place), then the
    learner's value of the final observation and the GAE scan
    (train/ppo.py:197-314, :101-110).  `--steps` counts env-steps per env
    (rounded up to whole collects)."""
    from qqtsim import HipRolloutBuffer, compute_gae

    n, W = args.envs, args.warmup
    reps = max(1, -(-args.steps // COLLECT_T))
    cfg, spec, roll = build_workload(n, args.seed, dev)
    for _ in range(W):
        roll.step()
    buf = HipRolloutBuffer(COLLECT_T, n, cfg.obs_shape, dev)
    roll.collect(buf)                                    # warm-up collect
    net = roll.policy
    compute_gae(buf, net.forward(roll.sim.observe(), 0)[2], 0.995, 0.95)
    _capi.timing_arm(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        _capi.timing_arm(2 * 8)                          # the first 8 steps' launches
        roll.collect(buf)
        last_val = net.forward(roll.sim.observe(), 0)[2]
        _capi.timing_arm(1)
        adv, ret = compute_gae(buf, last_val, 0.995, 0.95)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    kms = kernel_ms()
    steps = reps * COLLECT_T
    gae_us = kms["gae_kernel"] * 1e3
    gae_gbs = GAE_BYTES * COLLECT_T * n / (gae_us * 1e-6) / 1e9
    act_ms, tick_ms = kms["mlp_act_kernel"], kms["tick_kernel"]
    mlp_tf = MLP_FLOP_PER_ENV * n / (act_ms * 1e-3) / 1e12
    cpu = cpu_baseline_collect(cfg, spec, n, args.seed, args.cpu_seconds) \
        if args.cpu_seconds > 0 else None
    res = {
        "metric": "env-steps/s at 5632 envs, self-play collect into the device rollout "
                  "buffer (128 steps) + last-value forward + GAE, 1 MI355X",
        "value": n * steps / el, "unit": "env-steps/s", "n_gpus": 1, "steps": steps,
        "warmup": W, "ms_per_step": el / steps * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 sim / f16 MFMA (f32 accumulate) / f32 GAE",
        "data": "synthetic: template maps from Philox draws, PyTorch default-init MLP weights",
        "config": {"workload": "self-play collect, 5632 envs x 128 steps into the rollout "
                               "buffer (obs slab 3.4 GB per 128 steps), GAE gamma 0.995 "
                               "lambda 0.95", "envs": n, "collect_steps": COLLECT_T,
                   "collects": reps, "parallelism": "single GPU"},
        "roofline": {"kernel": "mlp_act_kernel", "bound": "mfma", "achieved": round(mlp_tf, 3),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(mlp_tf / MFMA_F16_PEAK_TFLOPS, 5),
                     "traffic": read_traffic("mlp_act_kernel")},
        "kernels": {"mlp_act_kernel": {"us": round(act_ms * 1e3, 3)},
                    "tick_kernel": {"us": round(tick_ms * 1e3, 3)},
                    "gae_kernel": {"us": round(gae_us, 3), "bound": "hbm",
                                   "achieved": round(gae_gbs, 3), "peak": HBM_PEAK_GBS,
                                   "unit": "GB/s", "bytes_per_step_env": GAE_BYTES,
                                   "frac": round(gae_gbs / HBM_PEAK_GBS, 5)}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)

def _torch_mlp(torch, sd, dev):
    """The reference's mlp ActorCritic as plain torch modules (float32,
    eager): forward and evaluate of train/model.py:140-153, 192-196,
    215-256.  The PyTorch-on-GPU baseline of the PPO update."""
    nn = torch.nn
    from qqtsim.policy import column_permutation

    class Mlp(nn.Module):
        arch = "mlp"

        def __init__(self):
            super().__init__()
            self.shared = nn.Sequential(nn.Linear(2366, 128), nn.LayerNorm(128), nn.ReLU(),
                                        nn.Linear(128, 128), nn.LayerNorm(128), nn.ReLU())
            self.move_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 5))
            self.bomb_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 2))
            self.critic = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 1))
            self.cols = [column_permutation(p, 2, 14, 169).to(dev) for p in range(2)]

        def forward(self, obs, pid=0):
            x = obs.to(self.shared[0].weight.dtype).reshape(obs.shape[0], -1)
            x = torch.nn.functional.linear(x, self.shared[0].weight[:, self.cols[pid]],
                                           self.shared[0].bias)
            x = self.shared[1:](x)
            return self.move_head(x), self.bomb_head(x), self.critic(x).squeeze(-1)

        def evaluate(self, obs, mm, bm, act, pid=0):
            ml, bl, v = self(obs, pid)
            neg = torch.finfo(ml.dtype).min
            dm = torch.distributions.Categorical(
                logits=torch.where(mm.bool(), ml, torch.full_like(ml, neg)))
            db = torch.distributions.Categorical(
                logits=torch.where(bm.bool(), bl, torch.full_like(bl, neg)))
            logp = dm.log_prob(act[..., 0]) + db.log_prob(act[..., 1])
            return logp, dm.entropy() + db.entropy(), v

    m = Mlp()
    m.load_state_dict(sd)
    return m.to(dev)


# Algorithmic bytes and FLOP per row of the first-layer weight gradient:
# the float16 observation row and the float32 dz1 row read once; 2 x 128 x
# 2366 multiply-adds, twice (the hi and lo halves of dz1).
L1G_BYTES_PER_ROW = 2366 * 2 + 128 * 4
L1G_FLOP_PER_ROW = 2 * 2 * 128 * 2366


def _require_finite(what, stats):
    """Exit non-zero when an update's statistics are not all finite (a
    diverged learner makes the timing meaningless)."""
    bad = {k: v for k, v in stats.items() if not math.isfinite(v)}
    if bad:
        print(f"{what}: non-finite statistics {bad}", file=sys.stderr, flush=True)
        sys.exit(3)


def main_ppo(args, torch, dev):
    """One PPO update (train/ppo.py:364-437: GAE, 4 epochs x 4 minibatches of
    the clipped loss, backward, gradient clipping, Adam) over a buffer of
    5632 envs x 128 self-play steps collected by the kernels.  `value` counts
    rows processed per second (rows x epochs / update time).  The learner is
    HipMlpActorCritic (first layer forward and weight gradient on MFMA, the
    loss and the backward above the first layer fused in one kernel);
    `torch_gpu_baseline` runs the same update with the reference's network
    as float32 eager torch modules on the same GPU."""
    from qqtsim import HipMlpActorCritic, HipRolloutBuffer, PPOConfig, ppo_update
    from qqtsim.policy import reference_init

    n = args.envs
    cfg, spec, roll = build_workload(n, args.seed, dev)
    sd = reference_init(cfg.obs_shape)
    roll.policy.load_state_dict(sd)           # the learner acts (and is cloned as the opponent)
    for _ in range(max(1, args.warmup)):
        roll.step()
    buf = HipRolloutBuffer(COLLECT_T, n, cfg.obs_shape, dev)
    roll.collect(buf)
    last_val = roll.policy.forward(roll.sim.observe(), 0)[2]
    pcfg = PPOConfig()
    rows = COLLECT_T * n
    reps = 2 if args.steps >= 256 else max(1, min(args.steps, 3))   # whole updates timed

    def run(learner, timed_launches=0):
        """Warm-up update, then `reps` timed updates, each from the same
        weights and optimizer state (the first update's statistics on a
        buffer the weights acted are the ones a training run sees)."""
        start = {k: v.detach().clone() for k, v in learner.state_dict().items()}
        opt = torch.optim.Adam(learner.parameters(), lr=pcfg.lr)
        torch.manual_seed(0)
        ppo_update(learner, opt, buf, last_val, pcfg, pcfg.entropy_coef)     # warm-up
        torch.cuda.synchronize()
        best, stats = float("inf"), None
        for _ in range(reps):
            learner.load_state_dict(start)
            opt = torch.optim.Adam(learner.parameters(), lr=pcfg.lr)
            torch.manual_seed(0)
            torch.cuda.synchronize()
            if timed_launches:
                _capi.timing_arm(timed_launches)
            t0 = time.perf_counter()
            stats = ppo_update(learner, opt, buf, last_val, pcfg, pcfg.entropy_coef)
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        return best, stats

    _capi.timing_arm(0)
    learner = HipMlpActorCritic(cfg.obs_shape, device=dev, state_dict=sd)
    # GAE, then the first minibatch's four launches (forward, fused loss +
    # backward, weight gradient and its chunk reduction)
    el, stats = run(learner, timed_launches=1 + 4)
    tim = _capi.timing_collect()
    mb_rows = rows // pcfg.minibatches
    fwd_ms = tim["mlp_act_kernel"][0] / tim["mlp_act_kernel"][1]
    # weight-gradient kernel + chunk reduction, per minibatch
    l1g_ms = tim["l1grad_kernels"][0] / (tim["l1grad_kernels"][1] / 2)
    l1g_gbs = L1G_BYTES_PER_ROW * mb_rows / (l1g_ms * 1e-3) / 1e9
    l1g_tf = L1G_FLOP_PER_ROW * mb_rows / (l1g_ms * 1e-3) / 1e12
    fwd_gbs = 2366 * 2 * mb_rows / (fwd_ms * 1e-3) / 1e9
    ppo_ms = tim["ppo_grad_kernel"][0] / tim["ppo_grad_kernel"][1]
    if args.no_torch_baseline:
        el_ref, ref_stats = None, None
    else:
        ref = _torch_mlp(torch, sd, dev)
        el_ref, ref_stats = run(ref)
    samples = rows * pcfg.epochs
    cpu = None
    if args.cpu_seconds > 0:
        cores = _cores(torch)
        cpu_net = _torch_mlp(torch, sd, torch.device("cpu"))
        opt = torch.optim.Adam(cpu_net.parameters(), lr=pcfg.lr)
        b = 4096
        obs = buf.obs.reshape(-1, 14, 13, 13)[:b].cpu()
        mm, bm = buf.mmask.reshape(-1, 5)[:b].cpu(), buf.bmask.reshape(-1, 2)[:b].cpu()
        act = buf.act.reshape(-1, 2)[:b].cpu()
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or done == 0:
            logp, ent, v = cpu_net.evaluate(obs, mm, bm, act)
            loss = -(logp.mean()) + 0.5 * (v ** 2).mean() - 0.05 * ent.mean()
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            done += 1
        elc = time.perf_counter() - t0
        cpu = {"value": b * done / elc, "unit": "samples/s", "cores": cores, "kind": "port",
               "sample": f"the reference's mlp ActorCritic as float32 torch modules on the "
                         f"host: {done} minibatches of {b} rows (evaluate + loss + backward + "
                         f"Adam), {elc:.1f} s"}
    res = {
        "metric": "PPO update samples/s (5632 envs x 128 steps, 4 epochs x 4 minibatches), "
                  "1 MI355X",
        "value": samples / el, "unit": "samples/s", "n_gpus": 1, "steps": reps,
        "warmup": 1, "ms_per_step": el * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA first layer (f32 accumulate) / f32 fused loss + backward / f32 torch "
                 "weight-gradient products and Adam",
        "data": "synthetic: a buffer collected by the kernels from template maps, acted by "
                "the learner's weights (the reference ActorCritic's orthogonal init)",
        "config": {"workload": "PPO update over a 5632 x 128 rollout buffer "
                               "(train/ppo.py:364-437)", "rows": rows,
                   "epochs": pcfg.epochs, "minibatches": pcfg.minibatches,
                   "minibatch_rows": mb_rows, "parallelism": "single GPU"},
        "roofline": {"kernel": "l1_grad_kernel + l1_grad_reduce", "bound": "hbm",
                     "achieved": round(l1g_gbs, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(l1g_gbs / HBM_PEAK_GBS, 5), "traffic": None},
        "kernels": {"l1_grad (per minibatch)": {"us": round(l1g_ms * 1e3, 3),
                                                "achieved_gbs": round(l1g_gbs, 3),
                                                "tflops": round(l1g_tf, 3),
                                                "bytes_per_row": L1G_BYTES_PER_ROW},
                    "first-layer forward (per minibatch)": {
                        "us": round(fwd_ms * 1e3, 3), "obs_gbs": round(fwd_gbs, 3)},
                    "ppo_grad_kernel (per minibatch)": {"us": round(ppo_ms * 1e3, 3)}},
        "torch_gpu_baseline": None if el_ref is None else {
            "value": samples / el_ref, "unit": "samples/s", "ms_per_update": el_ref * 1e3,
            "speedup": round(el_ref / el, 3), "update_stats": ref_stats,
            "note": "same update, the reference's network as float32 eager torch modules"},
        "update_stats": stats,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    _require_finite("ppo update", stats)


def main_train(args, torch, dev):
    """Whole training iterations of the reference's loop (train/ppo.py:197-314
    collect + :364-437 update): 128 self-play steps of 5632 envs into the
    device rollout buffer (both players acted by the current network), the
    learner's value of the last observation, one PPO update (4 epochs x 4
    minibatches) and the copy of the updated weights into the acting
    network.  `value` is env-steps per second of the whole iteration (the
    reference's "sps")."""
    from qqtsim import HipMlpActorCritic, HipRolloutBuffer, PPOConfig, ppo_update
    from qqtsim.policy import reference_init

    n = args.envs
    cfg, spec, roll = build_workload(n, args.seed, dev)
    sd = reference_init(cfg.obs_shape)
    actor = roll.policy
    actor.load_state_dict(sd)                 # the learner acts (and is cloned as the opponent)
    for _ in range(max(1, args.warmup)):
        roll.step()
    buf = HipRolloutBuffer(COLLECT_T, n, cfg.obs_shape, dev)
    pcfg = PPOConfig()
    learner = HipMlpActorCritic(cfg.obs_shape, device=dev, state_dict=sd)
    opt = torch.optim.Adam(learner.parameters(), lr=pcfg.lr)

    def iteration():
        roll.collect(buf)
        last_val = actor.forward(roll.sim.observe(), 0)[2]
        st = ppo_update(learner, opt, buf, last_val, pcfg, pcfg.entropy_coef)
        actor.load_state_dict(learner.state_dict())
        return st

    torch.manual_seed(0)
    history = [iteration()]                          # warm-up iteration
    torch.cuda.synchronize()
    iters = 3 if args.steps >= 256 else max(1, min(args.steps, 3))
    t0 = time.perf_counter()
    for _ in range(iters):
        history.append(iteration())
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    st = history[-1]
    steps = iters * COLLECT_T * n
    res = {
        "metric": "training env-steps/s (collect 128 steps x 5632 envs + PPO update + weight "
                  "sync), 1 MI355X",
        "value": steps / el, "unit": "env-steps/s", "n_gpus": 1, "steps": iters, "warmup": 1,
        "ms_per_step": el / iters * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 sim / f16 MFMA acting / f16 MFMA first layer + f32 fused loss and "
                 "backward in the update",
        "data": "synthetic: template maps from Philox draws, the reference ActorCritic's "
                "orthogonal init for the learner (acting for both players)",
        "config": {"workload": "training iteration: collect (5632 envs x 128 steps) + PPO "
                               "update (4 epochs x 4 minibatches) + weight sync",
                   "envs": n, "collect_steps": COLLECT_T, "parallelism": "single GPU"},
        "last_update_stats": st,
        "update_stats_per_iteration": history,
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)
    for i, h in enumerate(history):
        _require_finite(f"training iteration {i}", h)



# Algorithmic FLOP of the cnn actor/critic for one player view: 2 x MACs of
# conv0 14->16 3x3, conv 16->32 3x3, conv 32->64 3x3, conv 64->8 1x1 on
# 169 positions, Linear 1352->128, 128->128, three 128->64 heads and their
# 64->(5+2+1) outputs.
CNN_MACS = (169 * (14 * 9 * 16 + 16 * 9 * 32 + 32 * 9 * 64 + 64 * 8)
            + 1352 * 128 + 128 * 128 + 3 * 128 * 64 + 64 * 8)
CNN_FLOP_PER_ENV = 2 * 2 * CNN_MACS            # both players
# MACs of the convolutions and Linear(1352,128) (run as three float16
# products each) and of the rest (float32 MFMA)
CNN_CONV_MACS = 169 * (14 * 9 * 16 + 16 * 9 * 32 + 32 * 9 * 64 + 64 * 8)
CNN_F16_MACS = CNN_CONV_MACS + 1352 * 128
MFMA_F32_PEAK_TFLOPS = 157.3


def _torch_cnn(torch, sd, dev):
    """The reference's cnn ActorCritic as plain float32 eager torch modules
    (train/model.py:79-96, 140-153, 186-196, 230-245): forward through the
    view-permuted conv0 and act() with masked Categorical sampling."""
    nn = torch.nn
    F = torch.nn.functional
    from qqtsim.config import view_perm

    class Cnn(nn.Module):
        def __init__(self):
            super().__init__()
            self.conv0 = nn.Conv2d(14, 16, 3, padding=1)
            self.conv = nn.Sequential(
                nn.LayerNorm([16, 13, 13]), nn.ReLU(), nn.Conv2d(16, 32, 3, padding=1),
                nn.LayerNorm([32, 13, 13]), nn.ReLU(), nn.Conv2d(32, 64, 3, padding=1),
                nn.LayerNorm([64, 13, 13]), nn.ReLU(), nn.Conv2d(64, 8, 1),
                nn.LayerNorm([8, 13, 13]), nn.ReLU())
            self.shared = nn.Sequential(nn.Linear(1352, 128), nn.LayerNorm(128), nn.ReLU(),
                                        nn.Linear(128, 128), nn.LayerNorm(128), nn.ReLU())
            self.move_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 5))
            self.bomb_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 2))
            self.critic = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 1))
            self.inv = [torch.argsort(torch.tensor(view_perm(p, 2, 14))).to(dev) for p in range(2)]

        def forward(self, obs, pid=0):
            x = F.conv2d(obs.float(), self.conv0.weight[:, self.inv[pid]], self.conv0.bias,
                         padding=1)
            x = self.shared(self.conv(x).flatten(1))
            return self.move_head(x), self.bomb_head(x), self.critic(x).squeeze(-1)

        @torch.no_grad()
        def act(self, obs, mm, bm, pid=0):
            ml, bl, v = self(obs, pid)
            neg = torch.finfo(ml.dtype).min
            dm = torch.distributions.Categorical(logits=torch.where(mm, ml, torch.full_like(ml, neg)))
            db = torch.distributions.Categorical(logits=torch.where(bm, bl, torch.full_like(bl, neg)))
            a = torch.stack([dm.sample(), db.sample()], -1)
            return a, dm.log_prob(a[:, 0]) + db.log_prob(a[:, 1]), v

    m = Cnn()
    m.load_state_dict(sd)
    return m.to(dev)


def main_cnn(args, torch, dev):
    """The self-play rollout of the headline workload with the reference's cnn
    actor/critic as the policy (both players: the cnn_trunk_kernel and
    cnn_head_kernel launches, then the tick).  `torch_gpu_baseline` times the reference's act() for both
    players with the same network as float32 eager torch modules (MIOpen
    convolutions) on the same GPU and observations."""
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.policy import HipCnnActorCritic, default_init_cnn
    from qqtsim.rollout import Rollout
    from qqtsim.sim import HipBatchedSim

    n, K, W = args.envs, args.steps, args.warmup
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    sim = HipBatchedSim(cfg, n, device=dev, seed=args.seed, map_spec=spec)
    sd = default_init_cnn(cfg.obs_shape)
    roll = Rollout(sim, HipCnnActorCritic(sd, device=dev, seed=args.seed))
    for _ in range(W):
        roll.step()
    torch.cuda.synchronize()
    _capi.timing_arm(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        if sampled(k, K):
            _capi.timing_arm(3)
        roll.launch_act()
        roll.launch_tick()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    kms = kernel_ms()
    trunk_ms, head_ms, tick_ms = kms["cnn_trunk_kernel"], kms["cnn_head_kernel"], kms["tick_kernel"]
    act_ms = trunk_ms + head_ms
    kernels = {
        "cnn_act": {"us": act_ms * 1e3, "trunk_us": trunk_ms * 1e3, "head_us": head_ms * 1e3,
                    "bound": "mfma",
                    "achieved": CNN_FLOP_PER_ENV * n / (act_ms * 1e-3) / 1e12,
                    "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "flop_per_env": CNN_FLOP_PER_ENV,
                    "executed_tflops": 2 * 2 * (3 * CNN_F16_MACS + CNN_MACS - CNN_F16_MACS)
                    * n / (act_ms * 1e-3) / 1e12,
                    "f32_equivalent_frac": CNN_FLOP_PER_ENV * n / (act_ms * 1e-3) / 1e12
                    / MFMA_F32_PEAK_TFLOPS},
        "tick_kernel": {"us": tick_ms * 1e3, "bound": "hbm",
                        "achieved": TICK_BYTES_PER_ENV * n / (tick_ms * 1e-3) / 1e9,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "bytes_per_env": TICK_BYTES_PER_ENV},
    }
    for v in kernels.values():
        v["frac"] = v["achieved"] / v["peak"]
    d = kernels["cnn_act"]

    # the reference's act() for both players, eager float32 torch on this GPU
    ref = _torch_cnn(torch, sd, dev)
    obs = sim.observe().clone()
    mm, bm = (m.bool().clone() for m in sim.legal_mask())
    for _ in range(3):
        for pid in range(2):
            ref.act(obs, mm[:, pid], bm[:, pid], pid)
    torch.cuda.synchronize()
    reps = 10
    t1 = time.perf_counter()
    for _ in range(reps):
        for pid in range(2):
            ref.act(obs, mm[:, pid], bm[:, pid], pid)
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t1) / reps * 1e3

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(cfg, spec, 512, args.seed, args.cpu_seconds, arch="cnn")
    value = n * K / el
    out = {
        "metric": "env-steps/s at 5632 envs (step+obs+cnn act), 1 MI355X; % MFMA roofline",
        "value": value, "unit": "env-steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": el / K * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 sim / cnn convs and Linear(1352,128) as three f16 MFMA products (hi/lo "
                 "split, f32 accumulate), f32 MFMA for the later head layers",
        "data": "synthetic: template maps from Philox draws, PyTorch default-init cnn weights",
        "config": {"workload": "self-play rollout, 5632 envs, 13x13 pillars + 70% bricks, "
                               "P=2, 14-ch f16 obs, cnn act both players + masked sampling, "
                               "auto-reset", "envs": n, "parallelism": "single GPU"},
        "roofline": {"kernel": "cnn_trunk_kernel + cnn_head_kernel", "bound": d["bound"],
                     "achieved": round(d["achieved"], 3), "peak": d["peak"], "unit": d["unit"],
                     "frac": round(d["frac"], 5), "traffic": None,
                     "note": "algorithmic FLOP of the whole act over the summed durations of "
                             "its two launches, against the dense float16 MFMA peak (the "
                             "convolutions and the first head layer run there, three products "
                             "per float32-accurate product); executed_tflops and "
                             "f32_equivalent_frac in kernels"},
        "torch_gpu_baseline": {"act_ms_both_players": round(ref_ms, 3),
                               "hip_act_ms_both_players": round(act_ms, 4),
                               "speedup": round(ref_ms / act_ms, 2),
                               "note": "the reference's act() (forward + masked Categorical "
                                       "sampling) for both players, float32 eager torch with "
                                       "MIOpen convolutions, same observations"},
        "cpu_baseline": cpu,
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in kernels.items()},
    }
    print(json.dumps(out), flush=True)



# Multiply-accumulates of one row (one player) of the lstm network
# (train/model.py:103-120): conv 3x3 14->32 and 32->64 over 49 positions,
# Linear 576->128, rel 60->64->32, glob 5->16->8, fusion 168->256, the LSTM
# gates (256 + 128 inputs, 512 outputs), the heads 128->3x64 and 3x64->8.
LSTM_MACS = (49 * 126 * 32 + 49 * 288 * 64 + 576 * 128 + 60 * 64 + 64 * 32 + 5 * 16 + 16 * 8
             + 168 * 256 + 384 * 512 + 128 * 192 + 64 * 8)
LSTM_FLOP_PER_ROW = 2 * LSTM_MACS
# MACs the kernel issues per row on float16 MFMA: conv1 over 196 of 208
# tile positions x 160 K (two products, the windows being float16), conv2 at
# the 36 pooled positions x 288 K and the head (three products each).
LSTM_ISSUED_MACS = (2 * (208 / 4) * 160 * 32 + 3 * 36 * 288 * 64
                    + 3 * (576 * 128 + 64 * 64 + 64 * 32 + 2 * 32 * 16 + 192 * 256 + 384 * 512
                           + 128 * 192 + 192 * 16))
MFMA_F32_PEAK = 157.3
# Algorithmic bytes of the feature kernel per env (one player): the packed
# cells (169 x 4 B), the player rows (2 x 48 B), t (4 B), the 14 x 7 x 7
# float16 window read and written, rel (120 B) and glob (10 B) written.
LSTM_FEAT_BYTES_PER_ENV = 169 * 4 + 2 * 48 + 4 + 2 * 14 * 49 * 2 + 120 + 10


def _torch_lstm(torch, sd, dev):
    """The reference's lstm ActorCritic (train/model.py:103-120, 176-185,
    198-214, 230-245) as plain float32 eager torch modules: extract_fused,
    nn.LSTM over one step, the heads and masked Categorical sampling."""
    nn = torch.nn

    class Lstm(nn.Module):
        def __init__(self):
            super().__init__()
            self.l_conv1 = nn.Conv2d(14, 32, 3, padding=1)
            self.l_conv2 = nn.Conv2d(32, 64, 3, padding=1)
            self.l_pool = nn.MaxPool2d(2)
            self.l_cnn_fc = nn.Linear(576, 128)
            self.l_rel_fc1 = nn.Linear(60, 64)
            self.l_rel_fc2 = nn.Linear(64, 32)
            self.l_glob_fc1 = nn.Linear(5, 16)
            self.l_glob_fc2 = nn.Linear(16, 8)
            self.l_fusion = nn.Linear(168, 256)
            self.lstm = nn.LSTM(256, 128, 1, batch_first=True)
            self.move_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 5))
            self.bomb_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 2))
            self.critic = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 1))

        def forward(self, local, rel, glob, hidden):
            r = torch.relu
            x = r(self.l_conv1(local.float()))
            x = self.l_pool(r(self.l_conv2(x)))
            x = r(self.l_cnn_fc(x.view(x.size(0), -1)))
            e = r(self.l_rel_fc2(r(self.l_rel_fc1(rel.float().view(rel.size(0), -1)))))
            g = r(self.l_glob_fc2(r(self.l_glob_fc1(glob.float()))))
            f = r(self.l_fusion(torch.cat([x, e, g], 1)))
            lo, nh = self.lstm(f.unsqueeze(1), hidden)
            lo = lo.squeeze(1)
            return self.move_head(lo), self.bomb_head(lo), self.critic(lo).squeeze(-1), nh

        @torch.no_grad()
        def act(self, local, rel, glob, mm, bm, hidden):
            ml, bl, v, nh = self(local, rel, glob, hidden)
            neg = torch.finfo(ml.dtype).min
            dm = torch.distributions.Categorical(logits=torch.where(mm, ml, torch.full_like(ml, neg)))
            db = torch.distributions.Categorical(logits=torch.where(bm, bl, torch.full_like(bl, neg)))
            a = torch.stack([dm.sample(), db.sample()], -1)
            return a, dm.log_prob(a[:, 0]) + db.log_prob(a[:, 1]), v, nh

    m = Lstm()
    m.load_state_dict(sd)
    return m.to(dev)


def cpu_baseline_lstm(cfg, spec, n, seed, budget_s):
    """The oracle's lstm learner-vs-astar env-step on the host cores:
    local_view_features (only_p0), the lstm forward with the state carried
    and zeroed on done, masked sampling, the astar bot, step."""
    import numpy as np
    import torch

    from oracle import philox
    from oracle.bots import astar_act
    from oracle.obs import local_view_features
    from oracle.policy import lstm_forward, sample_masked
    from oracle.sim import OracleSim
    from qqtsim.policy import reference_init

    cores = _cores(torch)
    params = reference_init(cfg.obs_shape, arch="lstm")
    sim = OracleSim(cfg, n, spec, seed=seed)
    envs = np.arange(n)
    state = {"hidden": None}

    def env_step(t):
        obs = sim.observe()
        mm, bm = sim.legal_mask()
        s = sim.state_dict()
        loc, rel, glb = local_view_features(cfg, obs, s["pos"], s["alive"], s["t"], s["fuse"],
                                            s["hp"], only_p0=True)
        ml, bl, _, hid = lstm_forward(params, loc[:, 0], rel[:, 0], glb[:, 0], state["hidden"])
        u = philox.uniforms(seed, envs, t, philox.STREAM_POLICY, 2)
        ub = torch.from_numpy(philox.uniforms(seed, envs, t, philox.STREAM_BOT, 5))
        acts = torch.zeros((n, 2, 2), dtype=torch.int64)
        acts[:, 0, 0] = torch.from_numpy(sample_masked(ml.numpy(), mm[:, 0].numpy(), u[:, 0])[0])
        acts[:, 0, 1] = torch.from_numpy(sample_masked(bl.numpy(), bm[:, 0].numpy(), u[:, 1])[0])
        acts[:, 1] = astar_act(cfg, s, obs, mm[:, 1], bm[:, 1], 1, ub)
        _, done, _ = sim.step(acts, auto_reset=True)
        keep = (~done.bool()).float().view(-1, 1)
        state["hidden"] = (hid[0] * keep, hid[1] * keep)

    env_step(0)
    ticks, t0 = 0, time.perf_counter()
    while True:
        env_step(1 + ticks)
        ticks += 1
        el = time.perf_counter() - t0
        if el >= budget_s or ticks >= 128:
            break
    return {"value": n * ticks / el, "unit": "env-steps/s", "cores": cores, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": f"oracle (torch CPU restatement) lstm-learner-vs-astar env-step, {n} envs x "
                      f"{ticks} timed ticks after 1 warm-up tick, {el:.1f} s"}


def main_lstm(args, torch, dev):
    """The lstm arch's collect loop: player 0 = the lstm network (local
    features, LSTM state carried and zeroed on done, masked sampling),
    player 1 = the astar bot; tick with auto-reset.  Four launches per step
    plus the bot's reach reduction.  `torch_gpu_baseline` times the
    reference's act() for player 0 with the same network as float32 eager
    torch modules (MIOpen convolutions, MIOpen LSTM) on the same GPU and
    features."""
    from qqtsim.bots import HipAstarBot
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.policy import HipLstmActorCritic, reference_init
    from qqtsim.rollout import LstmRollout
    from qqtsim.sim import HipBatchedSim

    n, K, W = args.envs, args.steps, args.warmup
    cfg = corridor_training_config()
    spec = MapSpec(kind="pillars", brick_p=0.7, swap_spawns=True)
    sim = HipBatchedSim(cfg, n, device=dev, seed=args.seed, map_spec=spec)
    sd = reference_init(cfg.obs_shape, seed=args.seed, arch="lstm")
    net = HipLstmActorCritic(sd, device=dev, seed=args.seed)
    roll = LstmRollout(sim, net, HipAstarBot(sim, pid=1))
    for _ in range(W):
        roll.step()
    torch.cuda.synchronize()
    _capi.timing_arm(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        if sampled(k, K):
            _capi.timing_arm(5)          # features, act, bot reach, bot, tick
        roll.step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    kms = kernel_ms()
    us = {k: v * 1e3 for k, v in kms.items()}
    bot_us = us["bot_kernel"] + us.get("reach_kernel", 0.0)
    kernels = {
        "lstm_act_kernel": {"us": us["lstm_act_kernel"], "bound": "mfma",
                            "achieved": LSTM_FLOP_PER_ROW * n / (us["lstm_act_kernel"] * 1e-6)
                            / 1e12,
                            "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "flop_per_row": LSTM_FLOP_PER_ROW,
                            "executed_tflops": 2 * LSTM_ISSUED_MACS * n
                            / (us["lstm_act_kernel"] * 1e-6) / 1e12,
                            "f32_equivalent_frac": LSTM_FLOP_PER_ROW * n
                            / (us["lstm_act_kernel"] * 1e-6) / 1e12 / MFMA_F32_PEAK},
        "lstm_feat_kernel": {"us": us["lstm_feat_kernel"], "bound": "hbm",
                             "achieved": LSTM_FEAT_BYTES_PER_ENV * n
                             / (us["lstm_feat_kernel"] * 1e-6) / 1e9,
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "bytes_per_env": LSTM_FEAT_BYTES_PER_ENV},
        "bot_kernel": {"us": bot_us, "bound": "hbm",
                       "achieved": BOT_BYTES_PER_ENV * n / (bot_us * 1e-6) / 1e9,
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "bytes_per_env": BOT_BYTES_PER_ENV},
        "tick_kernel": {"us": us["tick_kernel"], "bound": "hbm",
                        "achieved": TICK_BYTES_PER_ENV * n / (us["tick_kernel"] * 1e-6) / 1e9,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "bytes_per_env": TICK_BYTES_PER_ENV},
    }
    for v in kernels.values():
        v["frac"] = v["achieved"] / v["peak"]
    d = kernels["lstm_act_kernel"]

    # the reference's act() for player 0, eager float32 torch on this GPU
    ref = _torch_lstm(torch, sd, dev)
    loc, rel, glb = (x[:, 0].clone() for x in sim.local_view_features(only_p0=True))
    mm, bm = (m[:, 0].bool().clone() for m in sim.legal_mask())
    hid = (roll.h[None].clone(), roll.c[None].clone())
    for _ in range(3):
        ref.act(loc, rel, glb, mm, bm, hid)
    torch.cuda.synchronize()
    reps = 10
    t1 = time.perf_counter()
    for _ in range(reps):
        ref.act(loc, rel, glb, mm, bm, hid)
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t1) / reps * 1e3
    hip_ms = us["lstm_act_kernel"] * 1e-3

    cpu = cpu_baseline_lstm(cfg, spec, 256, args.seed, args.cpu_seconds) \
        if args.cpu_seconds > 0 else None
    out = {
        "metric": "env-steps/s at 5632 envs, lstm learner vs astar bot "
                  "(step+obs+features+lstm act+bot), 1 MI355X",
        "value": n * K / el, "unit": "env-steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": el / K * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 sim and bot; network as float16 MFMA products of hi/lo-split float32 "
                 "operands (f32 accumulate, float32 accuracy); f16 features",
        "data": "synthetic: template maps from Philox draws, the reference's lstm init "
                "(orthogonal, torch.nn.LSTM uniform)",
        "config": {"workload": "lstm learner (player 0: 7x7 local features + LSTM, state "
                               "carried) vs astar bot (player 1), 5632 envs, 13x13 pillars "
                               "+ 70% bricks, auto-reset",
                   "envs": n, "parallelism": "single GPU"},
        "roofline": {"kernel": "lstm_act_kernel", "bound": d["bound"],
                     "achieved": round(d["achieved"], 3), "peak": d["peak"], "unit": d["unit"],
                     "frac": round(d["frac"], 5), "traffic": None,
                     "note": "algorithmic FLOP of the reference network over the dense float16 "
                             "MFMA peak (the products run there, three per float32-accurate "
                             "product); executed_tflops and f32_equivalent_frac in kernels"},
        "torch_gpu_baseline": {"act_ms_player0": round(ref_ms, 3),
                               "hip_act_ms_player0": round(hip_ms, 4),
                               "speedup": round(ref_ms / hip_ms, 2),
                               "note": "the reference's act() (extract_fused, nn.LSTM step, "
                                       "heads, masked Categorical sampling), float32 eager "
                                       "torch, same features and state"},
        "cpu_baseline": cpu,
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in kernels.items()},
    }
    print(json.dumps(out), flush=True)

if __name__ == "__main__":
    main()
