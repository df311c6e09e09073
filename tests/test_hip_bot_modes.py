"""HIP astar bot with behaviour modes (sim/bots.py:241-264, 433-443, 496-503;
needs an MI355X): the reference's flee-mode decisions reproduced bit for bit
given the modes, and the device mode ticker equal to the oracle's, call by
call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_io import GOLDEN

pytestmark = pytest.mark.gpu

KEYS = ("wall", "brick", "fuse", "owner", "pos", "alive", "blast_cap")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _sim_bot(dev, n, seed):
    from qqtsim import HipAstarBot, HipBatchedSim, MapSpec, corridor_training_config

    cfg = corridor_training_config()
    sim = HipBatchedSim(cfg, n, device=dev, seed=0, map_spec=MapSpec(kind="open"))
    return sim, HipAstarBot(sim, pid=1, seed=seed, mode=True)


def test_hip_bot_flee_mode_matches_reference_vectors(dev):
    """Per tick the fixture's approach / flee modes are given to the bot (timers
    far from 0, so this call's ticker step switches nothing) and its actions
    equal the reference's astar_attack with those modes."""
    z = np.load(f"{GOLDEN}/astar_flee.npz")
    sim, bot = _sim_bot(dev, z["bot"].shape[1], seed=3)
    for t in range(z["bot"].shape[0]):
        sim.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(z[k][t])) for k in KEYS})
        bot.modes.copy_(torch.from_numpy(z["mode"][t]))
        bot.mode_timers.fill_(1 << 30)
        got = bot.act(torch.from_numpy(z["obs"][t]), torch.from_numpy(z["mm1"][t]),
                      torch.from_numpy(z["bm1"][t]), 1, uniforms=torch.from_numpy(z["u"][t]))
        np.testing.assert_array_equal(got.cpu().numpy(), z["bot"][t], err_msg=f"tick {t}")


def test_hip_bot_mode_ticker_matches_oracle(dev):
    """40 calls from random modes and timers (some already due): after every
    call the device's modes and timers equal the oracle ticker's (the same
    Philox draws), switches happen, and the actions follow the new modes
    (the oracle bot with the ticker's modes)."""
    from oracle.bots import astar_act, mode_tick
    from qqtsim.config import corridor_training_config

    z = np.load(f"{GOLDEN}/astar_flee.npz")
    n, t0, seed = z["bot"].shape[1], 40, 77
    sim, bot = _sim_bot(dev, n, seed)
    st = {k: torch.from_numpy(np.ascontiguousarray(z[k][t0])) for k in KEYS}
    sim.load_state_dict(st)
    g = torch.Generator().manual_seed(1)
    mode = torch.randint(0, 2, (n,), generator=g, dtype=torch.int8)
    timer = torch.randint(-5, 40, (n,), generator=g, dtype=torch.int32)
    bot.modes.copy_(mode)
    bot.mode_timers.copy_(timer)
    inputs = (torch.from_numpy(z["obs"][t0]), torch.from_numpy(z["mm1"][t0]),
              torch.from_numpy(z["bm1"][t0]))
    u = torch.from_numpy(z["u"][t0])
    cfg = corridor_training_config()
    switched = 0
    for count in range(1, 41):
        got = bot.act(*inputs, 1, uniforms=u)
        m2, timer = mode_tick(mode, timer, count, seed)
        switched += int((m2 != mode).sum())
        mode = m2
        np.testing.assert_array_equal(bot.modes.cpu().numpy(), mode.numpy(), err_msg=f"call {count}")
        np.testing.assert_array_equal(bot.mode_timers.cpu().numpy(), timer.numpy(),
                                      err_msg=f"call {count}")
        want = astar_act(cfg, st, *inputs, 1, u, mode=mode.long())
        np.testing.assert_array_equal(got.cpu().numpy(), want.numpy(), err_msg=f"call {count}")
    assert switched > 0
