"""The lstm arch on the GPU: qqt_lstm_features and qqt_lstm_act against
the reference's vectors and the oracle, and the lstm collect loop.

Bars: features bit for bit (float16) against the oracle's
local_view_features (the tie rule of ascending cell index) and, against the
reference's own vectors (tests/golden/lstm.npz), bit for bit except the
order of bombs at equal distance; logits, values and the LSTM state within
1e-4 absolute of the reference's float32 forward (the kernel computes in
float32 on MFMA in another summation order); sampled actions bit-exact
against the host sampler on the kernel's own logits with the same uniforms
(injected or Philox), logp within 1e-6; the collect loop's buffer equal to
a step-by-step replay through the public API.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from golden_io import GOLDEN, check_features, lstm_params

pytestmark = pytest.mark.gpu

# Logits, values and (h, c) against the reference module / the float64 oracle:
# the products run as float16 hi/lo splits with float32 accumulation (a few
# 1e-6 measured); the bound is a few times that, tight enough that dropping
# one cross product of a split (~5e-4 relative) fails.
ATOL = 2e-5
LOGP_ATOL = 4e-5


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.set_num_threads(16)
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def z():
    return np.load(os.path.join(GOLDEN, "lstm.npz"))


def _bits(t):
    return t.cpu().numpy().view(np.uint16)


def _oracle_features(sim, only_p0):
    from oracle.obs import local_view_features

    s = sim.state_dict()
    obs = sim.observe().cpu()
    return local_view_features(sim.cfg, obs, s["pos"].cpu(), s["alive"].cpu(), s["t"].cpu(),
                               s["fuse"].cpu(), s["hp"].cpu(), only_p0=only_p0)


def test_lstm_features_match_reference_golden(dev, z):
    """The reference's local_view_features on 12 bomb-rich frames, loaded
    into the sim's state (positions, life, hp, fuses, t) and observation."""
    from qqtsim import HipBatchedSim, corridor_training_config
    from oracle.obs import local_view_features

    cfg = corridor_training_config()
    n = z["obs"].shape[1]
    sim = HipBatchedSim(cfg, n, device=dev, seed=1)
    for i in range(z["obs"].shape[0]):
        print(f"[lstm] golden features frame {i}", flush=True)
        snap = {k: torch.from_numpy(z[k][i]) for k in ("pos", "alive", "hp", "fuse", "t")}
        sim.load_state_dict(snap)
        sim._obs.copy_(torch.from_numpy(z["obs"][i]))
        sim._fresh = True
        args = [torch.from_numpy(z[k][i]) for k in ("obs", "pos", "alive", "t", "fuse", "hp")]
        for only, sfx in ((False, ""), (True, "0")):
            got = sim.local_view_features(only_p0=only)
            check_features([z[k + sfx][i] for k in ("local", "rel", "glob")],
                           [t.cpu().numpy() for t in got])
            want = local_view_features(cfg, *args, only_p0=only)
            for g, w in zip(got, want):
                np.testing.assert_array_equal(_bits(g), w.numpy().view(np.uint16))


def test_lstm_features_match_oracle_5632(dev):
    """Bomb-stress states at 5632 envs (5-tick fuse, caps up to 4 bombs):
    both feature layouts, and the strided `out=` path of a buffer slot."""
    from qqtsim import BOMB_STRESS_40, HipBatchedSim, corridor_training_config
    from qqtsim.rollout import TickLoop

    n, seed = 5632, 4
    cfg = corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=12)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=BOMB_STRESS_40)
    loop = TickLoop(sim)
    g = torch.Generator().manual_seed(seed)
    slab = [torch.zeros((3, n) + s, dtype=torch.float16, device=dev)
            for s in ((1, 14, 7, 7), (1, 10, 6), (1, 5))]
    bombs = 0
    for t in range(10):
        mv = torch.randint(0, 5, (n, 2), generator=g)
        bb = (torch.rand((n, 2), generator=g) < 0.5).long()
        loop.launch_tick(torch.stack([mv, bb], -1).to(torch.int8).to(dev).contiguous())
        if t % 3 != 2:
            continue
        print(f"[lstm] features n={n} tick {t}", flush=True)
        bombs += int((sim.state_dict()["fuse"] > 0).sum())
        for only in (False, True):
            got = sim.local_view_features(only_p0=only)
            want = _oracle_features(sim, only)
            for a, b in zip(got, want):
                np.testing.assert_array_equal(_bits(a), b.numpy().view(np.uint16))
        out = sim.local_view_features(only_p0=True, out=tuple(s[1] for s in slab))
        assert all(o.data_ptr() == s[1].data_ptr() for o, s in zip(out, slab))
        for a, b in zip(out, want):
            np.testing.assert_array_equal(_bits(a), b.numpy().view(np.uint16))
        assert all(not s[0].any() and not s[2].any() for s in slab)
    assert bombs > n


def test_lstm_forward_matches_reference_sequence(dev, z):
    """The reference's lstm ActorCritic over 12 frames as sequences, hidden
    carried and zeroed after the flagged frames; evaluate()'s logp and
    entropy of the recorded actions."""
    from qqtsim import HipLstmActorCritic

    net = HipLstmActorCritic(lstm_params(z), device=dev)
    assert net.n_params() == int(z["param_count"]) == 368816
    hidden, worst = None, 0.0
    for i in range(z["local0"].shape[0]):
        f = tuple(torch.from_numpy(z[k][i][:, 0]).to(dev) for k in ("local0", "rel0", "glob0"))
        mm = torch.from_numpy(z["mm"][i][:, 0]).to(dev)
        bm = torch.from_numpy(z["bm"][i][:, 0]).to(dev)
        lp, ent, _ = net.evaluate(f, mm, bm, torch.from_numpy(z["actions"][i]).to(dev), 0, hidden)
        ml, bl, v, hidden = net.forward(f, 0, hidden)
        for got, key in ((ml, "move_logits"), (bl, "bomb_logits"), (v, "value"),
                         (hidden[0][0], "h"), (hidden[1][0], "c")):
            worst = max(worst, float(np.abs(got.cpu().numpy() - z[key][i]).max()))
        np.testing.assert_allclose(lp.cpu().numpy(), z["logp"][i], atol=LOGP_ATOL, rtol=0)
        np.testing.assert_allclose(ent.cpu().numpy(), z["entropy"][i], atol=LOGP_ATOL, rtol=0)
        keep = (~torch.from_numpy(z["reset"][i])).float().to(dev).view(1, -1, 1)
        hidden = (hidden[0] * keep, hidden[1] * keep)
    print(f"lstm sequence: max |err| {worst:.2e}")
    assert worst <= ATOL


def _random_features(b, seed, dev):
    g = torch.Generator().manual_seed(seed)
    local = (torch.rand((b, 14, 7, 7), generator=g) < 0.3).half()
    rel = (torch.randn((b, 10, 6), generator=g) * 3).round().half()
    glob = torch.rand((b, 5), generator=g).half()
    hidden = tuple(torch.randn((1, b, 128), generator=g) * 0.5 for _ in range(2))
    return (local.to(dev), rel.to(dev), glob.to(dev)), tuple(h.to(dev) for h in hidden)


def test_lstm_forward_matches_oracle_default_init(dev):
    """PyTorch default init, random features and state (ragged batch of
    1001 rows), against the oracle in float64."""
    from oracle.policy import lstm_forward
    from qqtsim import HipLstmActorCritic
    from qqtsim.policy import _layer_tree, _tree_state

    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(7)
        params = _tree_state(_layer_tree("lstm", (14, 13, 13), 5, 2))
    net = HipLstmActorCritic(params, device=dev)
    f, hid = _random_features(1001, 3, dev)
    ml, bl, v, (h, c) = net.forward(f, 0, hid)
    rml, rbl, rv, (rh, rc) = lstm_forward(params, *(t.cpu() for t in f),
                                          tuple(t[0].cpu() for t in hid), dtype=torch.float64)
    worst = 0.0
    for a, b in ((ml, rml), (bl, rbl), (v, rv), (h[0], rh), (c[0], rc)):
        worst = max(worst, float((a.cpu().double() - b).abs().max()))
    print(f"lstm default init: max |err| {worst:.2e}")
    assert worst <= ATOL
    # rows are independent: a prefix of the batch gives the same outputs
    ml2, _, v2, (h2, _) = net.forward(tuple(t[:37] for t in f), 0, tuple(t[:, :37] for t in hid))
    assert torch.equal(ml2, ml[:37]) and torch.equal(v2, v[:37]) and torch.equal(h2, h[:, :37])


def test_lstm_sampling_bit_exact_given_logits(dev):
    """Same logits, masks and uniforms -> same actions as the host sampler,
    including all-masked rows and the uniforms' end points."""
    from oracle.policy import sample_masked
    from qqtsim import HipLstmActorCritic

    net = HipLstmActorCritic(device=dev, seed=3)
    b = 700
    f, hid = _random_features(b, 5, dev)
    g = torch.Generator().manual_seed(0)
    mm = torch.rand((b, 5), generator=g) < 0.6
    bm = torch.rand((b, 2), generator=g) < 0.6
    mm[:, 4] |= torch.rand(b, generator=g) < 0.5
    mm[:5] = False
    u = torch.rand((b, 2), generator=g)
    u[5:12] = torch.tensor([0.0, 1.0 - 2 ** -24])
    acts, logp, val, (h, c) = net.act(f, mm.to(dev), bm.to(dev), 0, hid, uniforms=u.to(dev))
    ml, bl, v, (h2, c2) = net.forward(f, 0, hid)
    assert torch.equal(val, v) and torch.equal(h, h2) and torch.equal(c, c2)
    am, lpm = sample_masked(ml.cpu().numpy(), mm.numpy(), u[:, 0].numpy())
    ab, lpb = sample_masked(bl.cpu().numpy(), bm.numpy(), u[:, 1].numpy())
    np.testing.assert_array_equal(acts[:, 0].cpu().numpy(), am)
    np.testing.assert_array_equal(acts[:, 1].cpu().numpy(), ab)
    np.testing.assert_allclose(logp.cpu().numpy(), lpm + lpb, atol=1e-6, rtol=0)


def test_lstm_philox_draws_match_oracle_uniforms(dev):
    """Without injected uniforms the kernel draws Philox(seed, env, tick,
    policy stream) at player 0's slots, tick after tick."""
    from oracle import philox
    from oracle.policy import sample_masked
    from qqtsim import HipLstmActorCritic

    seed, b = 11, 512
    net = HipLstmActorCritic(device=dev, seed=seed)
    f, hid = _random_features(b, 9, dev)
    g = torch.Generator().manual_seed(2)
    mm = (torch.rand((b, 5), generator=g) < 0.7).to(dev)
    bm = (torch.rand((b, 2), generator=g) < 0.7).to(dev)
    rows = np.arange(b)
    for _ in range(3):
        u = philox.uniforms(seed, rows, net.tick, philox.STREAM_POLICY, 4)
        acts, _, _, _ = net.act(f, mm, bm, 0, hid)
        ml, bl, _, _ = net.forward(f, 0, hid)
        am, _ = sample_masked(ml.cpu().numpy(), mm.cpu().numpy(), u[:, 0])
        ab, _ = sample_masked(bl.cpu().numpy(), bm.cpu().numpy(), u[:, 1])
        np.testing.assert_array_equal(acts[:, 0].cpu().numpy(), am)
        np.testing.assert_array_equal(acts[:, 1].cpu().numpy(), ab)


def test_lstm_state_in_place_with_reset(dev):
    """The in-place state update with per-env reset flags equals the
    functional forward on the state zeroed for those envs."""
    from qqtsim import HipLstmActorCritic

    net = HipLstmActorCritic(device=dev, seed=2)
    b = 300
    f, (h0, c0) = _random_features(b, 1, dev)
    reset = (torch.arange(b) % 3 == 0).to(torch.uint8).to(dev)
    keep = (1 - reset.float()).view(1, -1, 1)
    ml, _, v, (h1, c1) = net.forward(f, 0, (h0 * keep, c0 * keep))
    h, c = h0[0].clone(), c0[0].clone()
    flat = [t.reshape(b, -1) for t in f]
    a = net.args(*flat, h, c, reset=reset)
    lg = torch.empty((b, 8), dtype=torch.float32, device=dev)
    a.logits_out = lg.data_ptr()
    net.launch(a)
    assert torch.equal(lg[:, :5], ml) and torch.equal(lg[:, 7], v)
    assert torch.equal(h, h1[0]) and torch.equal(c, c1[0])


def _setup_rollout(dev, n, seed, cfg=None):
    from qqtsim import (HipAstarBot, HipBatchedSim, HipLstmActorCritic, LstmRollout, MapSpec,
                        corridor_training_config)

    cfg = cfg or corridor_training_config(fuse=5, max_hp=2, invuln_ticks=3, max_steps=10)
    spec = MapSpec(kind="pillars", brick_p=0.5, swap_spawns=True)
    sim = HipBatchedSim(cfg, n, device=dev, seed=seed, map_spec=spec)
    net = HipLstmActorCritic(device=dev, seed=seed)
    roll = LstmRollout(sim, net, HipAstarBot(sim, pid=1))
    return sim, net, roll


def test_lstm_rollout_matches_the_public_api(dev):
    """LstmRollout.step against a replay on a twin sim through the public
    API (local_view_features(only_p0), act with the hidden state zeroed for
    envs done at the last tick, the astar bot, step)."""
    from qqtsim import HipAstarBot, HipLstmActorCritic

    n, seed, T = 256, 17, 24
    sim, net, roll = _setup_rollout(dev, n, seed)
    twin, _, _ = _setup_rollout(dev, n, seed)
    ref = HipLstmActorCritic(device=dev, seed=seed)
    bot = HipAstarBot(twin, pid=1)
    hidden, done_any = None, 0
    for t in range(T):
        feats = twin.local_view_features(only_p0=True)
        f0 = tuple(x[:, 0] for x in feats)
        mm, bm = (m.clone() for m in twin.legal_mask())
        a0, lp, v, hidden = ref.act(f0, mm[:, 0], bm[:, 0], 0, hidden)
        acts = torch.zeros((n, 2, 2), dtype=torch.int64, device=dev)
        acts[:, 0] = a0
        acts[:, 1] = bot.act(twin.observe(), mm[:, 1], bm[:, 1], 1)
        _, done, _ = twin.step(acts)
        roll.step()
        assert torch.equal(roll.actions.long(), acts), t
        assert torch.equal(roll.logp[:, 0], lp) and torch.equal(roll.value[:, 0], v), t
        assert torch.equal(roll.h, hidden[0][0]) and torch.equal(roll.c, hidden[1][0]), t
        assert torch.equal(roll.done, done), t
        done_any += int(done.sum())
        dk = done.float().view(1, -1, 1)
        hidden = (hidden[0] * (1 - dk), hidden[1] * (1 - dk))
    assert done_any > 0


def test_lstm_collect_fills_the_buffer(dev):
    """LstmRollout.collect into an lstm HipRolloutBuffer equals T calls of
    step() on a twin (features, masks, actions, logp, values, rewards, done)
    with the recycle flush after the 4th step; last_value() equals the
    forward under the carried state."""
    from qqtsim import HipRolloutBuffer

    n, seed, T = 128, 5, 10
    sim, net, roll = _setup_rollout(dev, n, seed)
    twin, tnet, troll = _setup_rollout(dev, n, seed)
    buf = HipRolloutBuffer(T, n, sim.cfg.obs_shape, dev, arch="lstm")
    assert buf.obs.shape == (T, n, 14, 13, 13) and buf.local.shape == (T, n, 14, 7, 7)
    roll.collect(buf, flush_every=4)
    for k in range(T):
        f = twin.local_view_features(only_p0=True)
        mm, bm = (m.clone() for m in twin.legal_mask())
        troll.step()
        for a, b in ((buf.local[k], f[0][:, 0]), (buf.rel[k], f[1][:, 0]),
                     (buf.glob[k], f[2][:, 0])):
            assert torch.equal(a, b), k
        assert torch.equal(buf.mmask[k], mm[:, 0]) and torch.equal(buf.bmask[k], bm[:, 0]), k
        assert torch.equal(buf.act[k], troll.actions[:, 0].long()), k
        assert torch.equal(buf.logp[k], troll.logp[:, 0]), k
        assert torch.equal(buf.val[k], troll.value[:, 0]), k
        assert torch.equal(buf.rew[k], twin._reward[:, 0]), k
        assert torch.equal(buf.done[k], twin._done.float()), k
        if k % 4 == 3 and k + 1 < T:
            twin.flush_recycle()
    twin.flush_recycle()
    assert torch.equal(roll.h, troll.h) and torch.equal(roll.c, troll.c)
    lv = roll.last_value()
    f = twin.local_view_features(only_p0=True)
    keep = (1 - twin._done.float()).view(1, -1, 1)
    _, _, v, _ = tnet.forward(tuple(x[:, 0] for x in f), 0,
                              (troll.h[None] * keep, troll.c[None] * keep))
    assert torch.equal(lv, v)
    assert torch.equal(roll.h, troll.h)


def test_lstm_large_batch_workgroup_shape(dev):
    """5000 rows take the 24-row workgroups (one round of the CUs), 300 rows
    the 16-row ones: both against the oracle in float64, and the rows they
    share equal bit for bit (the per-row arithmetic does not depend on the
    row's place in a workgroup)."""
    from oracle.policy import lstm_forward
    from qqtsim import HipLstmActorCritic

    net = HipLstmActorCritic(device=dev, seed=4)
    f, hid = _random_features(5000, 8, dev)
    ml, bl, v, (h, c) = net.forward(f, 0, hid)
    sub = slice(2000, 2300)
    ml2, bl2, v2, (h2, c2) = net.forward(tuple(t[sub] for t in f), 0, tuple(t[:, sub] for t in hid))
    for x, y in ((ml[sub], ml2), (bl[sub], bl2), (v[sub], v2), (h[:, sub], h2), (c[:, sub], c2)):
        assert torch.equal(x, y)
    rml, rbl, rv, (rh, rc) = lstm_forward(net.state_dict(), *(t.cpu() for t in f),
                                          tuple(t[0].cpu() for t in hid), dtype=torch.float64)
    worst = 0.0
    for a, b in ((ml, rml), (bl, rbl), (v, rv), (h[0], rh), (c[0], rc)):
        worst = max(worst, float((a.cpu().double() - b).abs().max()))
    print(f"lstm 5000 rows: max |err| {worst:.2e}")
    assert worst <= ATOL


def test_lstm_large_activations_stay_finite(dev):
    """conv1 weights scaled so its activations pass float16's 65504: the
    saturating hi/lo split keeps every product finite (an unsaturated split
    gives hi = inf, lo = -inf and NaN outputs).  Past 65504 the remainder in
    lo keeps float16's 11 bits, so products lose accuracy (1.3% measured on
    the logits at activations near 1e5, against 4e-6 in range): finite, and
    within 5% of the float64 oracle."""
    from oracle.policy import lstm_forward
    from qqtsim import HipLstmActorCritic

    net = HipLstmActorCritic(device=dev, seed=4)
    params = {k: v.clone() for k, v in net.state_dict().items()}
    f, hid = _random_features(256, 9, dev)
    w = params["l_conv1.weight"]
    pre = torch.nn.functional.conv2d(f[0].cpu().float(), w, params["l_conv1.bias"], padding=1)
    scale = 100000.0 / float(pre.max())   # the largest activation after the ReLU near 1e5
    params["l_conv1.weight"] = w * scale
    params["l_conv1.bias"] = params["l_conv1.bias"] * scale
    big = HipLstmActorCritic(params, device=dev)
    ml, bl, v, (h, c) = big.forward(f, 0, hid)
    outs = (ml, bl, v, h, c)
    assert all(bool(torch.isfinite(t).all()) for t in outs)
    rml, rbl, rv, (rh, rc) = lstm_forward(params, *(t.cpu() for t in f),
                                          tuple(t[0].cpu() for t in hid), dtype=torch.float64)
    for a, b in ((ml, rml), (bl, rbl), (v, rv), (h[0], rh), (c[0], rc)):
        err = float(((a.cpu().double() - b).abs() / (b.abs() + 1.0)).max())
        assert err <= 5e-2, err
