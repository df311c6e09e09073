"""The PPO update's MFMA kernels (needs an MI355X): the first layer's weight
gradient `qqt_l1_grad` and its forward (`qqt_mlp_act` with `z1_out`), both
through the C ABI against float64 products of the same operands, then
`HipMlpActorCritic` against a float32 torch restatement of the reference's
mlp ActorCritic (train/model.py:121-256) on the reference's PPO loss
(train/ppo.py:408-421): outputs and every parameter gradient, and a full
`ppo_update` over a collected device buffer."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

K0 = 2366


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _obs(b, g, stride=K0):
    """Observation-like float16 rows: mostly 0/1 with fractions (exact in
    float16), in a buffer of the given row stride."""
    x = (torch.rand((b, stride), generator=g) < 0.2).float()
    x = x * torch.where(torch.rand((b, stride), generator=g) < 0.7, torch.ones(1),
                        torch.rand((b, stride), generator=g))
    return x.half()


def _l1_grad(dev, x16, dz1, scale=None):
    from qqtsim import _capi

    lib = _capi.lib()
    b = x16.shape[0]
    need = lib.qqt_l1_grad_workspace_floats(b, K0)
    ws = torch.empty(need, dtype=torch.float32, device=dev)
    out = torch.full((128, K0), float("nan"), dtype=torch.float32, device=dev)
    a = _capi.L1GradArgsC()
    a.batch, a.k0, a.obs_stride, a.workspace_floats = b, K0, x16.stride(0), need
    a.obs, a.dz1 = x16.data_ptr(), dz1.data_ptr()
    a.dz_scale = _capi.ptr(scale)
    a.workspace, a.dw0 = ws.data_ptr(), out.data_ptr()
    _capi.check(lib.qqt_l1_grad(a, _capi.stream_handle(dev)))
    return out


@pytest.mark.parametrize("b,stride,mag", [(1, K0, 1.0), (33, K0, 1e-6), (2049, K0 + 6, 3e3),
                                          (5000, K0, 1.0), (40001, K0, 1e-2)])
def test_l1_grad_matches_float64(dev, b, stride, mag):
    """dw0 = dz1^T x over ragged batches (partial chunks and steps), a
    strided observation buffer and dz1 magnitudes from 1e-6 to 3e3 (the
    power-of-two scale keeps the float16 split accurate)."""
    g = torch.Generator().manual_seed(b)
    xs = _obs(b, g, stride)
    x16 = xs.to(dev)[:, :K0]
    dz = (torch.randn((b, 128), generator=g) * mag).float()
    amax = float(dz.abs().max())
    scale = torch.tensor([2.0 ** (14 - math.ceil(math.log2(amax)))], device=dev)
    got = _l1_grad(dev, x16, dz.to(dev), scale).cpu().double()
    want = dz.double().T @ xs[:, :K0].double()
    err = float((got - want).abs().max()) / float(want.abs().max())
    assert err <= 1e-5, err


def test_l1_grad_planted_transpose_fails(dev):
    """A transposed operand pairing (dz1 rows against shifted rows) is far
    off: the check above is sensitive to row alignment."""
    g = torch.Generator().manual_seed(1)
    xs = _obs(96, g)
    dz = torch.randn((96, 128), generator=g)
    got = _l1_grad(dev, xs.to(dev), dz.to(dev)).cpu().double()
    wrong = dz.double().roll(1, 0).T @ xs.double()
    assert float((got - wrong).abs().max()) > 1e-2 * float(wrong.abs().max())


@pytest.mark.parametrize("b", [1, 63, 65, 1000, 70001])
def test_first_layer_forward(dev, b):
    """z1 = x W0[pid]^T + b0 with W0 rounded to float16: exact products and
    float32 sums (<= 2e-5 of the float64 value on float16 weights), and
    within 2e-3 of the float32 weights; both block sizes (70001 rows take
    two 64-row blocks per workgroup)."""
    from qqtsim.learn import HipMlpActorCritic
    from qqtsim.policy import column_permutation

    net = HipMlpActorCritic(device=dev)
    g = torch.Generator().manual_seed(b)
    xs = _obs(b, g)
    for pid in (0, 1):
        z = net._l1_forward(xs.to(dev), net.shared[0].weight, net.shared[0].bias, pid).cpu()
        w = net.shared[0].weight.detach().cpu()[:, column_permutation(pid, 2, 14, 169)]
        bias = net.shared[0].bias.detach().cpu().double()
        exact = xs.double() @ w.half().double().T + bias
        full = xs.double() @ w.double().T + bias
        assert float((z.double() - exact).abs().max()) <= 2e-5 * max(1.0, float(exact.abs().max()))
        assert float((z.double() - full).abs().max()) <= 2e-3


class RefMlp(torch.nn.Module):
    """float32 torch restatement of the reference's mlp ActorCritic forward
    and evaluate (train/model.py:140-153, 192-196, 215-256)."""

    def __init__(self, sd, w0_half=False):
        super().__init__()
        nn = torch.nn
        self.shared = nn.Sequential(nn.Linear(K0, 128), nn.LayerNorm(128), nn.ReLU(),
                                    nn.Linear(128, 128), nn.LayerNorm(128), nn.ReLU())
        self.move_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 5))
        self.bomb_head = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 2))
        self.critic = nn.Sequential(nn.Linear(128, 64), nn.ReLU(), nn.Linear(64, 1))
        self.load_state_dict(sd)
        self.w0_half = w0_half

    def forward(self, obs, pid):
        from qqtsim.policy import column_permutation

        x = obs.float().reshape(obs.shape[0], -1)
        w0 = self.shared[0].weight[:, column_permutation(pid, 2, 14, 169).to(obs.device)]
        if self.w0_half:
            w0 = w0 + (w0.half().float() - w0).detach()     # forward on float16 weights
        x = torch.nn.functional.linear(x, w0, self.shared[0].bias)
        x = self.shared[1:](x)
        return self.move_head(x), self.bomb_head(x), self.critic(x).squeeze(-1)

    def evaluate(self, obs, mm, bm, act, pid=0):
        ml, bl, v = self(obs, pid)
        neg = torch.finfo(torch.float32).min
        dm = torch.distributions.Categorical(logits=torch.where(mm, ml, torch.full_like(ml, neg)))
        db = torch.distributions.Categorical(logits=torch.where(bm, bl, torch.full_like(bl, neg)))
        return dm.log_prob(act[:, 0]) + db.log_prob(act[:, 1]), dm.entropy() + db.entropy(), v


def _ortho_init(seed):
    """The reference's ActorCritic init (train/model.py:154-165)."""
    from qqtsim.policy import reference_init

    return reference_init(seed=seed)


def _loss(net, obs, mm, bm, act, old_logp, adv, ret, old_val, pid):
    """The reference's clipped PPO loss (train/ppo.py:408-421)."""
    logp, ent, v = net.evaluate(obs, mm, bm, act, pid)
    ratio = (logp - old_logp).exp()
    pg = -torch.min(ratio * adv, ratio.clamp(0.8, 1.2) * adv).mean()
    vc = old_val + (v - old_val).clamp(-0.2, 0.2)
    vf = 0.5 * torch.max((v - ret) ** 2, (vc - ret) ** 2).mean()
    return pg + 0.5 * vf - 0.05 * ent.mean(), (logp, ent, v)


@pytest.mark.parametrize("pid", [0, 1])
def test_module_gradients_match_torch(dev, pid):
    from qqtsim.learn import HipMlpActorCritic

    sd = _ortho_init(7)
    net = HipMlpActorCritic(device=dev, state_dict=sd)
    g = torch.Generator().manual_seed(3)
    b = 3000
    obs = _obs(b, g).reshape(b, 14, 13, 13).to(dev)
    mm = (torch.rand((b, 5), generator=g) < 0.7).to(dev)
    mm[:, 4] = True
    bm = torch.ones((b, 2), dtype=torch.bool, device=dev)
    bm[:, 1] = (torch.rand(b, generator=g) < 0.5).to(dev)
    act = torch.stack([torch.multinomial(mm.float().cpu(), 1, generator=g)[:, 0],
                       torch.multinomial(bm.float().cpu(), 1, generator=g)[:, 0]], 1).to(dev)
    old_logp = (torch.randn(b, generator=g) * 0.1 - 2.0).to(dev)
    adv = torch.randn(b, generator=g).to(dev)
    ret = torch.randn(b, generator=g).to(dev)
    old_val = torch.randn(b, generator=g).to(dev)
    args = (obs, mm, bm, act, old_logp, adv, ret, old_val, pid)

    loss, (lp, ent, v) = _loss(net, *args)
    loss.backward()
    for w0_half, tol in ((True, 2e-4), (False, 3e-2)):
        ref = RefMlp(sd, w0_half).to(dev)
        rloss, (rlp, rent, rv) = _loss(ref, *args)
        rloss.backward()
        assert float((lp - rlp).abs().max()) <= (1e-4 if w0_half else 2e-3)
        assert float((v - rv).abs().max()) <= (1e-4 if w0_half else 2e-3)
        for (name, p), (_, q) in zip(net.named_parameters(), ref.named_parameters()):
            err = float((p.grad - q.grad).norm() / q.grad.norm().clamp_min(1e-12))
            assert err <= tol, (w0_half, name, err)


def test_ppo_update_runs_on_a_collected_buffer(dev):
    """ppo_update (train/ppo.py:364-437) over a 64 x 256 device buffer from
    Rollout.collect: finite statistics, every parameter moves, and the
    loss on the first minibatch falls."""
    from qqtsim import (HipActorCritic, HipBatchedSim, HipMlpActorCritic, HipRolloutBuffer,
                        MapSpec, PPOConfig, Rollout, corridor_training_config, ppo_update)

    cfg = corridor_training_config(max_steps=60)
    n, t = 256, 64
    sim = HipBatchedSim(cfg, n, device=dev, seed=1,
                        map_spec=MapSpec(kind="pillars", brick_p=0.5, bombs_cap=(2, 3)))
    sd = _ortho_init(2)
    actor = HipActorCritic(sd, device=dev, seed=1)
    roll = Rollout(sim, actor)
    buf = HipRolloutBuffer(t, n, cfg.obs_shape, dev)
    roll.collect(buf)
    learner = HipMlpActorCritic(device=dev, state_dict=sd)
    before = {k: v.detach().clone() for k, v in learner.state_dict().items()}
    opt = torch.optim.Adam(learner.parameters(), lr=3e-4)
    last_val = actor.forward(sim.observe(), 0)[2]
    torch.manual_seed(0)
    stats = ppo_update(learner, opt, buf, last_val, PPOConfig(), 0.05)
    assert all(np.isfinite(v) for v in stats.values()), stats
    after = learner.state_dict()
    for k, v in before.items():
        assert not torch.equal(v, after[k]), k


def test_fused_ppo_grads_match_autograd(dev):
    """qqt_ppo_grad (+ the first layer's kernels): every parameter gradient
    and the five statistics equal what loss.backward() through evaluate()
    gives on the same module (float32, summation order aside), on a ragged
    batch (3001 rows: the last 16-row block is partial) with masked moves,
    masked bombs, clipped and unclipped ratios and value errors."""
    from qqtsim.learn import HipMlpActorCritic, PPOConfig

    sd = _ortho_init(11)
    net = HipMlpActorCritic(device=dev, state_dict=sd)
    g = torch.Generator().manual_seed(5)
    b = 3001
    obs = _obs(b, g).reshape(b, 14, 13, 13).to(dev)
    mm = (torch.rand((b, 5), generator=g) < 0.6).to(dev)
    mm[:, 4] = True
    bm = torch.ones((b, 2), dtype=torch.bool, device=dev)
    bm[:, 1] = (torch.rand(b, generator=g) < 0.5).to(dev)
    act = torch.stack([torch.multinomial(mm.float().cpu(), 1, generator=g)[:, 0],
                       torch.multinomial(bm.float().cpu(), 1, generator=g)[:, 0]], 1).to(dev)
    with torch.no_grad():
        lp0, _, v0 = net.evaluate(obs, mm, bm, act)
    # old log-probs and values around the current ones: ratios and value
    # moves on both sides of the clip range
    old_logp = lp0 + (torch.randn(b, generator=g) * 0.3).to(dev)
    old_val = v0 + (torch.randn(b, generator=g) * 0.3).to(dev)
    adv = torch.randn(b, generator=g).to(dev)
    ret = old_val + torch.randn(b, generator=g).to(dev)
    cfg = PPOConfig()

    loss, (lp, ent, v) = _loss(net, obs, mm, bm, act, old_logp, adv, ret, old_val, 0)
    loss.backward()
    want = {k: p.grad.detach().clone() for k, p in net.named_parameters()}
    ratio = (lp - old_logp).exp()
    want_st = torch.stack([
        -torch.min(ratio * adv, ratio.clamp(0.8, 1.2) * adv).mean(),
        0.5 * torch.max((v - ret) ** 2, (old_val + (v - old_val).clamp(-0.2, 0.2) - ret) ** 2).mean(),
        ent.mean(), (old_logp - lp).mean(), ((ratio - 1).abs() > 0.2).float().mean()]).detach()
    clipped = float(((ratio - 1).abs() > 0.2).float().mean())
    assert 0.1 < clipped < 0.9, clipped
    net.zero_grad(set_to_none=True)
    st = net.ppo_grads(obs, mm, bm, act, old_logp, adv, ret, old_val, cfg, 0.05)
    for k, p in net.named_parameters():
        err = float((p.grad - want[k]).norm() / want[k].norm().clamp_min(1e-12))
        assert err <= 2e-4, (k, err)
    assert float((st - want_st).abs().max()) <= 1e-5 * max(1.0, float(want_st.abs().max()))


def test_gather_rows_matches_torch_indexing(dev):
    """qqt_gather_rows (the PPO minibatch's observation rows) equals torch's
    row indexing bit for bit, repeated and out-of-order indices included;
    rows with an index outside the source are left untouched."""
    from qqtsim import _capi
    from qqtsim.learn import _gather_rows

    g = torch.Generator().manual_seed(4)
    n, b = 3001, 2048
    x = (torch.randn((n, 14, 13, 13), generator=g) * 3).half().to(dev)
    idx = torch.randint(0, n, (b,), generator=g).to(dev)
    idx[:30] = idx[30]
    assert torch.equal(_gather_rows(x, idx), x[idx])
    out = torch.full((3, 1183), 7, dtype=torch.int32, device=dev)
    bad = torch.tensor([5, -1, n], dtype=torch.int64, device=dev)
    a = _capi.GatherArgsC()
    a.n, a.row_words, a.src_rows, a.src_stride, a.dst_stride = 3, 1183, n, 1183, 1183
    a.src, a.dst, a.index = x.data_ptr(), out.data_ptr(), bad.data_ptr()
    _capi.check(_capi.lib().qqt_gather_rows(a, _capi.stream_handle(dev)))
    assert torch.equal(out[0], x[5].reshape(-1).view(torch.int32))
    assert bool((out[1:] == 7).all())


@pytest.mark.parametrize("b", [3001, 70001])
def test_row_index_reads_equal_gathered_rows(dev, b):
    """Batch rows read in place through `row_index` (repeated and
    out-of-order indices, and two outside the buffer, which are clamped)
    give exactly what the gathered rows give: the policy forward of
    `qqt_mlp_act` (the act kernel at 3001 rows, the streaming forward at
    70001), the first layer's forward and weight gradient, and every
    gradient and statistic of the fused PPO minibatch (its masks, actions,
    log-probs, advantages, returns and values read by index too)."""
    from qqtsim import _capi
    from qqtsim.learn import HipMlpActorCritic, PPOConfig
    from qqtsim.policy import HipActorCritic

    sd = _ortho_init(3)
    g = torch.Generator().manual_seed(b)
    n = b + 917
    base = _obs(n, g).to(dev)
    idx = torch.randint(0, n, (b,), generator=g)
    idx[:40] = idx[40]
    idx[7], idx[b - 1] = -5, n + 3
    clamped = idx.clamp(0, n - 1)
    idx, clamped = idx.to(dev), clamped.to(dev)
    gathered = base[clamped].contiguous()

    # policy forward (logits and values)
    pol = HipActorCritic(sd, device=dev, seed=0)
    want = torch.empty((b, 1, 8), dtype=torch.float32, device=dev)
    pol._run(gathered, 1, 1, False, logits=want)
    got = torch.full((b, 1, 8), float("nan"), dtype=torch.float32, device=dev)
    a = pol._args(b, 1, 1, 0, base.data_ptr(), base.stride(0))
    a.logits_out, a.row_index, a.obs_rows = got.data_ptr(), idx.data_ptr(), n
    pol._launch(a, _capi.stream_handle(dev))
    assert torch.equal(got, want)

    # first layer forward and weight gradient
    net = HipMlpActorCritic(device=dev, state_dict=sd)
    w, bias = net.shared[0].weight, net.shared[0].bias
    assert torch.equal(net._l1_forward(base, w, bias, 0, idx), net._l1_forward(gathered, w, bias, 0))
    dz1 = torch.randn((b, 128), generator=g).to(dev)
    assert torch.equal(net._l1_weight_grad(base, dz1, 0, rows=idx),
                       net._l1_weight_grad(gathered, dz1, 0))

    # the fused minibatch: every per-row input of the whole buffer, read by index
    mm = (torch.rand((n, 5), generator=g) < 0.6).to(dev)
    mm[:, 4] = True
    bm = torch.ones((n, 2), dtype=torch.bool, device=dev)
    bm[:, 1] = (torch.rand(n, generator=g) < 0.5).to(dev)
    act = torch.stack([torch.multinomial(mm.float().cpu(), 1, generator=g)[:, 0],
                       torch.multinomial(bm.float().cpu(), 1, generator=g)[:, 0]], 1).to(dev)
    old_logp = (torch.randn(n, generator=g) * 0.3 - 2.0).to(dev)
    old_val, adv, ret = (torch.randn(n, generator=g).to(dev) for _ in range(3))
    per_row = (mm, bm, act, old_logp, adv, ret, old_val)
    cfg = PPOConfig()
    shape = (-1, 14, 13, 13)
    st_want = net.ppo_grads(gathered.reshape(shape), *(x[clamped] for x in per_row), cfg, 0.05)
    want_g = {k: p.grad.detach().clone() for k, p in net.named_parameters()}
    net.zero_grad(set_to_none=True)
    st_got = net.ppo_grads(base.reshape(shape), *per_row, cfg, 0.05, rows=idx)
    assert torch.equal(st_got, st_want)
    for k, p in net.named_parameters():
        assert torch.equal(p.grad, want_g[k]), k
