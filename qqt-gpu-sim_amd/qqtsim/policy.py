"""`HipActorCritic`: the reference's mlp `ActorCritic` on the MFMA kernel.

Drop-in for `train/model.py::ActorCritic` (arch "mlp", :54-259) on the
rollout path: `act(obs, move_mask, bomb_mask, pid)` -> (actions (B,2) int64,
logp (B,), value (B,)) and `forward(obs, pid)` -> (move logits (B,5), bomb
logits (B,2), value (B,)), plus `act_pair` which serves both players from one
pass over the shared observation (the collect loop's learner + self-play
opponent, train/ppo.py:213-249).

Weights come from an ActorCritic mlp state_dict (keys `shared.0.weight`, ...,
`critic.2.bias`) and are packed once into the kernel's layout: float16
matrices in MFMA B-fragment order (see qqt-gpu-sim_amd/csrc/mlp.hip) with each
player's view permutation folded into the first layer (train/model.py:121-139),
float32 bias / LayerNorm vectors.

Sampling replaces `Categorical.sample` (torch.multinomial, which cannot take
injected randomness) with an inverse-CDF draw on uniforms: given the same
logits, masks and uniforms it is reproducible bit for bit on the host.  The
uniforms come from Philox(seed, row, tick) unless passed explicitly.
"""

from __future__ import annotations

import math

import torch

from . import _capi
from .config import n_obs_channels, view_perm

KBLOCK = 64
HID = 128
HEAD = 64
LSTM_HIDDEN = 128          # train/model.py LSTM_HIDDEN
LSTM_MAX_T = 10            # rel target slots (sim/obs.py MAX_T)
LSTM_GLOB = 5              # global scalars (sim/obs.py GLOB_FEAT)


def column_permutation(pid: int, p: int, c: int, hw: int) -> torch.Tensor:
    """First-layer columns of player `pid`'s view: block k of the permuted
    weight is block argsort(view_perm)[k] of the original."""
    inv = torch.argsort(torch.tensor(view_perm(pid, p, c)))
    return (inv.view(c, 1) * hw + torch.arange(hw).view(1, hw)).reshape(-1)


def _frag(w: torch.Tensor, kpad: int, residual: bool = False) -> torch.Tensor:
    """(n_out, k) float matrix -> float16 B fragments [tile][kblock][lane][16]
    (of w itself, or of its float16 residual w - float16(w)), on w's
    device."""
    n, k = w.shape
    assert n % 16 == 0
    out = torch.zeros((n, kpad), dtype=torch.float32, device=w.device)
    out[:, :k] = w.float()
    if residual:
        out = out - out.half().float()
    kb = kpad // KBLOCK
    f = out.view(n // 16, 16, kb, 4, 16).permute(0, 2, 3, 1, 4).contiguous()
    return f.half().reshape(-1)


# K order of one 32-deep step of the later layers: MFMA K index 8q + i
# (lane group q, element i) reads input feature 32 s + CHAIN_KPERM[8q + i],
# the order in which the previous product's output tiles 2s, 2s+1 sit in a
# lane (features 4q..4q+3 of each).
CHAIN_KPERM = [4 * q + i if i < 4 else 16 + 4 * q + (i - 4) for q in range(4) for i in range(8)]


def _chain_frag(w: torch.Tensor, residual: bool = False) -> torch.Tensor:
    """(n_out, k) float matrix (n_out % 16 == 0, k % 32 == 0) -> float16 A
    fragments [tile][kstep][lane][8] = W[16 tile + lane%16][32 kstep +
    CHAIN_KPERM[8 (lane/16) + i]] (of w itself, or of its float16 residual)."""
    n, k = w.shape
    assert n % 16 == 0 and k % 32 == 0
    out = w.float()
    if residual:
        out = out - out.half().float()
    perm = torch.tensor(CHAIN_KPERM, device=w.device)
    f = out.reshape(n // 16, 16, k // 32, 32)[..., perm]           # [tile][r][s][8q + i]
    f = f.reshape(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()
    return f.half().reshape(-1)                                     # [tile][s][16q + r][i]


def pack_mlp(params: dict, n_players: int = 2, obs_shape=(14, 13, 13)) -> dict:
    """Packing of an ActorCritic mlp state_dict into the kernel's operand
    layout, on the device the weights live on."""
    c, h, w = obs_shape
    hw = h * w
    k0 = c * hw
    kpad = math.ceil(k0 / KBLOCK) * KBLOCK
    W0 = params["shared.0.weight"].float()
    dev = W0.device
    if W0.shape != (HID, k0):
        raise ValueError(f"shared.0.weight must be {(HID, k0)}, got {tuple(W0.shape)}")
    per_pid = [W0[:, column_permutation(pid, n_players, c, hw).to(dev)]
               for pid in range(n_players)]
    w0 = torch.cat([_frag(wp, kpad) for wp in per_pid])
    w1_src = params["shared.3.weight"].to(dev)
    w1, w1_lo = _chain_frag(w1_src), _chain_frag(w1_src, True)
    heads = ("move_head", "bomb_head", "critic")
    wh_src = torch.cat([params[f"{n}.0.weight"].to(dev).float() for n in heads])
    wh, wh_lo = _chain_frag(wh_src), _chain_frag(wh_src, True)
    wfin = torch.zeros((16, 3 * HEAD), dtype=torch.float32, device=dev)
    outs = [params[f"{n}.2.weight"].to(dev).float() for n in heads]
    row = 0
    for i, o in enumerate(outs):
        wfin[row:row + o.shape[0], i * HEAD:(i + 1) * HEAD] = o
        row += o.shape[0]
    if row != 8:
        raise ValueError("heads must produce 5 + 2 + 1 outputs")
    wf, wf_lo = _chain_frag(wfin), _chain_frag(wfin, True)
    vec = lambda k: params[k].to(dev).float().contiguous()  # noqa: E731
    w0g, w0d = _sparse_tables(W0, c, hw)
    vmap = [torch.argsort(torch.tensor(view_perm(pid, n_players, c))).tolist()
            for pid in range(n_players)]
    return dict(
        w0=w0, w1=w1, wh=wh, wf=wf, w1_lo=w1_lo, wh_lo=wh_lo, wf_lo=wf_lo, w0g=w0g, w0d=w0d,
        b0=vec("shared.0.bias"), ln1_w=vec("shared.1.weight"), ln1_b=vec("shared.1.bias"),
        b1=vec("shared.3.bias"), ln2_w=vec("shared.4.weight"), ln2_b=vec("shared.4.bias"),
        bh=torch.cat([vec(f"{n}.0.bias") for n in heads]),
        bf=torch.cat([vec(f"{n}.2.bias") for n in heads]),
        k0=k0, kblocks0=kpad // KBLOCK,
        # dense channels: wall | brick and the progress t / max_steps (sim/obs.py:88-101)
        sparse_info=dict(channels=c, cells=hw, vmap=vmap,
                         dense_mask=(1 << (2 * n_players)) | (1 << (2 * n_players + 2))))


def _sparse_tables(W0: torch.Tensor, c: int, hw: int):
    """Operands of the sparse first layer (csrc/mlp_sparse.hip) from the
    (128, c * hw) weight in the network's own input order: the float16
    gather table [k0][128] (row k = W0[:, k]) and the dense channels' MFMA A
    fragments [c][8 tiles][ceil(hw/32)][2 planes][64 lanes][8], lane (r, g)
    = (lane % 16, lane / 16) holding W0[16 tile + r][j hw + 32 s + 8 g + i]
    (0 past the channel), plane 0 float16(w) and plane 1 float16(w - plane
    0)."""
    dev = W0.device
    tab = W0.t().contiguous().half()
    ksc = -(-hw // 32)
    wpad = torch.zeros((HID, c, ksc * 32), dtype=torch.float32, device=dev)
    wpad[:, :, :hw] = W0.float().reshape(HID, c, hw)
    hi = wpad.half()
    lo = (wpad - hi.float()).half()

    def frag(x):   # (128, c, 32 ksc) -> [c][tile][s][64 lanes][8]
        return x.reshape(8, 16, c, ksc, 4, 8).permute(2, 0, 3, 4, 1, 5).reshape(c, 8, ksc, 64, 8)

    w0d = torch.stack([frag(hi), frag(lo)], dim=3).contiguous().reshape(-1)
    return tab.reshape(-1), w0d


def _layer_tree(arch: str, obs_shape, n_moves: int, n_bomb: int) -> torch.nn.Module:
    """The ActorCritic layers of `arch` as plain torch modules, created (and
    so drawing their PyTorch default init) in the reference's registration
    order: the cnn trunk `conv0`, `conv` (train/model.py:76-93) or the lstm
    arch's `l_conv1` .. `l_fusion`, `lstm` (:103-120; nn.LSTM draws its own
    uniform init when built), then `shared` (not for lstm), `move_head`,
    `bomb_head`, `critic` (:140-153)."""
    c, h, w = obs_shape
    nn = torch.nn
    tree = nn.Module()
    if arch == "cnn":
        tree.conv0 = nn.Conv2d(c, 16, 3, padding=1)
        tree.conv = nn.Sequential(
            nn.LayerNorm([16, h, w]), nn.ReLU(), nn.Conv2d(16, 32, 3, padding=1),
            nn.LayerNorm([32, h, w]), nn.ReLU(), nn.Conv2d(32, 64, 3, padding=1),
            nn.LayerNorm([64, h, w]), nn.ReLU(), nn.Conv2d(64, 8, 1),
            nn.LayerNorm([8, h, w]), nn.ReLU())
        flat = 8 * h * w
    elif arch == "lstm":
        tree.l_conv1 = nn.Conv2d(c, 32, 3, padding=1)
        tree.l_conv2 = nn.Conv2d(32, 64, 3, padding=1)
        tree.l_cnn_fc = nn.Linear(64 * 3 * 3, HID)
        tree.l_rel_fc1 = nn.Linear(LSTM_MAX_T * 6, 64)
        tree.l_rel_fc2 = nn.Linear(64, 32)
        tree.l_glob_fc1 = nn.Linear(LSTM_GLOB, 16)
        tree.l_glob_fc2 = nn.Linear(16, 8)
        tree.l_fusion = nn.Linear(HID + 32 + 8, 256)
        tree.lstm = nn.LSTM(256, LSTM_HIDDEN, 1, batch_first=True)
    elif arch == "mlp":
        flat = c * h * w
    else:
        raise ValueError(f"no layer tree for arch {arch!r}")
    if arch != "lstm":
        tree.shared = nn.Sequential(nn.Linear(flat, HID), nn.LayerNorm(HID), nn.ReLU(),
                                    nn.Linear(HID, HID), nn.LayerNorm(HID), nn.ReLU())
    tree.move_head = nn.Sequential(nn.Linear(HID, HEAD), nn.ReLU(), nn.Linear(HEAD, n_moves))
    tree.bomb_head = nn.Sequential(nn.Linear(HID, HEAD), nn.ReLU(), nn.Linear(HEAD, n_bomb))
    tree.critic = nn.Sequential(nn.Linear(HID, HEAD), nn.ReLU(), nn.Linear(HEAD, 1))
    return tree


def _tree_state(tree: torch.nn.Module) -> dict:
    return {k: v.detach().clone() for k, v in tree.state_dict().items()}


def default_init(obs_shape=(14, 13, 13), n_moves: int = 5, n_bomb: int = 2,
                 seed: int = 0) -> dict:
    """PyTorch default init of the mlp ActorCritic layers (nn.Linear
    kaiming-uniform(a=sqrt(5)) weights, U(+-1/sqrt(fan_in)) biases, LayerNorm
    1/0) under torch.manual_seed(seed), layers created in module order
    (train/model.py:140-153).  The global RNG state is restored afterwards.
    This is not what the reference's ActorCritic holds after construction
    (see `reference_init`); benchmark workloads that name PyTorch default
    init use it."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        return _tree_state(_layer_tree("mlp", obs_shape, n_moves, n_bomb))


def reference_init(obs_shape=(14, 13, 13), n_moves: int = 5, n_bomb: int = 2,
                   seed: int = 0, arch: str = "mlp") -> dict:
    """The weights `torch.manual_seed(seed); ActorCritic(obs_shape, arch=arch)`
    holds (train/model.py:154-165): every Conv2d / Linear weight orthogonal
    with gain sqrt(2) and its bias zero, visited in module order after all
    layers were created, then the move and bomb heads' output weights drawn
    again orthogonal with gain 0.01 (biases zero); LayerNorm 1 / 0.  The
    random draws follow the reference's order, so the result equals the
    reference module's state_dict bit for bit.  The global RNG state is
    restored afterwards."""
    nn = torch.nn
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        tree = _layer_tree(arch, obs_shape, n_moves, n_bomb)
        with torch.no_grad():
            for mod in tree.modules():
                if isinstance(mod, (nn.Conv2d, nn.Linear)):
                    nn.init.orthogonal_(mod.weight, gain=2 ** 0.5)
                    nn.init.zeros_(mod.bias)
            for head in (tree.move_head, tree.bomb_head):
                nn.init.orthogonal_(head[-1].weight, gain=0.01)
                nn.init.zeros_(head[-1].bias)
        return _tree_state(tree)


class HipActorCritic:
    arch = "mlp"

    def __init__(self, state_dict: dict | None = None, obs_shape=(14, 13, 13),
                 n_players: int = 2, device="cuda", seed: int = 0, sparse: bool = False):
        self.obs_shape = tuple(obs_shape)
        # sparse=True: the first layer over the observation's nonzero cells
        # (csrc/mlp_sparse.hip) where the launch qualifies: logits within
        # ~4e-5 of float32 instead of ~4e-4, at 30 us instead of 23 us per
        # 5632-row pair launch on MI355X
        self.sparse = bool(sparse)
        self.n_players = n_players
        if n_obs_channels(n_players) != self.obs_shape[0]:
            raise ValueError("observation channels do not match n_players")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HipActorCritic runs on a ROCm device")
        self.seed = int(seed)
        self.tick = 0
        self._lib = _capi.lib()
        self._w = None
        self.load_state_dict(state_dict if state_dict is not None
                             else reference_init(obs_shape, seed=0, arch=self.arch))

    def _pack(self, params: dict) -> dict:
        packed = pack_mlp(params, self.n_players, self.obs_shape)
        self.k0, self.kblocks0 = packed.pop("k0"), packed.pop("kblocks0")
        self._sparse_info = packed.pop("sparse_info")
        return packed

    def load_state_dict(self, state_dict: dict) -> None:
        """Repack the weights (on the device) and copy them over the packed
        buffers in place.  Argument blocks built before (a `Rollout`'s) keep
        the buffers' addresses, so they stay valid and the next launch uses
        the new weights; the copies are ordered on the current stream."""
        params = {k: v.detach().to(self.device, torch.float32).clone()
                  for k, v in state_dict.items()}
        packed = self._pack(params)
        if self._w is None:
            self._w = {k: v.to(self.device).contiguous() for k, v in packed.items()}
        else:
            if set(packed) != set(self._w) or any(
                    packed[k].shape != self._w[k].shape for k in packed):
                raise ValueError("state_dict does not match the network's layer shapes")
            for k, v in packed.items():
                self._w[k].copy_(v)
        self.params = params

    def state_dict(self) -> dict:
        """The float32 weights last loaded, under the reference's keys."""
        return {k: v.clone() for k, v in self.params.items()}

    def n_params(self) -> int:
        return sum(v.numel() for v in self.params.values())

    # ------------------------------------------------------------ launch
    def _args(self, b, npid, pid0, sample, obs_ptr, obs_stride):
        """Kernel argument block with the weights, sizes and Philox key set
        (masks, uniforms and outputs left NULL)."""
        a = _capi.MlpArgsC()
        a.batch, a.npid, a.pid0, a.sample = b, npid, pid0, int(sample)
        a.k0, a.kblocks0, a.obs_stride = self.k0, self.kblocks0, obs_stride
        a.seed = self.seed & 0xFFFFFFFFFFFFFFFF
        a.w0_players = self.n_players
        a.obs = obs_ptr
        for k, v in self._w.items():
            setattr(a, k, v.data_ptr())
        si = self._sparse_info
        a.sparse = int(self.sparse)
        a.channels, a.cells = si["channels"], si["cells"]
        a.dense_mask = si["dense_mask"]
        for p, row in enumerate(si["vmap"]):
            for ch, v in enumerate(row):
                a.vmap[p][ch] = v
        return a

    def _launch(self, a, stream) -> None:
        _capi.check(self._lib.qqt_mlp_act(a, stream))

    def _run(self, obs, npid, pid0, sample, mm=None, bm=None, mm_strides=(0, 0),
             bm_strides=(0, 0), uniforms=None, actions=None, actions_i8=None, logp=None,
             value=None, logits=None, tick=None):
        b = obs.shape[0]
        flat = obs.reshape(b, -1) if obs.is_contiguous() else obs.contiguous().reshape(b, -1)
        if flat.dtype != torch.float16:
            flat = flat.half()
        if flat.shape[1] != self.k0:
            raise ValueError(f"observation rows must have {self.k0} values")
        a = self._args(b, npid, pid0, sample, flat.data_ptr(), flat.stride(0))
        a.mm_row_stride, a.mm_pid_stride = mm_strides
        a.bm_row_stride, a.bm_pid_stride = bm_strides
        a.tick = (self.tick if tick is None else tick) & 0xFFFFFFFF
        a.move_mask = _capi.ptr(mm)
        a.bomb_mask = _capi.ptr(bm)
        a.uniforms = _capi.ptr(uniforms)
        a.actions = _capi.ptr(actions)
        a.actions_i8 = _capi.ptr(actions_i8)
        a.logp_out = _capi.ptr(logp)
        a.value_out = _capi.ptr(value)
        a.logits_out = _capi.ptr(logits)
        self._launch(a, _capi.stream_handle(self.device))
        return flat

    @staticmethod
    def _u8(mask):
        m = mask if mask.dtype == torch.uint8 else mask.to(torch.uint8)
        return m.contiguous()

    # ------------------------------------------------------------ API
    def forward(self, obs, pid: int = 0):
        """(move logits (B,5), bomb logits (B,2), value (B,)) of player `pid`."""
        b = obs.shape[0]
        out = torch.empty((b, 1, 8), dtype=torch.float32, device=self.device)
        keep = self._run(obs, 1, pid, False, logits=out)  # noqa: F841
        return out[:, 0, :5], out[:, 0, 5:7], out[:, 0, 7]

    __call__ = forward

    def act(self, obs, move_mask, bomb_mask, pid: int = 0, uniforms=None):
        """Sample one step for player `pid` (train/model.py:230-245)."""
        b = obs.shape[0]
        mm = self._u8(move_mask)
        bm = self._u8(bomb_mask)
        acts = torch.empty((b, 1, 2), dtype=torch.int64, device=self.device)
        logp = torch.empty((b, 1), dtype=torch.float32, device=self.device)
        val = torch.empty((b, 1), dtype=torch.float32, device=self.device)
        u = None if uniforms is None else uniforms.to(self.device, torch.float32).reshape(b, 1, 2).contiguous()
        self._run(obs, 1, pid, True, mm=mm, bm=bm, mm_strides=(5, 0), bm_strides=(2, 0),
                  uniforms=u, actions=acts, logp=logp, value=val)
        if uniforms is None:
            self.tick += 1
        return acts[:, 0], logp[:, 0], val[:, 0]

    def act_pair(self, obs, move_mask, bomb_mask, uniforms=None, out=None, logits=False):
        """Both players from one pass: masks (B,P,5)/(B,P,2); returns
        (actions (B,P,2) int64, logp (B,P), value (B,P)[, logits (B,P,8)])."""
        b, p = obs.shape[0], self.n_players
        if p != 2:
            raise ValueError("act_pair serves two players")
        mm = self._u8(move_mask)
        bm = self._u8(bomb_mask)
        if out is None:
            out = dict(actions=torch.empty((b, p, 2), dtype=torch.int64, device=self.device),
                       logp=torch.empty((b, p), dtype=torch.float32, device=self.device),
                       value=torch.empty((b, p), dtype=torch.float32, device=self.device))
        lg = torch.empty((b, p, 8), dtype=torch.float32, device=self.device) if logits else None
        u = None if uniforms is None else uniforms.to(self.device, torch.float32).reshape(b, p, 2).contiguous()
        self._run(obs, 2, 0, True, mm=mm, bm=bm, mm_strides=(5 * p, 5), bm_strides=(2 * p, 2),
                  uniforms=u, actions=out.get("actions"), actions_i8=out.get("actions_i8"),
                  logp=out.get("logp"), value=out.get("value"), logits=lg)
        if uniforms is None:
            self.tick += 1
        res = (out.get("actions", out.get("actions_i8")), out.get("logp"), out.get("value"))
        return res + ((lg,) if logits else ())

    def evaluate(self, obs, move_mask, bomb_mask, actions, pid: int = 0):
        """(logp, entropy, value) of given actions (train/model.py:247-256)."""
        ml, bl, v = self.forward(obs, pid)
        neg = torch.finfo(torch.float32).min
        lp, ent = 0.0, 0.0
        for logits, mask, act in ((ml, move_mask, actions[..., 0]), (bl, bomb_mask, actions[..., 1])):
            d = torch.distributions.Categorical(
                logits=torch.where(mask.bool(), logits, torch.full_like(logits, neg)))
            lp = lp + d.log_prob(act)
            ent = ent + d.entropy()
        return lp, ent, v


# ---------------------------------------------------------------- cnn arch
CNN_CHANNELS = (16, 32, 64, 8)


def _conv_operand(w: torch.Tensor, n_tiles: int) -> torch.Tensor:
    """[out][in][k][k] conv weight -> float32 [tile][step][lane][8] in the cnn
    kernel's K order: lane l holds output 16 tile + l % 16 and the 8 input
    channels of its lane group g = l // 16 at one tap: 16 inputs (conv0's 14
    padded with zeros): combination c = 4 step + g, tap c // 2 (zero past
    tap 8), channels 8 (c % 2)..; 32 inputs: tap = step, channels 8 g..; a
    1x1 conv over 64 inputs: channels 8 (4 step + g)...  Outputs past `out`
    are zero."""
    cout, cin, kh, kw = w.shape
    taps = kh * kw
    if taps == 1:
        cinp, steps = 64, 2
    elif cin <= 16:
        cinp, steps = 16, 5
    else:
        cinp, steps = 32, 9
    if cin > cinp:
        raise ValueError(f"{cin} input channels do not fit the kernel's layout")
    wp = torch.zeros((n_tiles * 16, cinp, taps), dtype=torch.float32)
    wp[:cout, :cin] = w.float().reshape(cout, cin, taps)
    out = torch.zeros((n_tiles, 16, steps, 4, 8), dtype=torch.float32)   # [tile][i16][step][g][j]
    wt = wp.view(n_tiles, 16, cinp, taps)
    for st in range(steps):
        for g in range(4):
            if taps == 1:
                tap, cb = 0, 4 * st + g
            elif cinp == 16:
                c = 4 * st + g
                tap, cb = c // 2, c % 2
                if tap >= taps:
                    continue
            else:
                tap, cb = st, g
            out[:, :, st, g, :] = wt[:, :, 8 * cb:8 * cb + 8, tap]
    return out.permute(0, 2, 3, 1, 4).reshape(-1).contiguous()          # [tile][step][g*16+i16][j]


HALF_MAX = 65504.0


def _split16(x: torch.Tensor):
    """float32 -> float16 hi and lo (x = hi + lo to ~2^-22 relative for
    |x| <= 65504).  Saturating like the kernels' split: past float16's range
    hi stays at +-65504 and lo takes the clamped remainder (finite, never
    inf - inf)."""
    hi = x.clamp(-HALF_MAX, HALF_MAX).half()
    return hi, (x - hi.float()).clamp(-HALF_MAX, HALF_MAX).half()


def _pack_linear(w: torch.Tensor) -> torch.Tensor:
    """[out][in] Linear weight -> [tile][step][lane]: lane l of step j holds
    output 16 tile + l % 16, input 4 j + l // 16."""
    n, k = w.shape
    x = w.float().reshape(n // 16, 16, k // 4, 4)             # [tile][i16][j][kq]
    return x.permute(0, 2, 3, 1).reshape(-1).contiguous()


def _frag16_planes(w: torch.Tensor, kpad: int):
    """[out][in] Linear weight -> float16 hi and lo planes of the k-major
    [kpad][out] matrix (rows past `in` zero) in the B-fragment order of
    v_mfma_f32_16x16x32_f16: half i of lane 16 q + r in K step s of column
    tile t is W[32 s + 8 q + i][16 t + r]."""
    n, k = w.shape
    wk = torch.zeros((kpad, n), dtype=torch.float32)
    wk[:k] = w.float().t()
    hi, lo = _split16(wk)

    def frag(x):
        return x.reshape(kpad // 32, 4, 8, n // 16, 16).permute(3, 0, 1, 4, 2).reshape(-1)

    return frag(hi).contiguous(), frag(lo).contiguous()


def _pack_ln(g: torch.Tensor, n_tiles: int) -> torch.Tensor:
    """[C][13][13] LayerNorm affine -> [tile][13][lane][4]: value q of lane l
    in row tile y is channel 16 tile + 4 (l // 16) + q at position (y, x =
    l % 16) (zero for x >= 13 or past C channels), the layout of the
    kernel's transposed convolution accumulators."""
    c = g.shape[0]
    gp = torch.zeros((n_tiles * 16, 13, 16), dtype=torch.float32)
    gp[:c, :, :13] = g.float().reshape(c, 13, 13)
    x = gp.view(n_tiles, 4, 4, 13, 16)                        # [tile][kq][q][y][x]
    return x.permute(0, 3, 1, 4, 2).reshape(-1).contiguous()


def _conv3_frag(w: torch.Tensor) -> torch.Tensor:
    """1x1 conv weight [8][64][1][1] -> [block][lane][4]: value j of lane l in
    input block b is W[o = l % 16][c = 16 b + 4 (l // 16) + j] (zero for
    o >= 8), the A operand of v_mfma_f32_16x16x16_f16 for each block of 16
    input channels."""
    wk = torch.zeros((16, 64), dtype=torch.float32)
    wk[:8] = w.float().reshape(8, 64)
    x = wk.view(16, 4, 4, 4)                                  # [o][block][kq][j]
    return x.permute(1, 2, 0, 3).reshape(-1).contiguous()


CNN_FLAT_PAD = 1376            # flattened trunk features padded to 43 K steps of 32
CNN_WS_BYTES_PER_ITEM = 5504   # QQT_CNN_WS_BYTES_PER_ITEM


def pack_cnn(params: dict, n_players: int = 2, obs_shape=(14, 13, 13)) -> dict:
    """Host-side packing of an ActorCritic cnn state_dict (train/model.py:79-96)
    into the operand layout of qqt_cnn_act (CPU tensors out: conv weights as
    float16 hi / lo planes, the rest float32), plus the view
    permutation table: conv0 input plane j of player p is observation channel
    view_perm(p)[j], which equals the reference's conv0.weight[:,
    argsort(view_perm)] over the stored observation (:186-190)."""
    c, h, w = obs_shape
    if (c, h, w) != (14, 13, 13) or n_players != 2:
        raise ValueError("the cnn kernel is built for 2 players on a 13 x 13 grid (14 channels)")
    f = lambda k: params[k].float().cpu()  # noqa: E731
    shapes = {"conv0.weight": (16, c, 3, 3), "conv.2.weight": (32, 16, 3, 3),
              "conv.5.weight": (64, 32, 3, 3), "conv.8.weight": (8, 64, 1, 1),
              "shared.0.weight": (HID, 8 * h * w), "shared.3.weight": (HID, HID)}
    for k, shp in shapes.items():
        if tuple(params[k].shape) != shp:
            raise ValueError(f"{k} must be {shp}, got {tuple(params[k].shape)}")
    heads = ("move_head", "bomb_head", "critic")
    fw = torch.cat([f(f"{n}.2.weight") for n in heads])
    if fw.shape != (8, HEAD):
        raise ValueError("heads must produce 5 + 2 + 1 outputs from 64 hidden units")
    c3b = torch.zeros(16)
    c3b[:8] = f("conv.8.bias")
    out = dict(
        view_perm=torch.tensor([view_perm(p, n_players, c) for p in range(n_players)],
                               dtype=torch.int32).reshape(-1),
        c0b=f("conv0.bias"),
        ln0w=_pack_ln(f("conv.0.weight"), 1), ln0b=_pack_ln(f("conv.0.bias"), 1),
        c1b=f("conv.2.bias"),
        ln1w=_pack_ln(f("conv.3.weight"), 2), ln1b=_pack_ln(f("conv.3.bias"), 2),
        c2b=f("conv.5.bias"),
        ln2w=_pack_ln(f("conv.6.weight"), 4), ln2b=_pack_ln(f("conv.6.bias"), 4),
        c3b=c3b,
        ln3w=f("conv.9.weight").reshape(-1), ln3b=f("conv.9.bias").reshape(-1),
        s0b=f("shared.0.bias"),
        s1w=f("shared.1.weight"), s1b=f("shared.1.bias"),
        s3p=_pack_linear(f("shared.3.weight")), s3b=f("shared.3.bias"),
        s4w=f("shared.4.weight"), s4b=f("shared.4.bias"),
        hp=_pack_linear(torch.cat([f(f"{n}.0.weight") for n in heads])),
        hb=torch.cat([f(f"{n}.0.bias") for n in heads]),
        fw=fw, fb=torch.cat([f(f"{n}.2.bias") for n in heads]))
    for key, src, nt in (("c0w", "conv0.weight", 1), ("c1w", "conv.2.weight", 2),
                         ("c2w", "conv.5.weight", 4)):
        out[key], out[key + "_lo"] = _split16(_conv_operand(f(src), nt))
    out["c3w"], out["c3w_lo"] = _split16(_conv3_frag(f("conv.8.weight")))
    out["s0h"], out["s0l"] = _frag16_planes(f("shared.0.weight"), CNN_FLAT_PAD)
    expect = dict(c0w=5 * 64 * 8, c1w=2 * 5 * 64 * 8, c2w=4 * 9 * 64 * 8, c3w=4 * 64 * 4,
                  ln3w=8 * 169,
                  s0h=8 * 43 * 64 * 8, s3p=8 * 32 * 64, hp=12 * 32 * 64, ln2w=4 * 13 * 64 * 4)
    for k, numel in expect.items():
        if out[k].numel() != numel:
            raise ValueError(f"{k} packs to {out[k].numel()} values, expected {numel}")
    return {k: v.contiguous() for k, v in out.items()}


def default_init_cnn(obs_shape=(14, 13, 13), n_moves: int = 5, n_bomb: int = 2,
                     seed: int = 0) -> dict:
    """PyTorch default init of the cnn ActorCritic layers (Conv2d / Linear
    kaiming-uniform(a=sqrt(5)), LayerNorm 1/0) under torch.manual_seed(seed),
    layers created in module order (train/model.py:79-96, 140-153).  The
    global RNG state is restored afterwards."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        return _tree_state(_layer_tree("cnn", obs_shape, n_moves, n_bomb))


class HipCnnActorCritic(HipActorCritic):
    """The reference's cnn `ActorCritic` (train/model.py:79-96, 186-190) on
    qqt_cnn_act: the same forward / act / act_pair / evaluate as the mlp
    class, with float32 weights (the trunk computes in float32 on MFMA)."""

    arch = "cnn"

    def _pack(self, params: dict) -> dict:
        # the conv operand layout is built on the host (a few hundred KB)
        packed = pack_cnn({k: v.cpu() for k, v in params.items()}, self.n_players,
                          self.obs_shape)
        self.k0 = self.obs_shape[0] * self.obs_shape[1] * self.obs_shape[2]
        return packed

    def _workspace(self, items: int) -> torch.Tensor:
        """The trunk's feature rows for launches of `items` (row, player)
        items: one buffer per item count, kept for the policy's lifetime so
        that argument blocks built earlier (a `Rollout`'s) stay valid.
        Launches share it in stream order."""
        ws = getattr(self, "_ws", None)
        if ws is None:
            ws = self._ws = {}
        if items not in ws:
            blocks = (items + 31) // 32             # the kernels' 32-item blocks
            ws[items] = torch.empty(blocks * 32 * CNN_WS_BYTES_PER_ITEM, dtype=torch.uint8,
                                    device=self.device)
        return ws[items]

    def _args(self, b, npid, pid0, sample, obs_ptr, obs_stride):
        a = _capi.CnnArgsC()
        a.batch, a.npid, a.pid0, a.sample = b, npid, pid0, int(sample)
        a.obs_stride = obs_stride
        a.w_players = self.n_players
        a.seed = self.seed & 0xFFFFFFFFFFFFFFFF
        a.obs = obs_ptr
        for k, v in self._w.items():
            setattr(a, k, v.data_ptr())
        ws = self._workspace(b * npid)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        return a

    def _launch(self, a, stream) -> None:
        _capi.check(self._lib.qqt_cnn_act(a, stream))


# ---------------------------------------------------------------- lstm arch
LSTM_PARAMS = 378880       # QQT_LSTM_PARAMS
# blocks of the packed parameters in order: (key, rows K, columns N, layout)
# with layout "k" = float32 k-major [K][N], "h" = float16 hi / lo MFMA
# fragments (see _lstm_frag16), "v" = a float32 vector in a block of N
# (qqt-gpu-sim_amd/csrc/lstm.hip OFF_*)
_LSTM_BLOCKS = (("c1w", 144, 32, "k"), ("c1b", 1, 64, "v"), ("c2w", 288, 64, "k"),
                ("c2b", 1, 64, "v"), ("fcw", 576, 128, "h"), ("fcb", 1, 128, "v"),
                ("r1w", 64, 64, "h"), ("r1b", 1, 64, "v"), ("r2w", 64, 32, "h"),
                ("r2b", 1, 64, "v"), ("g1w", 32, 16, "h"), ("g1b", 1, 64, "v"),
                ("g2w", 32, 16, "h"), ("g2b", 1, 64, "v"), ("fuw", 192, 256, "h"),
                ("fub", 1, 256, "v"), ("lw", 384, 512, "h"), ("lb", 1, 512, "v"),
                ("hw", 128, 192, "h"), ("hb", 1, 192, "v"), ("ow", 192, 16, "h"),
                ("ob", 1, 64, "v"))


def _lstm_frag16(w: torch.Tensor) -> torch.Tensor:
    """float32 k-major [K][N] (K a multiple of 32, N of 16) -> K N float32
    words holding two float16 planes, hi = fp16(w) then lo = fp16(w - hi),
    each in the B-fragment order of v_mfma_f32_16x16x32_f16: half i of lane
    16 q + r in K step s of column tile t is W[32 s + 8 q + i][16 t + r]."""
    k, n = w.shape
    hi, lo = _split16(w)

    def frag(x):
        return x.reshape(k // 32, 4, 8, n // 16, 16).permute(3, 0, 1, 4, 2).reshape(-1)

    return torch.cat([frag(hi), frag(lo)]).contiguous().view(torch.float32)


def pack_lstm(params: dict, obs_channels: int = 14) -> torch.Tensor:
    """One float32 block of QQT_LSTM_PARAMS values for qqt_lstm_act from an
    lstm ActorCritic state_dict (train/model.py:103-120, 140-153): every
    weight transposed to k-major [in][out], zero-padded to the block's shape
    and, for the head's layers, stored as float16 hi / lo MFMA B fragments
    (`_lstm_frag16`).
    Convolution rows are tap-major: k = (ky * 3 + kx) * S + in_channel
    with S = 16 channel slots for conv1 (14 used, 144 rows) and S = 32 for
    conv2 (288 rows); the LSTM block stacks W_ih^T over W_hh^T with the bias
    b_ih + b_hh, gate columns in torch's i, f, g, o order; the heads' hidden
    layers sit side by side (move | bomb | critic, 192 columns) and their
    output layers form one block-diagonal [192][16] matrix whose columns
    0-4, 5-6, 7 are the move logits, bomb logits and value."""
    c = obs_channels
    f = lambda k: params[k].detach().float().cpu()  # noqa: E731
    shapes = {"l_conv1.weight": (32, c, 3, 3), "l_conv2.weight": (64, 32, 3, 3),
              "l_cnn_fc.weight": (HID, 576), "l_rel_fc1.weight": (64, LSTM_MAX_T * 6),
              "l_rel_fc2.weight": (32, 64), "l_glob_fc1.weight": (16, LSTM_GLOB),
              "l_glob_fc2.weight": (8, 16), "l_fusion.weight": (256, HID + 40),
              "lstm.weight_ih_l0": (4 * LSTM_HIDDEN, 256),
              "lstm.weight_hh_l0": (4 * LSTM_HIDDEN, LSTM_HIDDEN),
              "move_head.0.weight": (HEAD, HID), "move_head.2.weight": (5, HEAD),
              "bomb_head.0.weight": (HEAD, HID), "bomb_head.2.weight": (2, HEAD),
              "critic.0.weight": (HEAD, HID), "critic.2.weight": (1, HEAD)}
    if c > 14:
        raise ValueError("the lstm kernel takes at most 14 observation channels")
    for k, shp in shapes.items():
        if tuple(params[k].shape) != shp:
            raise ValueError(f"{k} must be {shp}, got {tuple(params[k].shape)}")
    src = {
        "c1b": f("l_conv1.bias"),
        "c2w": f("l_conv2.weight").permute(2, 3, 1, 0).reshape(288, 64), "c2b": f("l_conv2.bias"),
        "fcw": f("l_cnn_fc.weight").t(), "fcb": f("l_cnn_fc.bias"),
        "r1w": f("l_rel_fc1.weight").t(), "r1b": f("l_rel_fc1.bias"),
        "r2w": f("l_rel_fc2.weight").t(), "r2b": f("l_rel_fc2.bias"),
        "g1w": f("l_glob_fc1.weight").t(), "g1b": f("l_glob_fc1.bias"),
        "g2w": f("l_glob_fc2.weight").t(), "g2b": f("l_glob_fc2.bias"),
        "fuw": f("l_fusion.weight").t(), "fub": f("l_fusion.bias"),
        "lw": torch.cat([f("lstm.weight_ih_l0").t(), f("lstm.weight_hh_l0").t()]),
        "lb": f("lstm.bias_ih_l0") + f("lstm.bias_hh_l0"),
        "hw": torch.cat([f(f"{n}.0.weight") for n in ("move_head", "bomb_head", "critic")]).t(),
        "hb": torch.cat([f(f"{n}.0.bias") for n in ("move_head", "bomb_head", "critic")]),
        "ob": torch.cat([f(f"{n}.2.bias") for n in ("move_head", "bomb_head", "critic")]),
    }
    c1w = torch.zeros((9, 16, 32))
    c1w[:, :c] = f("l_conv1.weight").permute(2, 3, 1, 0).reshape(9, c, 32)
    src["c1w"] = c1w.reshape(144, 32)
    ow = torch.zeros((3 * HEAD, 16))
    ow[0:HEAD, 0:5] = f("move_head.2.weight").t()
    ow[HEAD:2 * HEAD, 5:7] = f("bomb_head.2.weight").t()
    ow[2 * HEAD:, 7:8] = f("critic.2.weight").t()
    src["ow"] = ow
    out = torch.zeros(LSTM_PARAMS, dtype=torch.float32)
    off = 0
    for key, rows, cols, layout in _LSTM_BLOCKS:
        v = src[key]
        if layout == "v":
            out[off:off + v.numel()] = v
        else:
            blk = torch.zeros((rows, cols))
            blk[:v.shape[0], :v.shape[1]] = v
            out[off:off + rows * cols] = blk.reshape(-1) if layout == "k" else _lstm_frag16(blk)
        off += rows * cols
    if off != LSTM_PARAMS:
        raise AssertionError("packed block size")
    return out


def lstm_block_offsets() -> dict:
    """Float offset of each block of the packed lstm parameters."""
    offs, off = {}, 0
    for key, rows, cols, _ in _LSTM_BLOCKS:
        offs[key] = off
        off += rows * cols
    return offs


class HipLstmActorCritic:
    """The reference's lstm `ActorCritic` (train/model.py:103-120, 176-185,
    198-256) on qqt_lstm_act.  `obs` is the per-player feature triple
    (local (B,C,7,7), rel (B,10,6), glob (B,5)) of
    `HipBatchedSim.local_view_features` (float16), `hidden` the LSTM state
    as torch.nn.LSTM holds it ((1,B,128), (1,B,128)) or None for zeros.

    forward(obs, pid, hidden) -> (move logits, bomb logits, value, hidden')
    act(obs, mm, bm, pid, hidden) -> (actions (B,2), logp, value, hidden')
    evaluate(obs, mm, bm, actions, pid, hidden) -> (logp, entropy, value)

    Every step runs the whole network in one kernel (float32 arithmetic);
    hidden' is a new pair of tensors.  `step_` runs one frame of a rollout
    with the state held in place and zeroed for the envs flagged in `reset`
    (the reference's hidden * (1 - done) after each tick)."""

    arch = "lstm"

    def __init__(self, state_dict: dict | None = None, obs_shape=(14, 13, 13),
                 n_players: int = 2, device="cuda", seed: int = 0, sparse: bool = False):
        self.obs_shape = tuple(obs_shape)
        # sparse=True: the first layer over the observation's nonzero cells
        # (csrc/mlp_sparse.hip) where the launch qualifies: logits within
        # ~4e-5 of float32 instead of ~4e-4, at 30 us instead of 23 us per
        # 5632-row pair launch on MI355X
        self.sparse = bool(sparse)
        self.n_players = n_players
        if n_obs_channels(n_players) != self.obs_shape[0]:
            raise ValueError("observation channels do not match n_players")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HipLstmActorCritic runs on a ROCm device")
        self.seed = int(seed)
        self.tick = 0
        self._lib = _capi.lib()
        self._w = None
        self.load_state_dict(state_dict if state_dict is not None
                             else reference_init(obs_shape, seed=0, arch="lstm"))

    def load_state_dict(self, state_dict: dict) -> None:
        """Repack and copy over the packed block in place (ordered on the
        current stream), so argument blocks built before stay valid."""
        params = {k: v.detach().float().cpu().clone() for k, v in state_dict.items()}
        packed = pack_lstm(params, self.obs_shape[0]).to(self.device)
        if self._w is None:
            self._w = packed
        else:
            self._w.copy_(packed)
        self.params = params

    def state_dict(self) -> dict:
        return {k: v.clone() for k, v in self.params.items()}

    def n_params(self) -> int:
        return sum(v.numel() for v in self.params.values())

    # ------------------------------------------------------------ launch
    def _feat(self, obs):
        local, rel, glob = obs
        b = local.shape[0]
        c = self.obs_shape[0]
        if tuple(local.shape[1:]) != (c, 7, 7) or tuple(rel.shape[1:]) != (LSTM_MAX_T, 6) \
                or tuple(glob.shape[1:]) != (LSTM_GLOB,) or rel.shape[0] != b or glob.shape[0] != b:
            raise ValueError("features must be local (B,C,7,7), rel (B,10,6), glob (B,5)")
        out = []
        for t in (local, rel, glob):
            t = t if t.dtype == torch.float16 else t.half()
            t = t.reshape(b, -1)
            if t.stride(1) != 1:
                t = t.contiguous()
            out.append(t)
        return out

    def args(self, local, rel, glob, h, c, rows_per_env=1, pid0=0, reset=None):
        """Argument block over row-strided float16 feature planes and
        float32 [B][128] state (masks, uniforms and outputs left NULL)."""
        a = _capi.LstmArgsC()
        a.batch = local.shape[0]
        a.c_in = self.obs_shape[0]
        a.rows_per_env = rows_per_env
        a.pid0 = pid0
        a.seed = self.seed & 0xFFFFFFFFFFFFFFFF
        a.local, a.rel, a.glob = local.data_ptr(), rel.data_ptr(), glob.data_ptr()
        a.local_stride, a.rel_stride, a.glob_stride = local.stride(0), rel.stride(0), glob.stride(0)
        a.params = self._w.data_ptr()
        a.h, a.c = h.data_ptr(), c.data_ptr()
        a.reset = _capi.ptr(reset)
        a.out_stride, a.out_slot = 1, 0
        return a

    def launch(self, a) -> None:
        _capi.check(self._lib.qqt_lstm_act(a, _capi.stream_handle(self.device)))

    def _state(self, hidden, b):
        if hidden is None:
            z = torch.zeros((b, LSTM_HIDDEN), dtype=torch.float32, device=self.device)
            return z, z.clone()
        h, c = hidden
        h = h.reshape(b, LSTM_HIDDEN).to(self.device, torch.float32).clone()
        c = c.reshape(b, LSTM_HIDDEN).to(self.device, torch.float32).clone()
        return h, c

    def _run(self, obs, hidden, pid, mm=None, bm=None, uniforms=None, tick=None):
        local, rel, glob = self._feat(obs)
        b = local.shape[0]
        h, c = self._state(hidden, b)
        a = self.args(local, rel, glob, h, c, 1, pid)
        lg = torch.empty((b, 8), dtype=torch.float32, device=self.device)
        a.logits_out = lg.data_ptr()
        res = {}
        if mm is not None:
            mm = (mm if mm.dtype == torch.uint8 else mm.to(torch.uint8)).contiguous()
            bm = (bm if bm.dtype == torch.uint8 else bm.to(torch.uint8)).contiguous()
            res["actions"] = torch.empty((b, 2), dtype=torch.int64, device=self.device)
            res["logp"] = torch.empty((b,), dtype=torch.float32, device=self.device)
            a.sample = 1
            a.move_mask, a.bomb_mask = mm.data_ptr(), bm.data_ptr()
            a.mm_row_stride, a.bm_row_stride = mm.stride(0), bm.stride(0)
            a.tick = (self.tick if tick is None else tick) & 0xFFFFFFFF
            if uniforms is not None:
                uniforms = uniforms.to(self.device, torch.float32).reshape(b, 2).contiguous()
                a.uniforms = uniforms.data_ptr()
            a.actions, a.logp_out = res["actions"].data_ptr(), res["logp"].data_ptr()
        self.launch(a)
        hid = (h.view(1, b, LSTM_HIDDEN), c.view(1, b, LSTM_HIDDEN))
        return lg, hid, res

    # ------------------------------------------------------------ API
    def forward(self, obs, pid: int = 0, hidden=None):
        lg, hid, _ = self._run(obs, hidden, pid)
        return lg[:, :5], lg[:, 5:7], lg[:, 7], hid

    __call__ = forward

    def act(self, obs, move_mask, bomb_mask, pid: int = 0, hidden=None, uniforms=None):
        """Sample one step (train/model.py:230-245, lstm branch)."""
        lg, hid, res = self._run(obs, hidden, pid, move_mask, bomb_mask, uniforms)
        if uniforms is None:
            self.tick += 1
        return res["actions"], res["logp"], lg[:, 7], hid

    def evaluate(self, obs, move_mask, bomb_mask, actions, pid: int = 0, hidden=None):
        """(logp, entropy, value) of given actions (train/model.py:247-256)."""
        ml, bl, v, _ = self.forward(obs, pid, hidden)
        neg = torch.finfo(torch.float32).min
        lp, ent = 0.0, 0.0
        for logits, mask, act in ((ml, move_mask, actions[..., 0]), (bl, bomb_mask, actions[..., 1])):
            d = torch.distributions.Categorical(
                logits=torch.where(mask.bool(), logits, torch.full_like(logits, neg)))
            lp = lp + d.log_prob(act)
            ent = ent + d.entropy()
        return lp, ent, v
