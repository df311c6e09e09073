"""Host-side layout logic (CPU only): the packed device state, the MFMA
fragment packing of the MLP weights, and the float32 rule constants."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from qqtsim import state as st
from qqtsim.config import corridor_training_config
from qqtsim.maps import MapSpec
from qqtsim.policy import KBLOCK, _frag, default_init, pack_mlp
from qqtsim.sim import config_struct


def _random_state(n=5, h=13, w=13, p=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    ri = lambda lo, hi, shape, dt=torch.long: torch.randint(lo, hi, shape, generator=g).to(dt)  # noqa: E731
    return dict(
        wall=ri(0, 2, (n, h, w), torch.bool), brick=ri(0, 2, (n, h, w), torch.bool),
        crate=ri(0, 2, (n, h, w), torch.bool), recycle=ri(0, 2, (n, h, w), torch.bool),
        fuse=ri(0, 256, (n, h, w), torch.int16), owner=ri(-1, 4, (n, h, w), torch.int8),
        bomb_blast=ri(0, 256, (n, h, w), torch.int16),
        pos=torch.rand((n, p, 2), generator=g) * 12.0 + 0.3,
        alive=ri(0, 2, (n, p), torch.bool), hp=ri(0, 6, (n, p), torch.uint8),
        since_bomb=ri(-5, 100, (n, p), torch.int32), bombs_cap=ri(0, 11, (n, p)),
        blast_cap=ri(0, 8, (n, p)), spd_g=torch.rand((n, p), generator=g) + 0.5,
        invuln=ri(0, 31, (n, p)), combo=ri(0, 9, (n, p)), last_hit=ri(-1000, 2000, (n, p)),
        pending_lost=ri(0, 7, (n, p)), lo_bombs=ri(0, 3, (n, p)), lo_blast=ri(0, 3, (n, p)),
        lo_spd=torch.rand((n, p), generator=g), t=ri(0, 1800, (n,)),
        crate_prob=torch.rand((n,), generator=g), map_kind=ri(0, 2, (n,)))


def _packed(n=5, h=13, w=13, p=2):
    return (torch.zeros((n, h * w), dtype=torch.int32),
            torch.zeros((n, p, st.P_SLOTS), dtype=torch.int32),
            torch.zeros((n, st.E_SLOTS), dtype=torch.int32))


def test_state_round_trip_is_exact():
    snap = _random_state()
    cells, players, envs = _packed()
    st.pack_into(cells, players, envs, snap, 13, 13)
    back = st.unpack(cells, players, envs, 13, 13)
    assert set(back) == set(st.ALL_KEYS)
    for k, v in snap.items():
        b = back[k]
        if v.dtype.is_floating_point:
            assert torch.equal(b.view(torch.int32), v.float().view(torch.int32)), k
        else:
            assert torch.equal(b.long(), v.long()), k


def test_cell_word_bit_layout():
    """bits 0-7 fuse, 8-15 owner (int8), 16-23 bomb_blast, 24 wall, 25 brick,
    26 crate, 27 recycle-crate (the layout the C header documents)."""
    snap = {k: torch.zeros(1, 13, 13, dtype=dt) for k, dt in (
        ("wall", torch.bool), ("brick", torch.bool), ("crate", torch.bool),
        ("recycle", torch.bool), ("fuse", torch.int16), ("owner", torch.int8),
        ("bomb_blast", torch.int16))}
    snap["fuse"][0, 2, 3] = 30
    snap["owner"][0, 2, 3] = -1
    snap["bomb_blast"][0, 2, 3] = 5
    snap["wall"][0, 0, 0] = True
    snap["recycle"][0, 12, 12] = True
    cells, players, envs = _packed(n=1)
    st.pack_into(cells, players, envs, snap, 13, 13)
    assert int(cells[0, 2 * 13 + 3]) == 30 | (0xFF << 8) | (5 << 16)
    assert int(cells[0, 0]) == 1 << 24
    assert int(cells[0, 168]) == 1 << 27


@pytest.mark.parametrize("key,val", [("fuse", 256), ("bomb_blast", -1), ("t", -3)])
def test_pack_rejects_values_the_word_cannot_hold(key, val):
    snap = _random_state(n=2)
    snap[key] = torch.full_like(snap[key], val)
    cells, players, envs = _packed(n=2)
    with pytest.raises(ValueError):
        st.pack_into(cells, players, envs, snap, 13, 13)


def test_unpack_bits():
    words = torch.zeros((2, 8), dtype=torch.int32)
    words[0, 0] = 1 << 5
    words[1, 5] = 1 << 8          # cell 168
    m = st.unpack_bits(words, 13, 13)
    assert m.shape == (2, 13, 13) and int(m.sum()) == 2
    assert m[0, 0, 5] and m[1, 12, 12]


def test_fragment_layout():
    """frag[tile][kblock][lane][j] = W[16 tile + lane%16][64 kblock + 16 (lane/16) + j],
    zero past the matrix's K."""
    g = torch.Generator().manual_seed(3)
    wm = torch.randn((32, 100), generator=g)
    f = _frag(wm, 128).float().view(2, 2, 64, 16)
    for tile in range(2):
        for kb in range(2):
            for lane in range(64):
                for j in range(16):
                    r, k = 16 * tile + lane % 16, KBLOCK * kb + 16 * (lane // 16) + j
                    want = float(wm[r, k].half()) if k < 100 else 0.0
                    assert float(f[tile, kb, lane, j]) == want


def test_fragment_residual_split():
    g = torch.Generator().manual_seed(4)
    wm = torch.randn((16, 64), generator=g) * 0.3
    hi = _frag(wm, 64).float()
    lo = _frag(wm, 64, residual=True).float()
    flat = wm.view(1, 16, 1, 4, 16).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(lo, (flat - flat.half().float()).half().float())
    # hi + lo carries ~22 significant bits; residuals below the float16
    # normal range keep an absolute error of half the subnormal spacing
    err = (flat - (hi + lo)).abs()
    assert bool((err <= flat.abs() * 2.0 ** -22 + 2.0 ** -25).all())


def _mfma_16x16x32(a_lanes, b_lanes, c_lanes):
    """v_mfma_f32_16x16x32_f16 on lane registers (float64 here): lane l holds
    A[l%16][8(l/16) + i], B[8(l/16) + i][l%16] (i < 8) and D[4(l/16) + j][l%16]
    (j < 4)."""
    lane = np.arange(64)
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for i in range(8):
        A[lane % 16, 8 * (lane // 16) + i] = a_lanes[:, i]
        B[8 * (lane // 16) + i, lane % 16] = b_lanes[:, i]
    D = A @ B
    return c_lanes + np.stack([D[4 * (lane // 16) + j, lane % 16] for j in range(4)], 1)


def test_chain_fragments_take_the_previous_output_tiles_as_is():
    """The later layers' A fragments (_chain_frag) against activations held in
    the MFMA output layout (lane 16q + r: features 16t + 4q + j of row r): K
    step s of the next product packs output tiles 2s, 2s+1 of a lane into its
    8-element B fragment, and the products equal W h^T."""
    from qqtsim.policy import CHAIN_KPERM, _chain_frag

    g = torch.Generator().manual_seed(5)
    n_out, k_in = 48, 64
    W = torch.randn((n_out, k_in), generator=g).double()
    h = torch.randn((16, k_in), generator=g).double()       # 16 batch rows
    frag = _chain_frag(W).double().view(n_out // 16, k_in // 32, 64, 8).numpy()
    lane = np.arange(64)
    q, r = lane // 16, lane % 16
    # previous product's output tiles: v[t][lane][j] = h[r][16t + 4q + j]
    v = np.stack([np.stack([h.numpy()[r, 16 * t + 4 * q + j] for j in range(4)], 1)
                  for t in range(k_in // 16)])
    want = (W.half().double() @ h.numpy().T)                  # [feature][row]
    for T in range(n_out // 16):
        acc = np.zeros((64, 4))
        for s in range(k_in // 32):
            b = np.concatenate([v[2 * s], v[2 * s + 1]], 1)   # element i: tile 2s + i // 4
            acc = _mfma_16x16x32(frag[T, s], b, acc)
        for j in range(4):
            assert np.allclose(acc[:, j], want.numpy()[16 * T + 4 * q + j, r], atol=1e-12)
    assert sorted(CHAIN_KPERM) == list(range(32))
    # hi + lo planes carry W to ~22 bits in the same element order
    lo = _chain_frag(W, residual=True).double().view(frag.shape).numpy()
    kperm = np.array(CHAIN_KPERM)
    for T in range(n_out // 16):
        for s in range(k_in // 32):
            exact = W.numpy()[16 * T + r[:, None], 32 * s + kperm[8 * q[:, None] + np.arange(8)]]
            assert np.all(np.abs(frag[T, s] + lo[T, s] - exact) <= np.abs(exact) * 2.0 ** -21 + 2.0 ** -24)


def test_pack_mlp_folds_each_players_view_into_w0():
    from oracle.policy import column_permutation

    params = default_init()
    packed = pack_mlp(params)
    assert packed["k0"] == 2366 and packed["kblocks0"] == 37
    w0 = packed["w0"].float().view(2, 8, 37, 64, 16)
    W0 = params["shared.0.weight"]
    for pid in range(2):
        cols = column_permutation(pid, 2, 14, 169)
        # unpack the fragments back into a (128, 2368) matrix
        f = w0[pid].view(8, 37, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(128, 37 * 64)
        assert torch.equal(f[:, :2366], W0[:, cols].half().float())
        assert float(f[:, 2366:].abs().max()) == 0.0
    assert packed["bf"].numel() == 8 and packed["bh"].numel() == 192


def test_config_struct_float32_constants():
    c = config_struct(corridor_training_config(), MapSpec(kind="pillars", brick_p=0.7))
    f32 = lambda x: float(np.float32(x))  # noqa: E731
    assert c.step_len == f32(0.3)
    assert c.pos_hi_y == f32(13 - 0.3) and c.pos_hi_x == f32(13 - 0.3)
    assert c.chain_time_rest == f32(1.0 - 0.15)
    assert c.win_per_hp == f32(10.0 / 5)
    assert c.hit_speed_drop == f32(2 * 0.15)
    assert c.fuse == 30 and c.blast == 2 and c.max_steps == 1800 and c.corridor == 1
    assert c.brick_p == f32(0.7) and c.map_kind == 0


@pytest.mark.parametrize("kw", [dict(kind="ring"), dict(brick_p=1.5), dict(bombs_cap=(3, 2))])
def test_map_spec_validation(kw):
    with pytest.raises(ValueError):
        MapSpec(**kw)


def test_pack_cnn_operands_reproduce_the_reference_layers():
    """The cnn kernel's operand addressing over the packed tensors reproduces
    the reference's layers.  Each conv: the activations as zero-bordered
    15 x 15 grids of positions with contiguous channels; lane group g of step
    s reads the 8 channels of its block at its tap (16 inputs: combination
    4 s + g -> tap c // 2 (clamped to 8), block c % 2; 32 inputs: tap s,
    block g; 1x1: block 4 s + g, centre) and multiplies them with the packed
    B values [tile][s][g * 16 + n % 16][8] (hi + lo); the sum over steps
    equals F.conv2d with the same (hi + lo) weights in float64, which differ
    from the reference's by <= 2^-22 relative + 2^-24; conv0 runs on the observation
    channels permuted by the view table.  The Linear packing gives W[n][4 j +
    kq]; the LayerNorm tables give gamma[n][16 mt + 4 kq + q]."""
    import torch.nn.functional as F

    from qqtsim.policy import default_init_cnn, pack_cnn

    params = default_init_cnn(seed=3)
    pk = pack_cnn(params)
    g = torch.Generator().manual_seed(0)

    def tap_off(tap):
        return (tap // 3) * 15 + tap % 3

    def kernel_conv(x, key, n_tiles, steps, kind, cout):
        cin = x.shape[0]
        grid = torch.zeros((225, 64), dtype=torch.float64)       # [padded position][channel]
        grid[:, :cin] = F.pad(x, (1, 1, 1, 1)).reshape(cin, 225).t()
        w = (pk[key].double() + pk[key + "_lo"].double()).view(n_tiles, steps, 4, 16, 8)
        pos = torch.arange(169)
        pb = (pos // 13) * 15 + pos % 13
        out = torch.zeros((n_tiles * 16, 169), dtype=torch.float64)
        for st in range(steps):
            for gq in range(4):
                if kind == 0:
                    c = 4 * st + gq
                    tap, cb = min(c // 2, 8), c % 2
                    off = tap_off(tap)
                elif kind == 1:
                    cb, off = gq, tap_off(st)
                else:
                    cb, off = 4 * st + gq, 16
                a = grid[pb + off, 8 * cb:8 * cb + 8]                   # [169][8]
                bw = w[:, st, gq]                                        # [tile][16][8]
                out += torch.einsum("pj,tnj->tnp", a, bw).reshape(n_tiles * 16, 169)
        return out[:cout].view(cout, 13, 13)

    def dense(key, src, n_tiles, steps, kind):
        """The reference weight rounded as the kernel holds it (hi + lo)."""
        w = params[src].double()
        cout, cin, kh, _ = w.shape
        back = torch.zeros_like(w)
        pw = (pk[key].double() + pk[key + "_lo"].double()).view(n_tiles, steps, 4, 16, 8)
        for st in range(steps):
            for gq in range(4):
                if kind == 0:
                    c = 4 * st + gq
                    tap, cb = c // 2, c % 2
                    if tap > 8:
                        assert float(pw[:, st, gq].abs().max()) == 0.0
                        continue
                elif kind == 1:
                    tap, cb = st, gq
                else:
                    tap, cb = 0, 4 * st + gq
                blk = pw[:, st, gq].reshape(n_tiles * 16, 8)[:cout]
                for j in range(8):
                    ci = 8 * cb + j
                    if ci < cin:
                        back[:, ci, tap // kh, tap % kh] = blk[:, j]
                    else:
                        assert float(blk[:, j].abs().max()) == 0.0
        # hi + lo keeps ~22 bits; a lo below float16's normal range keeps 2^-24 absolute
        assert bool(((back - w).abs() <= 2.0 ** -22 * w.abs() + 2.0 ** -24).all())
        return back

    x = torch.rand((14, 13, 13), generator=g, dtype=torch.float64)
    vp = pk["view_perm"].view(2, 14)
    w0 = dense("c0w", "conv0.weight", 1, 5, 0)
    for pid in range(2):
        inv = torch.argsort(vp[pid].long())
        want = F.conv2d(x[None], w0[:, inv], params["conv0.bias"].double(), padding=1)[0]
        got = kernel_conv(x[vp[pid].long()], "c0w", 1, 5, 0, 16) + \
            params["conv0.bias"].double()[:, None, None]
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    for key, src, bk, cin, nt, steps, kind in (("c1w", "conv.2.weight", "conv.2.bias", 16, 2, 5, 0),
                                               ("c2w", "conv.5.weight", "conv.5.bias", 32, 4, 9, 1)):
        x = torch.rand((cin, 13, 13), generator=g, dtype=torch.float64)
        wd = dense(key, src, nt, steps, kind)
        want = F.conv2d(x[None], wd, params[bk].double(), padding=wd.shape[-1] // 2)[0]
        got = kernel_conv(x, key, nt, steps, kind, wd.shape[0]) + params[bk].double()[:, None, None]
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    p = pk["s3p"].view(8, 32, 4, 16)                             # [tile][j][kq][i16]
    assert torch.equal(p.permute(0, 3, 1, 2).reshape(128, 128), params["shared.3.weight"])
    # Linear(1352,128) as float16 hi / lo B fragments [tile][step][q * 16 + r][i]:
    # W^T[32 step + 8 q + i][16 tile + r], inputs 1352..1375 zero
    w0 = params["shared.0.weight"]
    planes = [pk[k].float().view(8, 43, 4, 16, 8) for k in ("s0h", "s0l")]
    kn = [x.permute(1, 2, 4, 0, 3).reshape(1376, 128) for x in planes]
    assert torch.count_nonzero(kn[0][1352:]) == 0 and torch.count_nonzero(kn[1][1352:]) == 0
    assert float(planes[0][3, 7, 2, 5, 1]) == float(w0[16 * 3 + 5, 32 * 7 + 8 * 2 + 1].half())
    wt = w0.t().double()
    err = (kn[0][:1352].double() + kn[1][:1352].double() - wt).abs()
    assert bool((err <= 2.0 ** -22 * wt.abs() + 2.0 ** -24).all())
    ln = pk["ln2w"].view(4, 13, 4, 16, 4)                        # [tile][row][kq][x][q]
    gam = params["conv.6.weight"].reshape(64, 13, 13)
    assert float(ln[1, 3, 2, 5, 1]) == float(gam[16 + 4 * 2 + 1, 3, 5])
    assert float(ln[2, 12, 3, 12, 0]) == float(gam[32 + 12, 12, 12])
    assert float(ln[0, 10, 3, 13, 1]) == 0.0                     # x = 13 is past the row
    assert torch.equal(ln.permute(0, 2, 4, 1, 3).reshape(64, 13, 16)[:, :, :13], gam)
    assert torch.equal(pk["ln3w"], params["conv.9.weight"].reshape(-1))   # plain [8][13][13]
    # the 1x1 conv as per-block A operands [block][kq * 16 + o][j] = W[o][16 block + 4 kq + j]
    w3 = params["conv.8.weight"].reshape(8, 64).double()
    f3 = (pk["c3w"].double() + pk["c3w_lo"].double()).view(4, 4, 16, 4)
    back = f3.permute(2, 0, 1, 3).reshape(16, 64)
    assert float(back[8:].abs().max()) == 0.0
    assert bool(((back[:8] - w3).abs() <= 2.0 ** -22 * w3.abs() + 2.0 ** -24).all())
    assert float(pk["c3w"][(2 * 64 + 16 * 3 + 5) * 4 + 2]) == \
        float(params["conv.8.weight"][5, 16 * 2 + 4 * 3 + 2].half())
    assert torch.equal(pk["fw"][5:7], params["bomb_head.2.weight"])
    assert sum(v.numel() for v in params.values()) == 281744


def test_gather_rows_equals_advanced_indexing():
    """The minibatch row gather of ppo_update (4-byte words for float16 rows
    of even width) returns exactly obs[sel], and falls back for other rows."""
    from qqtsim.learn import _gather_rows

    g = torch.Generator().manual_seed(0)
    obs = torch.rand((50, 14, 13, 13), generator=g).half()
    sel = torch.randint(0, 50, (37,), generator=g)
    assert torch.equal(_gather_rows(obs, sel), obs[sel])
    odd = torch.rand((20, 3), generator=g).half()
    s2 = torch.tensor([4, 1, 1, 19])
    assert torch.equal(_gather_rows(odd, s2), odd[s2])
    f32 = torch.rand((20, 6), generator=g)
    assert torch.equal(_gather_rows(f32, s2), f32[s2])


def test_sim_rejects_chain_blast_bonus():
    """A non-zero chain_blast_bonus (sim/torch_sim.py:981-1005) is refused
    before any device work, instead of being dropped from the rewards."""
    import dataclasses

    from qqtsim.sim import HipBatchedSim

    cfg = dataclasses.replace(corridor_training_config(), chain_blast_bonus=0.08)
    with pytest.raises(ValueError, match="chain_blast_bonus"):
        HipBatchedSim(cfg, 4, device="cpu")


def test_unpack_key_matches_unpack():
    snap = _random_state(seed=3)
    cells, players, envs = _packed()
    st.pack_into(cells, players, envs, snap, 13, 13)
    full = st.unpack(cells, players, envs, 13, 13)
    for k in st.ALL_KEYS:
        one = st.unpack_key(cells, players, envs, 13, 13, k)
        assert one.dtype == full[k].dtype and torch.equal(one, full[k]), k
    with pytest.raises(KeyError):
        st.unpack_key(cells, players, envs, 13, 13, "nope")


def _sparse_first_layer(packed, obs16, pid):
    """CPU emulation, in float64, of the sparse act kernel's first layer
    (csrc/mlp_sparse.hip) from the packed operands: the dense channels from
    the hi + lo MFMA A fragments read in the kernel's lane layout, every
    other channel c as its nonzero cells times the gather table's rows of
    view channel vmap[pid][c]."""
    si = packed["sparse_info"]
    c_n, hw = si["channels"], si["cells"]
    k0 = c_n * hw
    ksc = -(-hw // 32)
    tab = packed["w0g"].double().view(k0, 128)
    w0d = packed["w0d"].double().view(c_n, 8, ksc, 2, 64, 8)
    x = obs16.double().reshape(obs16.shape[0], c_n, hw)
    z = torch.zeros((x.shape[0], 128), dtype=torch.float64)
    for c in range(c_n):
        j = si["vmap"][pid][c]
        if (si["dense_mask"] >> c) & 1:
            # lane 16 g + r of (tile, step) holds W[16 tile + r][j hw + 32 step + 8 g + i]
            wd = (w0d[j, :, :, 0] + w0d[j, :, :, 1]).view(8, ksc, 4, 16, 8)
            wd = wd.permute(0, 3, 1, 2, 4).reshape(128, ksc * 32)
            assert float(wd[:, hw:].abs().max()) == 0.0
            z += x[:, c] @ wd[:, :hw].t()
        else:
            xc = x[:, c]
            nz = xc != 0
            z += torch.where(nz, xc, torch.zeros_like(xc)) @ tab[j * hw:(j + 1) * hw]
    return z


def test_sparse_first_layer_operands_reproduce_the_view_folded_product():
    """The sparse kernel's first-layer operands (gather table, dense-channel
    fragments, view map, dense-channel mask) put together as the kernel does
    give the reference's x @ W0[:, inv_cols[pid]]^T (train/model.py:192-196)
    for both players, on observations from a reference trajectory and on
    the same rows with every cell perturbed."""
    from oracle.policy import column_permutation

    from golden_io import traj

    params = default_init()
    packed = pack_mlp(params)
    si = packed["sparse_info"]
    # wall | brick (channel 2P) and progress (2P + 2) are the dense channels (sim/obs.py:88-101)
    assert si["dense_mask"] == (1 << 4) | (1 << 6)
    W0 = params["shared.0.weight"].double()
    obs = torch.from_numpy(traj("pillars70")["obs"].reshape(-1, 14, 13, 13)[:64].copy())
    g = torch.Generator().manual_seed(1)
    noisy = (obs.float() + 0.01 * torch.randn(obs.shape, generator=g)).half()
    dense = torch.zeros(2366, dtype=torch.bool)
    dense[4 * 169:5 * 169] = True
    dense[6 * 169:7 * 169] = True
    for x16 in (obs, noisy):
        xf = x16.double().reshape(x16.shape[0], -1)
        for pid in range(2):
            cols = column_permutation(pid, 2, 14, 169)
            ref = xf @ W0[:, cols].t()
            got = _sparse_first_layer(packed, x16, pid)
            # the gathered columns are float16: |error| <= sum over them of |x| |w| 2^-11;
            # the dense channels' hi + lo weights are float32-accurate
            wabs = W0[:, cols].abs()
            bound = (xf * ~dense) @ wabs.t() * 2.0 ** -11 + (xf * dense) @ wabs.t() * 2.0 ** -20 + 1e-9
            assert bool(torch.all((got - ref).abs() <= bound)), pid
    # a planted slip: the other player's view map misplaces the player channels
    bad = dict(packed, sparse_info=dict(si, vmap=[si["vmap"][1], si["vmap"][0]]))
    xf = obs.double().reshape(obs.shape[0], -1)
    ref = xf @ W0[:, column_permutation(0, 2, 14, 169)].t()
    assert float((_sparse_first_layer(bad, obs, 0) - ref).abs().max()) > 1e-3
