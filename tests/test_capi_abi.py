"""The C ABI library (no GPU needed): it loads, exports every entry point the
header declares, its structs have the layout the header gives them, and its
argument checks reject bad calls before anything touches a device."""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qqt_hip.h")


def _lib_path():
    from qqtsim import _build

    if not os.path.exists(_build.LIB):
        _build.build(verbose=False)
    return _build.LIB


@pytest.fixture(scope="module")
def lib():
    from qqtsim import _capi

    _lib_path()
    return _capi.lib()


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[\w\s\*]+?\b(qqt_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    assert _declared_functions() == ["qqt_abi_version", "qqt_bot_act", "qqt_cnn_act", "qqt_gae",
                                     "qqt_gather_rows", "qqt_l1_grad", "qqt_l1_grad_noalloc",
                                     "qqt_l1_grad_workspace_floats",
                                     "qqt_last_error", "qqt_lstm_act", "qqt_lstm_features",
                                     "qqt_mlp_act", "qqt_ppo_grad", "qqt_tick",
                                     "qqt_timing_arm", "qqt_timing_collect"]


def test_library_exports_every_declared_symbol():
    path = _lib_path()
    lib = ctypes.CDLL(path)
    for name in _declared_functions():
        assert hasattr(lib, name), name
    if shutil.which("nm"):
        out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True,
                             text=True, check=True).stdout
        exported = set(re.findall(r"\bT (qqt_\w+)", out))
        assert set(_declared_functions()) <= exported


def test_abi_version(lib):
    from qqtsim import _capi

    m = re.search(r"#define QQT_ABI_VERSION (\d+)", open(HEADER).read())
    assert lib.qqt_abi_version() == int(m.group(1)) == _capi.ABI_VERSION


def test_header_constants_match_host_mirror():
    from qqtsim import _capi, state as st

    text = open(HEADER).read()
    enum = dict((k, int(v)) for k, v in re.findall(r"\b(QQT_[PE]_\w+) = (\d+)", text))
    assert enum["QQT_P_SLOTS"] == st.P_SLOTS and enum["QQT_E_SLOTS"] == st.E_SLOTS
    host = dict(Y=st.P_Y, X=st.P_X, ALIVE=st.P_ALIVE, HP=st.P_HP, SINCE_BOMB=st.P_SINCE,
                BOMBS_CAP=st.P_BOMBS, BLAST_CAP=st.P_BLAST, SPD=st.P_SPD, INVULN=st.P_INV,
                COMBO=st.P_COMBO, LAST_HIT=st.P_LAST, PENDING_LOST=st.P_PEND,
                LO_BOMBS=st.P_LOB, LO_BLAST=st.P_LOZ, LO_SPD=st.P_LOS)
    for name, v in host.items():
        assert enum["QQT_P_" + name] == v, name
    for name, v in dict(T=st.E_T, CRATE_PROB=st.E_CRATE_PROB, MAP_KIND=st.E_KIND).items():
        assert enum["QQT_E_" + name] == v, name
    modes = dict((k, int(v)) for k, v in re.findall(r"#define QQT_MODE_(\w+) (\d+)", text))
    assert (modes["STEP"], modes["OBSERVE"], modes["RESET"], modes["PROBE"]) == (
        _capi.MODE_STEP, _capi.MODE_OBSERVE, _capi.MODE_RESET, _capi.MODE_PROBE)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_struct_layouts_match_the_header(tmp_path):
    """offsetof/sizeof of every ctypes field, from a C program built against
    the header, must equal the ctypes mirror's."""
    from qqtsim import _capi

    structs = {"qqt_sim_config": _capi.SimConfigC, "qqt_tick_args": _capi.TickArgsC,
               "qqt_mlp_args": _capi.MlpArgsC, "qqt_bot_args": _capi.BotArgsC,
               "qqt_gae_args": _capi.GaeArgsC, "qqt_l1_grad_args": _capi.L1GradArgsC,
               "qqt_ppo_args": _capi.PpoArgsC, "qqt_cnn_args": _capi.CnnArgsC,
               "qqt_lstm_feat_args": _capi.LstmFeatArgsC, "qqt_lstm_args": _capi.LstmArgsC,
               "qqt_gather_args": _capi.GatherArgsC}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "qqt_hip.h"',
             'int main(void) {']
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ['  return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out.strip().splitlines()}
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def _tick_args(**kw):
    from qqtsim import _capi

    a = _capi.TickArgsC()
    a.n_envs, a.mode = 4, _capi.MODE_OBSERVE
    a.cells, a.players, a.envs = 0x1000, 0x2000, 0x3000   # never dereferenced on these paths
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _cfg(**kw):
    from qqtsim.config import corridor_training_config
    from qqtsim.maps import MapSpec
    from qqtsim.sim import config_struct

    c = config_struct(corridor_training_config(), MapSpec())
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@pytest.mark.parametrize("cfg_kw,args_kw,msg", [
    ({}, dict(n_envs=0), "n_envs"),
    ({}, dict(cells=None), "null state"),
    ({}, dict(mode=7), "bad mode"),
    ({}, dict(mode=0), "STEP needs actions"),
    ({}, dict(mode=2), "RESET needs reset_mask"),
    ({}, dict(mode=3), "PROBE"),
    ({}, dict(obs=0x1008), "16-byte aligned"),
    (dict(fuse=0), {}, "fuse"),
    (dict(fuse=300), {}, "fuse"),
    (dict(bombs_lo=3, bombs_hi=2), {}, "cap ranges"),
])
def test_tick_rejects_bad_arguments(lib, cfg_kw, args_kw, msg):
    rc = lib.qqt_tick(_cfg(**cfg_kw), _tick_args(**args_kw), None)
    assert rc == -1
    assert msg in lib.qqt_last_error().decode()


def test_tick_null_config(lib):
    assert lib.qqt_tick(None, None, None) == -1
    assert b"null" in lib.qqt_last_error()


def test_tick_unsupported_grid(lib):
    rc = lib.qqt_tick(_cfg(height=11, width=11), _tick_args(), None)
    assert rc == -3
    assert b"not compiled" in lib.qqt_last_error()


def _mlp_args(**kw):
    from qqtsim import _capi

    a = _capi.MlpArgsC()
    a.batch, a.npid, a.pid0, a.sample = 8, 2, 0, 0
    a.k0, a.kblocks0, a.obs_stride, a.w0_players = 2366, 37, 2366, 2
    for i, name in enumerate(("obs", "w0", "w1", "wh", "wf", "w1_lo", "wh_lo", "wf_lo", "b0",
                              "ln1_w", "ln1_b", "b1", "ln2_w", "ln2_b", "bh", "bf")):
        setattr(a, name, 0x10000 * (i + 1))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(w1_lo=None), "null pointer"),
    (dict(batch=0), "bad shape"),
    (dict(npid=3), "bad shape"),
    (dict(k0=2365), "bad shape"),
    (dict(kblocks0=36), "bad shape"),
    (dict(obs_stride=2000), "bad shape"),
    (dict(obs=0x10002), "bad shape"),
    (dict(npid=1, pid0=2), "bad shape"),
    (dict(w0_players=1), "bad shape"),
    (dict(sample=1), "sampling needs masks"),
])
def test_mlp_rejects_bad_arguments(lib, kw, msg):
    assert lib.qqt_mlp_act(_mlp_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(out_slot=2, npid=1, out_slots=2), "output slots"),
    (dict(out_slots=1), "output slots"),
    (dict(out_slots=-1), "output slots"),
])
def test_mlp_rejects_bad_output_slots(lib, kw, msg):
    assert lib.qqt_mlp_act(_mlp_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


_CNN_PTRS = ("obs", "view_perm", "c0w", "c0w_lo", "c0b", "ln0w", "ln0b", "c1w", "c1w_lo", "c1b",
             "ln1w", "ln1b", "c2w", "c2w_lo", "c2b", "ln2w", "ln2b", "c3w", "c3w_lo", "c3b",
             "ln3w", "ln3b", "s0h", "s0l", "s0b", "s1w", "s1b", "s3p", "s3b", "s4w", "s4b", "hp",
             "hb", "fw", "fb", "workspace")


def _cnn_args(**kw):
    from qqtsim import _capi

    a = _capi.CnnArgsC()
    a.batch, a.npid, a.obs_stride, a.w_players = 4, 2, 14 * 169, 2
    for i, name in enumerate(_CNN_PTRS):
        setattr(a, name, 0x10000 * (i + 1))
    a.workspace_bytes = 32 * 5504                 # 8 items, rounded up to one 32-item block
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(s3p=None), "null pointer"),
    (dict(view_perm=None), "null pointer"),
    (dict(ln2b=0x10004), "16-byte aligned"),
    (dict(c2w_lo=0x10008), "16-byte aligned"),
    (dict(c1w_lo=None), "null pointer"),
    (dict(obs=None), "null pointer"),
    (dict(batch=0), "bad batch"),
    (dict(npid=3), "bad batch"),
    (dict(obs_stride=2365), "bad batch"),
    (dict(npid=1, pid0=2), "bad batch"),
    (dict(w_players=1), "bad batch"),
    (dict(out_slots=1), "output slots"),
    (dict(npid=1, out_slots=2, out_slot=2), "output slots"),
    (dict(sample=1), "sampling needs masks"),
    (dict(s0l=None), "null pointer"),
    (dict(s0h=0x10002), "16-byte aligned"),
    (dict(workspace=None), "workspace"),
    (dict(workspace=0x10008), "workspace"),
    (dict(workspace_bytes=32 * 5504 - 1), "workspace"),
])
def test_cnn_rejects_bad_arguments(lib, kw, msg):
    assert lib.qqt_cnn_act(_cnn_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


def _lstm_args(**kw):
    from qqtsim import _capi

    a = _capi.LstmArgsC()
    a.batch, a.c_in, a.rows_per_env = 4, 14, 1
    a.local_stride, a.rel_stride, a.glob_stride = 14 * 49, 60, 5
    a.out_stride = 1
    for i, name in enumerate(("local", "rel", "glob", "params", "h", "c")):
        setattr(a, name, 0x10000 * (i + 1))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(params=None), "null pointer"),
    (dict(h=None), "null pointer"),
    (dict(batch=0), "bad shape"),
    (dict(c_in=15), "bad shape"),
    (dict(local_stride=14 * 49 - 1), "bad shape"),
    (dict(rel_stride=59), "bad shape"),
    (dict(rows_per_env=0), "bad shape"),
    (dict(out_slot=1), "bad shape"),
    (dict(sample=1), "sampling needs masks"),
])
def test_lstm_rejects_bad_arguments(lib, kw, msg):
    assert lib.qqt_lstm_act(_lstm_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


def _lstm_feat_args(**kw):
    from qqtsim import _capi

    a = _capi.LstmFeatArgsC()
    a.n_envs, a.p_out = 4, 2
    a.local_stride, a.rel_stride, a.glob_stride = 2 * 14 * 49, 120, 10
    for i, name in enumerate(("cells", "players", "envs", "obs", "local", "rel", "glob")):
        setattr(a, name, 0x10000 * (i + 1))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("cfg_kw,kw,msg", [
    ({}, dict(obs=None), "null pointer"),
    ({}, dict(n_envs=0), "bad sizes"),
    ({}, dict(p_out=3), "bad sizes"),
    (dict(max_hp=0), {}, "bad sizes"),
    ({}, dict(rel_stride=119), "strides"),
    ({}, dict(local_stride=2 * 14 * 49 - 1), "strides"),
    (dict(height=11, width=11), {}, "not compiled"),
])
def test_lstm_features_reject_bad_arguments(lib, cfg_kw, kw, msg):
    assert lib.qqt_lstm_features(_cfg(**cfg_kw), _lstm_feat_args(**kw), None) < 0
    assert msg in lib.qqt_last_error().decode()


def test_lstm_block_size_matches_the_header():
    from qqtsim import policy

    m = re.search(r"#define QQT_LSTM_PARAMS (\d+)", open(HEADER).read())
    assert int(m.group(1)) == policy.LSTM_PARAMS == sum(r * c for _, r, c, _ in policy._LSTM_BLOCKS)


def _bot_args(**kw):
    from qqtsim import _capi

    b = _capi.BotArgsC()
    b.n_envs, b.pid = 4, 1
    for i, name in enumerate(("cells", "players", "obs", "move_mask", "bomb_mask", "actions")):
        setattr(b, name, 0x10000 * (i + 1))
    for k, v in kw.items():
        setattr(b, k, v)
    return b


@pytest.mark.parametrize("kw,msg", [
    (dict(n_envs=0), "null pointer or empty"),
    (dict(obs=None), "null pointer or empty"),
    (dict(actions=None), "null pointer or empty"),
    (dict(pid=2), "bad player id"),
    (dict(pid=-1), "bad player id"),
    (dict(reach_mode=1), "reach buffer"),
    (dict(reach_mode=4, reach=0x9000), "reach buffer"),
])
def test_bot_rejects_bad_arguments(lib, kw, msg):
    assert lib.qqt_bot_act(_cfg(), _bot_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


def test_bot_unsupported_grid(lib):
    assert lib.qqt_bot_act(_cfg(height=11, width=11), _bot_args(), None) == -3


def test_timing_rejects_bad_arguments(lib):
    import ctypes as ct

    assert lib.qqt_timing_arm(-1) == -1
    assert lib.qqt_timing_arm(4097) == -1
    assert b"launches" in lib.qqt_last_error()
    ms, cnt = (ct.c_double * 5)(), (ct.c_int32 * 5)()
    assert lib.qqt_timing_collect(None, cnt, 5) == -1
    assert lib.qqt_timing_collect(ms, cnt, 0) == -1
    # nothing armed or taken: collect succeeds without touching a device
    assert lib.qqt_timing_collect(ms, cnt, 5) == 0
    assert list(cnt) == [0, 0, 0, 0, 0]


def test_header_kernel_kinds_match_host_mirror():
    from qqtsim import _capi

    text = open(HEADER).read()
    kinds = dict((k, int(v)) for k, v in re.findall(r"\bQQT_KERNEL_(\w+) = (\d+)", text))
    assert kinds["KINDS"] == len(_capi.KERNEL_KINDS)
    for name in ("TICK", "MLP", "BOT", "REACH", "GAE", "L1GRAD", "PPO", "CNN"):
        assert _capi.KERNEL_KINDS[kinds[name]].startswith(name.lower()), name


def _gae_args(**kw):
    from qqtsim import _capi

    a = _capi.GaeArgsC()
    a.steps, a.n_envs, a.gamma, a.gamma_lam, a.step_stride, a.env_stride = 8, 4, 0.99, 0.94, 8, 2
    for i, name in enumerate(("rew", "val", "done", "last_val", "adv", "ret")):
        setattr(a, name, 0x10000 * (i + 1))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(rew=None), "null argument"),
    (dict(ret=None), "null argument"),
    (dict(steps=0), "positive"),
    (dict(n_envs=-3), "positive"),
    (dict(step_stride=0), "positive"),
    (dict(env_stride=-1), "positive"),
])
def test_gae_rejects_bad_arguments(lib, kw, msg):
    assert lib.qqt_gae(_gae_args(**kw), None) == -1
    assert msg in lib.qqt_last_error().decode()


def test_errors_raise_in_python(lib):
    from qqtsim import _capi

    with pytest.raises(ValueError, match="n_envs"):
        _capi.check(lib.qqt_tick(_cfg(), _tick_args(n_envs=-1), None))


def test_l1_grad_rejects_bad_arguments(lib):
    """Argument checks run before any launch (no GPU needed)."""
    from qqtsim import _capi

    assert lib.qqt_l1_grad_workspace_floats(0, 2366) == -1
    n = lib.qqt_l1_grad_workspace_floats(5000, 2366)
    assert n == 3 * 128 * 10 * 256          # 3 chunks of 1696 rows, 10 column tiles
    a = _capi.L1GradArgsC()
    assert lib.qqt_l1_grad(ctypes.byref(a), None) == -1
    assert b"null" in lib.qqt_last_error()
    a.batch, a.k0, a.obs_stride, a.workspace_floats = 5000, 2366, 2366, n - 1
    a.obs = a.dz1 = a.workspace = a.dw0 = 1 << 20
    assert lib.qqt_l1_grad(ctypes.byref(a), None) == -1
    assert b"workspace" in lib.qqt_last_error()
    a.workspace_floats, a.k0 = n, 2367
    assert lib.qqt_l1_grad(ctypes.byref(a), None) == -1


def test_integration_doc_lists_every_source():
    """INTEGRATION.md's build section names every source the build compiles."""
    from qqtsim import _build

    doc = open(os.path.join(os.path.dirname(os.path.dirname(__file__)), "INTEGRATION.md")).read()
    missing = [s for s in _build.SOURCES if f"csrc/{s}" not in doc]
    assert missing == [], missing


@pytest.mark.parametrize("kw,msg", [
    (dict(src=None), "null pointer"),
    (dict(index=None), "null pointer"),
    (dict(n=-1), "bad sizes"),
    (dict(row_words=0), "bad sizes"),
    (dict(src_stride=1182), "bad sizes"),
    (dict(dst_stride=1182), "bad sizes"),
])
def test_gather_rejects_bad_arguments(lib, kw, msg):
    from qqtsim import _capi

    a = _capi.GatherArgsC()
    a.n, a.row_words, a.src_rows, a.src_stride, a.dst_stride = 4, 1183, 10, 1183, 1183
    a.src, a.dst, a.index = 0x10000, 0x20000, 0x30000
    for k, v in kw.items():
        setattr(a, k, v)
    assert lib.qqt_gather_rows(a, None) == -1
    assert msg in lib.qqt_last_error().decode()
