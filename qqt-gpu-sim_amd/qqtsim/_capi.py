"""ctypes binding of libqqt_hip.so (include/qqt_hip.h).

The library is loaded after `torch` so that it binds to the HIP runtime torch
already loaded (same SONAME).  Nothing here falls back to a CPU path: a
missing library or a failed launch raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime first)

from ._build import LIB

ABI_VERSION = 25

MODE_STEP, MODE_OBSERVE, MODE_RESET, MODE_PROBE, MODE_FLUSH = 0, 1, 2, 3, 4
MAP_PILLARS, MAP_OPEN, MAP_REFERENCE = 0, 1, 2

_i32, _f32, _u32, _u64, _vp = (ctypes.c_int32, ctypes.c_float, ctypes.c_uint32,
                               ctypes.c_uint64, ctypes.c_void_p)


class SimConfigC(ctypes.Structure):
    _fields_ = [(n, _i32) for n in (
        "height", "width", "n_players", "fuse", "blast", "max_steps", "max_chain",
        "chain_cap_rounds", "max_hp", "invuln_ticks", "hit_attr_penalty",
        "place_dist_cooldown", "growth_bombs_max", "growth_blast_max", "corridor",
        "timeout_draw", "win_hp_scaled")] + [(n, _f32) for n in (
        "radius", "step_len", "pos_hi_y", "pos_hi_x", "step_penalty", "hit_reward",
        "win_bonus", "win_per_hp", "danger_penalty", "brick_reward", "place_cover_reward",
        "place_chain_reward", "place_dist_reward", "place_dist_radius", "chain_time_factor",
        "chain_time_rest", "combo_reward", "combo_gap_factor", "growth_speed_step",
        "growth_speed_max", "hit_speed_drop", "recycle_crate_prob", "growth_crate_prob")] + [
        (n, _i32) for n in ("map_kind", "swap_spawns", "bombs_lo", "bombs_hi", "blast_lo",
                            "blast_hi", "spawn_cooldown")] + [
        (n, _f32) for n in ("brick_p", "spawn_speed")] + [
        (n, _i32) for n in ("top_wall_rows", "random_wall_rows", "corridor_width",
                            "open_obstacle_max", "ring_center_h", "ring_center_w",
                            "open_crate_cross", "max_bombs", "growth_bombs_start",
                            "growth_blast_start", "open_growth_bombs", "open_growth_blast",
                            "opp_growth_bombs", "opp_growth_blast")] + [
        (n, _f32) for n in ("thr_pure", "thr_open", "thr_ring", "wall_density",
                            "ring_brick_density", "ring_crate_prob", "growth_speed_start",
                            "open_growth_speed", "opp_growth_speed", "opp_hist_mult")] + [
        ("ref_spawn_y", (_f32 * 4) * 3), ("ref_spawn_x", (_f32 * 4) * 3),
        ("ref_spawn_cell", (_i32 * 4) * 3)]


class TickArgsC(ctypes.Structure):
    _fields_ = [("n_envs", _i32), ("mode", _i32), ("auto_reset", _i32),
                ("resolve_tiers", _i32), ("explore_coef", _f32), ("danger_coef", _f32),
                ("seed", _u64), ("tick", _u32), ("epoch", _u32)] + [
        (n, _vp) for n in ("cells", "players", "envs", "actions", "actions_i8", "crate_u",
                           "reset_mask", "reward", "done", "n_alive", "died", "winner",
                           "covered", "triggered", "obs", "move_mask", "bomb_mask",
                           "probe_out", "damaged", "recycle_excl")] + [("opp_boost", _i32),
                                                                        ("danger_out", _vp),
                                                                        ("tick_stats", _vp),
                                                                        ("reach_caps", _vp),
                                                                        ("reach_pid", _i32)]


class MlpArgsC(ctypes.Structure):
    _fields_ = [(n, _i32) for n in (
        "batch", "npid", "pid0", "sample", "k0", "kblocks0", "obs_stride", "mm_row_stride",
        "mm_pid_stride", "bm_row_stride", "bm_pid_stride")] + [
        ("seed", _u64), ("tick", _u32), ("w0_players", _i32)] + [
        (n, _vp) for n in ("obs", "w0", "w1", "wh", "wf", "w1_lo", "wh_lo", "wf_lo", "b0", "ln1_w", "ln1_b", "b1",
                           "ln2_w", "ln2_b", "bh", "bf", "move_mask", "bomb_mask", "uniforms",
                           "actions", "actions_i8", "logp_out", "value_out", "logits_out")] + [
        ("out_slots", _i32), ("out_slot", _i32), ("z1_out", _vp), ("row_index", _vp),
        ("obs_rows", ctypes.c_int64)] + [
        (n, _i32) for n in ("sparse", "channels", "cells")] + [
        ("dense_mask", _u32), ("w0g", _vp), ("w0d", _vp),
        ("vmap", (ctypes.c_int8 * 16) * 4)]


class BotArgsC(ctypes.Structure):
    _fields_ = [("n_envs", _i32), ("pid", _i32), ("seed", _u64), ("tick", _u32),
                ("reach_mode", _i32), ("reach_slot", _i32)] + [
        (n, _vp) for n in ("cells", "players", "obs", "move_mask", "bomb_mask", "uniforms",
                           "reach", "reach_caps", "actions", "actions_i8", "mode",
                           "mode_timer")] + [("mode_tick", _u32), ("reserved", _i32)]


class L1GradArgsC(ctypes.Structure):
    _fields_ = [("batch", _i32), ("k0", _i32), ("obs_stride", _i32), ("reserved", _i32),
                ("workspace_floats", ctypes.c_int64)] + [
        (n, _vp) for n in ("obs", "dz1", "dz_scale", "workspace", "dw0", "row_index")] + [
        ("obs_rows", ctypes.c_int64)]


class PpoArgsC(ctypes.Structure):
    _fields_ = [("batch", _i32)] + [(n, _f32) for n in (
        "clip_eps", "ratio_lo", "ratio_hi", "value_coef", "entropy_coef")] + [
        (n, _vp) for n in ("z1", "ln1_w", "ln1_b", "w1", "w1t", "b1", "ln2_w", "ln2_b", "wh",
                           "wht", "bh", "wf", "bf", "actions", "move_mask", "bomb_mask",
                           "old_logp", "adv", "ret", "old_val", "dz1", "h1", "dz2", "h2", "hy",
                           "dhy", "dl", "ln_part", "stats_part", "bias_part",
                           "dz1_absmax_part")] + [("t_chunk", _i32), ("reserved", _i32),
                                                   ("row_index", _vp), ("src_rows", ctypes.c_int64)]


class CnnArgsC(ctypes.Structure):
    _fields_ = [(n, _i32) for n in (
        "batch", "npid", "pid0", "sample", "obs_stride", "mm_row_stride", "mm_pid_stride",
        "bm_row_stride", "bm_pid_stride", "w_players")] + [
        ("seed", _u64), ("tick", _u32), ("out_slots", _i32), ("out_slot", _i32),
        ("reserved", _i32)] + [
        (n, _vp) for n in ("obs", "view_perm", "c0w", "c0w_lo", "c0b", "ln0w", "ln0b", "c1w",
                           "c1w_lo", "c1b", "ln1w", "ln1b", "c2w", "c2w_lo", "c2b", "ln2w",
                           "ln2b", "c3w", "c3w_lo", "c3b", "ln3w", "ln3b", "s0h", "s0l", "s0b", "s1w", "s1b",
                           "s3p", "s3b", "s4w", "s4b", "hp", "hb", "fw", "fb", "move_mask",
                           "bomb_mask", "uniforms", "actions", "actions_i8", "logp_out",
                           "value_out", "logits_out", "workspace")] + [
        ("workspace_bytes", ctypes.c_int64)]


class GatherArgsC(ctypes.Structure):
    _fields_ = [("n", _i32), ("row_words", _i32)] + [
        (n, ctypes.c_int64) for n in ("src_rows", "src_stride", "dst_stride")] + [
        (n, _vp) for n in ("src", "dst", "index")]


class LstmFeatArgsC(ctypes.Structure):
    _fields_ = [("n_envs", _i32), ("p_out", _i32)] + [
        (n, _vp) for n in ("cells", "players", "envs", "obs", "local", "rel", "glob")] + [
        (n, ctypes.c_int64) for n in ("local_stride", "rel_stride", "glob_stride")]


class LstmArgsC(ctypes.Structure):
    _fields_ = [(n, _i32) for n in ("batch", "c_in", "rows_per_env", "pid0", "sample")] + [
        ("seed", _u64), ("tick", _u32)] + [
        (n, _vp) for n in ("local", "rel", "glob")] + [
        (n, ctypes.c_int64) for n in ("local_stride", "rel_stride", "glob_stride")] + [
        (n, _vp) for n in ("params", "h", "c", "reset", "move_mask", "bomb_mask")] + [
        ("mm_row_stride", _i32), ("bm_row_stride", _i32), ("uniforms", _vp),
        ("out_stride", _i32), ("out_slot", _i32)] + [
        (n, _vp) for n in ("actions", "actions_i8", "logp_out", "value_out", "logits_out")]


class GaeArgsC(ctypes.Structure):
    _fields_ = [("steps", _i32), ("n_envs", _i32), ("gamma", _f32), ("gamma_lam", _f32),
                ("step_stride", ctypes.c_int64), ("env_stride", ctypes.c_int64)] + [
        (n, _vp) for n in ("rew", "val", "done", "last_val", "adv", "ret")]


_LIB = None


def lib():
    """The loaded library (raises if it is missing or has another ABI)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB):
            raise RuntimeError(
                f"{LIB} is not built; run `python -m qqtsim._build` (HIP path required)")
        L = ctypes.CDLL(LIB)
        L.qqt_abi_version.restype = ctypes.c_int
        L.qqt_last_error.restype = ctypes.c_char_p
        L.qqt_tick.restype = ctypes.c_int
        L.qqt_tick.argtypes = [ctypes.POINTER(SimConfigC), ctypes.POINTER(TickArgsC), _vp]
        L.qqt_mlp_act.restype = ctypes.c_int
        L.qqt_mlp_act.argtypes = [ctypes.POINTER(MlpArgsC), _vp]
        L.qqt_bot_act.restype = ctypes.c_int
        L.qqt_bot_act.argtypes = [ctypes.POINTER(SimConfigC), ctypes.POINTER(BotArgsC), _vp]
        L.qqt_gae.restype = ctypes.c_int
        L.qqt_gae.argtypes = [ctypes.POINTER(GaeArgsC), _vp]
        L.qqt_l1_grad.restype = ctypes.c_int
        L.qqt_l1_grad.argtypes = [ctypes.POINTER(L1GradArgsC), _vp]
        L.qqt_l1_grad_noalloc.restype = ctypes.c_int
        L.qqt_l1_grad_noalloc.argtypes = [ctypes.POINTER(L1GradArgsC), _vp]
        L.qqt_l1_grad_workspace_floats.restype = ctypes.c_int64
        L.qqt_l1_grad_workspace_floats.argtypes = [_i32, _i32]
        L.qqt_ppo_grad.restype = ctypes.c_int
        L.qqt_ppo_grad.argtypes = [ctypes.POINTER(PpoArgsC), _vp]
        L.qqt_cnn_act.restype = ctypes.c_int
        L.qqt_cnn_act.argtypes = [ctypes.POINTER(CnnArgsC), _vp]
        L.qqt_lstm_features.restype = ctypes.c_int
        L.qqt_lstm_features.argtypes = [ctypes.POINTER(SimConfigC), ctypes.POINTER(LstmFeatArgsC),
                                        _vp]
        L.qqt_gather_rows.restype = ctypes.c_int
        L.qqt_gather_rows.argtypes = [ctypes.POINTER(GatherArgsC), _vp]
        L.qqt_lstm_act.restype = ctypes.c_int
        L.qqt_lstm_act.argtypes = [ctypes.POINTER(LstmArgsC), _vp]
        L.qqt_timing_arm.restype = ctypes.c_int
        L.qqt_timing_arm.argtypes = [_i32]
        L.qqt_timing_collect.restype = ctypes.c_int
        L.qqt_timing_collect.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i32), _i32]
        if L.qqt_abi_version() != ABI_VERSION:
            raise RuntimeError("libqqt_hip.so ABI version mismatch; rebuild it")
        _LIB = L
    return _LIB


KERNEL_KINDS = ("tick_kernel", "mlp_act_kernel", "bot_kernel", "reach_kernel",
                "gae_kernel", "l1grad_kernels", "ppo_grad_kernel", "cnn_trunk_kernel",
                "lstm_feat_kernel", "lstm_act_kernel", "cnn_head_kernel")  # QQT_KERNEL_*


def timing_arm(launches: int) -> None:
    """Time the next `launches` kernel launches of the library (each on its
    own dispatch packet)."""
    check(lib().qqt_timing_arm(int(launches)))


def timing_collect() -> dict:
    """{kernel name: (summed ms, timed launches)} of the armed launches since
    the last collect (waits for them)."""
    n = len(KERNEL_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int32 * n)()
    check(lib().qqt_timing_collect(ms, cnt, n))
    return {k: (ms[i], cnt[i]) for i, k in enumerate(KERNEL_KINDS) if cnt[i]}


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().qqt_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(msg)
        raise RuntimeError(f"qqt_hip error {rc}: {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
