// The STEP tick for gfx950 with a group of envs per wavefront: step +
// auto-reset + danger + observation + legality masks of four envs per
// 64-lane wavefront, one env per 16-lane DPP row.
//
// Layout:
// * lane l of an env's row holds the env's cells c = l + 16k (k < KC) as
//   packed cell words in registers; every cell-parallel phase (fuse
//   countdown, live counts, bomb lists, brick burn, clears, observation
//   channels, state store) runs on those registers;
// * lane i < P of the row holds player i's record in registers; the
//   per-player phases (placement, movement, damage, rewards, splat) run on
//   those lanes for the four envs of the wavefront at once, and any lane
//   reads player i's value with one DPP row broadcast (row_newbcast:i);
// * LDS holds per env, in a 2.4 KB block, only what is read at random
//   (a copy of the cell words for ray walks and movement probes) or
//   scattered into (the flame cover bytes, the danger map, the danger
//   front): a workgroup is one wavefront, so all 16,384 envs of a large
//   batch are resident at once (16 wavefronts per CU);
// * the observation is staged in the env's (then dead) LDS block in output
//   layout and copied out with 16-byte stores: all channels in one pass for
//   two-player envs at 32 lanes (a 4.75 KB block: 16 wavefronts per CU at
//   8192 envs still fit), else in passes of seven channels.
//
// Semantics and float32 operation order follow the per-env kernel in
// tick.hip, which follows the reference tick (sim/torch_sim.py:895-1261)
// stage by stage; the library is built with -ffp-contract=off.
//
// The explosion trigger stamp of a cell (0 = not triggered, else the round
// that triggered it + 1, saturating at 15) lives in bits 28-31 of the LDS
// copy of its word while the explosion resolves; the words written back
// carry no stamp.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"
#include "tick_rules.h"

namespace qqt {

int fail(int code, const char* msg);

namespace grp {

constexpr uint32_t STAMP_MASK = 0xF0000000u;
constexpr int STAMP_SHIFT = 28;

template <int H, int W, int P, int L>
struct Geo {
  static_assert(L == 16 || L == 32, "an env takes one or two DPP rows");
  static constexpr int C = H * W;
  static constexpr int KC = (C + L - 1) / L;       // cells per lane
  static constexpr int NCH = 5 * P + 4;
  static constexpr int OBS = NCH * C;
  // observation channels per staging pass
  static constexpr int CPP = (L == 32 && NCH * C * 2 <= 5120) ? NCH : 7;
  static constexpr int NPASS = (NCH + CPP - 1) / CPP;
  static constexpr int C4 = (C + 3) / 4 * 4;
  // block: cell words | danger front / weight by cell | danger map | cover bytes | bomb list
  static constexpr int O_FW = 4 * C, O_DNG = 8 * C, O_COV = 12 * C, O_LIST = 12 * C + C4;
  static constexpr int STATE = 12 * C + 2 * C4;
  static constexpr int STAGE = CPP * C * 2 + 15;   // one pass, placed at the output's address mod 16
  static constexpr int BLOCK = ((STATE > STAGE ? STATE : STAGE) + 15) / 16 * 16;
  static_assert(C <= 255, "cell indices are stored as bytes");
};

// ---------------------------------------------------------------- row helpers
template <int K>
__device__ __forceinline__ int rbc(int v) {      // lane K of this lane's row
  return __builtin_amdgcn_update_dpp(0, v, 0x150 + K, 0xF, 0xF, false);
}
template <int K>
__device__ __forceinline__ float rbcf(float v) {
  return __int_as_float(rbc<K>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// sum over the 16 lanes of the row, in every lane
__device__ __forceinline__ int row_sum(int v) {
  v += dpp<0x128>(v);   // row_ror:8
  v += dpp<0x124>(v);   // row_ror:4
  v += dpp<0x122>(v);   // row_ror:2
  v += dpp<0x121>(v);   // row_ror:1
  return v;
}
// sum over the L lanes of the env, in every lane
template <int L>
__device__ __forceinline__ int env_sum(int v) {
  v = row_sum(v);
  if constexpr (L == 32) {
    // v_permlane16_swap of v with itself: element 0 holds the even row's
    // values in both rows of each pair, element 1 the odd row's
    const auto pr = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = (int)(pr[0] + pr[1]);
  }
  return v;
}
// the L ballot bits of env e
template <int L>
__device__ __forceinline__ uint32_t env_bits(bool pred, int e) {
  const uint64_t b = __ballot(pred);
  return (uint32_t)(b >> (L * e)) & (L == 32 ? 0xFFFFFFFFu : 0xFFFFu);
}
// partner lanes l ^ 1 and l ^ 2 of a quad
__device__ __forceinline__ float qx1(float v) { return __int_as_float(dpp<0xB1>(__float_as_int(v))); }
__device__ __forceinline__ float qx2(float v) { return __int_as_float(dpp<0x4E>(__float_as_int(v))); }
__device__ __forceinline__ int qx1i(int v) { return dpp<0xB1>(v); }
__device__ __forceinline__ int qx2i(int v) { return dpp<0x4E>(v); }

template <int P>
__device__ __forceinline__ int sel(const int (&v)[P], int i) {
  int r = v[0];
#pragma unroll
  for (int j = 1; j < P; ++j) r = i == j ? v[j] : r;
  return r;
}
template <int P>
__device__ __forceinline__ float self(const float (&v)[P], int i) {
  float r = v[0];
#pragma unroll
  for (int j = 1; j < P; ++j) r = i == j ? v[j] : r;
  return r;
}
template <int P>
__device__ __forceinline__ void bcast_all(int v, int (&out)[P]) {
  out[0] = rbc<0>(v);
  if constexpr (P > 1) out[1] = rbc<1>(v);
  if constexpr (P > 2) out[2] = rbc<2>(v);
  if constexpr (P > 3) out[3] = rbc<3>(v);
}
template <int P>
__device__ __forceinline__ void bcast_allf(float v, float (&out)[P]) {
  out[0] = rbcf<0>(v);
  if constexpr (P > 1) out[1] = rbcf<1>(v);
  if constexpr (P > 2) out[2] = rbcf<2>(v);
  if constexpr (P > 3) out[3] = rbcf<3>(v);
}

__device__ __forceinline__ uint16_t h16(float v) { return __half_as_ushort(__float2half_rn(v)); }

// f / F correctly rounded, for integers 0 <= f <= 255 and 1 <= F <= 255,
// from rcp = f32(1 / F): the product's residual, one fused correction.
// Equal to the IEEE quotient for every such pair (checked exhaustively in
// exact rational arithmetic).
__device__ __forceinline__ float qdiv(int f, float F, float rcp) {
  const float ff = (float)f;
  const float q0 = ff * rcp;
  return fmaf(fmaf(-q0, F, ff), rcp, q0);
}
// Danger weight (1 - (f-1)/F)^2 clamped at 0 (sim/blast.py:218-220) for a
// bomb's fuse f >= 1.
__device__ __forceinline__ float fuse_weight(int f, float F, float rcp) {
  const float raw = 1.0f - qdiv(f - 1, F, rcp);
  const float v = raw > 0.0f ? raw : 0.0f;
  return v * v;
}

// Player record (slots QQT_P_*) in the registers of the player's lane.
struct Rec {
  float y, x;
  int alive, hp, since, bcap, zcap;
  float spd;
  int inv, combo, last_hit, pend, lob, loz;
  float los;
  int pad;
};

// The kernel's argument segment: the config at offset 0, the arguments after
// it at their 8-byte alignment (the by-value parameter layout).
typedef const __attribute__((address_space(4))) qqt_sim_config* CfgP;
typedef const __attribute__((address_space(4))) qqt_tick_args* ArgP;
constexpr size_t ARGS_OFFSET = (sizeof(qqt_sim_config) + alignof(qqt_tick_args) - 1) /
                               alignof(qqt_tick_args) * alignof(qqt_tick_args);
__device__ __forceinline__ CfgP cfg_ptr() { return (CfgP)__builtin_amdgcn_kernarg_segment_ptr(); }
__device__ __forceinline__ ArgP args_ptr() {
  return (ArgP)((const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr() +
                ARGS_OFFSET);
}

// ---------------------------------------------------------------- kernel
template <int H, int W, int P, int MAPS, int L>
__global__ __launch_bounds__(64, 4) void tick_group_kernel(const qqt_sim_config cf,
                                                           const qqt_tick_args a) {
  using G = Geo<H, W, P, L>;
  constexpr int EPW = 64 / L;   // envs per wavefront (= workgroup)
  constexpr int C = G::C, KC = G::KC, OBS = G::OBS;
  // The config and arguments are read through pointers into the kernel's own
  // argument segment, so each field is loaded (scalar loads) where it is used
  // instead of all of them at entry and kept live through the whole tick.
  const CfgP CF = cfg_ptr();
  const ArgP A = args_ptr();
  static_assert(XCD_ROWS % EPW == 0, "whole wavefronts per row block");
  constexpr int WGRB = XCD_ROWS / EPW;
  __shared__ __align__(16) uint8_t lds[EPW * G::BLOCK];

  const int lane = threadIdx.x;
  // env e of the wavefront; lane l of the env (its cells are l + L k); lane
  // lr of the 16-lane row (a two-row env holds its player records in both
  // rows, so that player values move with row broadcasts)
  const int e = lane / L, l = lane % L, lr = lane & 15;
  // workgroups are dealt to the 8 XCDs round robin; block b takes the envs
  // of XCD_ROWS-env row block (b / 8 / WGRB) * 8 + b % 8, as the act kernel
  // deals its rows, so an env stays in one XCD's L2 from kernel to kernel
  const int seq = blockIdx.x >> 3;
  const int rb = (seq / WGRB) * 8 + (blockIdx.x & 7);
  const int g0 = rb * XCD_ROWS + (seq % WGRB) * EPW;
  if (g0 >= A->n_envs) return;
  const int n_envs = A->n_envs;
  const int g = g0 + e;
  const bool valid = g < n_envs;
  const size_t gs = valid ? (size_t)g : (size_t)g0;

  uint8_t* blk = lds + e * G::BLOCK;
  uint32_t* cwl = reinterpret_cast<uint32_t*>(blk);
  float* fw = reinterpret_cast<float*>(blk + G::O_FW);
  float* dng = reinterpret_cast<float*>(blk + G::O_DNG);
  uint8_t* cov = blk + G::O_COV;
  uint8_t* list = blk + G::O_LIST;
  const float rad = CF->radius;
  const float fmax_f = (float)CF->fuse;
  const float frcp = __fdiv_rn(1.0f, fmax_f);
  const int cfg_blast = CF->blast;
  const bool corridor = CF->corridor != 0;

  // ---- load: cells into registers, players into their lanes, env record
  const int32_t* const cells_in = A->cells + gs * C;
  uint32_t cw[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    cw[k] = (valid && c < C) ? (uint32_t)cells_in[c] : (F_WALL | EMPTY_CELL);
  }
  const int pi = lr < P ? lr : 0;   // player of this lane (other lanes carry a copy of player 0)
  Rec r;
  {
    const int4* q = reinterpret_cast<const int4*>(A->players + (gs * P + pi) * QQT_P_SLOTS);
    const int4 q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
    r.y = __int_as_float(q0.x); r.x = __int_as_float(q0.y); r.alive = q0.z; r.hp = q0.w;
    r.since = q1.x; r.bcap = q1.y; r.zcap = q1.z; r.spd = __int_as_float(q1.w);
    r.inv = q2.x; r.combo = q2.y; r.last_hit = q2.z; r.pend = q2.w;
    r.lob = q3.x; r.loz = q3.y; r.los = __int_as_float(q3.z); r.pad = q3.w;
  }
  int4 ev = *reinterpret_cast<const int4*>(A->envs + gs * QQT_E_SLOTS);
  int in_mv = 4, in_bb = 0;
  float in_uh = 0.0f, in_ug = 0.0f;
  if (lr < P && valid) {
    const size_t ai = (gs * P + lr) * 2;
    if (A->actions) {
      in_mv = (int)A->actions[ai];
      in_bb = (int)A->actions[ai + 1];
    } else {
      in_mv = A->actions_i8[ai];
      in_bb = A->actions_i8[ai + 1];
    }
    if (A->crate_u) {
      in_uh = A->crate_u[((size_t)lr * 2 + 0) * n_envs + g];
      in_ug = A->crate_u[((size_t)lr * 2 + 1) * n_envs + g];
    }
  }

  // ---- 1. snapshots, fuse countdown, live counts (8 bits per player)
  const int alive0 = r.alive, hp0 = r.hp;
  const int fpre = min(max((int)floorf(r.y) * W + (int)floorf(r.x), 0), C - 1);
  int livepack = 0;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int f = cw_fuse(cw[k]);
    if (f > 0) cw[k] -= 1u;
    const int o = cw_owner(cw[k]);
    if (cw_fuse(cw[k]) > 0 && o >= 0 && o < P) livepack += 1 << (8 * o);
  }
  livepack = env_sum<L>(livepack);
  const int my_live = (livepack >> (8 * pi)) & 0xFF;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    if (c < C) cwl[c] = cw[k];
  }
  wave_sync();

  // ---- 2. placement, players in id order (sim/torch_sim.py:1357-1402):
  // a player's bomb also blocks the cell for every later player
  const uint32_t wpre = cwl[fpre];
  int placed = (lr < P && alive0 && in_bb == 1 && cw_fuse(wpre) <= 0 && !(wpre & F_BRICK) &&
                my_live < r.bcap) ? 1 : 0;
  int fpre_b[P], alive_b[P], placed_b[P];
  bcast_all<P>(fpre, fpre_b);
  bcast_all<P>(alive0, alive_b);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int pb = i == 0 ? rbc<0>(placed) : i == 1 ? rbc<1>(placed) : i == 2 ? rbc<2>(placed)
                                                                       : rbc<3>(placed);
    placed_b[i] = pb;
    if (lr > i && pb && fpre_b[i] == fpre) placed = 0;
  }
  const bool any_placed = __any(placed != 0);
  if (any_placed) {
    if (placed && l < P) cwl[fpre] = cw_make(wpre, CF->fuse, lr, r.zcap);
    int zcap_b[P];
    bcast_all<P>(r.zcap, zcap_b);
#pragma unroll
    for (int i = 0; i < P; ++i) {
#pragma unroll
      for (int k = 0; k < KC; ++k)
        if (placed_b[i] && fpre_b[i] == l + L * k) cw[k] = cw_make(cw[k], CF->fuse, i, zcap_b[i]);
    }
  }
  wave_sync();

  // ---- 3. placement reward (sim/torch_sim.py:1263-1355): lane = me*4 + dir
  float pbonus = 0.0f;
  if (any_placed) {
    const int me = lr >> 2, d = lr & 3;
    const float ctf = CF->chain_time_factor, ctr = CF->chain_time_rest;
    float ypre_b[P], xpre_b[P];
    int since_b[P];
    bcast_allf<P>(r.y, ypre_b);
    bcast_allf<P>(r.x, xpre_b);
    bcast_all<P>(r.since, since_b);
    float chain = 0.0f;
    int cover_bits = 0;
    const bool me_placed = me < P && sel<P>(placed_b, me);
    if (me_placed) {
      const int s0 = sel<P>(fpre_b, me);
      const uint32_t w0 = cwl[s0];
      if (!(w0 & (F_WALL | F_BRICK))) {
        auto visit = [&](int x, uint32_t wx) {
#pragma unroll
          for (int o = 0; o < P; ++o)
            if (o != me && fpre_b[o] == x && alive_b[o]) cover_bits |= 1 << o;
          const int fx = cw_fuse(wx);
          if (fx > 0 && cw_owner(wx) >= 0) {
            int pm = 0;
#pragma unroll
            for (int i = 0; i < P; ++i)
              if (fpre_b[i] == x) pm = placed_b[i];
            if (!pm) {
              float frac = qdiv(fx, fmax_f, frcp);
              frac = fminf(fmaxf(frac, 0.0f), 1.0f);
              const float wt = ctf + ctr * (1.0f - frac);
              chain = chain + wt;
            }
          }
        };
        if (d == 0) visit(s0, w0);
        walk_ray<H, W>(cwl, s0, d, blast_of(w0, cfg_blast), 1, [&](int, int x, uint32_t wx) {
          if (wx & F_WALL) return false;
          visit(x, wx);
          return !cw_solid(wx);
        });
      }
    }
    chain += qx1(chain);
    chain += qx2(chain);
    cover_bits |= qx1i(cover_bits);
    cover_bits |= qx2i(cover_bits);
    float bonus = 0.0f;
    if (me_placed && d == 0) {
      float cover = 0.0f, dist = 0.0f;
#pragma unroll
      for (int o = 0; o < P; ++o) cover += (float)((cover_bits >> o) & 1);
      if (CF->place_dist_reward > 0.0f) {
        // the players' positions and cooldowns are pre-move values here
        const float ym = floorf(self<P>(ypre_b, me)), xm = floorf(self<P>(xpre_b, me));
        const bool cool = sel<P>(since_b, me) >= CF->place_dist_cooldown;
#pragma unroll
        for (int o = 0; o < P; ++o) {
          if (o == me) continue;
          const float dy = ym - floorf(ypre_b[o]);
          const float dx = xm - floorf(xpre_b[o]);
          const float dd = sqrtf(dy * dy + dx * dx);
          const bool under = (cover_bits >> o) & 1;
          const bool ok = !under && dd < CF->place_dist_radius && cool && alive_b[o];
          const float gain = 1.0f - __fdiv_rn(dd, CF->place_dist_radius);
          dist = dist + (ok ? fmaxf(gain, 0.0f) : 0.0f);
        }
      }
      bonus = (CF->place_cover_reward * cover + CF->place_dist_reward * dist) +
              CF->place_chain_reward * chain;
      bonus = bonus * (float)sel<P>(alive_b, me);
    }
    // lane 4i holds player i's bonus
    float bb[P];
    bb[0] = rbcf<0>(bonus);
    if constexpr (P > 1) bb[1] = rbcf<4>(bonus);
    if constexpr (P > 2) bb[2] = rbcf<8>(bonus);
    if constexpr (P > 3) bb[3] = rbcf<12>(bonus);
    pbonus = self<P>(bb, pi);
  }

  // ---- 4. since_bomb; 5. movement (sim/move.py:234-279), both axes from
  // the pre-move box, in the player's lane
  if (lr < P) {
    const int mc = min(max(in_mv, 0), 4);
    const float st = CF->step_len;
    const float tvy = mc == 0 ? -st : (mc == 1 ? st : 0.0f);
    const float tvx = mc == 2 ? -st : (mc == 3 ? st : 0.0f);
    float dy = tvy * r.spd, dx = tvx * r.spd;
    if (!(alive0 && in_mv != 4)) { dy = 0.0f; dx = 0.0f; }
    const float ny = resolve_axis<H, W>(cwl, r.y + dy, dy, r.y, r.x, rad, true);
    const float nx = resolve_axis<H, W>(cwl, r.x + dx, dx, r.y, r.x, rad, false);
    float oy = dy != 0.0f ? ny : r.y;
    float ox = dx != 0.0f ? nx : r.x;
    oy = fminf(fmaxf(oy, rad), CF->pos_hi_y);
    ox = fminf(fmaxf(ox, rad), CF->pos_hi_x);
    r.since = placed ? 0 : r.since + 1;
    r.y = oy;
    r.x = ox;
  }

  // ---- 6. explosions (sim/blast.py:101-155), fixed synchronous rounds over
  // the list of bomb cells (live or due)
  {
    uint32_t* cv32 = reinterpret_cast<uint32_t*>(cov);
#pragma unroll
    for (int m = 0; m < (G::C4 / 4 + L - 1) / L; ++m)
      if (l + L * m < G::C4 / 4) cv32[l + L * m] = 0u;
  }
  bool boom = false;
  int nl = 0;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    const uint32_t w = cw[k];
    const bool in = c < C && (cw_fuse(w) > 0 || cw_owner(w) >= 0);
    const uint32_t bits = env_bits<L>(in, e);
    if (in) list[nl + __popc(bits & ((1u << l) - 1u))] = (uint8_t)c;
    nl += __popc(bits);
    const bool due = c < C && cw_fuse(w) == 0 && cw_owner(w) >= 0;
    if (due) {
      cwl[c] = w | (1u << STAMP_SHIFT);
      if (!(w & (F_WALL | F_BRICK))) cov[c] = 1;
    }
    boom |= due;
  }
  const bool env_boom = env_bits<L>(boom, e) != 0;
  const bool wave_boom = __any(boom);
  if (wave_boom) {
    wave_sync();
    // rays of the list entries whose trigger stamp is `stamp`, one (entry,
    // direction) per lane: walls stop a ray before the cell, other solids after it
    // a ray that covers a live bomb not yet triggered makes another round
    // necessary; without one the remaining rounds trigger nothing
    bool hit_live = false;
    const int tiers = A->resolve_tiers;
    auto fire = [&](uint32_t stamp) {
      hit_live = false;
      for (int it = l; it < 4 * nl; it += L) {
        const int src = list[it >> 2], d = it & 3;
        const uint32_t w = cwl[src];
        const int b = blast_of(w, cfg_blast);
        if ((w >> STAMP_SHIFT) != stamp || (w & (F_WALL | F_BRICK)) || b > tiers) continue;
        walk_ray<H, W>(cwl, src, d, b, 1, [&](int, int x, uint32_t wx) {
          if (wx & F_WALL) return false;
          cov[x] = 1;
          if (cw_fuse(wx) > 0 && (wx >> STAMP_SHIFT) == 0u) hit_live = true;
          return !cw_solid(wx);
        });
      }
    };
    // round 0 fires the due bombs; round r >= 1 first marks the live bombs
    // the flames cover (stamp r + 1), then fires them
    const int rounds = min(CF->max_chain - 1, CF->chain_cap_rounds);
    for (int rr = 0; rr <= rounds; ++rr) {
      // stamps saturate at 15: from round 14 on, the bombs stamped 15 fire
      // again each round, which changes nothing (cover writes are idempotent)
      const uint32_t stamp = (uint32_t)min(rr + 1, 15);
      if (rr > 0) {
        wave_sync();
        bool newly = false;
        for (int j = l; j < nl; j += L) {
          const int c = list[j];
          const uint32_t w = cwl[c];
          if (cw_fuse(w) > 0 && cov[c] && (w >> STAMP_SHIFT) == 0u) {
            cwl[c] = w | (stamp << STAMP_SHIFT);
            newly = true;
          }
        }
        if (!__any(newly)) break;
        wave_sync();
      }
      fire(stamp);
      if (!__any(hit_live)) break;
    }
    wave_sync();
  }

  // ---- 7. damage at the post-move centre cell (sim/torch_sim.py:1007-1034)
  int n_died = 0;                 // deaths among the players of row 0 (tick_stats)
  const int fpost = min(max((int)floorf(r.y) * W + (int)floorf(r.x), 0), C - 1);
  {
    const bool hit = alive0 && cov[fpost];
    const bool hit_eff = hit && r.inv <= 0;
    const int hp_new = max(r.hp - (int)hit_eff, 0);
    const bool died = hit_eff && hp_new == 0;
    r.hp = hp_new;
    r.alive = alive0 && !died;
    int inv = max(r.inv - 1, 0);
    if (hit_eff) inv = CF->invuln_ticks;
    r.inv = inv;
    if (valid && l < P && A->died) A->died[gs * P + l] = died;
    n_died = (valid && l < P && died) ? 1 : 0;
  }

  // ---- 8. burnt bricks (corridor: into crates), info bitsets, clear the
  // exploded cells, then the LDS copy takes the cleared words
  uint32_t covw = 0, trgw = 0;   // lane w < 8: word w of the env's bitsets
  int n_trg = 0;                  // exploded bombs among this lane's cells (tick_stats)
  if (wave_boom) {
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int c = l + L * k;
      bool cvd = false, trg = false;
      if (c < C) {
        cvd = cov[c] != 0;
        trg = (cwl[c] >> STAMP_SHIFT) != 0u;
        uint32_t w = cw[k];
        if (env_boom && cvd && (w & F_BRICK)) {
          if (corridor) w |= F_CRATE;
          w &= ~F_BRICK;
        }
        if (trg) w = cw_make(w, 0, -1, 0);
        n_trg += trg && valid;
        cw[k] = w;
        cwl[c] = w;
      }
      const uint32_t bc = env_bits<L>(cvd, e), bt = env_bits<L>(trg, e);
      if (((L * k) >> 5) == l) {   // cells L k .. L k + L - 1 sit at bit (L k) % 32 of word (L k) / 32
        covw |= bc << ((L * k) & 31);
        trgw |= bt << ((L * k) & 31);
      }
    }
  }
  if (valid && l < 8) {
    if (A->covered) A->covered[gs * 8 + l] = covw;
    if (A->triggered) A->triggered[gs * 8 + l] = trgw;
  }

  // ---- 9. danger map of the post-clear state (sim/blast.py:158-317)
  int nb = 0;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    const bool in = c < C && cw_fuse(cw[k]) > 0;
    const uint32_t bits = env_bits<L>(in, e);
    if (in) list[nb + __popc(bits & ((1u << l) - 1u))] = (uint8_t)c;
    nb += __popc(bits);
  }
  bool has_danger = nb > 0;
  if (__any(has_danger)) {
    wave_sync();
    // Stage A, synchronous relay rounds over (bomb, direction) items, one per
    // lane: bomb j = item / 4 looks back along direction item % 4 for its
    // in-neighbour, the first solid cell behind it, kept if it is a bomb
    // whose range reaches j (bombs on walls have none; walls are senders
    // like any bomb: the reference's stage-A origins are not masked by
    // passability).  The quad's largest sender front is j's spread; a bomb
    // whose spread beats its weight takes the spread as weight and as next
    // round's front, every other bomb's next front is 0.  Weights by cell
    // live in fw (read by stage B), fronts of rounds >= 1 in the danger
    // map's space (zeroed before stage B), update flags by list index in
    // the dead cover bytes.  Round 0's fronts are the fuse weights of the
    // senders themselves, computed from the cell words the walk reads.
    float* front = dng;
    uint8_t* upd_f = cov;
    const int rounds = CF->max_chain > 1 ? min(CF->max_chain, CF->chain_cap_rounds) : 0;
    // the first L items (bombs 0 .. L/4 - 1 of the env) keep their cell, sender and
    // weight in registers from round 0 on
    int c0 = 0, snd0 = 255;
    float w0r = 0.0f;
    bool more = true;
    for (int rr = 0; rr < rounds + (rounds == 0 ? 1 : 0) && more; ++rr) {
      if (rr > 0) wave_sync();
      bool upd = false, flag0 = false;
      for (int it0 = 0; it0 < 4 * nb; it0 += L) {   // the env's items in passes of L
        const int it = it0 + l;
        const int j = it >> 2, d = it & 3;
        const bool live = it < 4 * nb;
        float spread = 0.0f;
        if (it0 == 0 && rr > 0) {
          if (live && snd0 != 255) spread = front[snd0];
          spread = fmaxf(spread, qx1(spread));
          spread = fmaxf(spread, qx2(spread));
          if (live && d == 0) {
            const bool f = spread > w0r;
            if (f) {
              w0r = spread;
              fw[c0] = spread;
            }
            flag0 = f;
            upd |= f;
          }
          continue;
        }
        const int c = live ? list[j] : 0;
        const uint32_t wc = cwl[c];
        int snd = 255;
        if (live && rounds > 0 && !(wc & F_WALL)) {
          walk_ray<H, W>(cwl, c, d, H + W, -1, [&](int k, int u, uint32_t wu) {
            if (cw_fuse(wu) > 0) {
              if (blast_of(wu, cfg_blast) >= k) {
                snd = u;
                spread = rr == 0 ? fuse_weight(cw_fuse(wu), fmax_f, frcp) : front[u];
              }
              return false;
            }
            return !(wu & (F_WALL | F_BRICK));
          });
        }
        spread = fmaxf(spread, qx1(spread));
        spread = fmaxf(spread, qx2(spread));
        const float wj = (live && d == 0) ? (rr == 0 ? fuse_weight(cw_fuse(wc), fmax_f, frcp) : fw[c]) : 0.0f;
        const bool f = spread > wj;
        if (it0 == 0) {       // round 0 of the first pass
          c0 = c;
          snd0 = snd;
          w0r = f ? spread : wj;
        }
        if (live && d == 0) {
          fw[c] = f ? spread : wj;
          if (rr == 0) front[c] = f ? spread : 0.0f;   // nobody reads fronts in round 0
          else upd_f[j] = f ? 1 : 0;
          upd |= f;
        }
      }
      if (rr > 0) {
        wave_sync();
        if (l < 4 * nb && (l & 3) == 0) front[c0] = flag0 ? w0r : 0.0f;
        for (int j = L / 4 + l; j < nb; j += L) {
          const int c = list[j];
          front[c] = upd_f[j] ? fw[c] : 0.0f;
        }
      }
      more = __any(upd);
    }
    wave_sync();
    if (has_danger) {
#pragma unroll
      for (int k = 0; k < KC; ++k)
        if (l + L * k < C) dng[l + L * k] = 0.0f;
    }
    wave_sync();
    // stage B: every (bomb, direction) ray max-updates the danger map.
    // Danger values are >= 0, so their float bits order like ints and an LDS
    // integer max is exact whatever the order of the rays.
    int* dngi = reinterpret_cast<int*>(dng);
    for (int it = l; it < 4 * nb; it += L) {
      const int j = it >> 2, d = it & 3;
      const int c = list[j];
      const uint32_t wc = cwl[c];
      const int v = __float_as_int(fw[c]);
      if (wc & F_WALL) continue;
      if (d == 0) atomicMax(&dngi[c], v);   // the bomb's own cell (seed)
      walk_ray<H, W>(cwl, c, d, blast_of(wc, cfg_blast), 1, [&](int, int x, uint32_t wx) {
        if (wx & F_WALL) return false;
        atomicMax(&dngi[x], v);
        return !cw_solid(wx);
      });
    }
    wave_sync();
  }

  // ---- 10. time, rewards, growth, combo, terminal terms (player lanes)
  int t = ev.x + 1;
  float crate_prob = __int_as_float(ev.y);
  int map_kind = ev.z;
  bool do_reset = false;
  {
    const auto k_max_steps = CF->max_steps;
    const auto k_explore_coef = A->explore_coef;
    const auto k_crate_u = A->crate_u;
    const auto k_seed = A->seed;
    const auto k_tick = A->tick;
    const auto k_step_penalty = CF->step_penalty;
    const auto k_hit_reward = CF->hit_reward;
    const auto k_hit_attr_penalty = CF->hit_attr_penalty;
    const auto k_hit_speed_drop = CF->hit_speed_drop;
    const auto k_growth_speed_step = CF->growth_speed_step;
    const auto k_brick_reward = CF->brick_reward;
    const auto k_recycle_crate_prob = CF->recycle_crate_prob;
    const auto k_growth_bombs_max = CF->growth_bombs_max;
    const auto k_growth_blast_max = CF->growth_blast_max;
    const auto k_growth_speed_max = CF->growth_speed_max;
    const auto k_danger_coef = A->danger_coef;
    const auto k_combo_reward = CF->combo_reward;
    const auto k_combo_gap_factor = CF->combo_gap_factor;
    const auto k_timeout_draw = CF->timeout_draw;
    const auto k_win_hp_scaled = CF->win_hp_scaled;
    const auto k_win_per_hp = CF->win_per_hp;
    const auto k_win_bonus = CF->win_bonus;
    const auto k_reward = A->reward;
    const auto k_winner = A->winner;
    const auto k_done = A->done;
    const auto k_n_alive = A->n_alive;
    const auto k_auto_reset = A->auto_reset;
    int alv_b[P], hp_b[P], hp0_b[P], stood_b[P];
    const uint32_t wcell = cwl[fpost];
    const int stood = corridor && (wcell & F_CRATE) ? 1 : 0;
    bcast_all<P>(r.alive, alv_b);
    bcast_all<P>(r.hp, hp_b);
    bcast_all<P>(hp0, hp0_b);
    bcast_all<P>(stood, stood_b);
    int n_alive = 0, dsum_int = 0, hsum_int = 0;
    bool any_stood = false;
#pragma unroll
    for (int o = 0; o < P; ++o) {
      n_alive += alv_b[o] != 0;
      dsum_int += max(hp0_b[o] - hp_b[o], 0);
      hsum_int += hp_b[o];
      any_stood |= stood_b[o] != 0;
    }
    const bool done = (n_alive <= 1) || (t >= k_max_steps);
    const float alpha = k_explore_coef;
    const float dmg = (float)max(hp0 - r.hp, 0);
    const float dng_here = has_danger ? dng[fpost] : 0.0f;
    // crate uniforms: injected, or Philox per tick (both players' pairs in one block)
    float uh = in_uh, ug = in_ug;
    if (any_stood && !k_crate_u) {
      float u4[4];
      philox_block(k_seed, (uint32_t)gs, k_tick, STREAM_CRATE, (uint32_t)((2 * pi) >> 2), u4);
      const bool hi = ((2 * pi) & 3) != 0;   // player pairs sit at words 0-1 and 2-3
      uh = hi ? u4[2] : u4[0];
      ug = hi ? u4[3] : u4[1];
    }
    if (lr < P) {
      const float a0 = (float)(alive0 != 0);
      const float dsum = (float)dsum_int;  // exact: a sum of small integers
      const float dealt = dsum - dmg;
      float rw = (-k_step_penalty) * a0;
      rw = rw + k_hit_reward * dealt;
      rw = rw - k_hit_reward * dmg;
      rw = rw + (alpha * pbonus) * a0;
      if (k_hit_attr_penalty > 0 && dmg > 0.0f && alive0) {
        const int pen = k_hit_attr_penalty;
        const int bc = r.bcap, zc = r.zcap;
        const float sp = r.spd;
        const int nbc = max(bc - pen, r.lob);
        const int nzc = max(zc - pen, r.loz);
        const float ns = fmaxf(sp - k_hit_speed_drop, r.los);
        const float lost_f = (float)((bc - nbc) + (zc - nzc)) +
                             rintf(__fdiv_rn(sp - ns, k_growth_speed_step));
        r.bcap = nbc;
        r.zcap = nzc;
        r.spd = ns;
        r.pend += (int)lost_f;
      }
      rw = rw + (alpha * 0.0f) * a0;  // chain_blast_bonus term (0: the host refuses other values)
      if (corridor) {
        rw = rw + (k_brick_reward * (float)stood) * a0;
        if (any_stood) {
          const float prob = (wcell & F_REC) ? k_recycle_crate_prob : crate_prob;
          const int h = stood && (uh < prob) && alive0;
          const int attr = (int)floorf(ug * 3.0f);
          r.bcap = min(r.bcap + (attr == 0) * h, k_growth_bombs_max);
          r.zcap = min(r.zcap + (attr == 1) * h, k_growth_blast_max);
          const float sp = r.spd + (float)((attr == 2) * h) * k_growth_speed_step;
          r.spd = fminf(sp, k_growth_speed_max);
        }
        cwl[fpost] = wcell & ~(F_CRATE | F_REC);
      }
      rw = rw - (k_danger_coef * dng_here) * a0;
      if (k_combo_reward > 0.0f) {
        const int c0 = r.combo;
        if (dealt > 0.0f) {
          const int gap = t - r.last_hit;
          const float factor = powf(k_combo_gap_factor, (float)max(gap, 0));
          const int combo_now = c0 + 1;
          const float pts = (((float)combo_now * k_combo_reward) * factor) * fminf(dealt, 1.0f);
          rw = rw + pts * a0;
          r.last_hit = t;
          r.combo = combo_now;
        } else {
          rw = rw + 0.0f * a0;
        }
        if (dmg > 0.0f) r.combo = 0;
      }
      const bool death_done = done && n_alive == 1;
      const bool all_alive = done && n_alive == P;
      const bool al = r.alive != 0;
      int win = death_done && al, lose = death_done && !al;
      const float hpf = (float)r.hp;
      float tscale = alpha;
      if (!k_timeout_draw) {
        bool gt = true, lt = false;
#pragma unroll
        for (int o = 0; o < P; ++o) {
          if (o == lr) continue;
          const float ho = (float)hp_b[o];
          gt = gt && (hpf > ho);
          lt = lt || (hpf < ho);
        }
        win |= all_alive && gt;
        lose |= all_alive && lt;
        tscale = 1.0f;
      }
      const float diff = hpf - __fdiv_rn((float)hsum_int - hpf, (float)(P - 1));
      if (k_win_hp_scaled) {
        const float base = k_win_per_hp * diff;
        rw = rw + (base * (float)death_done + (base * (float)all_alive) * tscale);
      } else {
        rw = rw + k_win_bonus * ((float)win - (float)lose);
        if (k_timeout_draw) rw = rw + ((k_win_per_hp * diff) * (float)all_alive) * tscale;
      }
      if (valid && l < P) {
        if (k_reward) k_reward[gs * P + l] = rw;
        if (k_winner) k_winner[gs * P + l] = win;
      }
    }
    if (valid && l == 0) {
      if (k_done) k_done[gs] = done;
      if (k_n_alive) k_n_alive[gs] = n_alive;
    }
    do_reset = done && k_auto_reset && valid;
  }

  // ---- 11. auto-reset of finished envs (sim/torch_sim.py:178-420)
  if (__any(do_reset)) {
    wave_sync();
    if (do_reset) {
      has_danger = false;   // a fresh map has no bombs
      const uint32_t env_id = (uint32_t)g;
      if constexpr (MAPS == 0) {
        // template maps (qqtsim/maps.py): border + even/even pillars for
        // map_kind 0, bricks w.p. brick_p off the spawn L; one Philox block
        // keys four consecutive cells
#pragma unroll 1
        for (int k = 0; k < KC; ++k) {
          const int c = l + L * k;
          if (c >= C) continue;
          const int rr = c / W, col = c % W;
          bool wall = false;
          if (CF->map_kind == 0)
            wall = rr == 0 || rr == H - 1 || col == 0 || col == W - 1 || ((rr % 2 == 0) && (col % 2 == 0));
          bool keep = false;
#pragma unroll
          for (int i = 0; i < P; ++i) {
            const int sr = (i == 0 || i == 2) ? 1 : H - 2;
            const int sc = (i == 0 || i == 3) ? 1 : W - 2;
            const int dr = sr < H / 2 ? 1 : -1, dc = sc < W / 2 ? 1 : -1;
            keep |= (rr == sr && col == sc) || (rr == sr && col == sc + dc) || (rr == sr + dr && col == sc);
          }
          bool brick = false;
          if (!wall && !keep && CF->brick_p > 0.0f)
            brick = philox_uniform(A->seed, env_id, A->epoch, STREAM_RESET_CELL, (uint32_t)c) < CF->brick_p;
          cwl[c] = (wall ? F_WALL : 0u) | (brick ? F_BRICK : 0u) | EMPTY_CELL;
        }
        // misc values 0..11: lane j draws block min(j, 2)
        float ub[4];
        philox_block(A->seed, env_id, A->epoch, STREAM_RESET_MISC, (uint32_t)min(l, 2), ub);
        float u[12];
#pragma unroll
        for (int j = 0; j < 12; ++j) u[j] = __shfl(ub[j % 4], (lane & ~(L - 1)) + j / 4);
        if (lr < P) {
          float py[P], px[P];
#pragma unroll
          for (int i = 0; i < P; ++i) {
            py[i] = (float)((i == 0 || i == 2) ? 1 : H - 2) + 0.5f;
            px[i] = (float)((i == 0 || i == 3) ? 1 : W - 2) + 0.5f;
          }
          if (CF->swap_spawns && u[0] < 0.5f) {
            const float ty = py[0], tx = px[0];
            py[0] = py[1]; px[0] = px[1]; py[1] = ty; px[1] = tx;
          }
          const int bspan = CF->bombs_hi - CF->bombs_lo + 1, zspan = CF->blast_hi - CF->blast_lo + 1;
          float ub1 = u[1], ub2 = u[2];
#pragma unroll
          for (int i = 1; i < P; ++i)
            if (lr == i) { ub1 = u[1 + 2 * i]; ub2 = u[2 + 2 * i]; }
          const int bc = CF->bombs_lo + min((int)floorf(ub1 * (float)bspan), bspan - 1);
          const int zc = CF->blast_lo + min((int)floorf(ub2 * (float)zspan), zspan - 1);
          r.y = self<P>(py, lr);
          r.x = self<P>(px, lr);
          r.alive = 1;
          r.hp = CF->max_hp;
          r.since = CF->spawn_cooldown;
          r.bcap = bc;
          r.zcap = zc;
          r.spd = CF->spawn_speed;
          r.inv = 0;
          r.combo = 0;
          r.last_hit = -1000000000;
          r.pend = 0;
          r.lob = bc;
          r.loz = zc;
          r.los = CF->spawn_speed;
          r.pad = 0;
        }
        t = 0;
        crate_prob = CF->growth_crate_prob;
        map_kind = 0;
      } else {
        // the reference's map modes (generators sim/mapgen.py:15-242).
        // Draws: STREAM_RESET_MISC values 0 map type, 1 top wall rows,
        // 2 spawn swap, 3 obstacle count, 4.. the corridor edge segments
        // (start, length, on) x 4 columns then the horizontal one;
        // STREAM_RESET_CELL value c the ring band's brick draw, C + c the
        // open obstacles' keys (the n cells with the smallest (key, cell)).
        float ub[4];
        philox_block(A->seed, env_id, A->epoch, STREAM_RESET_MISC, (uint32_t)min(l, 4), ub);
        float u[19];
#pragma unroll
        for (int j = 0; j < 19; ++j) u[j] = __shfl(ub[j % 4], (lane & ~(L - 1)) + j / 4);
        int kind = 1;
        bool pure = false;
        if (corridor) {
          kind = u[0] < CF->thr_open ? 1 : u[0] < CF->thr_ring ? 2 : 0;
          pure = u[0] < CF->thr_pure;
        }
        const int T = CF->top_wall_rows;
        const int top = CF->random_wall_rows ? min((int)floorf(u[1] * (float)(T + 1)), T) : T;
        const int bot = CF->random_wall_rows ? T - top : 0;
        const int sp_mode = corridor ? 0 : 1;
        const int sp_kind = kind == 0 ? 0 : kind == 2 ? 2 : 1;
        auto near_spawn = [&](int set, int rr, int col) {
          bool nbh = false;
#pragma unroll
          for (int i = 0; i < P; ++i) {
            const int sc = CF->ref_spawn_cell[set][i];
            const int dr = rr - sc / W, dc = col - sc % W;
            nbh |= (dr == 0 && (dc == 0 || dc == 1 || dc == -1)) || (dc == 0 && (dr == 1 || dr == -1));
          }
          return nbh;
        };
        // open obstacles: bit k marks cell l + 16k
        uint32_t obst = 0;
        const int nmax = CF->open_obstacle_max;
        const int nobst = nmax > 0 ? min((int)floorf(u[3] * (float)(nmax + 1)), nmax) : 0;
        if (kind == 1 && !pure && nobst > 0) {
          uint64_t key[KC];
#pragma unroll
          for (int k = 0; k < KC; ++k) {
            const int c = l + L * k;
            key[k] = ~0ull;
            if (c < C) {
              const float uk = philox_uniform(A->seed, env_id, A->epoch, STREAM_RESET_CELL,
                                              (uint32_t)(C + c));
              key[k] = ((uint64_t)__float_as_uint(uk) << 32) | (uint32_t)c;
            }
          }
          for (int tt = 0; tt < nobst; ++tt) {
            uint64_t mn = key[0];
#pragma unroll
            for (int k = 1; k < KC; ++k) mn = key[k] < mn ? key[k] : mn;
#pragma unroll
            for (int m = 1; m < L; m <<= 1) {
              const uint64_t o = __shfl_xor(mn, m, L);
              mn = o < mn ? o : mn;
            }
#pragma unroll
            for (int k = 0; k < KC; ++k)
              if (key[k] == mn) {
                obst |= 1u << k;
                key[k] = ~0ull;
              }
          }
        }
        const int c0 = (W - CF->corridor_width) / 2, c1 = c0 + CF->corridor_width;
        const bool segs = kind == 0 && CF->wall_density > 0.0f;
        const int ecol[4] = {c0, c0 + 1, c1 - 2, c1 - 1};
        int vs[4], vl[4];
        bool va[4];
#pragma unroll
        for (int ci = 0; ci < 4; ++ci) {
          const float us = u[4 + 3 * ci], ul = u[5 + 3 * ci], ua = u[6 + 3 * ci];
          vs[ci] = CF->random_wall_rows
              ? (int)(us * (float)max(H - bot - 4 - top, 1) + (float)top)
              : (int)(us * (float)(H - T - 4) + (float)T);
          vl[ci] = 2 + (int)(ul * 3.0f);
          va[ci] = segs && ua < CF->wall_density && ecol[ci] >= c0 && ecol[ci] < c1;
        }
        const int hs = (int)(u[16] * (float)(c1 - c0 - 4) + (float)c0);
        const int hl = 2 + (int)(u[17] * 3.0f);
        const bool ha = segs && c1 - c0 > 4 && u[18] < CF->wall_density;
        const int hr0 = CF->random_wall_rows ? top : T;
        const int hr1 = CF->random_wall_rows ? top + 2 : T + min(2, H - T);
        const int r0 = (H - CF->ring_center_h) / 2, q0 = (W - CF->ring_center_w) / 2;
        const int r1 = r0 + CF->ring_center_h, q1 = q0 + CF->ring_center_w;
        const int cy = (H - 1) / 2, cx = (W - 1) / 2;
#pragma unroll 1
        for (int k = 0; k < KC; ++k) {
          const int c = l + L * k;
          if (c >= C) continue;
          const int rr = c / W, col = c % W;
          bool wall = false, brick = false, crate = false;
          if (kind == 0) {
            wall = CF->random_wall_rows ? (rr < top || rr >= H - bot) : rr < T;
            brick = (col < c0 || col >= c1) && rr >= (CF->random_wall_rows ? top : T);
#pragma unroll
            for (int ci = 0; ci < 4; ++ci)
              brick |= va[ci] && col == ecol[ci] && rr >= vs[ci] && rr < vs[ci] + vl[ci];
            brick |= ha && rr >= hr0 && rr < hr1 && col >= c0 && col < c1 && col >= hs && col < hs + hl;
            if (near_spawn(sp_mode, rr, col)) wall = brick = false;
          } else if (kind == 2) {
            wall = rr >= r0 && rr < r1 && col >= q0 && col < q1;
            const bool band = !wall && rr >= r0 - 1 && rr <= r1 && col >= q0 - 1 && col <= q1;
            if (band && !near_spawn(2, rr, col))
              brick = philox_uniform(A->seed, env_id, A->epoch, STREAM_RESET_CELL, (uint32_t)c) <
                      CF->ring_brick_density;
          } else {
            wall = ((obst >> k) & 1u) && !near_spawn(sp_mode, rr, col);
            crate = corridor && CF->open_crate_cross &&
                    (rr == cy - 1 || rr == cy || col == cx - 1 || col == cx) && !near_spawn(1, rr, col);
          }
          cwl[c] = (wall ? F_WALL : 0u) | (brick ? F_BRICK : 0u) | (crate ? F_CRATE : 0u) | EMPTY_CELL;
        }
        int b0, z0;
        float s0;
        if (!corridor) {
          b0 = CF->max_bombs; z0 = cfg_blast; s0 = 1.0f;
        } else if (kind == 1) {
          b0 = CF->open_growth_bombs; z0 = CF->open_growth_blast; s0 = CF->open_growth_speed;
        } else {
          b0 = CF->growth_bombs_start; z0 = CF->growth_blast_start; s0 = CF->growth_speed_start;
        }
        int b1 = b0, z1 = z0;
        float s1 = s0;
        if (A->opp_boost == 2) {
          b1 = CF->opp_growth_bombs; z1 = CF->opp_growth_blast; s1 = CF->opp_growth_speed;
        } else if (A->opp_boost == 1) {
          b1 = (int)fminf(rintf((float)b0 * CF->opp_hist_mult), (float)CF->growth_bombs_max);
          z1 = (int)fminf(rintf((float)z0 * CF->opp_hist_mult), (float)CF->growth_blast_max);
          s1 = fminf(s0 * CF->opp_hist_mult, CF->growth_speed_max);
        }
        const bool swap = u[2] < 0.5f;
        if (lr < P) {
          const int i = lr;
          const int si = (swap && i < 2) ? 1 - i : i;
          float sy = CF->ref_spawn_y[sp_kind][0], sx = CF->ref_spawn_x[sp_kind][0];
#pragma unroll
          for (int j = 1; j < P; ++j)
            if (si == j) { sy = CF->ref_spawn_y[sp_kind][j]; sx = CF->ref_spawn_x[sp_kind][j]; }
          r.y = sy;
          r.x = sx;
          r.alive = 1;
          r.hp = CF->max_hp;
          r.since = CF->spawn_cooldown;
          r.inv = 0;
          r.combo = 0;
          r.last_hit = -1000000000;
          r.pend = 0;
          if (i < 2) {            // players 2 and 3 keep caps, speed and floors
            const int bc = i == 0 ? b0 : b1, zc = i == 0 ? z0 : z1;
            const float sp = i == 0 ? s0 : s1;
            r.bcap = bc;
            r.zcap = zc;
            r.spd = sp;
            r.lob = bc;
            r.loz = zc;
            r.los = sp;
          }
        }
        t = 0;
        if (corridor)
          crate_prob = kind == 1 ? 1.0f : kind == 2 ? CF->ring_crate_prob : CF->growth_crate_prob;
        map_kind = kind;
      }
    }
    wave_sync();
  }
  // hp fell this tick, judged on the post-reset record (the collect loop
  // compares after step() returns)
  if (A->damaged && valid && l < P) A->damaged[gs * P + l] = hp0 - r.hp > 0 ? 1 : 0;

  // ---- 12. the cells of the final state back into registers; legality
  // masks (sim/obs.py:139-229): lane = me*4 + probe (up, down, left, right)
  const auto m_step_len = CF->step_len;
  const auto m_move_mask = A->move_mask;
  const auto m_bomb_mask = A->bomb_mask;
  livepack = 0;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    if (c < C) cw[k] = cwl[c];
    const int o = cw_owner(cw[k]);
    if (cw_fuse(cw[k]) > 0 && o >= 0 && o < P) livepack += 1 << (8 * o);
  }
  livepack = env_sum<L>(livepack);
  float y_b[P], x_b[P];
  int al_b[P], bcap_b[P];
  bcast_allf<P>(r.y, y_b);
  bcast_allf<P>(r.x, x_b);
  bcast_all<P>(r.alive, al_b);
  bcast_all<P>(r.bcap, bcap_b);
  {
    const int me = lr >> 2, pr = lr & 3;
    if (me < P && l < 16 && valid) {
      const float y = self<P>(y_b, me), x = self<P>(x_b, me);
      const bool al = sel<P>(al_b, me) != 0;
      const float st = m_step_len;
      const float d = (pr & 1) ? st : -st;
      const bool vert = pr < 2;
      const float own = vert ? y : x;
      const float nv = resolve_axis<H, W>(cwl, own + d, d, y, x, rad, vert);
      const bool moved = fabsf(nv - own) > 2e-4f;
      if (m_move_mask) {
        m_move_mask[(gs * P + me) * 5 + pr] = al ? moved : 1;
        if (pr == 0) m_move_mask[(gs * P + me) * 5 + 4] = 1;
      }
      if (pr == 0 && m_bomb_mask) {
        const int flat = min(max((int)floorf(y) * W + (int)floorf(x), 0), C - 1);
        const uint32_t wc = cwl[flat];
        const bool under = cw_fuse(wc) > 0;
        const int live_me = (livepack >> (8 * me)) & 0xFF;
        const bool can = !under && !(wc & F_BRICK) && live_me < sel<P>(bcap_b, me);
        m_bomb_mask[(gs * P + me) * 2 + 0] = 1;
        m_bomb_mask[(gs * P + me) * 2 + 1] = (can && al) || !al;
      }
    }
  }

  // ---- 13. observation (sim/obs.py:25-136): the float32 danger of my
  const auto o_growth_bombs_max = CF->growth_bombs_max;
  const auto o_max_steps = CF->max_steps;
  const auto o_obs = A->obs;
  // cells, the per-player values, then the channels in staging passes
  float dv[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int c = l + L * k;
    dv[k] = (has_danger && c < C) ? dng[c] : 0.0f;
  }
  // splat corners in order (0,0),(0,1),(1,0),(1,1) with running sums where
  // corners coincide; the player-cell channels
  int sid[4];
  uint16_t sval[4];
  int pcell;
  uint16_t h_inv, h_avail, h_cap;
  {
    const bool al = r.alive != 0;
    const float gate = (float)al;
    const float fy = fminf(fmaxf(r.y - 0.5f, 0.0f), (float)(H - 1));
    const float fx = fminf(fmaxf(r.x - 0.5f, 0.0f), (float)(W - 1));
    const int y0 = min(max((int)floorf(fy), 0), H - 1);
    const int x0 = min(max((int)floorf(fx), 0), W - 1);
    const int y1 = min(y0 + 1, H - 1), x1 = min(x0 + 1, W - 1);
    const float wy = fminf(fmaxf(fy - (float)y0, 0.0f), 1.0f);
    const float wx = fminf(fmaxf(fx - (float)x0, 0.0f), 1.0f);
    const float ky0 = 1.0f - wy, kx0 = 1.0f - wx;
    sid[0] = y0 * W + x0; sid[1] = y0 * W + x1; sid[2] = y1 * W + x0; sid[3] = y1 * W + x1;
    const float wt[4] = {(ky0 * kx0) * gate, (ky0 * wx) * gate, (wy * kx0) * gate, (wy * wx) * gate};
    float run[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float prev = 0.0f;
#pragma unroll
      for (int j = 0; j < q; ++j)
        if (sid[j] == sid[q]) prev = run[j];
      run[q] = prev + wt[q];
      sval[q] = h16(run[q]);
    }
    pcell = min(max((int)floorf(r.y) * W + (int)floorf(r.x), 0), C - 1);
    const int live_i = (livepack >> (8 * pi)) & 0xFF;
    const float cap = fmaxf((float)r.bcap, 1.0f);
    const float avail = fmaxf((float)(r.bcap - live_i), 0.0f);
    const float invf = (r.inv > 0 && al) ? 1.0f : 0.0f;
    h_inv = h16(invf);
    h_avail = h16(__fdiv_rn(avail, cap) * gate);
    h_cap = h16(__fdiv_rn(cap, (float)o_growth_bombs_max) * gate);
  }
  const uint16_t h_one = h16(1.0f);
  const uint16_t h_t = h16(__fdiv_rn((float)t, (float)o_max_steps));
  wave_sync();

  if (o_obs) {
    const size_t obs_base = gs * OBS;
#pragma unroll
    for (int pass = 0; pass < G::NPASS; ++pass) {
      constexpr int CPP = G::CPP;
      const int ch0 = pass * CPP;
      const int nch = (G::NCH - ch0) < CPP ? (G::NCH - ch0) : CPP;
      const int nbytes = nch * C * 2;
      uint16_t* dst = o_obs + obs_base + (size_t)ch0 * C;
      const int opad = (int)(((uintptr_t)dst) & 15u);
      uint16_t* sb = reinterpret_cast<uint16_t*>(blk + opad);
      if (pass > 0) wave_sync();   // the previous pass's copy-out has read the block
      // Every cell of the cell-parallel channels is written below; only the
      // players' sparse channels (splat [0, P) and the player-cell channels
      // [2P + 4, 5P + 4)) start from zero.  The 16-byte units that hold them
      // are cleared first (a unit shared with a cell-parallel channel gets
      // that channel's values afterwards: one wavefront's LDS accesses
      // complete in order).
      {
        uint4* z = reinterpret_cast<uint4*>(blk);
        auto clear = [&](int lo, int hi) {   // channels [lo, hi) of the pass, when not empty
          const int zlo = max(lo, ch0), zhi = min(hi, ch0 + nch);
          if (zlo >= zhi) return;
          const int b0 = (opad + (zlo - ch0) * C * 2) & ~15;
          const int b1 = min((opad + (zhi - ch0) * C * 2 + 15) & ~15, G::BLOCK);
          for (int i = b0 / 16 + l; i < b1 / 16; i += L) z[i] = make_uint4(0u, 0u, 0u, 0u);
        };
        clear(0, P);
        clear(2 * P + 4, 5 * P + 4);
      }
      // cell-parallel channels (relative to ch0): walls+bricks, danger, time,
      // crates, and the own-bomb fuse channels
      constexpr int CW_CH = 2 * P, DG_CH = 2 * P + 1, T_CH = 2 * P + 2, CR_CH = 2 * P + 3;
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int c = l + L * k;
        if (c >= C) continue;
        const uint32_t w = cw[k];
        if (CW_CH >= ch0 && CW_CH < ch0 + nch)
          sb[(CW_CH - ch0) * C + c] = (w & (F_WALL | F_BRICK)) ? h_one : (uint16_t)0;
        if (DG_CH >= ch0 && DG_CH < ch0 + nch) sb[(DG_CH - ch0) * C + c] = h16(dv[k]);
        if (T_CH >= ch0 && T_CH < ch0 + nch) sb[(T_CH - ch0) * C + c] = h_t;
        if (CR_CH >= ch0 && CR_CH < ch0 + nch)
          sb[(CR_CH - ch0) * C + c] = (w & F_CRATE) ? h_one : (uint16_t)0;
        if (P + P > ch0 && P < ch0 + nch) {
          const int f = cw_fuse(w), o = cw_owner(w);
          const uint16_t hq = f > 0 ? h16(qdiv(f, fmax_f, frcp)) : (uint16_t)0;
#pragma unroll
          for (int i = 0; i < P; ++i)
            if (P + i >= ch0 && P + i < ch0 + nch) sb[(P + i - ch0) * C + c] = o == i ? hq : (uint16_t)0;
        }
      }
      // the players' channels, written after the cell-parallel ones
      if (l < P) {
        if (l >= ch0 && l < ch0 + nch) {
#pragma unroll
          for (int q = 0; q < 4; ++q) sb[(l - ch0) * C + sid[q]] = sval[q];
        }
        const int ci = 2 * P + 4 + l, ca = 3 * P + 4 + l, cc = 4 * P + 4 + l;
        if (ci >= ch0 && ci < ch0 + nch) sb[(ci - ch0) * C + pcell] = h_inv;
        if (ca >= ch0 && ca < ch0 + nch) sb[(ca - ch0) * C + pcell] = h_avail;
        if (cc >= ch0 && cc < ch0 + nch) sb[(cc - ch0) * C + pcell] = h_cap;
      }
      wave_sync();
      // copy-out: staging and destination share their address mod 16, so a
      // u16 head, a 16-byte body and a u16 tail
      if (valid) {
        uint8_t* d8 = reinterpret_cast<uint8_t*>(dst);
        const uint8_t* src = blk + opad;
        const int head = min((16 - opad) & 15, nbytes);
        const int n16 = (nbytes - head) / 16;
        const int tail0 = head + n16 * 16;
        // every LDS read of the lane (head and tail halfwords, 16-byte units,
        // all at clamped in-block addresses) is issued before the first store,
        // so the copy waits on LDS once
        constexpr int NU = (CPP * C * 2 / 16 + L - 1) / L;
        const uint4* s16 = reinterpret_cast<const uint4*>(src + head);
        uint4* d16 = reinterpret_cast<uint4*>(d8 + head);
        uint32_t hv = *reinterpret_cast<const uint16_t*>(src + min(l * 2, max(head - 2, 0)));
        uint32_t tv = *reinterpret_cast<const uint16_t*>(src + min(tail0 + l * 2, nbytes - 2));
        uint4 u16[NU];
#pragma clang loop unroll(full)
        for (int m = 0; m < NU; ++m) u16[m] = s16[min(l + L * m, n16 - 1)];
        // the values are materialised here: no read sinks below a store
        asm volatile("" : "+v"(hv), "+v"(tv));
#pragma clang loop unroll(full)
        for (int m = 0; m < NU; ++m) asm volatile("" : "+v"(u16[m].x), "+v"(u16[m].y), "+v"(u16[m].z), "+v"(u16[m].w));
        if (l * 2 < head) *reinterpret_cast<uint16_t*>(d8 + l * 2) = (uint16_t)hv;
#pragma clang loop unroll(full)
        for (int m = 0; m < NU; ++m)
          if (l + L * m < n16) d16[l + L * m] = u16[m];
        if (tail0 + l * 2 < nbytes) *reinterpret_cast<uint16_t*>(d8 + tail0 + l * 2) = (uint16_t)tv;
      }
    }
  }

  // ---- 14. store the state
  if (valid) {
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int c = l + L * k;
      if (c < C) A->cells[gs * C + c] = (int32_t)cw[k];
    }
    if (l < P) {
      int4* q = reinterpret_cast<int4*>(A->players + (gs * P + l) * QQT_P_SLOTS);
      q[0] = make_int4(__float_as_int(r.y), __float_as_int(r.x), r.alive, r.hp);
      q[1] = make_int4(r.since, r.bcap, r.zcap, __float_as_int(r.spd));
      q[2] = make_int4(r.inv, r.combo, r.last_hit, r.pend);
      q[3] = make_int4(r.lob, r.loz, __float_as_int(r.los), r.pad);
    }
    if (l == 0)
      *reinterpret_cast<int4*>(A->envs + gs * QQT_E_SLOTS) =
          make_int4(t, __float_as_int(crate_prob), map_kind, ev.w);
  }

  // ---- 15. optional per-env counters: exploded bombs, deaths, auto-resets
  // (each env's own int4, added to by lane 0 of the env: no atomics and no
  // contention between envs)
  int32_t* const stats = A->tick_stats;
  if (stats) {
    const int v0 = env_sum<L>(n_trg), v1 = env_sum<L>(n_died);
    if (valid && l == 0) {
      int4* sp = reinterpret_cast<int4*>(stats) + gs;
      const int4 o = *sp;
      *sp = make_int4(o.x + v0, o.y + v1, o.z + (do_reset ? 1 : 0), o.w);
    }
  }

  // ---- 16. optional blast-cap maximum of one player over the wavefront's
  // envs (int8, one per wavefront), the astar bot's chain-check reach source
  // for its next call
  int8_t* const rcaps = A->reach_caps;
  if (rcaps) {
    const int cap = (valid && l == A->reach_pid) ? min(r.zcap, 127) : 0;
    int m = 0;
#pragma unroll
    for (int ee = 0; ee < EPW; ++ee) m = max(m, __builtin_amdgcn_readlane(cap, L * ee + A->reach_pid));
    if (lane == 0) rcaps[g0 / EPW] = (int8_t)m;
  }
}

}  // namespace grp

// STEP launch of the group kernel: XCD_ROWS-env row blocks, a multiple of 8
// of them (one per XCD in turn), one-wavefront workgroups.  Up to
// GROUP32_MAX_ENVS envs an env takes 32 lanes (two envs per wavefront: at
// 5632 envs, 2816 wavefronts keep every SIMD at two or three of them and
// halve the per-wavefront cell work); larger batches take 16 lanes per env
// (four per wavefront), which keeps 16,384 envs resident in one round
// (GROUP32_MAX_ENVS, tick_envs_per_wave in qqt_common.h).

template <int H, int W, int P, int L>
int launch_group(const qqt_sim_config* cfg, const qqt_tick_args* a, hipStream_t st) {
  const int nrb = (a->n_envs + XCD_ROWS - 1) / XCD_ROWS;
  const int blocks = ((nrb + 7) / 8) * 8 * (XCD_ROWS / (64 / L));
  const dim3 grid(blocks), block(64);
  if (cfg->map_kind == QQT_MAP_REFERENCE)
    QQT_LAUNCH(QQT_KERNEL_TICK, (grp::tick_group_kernel<H, W, P, 1, L>), grid, block, st, *cfg, *a);
  else
    QQT_LAUNCH(QQT_KERNEL_TICK, (grp::tick_group_kernel<H, W, P, 0, L>), grid, block, st, *cfg, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    char msg[256];
    snprintf(msg, sizeof(msg), "tick launch failed: %s", hipGetErrorString(err));
    return fail(QQT_E_LAUNCH, msg);
  }
  return QQT_OK;
}

template <int H, int W, int P>
int launch_step_group(const qqt_sim_config* cfg, const qqt_tick_args* a, hipStream_t st) {
  return a->n_envs <= GROUP32_MAX_ENVS ? launch_group<H, W, P, 32>(cfg, a, st)
                                       : launch_group<H, W, P, 16>(cfg, a, st);
}

template int launch_step_group<13, 13, 2>(const qqt_sim_config*, const qqt_tick_args*, hipStream_t);
template int launch_step_group<7, 7, 2>(const qqt_sim_config*, const qqt_tick_args*, hipStream_t);
template int launch_step_group<9, 9, 2>(const qqt_sim_config*, const qqt_tick_args*, hipStream_t);
template int launch_step_group<13, 13, 3>(const qqt_sim_config*, const qqt_tick_args*, hipStream_t);
template int launch_step_group<13, 13, 4>(const qqt_sim_config*, const qqt_tick_args*, hipStream_t);

}  // namespace qqt
