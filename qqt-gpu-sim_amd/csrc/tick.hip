// Fused rollout tick for gfx950: step + auto-reset + danger + observation +
// legality masks of a batch of envs in one launch.
//
// Mapping: one 64-lane wavefront owns EPW = 64 / LPE consecutive envs; each
// env gets LPE lanes (LPE = 64 on MI355X: a wavefront per env).  Lane l of an
// env walks the cells c = l, l + LPE, ...  A workgroup holds WPB independent
// wavefronts (own envs, own LDS, wave-level syncs only): with WPB = 2 a CU
// keeps 11 workgroups = 22 envs resident (LDS-bound, 6.8 KB per env), so a
// 5632-env batch runs in one round on 256 CUs; one-wave workgroups would hit
// the per-CU workgroup-slot limit first.  Per-env grids live in LDS for the
// whole tick; the observation is staged in LDS in its final (N, C, H, W)
// float16 layout and leaves with wide, fully coalesced stores.
//
// Semantics follow the reference tick (sim/torch_sim.py:895-1261) stage by
// stage in float32 with the reference's operation order; the library is built
// with -ffp-contract=off so no product is fused into an add.
//
// Explosions and danger work on a per-env list of bomb cells built with a
// wavefront ballot, not on all H*W cells:
// * chain explosion: each source scatters its four rays into a byte cover
//   map; stores of 1 are idempotent, so overlapping rays need no atomics;
// * danger stage A: each bomb gathers from its (at most four) in-neighbours,
//   the first solid cell behind it in each direction, for a fixed number of
//   synchronous rounds;
// * danger stage B: every (bomb, direction) ray scatters the bomb's corrected
//   weight along its cells.  Rays of different bombs may share a cell; danger values are >= 0,
//   so an LDS integer atomic max on their float bits is exact in any order.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "qqt_common.h"
#include "qqt_hip.h"
#include "tick_rules.h"

namespace qqt {

template <int H, int W, int P, int LPE_>
struct Geo {
  static constexpr int LPE = LPE_;
  static constexpr int EPW = 64 / LPE;
  static constexpr int C = H * W;
  static constexpr int CW4 = (C + 3) / 4;       // dwords of a byte map
  static constexpr int NCH = 5 * P + 4;
  static constexpr int OBS = NCH * C;          // float16 values per env
  static constexpr int KMAX = (C + LPE - 1) / LPE;
};

template <class G>
struct DangerScratch {
  float fw[G::EPW][G::C];          // danger stage-A front (by cell)
  float wl[G::EPW][G::C];          // per listed bomb: corrected weight
  uint16_t edge[G::EPW][G::C][4];  // stage-A in-edge per listed bomb: sender | dist << 8
};

template <class G, int P>
struct __align__(16) Lds {
  // The danger map's scratch is dead before the observation is staged, so
  // the two share LDS (fewer bytes per env -> more envs resident per CU).
  union {
    DangerScratch<G> dz;
    // observation staging: envs back to back in output layout, placed at byte
    // offset (output address mod 16) so that copy-out can use 16-byte units
    uint8_t obs_raw[(G::EPW * G::OBS * 2 + 16 + 15) / 16 * 16];
  };
  uint32_t cw[G::EPW][G::C];
  float dng[G::EPW][G::C];   // danger map
  uint8_t list[G::EPW][G::C];
  int32_t pl[G::EPW][P][QQT_P_SLOTS];
  int32_t ev[G::EPW][QQT_E_SLOTS];
  int32_t alive0[G::EPW][P], live[G::EPW][P], fpre[G::EPW][P], act_b[G::EPW][P];
  int32_t done[G::EPW];
};

// ---------------------------------------------------------------- lane helpers
template <int LPE>
__device__ __forceinline__ int env_sum(int v) {
#pragma unroll
  for (int m = LPE / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, LPE);
  return v;
}
template <int LPE>
__device__ __forceinline__ int env_max(int v) {
#pragma unroll
  for (int m = LPE / 2; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, LPE));
  return v;
}
template <int LPE>
__device__ __forceinline__ uint64_t env_bits(bool pred, int e) {
  const uint64_t b = __ballot(pred);
  return LPE == 64 ? b : ((b >> (LPE * e)) & ((1ull << LPE) - 1ull));
}

// Number of cells c = l + LPE*k (k < KMAX) of this env satisfying pred (same
// result in every lane of the env; the popcounts run on the scalar unit).
template <class G, class Pred>
__device__ __forceinline__ int env_count(int e, int l, Pred pred) {
  int n = 0;
#pragma unroll
  for (int k = 0; k < G::KMAX; ++k) {
    const int c = l + G::LPE * k;
    n += __popcll(env_bits<G::LPE>(c < G::C && pred(c), e));
  }
  return n;
}

// Collect the cells satisfying `pred` into list[] (ascending cell order).
template <class G, class Pred>
__device__ __forceinline__ int build_list(uint8_t* list, int e, int l, Pred pred) {
  int base = 0;
#pragma unroll
  for (int k = 0; k < G::KMAX; ++k) {
    const int c = l + G::LPE * k;
    const bool p = c < G::C && pred(c);
    const uint64_t bits = env_bits<G::LPE>(p, e);
    if (p) list[base + __popcll(bits & ((1ull << l) - 1ull))] = (uint8_t)c;
    base += __popcll(bits);
  }
  return base;
}

// ---------------------------------------------------------------- kernel
// KMODE = QQT_MODE_FLUSH fixes the flush at compile time (its code lives
// only in that instantiation); KMODE = -1 serves RESET, OBSERVE and PROBE
// from a.mode.  MAPS selects the reset's map source: 0 the templates, 1 the
// reference's map modes (each kernel carries one of the two).
template <int H, int W, int P, int LPE, int WPB, int KMODE, int MAPS>
__global__ __launch_bounds__(64 * WPB) void tick_kernel(const qqt_sim_config cf, const qqt_tick_args a) {
  using G = Geo<H, W, P, LPE>;
  constexpr int C = G::C;
  constexpr int EPW = G::EPW;
  constexpr int OBS = G::OBS;
  constexpr int KMAX = G::KMAX;
  __shared__ Lds<G, P> sh[WPB];

  // waves of one workgroup share nothing: each owns its envs and its LDS.
  // Workgroups are dealt to the 8 XCDs round robin; block b takes XCD_ROWS-env
  // row block (b / 8 / WGRB) * 8 + b % 8, so a row block's state, observation
  // and masks stay in the L2 of the XCD whose policy workgroups read them
  // (the act kernel deals its row blocks the same way).
  constexpr int WGRB = XCD_ROWS / (WPB * EPW);      // workgroups per row block
  static_assert(WGRB * WPB * EPW == XCD_ROWS, "whole workgroups per row block");
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int seq = blockIdx.x >> 3;
  const int rb = (seq / WGRB) * 8 + (blockIdx.x & 7);
  const int g0 = rb * XCD_ROWS + ((seq % WGRB) * WPB + wv) * EPW;
  if (g0 >= a.n_envs) return;
  Lds<G, P>& s = sh[wv];
  const int lane = threadIdx.x & 63;
  const int e = lane / LPE;
  const int l = lane % LPE;
  const int g = g0 + e;
  const bool valid = g < a.n_envs;
  const int mode = KMODE >= 0 ? KMODE : a.mode;
  const float rad = cf.radius;
  const float fmax_f = (float)cf.fuse;

  uint32_t* cw = s.cw[e];
  int32_t(*pl)[QQT_P_SLOTS] = s.pl[e];
  uint8_t* list = s.list[e];

  // ---- load
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = l + LPE * k;
    if (c < C) cw[c] = valid ? (uint32_t)a.cells[(size_t)g * C + c] : (F_WALL | EMPTY_CELL);
  }
  for (int i = l; i < P * QQT_P_SLOTS; i += LPE)
    pl[i / QQT_P_SLOTS][i % QQT_P_SLOTS] = valid ? a.players[(size_t)g * P * QQT_P_SLOTS + i] : 0;
  if (l < QQT_E_SLOTS) s.ev[e][l] = valid ? a.envs[(size_t)g * QQT_E_SLOTS + l] : 0;
  if (l == 0) s.done[e] = 0;
  // PROBE's bomb actions, issued together with the state loads
  int in_bb = 0;
  if (mode == QQT_MODE_PROBE && l < P && valid)
    in_bb = a.actions ? (int)a.actions[((size_t)g * P + l) * 2 + 1]
                      : a.actions_i8[((size_t)g * P + l) * 2 + 1];
  wave_sync();

  if (mode == QQT_MODE_PROBE) {
    // fuse countdown, live counts, placement as the tick makes them
    // (sim/torch_sim.py:1357-1402), then the largest bomb_blast
    if (l < P) {
      s.alive0[e][l] = pl[l][QQT_P_ALIVE];
      s.act_b[e][l] = in_bb;
      const float y = __int_as_float(pl[l][QQT_P_Y]), x = __int_as_float(pl[l][QQT_P_X]);
      s.fpre[e][l] = min(max((int)floorf(y) * W + (int)floorf(x), 0), C - 1);
    }
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      if (c < C) {
        const uint32_t w = cw[c];
        const int f = cw_fuse(w);
        if (f > 0) cw[c] = (w & ~0xFFu) | (uint32_t)(f - 1);
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int t = env_count<G>(e, l, [&](int c) {
        const uint32_t w = cw[c];
        return cw_fuse(w) > 0 && cw_owner(w) == i;
      });
      if (l == 0) s.live[e][i] = t;
    }
    wave_sync();

    // ---- 2. placement, players in id order (sim/torch_sim.py:1357-1402)
    if (l == 0) {
      for (int me = 0; me < P; ++me) {
        const int idx = s.fpre[e][me];
        const uint32_t w = cw[idx];
        const bool ok = s.alive0[e][me] && s.act_b[e][me] == 1 && cw_fuse(w) <= 0 &&
                        !(w & F_BRICK) && s.live[e][me] < pl[me][QQT_P_BOMBS_CAP];
        if (ok) cw[idx] = cw_make(w, cf.fuse, me, pl[me][QQT_P_BLAST_CAP]);
      }
    }
    wave_sync();

    {   // PROBE: the largest bomb_blast after placement
      int mb = 0;
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        if (c < C) mb = max(mb, cw_bb(cw[c]));
      }
      mb = env_max<LPE>(mb);
      if (valid && l == 0) a.probe_out[g] = mb;
      return;
    }
  }

  auto template_reset = [&]() {  // qqtsim/maps.py; re-init of sim/torch_sim.py:178-420
    const uint32_t env_id = (uint32_t)g;
    // rolled: one copy of the per-cell Philox draw (this code runs rarely,
    // and its size slows every tick)
#pragma unroll 1
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      if (c >= C) continue;
      const int r = c / W, col = c % W;
      bool wall = false;
      if (cf.map_kind == 0)
        wall = r == 0 || r == H - 1 || col == 0 || col == W - 1 || ((r % 2 == 0) && (col % 2 == 0));
      bool keep = false;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int sr = (i == 0 || i == 2) ? 1 : H - 2;
        const int sc = (i == 0 || i == 3) ? 1 : W - 2;
        const int dr = sr < H / 2 ? 1 : -1, dc = sc < W / 2 ? 1 : -1;
        keep |= (r == sr && col == sc) || (r == sr && col == sc + dc) || (r == sr + dr && col == sc);
      }
      bool brick = false;
      if (!wall && !keep && cf.brick_p > 0.0f)
        brick = philox_uniform(a.seed, env_id, a.epoch, STREAM_RESET_CELL, (uint32_t)c) < cf.brick_p;
      cw[c] = (wall ? F_WALL : 0u) | (brick ? F_BRICK : 0u) | EMPTY_CELL;
      s.dng[e][c] = 0.0f;
    }
    // the misc values 0..11: lane j draws block min(j, 2), lane 0 gathers
    float ub[4];
    philox_block(a.seed, env_id, a.epoch, STREAM_RESET_MISC, (uint32_t)min(l, 2), ub);
    float u[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) u[j] = __shfl(ub[j % 4], j / 4, LPE);
    if (l == 0) {
      float py[P], px[P];
#pragma unroll
      for (int i = 0; i < P; ++i) {
        py[i] = (float)((i == 0 || i == 2) ? 1 : H - 2) + 0.5f;
        px[i] = (float)((i == 0 || i == 3) ? 1 : W - 2) + 0.5f;
      }
      if (cf.swap_spawns && u[0] < 0.5f) {
        const float ty = py[0], tx = px[0];
        py[0] = py[1]; px[0] = px[1]; py[1] = ty; px[1] = tx;
      }
      const int bspan = cf.bombs_hi - cf.bombs_lo + 1, zspan = cf.blast_hi - cf.blast_lo + 1;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int bc = cf.bombs_lo + min((int)floorf(u[1 + 2 * i] * (float)bspan), bspan - 1);
        const int zc = cf.blast_lo + min((int)floorf(u[2 + 2 * i] * (float)zspan), zspan - 1);
        int32_t* q = pl[i];
        q[QQT_P_Y] = __float_as_int(py[i]);
        q[QQT_P_X] = __float_as_int(px[i]);
        q[QQT_P_ALIVE] = 1;
        q[QQT_P_HP] = cf.max_hp;
        q[QQT_P_SINCE_BOMB] = cf.spawn_cooldown;
        q[QQT_P_BOMBS_CAP] = bc;
        q[QQT_P_BLAST_CAP] = zc;
        q[QQT_P_SPD] = __float_as_int(cf.spawn_speed);
        q[QQT_P_INVULN] = 0;
        q[QQT_P_COMBO] = 0;
        q[QQT_P_LAST_HIT] = -1000000000;
        q[QQT_P_PENDING_LOST] = 0;
        q[QQT_P_LO_BOMBS] = bc;
        q[QQT_P_LO_BLAST] = zc;
        q[QQT_P_LO_SPD] = __float_as_int(cf.spawn_speed);
        q[15] = 0;
      }
      s.ev[e][QQT_E_T] = 0;
      s.ev[e][QQT_E_CRATE_PROB] = __float_as_int(cf.growth_crate_prob);
      s.ev[e][QQT_E_MAP_KIND] = 0;
    }
  };

  // The reference's reset map modes (BatchedSim.reset_, sim/torch_sim.py:
  // 178-420; generators sim/mapgen.py:15-242).  Every lane of the env runs
  // it.  Draws: STREAM_RESET_MISC values 0 map type, 1 top wall rows,
  // 2 spawn swap, 3 obstacle count, 4.. the corridor edge segments (start,
  // length, on) x 4 columns then the horizontal one; STREAM_RESET_CELL value
  // c the ring band's brick draw, C + c the open obstacles' keys (the n
  // cells with the smallest (key, cell)).
  auto reference_reset = [&]() {
    const uint32_t env_id = (uint32_t)g;
    float ub[4];
    philox_block(a.seed, env_id, a.epoch, STREAM_RESET_MISC, (uint32_t)min(l, 4), ub);
    float u[19];
#pragma unroll
    for (int j = 0; j < 19; ++j) u[j] = __shfl(ub[j % 4], j / 4, LPE);
    // map kind (uniform over the env's lanes): 0 corridor, 1 open, 2 ring
    int kind = 1;
    bool pure = false;
    if (cf.corridor) {
      kind = u[0] < cf.thr_open ? 1 : u[0] < cf.thr_ring ? 2 : 0;
      pure = u[0] < cf.thr_pure;
    }
    const int T = cf.top_wall_rows;
    const int top = cf.random_wall_rows ? min((int)floorf(u[1] * (float)(T + 1)), T) : T;
    const int bot = cf.random_wall_rows ? T - top : 0;
    const int sp_mode = cf.corridor ? 0 : 1;    // cfg.spawn_cells(): the mode's own spawns
    const int sp_kind = kind == 0 ? 0 : kind == 2 ? 2 : 1;
    auto near_spawn = [&](int set, int r, int col) {
      bool nb = false;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int sc = cf.ref_spawn_cell[set][i];
        const int dr = r - sc / W, dc = col - sc % W;
        nb |= (dr == 0 && (dc == 0 || dc == 1 || dc == -1)) || (dc == 0 && (dr == 1 || dr == -1));
      }
      return nb;
    };
    // open obstacles: bit k marks cell l + LPE k
    uint32_t obst = 0;
    const int nmax = cf.open_obstacle_max;
    const int nobst = nmax > 0 ? min((int)floorf(u[3] * (float)(nmax + 1)), nmax) : 0;
    if (kind == 1 && !pure && nobst > 0) {
      uint64_t key[KMAX];
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        key[k] = ~0ull;
        if (c < C) {
          const float uk = philox_uniform(a.seed, env_id, a.epoch, STREAM_RESET_CELL,
                                          (uint32_t)(C + c));
          key[k] = ((uint64_t)__float_as_uint(uk) << 32) | (uint32_t)c;
        }
      }
      for (int t = 0; t < nobst; ++t) {
        uint64_t mn = key[0];
#pragma unroll
        for (int k = 1; k < KMAX; ++k) mn = key[k] < mn ? key[k] : mn;
#pragma unroll
        for (int m = 1; m < LPE; m <<= 1) {
          const uint64_t o = __shfl_xor(mn, m, LPE);
          mn = o < mn ? o : mn;
        }
#pragma unroll
        for (int k = 0; k < KMAX; ++k)
          if (key[k] == mn) {
            obst |= 1u << k;
            key[k] = ~0ull;
          }
      }
    }
    // corridor geometry and edge segments (sim/mapgen.py:101-199)
    const int c0 = (W - cf.corridor_width) / 2, c1 = c0 + cf.corridor_width;
    const bool segs = kind == 0 && cf.wall_density > 0.0f;
    const int ecol[4] = {c0, c0 + 1, c1 - 2, c1 - 1};
    int vs[4], vl[4];
    bool va[4];
#pragma unroll
    for (int ci = 0; ci < 4; ++ci) {
      const float us = u[4 + 3 * ci], ul = u[5 + 3 * ci], ua = u[6 + 3 * ci];
      vs[ci] = cf.random_wall_rows
          ? (int)(us * (float)max(H - bot - 4 - top, 1) + (float)top)
          : (int)(us * (float)(H - T - 4) + (float)T);
      vl[ci] = 2 + (int)(ul * 3.0f);
      va[ci] = segs && ua < cf.wall_density && ecol[ci] >= c0 && ecol[ci] < c1;
    }
    const int hs = (int)(u[16] * (float)(c1 - c0 - 4) + (float)c0);
    const int hl = 2 + (int)(u[17] * 3.0f);
    const bool ha = segs && c1 - c0 > 4 && u[18] < cf.wall_density;
    const int hr0 = cf.random_wall_rows ? top : T;
    const int hr1 = cf.random_wall_rows ? top + 2 : T + min(2, H - T);
    // ring geometry (sim/mapgen.py:202-242)
    const int r0 = (H - cf.ring_center_h) / 2, q0 = (W - cf.ring_center_w) / 2;
    const int r1 = r0 + cf.ring_center_h, q1 = q0 + cf.ring_center_w;
    const int cy = (H - 1) / 2, cx = (W - 1) / 2;
#pragma unroll 1
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      if (c >= C) continue;
      const int r = c / W, col = c % W;
      bool wall = false, brick = false, crate = false;
      if (kind == 0) {
        wall = cf.random_wall_rows ? (r < top || r >= H - bot) : r < T;
        brick = (col < c0 || col >= c1) && r >= (cf.random_wall_rows ? top : T);
#pragma unroll
        for (int ci = 0; ci < 4; ++ci)
          brick |= va[ci] && col == ecol[ci] && r >= vs[ci] && r < vs[ci] + vl[ci];
        brick |= ha && r >= hr0 && r < hr1 && col >= c0 && col < c1 && col >= hs && col < hs + hl;
        if (near_spawn(sp_mode, r, col)) wall = brick = false;
      } else if (kind == 2) {
        wall = r >= r0 && r < r1 && col >= q0 && col < q1;
        const bool band = !wall && r >= r0 - 1 && r <= r1 && col >= q0 - 1 && col <= q1;
        if (band && !near_spawn(2, r, col))
          brick = philox_uniform(a.seed, env_id, a.epoch, STREAM_RESET_CELL, (uint32_t)c) <
                  cf.ring_brick_density;
      } else {
        wall = ((obst >> k) & 1u) && !near_spawn(sp_mode, r, col);
        crate = cf.corridor && cf.open_crate_cross &&
                (r == cy - 1 || r == cy || col == cx - 1 || col == cx) && !near_spawn(1, r, col);
      }
      cw[c] = (wall ? F_WALL : 0u) | (brick ? F_BRICK : 0u) | (crate ? F_CRATE : 0u) | EMPTY_CELL;
      s.dng[e][c] = 0.0f;
    }
    if (l == 0) {
      int b0, z0;
      float s0;
      if (!cf.corridor) {
        b0 = cf.max_bombs; z0 = cf.blast; s0 = 1.0f;
      } else if (kind == 1) {
        b0 = cf.open_growth_bombs; z0 = cf.open_growth_blast; s0 = cf.open_growth_speed;
      } else {
        b0 = cf.growth_bombs_start; z0 = cf.growth_blast_start; s0 = cf.growth_speed_start;
      }
      int b1 = b0, z1 = z0;
      float s1 = s0;
      if (a.opp_boost == 2) {
        b1 = cf.opp_growth_bombs; z1 = cf.opp_growth_blast; s1 = cf.opp_growth_speed;
      } else if (a.opp_boost == 1) {
        b1 = (int)fminf(rintf((float)b0 * cf.opp_hist_mult), (float)cf.growth_bombs_max);
        z1 = (int)fminf(rintf((float)z0 * cf.opp_hist_mult), (float)cf.growth_blast_max);
        s1 = fminf(s0 * cf.opp_hist_mult, cf.growth_speed_max);
      }
      const bool swap = u[2] < 0.5f;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int si = (swap && i < 2) ? 1 - i : i;
        int32_t* q = pl[i];
        q[QQT_P_Y] = __float_as_int(cf.ref_spawn_y[sp_kind][si]);
        q[QQT_P_X] = __float_as_int(cf.ref_spawn_x[sp_kind][si]);
        q[QQT_P_ALIVE] = 1;
        q[QQT_P_HP] = cf.max_hp;
        q[QQT_P_SINCE_BOMB] = cf.spawn_cooldown;
        q[QQT_P_INVULN] = 0;
        q[QQT_P_COMBO] = 0;
        q[QQT_P_LAST_HIT] = -1000000000;
        q[QQT_P_PENDING_LOST] = 0;
        if (i < 2) {            // players 2 and 3 keep caps, speed and floors
          const int bc = i == 0 ? b0 : b1, zc = i == 0 ? z0 : z1;
          const float sp = i == 0 ? s0 : s1;
          q[QQT_P_BOMBS_CAP] = bc;
          q[QQT_P_BLAST_CAP] = zc;
          q[QQT_P_SPD] = __float_as_int(sp);
          q[QQT_P_LO_BOMBS] = bc;
          q[QQT_P_LO_BLAST] = zc;
          q[QQT_P_LO_SPD] = __float_as_int(sp);
        }
      }
      s.ev[e][QQT_E_T] = 0;
      if (cf.corridor)
        s.ev[e][QQT_E_CRATE_PROB] = __float_as_int(
            kind == 1 ? 1.0f : kind == 2 ? cf.ring_crate_prob : cf.growth_crate_prob);
      s.ev[e][QQT_E_MAP_KIND] = kind;
    }
  };

  // RESET mode marks its envs here and resets them at the auto-reset site
  // below (one inline copy of the reset code); their danger map, computed
  // in between from the old state, is cleared by the reset.
  if (mode == QQT_MODE_RESET && l == 0) s.done[e] = valid && a.reset_mask[g] != 0;

  // ---- recycle flush (sim/torch_sim.py:549-596): player by player, the
  // pending lost growth becomes that many recycle crates on distinct free
  // cells (no wall, no brick, not excluded), then the counts reset.  The
  // reference takes the first k of a random permutation of the free cells;
  // here the k free cells with the smallest Philox keys (stream 8, value
  // p*C + c) are taken, the same uniform k-subset law.
  if constexpr (KMODE == QQT_MODE_FLUSH) {
    bool freec[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      freec[k] = c < C && !(cw[c] & (F_WALL | F_BRICK)) && !a.recycle_excl[c];
    }
    for (int i = 0; i < P; ++i) {
      const int want = valid ? pl[i][QQT_P_PENDING_LOST] : 0;
      uint64_t key[KMAX];
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        key[k] = ~0ull;
        if (want > 0 && freec[k]) {
          const float u = philox_uniform(a.seed, (uint32_t)g, a.epoch, STREAM_RECYCLE,
                                         (uint32_t)(i * C + c));
          key[k] = ((uint64_t)__float_as_uint(u) << 32) | (uint32_t)c;   // u >= 0: bits order
        }
      }
      // every lane runs the same number of rounds (the wave's largest count)
      int rounds = want;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) rounds = max(rounds, __shfl_xor(rounds, m, 64));
      for (int t = 0; t < rounds; ++t) {
        uint64_t mn = key[0];
#pragma unroll
        for (int k = 1; k < KMAX; ++k) mn = key[k] < mn ? key[k] : mn;
#pragma unroll
        for (int m = 1; m < LPE; m <<= 1) {
          const uint64_t o = __shfl_xor(mn, m, 64);
          mn = o < mn ? o : mn;
        }
        if (t < want && mn != ~0ull) {
          const int c = (int)(mn & 0xFFu);
#pragma unroll
          for (int k = 0; k < KMAX; ++k)
            if (c == l + LPE * k) {
              cw[c] |= F_CRATE | F_REC;
              key[k] = ~0ull;
            }
        }
      }
    }
    wave_sync();
    if (l < P && valid) pl[l][QQT_P_PENDING_LOST] = 0;
    wave_sync();
  }

  // ---- danger map of the current state (sim/blast.py:158-317)
  {
    float* dng = s.dng[e];
    float* fw = s.dz.fw[e];
    float* wl = s.dz.wl[e];
    const int nb = build_list<G>(list, e, l, [&](int c) { return cw_fuse(cw[c]) > 0; });
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      if (c < C) dng[c] = 0.0f;
    }
    const bool wave_bombs = __any(nb > 0);
    if (wave_bombs) {
      // weights; stage-A front = weight at every bomb (walls included: the
      // reference's stage-A origins are not masked by passability)
      for (int j = l; j < nb; j += LPE) {
        const int c = list[j];
        const float w0 = bomb_weight(cw_fuse(cw[c]), fmax_f);
        wl[j] = w0;
        fw[c] = w0;
      }
      if (cf.max_chain > 1) {
        // in-edges, one (bomb, direction) per item: the first solid cell
        // behind the bomb, kept if it is a bomb whose range reaches it
        for (int it = l; it < 4 * nb; it += LPE) {
          const int j = it >> 2, d = it & 3;
          const int c = list[j];
          uint16_t ed = 0;
          if (!(cw[c] & F_WALL)) {
            // backwards from the bomb: the first solid cell behind it
            walk_ray<H, W>(cw, c, d, H + W, -1, [&](int k, int u, uint32_t wu) {
              if (cw_fuse(wu) > 0) {
                if (blast_of(wu, cf.blast) >= k) ed = (uint16_t)(u | (k << 8));
                return false;
              }
              return !(wu & (F_WALL | F_BRICK));
            });
          }
          s.dz.edge[e][j][d] = ed;
        }
        // stage A: synchronous relay rounds
        const int rounds = min(cf.max_chain, cf.chain_cap_rounds);
        for (int r = 0; r < rounds; ++r) {
          wave_sync();
          float nf[KMAX];
          bool upd = false;
#pragma unroll
          for (int i = 0; i < KMAX; ++i) {
            const int j = l + LPE * i;
            nf[i] = 0.0f;
            if (j >= nb) continue;
            float spread = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint16_t ed = s.dz.edge[e][j][d];
              if (ed) spread = fmaxf(spread, fw[ed & 0xFF]);
            }
            const float nv = spread > wl[j] ? spread : 0.0f;
            nf[i] = nv;
            upd |= nv > 0.0f;
          }
          wave_sync();
#pragma unroll
          for (int i = 0; i < KMAX; ++i) {
            const int j = l + LPE * i;
            if (j >= nb) continue;
            const float nv = nf[i];
            if (nv > 0.0f) wl[j] = nv;
            fw[list[j]] = nv;
          }
          if (!__any(upd)) break;
        }
      }
      wave_sync();
      // stage B: every (bomb, direction) ray max-updates the danger map.
      // Danger values are >= 0, so their float bits order like ints and an
      // LDS integer atomic max is exact whatever the order of the rays.
      int* dngi = reinterpret_cast<int*>(dng);
      for (int it = l; it < 4 * nb; it += LPE) {
        const int j = it >> 2, d = it & 3;
        const int c = list[j];
        const uint32_t wc = cw[c];
        const float v = wl[j];
        if (wc & F_WALL) continue;
        if (d == 0) atomicMax(&dngi[c], __float_as_int(v));  // the bomb's own cell (seed)
        walk_ray<H, W>(cw, c, d, blast_of(wc, cf.blast), 1, [&](int, int x, uint32_t wx) {
          if (wx & F_WALL) return false;
          atomicMax(&dngi[x], __float_as_int(v));
          return !cw_solid(wx);
        });
      }
    }
    wave_sync();
  }
  // the float32 danger map itself, for callers that read it (OBSERVE launches;
  // the STEP and FLUSH instantiations carry no such code)
  if constexpr (KMODE < 0) {
    if (mode == QQT_MODE_OBSERVE && a.danger_out && valid) {
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        if (c < C) a.danger_out[(size_t)g * C + c] = s.dng[e][c];
      }
    }
  }

  if (mode == QQT_MODE_RESET) {
    wave_sync();
    if (s.done[e]) {
      if constexpr (MAPS == 1) reference_reset();
      else template_reset();
    }
    wave_sync();
  }

  // ---- observation + legality masks of the current state (sim/obs.py:25-229)
  const int opad = (int)(((uintptr_t)(a.obs + (size_t)g0 * OBS)) & 15u);  // staging offset
  {
    // everything starts as zero; only nonzero values are written afterwards
    {
      uint4* z = reinterpret_cast<uint4*>(s.obs_raw);
      constexpr int N16 = sizeof(s.obs_raw) / 16;
      for (int i = lane; i < N16; i += 64) z[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    wave_sync();
    uint16_t* ob = reinterpret_cast<uint16_t*>(s.obs_raw + opad) + (size_t)e * OBS;
    const float tplane = __fdiv_rn((float)s.ev[e][QQT_E_T], (float)cf.max_steps);
    const uint16_t h_one = __half_as_ushort(__float2half_rn(1.0f));
    const uint16_t h_t = __half_as_ushort(__float2half_rn(tplane));
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      if (c >= C) continue;
      const uint32_t w = cw[c];
      const float dv = s.dng[e][c];
      if (w & (F_WALL | F_BRICK)) ob[(2 * P) * C + c] = h_one;
      if (dv != 0.0f) ob[(2 * P + 1) * C + c] = __half_as_ushort(__float2half_rn(dv));
      ob[(2 * P + 2) * C + c] = h_t;
      if (w & F_CRATE) ob[(2 * P + 3) * C + c] = h_one;
    }
    // fuse channels from the bomb cells: list[] still holds them unless this
    // env was reset (then it has no bombs)
    const int nbo = build_list<G>(list, e, l, [&](int c) { return cw_fuse(cw[c]) > 0; });
    for (int j = l; j < nbo; j += LPE) {
      const int c = list[j];
      const uint32_t w = cw[c];
      const int o = cw_owner(w);
      if (o >= 0 && o < P)
        ob[(P + o) * C + c] = __half_as_ushort(__float2half_rn(__fdiv_rn((float)cw_fuse(w), fmax_f)));
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int t = env_count<G>(e, l, [&](int c) {
        const uint32_t w = cw[c];
        return cw_fuse(w) > 0 && cw_owner(w) == i;
      });
      if (l == 0) s.live[e][i] = t;
    }
    wave_sync();
    if (l < P) {
      // splat: the four corner terms accumulate in order (0,0),(0,1),(1,0),(1,1)
      const int i = l;
      const float py = __int_as_float(pl[i][QQT_P_Y]), px = __int_as_float(pl[i][QQT_P_X]);
      const bool al = pl[i][QQT_P_ALIVE] != 0;
      const float gate = (float)al;
      const float fy = fminf(fmaxf(py - 0.5f, 0.0f), (float)(H - 1));
      const float fx = fminf(fmaxf(px - 0.5f, 0.0f), (float)(W - 1));
      const int y0 = min(max((int)floorf(fy), 0), H - 1);
      const int x0 = min(max((int)floorf(fx), 0), W - 1);
      const int y1 = min(y0 + 1, H - 1), x1 = min(x0 + 1, W - 1);
      const float wy = fminf(fmaxf(fy - (float)y0, 0.0f), 1.0f);
      const float wx = fminf(fmaxf(fx - (float)x0, 0.0f), 1.0f);
      const float ky0 = 1.0f - wy, kx0 = 1.0f - wx;
      const int id[4] = {y0 * W + x0, y0 * W + x1, y1 * W + x0, y1 * W + x1};
      const float wt[4] = {(ky0 * kx0) * gate, (ky0 * wx) * gate, (wy * kx0) * gate, (wy * wx) * gate};
      float run[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float prev = 0.0f;
#pragma unroll
        for (int j = 0; j < q; ++j)
          if (id[j] == id[q]) prev = run[j];
        run[q] = prev + wt[q];
        ob[i * C + id[q]] = __half_as_ushort(__float2half_rn(run[q]));
      }
      const int cell = min(max((int)floorf(py) * W + (int)floorf(px), 0), C - 1);
      const int capi = pl[i][QQT_P_BOMBS_CAP];
      const float cap = fmaxf((float)capi, 1.0f);
      const float avail = fmaxf((float)(capi - s.live[e][i]), 0.0f);
      const float inv = (pl[i][QQT_P_INVULN] > 0 && al) ? 1.0f : 0.0f;
      ob[(2 * P + 4 + i) * C + cell] = __half_as_ushort(__float2half_rn(inv));
      ob[(3 * P + 4 + i) * C + cell] = __half_as_ushort(__float2half_rn(__fdiv_rn(avail, cap) * gate));
      ob[(4 * P + 4 + i) * C + cell] =
          __half_as_ushort(__float2half_rn(__fdiv_rn(cap, (float)cf.growth_bombs_max) * gate));
    }

    // masks: lane = me*4 + probe (up, down, left, right)
    const int me = l >> 2, pr = l & 3;
    if (me < P && valid) {
      const float y = __int_as_float(pl[me][QQT_P_Y]), x = __int_as_float(pl[me][QQT_P_X]);
      const bool al = pl[me][QQT_P_ALIVE] != 0;
      const float st = cf.step_len;
      const float d = (pr & 1) ? st : -st;
      bool moved;
      const bool vert = pr < 2;
      const float own = vert ? y : x;
      const float nv = resolve_axis<H, W>(cw, own + d, d, y, x, rad, vert);
      moved = fabsf(nv - own) > 2e-4f;
      if (a.move_mask) {
        a.move_mask[((size_t)g * P + me) * 5 + pr] = al ? moved : 1;
        if (pr == 0) a.move_mask[((size_t)g * P + me) * 5 + 4] = 1;
      }
      if (pr == 0 && a.bomb_mask) {
        const int flat = min(max((int)floorf(y) * W + (int)floorf(x), 0), C - 1);
        const uint32_t wc = cw[flat];
        const bool under = cw_fuse(wc) > 0;
        const bool can = !under && !(wc & F_BRICK) && s.live[e][me] < pl[me][QQT_P_BOMBS_CAP];
        a.bomb_mask[((size_t)g * P + me) * 2 + 0] = 1;
        a.bomb_mask[((size_t)g * P + me) * 2 + 1] = (can && al) || !al;
      }
    }
  }
  wave_sync();

  // ---- store state and the staged observation
  if (mode == QQT_MODE_RESET || mode == QQT_MODE_FLUSH) {
    if (valid) {
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        if (c < C) a.cells[(size_t)g * C + c] = (int32_t)cw[c];
      }
      for (int i = l; i < P * QQT_P_SLOTS; i += LPE)
        a.players[(size_t)g * P * QQT_P_SLOTS + i] = pl[i / QQT_P_SLOTS][i % QQT_P_SLOTS];
      if (l < QQT_E_SLOTS) a.envs[(size_t)g * QQT_E_SLOTS + l] = s.ev[e][l];
    }
  }
  if (a.obs) {
    // staging and destination share their address mod 16: u16 head, 16-byte
    // body, u16 tail
    const int nvalid = min(EPW, a.n_envs - g0);
    const int bytes = nvalid * OBS * 2;
    uint8_t* dst = (uint8_t*)(a.obs + (size_t)g0 * OBS);
    const uint8_t* src = s.obs_raw + opad;
    const int head = min((16 - opad) & 15, bytes);
    const int n16 = (bytes - head) / 16;
    if (lane * 2 < head)
      *reinterpret_cast<uint16_t*>(dst + lane * 2) = *reinterpret_cast<const uint16_t*>(src + lane * 2);
    for (int i = lane; i < n16; i += 64)
      reinterpret_cast<uint4*>(dst + head)[i] = reinterpret_cast<const uint4*>(src + head)[i];
    const int tail0 = head + n16 * 16;
    if (tail0 + lane * 2 < bytes)
      *reinterpret_cast<uint16_t*>(dst + tail0 + lane * 2) =
          *reinterpret_cast<const uint16_t*>(src + tail0 + lane * 2);
  }
}

// ---------------------------------------------------------------- host side
thread_local char g_err[512] = "";

int fail(int code, const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

#ifndef QQT_LPE
#define QQT_LPE 64
#endif
#ifndef QQT_TICK_WPB
#define QQT_TICK_WPB 2
#endif

// The STEP tick (tick_group.hip): two envs per wavefront up to 8192 envs,
// four above.
template <int H, int W, int P>
int launch_step_group(const qqt_sim_config* cfg, const qqt_tick_args* a, hipStream_t st);

template <int H, int W, int P>
int launch(const qqt_sim_config* cfg, const qqt_tick_args* a, hipStream_t st) {
  if (a->mode == QQT_MODE_STEP) return launch_step_group<H, W, P>(cfg, a, st);
  constexpr int LPE = QQT_LPE;
  constexpr int WPB = QQT_TICK_WPB;
  constexpr int EPW = 64 / LPE;
  // XCD_ROWS-env row blocks, a multiple of 8 of them (one per XCD in turn)
  const int nrb = (a->n_envs + XCD_ROWS - 1) / XCD_ROWS;
  const int blocks = ((nrb + 7) / 8) * 8 * (XCD_ROWS / (WPB * EPW));
  const bool ref = cfg->map_kind == QQT_MAP_REFERENCE;
  const dim3 grid(blocks), block(64 * WPB);
  if (a->mode == QQT_MODE_FLUSH)     // no reset in a flush
    QQT_LAUNCH(QQT_KERNEL_TICK, (tick_kernel<H, W, P, LPE, WPB, QQT_MODE_FLUSH, 0>), grid, block, st,
               *cfg, *a);
  else if (!ref)
    QQT_LAUNCH(QQT_KERNEL_TICK, (tick_kernel<H, W, P, LPE, WPB, -1, 0>), grid, block, st, *cfg, *a);
  else
    QQT_LAUNCH(QQT_KERNEL_TICK, (tick_kernel<H, W, P, LPE, WPB, -1, 1>), grid, block, st, *cfg, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "tick launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // namespace qqt

extern "C" {

int qqt_abi_version(void) { return QQT_ABI_VERSION; }

const char* qqt_last_error(void) { return qqt::g_err; }

int qqt_tick(const qqt_sim_config* cfg, const qqt_tick_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!cfg || !a) return fail(QQT_E_ARG, "null config or args");
  if (a->n_envs <= 0) return fail(QQT_E_ARG, "n_envs must be positive");
  if (!a->cells || !a->players || !a->envs) return fail(QQT_E_ARG, "null state pointer");
  if (a->mode < QQT_MODE_STEP || a->mode > QQT_MODE_FLUSH) return fail(QQT_E_ARG, "bad mode");
  if (a->mode == QQT_MODE_FLUSH && !a->recycle_excl)
    return fail(QQT_E_ARG, "FLUSH needs recycle_excl");
  if (a->mode == QQT_MODE_STEP && !a->actions && !a->actions_i8)
    return fail(QQT_E_ARG, "STEP needs actions");
  if (a->mode == QQT_MODE_PROBE && !a->actions && !a->actions_i8)
    return fail(QQT_E_ARG, "PROBE needs actions");
  if (a->mode == QQT_MODE_RESET && !a->reset_mask) return fail(QQT_E_ARG, "RESET needs reset_mask");
  if (a->mode == QQT_MODE_PROBE && !a->probe_out) return fail(QQT_E_ARG, "PROBE needs probe_out");
  if (a->obs && (((uintptr_t)a->obs) & 15)) return fail(QQT_E_ARG, "obs must be 16-byte aligned");
  if (a->tick_stats && (((uintptr_t)a->tick_stats) & 15))
    return fail(QQT_E_ARG, "tick_stats must be 16-byte aligned");
  if (a->reach_caps && (a->reach_pid < 0 || a->reach_pid >= cfg->n_players))
    return fail(QQT_E_ARG, "reach_pid out of range");
  if (cfg->fuse < 1 || cfg->fuse > 255) return fail(QQT_E_ARG, "fuse must be in 1..255");
  if (cfg->chain_cap_rounds < 0 || cfg->chain_cap_rounds > 64)
    return fail(QQT_E_ARG, "chain_cap_rounds must be in 0..64");
  if (cfg->bombs_lo > cfg->bombs_hi || cfg->blast_lo > cfg->blast_hi)
    return fail(QQT_E_ARG, "bad cap ranges");
  if (cfg->map_kind < QQT_MAP_PILLARS || cfg->map_kind > QQT_MAP_REFERENCE)
    return fail(QQT_E_ARG, "bad map_kind");
  if (cfg->map_kind == QQT_MAP_REFERENCE) {
    const int h = cfg->height, w = cfg->width, p = cfg->n_players;
    if (cfg->corridor_width < 3 || cfg->corridor_width > w - 2 || cfg->top_wall_rows < 1 ||
        cfg->top_wall_rows > h - 3 || cfg->ring_center_h < 3 || cfg->ring_center_h > h - 4 ||
        cfg->ring_center_w < 3 || cfg->ring_center_w > w - 4 || cfg->open_obstacle_max < 0 ||
        cfg->open_obstacle_max > h * w || a->opp_boost < 0 || a->opp_boost > 2)
      return fail(QQT_E_ARG, "reference map mode geometry out of range");
    for (int k = 0; k < 3; ++k)
      for (int i = 0; i < p; ++i)
        if (cfg->ref_spawn_cell[k][i] < 0 || cfg->ref_spawn_cell[k][i] >= h * w)
          return fail(QQT_E_ARG, "reference spawn cell outside the grid");
  }
  hipStream_t st = (hipStream_t)stream;
  const int h = cfg->height, w = cfg->width, p = cfg->n_players;
  if (h == 13 && w == 13 && p == 2) return launch<13, 13, 2>(cfg, a, st);
  if (h == 7 && w == 7 && p == 2) return launch<7, 7, 2>(cfg, a, st);
  if (h == 9 && w == 9 && p == 2) return launch<9, 9, 2>(cfg, a, st);
  if (h == 13 && w == 13 && p == 3) return launch<13, 13, 3>(cfg, a, st);
  if (h == 13 && w == 13 && p == 4) return launch<13, 13, 4>(cfg, a, st);
  snprintf(g_err, sizeof(g_err), "grid %dx%d with %d players is not compiled", h, w, p);
  return QQT_E_UNSUPPORTED;
}

}  // extern "C"
