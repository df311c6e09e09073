// Fused rollout tick for gfx950: step + auto-reset + danger + observation +
// legality masks of a batch of envs in one launch.
//
// Mapping: one 64-lane wavefront (= one workgroup) owns EPW = 4 consecutive
// envs; each env gets 16 lanes.  Lane l of an env walks the cells
// c = l, l+16, l+32, ...  Per-env grids live in LDS for the whole tick; the
// observation is staged in LDS in its final (N, C, H, W) float16 layout and
// leaves with 16-byte stores, so the output stream is written once, fully
// coalesced.  Per-player scalar work (placement, movement, damage, rewards,
// masks) runs on a few lanes per env while the grid phases use all 16.
//
// Semantics follow the reference tick (sim/torch_sim.py:895-1261) stage by
// stage in float32 with the reference's operation order; the library is
// built with -ffp-contract=off so no product is fused into an add.
//
// Chain explosion: flame is scattered from each source cell along its four
// rays (byte stores of 1 into an LDS cover map are idempotent, so lanes that
// reach the same cell need no atomics), one synchronous round at a time.
// Danger map: gathered (each cell scans back along the four directions to
// the first bomb/brick/wall), never scattered, so max-combining needs no
// atomics either.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

constexpr int EPW = 4;   // envs per wavefront
constexpr int LPE = 16;  // lanes per env

constexpr uint32_t F_WALL = 1u << 24, F_BRICK = 1u << 25, F_CRATE = 1u << 26, F_REC = 1u << 27;

__device__ __forceinline__ int cw_fuse(uint32_t w) { return (int)(w & 0xFFu); }
__device__ __forceinline__ int cw_owner(uint32_t w) { return (int)(int8_t)((w >> 8) & 0xFFu); }
__device__ __forceinline__ int cw_bb(uint32_t w) { return (int)((w >> 16) & 0xFFu); }
__device__ __forceinline__ uint32_t cw_make(uint32_t flags, int fuse, int owner, int bb) {
  return (flags & 0xFF000000u) | ((uint32_t)fuse & 0xFFu) | (((uint32_t)owner & 0xFFu) << 8) |
         (((uint32_t)bb & 0xFFu) << 16);
}

// Sum / max over the 16 lanes of one env (all 16 lanes receive the result).
__device__ __forceinline__ int sum16(int v) {
  v += __shfl_xor(v, 8, 16);
  v += __shfl_xor(v, 4, 16);
  v += __shfl_xor(v, 2, 16);
  v += __shfl_xor(v, 1, 16);
  return v;
}
__device__ __forceinline__ int max16(int v) {
  v = max(v, __shfl_xor(v, 8, 16));
  v = max(v, __shfl_xor(v, 4, 16));
  v = max(v, __shfl_xor(v, 2, 16));
  v = max(v, __shfl_xor(v, 1, 16));
  return v;
}

template <int H, int W, int P>
struct Geo {
  static constexpr int C = H * W;
  static constexpr int NCH = 5 * P + 4;
  static constexpr int OBS = NCH * C;  // float16 values per env
  static constexpr int MAXR = (H > W ? H : W) - 1;  // longest in-grid ray
};

template <int H, int W, int P>
struct __align__(16) Lds {
  using G = Geo<H, W, P>;
  uint16_t obs[EPW][G::OBS];
  uint32_t cw[EPW][G::C];
  float fw[EPW][G::C];   // danger: stage-A front / stage-B sender weight
  float dng[EPW][G::C];  // danger output
  uint8_t cov[EPW][G::C];
  uint8_t trg[EPW][G::C];
  int32_t pl[EPW][P][QQT_P_SLOTS];
  int32_t ev[EPW][QQT_E_SLOTS];
  int32_t alive0[EPW][P], hp0[EPW][P], placed[EPW][P], live[EPW][P];
  int32_t fpre[EPW][P], fpost[EPW][P], act_m[EPW][P], act_b[EPW][P];
  float pbonus[EPW][P];
  float splat_w[EPW][P][4];
  int32_t splat_i[EPW][P][4];
  int32_t done[EPW];
  int32_t any[EPW];
};

struct DevCfg {
  qqt_sim_config c;
};

// ---------------------------------------------------------------- movement
// One axis of the AABB slide-stop resolution (sim/move.py:154-231).
template <int H, int W>
__device__ __forceinline__ bool blocked_pair(const uint32_t* cw, int r0, int c0, int r1, int c1,
                                             float yb, float xb, float rad) {
  const bool oob = (r0 < 0) | (r0 >= H) | (c0 < 0) | (c0 >= W) | (r1 < 0) | (r1 >= H) |
                   (c1 < 0) | (c1 >= W);
  const int i0 = min(max(r0, 0), H - 1) * W + min(max(c0, 0), W - 1);
  const int i1 = min(max(r1, 0), H - 1) * W + min(max(c1, 0), W - 1);
  const uint32_t w0 = cw[i0], w1 = cw[i1];
  const bool s0 = (w0 & (F_WALL | F_BRICK)) || cw_fuse(w0) > 0;
  const bool s1 = (w1 & (F_WALL | F_BRICK)) || cw_fuse(w1) > 0;
  const int top = (int)floorf(yb - rad), bot = (int)floorf(yb + rad);
  const int lef = (int)floorf(xb - rad), rig = (int)floorf(xb + rad);
  const bool in0 = (r0 >= top) & (r0 <= bot) & (c0 >= lef) & (c0 <= rig);
  const bool in1 = (r1 >= top) & (r1 <= bot) & (c1 >= lef) & (c1 <= rig);
  return oob | (s0 & !in0) | (s1 & !in1);
}

template <int H, int W>
__device__ __forceinline__ float resolve_axis(const uint32_t* cw, float coord, float delta,
                                              float other, float y, float x, float rad,
                                              bool vertical) {
  const float eps = 1e-4f;
  const float sgn = delta > 0.0f ? 1.0f : (delta < 0.0f ? -1.0f : 0.0f);
  const int old_lead = (int)floorf((coord - delta) + sgn * rad);
  const int new_lead = (int)floorf(coord + sgn * rad);
  const int lo = min(old_lead, new_lead), hi = max(old_lead, new_lead);
  const int a0 = (int)floorf(other - rad), a1 = (int)floorf(other + rad);
  bool hit_lo, hit_hi;
  if (vertical) {
    hit_lo = blocked_pair<H, W>(cw, lo, a0, lo, a1, y, x, rad);
    hit_hi = blocked_pair<H, W>(cw, hi, a0, hi, a1, y, x, rad);
  } else {
    hit_lo = blocked_pair<H, W>(cw, a0, lo, a1, lo, y, x, rad);
    hit_hi = blocked_pair<H, W>(cw, a0, hi, a1, hi, y, x, rad);
  }
  const bool fwd = sgn > 0.0f;
  const int first_lead = fwd ? hi : lo, second_lead = fwd ? lo : hi;
  const bool fh = fwd ? hit_hi : hit_lo, sh = fwd ? hit_lo : hit_hi;
  const int stop_cell = fh ? first_lead : (sh ? second_lead : 0);
  const float sc = (float)stop_cell;
  const float stop = fwd ? ((sc - rad) - eps) : (((sc + 1.0f) + rad) + eps);
  return (fh | sh) ? stop : coord;
}

__device__ __forceinline__ int blast_of(uint32_t w, int cfg_blast) {
  const int b = cw_bb(w);
  return b > 0 ? b : cfg_blast;
}

// Danger weight (1 - (f-1)/FUSE)^2 clamped at 0 (sim/blast.py:218-220).
__device__ __forceinline__ float bomb_weight(int f, float fuse_max) {
  if (f <= 0) return 0.0f;
  const float raw = 1.0f - __fdiv_rn((float)f - 1.0f, fuse_max);
  const float v = raw > 0.0f ? raw : 0.0f;
  return v * v;
}

// ---------------------------------------------------------------- kernel
template <int H, int W, int P>
__global__ __launch_bounds__(64) void tick_kernel(const DevCfg dc, const qqt_tick_args a) {
  using G = Geo<H, W, P>;
  constexpr int C = G::C;
  constexpr int NCH = G::NCH;
  constexpr int OBS = G::OBS;
  __shared__ Lds<H, W, P> s;
  const qqt_sim_config& cf = dc.c;

  const int lane = threadIdx.x;
  const int e = lane >> 4;
  const int l = lane & 15;
  const int g = blockIdx.x * EPW + e;
  const bool valid = g < a.n_envs;
  const int mode = a.mode;
  const float rad = cf.radius;
  const float fmax_f = (float)cf.fuse;

  uint32_t* cw = s.cw[e];
  int32_t(*pl)[QQT_P_SLOTS] = s.pl[e];

  // ---- load
  for (int c = l; c < C; c += LPE)
    cw[c] = valid ? (uint32_t)a.cells[(size_t)g * C + c] : (F_WALL | 0x0000FF00u);
  for (int i = l; i < P * QQT_P_SLOTS; i += LPE)
    pl[i / QQT_P_SLOTS][i % QQT_P_SLOTS] = valid ? a.players[(size_t)g * P * QQT_P_SLOTS + i] : 0;
  if (l < QQT_E_SLOTS) s.ev[e][l] = valid ? a.envs[(size_t)g * QQT_E_SLOTS + l] : 0;
  if (l == 0) { s.done[e] = 0; s.any[e] = 0; }
  __syncthreads();

  bool do_reset = false;

  if (mode == QQT_MODE_STEP || mode == QQT_MODE_PROBE) {
    // ---- 1. snapshots, actions, fuse countdown
    if (l < P) {
      s.alive0[e][l] = pl[l][QQT_P_ALIVE];
      s.hp0[e][l] = pl[l][QQT_P_HP];
      int mv = 4, bb = 0;
      if (valid) {
        if (a.actions) {
          mv = (int)a.actions[((size_t)g * P + l) * 2 + 0];
          bb = (int)a.actions[((size_t)g * P + l) * 2 + 1];
        } else if (a.actions_i8) {
          mv = a.actions_i8[((size_t)g * P + l) * 2 + 0];
          bb = a.actions_i8[((size_t)g * P + l) * 2 + 1];
        }
      }
      s.act_m[e][l] = mv;
      s.act_b[e][l] = bb;
      const float y = __int_as_float(pl[l][QQT_P_Y]), x = __int_as_float(pl[l][QQT_P_X]);
      const int cy = (int)floorf(y), cx = (int)floorf(x);
      s.fpre[e][l] = min(max(cy * W + cx, 0), C - 1);
    }
    int cnt[P];
#pragma unroll
    for (int i = 0; i < P; ++i) cnt[i] = 0;
    for (int c = l; c < C; c += LPE) {
      uint32_t w = cw[c];
      const int f = cw_fuse(w);
      if (f > 0) { w = (w & ~0xFFu) | (uint32_t)(f - 1); cw[c] = w; }
      const int o = cw_owner(w);
      if (cw_fuse(w) > 0) {
#pragma unroll
        for (int i = 0; i < P; ++i) cnt[i] += (o == i);
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int t = sum16(cnt[i]);
      if (l == 0) s.live[e][i] = t;
    }
    __syncthreads();

    // ---- 2. placement, players in id order (sim/torch_sim.py:1357-1402)
    if (l == 0) {
      for (int me = 0; me < P; ++me) {
        const int idx = s.fpre[e][me];
        const uint32_t w = cw[idx];
        const bool ok = s.alive0[e][me] && s.act_b[e][me] == 1 && cw_fuse(w) <= 0 &&
                        !(w & F_BRICK) && s.live[e][me] < pl[me][QQT_P_BOMBS_CAP];
        s.placed[e][me] = ok;
        if (ok) cw[idx] = cw_make(w, cf.fuse, me, pl[me][QQT_P_BLAST_CAP]);
      }
    }
    __syncthreads();

    if (mode == QQT_MODE_PROBE) {
      int mb = 0;
      for (int c = l; c < C; c += LPE) mb = max(mb, cw_bb(cw[c]));
      mb = max16(mb);
      if (valid && l == 0) a.probe_out[g] = mb;
      return;
    }

    // ---- 3. placement reward (sim/torch_sim.py:1263-1355): lane = me*4 + dir
    {
      const int me = l >> 2, d = l & 3;
      float chain = 0.0f;
      int cover_bits = 0;
      if (me < P && s.placed[e][me]) {
        const int s0 = s.fpre[e][me];
        const uint32_t w0 = cw[s0];
        const bool seed_ok = !(w0 & (F_WALL | F_BRICK));
        if (seed_ok) {
          const int r0 = s0 / W, c0 = s0 % W;
          const int dr = d == 0 ? -1 : (d == 1 ? 1 : 0);
          const int dcol = d == 2 ? -1 : (d == 3 ? 1 : 0);
          auto visit = [&](int x) {
            for (int o = 0; o < P; ++o)
              if (o != me && s.fpre[e][o] == x && s.alive0[e][o]) cover_bits |= 1 << o;
            const uint32_t wx = cw[x];
            const int fx = cw_fuse(wx);
            if (fx > 0 && cw_owner(wx) >= 0) {
              int pm = 0;
              for (int i = 0; i < P; ++i)
                if (s.fpre[e][i] == x) pm = s.placed[e][i];
              if (!pm) {
                float frac = __fdiv_rn((float)fx, fmax_f);
                frac = fminf(fmaxf(frac, 0.0f), 1.0f);
                const float wt = cf.chain_time_factor + cf.chain_time_rest * (1.0f - frac);
                chain = chain + wt;
              }
            }
          };
          if (d == 0) visit(s0);
          const int b = blast_of(w0, cf.blast);
          for (int k = 1; k <= b; ++k) {
            const int rr = r0 + k * dr, cc = c0 + k * dcol;
            if (rr < 0 || rr >= H || cc < 0 || cc >= W) break;
            const int x = rr * W + cc;
            const uint32_t wx = cw[x];
            if (wx & F_WALL) break;
            visit(x);
            if ((wx & F_BRICK) || cw_fuse(wx) > 0) break;
          }
        }
      }
      // combine the four direction lanes of each player
      chain += __shfl_xor(chain, 1, 16);
      chain += __shfl_xor(chain, 2, 16);
      cover_bits |= __shfl_xor(cover_bits, 1, 16);
      cover_bits |= __shfl_xor(cover_bits, 2, 16);
      if (me < P && d == 0) {
        float bonus = 0.0f;
        if (s.placed[e][me]) {
          float cover = 0.0f, dist = 0.0f;
          for (int o = 0; o < P; ++o) cover += (float)((cover_bits >> o) & 1);
          if (cf.place_dist_reward > 0.0f) {
            const float ym = floorf(__int_as_float(pl[me][QQT_P_Y]));
            const float xm = floorf(__int_as_float(pl[me][QQT_P_X]));
            const bool cool = pl[me][QQT_P_SINCE_BOMB] >= cf.place_dist_cooldown;
            for (int o = 0; o < P; ++o) {
              if (o == me) continue;
              const float dy = ym - floorf(__int_as_float(pl[o][QQT_P_Y]));
              const float dx = xm - floorf(__int_as_float(pl[o][QQT_P_X]));
              const float dd = sqrtf(dy * dy + dx * dx);
              const bool under = (cover_bits >> o) & 1;
              const bool ok = !under && dd < cf.place_dist_radius && cool && s.alive0[e][o];
              const float gain = 1.0f - __fdiv_rn(dd, cf.place_dist_radius);
              dist = dist + (ok ? fmaxf(gain, 0.0f) : 0.0f);
            }
          }
          bonus = (cf.place_cover_reward * cover + cf.place_dist_reward * dist) +
                  cf.place_chain_reward * chain;
        }
        s.pbonus[e][me] = bonus * (float)s.alive0[e][me];
      }
    }
    __syncthreads();

    // ---- 4. since_bomb; 5. movement (sim/move.py:234-279)
    if (l < P) {
      const int me = l;
      int sb = pl[me][QQT_P_SINCE_BOMB] + 1;
      if (s.placed[e][me]) sb = 0;
      const float y = __int_as_float(pl[me][QQT_P_Y]), x = __int_as_float(pl[me][QQT_P_X]);
      const int mv = s.act_m[e][me];
      const int mc = min(max(mv, 0), 4);
      const float spd = __int_as_float(pl[me][QQT_P_SPD]);
      const float st = cf.step_len;
      float ty = 0.0f, tx = 0.0f;
      if (mc == 0) ty = -st; else if (mc == 1) ty = st; else if (mc == 2) tx = -st; else if (mc == 3) tx = st;
      float dy = ty * spd, dx = tx * spd;
      const bool moving = s.alive0[e][me] && mv != 4;
      if (!moving) { dy = 0.0f; dx = 0.0f; }
      const float ny = resolve_axis<H, W>(cw, y + dy, dy, x, y, x, rad, true);
      const float nx = resolve_axis<H, W>(cw, x + dx, dx, y, y, x, rad, false);
      float oy = dy != 0.0f ? ny : y;
      float ox = dx != 0.0f ? nx : x;
      oy = fminf(fmaxf(oy, rad), cf.pos_hi_y);
      ox = fminf(fmaxf(ox, rad), cf.pos_hi_x);
      pl[me][QQT_P_SINCE_BOMB] = sb;
      pl[me][QQT_P_Y] = __float_as_int(oy);
      pl[me][QQT_P_X] = __float_as_int(ox);
    }
    __syncthreads();

    // ---- 6. explosions (sim/blast.py:101-155), fixed synchronous rounds
    for (int c = l; c < C; c += LPE) {
      const uint32_t w = cw[c];
      const bool t0 = cw_fuse(w) == 0 && cw_owner(w) >= 0;
      s.trg[e][c] = t0;
      s.cov[e][c] = t0 && !(w & (F_WALL | F_BRICK));
    }
    __syncthreads();
    auto fire = [&](int src) {  // rays of one seed cell into cov
      const uint32_t w = cw[src];
      if (w & (F_WALL | F_BRICK)) return;
      const int b = blast_of(w, cf.blast);
      if (b > a.resolve_tiers) return;
      const int r0 = src / W, c0 = src % W;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int dr = d == 0 ? -1 : (d == 1 ? 1 : 0);
        const int dcol = d == 2 ? -1 : (d == 3 ? 1 : 0);
        for (int k = 1; k <= b; ++k) {
          const int rr = r0 + k * dr, cc = c0 + k * dcol;
          if (rr < 0 || rr >= H || cc < 0 || cc >= W) break;
          const int x = rr * W + cc;
          const uint32_t wx = cw[x];
          if (wx & F_WALL) break;
          s.cov[e][x] = 1;
          if ((wx & F_BRICK) || cw_fuse(wx) > 0) break;
        }
      }
    };
    for (int c = l; c < C; c += LPE)
      if (s.trg[e][c]) fire(c);
    const int rounds = min(cf.max_chain - 1, cf.chain_cap_rounds);
    for (int r = 0; r < rounds; ++r) {
      __syncthreads();
      uint32_t newly_bits = 0;  // bit k: cell l + 16k
      int kk = 0;
      for (int c = l; c < C; c += LPE, ++kk) {
        const bool nw = cw_fuse(cw[c]) > 0 && s.cov[e][c] && !s.trg[e][c];
        if (nw) newly_bits |= 1u << kk;
      }
      if (!__any(newly_bits != 0)) break;
      __syncthreads();
      kk = 0;
      for (int c = l; c < C; c += LPE, ++kk) {
        if (newly_bits & (1u << kk)) {
          s.trg[e][c] = 1;
          fire(c);
        }
      }
    }
    __syncthreads();

    // ---- 7. bricks burn (corridor: into crates); 8. damage (sim/torch_sim.py:1004-1040)
    for (int c = l; c < C; c += LPE) {
      if (s.cov[e][c]) {
        uint32_t w = cw[c];
        if (w & F_BRICK) {
          if (cf.corridor) w |= F_CRATE;
          w &= ~F_BRICK;
          cw[c] = w;
        }
      }
    }
    if (l < P) {
      const int me = l;
      const float y = __int_as_float(pl[me][QQT_P_Y]), x = __int_as_float(pl[me][QQT_P_X]);
      const int flat = min(max((int)floorf(y) * W + (int)floorf(x), 0), C - 1);
      s.fpost[e][me] = flat;
      const bool hit = s.alive0[e][me] && s.cov[e][flat];
      const bool hit_eff = hit && pl[me][QQT_P_INVULN] <= 0;
      const int hp_new = max(pl[me][QQT_P_HP] - (int)hit_eff, 0);
      const bool died = hit_eff && hp_new == 0;
      pl[me][QQT_P_HP] = hp_new;
      pl[me][QQT_P_ALIVE] = s.alive0[e][me] && !died;
      int inv = max(pl[me][QQT_P_INVULN] - 1, 0);
      if (hit_eff) inv = cf.invuln_ticks;
      pl[me][QQT_P_INVULN] = inv;
      if (valid && a.died) a.died[(size_t)g * P + me] = died;
    }
    __syncthreads();

    // ---- 9. clear exploded cells; info bitsets (bit c of the env's words)
    {
      constexpr int KMAX = (C + LPE - 1) / LPE;
      uint32_t myc = 0, myt = 0;
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        const bool tc = c < C && s.cov[e][c];
        const bool tt = c < C && s.trg[e][c];
        if (tt) cw[c] = cw_make(cw[c], 0, -1, 0);
        const uint32_t hc = (uint32_t)(__ballot(tc) >> (16 * e)) & 0xFFFFu;
        const uint32_t ht = (uint32_t)(__ballot(tt) >> (16 * e)) & 0xFFFFu;
        if ((k >> 1) == l) {
          myc |= hc << (16 * (k & 1));
          myt |= ht << (16 * (k & 1));
        }
      }
      if (valid && l < 8) {
        if (a.covered) a.covered[(size_t)g * 8 + l] = myc;
        if (a.triggered) a.triggered[(size_t)g * 8 + l] = myt;
      }
    }
    __syncthreads();
  }

  // ---- danger map of the current state (sim/blast.py:158-317)
  {
    constexpr int KMAX = (C + LPE - 1) / LPE;
    float wreg[KMAX];
    bool any_bomb = false;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = l + LPE * k;
      wreg[k] = 0.0f;
      if (c < C) {
        const int f = cw_fuse(cw[c]);
        const float w0 = bomb_weight(f, fmax_f);
        wreg[k] = w0;
        s.fw[e][c] = w0;
        any_bomb |= f > 0;
      }
    }
    auto gather = [&](int c, float v) {  // max over senders whose range reaches c
      const int r0 = c / W, c0 = c % W;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int dr = d == 0 ? -1 : (d == 1 ? 1 : 0);
        const int dcol = d == 2 ? -1 : (d == 3 ? 1 : 0);
        for (int k = 1; k <= G::MAXR; ++k) {
          const int rr = r0 - k * dr, cc = c0 - k * dcol;
          if (rr < 0 || rr >= H || cc < 0 || cc >= W) break;
          const int u = rr * W + cc;
          const uint32_t wu = cw[u];
          if (cw_fuse(wu) > 0) {
            if (blast_of(wu, cf.blast) >= k) v = fmaxf(v, s.fw[e][u]);
            break;
          }
          if (wu & (F_WALL | F_BRICK)) break;
        }
      }
      return v;
    };
    if (__any(any_bomb)) {
      // stage A: synchronous relay of weights between bombs (front in s.fw)
      if (cf.max_chain > 1) {
        const int rounds = min(cf.max_chain, cf.chain_cap_rounds);
        for (int r = 0; r < rounds; ++r) {
          __syncthreads();
          float nfront[KMAX];
          bool newly_any = false;
#pragma unroll
          for (int k = 0; k < KMAX; ++k) {
            const int c = l + LPE * k;
            nfront[k] = 0.0f;
            if (c < C) {
              const uint32_t wc = cw[c];
              if (cw_fuse(wc) > 0 && !(wc & F_WALL)) {
                const float spread = gather(c, 0.0f);
                if (spread > wreg[k]) {
                  wreg[k] = spread;
                  nfront[k] = spread;
                  newly_any = true;
                }
              }
            }
          }
          __syncthreads();
#pragma unroll
          for (int k = 0; k < KMAX; ++k) {
            const int c = l + LPE * k;
            if (c < C) s.fw[e][c] = nfront[k];
          }
          if (!__any(newly_any)) break;
        }
        __syncthreads();
      }
      // stage B: each bomb's corrected weight spreads along its cross
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        const int c = l + LPE * k;
        if (c < C) {
          const uint32_t wc = cw[c];
          s.fw[e][c] = (cw_fuse(wc) > 0 && !(wc & F_WALL)) ? wreg[k] : 0.0f;
        }
      }
      __syncthreads();
      for (int c = l; c < C; c += LPE) {
        const uint32_t wc = cw[c];
        s.dng[e][c] = (wc & F_WALL) ? 0.0f : gather(c, s.fw[e][c]);
      }
    } else {
      for (int c = l; c < C; c += LPE) s.dng[e][c] = 0.0f;
    }
    __syncthreads();
  }

  if (mode == QQT_MODE_STEP) {
    // ---- 10. time, rewards, growth, combo, terminal terms (lane 0 of each env)
    if (l == 0) {
      const float alpha = a.explore_coef;
      int t = s.ev[e][QQT_E_T] + 1;
      s.ev[e][QQT_E_T] = t;
      int n_alive = 0;
      for (int i = 0; i < P; ++i) n_alive += pl[i][QQT_P_ALIVE] != 0;
      const bool done = (n_alive <= 1) || (t >= cf.max_steps);
      float dmg[P], rw[P], a0[P];
      float dsum = 0.0f;
      for (int i = 0; i < P; ++i) {
        dmg[i] = (float)max(s.hp0[e][i] - pl[i][QQT_P_HP], 0);
        dsum = dsum + dmg[i];
        a0[i] = (float)(s.alive0[e][i] != 0);
      }
      for (int i = 0; i < P; ++i) {
        const float dealt = dsum - dmg[i];
        float r = (-cf.step_penalty) * a0[i];
        r = r + cf.hit_reward * dealt;
        r = r - cf.hit_reward * dmg[i];
        r = r + (alpha * s.pbonus[e][i]) * a0[i];
        rw[i] = r;
      }
      if (cf.hit_attr_penalty > 0) {
        const int pen = cf.hit_attr_penalty;
        for (int i = 0; i < P; ++i) {
          if (!(dmg[i] > 0.0f && s.alive0[e][i])) continue;
          const int bc = pl[i][QQT_P_BOMBS_CAP], zc = pl[i][QQT_P_BLAST_CAP];
          const float sp = __int_as_float(pl[i][QQT_P_SPD]);
          const int nb = max(bc - pen, pl[i][QQT_P_LO_BOMBS]);
          const int nz = max(zc - pen, pl[i][QQT_P_LO_BLAST]);
          const float ns = fmaxf(sp - cf.hit_speed_drop, __int_as_float(pl[i][QQT_P_LO_SPD]));
          const float lost_f = (float)((bc - nb) + (zc - nz)) +
                               rintf(__fdiv_rn(sp - ns, cf.growth_speed_step));
          pl[i][QQT_P_BOMBS_CAP] = nb;
          pl[i][QQT_P_BLAST_CAP] = nz;
          pl[i][QQT_P_SPD] = __float_as_int(ns);
          pl[i][QQT_P_PENDING_LOST] += (int)lost_f;
        }
      }
      for (int i = 0; i < P; ++i) rw[i] = rw[i] + (alpha * 0.0f) * a0[i];
      if (cf.corridor) {
        int hits[P], stood_v[P];
        float ug[P];
        for (int i = 0; i < P; ++i) {
          const uint32_t wc = cw[s.fpost[e][i]];
          const int stood = (wc & F_CRATE) != 0;
          stood_v[i] = stood;
          rw[i] = rw[i] + (cf.brick_reward * (float)stood) * a0[i];
          float uh, ugr;
          if (a.crate_u) {
            uh = a.crate_u[((size_t)i * 2 + 0) * a.n_envs + g];
            ugr = a.crate_u[((size_t)i * 2 + 1) * a.n_envs + g];
          } else {
            uh = philox_uniform(a.seed, (uint32_t)g, a.tick, STREAM_CRATE, 2 * i);
            ugr = philox_uniform(a.seed, (uint32_t)g, a.tick, STREAM_CRATE, 2 * i + 1);
          }
          const float prob = (wc & F_REC) ? cf.recycle_crate_prob
                                          : __int_as_float(s.ev[e][QQT_E_CRATE_PROB]);
          hits[i] = stood && (uh < prob) && s.alive0[e][i];
          ug[i] = ugr;
        }
        (void)stood_v;
        for (int i = 0; i < P; ++i) {
          const int h = hits[i] * (s.alive0[e][i] != 0);
          const int attr = (int)floorf(ug[i] * 3.0f);
          pl[i][QQT_P_BOMBS_CAP] = min(pl[i][QQT_P_BOMBS_CAP] + (attr == 0) * h, cf.growth_bombs_max);
          pl[i][QQT_P_BLAST_CAP] = min(pl[i][QQT_P_BLAST_CAP] + (attr == 1) * h, cf.growth_blast_max);
          const float sp = __int_as_float(pl[i][QQT_P_SPD]) + (float)((attr == 2) * h) * cf.growth_speed_step;
          pl[i][QQT_P_SPD] = __float_as_int(fminf(sp, cf.growth_speed_max));
        }
        for (int i = 0; i < P; ++i) {
          const int f = s.fpost[e][i];
          cw[f] &= ~(F_CRATE | F_REC);
        }
      }
      for (int i = 0; i < P; ++i) {
        const float standing = s.dng[e][s.fpost[e][i]];
        rw[i] = rw[i] - (a.danger_coef * standing) * a0[i];
      }
      if (cf.combo_reward > 0.0f) {
        for (int i = 0; i < P; ++i) {
          const float dealt = dsum - dmg[i];
          const int c = pl[i][QQT_P_COMBO];
          const int gap = t - pl[i][QQT_P_LAST_HIT];
          const float factor = powf(cf.combo_gap_factor, (float)max(gap, 0));
          const int inc = dealt > 0.0f;
          const int combo_now = (c + inc) * inc;
          const float pts = (((float)combo_now * cf.combo_reward) * factor) * fminf(dealt, 1.0f);
          rw[i] = rw[i] + pts * a0[i];
          int cn = inc ? combo_now : c;
          if (inc) pl[i][QQT_P_LAST_HIT] = t;
          if (dmg[i] > 0.0f) cn = 0;
          pl[i][QQT_P_COMBO] = cn;
        }
      }
      const bool death_done = done && n_alive == 1;
      const bool all_alive = done && n_alive == P;
      float hpf[P];
      float hsum = 0.0f;
      for (int i = 0; i < P; ++i) { hpf[i] = (float)pl[i][QQT_P_HP]; hsum = hsum + hpf[i]; }
      int win[P], lose[P];
      for (int i = 0; i < P; ++i) {
        const bool al = pl[i][QQT_P_ALIVE] != 0;
        win[i] = death_done && al;
        lose[i] = death_done && !al;
      }
      float tscale = alpha;
      if (!cf.timeout_draw) {
        for (int i = 0; i < P; ++i) {
          bool gt = true, lt = false;
          for (int o = 0; o < P; ++o) {
            if (o == i) continue;
            gt = gt && (hpf[i] > hpf[o]);
            lt = lt || (hpf[i] < hpf[o]);
          }
          win[i] |= all_alive && gt;
          lose[i] |= all_alive && lt;
        }
        tscale = 1.0f;
      }
      for (int i = 0; i < P; ++i) {
        const float diff = hpf[i] - __fdiv_rn(hsum - hpf[i], (float)(P - 1));
        if (cf.win_hp_scaled) {
          const float base = cf.win_per_hp * diff;
          rw[i] = rw[i] + (base * (float)death_done + (base * (float)all_alive) * tscale);
        } else {
          rw[i] = rw[i] + cf.win_bonus * ((float)win[i] - (float)lose[i]);
          if (cf.timeout_draw)
            rw[i] = rw[i] + ((cf.win_per_hp * diff) * (float)all_alive) * tscale;
        }
      }
      if (valid) {
        for (int i = 0; i < P; ++i) {
          if (a.reward) a.reward[(size_t)g * P + i] = rw[i];
          if (a.winner) a.winner[(size_t)g * P + i] = win[i];
        }
        if (a.done) a.done[g] = done;
        if (a.n_alive) a.n_alive[g] = n_alive;
      }
      s.done[e] = done && a.auto_reset;
    }
    __syncthreads();
    do_reset = s.done[e] != 0;
  } else if (mode == QQT_MODE_RESET) {
    do_reset = valid && a.reset_mask[g] != 0;
  }

  // ---- template reset (qqtsim/maps.py; re-init values of sim/torch_sim.py:178-420)
  if (do_reset) {
    const uint32_t env_id = (uint32_t)g;
    for (int c = l; c < C; c += LPE) {
      const int r = c / W, col = c % W;
      bool wall = false;
      if (cf.map_kind == 0)
        wall = r == 0 || r == H - 1 || col == 0 || col == W - 1 || ((r % 2 == 0) && (col % 2 == 0));
      bool keep = false;
      for (int i = 0; i < P; ++i) {
        const int sr = (i == 0 || i == 2) ? 1 : H - 2;
        const int sc = (i == 0 || i == 3) ? 1 : W - 2;
        const int dr = sr < H / 2 ? 1 : -1, dcol = sc < W / 2 ? 1 : -1;
        keep |= (r == sr && col == sc) || (r == sr && col == sc + dcol) || (r == sr + dr && col == sc);
      }
      bool brick = false;
      if (!wall && !keep && cf.brick_p > 0.0f)
        brick = philox_uniform(a.seed, env_id, a.epoch, STREAM_RESET_CELL, (uint32_t)c) < cf.brick_p;
      cw[c] = (wall ? F_WALL : 0u) | (brick ? F_BRICK : 0u) | 0x0000FF00u;
      s.dng[e][c] = 0.0f;
    }
    if (l == 0) {
      float u[12];
      philox_block(a.seed, env_id, a.epoch, STREAM_RESET_MISC, 0, u);
      philox_block(a.seed, env_id, a.epoch, STREAM_RESET_MISC, 1, u + 4);
      philox_block(a.seed, env_id, a.epoch, STREAM_RESET_MISC, 2, u + 8);
      float py[P], px[P];
      for (int i = 0; i < P; ++i) {
        const int sr = (i == 0 || i == 2) ? 1 : H - 2;
        const int sc = (i == 0 || i == 3) ? 1 : W - 2;
        py[i] = (float)sr + 0.5f;
        px[i] = (float)sc + 0.5f;
      }
      if (cf.swap_spawns && u[0] < 0.5f) {
        float ty = py[0], tx = px[0];
        py[0] = py[1]; px[0] = px[1]; py[1] = ty; px[1] = tx;
      }
      for (int i = 0; i < P; ++i) {
        const int bspan = cf.bombs_hi - cf.bombs_lo + 1, zspan = cf.blast_hi - cf.blast_lo + 1;
        const float ub = u[1 + 2 * i];
        const float uz = u[2 + 2 * i];
        const int bc = cf.bombs_lo + min((int)floorf(ub * (float)bspan), bspan - 1);
        const int zc = cf.blast_lo + min((int)floorf(uz * (float)zspan), zspan - 1);
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
  }
  __syncthreads();

  // ---- observation + legality masks of the current state (sim/obs.py:25-229)
  {
    int cnt[P];
#pragma unroll
    for (int i = 0; i < P; ++i) cnt[i] = 0;
    for (int c = l; c < C; c += LPE) {
      const uint32_t w = cw[c];
      if (cw_fuse(w) > 0) {
        const int o = cw_owner(w);
#pragma unroll
        for (int i = 0; i < P; ++i) cnt[i] += (o == i);
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int t = sum16(cnt[i]);
      if (l == 0) s.live[e][i] = t;
    }
    if (l < P) {
      const int i = l;
      const float py = __int_as_float(pl[i][QQT_P_Y]), px = __int_as_float(pl[i][QQT_P_X]);
      const float gate = (float)(pl[i][QQT_P_ALIVE] != 0);
      const float fy = fminf(fmaxf(py - 0.5f, 0.0f), (float)(H - 1));
      const float fx = fminf(fmaxf(px - 0.5f, 0.0f), (float)(W - 1));
      const int y0 = min(max((int)floorf(fy), 0), H - 1);
      const int x0 = min(max((int)floorf(fx), 0), W - 1);
      const int y1 = min(y0 + 1, H - 1), x1 = min(x0 + 1, W - 1);
      const float wy = fminf(fmaxf(fy - (float)y0, 0.0f), 1.0f);
      const float wx = fminf(fmaxf(fx - (float)x0, 0.0f), 1.0f);
      const float ky0 = 1.0f - wy, kx0 = 1.0f - wx;
      s.splat_i[e][i][0] = y0 * W + x0; s.splat_w[e][i][0] = (ky0 * kx0) * gate;
      s.splat_i[e][i][1] = y0 * W + x1; s.splat_w[e][i][1] = (ky0 * wx) * gate;
      s.splat_i[e][i][2] = y1 * W + x0; s.splat_w[e][i][2] = (wy * kx0) * gate;
      s.splat_i[e][i][3] = y1 * W + x1; s.splat_w[e][i][3] = (wy * wx) * gate;
      s.fpost[e][i] = min(max((int)floorf(py) * W + (int)floorf(px), 0), C - 1);
    }
    __syncthreads();

    uint16_t* ob = s.obs[e];
    const float tplane = __fdiv_rn((float)s.ev[e][QQT_E_T], (float)cf.max_steps);
    for (int c = l; c < C; c += LPE) {
      const uint32_t w = cw[c];
      const int f = cw_fuse(w), o = cw_owner(w);
      const float fnorm = __fdiv_rn((float)f, fmax_f);
#pragma unroll
      for (int i = 0; i < P; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (s.splat_i[e][i][k] == c) v = v + s.splat_w[e][i][k];
        ob[i * C + c] = __half_as_ushort(__float2half_rn(v));
        ob[(P + i) * C + c] = __half_as_ushort(__float2half_rn((o == i && f > 0) ? fnorm : 0.0f));
      }
      ob[(2 * P) * C + c] = __half_as_ushort(__float2half_rn((w & (F_WALL | F_BRICK)) ? 1.0f : 0.0f));
      ob[(2 * P + 1) * C + c] = __half_as_ushort(__float2half_rn(s.dng[e][c]));
      ob[(2 * P + 2) * C + c] = __half_as_ushort(__float2half_rn(tplane));
      ob[(2 * P + 3) * C + c] = __half_as_ushort(__float2half_rn((w & F_CRATE) ? 1.0f : 0.0f));
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const bool here = s.fpost[e][i] == c;
        const bool al = pl[i][QQT_P_ALIVE] != 0;
        const int capi = pl[i][QQT_P_BOMBS_CAP];
        const float cap = fmaxf((float)capi, 1.0f);
        const float avail = fmaxf((float)(capi - s.live[e][i]), 0.0f);
        const float af = (float)al;
        const float inv = (pl[i][QQT_P_INVULN] > 0 && al) ? 1.0f : 0.0f;
        ob[(2 * P + 4 + i) * C + c] = __half_as_ushort(__float2half_rn(here ? inv : 0.0f));
        ob[(3 * P + 4 + i) * C + c] =
            __half_as_ushort(__float2half_rn(here ? __fdiv_rn(avail, cap) * af : 0.0f));
        ob[(4 * P + 4 + i) * C + c] = __half_as_ushort(
            __float2half_rn(here ? __fdiv_rn(cap, (float)cf.growth_bombs_max) * af : 0.0f));
      }
    }

    // masks: lane = me*4 + probe (up, down, left, right)
    const int me = l >> 2, pr = l & 3;
    if (me < P && valid) {
      const float y = __int_as_float(pl[me][QQT_P_Y]), x = __int_as_float(pl[me][QQT_P_X]);
      const bool al = pl[me][QQT_P_ALIVE] != 0;
      const float st = cf.step_len;
      const float d = (pr & 1) ? st : -st;
      bool moved;
      if (pr < 2) {
        const float ny = resolve_axis<H, W>(cw, y + d, d, x, y, x, rad, true);
        moved = fabsf(ny - y) > 2e-4f;
      } else {
        const float nx = resolve_axis<H, W>(cw, x + d, d, y, y, x, rad, false);
        moved = fabsf(nx - x) > 2e-4f;
      }
      if (a.move_mask) {
        a.move_mask[((size_t)g * P + me) * 5 + pr] = al ? moved : 1;
        if (pr == 0) a.move_mask[((size_t)g * P + me) * 5 + 4] = 1;
      }
      if (pr == 0 && a.bomb_mask) {
        const int cy = (int)floorf(y), cx = (int)floorf(x);
        const int flat = min(max(cy * W + cx, 0), C - 1);
        const uint32_t wc = cw[flat];
        const bool under = cw_fuse(wc) > 0;
        const bool blk = under || (wc & F_BRICK);
        const bool can = !under && !blk && s.live[e][me] < pl[me][QQT_P_BOMBS_CAP];
        a.bomb_mask[((size_t)g * P + me) * 2 + 0] = 1;
        a.bomb_mask[((size_t)g * P + me) * 2 + 1] = (can && al) || !al;
      }
    }
  }
  __syncthreads();

  // ---- store state and the staged observation
  if (mode == QQT_MODE_STEP || mode == QQT_MODE_RESET) {
    if (valid) {
      for (int c = l; c < C; c += LPE) a.cells[(size_t)g * C + c] = (int32_t)cw[c];
      for (int i = l; i < P * QQT_P_SLOTS; i += LPE)
        a.players[(size_t)g * P * QQT_P_SLOTS + i] = pl[i / QQT_P_SLOTS][i % QQT_P_SLOTS];
      if (l < QQT_E_SLOTS) a.envs[(size_t)g * QQT_E_SLOTS + l] = s.ev[e][l];
    }
  }
  if (a.obs) {
    const int g0 = blockIdx.x * EPW;
    const int nvalid = min(EPW, a.n_envs - g0);
    const size_t bytes = (size_t)nvalid * OBS * 2;
    uint8_t* dst = (uint8_t*)(a.obs + (size_t)g0 * OBS);
    const uint8_t* src = (const uint8_t*)&s.obs[0][0];
    if constexpr ((EPW * OBS * 2) % 16 == 0) {
      const size_t n16 = bytes / 16;
      for (size_t i = lane; i < n16; i += 64)
        reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
      for (size_t i = n16 * 16 + lane * 2; i < bytes; i += 128)
        *reinterpret_cast<uint16_t*>(dst + i) = *reinterpret_cast<const uint16_t*>(src + i);
    } else {
      for (size_t i = lane * 2; i < bytes; i += 128)
        *reinterpret_cast<uint16_t*>(dst + i) = *reinterpret_cast<const uint16_t*>(src + i);
    }
  }
}

// ---------------------------------------------------------------- host side
thread_local char g_err[512] = "";

int fail(int code, const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

template <int H, int W, int P>
int launch(const qqt_sim_config* cfg, const qqt_tick_args* a, hipStream_t st) {
  const int blocks = (a->n_envs + EPW - 1) / EPW;
  DevCfg dc;
  dc.c = *cfg;
  hipLaunchKernelGGL((tick_kernel<H, W, P>), dim3(blocks), dim3(64), 0, st, dc, *a);
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
  if (a->mode < QQT_MODE_STEP || a->mode > QQT_MODE_PROBE) return fail(QQT_E_ARG, "bad mode");
  if (a->mode == QQT_MODE_STEP && !a->actions && !a->actions_i8)
    return fail(QQT_E_ARG, "STEP needs actions");
  if (a->mode == QQT_MODE_RESET && !a->reset_mask) return fail(QQT_E_ARG, "RESET needs reset_mask");
  if (a->mode == QQT_MODE_PROBE && !a->probe_out) return fail(QQT_E_ARG, "PROBE needs probe_out");
  if (a->obs && (((uintptr_t)a->obs) & 15)) return fail(QQT_E_ARG, "obs must be 16-byte aligned");
  if (cfg->fuse < 1 || cfg->fuse > 255) return fail(QQT_E_ARG, "fuse must be in 1..255");
  if (cfg->bombs_lo > cfg->bombs_hi || cfg->blast_lo > cfg->blast_hi)
    return fail(QQT_E_ARG, "bad cap ranges");
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
