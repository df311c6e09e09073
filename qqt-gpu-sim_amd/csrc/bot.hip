// The astar rule bot for gfx950 (sim/bots.py:179-238, :267-508): two
// danger-weighted multi-source shortest-cost fields and steepest descent on
// them, for one player of a batch of envs, in one launch.
//
// Mapping: one 64-lane wavefront per env, two independent wavefronts per
// workgroup (a CU holds more waves than workgroups).  The env's obstacles,
// danger and threat maps and both cost fields live in LDS (~3.5 KB); lane l
// owns cells l, l + 64, l + 128.  Every global load (cells, danger, players,
// masks, noise) is issued at the start.
//
// Cost fields: dist = min(dist, min_4nbr(dist) + cost), cost = 1 + 2 danger
// (inf on blocked cells), sources at 0 even when blocked, relaxed in place
// until a full pass changes nothing (wavefront ballot).  float32 addition is
// monotone, so the in-place order reaches the same fixed point as the
// reference's synchronous passes, bit for bit.
//
// Decision: lane 0 scores the five candidate cells (4 moves + idle) exactly as
// the reference does (approach on V_opp, escape on V_safe, danger and threat
// penalties, 0.05-scaled noise, fallback to the least dangerous legal move);
// the chain check (a short-fuse bomb within `reach` cells in line) runs one
// (distance, direction) pair per lane.  The library is built with
// -ffp-contract=off, so every product and sum rounds separately like the
// reference's float32 tensor ops.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

namespace bot {

constexpr uint32_t F_WALL = 1u << 24, F_BRICK = 1u << 25;
__device__ __forceinline__ int fuse_of(uint32_t w) { return (int)(w & 0xFFu); }
__device__ __forceinline__ int owner_of(uint32_t w) { return (int)(int8_t)((w >> 8) & 0xFFu); }

template <int H, int W, int P>
struct BotLds {
  static constexpr int C = H * W;
  float dng[C];       // danger (the observation's float16 channel, widened)
  float vs[C];        // V_safe
  float vo[C];        // V_opp
  uint32_t cw[C];     // packed cell words
  uint8_t thr[C];     // threat map
  int32_t pl[P * QQT_P_SLOTS];  // player slots of the env
  float u[8];         // noise uniforms
  uint8_t mm[5], bm[2];         // the bot's legality masks
};

}  // namespace bot

template <int H, int W, int P, int WPB>
__global__ __launch_bounds__(64 * WPB) void bot_kernel(const qqt_sim_config cf, const qqt_bot_args a) {
  constexpr int C = H * W;
  constexpr int KMAX = (C + 63) / 64;
  constexpr int NPL = P * QQT_P_SLOTS;
  static_assert(NPL <= 64, "player slots must fit one wavefront");
  __shared__ bot::BotLds<H, W, P> sh[WPB];
  // the waves of a workgroup share nothing: each owns one env and its LDS.
  // XCD_ROWS-env row blocks are dealt to the XCDs as in the tick and act
  // kernels (block b: row block (b / 8 / WGRB) * 8 + b % 8), so the env's
  // state, observation and masks are read from the L2 that the tick wrote
  // them to.
  constexpr int WGRB = XCD_ROWS / WPB;              // workgroups per row block
  static_assert(WGRB * WPB == XCD_ROWS, "whole workgroups per row block");
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int seq = blockIdx.x >> 3;
  const int g = ((seq / WGRB) * 8 + (blockIdx.x & 7)) * XCD_ROWS + (seq % WGRB) * WPB + wv;
  if (g >= a.n_envs) return;
  bot::BotLds<H, W, P>& s = sh[wv];
  const int lane = threadIdx.x & 63;
  const int pid = a.pid;
  const float INF = __builtin_inff();
  const uint16_t* obs = a.obs + (size_t)g * (5 * P + 4) * C + (size_t)(2 * P + 1) * C;

  // ---- every global load is issued first; the Philox noise is computed
  // (lane 0: words 0-3, lane 1: words 4-7) while they are in flight
  // Every lane loads from a clamped in-bounds index and every use is guarded
  // by the lane's range: a select on a loaded value would make the kernel
  // wait for that load before issuing the rest.
  uint32_t wreg[KMAX];
  uint16_t dreg[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = min(lane + 64 * k, C - 1);
    wreg[k] = (uint32_t)a.cells[(size_t)g * C + c];
    dreg[k] = obs[c];
  }
  const int plv = a.players[(size_t)g * NPL + min(lane, NPL - 1)];
  const int mv = a.move_mask[((size_t)g * P + pid) * 5 + min(lane, 4)];
  const int bv = a.bomb_mask[((size_t)g * P + pid) * 2 + min(lane, 1)];
  // (loads are unconditional, so that the compiler counts them exactly: a
  // source that is not in use is read from a buffer that is, and ignored)
  const float* const usrc = a.uniforms ? a.uniforms + (size_t)g * 5
                                       : reinterpret_cast<const float*>(a.players);
  const float uv = usrc[min(lane, 4)];
  int reach_in = a.reach_mode == 1 ? a.reach[a.reach_slot & 1]
                 : a.reach_mode == 2 ? a.reach[0] : 0;
  // reach mode 3: the cap maxima the last STEP tick wrote (one per tick
  // wavefront), 16 per lane load; the first 4096 are loaded here with
  // everything else and reduced where the chain check needs them, so their
  // latency overlaps the cost fields
  const bool caps = a.reach_mode == 3;
  const uint4* const c16 = reinterpret_cast<const uint4*>(caps ? (const void*)a.reach_caps
                                                               : (const void*)a.cells);
  const int epw = tick_envs_per_wave(a.n_envs);
  const int n16 = caps ? ((a.n_envs + epw - 1) / epw + 15) >> 4 : 1;
  constexpr int CAPL = 4;   // loads per lane up front
  uint4 capv[CAPL];   // lanes past the maxima re-read the last unit (the max is unchanged)
#pragma unroll
  for (int j = 0; j < CAPL; ++j) capv[j] = c16[min(lane + 64 * j, n16 - 1)];
  if (!a.uniforms && lane < 2) {
    float ub[4];
    philox_block(a.seed, (uint32_t)g, a.tick, STREAM_BOT, (uint32_t)lane, ub);
#pragma unroll
    for (int q = 0; q < 4; ++q) s.u[lane * 4 + q] = ub[q];
  }
  if (a.uniforms && lane < 5) s.u[lane] = uv;
  if (lane < NPL) s.pl[lane] = plv;
  if (lane < 5) s.mm[lane] = (uint8_t)mv;
  if (lane < 2) s.bm[lane] = (uint8_t)bv;

  // ---- cells, danger, cost, V_safe sources
  float cst[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = lane + 64 * k;
    cst[k] = INF;
    if (c < C) {
      const uint32_t w = wreg[k];
      s.cw[c] = w;
      const float d = __half2float(__ushort_as_half(dreg[k]));
      s.dng[c] = d;
      const bool blocked = (w & (bot::F_WALL | bot::F_BRICK)) || bot::fuse_of(w) > 0;
      cst[k] = blocked ? INF : 1.0f + 2.0f * d;
      s.vs[c] = d < 0.35f ? 0.0f : INF;
      s.vo[c] = INF;
    }
  }

  // ---- threat: the bot's live bombs dilated growth_blast_max times with the
  // 4-neighbourhood, clipped at the border.  On a rectangle that is the set
  // of cells within L1 distance growth_blast_max of such a bomb (a monotone
  // path never leaves the bounding box), tested bomb by bomb.
  {
    const int gr = cf.growth_blast_max;
    bool thr[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) thr[k] = false;
#pragma unroll
    for (int kb = 0; kb < KMAX; ++kb) {
      const int cb = lane + 64 * kb;
      const uint32_t wb = wreg[kb];
      uint64_t m = __ballot(cb < C && bot::owner_of(wb) == pid && bot::fuse_of(wb) > 0);
      while (m) {
        const int b = 64 * kb + __builtin_ctzll(m);
        m &= m - 1;
        const int rb = b / W, colb = b % W;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
          const int c = lane + 64 * k;
          const int r = c / W, col = c % W;
          thr[k] |= abs(r - rb) + abs(col - colb) <= gr;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int c = lane + 64 * k;
      if (c < C) s.thr[c] = thr[k] ? 1 : 0;
    }
  }
  wave_sync();

  // opponents' cells: a later opponent overwrites an earlier one's flag
  // (the reference assigns alive[o] per opponent in id order)
  if (lane == 0) {
    for (int o = 0; o < P; ++o) {
      if (o == pid) continue;
      const float oy = __int_as_float(s.pl[o * QQT_P_SLOTS + QQT_P_Y]);
      const float ox = __int_as_float(s.pl[o * QQT_P_SLOTS + QQT_P_X]);
      const int ro = min(max((int)floorf(oy), 0), H - 1);
      const int co = min(max((int)floorf(ox), 0), W - 1);
      s.vo[ro * W + co] = s.pl[o * QQT_P_SLOTS + QQT_P_ALIVE] ? 0.0f : INF;
    }
  }
  wave_sync();

  // ---- both cost fields, relaxed in place to their fixed point; each lane
  // keeps its own cells' values in registers (only it writes them)
  float vsr[KMAX], vor[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int c = lane + 64 * k;
    vsr[k] = c < C ? s.vs[c] : INF;
    vor[k] = c < C ? s.vo[c] : INF;
  }
  // A cell can only improve when a neighbour changed since it was last
  // relaxed, so a pass relaxes the cells next to a change of the previous
  // pass or of an earlier slice of this one (every cell in the first pass).
  // Change sets are one 64-cell ballot per slice, shifted by 1 and W to find
  // the neighbours; a superset (row wrap-around) only costs work.
  uint64_t prev[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) prev[k] = ~0ull;
  // bit i: a neighbour (c - 1, c + 1, c - W, c + W) of cell c = 64k + i is in x
  auto near = [](const uint64_t (&x)[KMAX], int k) -> uint64_t {
    const uint64_t w = x[k], lo = k > 0 ? x[k - 1] : 0ull, hi = k + 1 < KMAX ? x[k + 1] : 0ull;
    return ((w << 1) | (lo >> 63)) | ((w >> 1) | (hi << 63)) |
           ((w << W) | (lo >> (64 - W))) | ((w >> W) | (hi << (64 - W)));
  };
  for (int pass = 0; pass < 4 * C; ++pass) {
    uint64_t seen[KMAX];   // the previous pass's changes, then this pass's of earlier slices
#pragma unroll
    for (int k = 0; k < KMAX; ++k) seen[k] = prev[k];
    bool any = false;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const uint64_t act = near(seen, k);
      const int c = lane + 64 * k;
      const float cc = cst[k];
      bool changed = false;
      if (((act >> lane) & 1ull) && c < C && cc != INF) {
        const int r = c / W, col = c % W;
        float ns = INF, no = INF;
        if (r > 0) { ns = fminf(ns, s.vs[c - W]); no = fminf(no, s.vo[c - W]); }
        if (r < H - 1) { ns = fminf(ns, s.vs[c + W]); no = fminf(no, s.vo[c + W]); }
        if (col > 0) { ns = fminf(ns, s.vs[c - 1]); no = fminf(no, s.vo[c - 1]); }
        if (col < W - 1) { ns = fminf(ns, s.vs[c + 1]); no = fminf(no, s.vo[c + 1]); }
        const float cs = ns + cc, co = no + cc;
        if (cs < vsr[k]) { vsr[k] = cs; s.vs[c] = cs; changed = true; }
        if (co < vor[k]) { vor[k] = co; s.vo[c] = co; changed = true; }
      }
      const uint64_t ch = __ballot(changed);
      prev[k] = ch;
      seen[k] |= ch;
      any |= ch != 0ull;
    }
    if (!any) break;
    wave_sync();
  }
  wave_sync();

  // ---- decision
  const int32_t* pl = s.pl;
  const float by = __int_as_float(pl[pid * QQT_P_SLOTS + QQT_P_Y]);
  const float bx = __int_as_float(pl[pid * QQT_P_SLOTS + QQT_P_X]);
  const int r = min(max((int)floorf(by), 0), H - 1);
  const int c = min(max((int)floorf(bx), 0), W - 1);
  const bool alive = pl[pid * QQT_P_SLOTS + QQT_P_ALIVE] != 0;
  const int cap = pl[pid * QQT_P_SLOTS + QQT_P_BLAST_CAP];
  if (a.reach_mode == 3) {   // the batch max of the caps (each in 0..127)
    auto bmax = [](uint32_t m, const uint4& v) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        m = max(m, max(max(w[q] & 0xffu, (w[q] >> 8) & 0xffu), max((w[q] >> 16) & 0xffu, w[q] >> 24)));
      return m;
    };
    uint32_t m = 0u;
#pragma unroll
    for (int j = 0; j < CAPL; ++j) m = bmax(m, capv[j]);
    for (int i = 64 * CAPL + lane; i < n16; i += 64) m = bmax(m, c16[i]);   // larger batches
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, sh, 64));
    reach_in = (int)m;
  }
  const int reach = a.reach_mode != 0 ? reach_in : cap;

  // chain: a bomb with fuse 1..10 within `reach` cells in line (lane = step, direction)
  bool chain_l = false;
  for (int i = lane; i < 4 * reach; i += 64) {
    const int k = i / 4 + 1, d = i % 4;
    const int rr = r + (d == 0 ? -k : d == 1 ? k : 0);
    const int cc2 = c + (d == 2 ? -k : d == 3 ? k : 0);
    if (rr >= 0 && rr < H && cc2 >= 0 && cc2 < W) {
      const int f = bot::fuse_of(s.cw[rr * W + cc2]);
      chain_l |= f > 0 && f <= 10;
    }
  }
  const bool chain = __ballot(chain_l) != 0ull;

  // the five candidate moves (up, down, left, right, stay), one per lane
  // 0-4, then read by lane 0 (the scoring below is one lane's work)
  const int kk = min(lane, 4);
  const int ck = kk == 0 ? max(r - 1, 0) * W + c : kk == 1 ? min(r + 1, H - 1) * W + c
               : kk == 2 ? r * W + max(c - 1, 0) : kk == 3 ? r * W + min(c + 1, W - 1) : r * W + c;
  const uint32_t wk = s.cw[ck];
  const bool legal_k = s.mm[kk] != 0 && !(wk & (bot::F_WALL | bot::F_BRICK));
  const bool thr_k = s.thr[ck] != 0;
  const float thf_k = thr_k ? 1.0f : 0.0f;
  const float noise_k = 0.05f * s.u[kk];
  const float dng_k = s.dng[ck];
  float ap_k = ((s.vo[ck] + 2.0f * dng_k) + 2.0f * thf_k) + noise_k;
  // flee (mode 1): away from the opponent, V_opp clamped at 1e3
  float fl_k = ((-fminf(s.vo[ck], 1e3f) + 2.0f * dng_k) + 2.0f * thf_k) + noise_k;
  if (dng_k >= 0.5f || !legal_k) ap_k = fl_k = INF;
  const float esc_k = ((s.vs[ck] * 100.0f) + 2.0f * thf_k) + noise_k;
  const int flags_k = (legal_k ? 1 : 0) | (thr_k ? 2 : 0);
  float app[5], esc[5], dngc[5], flee[5];
  bool legal[5], thr[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    app[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ap_k), k));
    esc[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(esc_k), k));
    dngc[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dng_k), k));
    flee[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fl_k), k));
    const int f = __builtin_amdgcn_readlane(flags_k, k);
    legal[k] = (f & 1) != 0;
    thr[k] = (f & 2) != 0;
  }

  if (lane == 0) {
    // behaviour mode of this env, after this call's ticker step
    int md = 0;
    if (a.mode) {
      md = a.mode[g];
      if (a.mode_tick != 0u) {
        int tmr = a.mode_timer[g] - 1;
        if ((a.mode_tick & 15u) == 0u && tmr <= 0) {
          float u4[4];
          philox_block(a.seed, (uint32_t)g, a.mode_tick, STREAM_BOT_MODE, 0u, u4);
          md = u4[0] >= 0.5f ? 1 : 0;
          tmr = 60 + min((int)(u4[1] * 180.0f), 179);
          a.mode[g] = (int8_t)md;
        }
        a.mode_timer[g] = tmr;
      }
    }
    const uint8_t* bm = s.bm;
    const float own_dng = s.dng[r * W + c];
    bool app_ok = false;
#pragma unroll
    for (int k = 0; k < 5; ++k) app_ok |= app[k] != INF;
    const bool use_esc = own_dng >= 0.35f || !app_ok;
    float score[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      float e = esc[k];
      if ((use_esc && k == 4) || !legal[k]) e = INF;
      score[k] = use_esc ? e : md == 1 ? flee[k] : app[k];
    }
    // argmin with the first index winning ties (all-inf -> 0)
    int move = 0;
    bool finite = score[0] != INF;
#pragma unroll
    for (int k = 1; k < 5; ++k) {
      if (score[k] < score[move]) move = k;
      finite |= score[k] != INF;
    }
    bool any_legal = false;
#pragma unroll
    for (int k = 0; k < 5; ++k) any_legal |= legal[k];
    if (!finite && any_legal) {
      float dl[5];
#pragma unroll
      for (int k = 0; k < 5; ++k) dl[k] = legal[k] ? dngc[k] : INF;
      int fm = 0, fi = 0;
#pragma unroll
      for (int k = 1; k < 4; ++k)
        if (dl[k] < dl[fm]) fm = k;
#pragma unroll
      for (int k = 1; k < 5; ++k)
        if (dl[k] < dl[fi]) fi = k;
      move = dl[fm] != INF ? fm : fi;
    }

    // placement
    long long dr_o = 1000000000LL, dc_o = 1000000000LL;
    for (int o = 0; o < P; ++o) {
      if (o == pid || !pl[o * QQT_P_SLOTS + QQT_P_ALIVE]) continue;
      const float oy = __int_as_float(pl[o * QQT_P_SLOTS + QQT_P_Y]);
      const float ox = __int_as_float(pl[o * QQT_P_SLOTS + QQT_P_X]);
      const int ro = min(max((int)floorf(oy), 0), H - 1);
      const int co = min(max((int)floorf(ox), 0), W - 1);
      dr_o = r > ro ? r - ro : ro - r;
      dc_o = c > co ? c - co : co - c;
    }
    const bool aligned = (dr_o == 0 && dc_o <= cap) || (dc_o == 0 && dr_o <= cap);
    const long long manh = min(dr_o + dc_o, 100000000LL);
    const bool near = manh <= (long long)max(cap + 1, 1);
    bool can_escape = false;
#pragma unroll
    for (int k = 0; k < 5; ++k) can_escape |= legal[k] && dngc[k] < 0.35f && !thr[k];
    // a fleeing bot places only on an opponent in reach, never for a chain
    int place = (bm[1] != 0 && (aligned || near || (chain && md != 1)) && own_dng < 0.2f &&
                 can_escape) ? 1 : 0;
    if (!alive) {
      move = 4;
      place = 0;
    }
    const size_t o = ((size_t)g * P + pid) * 2;
    if (a.actions) {
      a.actions[o] = move;
      a.actions[o + 1] = place;
    }
    if (a.actions_i8) {
      a.actions_i8[o] = (int8_t)move;
      a.actions_i8[o + 1] = (int8_t)place;
    }
  }
}

// Batch max of the bot's blast cap (the chain-check reach of the reference,
// `int(cap.max().item())`): one env per thread, a workgroup max, then one
// atomic max per workgroup into out[slot].  Workgroup 0 also resets the
// other slot, which the next call reduces into; the bot kernel that follows
// in stream order reads out[slot].
constexpr int REACH_THREADS = 256;
__global__ __launch_bounds__(REACH_THREADS) void reach_kernel(const int32_t* players, int n, int p,
                                                              int pid, int32_t* out, int slot) {
  __shared__ int part[REACH_THREADS / 64];
  const int g = blockIdx.x * REACH_THREADS + (int)threadIdx.x;
  int v = g < n ? players[((size_t)g * p + pid) * QQT_P_SLOTS + QQT_P_BLAST_CAP] : INT_MIN;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    int r = part[0];
#pragma unroll
    for (int i = 1; i < REACH_THREADS / 64; ++i) r = max(r, part[i]);
    atomicMax(&out[slot & 1], r);
    if (blockIdx.x == 0) out[(slot & 1) ^ 1] = INT_MIN;
  }
}

extern thread_local char g_err[512];

template <int H, int W, int P>
static int launch_bot(const qqt_sim_config* cfg, const qqt_bot_args* a, hipStream_t st) {
  if (a->reach_mode == 1)
    QQT_LAUNCH(QQT_KERNEL_REACH, reach_kernel, dim3((a->n_envs + REACH_THREADS - 1) / REACH_THREADS),
               dim3(REACH_THREADS), st, a->players, a->n_envs, P, a->pid, a->reach, a->reach_slot);
  constexpr int WPB = 2;  // two independent waves per workgroup (workgroup slots per CU)
  const int nrb = (a->n_envs + XCD_ROWS - 1) / XCD_ROWS;   // row blocks, a multiple of 8 of them
  QQT_LAUNCH(QQT_KERNEL_BOT, (bot_kernel<H, W, P, WPB>), dim3(((nrb + 7) / 8) * 8 * (XCD_ROWS / WPB)),
             dim3(64 * WPB), st, *cfg, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "bot launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // namespace qqt

extern "C" {

int qqt_bot_act(const qqt_sim_config* cfg, const qqt_bot_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!cfg || !a) {
    snprintf(g_err, sizeof(g_err), "qqt_bot_act: null config or args");
    return QQT_E_ARG;
  }
  if (a->n_envs <= 0 || !a->cells || !a->players || !a->obs || !a->move_mask ||
      !a->bomb_mask || (!a->actions && !a->actions_i8)) {
    snprintf(g_err, sizeof(g_err), "qqt_bot_act: null pointer or empty batch");
    return QQT_E_ARG;
  }
  if (a->reach_mode < 0 || a->reach_mode > 3 || ((a->reach_mode == 1 || a->reach_mode == 2) && !a->reach) ||
      (a->reach_mode == 3 && (!a->reach_caps || (((uintptr_t)a->reach_caps) & 15)))) {
    snprintf(g_err, sizeof(g_err), "qqt_bot_act: reach_mode 1/2 needs a reach buffer, 3 aligned reach_caps");
    return QQT_E_ARG;
  }
  if (a->pid < 0 || a->pid >= cfg->n_players || cfg->growth_blast_max < 0 ||
      cfg->growth_blast_max > 64) {
    snprintf(g_err, sizeof(g_err), "qqt_bot_act: bad player id or dilation count");
    return QQT_E_ARG;
  }
  if (a->mode && a->mode_tick != 0u && !a->mode_timer) {
    snprintf(g_err, sizeof(g_err), "qqt_bot_act: the mode ticker needs mode_timer");
    return QQT_E_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  const int h = cfg->height, w = cfg->width, p = cfg->n_players;
  if (h == 13 && w == 13 && p == 2) return launch_bot<13, 13, 2>(cfg, a, st);
  if (h == 7 && w == 7 && p == 2) return launch_bot<7, 7, 2>(cfg, a, st);
  if (h == 9 && w == 9 && p == 2) return launch_bot<9, 9, 2>(cfg, a, st);
  if (h == 13 && w == 13 && p == 3) return launch_bot<13, 13, 3>(cfg, a, st);
  if (h == 13 && w == 13 && p == 4) return launch_bot<13, 13, 4>(cfg, a, st);
  snprintf(g_err, sizeof(g_err), "grid %dx%d with %d players is not compiled", h, w, p);
  return QQT_E_UNSUPPORTED;
}

}  // extern "C"
