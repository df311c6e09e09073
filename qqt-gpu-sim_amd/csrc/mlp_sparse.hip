// MLP actor/critic act kernel with a sparse first layer (gfx950).
//
// Network (train/model.py:121-196, arch "mlp"): obs (B, C*H*W) float16 ->
// Linear(2366,128) -> LayerNorm -> ReLU -> Linear(128,128) -> LayerNorm ->
// ReLU -> three heads Linear(128,64) -> ReLU -> Linear(64, 5 | 2 | 1), then
// masked factored sampling (train/model.py:215-245).
//
// The observation (sim/obs.py:48-136) is mostly zeros: the player splats,
// the per-owner bomb fuses, the danger map, the crates and the one-hot
// invulnerability / bomb-count markers hold a few nonzero cells per env out
// of 169.  Only the wall|brick channel and the progress channel (one value
// over the whole grid) are dense.  So the first layer z1 = W0 x + b0 is
//   sum over the (at most two) dense channels c of W0[:, c] x[c]   (MFMA, hi/lo weights)
//   + sum over the nonzero cells k of every other channel of x[k] W0[:, k]
// with the gathered columns from a [k0][128] float16 table of W0's columns.
// A player's view permutation (sim/config.py:77-94) maps storage channel c to
// view channel vmap[pid][c]; channels that it leaves in place are shared by
// both players, so their terms are gathered once for the env.
//
// Workgroup = 8 wavefronts = 22 rows (half an XCD row block) and both
// players: 5632 rows make 256 workgroups, one per CU.
//   1. wavefront w takes rows w, w+8, w+16 in turn.  Stage 1 tests a row's
//      dwords 64 at a time against a per-lane mask of the gathered halves
//      and keeps the dwords with a nonzero one (candidates); the dense
//      channels' cells go to zero-padded LDS tiles.  Stage 2 classifies the
//      candidates lane-parallel into a shared list and one list per player
//      (table row, value).  Gathers: lane group q (16 lanes) sums z1 kind q
//      of the row (shared even / odd list positions, player 0, player 1),
//      8 features per lane, its columns in flight through the next row's
//      stage 1.
//   2. the dense channels' products run on MFMA (wavefront w = feature tile
//      w) from the LDS tiles and are added to z1.
//   3. the tail (LayerNorm 1, layer 2, LayerNorm 2, heads, sampling) runs
//      one 16-row tile (row tile, player) per wavefront in registers as in
//      the dense kernel (mlp.hip).
// A workgroup whose rows hold more nonzero cells than its lists take
// (random dense inputs, say) computes its first layer as the dense product
// instead (every K block on MFMA from the per-player W0 fragments).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "mlp_common.h"
#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

constexpr int SP_ROWS = XCD_ROWS / 2;     // rows per workgroup
static_assert(SP_ROWS > 16 && SP_ROWS <= 24, "two 16-row tiles, three rows per wavefront");
constexpr int SP_ND = 2;                  // dense channels
constexpr int SP_KSC = 6;                 // 32-K steps per channel (cells <= 192)
constexpr int SP_XS = SP_KSC * 32 + 8;    // dense tile row stride (halves): 400 B
constexpr int SP_NIT = 24;                // 64-dword chunks per row (k0 <= 3072)
constexpr int SP_CAND = 128;              // candidate dwords of one row
constexpr int SP_SCAP = 224;              // shared-list entries of one row
constexpr int SP_PCAP = 112;              // per-player-list entries of one row
constexpr int SP_LIST = SP_SCAP + 2 * SP_PCAP;
constexpr int SP_U = 8;                   // column loads in flight per lane group

struct SparseL1 {                         // first-layer scratch
  uint16_t xd[SP_ND][32][SP_XS];          // dense-channel tiles (other rows, cells zero)
  uint2 cand[8][SP_CAND];                 // per wavefront, its current row: (dword index, dword)
  uint2 list[8][SP_LIST];                 // per wavefront, its current row: (table row, value bits)
  int ovf[8];                             // per wavefront: a row past a capacity
};
static_assert(sizeof(SparseL1) <= 2 * W1_HALVES * 2, "layer-1 scratch fits under W1");

// z1 parts [row][kind][feature]: kinds 0 and 1 the shared entries (even and
// odd list positions; kind 0 also takes the shared dense products), 2 + p
// player p's.  The first-layer scratch and later W1 share one region; the
// head weights go over both once layer 2 is done.
struct __align__(16) SparseLds {
  float vec[V_N];
  uint16_t wf[2 * WF_HALVES];
  union {
    struct {
      float z[SP_ROWS][4][HID];
      union {
        SparseL1 l1;
        uint16_t w1[2 * W1_HALVES];
      } r;
    } a;
    uint16_t wh[2 * WH_HALVES];
  } u;
};

__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ __forceinline__ int mbcnt(uint64_t m, int base) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)base));
}

// View channel of storage channel c from a 4-bit-per-channel map.
__device__ __forceinline__ int vch(uint64_t vm, int c) { return (int)((vm >> (4 * c)) & 15u); }

template <int NP>
__global__ __launch_bounds__(NTHR) void mlp_sparse_kernel(const qqt_mlp_args a) {
  constexpr int W1_CH = 2 * W1_HALVES / 8 / NTHR;
  constexpr int WH_CH = 2 * WH_HALVES / 8 / NTHR;
  constexpr int WF_CH = 2 * WF_HALVES / 8;
  static_assert(WF_CH <= 2 * NTHR && WF_CH > NTHR, "two output-layer chunks per thread");
  __shared__ SparseLds s;
  const int xcd = blockIdx.x & 7, seq = blockIdx.x >> 3;
  const int row0 = ((seq >> 1) * 8 + xcd) * XCD_ROWS + (seq & 1) * SP_ROWS;
  if (row0 >= a.batch) return;                         // padding workgroup (uniform)
  const int nrows = min(SP_ROWS, a.batch - row0);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int C = a.channels, HW = a.cells, k0 = a.k0;
  const int nd = k0 >> 1, nit = (nd + 63) >> 6, ksc = (HW + 31) >> 5;
  const uint32_t dmask = a.dense_mask;
  const int cd0 = dmask ? __builtin_ctz(dmask) : -1;   // the dense channels
  const int cd1 = (dmask & (dmask - 1u)) ? __builtin_ctz(dmask & (dmask - 1u)) : -1;
  const int ndense = (cd0 >= 0) + (cd1 >= 0);
  const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;

  // players of this launch and their view maps (4 bits per storage channel)
  int pidv[2];
  uint64_t vmw[2] = {0u, 0u};
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    pidv[p] = NP == 2 ? p : a.pid0;
#pragma unroll
    for (int c = 0; c < 16; ++c) vmw[p] |= (uint64_t)(a.vmap[pidv[p]][c] & 15) << (4 * c);
  }
  if (NP == 1) { pidv[1] = pidv[0]; vmw[1] = vmw[0]; }
  // channels the packed players see differently (all of them, not just this
  // launch's: a one-player launch then lists and sums its player's terms
  // exactly as a two-player launch does, bit for bit)
  uint32_t ppmask = 0u;
  for (int p = 1; p < a.w0_players; ++p)
#pragma unroll
    for (int c = 0; c < 16; ++c) ppmask |= (uint32_t)(a.vmap[p][c] != a.vmap[0][c]) << c;

  // ---------------- loads in flight first: rows w, w + 8 (w + 16 once row w
  // is scanned, into its registers); the keep mask drops lanes past k0
  const uint32_t* const xbase = reinterpret_cast<const uint32_t*>(a.obs);
  const size_t xstride = (size_t)a.obs_stride / 2;     // dwords per row
  uint32_t xr[2][SP_NIT];
  uint16_t dx[2][SP_ND][3];                            // dense channels' cells lane + 64i
  auto load_row = [&](int jj) __attribute__((always_inline)) {
    const int j = w + 8 * jj;
    if (j < nrows) {
      const uint32_t* rp = xbase + obs_row(a, row0 + j) * xstride;
      const uint16_t* rh = reinterpret_cast<const uint16_t*>(rp);
#pragma unroll
      for (int it = 0; it < SP_NIT; ++it) {
        xr[jj & 1][it] = it < nit ? rp[min(64 * it + lane, nd - 1)] : 0u;
      }
#pragma unroll
      for (int d = 0; d < SP_ND; ++d) {
        const int c = d ? cd1 : cd0;
        if (c >= 0) {
#pragma unroll
          for (int i = 0; i < 3; ++i) dx[jj & 1][d][i] = rh[c * HW + min(lane + 64 * i, HW - 1)];
        }
      }
    }
  };
  load_row(0);
  load_row(1);

  // per-lane mask of the gathered halves of each chunk (the same for every
  // row): 0x7fff per half of a gathered channel below k0, 0 otherwise.  Only
  // chunks that meet a dense channel or k0 need per-lane tests.
  const int dlo0 = cd0 * HW, dlo1 = cd1 * HW;          // (unused when the channel is absent)
  uint32_t keepm[SP_NIT];
#pragma unroll
  for (int it = 0; it < SP_NIT; ++it) {
    const int lo = 128 * it;
    const bool meets = lo + 128 > k0 || (cd0 >= 0 && lo < dlo0 + HW && lo + 128 > dlo0) ||
                       (cd1 >= 0 && lo < dlo1 + HW && lo + 128 > dlo1);
    uint32_t km = 0x7fff7fffu;
    if (meets) {
      km = 0u;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = lo + 2 * lane + h;
        const bool dense = (cd0 >= 0 && (unsigned)(k - dlo0) < (unsigned)HW) ||
                           (cd1 >= 0 && (unsigned)(k - dlo1) < (unsigned)HW);
        if (k < k0 && !dense) km |= 0x7fffu << (16 * h);
      }
    }
    keepm[it] = km;
  }

  // parameter vectors and the output layer's weights
  auto vec_src = [&](int i) -> const float* {
    return i < V_G1 ? a.b0 + (i - V_B0) : i < V_BE1 ? a.ln1_w + (i - V_G1)
         : i < V_B1 ? a.ln1_b + (i - V_BE1) : i < V_G2 ? a.b1 + (i - V_B1)
         : i < V_BE2 ? a.ln2_w + (i - V_G2) : i < V_BH ? a.ln2_b + (i - V_BE2)
         : i < V_BF ? a.bh + (i - V_BH) : a.bf + (i - V_BF);
  };
  auto plane_src = [](const uint16_t* hi, const uint16_t* lo, int halves, int c) {
    const int per = halves / 8;
    return c < per ? reinterpret_cast<const u32x4*>(hi) + c
                   : reinterpret_cast<const u32x4*>(lo) + (c - per);
  };
  const int vi0 = threadIdx.x, vi1 = threadIdx.x + NTHR;
  const float vv0 = *vec_src(vi0);
  const float vv1 = vi1 < V_N ? *vec_src(vi1) : 0.0f;
  const int wc1 = threadIdx.x + NTHR;
  const u32x4 wfv0 = *plane_src(a.wf, a.wf_lo, WF_HALVES, threadIdx.x);
  const u32x4 wfv1 = wc1 < WF_CH ? *plane_src(a.wf, a.wf_lo, WF_HALVES, wc1) : u32x4{0u, 0u, 0u, 0u};

  // sampling inputs of the tail wavefronts' rows (tile t = (row tile t & 1, player t >> 1))
  const bool tail = w < 2 * NP;
  const int trt = w & 1, tp = NP == 2 ? (w >> 1) & 1 : 0;
  const int trow = 16 * trt + r16;                     // row of lanes r16, r16 + 16
  const int tpid = tp ? pidv[1] : pidv[0], toslot = NP == 2 ? tp : a.out_slot;
  const bool sown = tail && lane < 32 && trow < nrows;
  const RowSampler rs = load_sampler(a, a.sample && sown, q & 1, row0 + trow, tpid, oslots, toslot);

  s.vec[vi0] = vv0;
  if (vi1 < V_N) s.vec[vi1] = vv1;
  reinterpret_cast<u32x4*>(s.wf)[threadIdx.x] = wfv0;
  if (wc1 < WF_CH) reinterpret_cast<u32x4*>(s.wf)[wc1] = wfv1;

  SparseL1& L = s.u.a.r.l1;
  const float inv_hw = 1.0f / (float)HW;
  // the dense tiles' rows of this wavefront (w + 8i) start at zero
  if (ndense && lane < SP_XS / 8) {
#pragma unroll
    for (int d = 0; d < SP_ND; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        reinterpret_cast<u32x4*>(&L.xd[d][w + 8 * i][0])[lane] = u32x4{0u, 0u, 0u, 0u};
  }

  // ---------------- per row of the wavefront: scan (stage 1), lists (stage 2),
  // gathers.  A row's column loads stay in flight through the next row's stage 1.
  const uint16_t* const tab = a.w0g + r16 * 8;
  // stage 1: the row's dwords holding a nonzero gathered half; the dense
  // channels' cells into their tiles
  auto stage1 = [&](int jj, int j) __attribute__((always_inline)) {
    int cnt = 0;
#pragma unroll
    for (int it = 0; it < SP_NIT; ++it) {
      const uint32_t dw = xr[jj & 1][it];
      const bool hit = (dw & keepm[it]) != 0u;
      const uint64_t m = __ballot(hit);
      const int pos = min(mbcnt(m, cnt), SP_CAND - 1);   // (a full list only overflows)
      if (hit) L.cand[w][pos] = make_uint2(64 * it + lane, dw);
      cnt += __popcll(m);
    }
#pragma unroll
    for (int d = 0; d < SP_ND; ++d) {
      if (d < ndense) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          if (lane + 64 * i < HW) L.xd[d][j][lane + 64 * i] = dx[jj & 1][d][i];
      }
    }
    return cnt;
  };
  // appends the lanes' entries (where on) to a list holding n; returns its new length
  auto append = [&](bool on, int n, int cap, int off, uint32_t tr, float v) __attribute__((always_inline)) {
    const uint64_t m = __ballot(on);
    const int pos = min(mbcnt(m, n), cap - 1);
    if (on) L.list[w][off + pos] = make_uint2(tr, __float_as_uint(v));
    return n + __popcll(m);
  };
  // stage 2: candidates -> the shared list and one list per player; returns
  // whether a capacity was passed
  auto stage2 = [&](int cnt, int& nS, int& nP0, int& nP1) __attribute__((always_inline)) {
    const int nc = min(cnt, SP_CAND);
    nS = nP0 = nP1 = 0;
    for (int base = 0; base < nc; base += 64) {
      const int i = base + lane;
      const bool has = i < nc;
      const uint2 cdw = has ? L.cand[w][i] : make_uint2(0u, 0u);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * (int)cdw.x + h;
        const uint32_t bits = h ? cdw.y >> 16 : cdw.y & 0xffffu;
        const int c = min((int)(((float)k + 0.5f) * inv_hw), C - 1);
        const int cell = k - c * HW;
        const bool ex = has && (bits & 0x7fffu) != 0u && c != cd0 && c != cd1;
        const float v = h2f(bits);
        const bool pp = (ppmask >> c) & 1u;
        nS = append(ex && !pp, nS, SP_SCAP, 0, (uint32_t)(vch(vmw[0], c) * HW + cell), v);
        nP0 = append(ex && pp, nP0, SP_PCAP, SP_SCAP, (uint32_t)(vch(vmw[0], c) * HW + cell), v);
        if (NP == 2)
          nP1 = append(ex && pp, nP1, SP_PCAP, SP_SCAP + SP_PCAP,
                       (uint32_t)(vch(vmw[1], c) * HW + cell), v);
      }
    }
    return cnt > SP_CAND || nS > SP_SCAP || nP0 > SP_PCAP || nP1 > SP_PCAP;
  };
  // lane group q takes z1 kind q of a row (NP = 1: group 3 idles): its first
  // SP_U entries' columns are loaded by issue(), summed by consume() with the
  // rest of the entries, which are still in the lists then
  u32x4 gd[SP_U];
  float gv[SP_U];
  int gn = 0, glidx = 0, gstr = 1;
  auto issue = [&](int nS, int nP0, int nP1) __attribute__((always_inline)) {
    gn = 0;
    glidx = 0;
    gstr = 1;
    if (q < 2) {
      gn = q == 0 ? (nS + 1) >> 1 : nS >> 1;
      glidx = q;
      gstr = 2;
    } else if (q - 2 < NP) {
      gn = q == 2 ? nP0 : nP1;
      glidx = SP_SCAP + (q - 2) * SP_PCAP;
    }
#pragma unroll
    for (int u = 0; u < SP_U; ++u) {
      const bool ok = u < gn;
      const uint2 e = ok ? L.list[w][glidx + u * gstr] : make_uint2(0u, 0u);
      gv[u] = __uint_as_float(e.y);
      gd[u] = ok ? *reinterpret_cast<const u32x4*>(tab + (size_t)e.x * HID) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto consume = [&](int j) __attribute__((always_inline)) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int u = 0; u < SP_U; ++u) {
      const half8 hv = as_h8(gd[u]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(gv[u], (float)hv[i], acc[i]);
    }
    for (int m0 = SP_U; m0 < gn; m0 += SP_U) {        // long lists: the rest, batch by batch
#pragma unroll
      for (int u = 0; u < SP_U; ++u) {
        const bool ok = m0 + u < gn;
        const uint2 e = ok ? L.list[w][glidx + (m0 + u) * gstr] : make_uint2(0u, 0u);
        gv[u] = __uint_as_float(e.y);
        gd[u] = ok ? *reinterpret_cast<const u32x4*>(tab + (size_t)e.x * HID) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < SP_U; ++u) {
        const half8 hv = as_h8(gd[u]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(gv[u], (float)hv[i], acc[i]);
      }
    }
    if (q < 2 + NP) {
      float4* zp = reinterpret_cast<float4*>(&s.u.a.z[j][q][8 * r16]);
      zp[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      zp[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
  };
  bool wave_ovf = false;
  int jlive = -1;                                      // row whose gathers are in flight
#pragma unroll
  for (int jj = 0; jj < 3; ++jj) {
    const int j = w + 8 * jj;
    if (j >= nrows) continue;                          // uniform
    const int cnt = stage1(jj, j);
    if (jj == 0) load_row(2);                          // into row 0's registers
    if (jlive >= 0) consume(jlive);
    wave_sync();
    int nS, nP0, nP1;
    const bool row_ovf = stage2(cnt, nS, nP0, nP1);
    wave_ovf = wave_ovf || row_ovf;
    jlive = -1;
    if (row_ovf) continue;                             // the workgroup goes dense
    wave_sync();
    issue(nS, nP0, nP1);
    jlive = j;
  }
  if (jlive >= 0) consume(jlive);
  if (lane == 0) L.ovf[w] = wave_ovf ? 1 : 0;
  // rows past the batch: zero z1 parts (the tail reads them)
  for (int j = nrows + w; j < SP_ROWS; j += 8)
    if (q < 2 + NP) {
      float4* zp = reinterpret_cast<float4*>(&s.u.a.z[j][q][8 * r16]);
      zp[0] = zp[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

  // the dense channels' A fragments (player 0's view; a channel the players
  // see differently loads player 1's in the loop) and layer 2's weights: in
  // flight through the barrier
  int dj0[SP_ND], dj1[SP_ND];
  bool dsh[SP_ND];
#pragma unroll
  for (int d = 0; d < SP_ND; ++d) {
    const int c = d ? cd1 : cd0;
    dj0[d] = c >= 0 ? vch(vmw[0], c) : 0;
    dj1[d] = c >= 0 ? vch(vmw[1], c) : 0;
    dsh[d] = NP == 1 || dj0[d] == dj1[d];
  }
  half8 dah[SP_ND][SP_KSC], dal[SP_ND][SP_KSC];
#pragma unroll
  for (int d = 0; d < SP_ND; ++d)
#pragma unroll
    for (int st = 0; st < SP_KSC; ++st) {
      if (d < ndense && st < ksc) {
        const uint16_t* ap = a.w0d + ((((size_t)dj0[d] * 8 + w) * ksc + st) * 2) * 512 + lane * 8;
        dah[d][st] = *reinterpret_cast<const half8*>(ap);
        dal[d][st] = *reinterpret_cast<const half8*>(ap + 512);
      }
    }
  u32x4 w1v[W1_CH];
#pragma unroll
  for (int c = 0; c < W1_CH; ++c) w1v[c] = *plane_src(a.w1, a.w1_lo, W1_HALVES, threadIdx.x + NTHR * c);
  __syncthreads();   // every row's gathers and dense tile row are in LDS

  // a row past a capacity sends the whole workgroup down the dense path
  const bool ovf = __ballot(lane < 8 && L.ovf[lane] != 0) != 0ull;
  if (!ovf) {
    // ---------------- dense channels on MFMA: wavefront w = feature tile w
    floatx4 dk[3][2];                                  // shared, player 0, player 1
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) dk[t][rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    bool dk_on[3] = {false, false, false};
#pragma unroll
    for (int d = 0; d < SP_ND; ++d) {
      if (d >= ndense) continue;
      if (dsh[d]) dk_on[0] = true;
      else { dk_on[1] = true; dk_on[2] = NP == 2; }
#pragma unroll
      for (int st = 0; st < SP_KSC; ++st) {
        if (st >= ksc) continue;
        half8 b[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          b[rt] = *reinterpret_cast<const half8*>(&L.xd[d][16 * rt + r16][32 * st + 8 * q]);
        if (dsh[d]) {
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            dk[0][rt] = mfma(dah[d][st], b[rt], dk[0][rt]);
            dk[0][rt] = mfma(dal[d][st], b[rt], dk[0][rt]);
          }
        } else {
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            dk[1][rt] = mfma(dah[d][st], b[rt], dk[1][rt]);
            dk[1][rt] = mfma(dal[d][st], b[rt], dk[1][rt]);
          }
          if (NP == 2) {
            const uint16_t* ap = a.w0d + ((((size_t)dj1[d] * 8 + w) * ksc + st) * 2) * 512 + lane * 8;
            const half8 ahi = *reinterpret_cast<const half8*>(ap);
            const half8 alo = *reinterpret_cast<const half8*>(ap + 512);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              dk[2][rt] = mfma(ahi, b[rt], dk[2][rt]);
              dk[2][rt] = mfma(alo, b[rt], dk[2][rt]);
            }
          }
        }
      }
    }
    // into z1: lane (r16, q) owns features 16w + 4q .. +3 of its rows
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = 16 * rt + r16;
      if (row < SP_ROWS) {
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          if (!dk_on[t]) continue;
          float4* zp = reinterpret_cast<float4*>(&s.u.a.z[row][t ? 1 + t : 0][16 * w + 4 * q]);
          const float4 o = *zp;
          *zp = make_float4(o.x + dk[t][rt][0], o.y + dk[t][rt][1], o.z + dk[t][rt][2],
                            o.w + dk[t][rt][3]);
        }
      }
    }
  } else {
    // ---------------- dense first layer: every K block of the per-player W0 fragments
    floatx4 dk[2][2];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) dk[p][rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* xrow[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      xrow[rt] = a.obs + obs_row(a, row0 + min(16 * rt + r16, nrows - 1)) * (size_t)a.obs_stride;
    for (int kb = 0; kb < a.kblocks0; ++kb) {
      Frag16 bx[2];
      const int k = 64 * kb + 16 * q;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if (k + 16 <= k0) {
          u32x4 lo, hi;
          __builtin_memcpy(&lo, xrow[rt] + k, 16);
          __builtin_memcpy(&hi, xrow[rt] + k + 8, 16);
          bx[rt].lo = as_h8(lo);
          bx[rt].hi = as_h8(hi);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            bx[rt].lo[i] = k + i < k0 ? __builtin_bit_cast(_Float16, xrow[rt][k + i]) : (_Float16)0.0f;
            bx[rt].hi[i] =
                k + 8 + i < k0 ? __builtin_bit_cast(_Float16, xrow[rt][k + 8 + i]) : (_Float16)0.0f;
          }
        }
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const Frag16 aw =
            load_b(a.w0 + ((size_t)(pidv[p] * 8 + w) * a.kblocks0 + kb) * 1024 + lane * 16);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          dk[p][rt] = mfma(aw.lo, bx[rt].lo, dk[p][rt]);
          dk[p][rt] = mfma(aw.hi, bx[rt].hi, dk[p][rt]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = 16 * rt + r16;
      if (row < SP_ROWS) {
        const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *reinterpret_cast<float4*>(&s.u.a.z[row][0][16 * w + 4 * q]) = zero;
        *reinterpret_cast<float4*>(&s.u.a.z[row][1][16 * w + 4 * q]) = zero;
#pragma unroll
        for (int p = 0; p < NP; ++p)
          *reinterpret_cast<float4*>(&s.u.a.z[row][2 + p][16 * w + 4 * q]) =
              make_float4(dk[p][rt][0], dk[p][rt][1], dk[p][rt][2], dk[p][rt][3]);
      }
    }
  }
  __syncthreads();   // every wavefront is past its dense-tile reads
#pragma unroll
  for (int c = 0; c < W1_CH; ++c) reinterpret_cast<u32x4*>(s.u.a.r.w1)[threadIdx.x + NTHR * c] = w1v[c];
  __syncthreads();

  // head weights: in flight through LayerNorm 1 and layer 2
  u32x4 whv[WH_CH];
#pragma unroll
  for (int i = 0; i < WH_CH; ++i) whv[i] = *plane_src(a.wh, a.wh_lo, WH_HALVES, threadIdx.x + NTHR * i);

  // ---------------- LayerNorm 1, layer 2, LayerNorm 2: tail wavefront = (row tile, player)
  half8 hh[4], hl[4];
  if (tail) {
    floatx4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      floatx4 z = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (trow < SP_ROWS) {
        const floatx4 e0 = *reinterpret_cast<const floatx4*>(&s.u.a.z[trow][0][16 * t + 4 * q]);
        const floatx4 e1 = *reinterpret_cast<const floatx4*>(&s.u.a.z[trow][1][16 * t + 4 * q]);
        const floatx4 ep = *reinterpret_cast<const floatx4*>(&s.u.a.z[trow][2 + tp][16 * t + 4 * q]);
        z = (e0 + e1) + ep;
      }
      v[t] = z + vec4(s.vec + V_B0, t, q);
    }
    ln_relu_split(v, s.vec + V_G1, s.vec + V_BE1, q, hh, hl);
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = vec4(s.vec + V_B1, t, q);
    tail_gemm<8, 4>(v, s.u.a.r.w1, s.u.a.r.w1 + W1_HALVES, hh, hl, lane);
    ln_relu_split(v, s.vec + V_G2, s.vec + V_BE2, q, hh, hl);
  }
  __syncthreads();   // every tail wavefront is past layer 2: z1 and W1 are dead
#pragma unroll
  for (int i = 0; i < WH_CH; ++i) reinterpret_cast<u32x4*>(s.u.wh)[threadIdx.x + NTHR * i] = whv[i];
  __syncthreads();
  if (!tail) return;   // no barrier below

  // ---------------- heads: 128 -> 192 (+ bias, ReLU), then 192 -> 8 (block diagonal)
  half8 yh[6], yl[6];
  floatx4 o[1] = {vec4(s.vec + V_BF, 0, q & 1)};
  {
    floatx4 a3[12];
#pragma unroll
    for (int t = 0; t < 12; ++t) a3[t] = vec4(s.vec + V_BH, t, q);
    tail_gemm<12, 4>(a3, s.u.wh, s.u.wh + WH_HALVES, hh, hl, lane);
#pragma unroll
    for (int t = 0; t < 12; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        split_into(fmaxf(a3[t][j], 0.0f), yh[t >> 1], yl[t >> 1], 4 * (t & 1) + j);
  }
  tail_gemm<1, 6>(o, s.wf, s.wf + WF_HALVES, yh, yl, lane);

  // ---------------- outputs and sampling: lanes r and r + 16 own the tile's row r
  const float out4 = __shfl(o[0][0], lane + 16, 64);
  const bool half0 = q == 0;
  float lp = 0.0f;
  int act = 0;
  if (rs.on) {
    const float lg[5] = {half0 ? o[0][0] : o[0][1], half0 ? o[0][1] : o[0][2],
                         half0 ? o[0][2] : 0.0f, half0 ? o[0][3] : 0.0f, half0 ? out4 : 0.0f};
    act = sample_masked_n(lg, rs.m, half0 ? 5 : 2, rs.u, &lp);
  }
  const float lpb = __shfl(lp, lane + 16, 64);
  if (sown) {
    const size_t oo = (size_t)(row0 + trow) * oslots + toslot;
    if (a.logits_out) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a.logits_out[oo * NOUT + 4 * q + j] = o[0][j];
    }
    if (!half0 && a.value_out) a.value_out[oo] = o[0][3];
    if (rs.on) {
      if (a.actions) a.actions[oo * 2 + q] = act;
      if (a.actions_i8) a.actions_i8[oo * 2 + q] = (int8_t)act;
      if (half0 && a.logp_out) a.logp_out[oo] = lp + lpb;
    }
  }
}


bool mlp_sparse_eligible(const qqt_mlp_args& a) {
  if (!a.sparse || a.z1_out || !a.w0g) return false;
  if (a.npid != 1 && a.npid != 2) return false;
  if (a.cells < 128 || a.cells > 32 * SP_KSC || a.channels < 1 || a.channels > 16) return false;
  if (a.k0 != a.channels * a.cells || a.k0 > 128 * SP_NIT) return false;
  if (__builtin_popcount(a.dense_mask) > SP_ND || (a.dense_mask >> a.channels)) return false;
  if (a.dense_mask && !a.w0d) return false;
  for (int p = 0; p < a.w0_players; ++p)
    for (int c = 0; c < a.channels; ++c)
      if (a.vmap[p][c] < 0 || a.vmap[p][c] >= a.channels) return false;
  return true;
}

int mlp_sparse_launch(const qqt_mlp_args& a, hipStream_t st) {
  const int nrb = (a.batch + XCD_ROWS - 1) / XCD_ROWS;
  const int blocks = ((nrb + 7) / 8) * 8 * 2;
  if (a.npid == 2)
    QQT_LAUNCH(QQT_KERNEL_MLP, mlp_sparse_kernel<2>, dim3(blocks), dim3(NTHR), st, a);
  else
    QQT_LAUNCH(QQT_KERNEL_MLP, mlp_sparse_kernel<1>, dim3(blocks), dim3(NTHR), st, a);
  return 0;
}

}  // namespace qqt
