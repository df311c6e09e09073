// MLP actor/critic forward + masked factored sampling for gfx950 (MFMA).
//
// Network (train/model.py:121-196, arch "mlp"): obs (B, C*H*W) float16 ->
// Linear(2366,128) -> LayerNorm -> ReLU -> Linear(128,128) -> LayerNorm ->
// ReLU -> three heads Linear(128,64) -> ReLU -> Linear(64, 5 | 2 | 1).
// A player's view permutation is folded into the first-layer weights, so a
// player is just a column block of one shared weight buffer.
//
// mlp_act_kernel: workgroup = 8 wavefronts (2 per SIMD) = one row block of
// one player, an XCD row block of 44 rows (three 16-row tiles).  Forward
// batches without sampling from 65,536 rows take mlp_fwd_kernel instead
// (256-row workgroups, described at that kernel).  Both players'
// workgroups of a row block are dispatched back to back on the same XCD
// (workgroups are dealt to the 8 XCDs round robin), so the second read of
// the observation tile hits that XCD's L2, where the tick kernel wrote it.
//
// Every product is v_mfma_f32_16x16x32_f16 (float32 accumulation) with the
// weights as the A operand and the activations as the B operand, so a 16 x 16
// output tile holds features 4q..4q+3 of batch row r in lane 16q + r
// (q = lane / 16).
//
// Layer 1 (K = 2366) is split over two groups of four wavefronts: group g
// takes K blocks g, g+2, g+4, ...  Each group streams its observation tiles
// (16RT rows x 64 K) through its own double-buffered, XOR-swizzled LDS tile
// (loaded PD steps ahead into registers); the weight fragments go straight
// from L2 into registers, PD steps ahead.  Wavefront (g, c) owns features
// 32c..32c+31 of every row.  The groups' partial sums meet in LDS (group 1
// writes, group 0 adds), laid out by (row tile, feature tile, lane).
//
// Everything after layer 1 runs per 16-row tile inside one wavefront, in
// registers (wavefront w takes row tile w; wavefronts past the last tile
// only help stage weights).  A row's 128 features sit in lanes r, r+16, r+32,
// r+48, so LayerNorm reduces with two cross-lane exchanges, and the output
// tiles of one product are, unchanged, the B operand of the next: K step s
// of the next product reads feature tiles 2s and 2s+1, i.e. MFMA K index
// 8q + i is feature 32s + 4q + i (i < 4) or 32s + 16 + 4q + (i - 4) (i >= 4);
// the host stores the later layers' weights in that K order.  Those layers
// carry activations and weights as float16 hi/lo pairs (x = hi + lo) and sum
// hi*hi + hi*lo + lo*hi, which keeps logits within ~5e-4 of a float32 forward
// even for large (orthogonal, gain sqrt 2) weights.  Their weights are read
// from LDS: layer 2's (64 KB, both planes) is staged in the prologue; the
// heads' (96 KB) is loaded into registers while layer 2 runs and written over
// layer 2's weights and the dead observation tiles once every tail wavefront
// is past layer 2.
//
// Fragment layouts (built by qqtsim/policy.py):
//   w0:          frag[tile][kblock][lane][16] =
//                  W[16*tile + lane%16][64*kblock + 16*(lane/16) + j];
//                the observation row's 16 halves at the same K offsets form
//                the B operand (a K order inside the block shared by both);
//   w1, wh, wf:  frag[tile][kstep][lane][8] =
//   (hi and lo)    W[16*tile + lane%16][32*kstep + perm(lane/16, i)],
//                perm(q, i) = 4q + i (i < 4), 16 + 4q + (i - 4) (i >= 4).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <type_traits>
#include <utility>

#include "mlp_common.h"
#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

// Row tiles (16 rows each) per workgroup.  Rollout-sized batches take RT = 3
// tiles over an XCD row block of 44 rows: 5632 rows make 128 row blocks x 2
// players = 256 workgroups, one per CU (64-row blocks left 80 of the 256 CUs
// idle and put a third more MFMA work on each busy one).  Forward batches
// (no sampling) from MLP_BIG_ROWS rows go to mlp_fwd_kernel (256-row
// workgroups, W0 streamed once per 256 rows).
constexpr int RT_SMALL = (XCD_ROWS + 15) / 16;
constexpr int RT_HALF = (XCD_ROWS / 2 + 15) / 16;   // half an XCD row block
constexpr int MLP_BIG_ROWS = 1 << 16;
#ifndef QQT_MLP_PD
#define QQT_MLP_PD 2
#endif
constexpr int PD = QQT_MLP_PD;     // K blocks of layer 1 in flight per group (even)
static_assert(PD >= 2 && PD % 2 == 0, "the x tile ring pairs with an LDS double buffer");

// Observation tiles store rows of 64 float16 as eight 16-byte chunks; chunk c
// of row r sits at position c ^ (r & 7) ^ ((r >> 3) & 1).  The 16 rows of one
// fragment read then land on 16 distinct 16-byte bank groups of a 256-byte
// bank window (row r's window half is r & 1), and any 8 consecutive rows on 8
// distinct groups of a 128-byte window.
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ (row & 7) ^ ((row >> 3) & 1);
}

// LDS of a workgroup of RT row tiles.  xw holds the layer-1 x tiles
// [group][buffer] (16RT rows x 64 K each) and then layer 2's weight planes;
// after layer 1 the partial-sum exchange ([row tile][feature tile][lane]
// floatx4, exactly the x tiles' bytes) reuses the x tiles, and after layer 2
// the head weights overwrite the front of xw.
template <int RT>
struct __align__(16) MlpLds {
  static constexpr int XT = RT * 16 * 64;     // halves of one x tile
  static constexpr int XW = 4 * XT + 2 * W1_HALVES > 2 * WH_HALVES ? 4 * XT + 2 * W1_HALVES
                                                                   : 2 * WH_HALVES;
  uint16_t xw[XW];
  uint16_t wf[2 * WF_HALVES];                 // output-layer fragments, hi and lo planes
  float vec[V_N];                             // biases and LayerNorm affine parameters
};

// The B fragment (16 halves of row `row`, K 16q..16q+15 of the block) from a
// swizzled 64-K observation tile.
__device__ __forceinline__ Frag16 read_x(const uint16_t* tile, int row, int q) {
  const uint16_t* r = tile + row * 64;
  Frag16 f;
  f.lo = as_h8(*reinterpret_cast<const uint4*>(r + (swz(row, 2 * q) << 3)));
  f.hi = as_h8(*reinterpret_cast<const uint4*>(r + (swz(row, 2 * q + 1) << 3)));
  return f;
}


// RT row tiles (16RT rows) per workgroup.
// Z1: the first-layer-only instantiation of the training forward (z1_out).
// HALF: the workgroup owns half an XCD row block (one-player launches: 5632
// rows then make 256 workgroups instead of 128).
template <int RT, bool Z1, bool HALF = false>
__global__ __launch_bounds__(NTHR) void mlp_act_kernel(const qqt_mlp_args a) {
  static_assert(RT >= 1 && RT <= 8, "tail wavefronts take one row tile each");
  constexpr int ROWS = 16 * RT;            // rows of the workgroup's tiles
  // rows the workgroup owns: an XCD row block (or half of one) for
  // rollout-sized batches (the last tile's rows past it are computed on the
  // next block's rows and dropped)
  constexpr int BROWS = HALF ? XCD_ROWS / 2 : RT == RT_SMALL ? XCD_ROWS : ROWS;
  static_assert(BROWS <= ROWS && BROWS > ROWS - 16, "the tiles cover the block");
  constexpr int NX = 2 * RT;               // x load instructions per wavefront and K block
  constexpr int XT = MlpLds<RT>::XT;       // one x tile of the workgroup
  constexpr int W1_CH = 2 * W1_HALVES / 8 / NTHR;   // 16-byte chunks of W1 per thread
  constexpr int WH_CH = 2 * WH_HALVES / 8 / NTHR;   // ... of the head weights
  constexpr int WF_CH = 2 * WF_HALVES / 8;          // 16-byte chunks of the output layer
  static_assert(W1_CH * NTHR * 8 == 2 * W1_HALVES && WH_CH * NTHR * 8 == 2 * WH_HALVES,
                "weight staging divides over the threads");
  static_assert(WF_CH <= 2 * NTHR && WF_CH > NTHR, "two output-layer chunks per thread");
  __shared__ MlpLds<RT> s;
  const int nrb = (a.batch + BROWS - 1) / BROWS;
  const int xcd = blockIdx.x & 7, seq = blockIdx.x >> 3;
  const int slot = seq % a.npid;
  // (half blocks 2k, 2k + 1 of XCD row block k, on that block's XCD)
  const int rb = HALF ? (((seq / a.npid) >> 1) * 8 + xcd) * 2 + ((seq / a.npid) & 1)
                      : (seq / a.npid) * 8 + xcd;
  if (rb >= nrb) return;                   // padding workgroup (uniform, before any barrier)
  const int pid = a.npid == 2 ? slot : a.pid0;
  const int row0 = rb * BROWS;
  // wavefront index as a scalar: branches and addresses on it stay uniform
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int kg = w >> 2, cg = w & 3;       // layer-1 K group, column group
  const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;   // output row width (slots)
  const int oslot = a.npid == 2 ? slot : a.out_slot;
  uint16_t* const w1s = s.xw + 4 * XT;                         // layer-2 weights in LDS

  // Parameter vectors (two floats per thread), the output layer's and layer
  // 2's weights: loaded before the first tiles (vmcnt retires in order) and
  // written to LDS after those are issued.
  auto vec_src = [&](int i) -> const float* {
    return i < V_G1 ? a.b0 + (i - V_B0) : i < V_BE1 ? a.ln1_w + (i - V_G1)
         : i < V_B1 ? a.ln1_b + (i - V_BE1) : i < V_G2 ? a.b1 + (i - V_B1)
         : i < V_BE2 ? a.ln2_w + (i - V_G2) : i < V_BH ? a.ln2_b + (i - V_BE2)
         : i < V_BF ? a.bh + (i - V_BH) : a.bf + (i - V_BF);
  };
  const int vi0 = threadIdx.x, vi1 = threadIdx.x + NTHR;   // vi1 < V_N for the first 456
  const float vv0 = *vec_src(vi0);
  const float vv1 = vi1 < V_N ? *vec_src(vi1) : 0.0f;
  auto plane_src = [](const uint16_t* hi, const uint16_t* lo, int halves, int c) {
    const int per = halves / 8;
    return c < per ? reinterpret_cast<const u32x4*>(hi) + c
                   : reinterpret_cast<const u32x4*>(lo) + (c - per);
  };
  u32x4 wfv[2];
  const int wc1 = threadIdx.x + NTHR;
  if constexpr (!Z1) {
    wfv[0] = *plane_src(a.wf, a.wf_lo, WF_HALVES, threadIdx.x);
    wfv[1] = wc1 < WF_CH ? *plane_src(a.wf, a.wf_lo, WF_HALVES, wc1) : u32x4{0u, 0u, 0u, 0u};
  }
  // Layer 2's weights (64 KB) go to LDS in the prologue.  Staging them one
  // chunk per K step instead was measured 1.3 us slower: the conditional
  // stores split the K loop's body and the extra requests slow its stream.
  u32x4 w1v[W1_CH];
  if constexpr (!Z1) {
#pragma unroll
    for (int c = 0; c < W1_CH; ++c)
      w1v[c] = *plane_src(a.w1, a.w1_lo, W1_HALVES, threadIdx.x + NTHR * c);
  }

  // ---------------- layer 1: group kg, K blocks kg, kg+2, ...; features 32cg..32cg+31
  floatx4 acc[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // x loads: instruction i of wavefront (kg, cg) covers tile rows
  // 4RTcg+2i, 4RTcg+2i+1; lane l reads dword l&31 (two halves) of row
  // 4RTcg+2i+(l>>5).
  const int nkb = a.kblocks0;
  const int dw = lane & 31;
  // row addresses are formed at each load from one base row (clamped to
  // the batch for a ragged last block), not held as NX pointers
  const int xrow0 = row0 + 4 * RT * cg + (lane >> 5);
  const uint32_t* const xbase = reinterpret_cast<const uint32_t*>(a.obs);
  const size_t xstride = (size_t)a.obs_stride / 2;    // dwords per row
  const uint16_t* wb = a.w0 + (size_t)((pid * 8 + 2 * cg) * nkb) * 64 * 16 + lane * 16;
  const size_t wtile = (size_t)nkb * 64 * 16;   // halves between weight tiles
  uint16_t* const xt = s.xw + kg * 2 * XT;      // this group's two x tiles

  // Loads run PD group steps ahead and go to LDS unchanged (a select on them
  // is scheduled early and shortens the prefetch).  Lanes past k0 read dword 0
  // of their row (in bounds, finite): w0 is zero at K >= k0, so those
  // products add zero.
  const uint32_t* xrp[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) xrp[i] = xbase + obs_row(a, min(xrow0 + 2 * i, a.batch - 1)) * xstride;
  auto load_x = [&](int kb, uint32_t (&xr)[NX]) {
    const int k = 64 * kb + 2 * dw;              // first half of this lane's pair
    const int off = k < a.k0 ? (k >> 1) : 0;     // k0 is even: pairs never straddle
#pragma unroll
    for (int i = 0; i < NX; ++i) xr[i] = xrp[i][off];   // cached: two workgroups read each row
  };
  auto load_w = [&](int kb, Frag16 (&br)[2]) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) br[ct] = load_b(wb + ct * wtile + (size_t)kb * 64 * 16);
  };
  auto store_x = [&](const uint32_t (&xr)[NX], int buf, int) {
    uint32_t* t = reinterpret_cast<uint32_t*>(xt + buf * XT);
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int r = 4 * RT * cg + 2 * i + (lane >> 5);
      t[r * 32 + (swz(r, dw >> 2) << 2) + (dw & 3)] = xr[i];
    }
  };
  auto compute = [&](int buf, const Frag16 (&br)[2]) {
    const uint16_t* t = xt + buf * XT;
    Frag16 xf[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) xf[rt] = read_x(t, 16 * rt + r16, q);
    // low K halves over every tile pair, then the high halves
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          acc[rt][ct] = h ? mfma(br[ct].hi, xf[rt].hi, acc[rt][ct])
                          : mfma(br[ct].lo, xf[rt].lo, acc[rt][ct]);
  };

  // Group step i handles K block 2i + kg.  Register ring of PD steps in
  // flight, LDS double buffer per group, one barrier per step: prefetch
  // indices are clamped to the last block, and the step count is padded to a
  // multiple of PD.  A group has at most PD padded steps (nsteps - floor(nkb/2)
  // <= PD), so they all fall in the last PD steps, whose products are skipped
  // by a uniform branch (their tiles hold the clamped last block).
  uint32_t xr[PD][NX];
  Frag16 br[PD][2];
  const int last = nkb - 1;
  const int nsteps = (((nkb + 1) / 2 + PD - 1) / PD) * PD;
  auto kblk = [&](int i) { return 2 * i + kg; };
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    load_x(min(kblk(j), last), xr[j]);
    load_w(min(kblk(j), last), br[j]);
  }

  // output row of lanes l and l + 16 (l < 16) of tail wavefront w: row0 + 16w + l
  const int srow = row0 + 16 * w + r16;
  const bool sown = w < RT && lane < 32 && 16 * w + r16 < BROWS && srow < a.batch;
  const RowSampler rs = load_sampler(a, !Z1 && a.sample && sown, q & 1, srow, pid, oslots, oslot);

  s.vec[vi0] = vv0;
  if (vi1 < V_N) s.vec[vi1] = vv1;
  if constexpr (!Z1) {
    reinterpret_cast<u32x4*>(s.wf)[threadIdx.x] = wfv[0];
    if (wc1 < WF_CH) reinterpret_cast<u32x4*>(s.wf)[wc1] = wfv[1];
#pragma unroll
    for (int c = 0; c < W1_CH; ++c) reinterpret_cast<u32x4*>(w1s)[threadIdx.x + NTHR * c] = w1v[c];
  }
  store_x(xr[0], 0, kblk(0));
  load_x(min(kblk(PD), last), xr[0]);
  __syncthreads();
  for (int i0 = 0; i0 < nsteps - PD; i0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; ++j) {
      const int i = i0 + j;                 // LDS buffer j&1 holds block kblk(i)
      compute(j & 1, br[j]);
      load_w(min(kblk(i + PD), last), br[j]);
      store_x(xr[(j + 1) % PD], (j + 1) & 1, kblk(i + 1));
      load_x(min(kblk(i + 1 + PD), last), xr[(j + 1) % PD]);
      __syncthreads();
    }
  }
  // last PD steps: everything they need is already in flight
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    if (kblk(nsteps - PD + j) <= last) compute(j & 1, br[j]);
    if (j + 1 < PD) store_x(xr[(j + 1) % PD], (j + 1) & 1, kblk(nsteps - PD + j + 1));
    __syncthreads();
  }

  // Head weights: in flight through the partial-sum exchange and layer 2.
  u32x4 whv[WH_CH];
  if constexpr (!Z1) {
#pragma unroll
    for (int i = 0; i < WH_CH; ++i)
      whv[i] = *plane_src(a.wh, a.wh_lo, WH_HALVES, threadIdx.x + NTHR * i);
  }

  // ---------------- the groups' partial sums meet in the (now free) x tiles:
  // ex[(row tile * 8 + feature tile) * 64 + lane]; group 1 writes, group 0 adds.
  floatx4* const ex = reinterpret_cast<floatx4*>(s.xw);
  if (kg == 1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) ex[(rt * 8 + 2 * cg + ct) * 64 + lane] = acc[rt][ct];
  }
  __syncthreads();
  if (kg == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        floatx4& e = ex[(rt * 8 + 2 * cg + ct) * 64 + lane];
        e = acc[rt][ct] + e;
      }
  }
  __syncthreads();

  if constexpr (Z1) {   // first layer only (the training forward): z1 = (f + f1) + b0
#pragma unroll
    for (int hb = 0; hb < (ROWS + 63) / 64; ++hb) {
      // thread t: row 64hb + t/8 of the workgroup, features 16(t%8) .. +15 as four float4
      const int row = 64 * hb + (threadIdx.x >> 3), ft = threadIdx.x & 7;
      const int orow = row0 + row;
      if (row < BROWS && orow < a.batch) {
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const floatx4 e = ex[((row >> 4) * 8 + ft) * 64 + 16 * q2 + (row & 15)];
          const float4 b = *reinterpret_cast<const float4*>(&s.vec[V_B0 + 16 * ft + 4 * q2]);
          *reinterpret_cast<float4*>(a.z1_out + (size_t)orow * HID + 16 * ft + 4 * q2) =
              make_float4(e[0] + b.x, e[1] + b.y, e[2] + b.z, e[3] + b.w);
        }
      }
    }
    return;
  }

  // ---------------- LayerNorm 1, layer 2, LayerNorm 2: tail wavefront w, row tile w
  const bool tail = w < RT;
  half8 hh[4], hl[4];
  if (tail) {
    floatx4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = ex[(w * 8 + t) * 64 + lane];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = v[t] + vec4(s.vec + V_B0, t, q);   // z1 = (f + f1) + b0
    ln_relu_split(v, s.vec + V_G1, s.vec + V_BE1, q, hh, hl);
    // layer 2: the accumulators start at the bias
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = vec4(s.vec + V_B1, t, q);
    tail_gemm<8, 4>(v, w1s, w1s + W1_HALVES, hh, hl, lane);
    ln_relu_split(v, s.vec + V_G2, s.vec + V_BE2, q, hh, hl);
  }
  __syncthreads();   // every tail wavefront is past layer 2: x tiles and W1 are dead
#pragma unroll
  for (int i = 0; i < WH_CH; ++i) reinterpret_cast<u32x4*>(s.xw)[threadIdx.x + NTHR * i] = whv[i];
  __syncthreads();
  if (!tail) return;   // no barrier below

  // ---------------- heads: 128 -> 192 (+ bias, ReLU), then 192 -> 8 (block diagonal)
  // (accumulators start at the biases; lanes q >= 2 of the output tile hold
  // its 8 padding rows, seeded with bf[0..7] and never read)
  half8 yh[6], yl[6];
  floatx4 o[1] = {vec4(s.vec + V_BF, 0, q & 1)};
  {
    floatx4 a3[12];
#pragma unroll
    for (int t = 0; t < 12; ++t) a3[t] = vec4(s.vec + V_BH, t, q);
    tail_gemm<12, 4>(a3, s.xw, s.xw + WH_HALVES, hh, hl, lane);
#pragma unroll
    for (int t = 0; t < 12; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        split_into(fmaxf(a3[t][j], 0.0f), yh[t >> 1], yl[t >> 1], 4 * (t & 1) + j);
  }
  tail_gemm<1, 6>(o, s.wf, s.wf + WF_HALVES, yh, yl, lane);

  // ---------------- outputs and sampling: lanes r and r + 16 own row 16w + r
  // (outputs 0-3 in lane r, 4-7 in lane r + 16)
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
    const size_t oo = (size_t)srow * oslots + oslot;
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

// ---------------------------------------------------------------------------
// Large forward batches (no sampling): mlp_fwd_kernel.
//
// Workgroup = 8 wavefronts = FWD_ROWS = 256 rows of one player; wavefront w
// owns row tiles 2w, 2w+1 (rows 32w .. 32w+31) with all 128 features, so
// layer 1 needs no partial-sum exchange and the tail starts from the
// accumulators.  Layer 1: the observation B fragments go straight from HBM
// into registers (a lane's 16 halves of one 64-K block are 32 contiguous
// bytes of its row, read as two 16-byte loads at the row's 4-byte
// alignment).  Layer 1 walks K in steps of FWD_KPS = 1 block (128 bytes of
// each of the 256 rows), loaded FWD_PD = 1 step ahead.  Wider steps, deeper
// rings and non-temporal observation loads were all measured slower
// (4.19 M rows: 5.52 ms as built; two-block steps 6.08, rings of 2/3/4
// steps 6.07/5.95/6.03, non-temporal loads 9.07; likely causes, not
// measured: more in-flight observation lines of an XCD's 32 workgroups
// crowd W0 out of its L2, and non-temporal loads lose the L2's merging of a
// row's 16-byte requests into 128-byte lines).  W0's 16 KB per K block is
// loaded by the wavefront of each feature tile and shared through a
// double-buffered LDS stage (planes [block][tile][lo|hi][lane][8]: a
// wavefront's 16-byte reads are 1 KB contiguous, conflict-free).  One
// barrier per step.  The tail runs both row tiles of a wavefront together,
// so every later-layer weight fragment read from LDS feeds two products.
constexpr int FWD_RT = 16, FWD_ROWS = 16 * FWD_RT;
#ifndef QQT_FWD_KPS
#define QQT_FWD_KPS 1
#endif
#ifndef QQT_FWD_PD
#define QQT_FWD_PD 1
#endif
constexpr int FWD_KPS = QQT_FWD_KPS;    // K blocks per step
constexpr int FWD_PD = QQT_FWD_PD;      // steps of loads in flight (register ring depth)
constexpr int W0_BLOCK = 8 * 2 * 64 * 8;          // halves of one K block of W0 (16 KB)
constexpr int W0_STAGE = FWD_KPS * W0_BLOCK;      // halves of one step's stage

// [W0 stage 0 | W0 stage 1] during layer 1, then W1 (hi | lo) for layer 2,
// then the head weights (hi | lo)
// (the first-layer-only launch needs the W0 stages and the biases alone: 36
// KB instead of 114, so more than one workgroup fits on a CU)
template <bool Z1>
struct __align__(16) FwdLds {
  static constexpr int BIG = Z1 ? 2 * W0_STAGE
                                : (2 * W0_STAGE > 2 * WH_HALVES ? 2 * W0_STAGE : 2 * WH_HALVES);
  static_assert(Z1 || BIG >= 2 * W1_HALVES, "W1 reuses the stages");
  uint16_t big[BIG];
  uint16_t wf[Z1 ? 8 : 2 * WF_HALVES];
  float vec[V_N];
};

// acc[r][t] += W(tile t) h_r over KS K steps for R row tiles that share every
// weight fragment read (layout as tail_gemm).
template <int NT, int KS, int R>
__device__ __forceinline__ void tail_gemm_rows(floatx4 (&acc)[R][NT], const uint16_t* a_hi,
                                               const uint16_t* a_lo, const half8 (&bh)[R][KS],
                                               const half8 (&bl)[R][KS], int lane) {
  constexpr int G = NT < 2 ? NT : 2;
  static_assert(NT % G == 0, "whole chunks");
  constexpr int NG = NT / G, NC = KS * NG;
  half8 fa[2][2][G];
  auto fetch = [&](int c, half8 (&f)[2][G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int off = (((G * (c % NG) + g) * KS + c / NG) * 64 + lane) * 8;
      f[0][g] = *reinterpret_cast<const half8*>(a_hi + off);
      f[1][g] = *reinterpret_cast<const half8*>(a_lo + off);
    }
  };
  fetch(0, fa[0]);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c + 1 < NC) fetch(c + 1, fa[(c + 1) & 1]);
    const int s = c / NG, t0 = G * (c % NG);
    const half8 (&f)[2][G] = fa[c & 1];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][t0 + g] = mfma(f[0][g], bh[r][s], acc[r][t0 + g]);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][t0 + g] = mfma(f[0][g], bl[r][s], acc[r][t0 + g]);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][t0 + g] = mfma(f[1][g], bh[r][s], acc[r][t0 + g]);
  }
}

// f(std::integral_constant<int, J>) for each J of the sequence, in order.
template <int... J, class F>
__device__ __forceinline__ void for_each_index(std::integer_sequence<int, J...>, F&& f) {
  (f(std::integral_constant<int, J>{}), ...);
}

template <bool Z1>
__global__ __launch_bounds__(NTHR) void mlp_fwd_kernel(const qqt_mlp_args a) {
  constexpr int W1_CH = 2 * W1_HALVES / 8 / NTHR;
  constexpr int WH_CH = 2 * WH_HALVES / 8 / NTHR;
  constexpr int WF_CH = 2 * WF_HALVES / 8;
  __shared__ FwdLds<Z1> s;
  const int nrb = (a.batch + FWD_ROWS - 1) / FWD_ROWS;
  const int xcd = blockIdx.x & 7, seq = blockIdx.x >> 3;
  const int slot = seq % a.npid;
  const int rb = (seq / a.npid) * 8 + xcd;
  if (rb >= nrb) return;                   // padding workgroup (uniform, before any barrier)
  const int pid = a.npid == 2 ? slot : a.pid0;
  const int row0 = rb * FWD_ROWS;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;
  const int oslot = a.npid == 2 ? slot : a.out_slot;
  uint16_t* const w1s = s.big;

  auto vec_src = [&](int i) -> const float* {
    return i < V_G1 ? a.b0 + (i - V_B0) : i < V_BE1 ? a.ln1_w + (i - V_G1)
         : i < V_B1 ? a.ln1_b + (i - V_BE1) : i < V_G2 ? a.b1 + (i - V_B1)
         : i < V_BE2 ? a.ln2_w + (i - V_G2) : i < V_BH ? a.ln2_b + (i - V_BE2)
         : i < V_BF ? a.bh + (i - V_BH) : a.bf + (i - V_BF);
  };
  const int vi0 = threadIdx.x, vi1 = threadIdx.x + NTHR;
  const float vv0 = *vec_src(vi0);
  const float vv1 = vi1 < V_N ? *vec_src(vi1) : 0.0f;
  auto plane_src = [](const uint16_t* hi, const uint16_t* lo, int halves, int c) {
    const int per = halves / 8;
    return c < per ? reinterpret_cast<const u32x4*>(hi) + c
                   : reinterpret_cast<const u32x4*>(lo) + (c - per);
  };

  // ---------------- layer 1
  const int nkb = a.kblocks0;
  const int k0 = a.k0;
  constexpr int KPS = FWD_KPS;
  const int nsteps = (nkb + KPS - 1) / KPS, last_s = nsteps - 1;
  // W0: wavefront w loads feature tile w of each K block (32 bytes per lane);
  // blocks past the last (a step's padding) reload the last block, which
  // meets all-zero observation halves
  const uint16_t* const wsrc = a.w0 + (size_t)((pid * 8 + w) * nkb) * 64 * 16 + lane * 16;
  auto load_w = [&](int st, u32x4 (&wr)[KPS][2]) {
#pragma unroll
    for (int b = 0; b < KPS; ++b) {
      const u32x4* p =
          reinterpret_cast<const u32x4*>(wsrc + (size_t)min(KPS * st + b, nkb - 1) * 64 * 16);
      wr[b][0] = p[0];
      wr[b][1] = p[1];
    }
  };
  auto store_w = [&](const u32x4 (&wr)[KPS][2], int buf) {
    u32x4* stg = reinterpret_cast<u32x4*>(s.big + buf * W0_STAGE);
#pragma unroll
    for (int b = 0; b < KPS; ++b) {
      stg[((b * 8 + w) * 2 + 0) * 64 + lane] = wr[b][0];
      stg[((b * 8 + w) * 2 + 1) * 64 + lane] = wr[b][1];
    }
  };
  // x: row tile rt of this wavefront, row clamped to the batch (a ragged last
  // block computes copies of the last row and drops them)
  const uint16_t* xrow[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = min(row0 + 32 * w + 16 * rt + r16, a.batch - 1);
    xrow[rt] = a.obs + obs_row(a, r) * a.obs_stride;
  }
  // Chunk h (8 halves from k = 64kb + 16q + 8h) of this lane's rows.  Every
  // step but the last reads whole chunks below k0 (its blocks end at or
  // before 64 KPS (nsteps - 1) <= 64 (nkb - 1) < k0), at a per-lane base and
  // compile-time offsets.  The last step reads each chunk from
  // off = min(k, k0 - 8), which always ends inside the row, and, when it is
  // used, shifts it down by (k - off) / 2 words with zeros shifted in, so
  // halves at or past k0 (k0 is even: a word never straddles it) become zero
  // (a step's padding block entirely).  (The shift is applied at use so that
  // no load is waited on before its step.)
  const uint16_t* const xlane[2] = {xrow[0] + 16 * q, xrow[1] + 16 * q};
  auto chunk_off = [&](int kb, int h) { return min(64 * kb + 16 * q + 8 * h, k0 - 8); };
  auto load_x = [&](int st, u32x4 (&xr)[KPS][2][2]) {
    if (st < last_s) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int b = 0; b < KPS; ++b)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            __builtin_memcpy(&xr[b][rt][h], xlane[rt] + 64 * (KPS * st + b) + 8 * h, 16);
    } else {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int b = 0; b < KPS; ++b)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            __builtin_memcpy(&xr[b][rt][h], xrow[rt] + chunk_off(KPS * st + b, h), 16);
    }
  };
  auto shifted = [&](int kb, int h, const u32x4& v) {
    const int sh = min((64 * kb + 16 * q + 8 * h - chunk_off(kb, h)) >> 1, 4);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t e = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i + j < 4) e = sh == j ? v[i + j] : e;
      o[i] = e;
    }
    return o;
  };

  floatx4 acc[2][8];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[rt][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // Register rings of PD steps for the observation chunks and the W0
  // fragments: step st computes from ring slot st % PD, then refills that
  // slot with step st + PD's chunks, stores step st + 1's W0 (in slot
  // (st + 1) % PD) to the other LDS stage and refills its slot with step
  // st + 1 + PD's.  Each W0 load is issued before the chunks of the step
  // after it, so the in-order wait for a W0 slot never waits for chunks that
  // are needed later.  Prefetch steps are clamped to the last step (those
  // reloads are never used).
  constexpr int PD = FWD_PD;
  u32x4 xr[PD][KPS][2][2];
  u32x4 wr[PD][KPS][2];
#pragma unroll
  for (int j = 0; j < PD; ++j) {
    load_w(min(j, last_s), wr[j]);
    load_x(min(j, last_s), xr[j]);
  }
  u32x4 wfv[2];
  const int wc1 = threadIdx.x + NTHR;
  if constexpr (!Z1) {
    wfv[0] = *plane_src(a.wf, a.wf_lo, WF_HALVES, threadIdx.x);
    wfv[1] = wc1 < WF_CH ? *plane_src(a.wf, a.wf_lo, WF_HALVES, wc1) : u32x4{0u, 0u, 0u, 0u};
  }
  s.vec[vi0] = vv0;
  if (vi1 < V_N) s.vec[vi1] = vv1;
  store_w(wr[0], 0);
  load_w(min(PD, last_s), wr[0]);
  if constexpr (!Z1) {
    reinterpret_cast<u32x4*>(s.wf)[threadIdx.x] = wfv[0];
    if (wc1 < WF_CH) reinterpret_cast<u32x4*>(s.wf)[wc1] = wfv[1];
  }
  __syncthreads();

  auto compute = [&](int st, const u32x4 (&xraw)[KPS][2][2], auto last) {
#pragma unroll
    for (int b = 0; b < KPS; ++b) {
      const int kb = KPS * st + b;
      const half8* stg = reinterpret_cast<const half8*>(s.big + (st & 1) * W0_STAGE + b * W0_BLOCK);
      u32x4 x[2][2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int h = 0; h < 2; ++h) x[rt][h] = last ? shifted(kb, h, xraw[b][rt][h]) : xraw[b][rt][h];
#pragma unroll
      for (int tp = 0; tp < 4; ++tp) {       // feature tiles 2tp, 2tp+1
        half8 f[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          f[u][0] = stg[((2 * tp + u) * 2 + 0) * 64 + lane];
          f[u][1] = stg[((2 * tp + u) * 2 + 1) * 64 + lane];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
              acc[rt][2 * tp + u] = mfma(f[u][h], as_h8(x[rt][h]), acc[rt][2 * tp + u]);
      }
    }
  };

  // Step st (ring slot j = st % PD, W0 stage st & 1); every step but the
  // last, which only computes.
  auto step = [&](int st, auto jc) {
    constexpr int j = decltype(jc)::value;
    compute(st, xr[j], std::false_type{});
    load_x(min(st + PD, last_s), xr[j]);
    store_w(wr[(j + 1) % PD], (st + 1) & 1);
    load_w(min(st + 1 + PD, last_s), wr[(j + 1) % PD]);
    __syncthreads();
  };
  auto unrolled = [&](auto f) { for_each_index(std::make_integer_sequence<int, PD>{}, f); };
  int st0 = 0;
  for (; st0 + PD <= last_s; st0 += PD) unrolled([&](auto jc) { step(st0 + jc, jc); });
  unrolled([&](auto jc) {
    if (st0 + jc < last_s) step(st0 + jc, jc);
  });
  unrolled([&](auto jc) {
    if (st0 + jc == last_s) compute(last_s, xr[jc], std::true_type{});
  });
  __syncthreads();   // every wavefront is past its last read of the W0 stages

  if constexpr (Z1) {   // first layer only (the training forward): z1 = f + b0
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int row = 32 * w + 16 * rt + r16, orow = row0 + row;
      if (orow < a.batch) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const floatx4 b = vec4(s.vec + V_B0, t, q);
          *reinterpret_cast<float4*>(a.z1_out + (size_t)orow * HID + 16 * t + 4 * q) =
              make_float4(acc[rt][t][0] + b[0], acc[rt][t][1] + b[1], acc[rt][t][2] + b[2],
                          acc[rt][t][3] + b[3]);
        }
      }
    }
    return;
  }

  // ---------------- LayerNorm 1, layer 2, LayerNorm 2 on both row tiles.
  // W1 goes over the W0 stages (every wavefront is past its last read of
  // them: the loop ends with a barrier); its loads overlap LayerNorm 1.
  {
    u32x4 w1v[W1_CH];
#pragma unroll
    for (int c = 0; c < W1_CH; ++c)
      w1v[c] = *plane_src(a.w1, a.w1_lo, W1_HALVES, threadIdx.x + NTHR * c);
#pragma unroll
    for (int c = 0; c < W1_CH; ++c) reinterpret_cast<u32x4*>(w1s)[threadIdx.x + NTHR * c] = w1v[c];
  }
  half8 hh[2][4], hl[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    floatx4 v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = acc[rt][t] + vec4(s.vec + V_B0, t, q);
    ln_relu_split(v, s.vec + V_G1, s.vec + V_BE1, q, hh[rt], hl[rt]);
  }
  __syncthreads();
  {
    floatx4 v2[2][8];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 8; ++t) v2[rt][t] = vec4(s.vec + V_B1, t, q);
    tail_gemm_rows<8, 4, 2>(v2, w1s, w1s + W1_HALVES, hh, hl, lane);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) ln_relu_split(v2[rt], s.vec + V_G2, s.vec + V_BE2, q, hh[rt], hl[rt]);
  }
  // head weights over W1 once every wavefront is past layer 2
  {
    u32x4 whv[WH_CH];
#pragma unroll
    for (int i = 0; i < WH_CH; ++i) whv[i] = *plane_src(a.wh, a.wh_lo, WH_HALVES, threadIdx.x + NTHR * i);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < WH_CH; ++i) reinterpret_cast<u32x4*>(s.big)[threadIdx.x + NTHR * i] = whv[i];
  }
  __syncthreads();

  // ---------------- heads: 128 -> 192 (+ bias, ReLU), then 192 -> 8 (block diagonal)
  half8 yh[2][6], yl[2][6];
  floatx4 o[2][1];
  {
    floatx4 a3[2][12];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 12; ++t) a3[rt][t] = vec4(s.vec + V_BH, t, q);
    tail_gemm_rows<12, 4, 2>(a3, s.big, s.big + WH_HALVES, hh, hl, lane);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 12; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          split_into(fmaxf(a3[rt][t][j], 0.0f), yh[rt][t >> 1], yl[rt][t >> 1], 4 * (t & 1) + j);
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) o[rt][0] = vec4(s.vec + V_BF, 0, q & 1);
  tail_gemm_rows<1, 6, 2>(o, s.wf, s.wf + WF_HALVES, yh, yl, lane);

  // outputs: lanes r (outputs 0-3) and r + 16 (outputs 4-7) of each row tile
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int orow = row0 + 32 * w + 16 * rt + r16;
    if (q < 2 && orow < a.batch) {
      const size_t oo = (size_t)orow * oslots + oslot;
      if (a.logits_out) {
        float* lo = a.logits_out + oo * NOUT + 4 * q;
        if ((reinterpret_cast<uintptr_t>(a.logits_out) & 15u) == 0u)   // one 16-byte store
          *reinterpret_cast<float4*>(lo) = make_float4(o[rt][0][0], o[rt][0][1], o[rt][0][2], o[rt][0][3]);
        else
#pragma unroll
          for (int j = 0; j < 4; ++j) lo[j] = o[rt][0][j];
      }
      if (q == 1 && a.value_out) a.value_out[oo] = o[rt][0][3];
    }
  }
}

extern thread_local char g_err[512];

}  // namespace qqt

extern "C" {

int qqt_mlp_act(const qqt_mlp_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!a || !a->obs || !a->w0 || !a->w1 || !a->wh || !a->wf || !a->w1_lo || !a->wh_lo ||
      !a->wf_lo || !a->b0 || !a->ln1_w ||
      !a->ln1_b || !a->b1 || !a->ln2_w || !a->ln2_b || !a->bh || !a->bf) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: null pointer argument");
    return QQT_E_ARG;
  }
  if (a->batch <= 0 || (a->npid != 1 && a->npid != 2) || a->w0_players < a->npid ||
      a->w0_players > 4 || a->pid0 < 0 || (a->npid == 1 && a->pid0 >= a->w0_players) ||
      a->k0 <= 0 || a->k0 % 2 || a->kblocks0 != (a->k0 + 63) / 64 || a->obs_stride < a->k0 ||
      (a->obs_stride % 2) || (((uintptr_t)a->obs) & 3)) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: bad shape/stride/alignment");
    return QQT_E_ARG;
  }
  {
    const int oslots = a->out_slots > 0 ? a->out_slots : a->npid;
    if (a->out_slots < 0 || oslots < a->npid || oslots > 4 || a->out_slot < 0 ||
        (a->npid == 1 && a->out_slot >= oslots)) {
      snprintf(g_err, sizeof(g_err), "qqt_mlp_act: bad output slots");
      return QQT_E_ARG;
    }
  }
  if (a->sample && (!a->move_mask || !a->bomb_mask)) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: sampling needs masks");
    return QQT_E_ARG;
  }
  if (a->row_index && (a->obs_rows <= 0 || (((uintptr_t)a->row_index) & 7))) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: row_index needs obs_rows > 0 and 8-byte alignment");
    return QQT_E_ARG;
  }
  if (a->z1_out && (a->npid != 1 || a->sample || (((uintptr_t)a->z1_out) & 15))) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: z1_out needs npid 1, no sampling, 16-byte alignment");
    return QQT_E_ARG;
  }
  // one workgroup per (row block, player); row blocks are dealt to the 8
  // XCDs round robin with both players' workgroups adjacent on one XCD.
  // Large forward batches take the streaming kernel's 256-row blocks (W0
  // streamed once per 256 rows); everything else XCD row blocks.
  const bool big = !a->sample && a->batch >= MLP_BIG_ROWS && a->k0 >= 64;   // (the streaming
  // kernel's boundary loads read the 8 halves before k0)
  hipStream_t st = (hipStream_t)stream;
  if (!big && mlp_sparse_eligible(*a)) {
    mlp_sparse_launch(*a, st);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      snprintf(g_err, sizeof(g_err), "mlp launch failed: %s", hipGetErrorString(err));
      return QQT_E_LAUNCH;
    }
    return QQT_OK;
  }
  const int rows_wg = big ? FWD_ROWS : XCD_ROWS;
  const int nrb = (a->batch + rows_wg - 1) / rows_wg;
  // one-player rollout launches: two workgroups (half blocks) per XCD row block
  const bool half = !big && !a->z1_out && a->npid == 1;
  const int blocks = ((nrb + 7) / 8) * 8 * a->npid * (half ? 2 : 1);
  if (a->z1_out && big)
    QQT_LAUNCH(QQT_KERNEL_MLP, mlp_fwd_kernel<true>, dim3(blocks), dim3(NTHR), st, *a);
  else if (a->z1_out)
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<RT_SMALL, true>), dim3(blocks), dim3(NTHR), st, *a);
  else if (big)
    QQT_LAUNCH(QQT_KERNEL_MLP, mlp_fwd_kernel<false>, dim3(blocks), dim3(NTHR), st, *a);
  else if (half)
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<RT_HALF, false, true>), dim3(blocks), dim3(NTHR),
               st, *a);
  else
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<RT_SMALL, false>), dim3(blocks), dim3(NTHR), st,
               *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "mlp launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
