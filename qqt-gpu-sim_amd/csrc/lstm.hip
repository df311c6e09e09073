// The lstm arch on gfx950: per-player local features and the actor/critic
// step.
//
// lstm_feat_kernel (sim/obs.py:243-340 local_view_features): one wavefront
// per env.  The env's bomb cells come from a ballot over its fuse bytes; each
// player ranks them by (L1 distance to its centre cell, cell index) with one
// bomb per lane counting the keys below its own, so slot j holds the bomb of
// rank j; slots past the last bomb take the lowest-index cells without one.
// The 7x7 windows are gathered one float16 per lane from the env's
// observation row (L2-hot: the tick kernel wrote it).
//
// lstm_act_kernel (train/model.py:103-120, 176-185, 198-214): one workgroup
// of eight wavefronts (two per SIMD) per 16 or 24 rows.  Every product runs
// on v_mfma_f32_16x16x32_f16 with float32-level accuracy (within 5e-6 of the
// float32 module): float32 operands split into float16 hi + lo, each
// product taken as hi*hi + hi*lo + lo*hi with float32 accumulation (the
// float16 features need no lo part).  The split saturates at 65504, so
// larger activations stay finite, their remainder at float16 precision.  A: lane l
// holds row l%16, k = 8(l/16) .. + 7; B: k = 8(l/16) .. + 7 of column l%16;
// D: lane l holds D[4(l/16)+j][l%16].
// * Trunk, four rows at a time: the windows sit in LDS as zero-bordered 9 x 9
//   grids with a position's channels contiguous, so with K ordered tap-major
//   (k = tap * channels + channel) one K step of 32 is one 16-byte read per
//   lane at a per-lane base plus an immediate.  Each wavefront holds the hi
//   / lo fragments of its output-column tile of both convolutions in
//   registers for the whole launch.  conv1 runs over the 4 x 49 positions
//   and writes a second bordered grid (hi and lo planes); conv2 runs only at
//   the 36 positions per row that the 2x2 max pool reads (7 -> 3 drops row
//   and column 6), ordered so that each output lane's four values are one
//   pooling window: the pool is a max over the lane's accumulators.
// * Head, 16 rows at a time (M = 16): Linear(576,128), the rel and glob
//   MLPs, the fusion layer, the LSTM gates (K = 256 inputs + 128 hidden, N =
//   512, gate order i, f, g, o as torch.nn.LSTM stores them; each wavefront
//   takes the same 16 hidden units of all four gates, so the cell update
//   happens in registers), the three heads and the block-diagonal output
//   layer.  Weights come from L2 as hi / lo B fragments (16 bytes per lane
//   per K step), activations from LDS hi / lo planes whose row pitch is an
//   odd number of 16-byte chunks (the 16 rows of one read hit distinct bank
//   groups); then masked sampling, one thread per row.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "pipeline.h"
#include "qqt_hip.h"

namespace qqt {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

namespace lstm {

constexpr int MAX_T = 10, GLOB = 5, K7 = 7, HALF = 3;
constexpr int HID = 128, HEAD = 64;
constexpr int C_MAX = 14;                 // observation channels the packing allows
constexpr int CS1 = 16;                   // channel slots per conv1 tap (C_MAX used)
constexpr int K1 = 9 * CS1;               // conv1 K: tap-major, k = tap * 16 + channel
constexpr int K2 = 9 * 32;                // conv2 K: tap-major, k = tap * 32 + channel
constexpr int KS1 = (K1 + 31) / 32;       // conv1 K steps of 32 (the last half padding)
constexpr int KS2 = K2 / 32;              // conv2 K steps of 32 (one tap each)
// channel pitch (halves) of the position-major trunk planes: 16-byte
// aligned, chosen for few LDS bank conflicts of the 16-byte A reads
constexpr int CP1 = 24, CP2 = 40;
constexpr int FEAT = 576;                 // 64 x 3 x 3 pooled features
constexpr int XIN = 168;                  // 128 + 32 + 8 fusion inputs
constexpr int XINP = 192;                 // padded to whole 32-k MFMA steps
constexpr int GK = 32;                    // glob layers' K, padded likewise
constexpr int G4 = 512;                   // 4 x 128 gates
constexpr int NW = 8;                     // wavefronts per workgroup (two per SIMD)
constexpr int NTHR = 64 * NW;
constexpr int RG = 4;                     // rows per trunk group
constexpr int M1T = (RG * 49 + 15) / 16;  // conv1 position tiles per group (13)
constexpr int T1 = (M1T + 3) / 4;         // conv1 tiles per wavefront (four per column tile)
constexpr int M2T = RG * 36 / 16;         // conv2 pooled-position tiles per group (9)
constexpr int T2 = (M2T + 1) / 2;         // conv2 tiles per wavefront (two per column tile)
static_assert(RG * 36 % 16 == 0, "whole conv2 tiles per group");
// row pitches (halves) of the head's 16-row float16 planes: an odd number
// of 16-byte chunks, so the 16 rows of one 16-byte A read land in distinct
// bank groups
constexpr int PP = 584, PX = 200, PXH = 392, PHN = 136, PHD = 200, PR = 72, PG = 40;
constexpr int LD_LG = 16;                 // float32 outputs
#ifndef QQT_LSTM_GEMM_D
#define QQT_LSTM_GEMM_D 1
#endif
constexpr int GEMM_D = QQT_LSTM_GEMM_D;   // K steps the head GEMMs' weight fragments load ahead

// packed parameter block (floats; built by qqtsim/policy.py pack_lstm): the
// convolutions k-major [in][out]; each head layer W [K][N] as float16 hi
// and lo planes of K N / 2 floats each, in MFMA B fragments
// [column tile][K / 32][64 lanes][8 halves] (half i of lane 16 q + r in step
// s of tile t = W[32 s + 8 q + i][16 t + r])
constexpr int OFF_C1W = 0, OFF_C1B = OFF_C1W + K1 * 32, OFF_C2W = OFF_C1B + 64,
              OFF_C2B = OFF_C2W + K2 * 64, OFF_FCW = OFF_C2B + 64, OFF_FCB = OFF_FCW + FEAT * 128,
              OFF_R1W = OFF_FCB + 128, OFF_R1B = OFF_R1W + 64 * 64, OFF_R2W = OFF_R1B + 64,
              OFF_R2B = OFF_R2W + 64 * 32, OFF_G1W = OFF_R2B + 64, OFF_G1B = OFF_G1W + GK * 16,
              OFF_G2W = OFF_G1B + 64, OFF_G2B = OFF_G2W + GK * 16, OFF_FUW = OFF_G2B + 64,
              OFF_FUB = OFF_FUW + XINP * 256, OFF_LW = OFF_FUB + 256, OFF_LB = OFF_LW + 384 * G4,
              OFF_HW = OFF_LB + G4, OFF_HB = OFF_HW + 128 * 192, OFF_OW = OFF_HB + 192,
              OFF_OB = OFF_OW + 192 * 16, N_PARAMS = OFF_OB + 64;
static_assert(N_PARAMS == QQT_LSTM_PARAMS, "packed block size");

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }
__device__ __forceinline__ uint16_t f2h(float x) { return __half_as_ushort(__float2half_rn(x)); }

// ---------------------------------------------------------------- features
template <int H, int W, int P>
__global__ __launch_bounds__(64) void lstm_feat_kernel(const qqt_sim_config cf,
                                                       const qqt_lstm_feat_args a) {
  constexpr int C = H * W, NCH = 5 * P + 4, SLOTS = MAX_T - (P - 1);
  static_assert(SLOTS > 0 && SLOTS <= 64 && C <= 4 * 64, "slot and cell counts");
  const int g = blockIdx.x, lane = threadIdx.x;
  if (g >= a.n_envs) return;
  __shared__ uint8_t bomb_cell[C];
  __shared__ uint16_t relbuf[MAX_T * 6];
  __shared__ int nbomb;
  const int32_t* cells = a.cells + (size_t)g * C;
  const int32_t* pl = a.players + (size_t)g * P * QQT_P_SLOTS;
  const uint16_t* obs = a.obs + (size_t)g * NCH * C;
  // bomb list in ascending cell index, fuse total
  int fsum = 0, base = 0;
  for (int c0 = 0; c0 < C; c0 += 64) {
    const int c = c0 + lane;
    const int f = c < C ? (cells[c] & 0xFF) : 0;
    fsum += f;
    const uint64_t m = __ballot(f > 0);
    if (f > 0) bomb_cell[base + __popcll(m & ((1ull << lane) - 1ull))] = (uint8_t)c;
    base += __popcll(m);
  }
  for (int o = 32; o >= 1; o >>= 1) fsum += __shfl_xor(fsum, o, 64);
  if (lane == 0) nbomb = base;
  __syncthreads();
  const int nb = nbomb;
  // lowest-index cells without a bomb (for slots past the last bomb)
  const uint64_t free0 = __ballot(lane < C && (cells[lane] & 0xFF) == 0);
  const int t = a.envs[(size_t)g * QQT_E_SLOTS + QQT_E_T];
  const float tf = h2f(f2h((float)t));           // t as float16, as the reference casts it
  for (int me = 0; me < a.p_out; ++me) {
    const float py = __int_as_float(pl[me * QQT_P_SLOTS + QQT_P_Y]);
    const float px = __int_as_float(pl[me * QQT_P_SLOTS + QQT_P_X]);
    const int cy = (int)floorf(py), cx = (int)floorf(px);
    // ---- local window
    uint16_t* loc = a.local + (size_t)g * a.local_stride + (size_t)me * NCH * K7 * K7;
    for (int i = lane; i < NCH * K7 * K7; i += 64) {
      const int ch = i / (K7 * K7), r = i % (K7 * K7);
      const int y = cy + r / K7 - HALF, x = cx + r % K7 - HALF;
      loc[i] = (y >= 0 && y < H && x >= 0 && x < W) ? obs[ch * C + y * W + x] : (uint16_t)0;
    }
    // ---- relative targets, assembled in LDS and written once
    uint16_t* rel = relbuf;
    if (lane < MAX_T * 6) rel[lane] = 0;
    __syncthreads();
    if (lane < P - 1) {
      const int opp = (me + lane + 1) % P;
      const float oy = __int_as_float(pl[opp * QQT_P_SLOTS + QQT_P_Y]);
      const float ox = __int_as_float(pl[opp * QQT_P_SLOTS + QQT_P_X]);
      rel[lane * 6 + 0] = f2h(oy - py);
      rel[lane * 6 + 1] = f2h(ox - px);
      rel[lane * 6 + 2] = f2h(pl[opp * QQT_P_SLOTS + QQT_P_ALIVE] ? 1.0f : 0.0f);
    }
    // rank of each bomb by (distance, cell); nb <= H*W, lanes walk the list
    for (int j = lane; j < nb; j += 64) {
      const int c = bomb_cell[j];
      const int key = (abs(c / W - cy) + abs(c % W - cx)) * C + c;
      int rank = 0;
      for (int i = 0; i < nb; ++i) {
        const int ci = bomb_cell[i];
        rank += (abs(ci / W - cy) + abs(ci % W - cx)) * C + ci < key;
      }
      if (rank < SLOTS) {
        uint16_t* s = rel + (P - 1 + rank) * 6;
        s[0] = f2h((float)(c % W) - (float)cx);
        s[1] = f2h((float)(c / W) - (float)cy);
        s[3] = f2h(1.0f);
      }
    }
    if (lane < SLOTS && lane >= nb) {             // the (lane - nb)-th bomb-free cell
      uint64_t m = free0;
      for (int k = 0; k < lane - nb; ++k) m &= m - 1ull;
      const int c = __ffsll((unsigned long long)m) - 1;
      uint16_t* s = rel + (P - 1 + lane) * 6;
      s[0] = f2h((float)(c % W) - (float)cx);
      s[1] = f2h((float)(c / W) - (float)cy);
    }
    __syncthreads();
    if (lane < MAX_T * 6) a.rel[(size_t)g * a.rel_stride + (size_t)me * MAX_T * 6 + lane] = rel[lane];
    // ---- global scalars
    if (lane < GLOB) {
      uint16_t v;
      if (lane == 0) v = f2h(__fdiv_rn(tf, (float)cf.max_steps));
      else if (lane == 1) v = f2h(__fdiv_rn((float)pl[me * QQT_P_SLOTS + QQT_P_HP], (float)cf.max_hp));
      else if (lane == 2) v = obs[(2 * P + 1) * C + min(max(cy, 0), H - 1) * W + min(max(cx, 0), W - 1)];
      else if (lane == 3) v = f2h(__fdiv_rn((float)nb, (float)cf.max_bombs));
      else v = f2h(__fdiv_rn((float)fsum, (float)(cf.max_bombs * cf.fuse)));
      a.glob[(size_t)g * a.glob_stride + (size_t)me * GLOB + lane] = v;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- act
template <int ROWS>
struct __align__(16) ActLds {
  static constexpr int HT = (ROWS + 15) / 16;   // 16-row head tiles
  union {
    struct {                        // trunk: one group of RG rows, zero-bordered 9 x 9 grids
      uint16_t in[RG][81 * CP1];    // float16 windows [position][channel slot]
      uint16_t a1h[RG][81 * CP2];   // conv1 output [position][channel], float16 hi part
      uint16_t a1l[RG][81 * CP2];   // and lo part (v - hi)
    } t;
    struct {                        // head: one 16-row tile; float16 [hi plane][lo plane]
      uint16_t xin[2][16 * PX];     // fc | rel | glob outputs (192 K)
      uint16_t xh[2][16 * PXH];     // fused | previous h (384 K)
      uint16_t hn[2][16 * PHN];     // new h
      uint16_t hd[2][16 * PHD];     // heads' hidden layers
      uint16_t r1[2][16 * PR], g1[2][16 * PG];
      uint16_t rel[16 * PR];        // rel inputs (float16 already; 60 used)
      uint16_t glb[16 * PG];        // glob inputs (5 used)
      float lg[16 * LD_LG];         // outputs
    } h;
  };
  uint16_t pooled[2][HT * 16 * PP]; // 576 pooled features per row, hi and lo
};

// acc[t] += A (16 rows of float16 hi / lo planes in LDS, row pitch lda
// halves) x B over K (a multiple of 32), B's column tile tile(t) read from
// its float16 hi / lo fragments F (N columns).  Per K step: one 16-byte A
// read per plane (row r, k = 32 s + 8 q .. + 7) and one 16-byte fragment
// read per plane and tile feed hi*hi + hi*lo + lo*hi (LO = false: the A
// values are float16 exactly, hi*hi + hi*lo).
template <int NT, bool LO, int K, int N, class Tile>
__device__ __forceinline__ void gemmh(floatx4 (&acc)[NT], const uint16_t* Ah, const uint16_t* Al,
                                      int lda, const float* F, Tile tile, int lane) {
  static_assert(K % 32 == 0, "whole K steps");
  constexpr int ks = K / 32;
  const int r = lane & 15, q = lane >> 4;
  // the fragments' hi plane, then the lo plane, K * N halves each; loaded
  // GEMM_D steps ahead
  const Rsrc fr = rsrc(F, (uint32_t)K * N * 4);
  const uint16_t* ah = Ah + r * lda + 8 * q;
  const uint16_t* al = Al + r * lda + 8 * q;
  struct Frag { half8 h[NT], l[NT]; };
  pipeline<ks, GEMM_D>(
      [&](int st) {
        Frag f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const uint32_t o = (uint32_t)(((tile(t) * ks + st) * 64 + lane) * 16);
          f.h[t] = bld16<half8>(fr, o);
          f.l[t] = bld16<half8>(fr, o + (uint32_t)K * N * 2);
        }
        return f;
      },
      [&](int st, const Frag& f) {
        const half8 xh = *reinterpret_cast<const half8*>(ah + 32 * st);
        half8 xl;
        if constexpr (LO) xl = *reinterpret_cast<const half8*>(al + 32 * st);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          acc[t] = mfma16(xh, f.h[t], acc[t]);
          acc[t] = mfma16(xh, f.l[t], acc[t]);
          if constexpr (LO) acc[t] = mfma16(xl, f.h[t], acc[t]);
        }
      });
}

// NT consecutive column tiles from t0
struct Tiles {
  int t0;
  __device__ int operator()(int t) const { return t0 + t; }
};

// float32 v as float16 hi + lo (hi*w + lo*w carries v's product to float32
// accuracy for |v| <= 65504).  Saturating: past float16's range hi stays at
// +-65504 and lo takes the (clamped) remainder, so a large activation gives
// a large finite product instead of inf - inf = NaN; exact in hi + lo up to
// |v| = 131008, clamped beyond.
__device__ __forceinline__ void split16(float v, _Float16& hi, _Float16& lo) {
  constexpr float HMAX = 65504.0f;
  hi = (_Float16)fminf(fmaxf(v, -HMAX), HMAX);
  lo = (_Float16)fminf(fmaxf(v - (float)hi, -HMAX), HMAX);
}

// float32 v as float16 hi + lo into a plane pair
__device__ __forceinline__ void put_split(uint16_t* h, uint16_t* l, int at, float v) {
  _Float16 hi, lo;
  split16(v, hi, lo);
  h[at] = __half_as_ushort(hi);
  l[at] = __half_as_ushort(lo);
}

// bias + optional ReLU of the output tiles, split into a float16 plane pair
template <int NT>
__device__ __forceinline__ void store16h(const floatx4 (&acc)[NT], uint16_t* Dh, uint16_t* Dl,
                                         int ldd, int n0, const float* bias, int lane, int ncols) {
  const int c = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = n0 + 16 * t + c;
    if (n >= ncols) continue;
    const float b = bias[n];
#pragma unroll
    for (int j = 0; j < 4; ++j) put_split(Dh, Dl, (4 * q + j) * ldd + n, fmaxf(acc[t][j] + b, 0.0f));
  }
}

// bias + optional ReLU of the output tiles into a row-major LDS block
template <int NT>
__device__ __forceinline__ void store16(const floatx4 (&acc)[NT], float* D, int ldd, int n0,
                                        const float* bias, bool relu, int lane, int ncols) {
  const int c = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = n0 + 16 * t + c;
    if (n >= ncols) continue;
    const float b = bias[n];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = acc[t][j] + b;
      D[(4 * q + j) * ldd + n] = relu ? fmaxf(v, 0.0f) : v;
    }
  }
}

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ int tapoff(int tap) { return (tap / 3) * 9 + tap % 3; }

// ROWS rows per workgroup: the trunk in groups of RG rows, the head in
// 16-row tiles.
template <int ROWS>
__global__ __launch_bounds__(NTHR) void lstm_act_kernel(const qqt_lstm_args a) {
  static_assert(ROWS % RG == 0, "whole trunk groups");
  using L = ActLds<ROWS>;
  constexpr int HT = L::HT;
  __shared__ L s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, q = lane >> 4;
  const int row0 = blockIdx.x * ROWS;
  const float* P = a.params;
  const int cin = a.c_in;

  // The trunk multiplies on v_mfma_f32_16x16x32_f16 (A: lane l holds row
  // l%16, k = 8(l/16) .. + 7; B: k = 8(l/16) .. + 7 of column l%16; D as for
  // the float32 MFMA) with float32 accuracy: weights split into float16 hi
  // + lo, conv1's output likewise, and each product taken as hi*hi + hi*lo +
  // lo*hi (the windows are float16 already: two products).  This
  // wavefront's weight fragments stay in registers for the whole trunk:
  // conv1 column tile w & 1 (the four wavefronts w >> 1 take every fourth
  // position tile), conv2 column tile w & 3 (wavefronts w >> 2 take every
  // other position tile).  K step s covers k = 32 s .. 32 s + 31 of the
  // tap-major K (conv1: taps 2s, 2s+1 x 16 channel slots; conv2: tap s x 32
  // channels).
  const int n1 = 16 * (w & 1) + r16, n2 = 16 * (w & 3) + r16;
  half8 b1h[KS1], b1l[KS1], b2h[KS2], b2l[KS2];
#pragma unroll
  for (int st = 0; st < KS1; ++st)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = 32 * st + 8 * q + i;
      const float v = k < K1 ? P[OFF_C1W + k * 32 + n1] : 0.0f;
      _Float16 hi, lo;
      split16(v, hi, lo);
      b1h[st][i] = hi;
      b1l[st][i] = lo;
    }
#pragma unroll
  for (int st = 0; st < KS2; ++st)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = P[OFF_C2W + (32 * st + 8 * q + i) * 64 + n2];
      _Float16 hi, lo;
      split16(v, hi, lo);
      b2h[st][i] = hi;
      b2l[st][i] = lo;
    }
  const float bias1 = P[OFF_C1B + n1], bias2 = P[OFF_C2B + n2];

  // per-lane A-fragment addresses (halves; a K step adds its tap offset).
  // conv1 positions run row-major over the group's 4 x 49 positions; conv2
  // positions are ordered (row, pooling window, position in the window), so
  // each output lane's four values are one 2x2 window.
  auto tile1 = [&](int i) { return 4 * i + (w >> 1); };   // conv1 tile of slot i
  auto tile2 = [&](int i) { return 2 * i + (w >> 2); };   // conv2 tile of slot i
  int base1[T1];
#pragma unroll
  for (int i = 0; i < T1; ++i) {
    const int m = tile1(i) * 16 + r16;
    const bool ok = tile1(i) < M1T && m < RG * 49;     // else a valid dummy row, dropped
    const int rr = ok ? m / 49 : 0, p = ok ? m % 49 : 0;
    base1[i] = (rr * 81 + (p / 7) * 9 + p % 7) * CP1;
  }
  int base2[T2];
  bool ok2[T2];
#pragma unroll
  for (int i = 0; i < T2; ++i) {
    ok2[i] = tile2(i) < M2T;
    const int m = (ok2[i] ? tile2(i) : 0) * 16 + r16;
    const int rr = m / 36, wi = (m % 36) / 4, s4 = m % 4;
    const int y = 2 * (wi / 3) + (s4 >> 1), x = 2 * (wi % 3) + (s4 & 1);
    base2[i] = (rr * 81 + y * 9 + x) * CP2;
  }

  // zero the planes (borders and unused channel slots stay zero) and the
  // pooled rows past ROWS (read by the last head tile, dropped)
  for (int i = tid; i < RG * 81 * CP1 / 2; i += NTHR) reinterpret_cast<uint32_t*>(&s.t.in[0][0])[i] = 0u;
  for (int i = tid; i < RG * 81 * CP2 / 2; i += NTHR) {
    reinterpret_cast<uint32_t*>(&s.t.a1h[0][0])[i] = 0u;
    reinterpret_cast<uint32_t*>(&s.t.a1l[0][0])[i] = 0u;
  }
  for (int i = ROWS * PP + tid; i < HT * 16 * PP; i += NTHR) s.pooled[0][i] = s.pooled[1][i] = 0;
  __syncthreads();

  auto stage = [&](int g) {   // the group's float16 windows into the position-major planes
    const int n = cin * 49;
    for (int i = tid; i < RG * n; i += NTHR) {
      const int rr = i / n, rem = i % n, ci = rem / 49, p = rem % 49;
      const int row = min(row0 + g * RG + rr, a.batch - 1);   // past the batch: computed, dropped
      s.t.in[rr][((p / 7 + 1) * 9 + p % 7 + 1) * CP1 + ci] =
          a.local[(size_t)row * a.local_stride + rem];
    }
  };
  stage(0);
#pragma unroll 1
  for (int g = 0; g < ROWS / RG; ++g) {
    __syncthreads();   // in[] holds group g; a1 is free
    // conv1 (C -> 32, 3x3, pad 1) + ReLU into a1's interior, split hi / lo
    {
      floatx4 acc[T1];
#pragma unroll
      for (int i = 0; i < T1; ++i) acc[i] = floatx4{0, 0, 0, 0};
      const uint16_t* ib = &s.t.in[0][0];
#pragma unroll
      for (int st = 0; st < KS1; ++st) {
        // taps 2st + q/2 (the padding tap 9 reads tap 8 against zero weights)
        const int off = tapoff(min(2 * st + (q >> 1), 8)) * CP1 + 8 * (q & 1);
#pragma unroll
        for (int i = 0; i < T1; ++i) {
          const half8 av = *reinterpret_cast<const half8*>(ib + base1[i] + off);
          acc[i] = mfma16(av, b1h[st], acc[i]);
          acc[i] = mfma16(av, b1l[st], acc[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < T1; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = tile1(i) * 16 + 4 * q + j;
          if (tile1(i) < M1T && m < RG * 49) {
            const int rr = m / 49, p = m % 49;
            const float v = fmaxf(acc[i][j] + bias1, 0.0f);
            const int at = ((p / 7 + 1) * 9 + p % 7 + 1) * CP2 + n1;
            put_split(s.t.a1h[rr], s.t.a1l[rr], at, v);
          }
        }
      }
    }
    __syncthreads();   // a1 complete; in[] free
    if (g + 1 < ROWS / RG) stage(g + 1);
    // conv2 (32 -> 64) at the 36 positions the 2x2 pool reads, ReLU, max pool
    {
      floatx4 acc[T2];
#pragma unroll
      for (int i = 0; i < T2; ++i) acc[i] = floatx4{0, 0, 0, 0};
      const uint16_t* hb = &s.t.a1h[0][0];
      const uint16_t* lb = &s.t.a1l[0][0];
#pragma unroll
      for (int st = 0; st < KS2; ++st) {
        const int off = tapoff(st) * CP2 + 8 * q;
#pragma unroll
        for (int i = 0; i < T2; ++i) {
          const half8 ah = *reinterpret_cast<const half8*>(hb + base2[i] + off);
          const half8 al = *reinterpret_cast<const half8*>(lb + base2[i] + off);
          acc[i] = mfma16(ah, b2h[st], acc[i]);
          acc[i] = mfma16(ah, b2l[st], acc[i]);
          acc[i] = mfma16(al, b2h[st], acc[i]);
        }
      }
      // lane (q, j) of tile t holds window 4 t + q at its position j:
      // max_j relu(v_j + b) = relu(max_j v_j + b)
#pragma unroll
      for (int i = 0; i < T2; ++i) {
        if (!ok2[i]) continue;
        const int wdx = 4 * tile2(i) + q, rr = wdx / 9, w9 = wdx % 9;
        const float mx = fmaxf(fmaxf(acc[i][0], acc[i][1]), fmaxf(acc[i][2], acc[i][3]));
        put_split(s.pooled[0], s.pooled[1], (g * RG + rr) * PP + n2 * 9 + w9,
                  fmaxf(mx + bias2, 0.0f));
      }
    }
  }

#pragma unroll 1
  for (int ht = 0; ht < HT; ++ht) {
    __syncthreads();   // trunk done / previous tile's buffers consumed
    const int hr0 = row0 + 16 * ht;
    // rel / glob inputs (float16 bits as they are), previous hidden state
    // (zero for reset envs) split hi / lo, and the K padding of the layers
    for (int i = tid; i < 16 * 64; i += NTHR) {
      const int r = i / 64, k = i % 64, row = min(hr0 + r, a.batch - 1);
      s.h.rel[r * PR + k] = k < MAX_T * 6 ? a.rel[(size_t)row * a.rel_stride + k] : (uint16_t)0;
    }
    for (int i = tid; i < 16 * GK; i += NTHR) {
      const int r = i / GK, k = i % GK, row = min(hr0 + r, a.batch - 1);
      s.h.glb[r * PG + k] = k < GLOB ? a.glob[(size_t)row * a.glob_stride + k] : (uint16_t)0;
      if (k >= 16) s.h.g1[0][r * PG + k] = s.h.g1[1][r * PG + k] = 0;      // glob2 K padding
      if (k < XINP - XIN) s.h.xin[0][r * PX + XIN + k] = s.h.xin[1][r * PX + XIN + k] = 0;
    }
    for (int i = tid; i < 16 * HID; i += NTHR) {
      const int r = i / HID, k = i % HID, row = min(hr0 + r, a.batch - 1);
      const bool zero = a.reset && a.reset[row / a.rows_per_env];
      put_split(s.h.xh[0], s.h.xh[1], r * PXH + 256 + k, zero ? 0.0f : a.h[(size_t)row * HID + k]);
    }
    // Linear(576, 128) + ReLU: 8 column tiles, one per wavefront
    {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, true, FEAT, HID>(acc, s.pooled[0] + 16 * ht * PP, s.pooled[1] + 16 * ht * PP, PP, P + OFF_FCW,
                     Tiles{w}, lane);
      store16h<1>(acc, s.h.xin[0], s.h.xin[1], PX, 16 * w, P + OFF_FCB, lane, HID);
    }
    __syncthreads();
    // rel 60 -> 64 (wavefronts 0-3), glob 5 -> 16 (wavefront 4)
    if (w < 4) {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, false, 64, 64>(acc, s.h.rel, s.h.rel, PR, P + OFF_R1W, Tiles{w}, lane);
      store16h<1>(acc, s.h.r1[0], s.h.r1[1], PR, 16 * w, P + OFF_R1B, lane, 64);
    } else {
      if (w == 4) {
        floatx4 ag[1] = {floatx4{0, 0, 0, 0}};
        gemmh<1, false, GK, 16>(ag, s.h.glb, s.h.glb, PG, P + OFF_G1W, Tiles{0}, lane);
        store16h<1>(ag, s.h.g1[0], s.h.g1[1], PG, 0, P + OFF_G1B, lane, 16);
      }
    }
    __syncthreads();
    // rel 64 -> 32 (wavefronts 0, 1), glob 16 -> 8 (wavefront 2)
    if (w < 2) {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, true, 64, 32>(acc, s.h.r1[0], s.h.r1[1], PR, P + OFF_R2W, Tiles{w}, lane);
      store16h<1>(acc, s.h.xin[0] + HID, s.h.xin[1] + HID, PX, 16 * w, P + OFF_R2B, lane, 32);
    } else if (w == 2) {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, true, GK, 16>(acc, s.h.g1[0], s.h.g1[1], PG, P + OFF_G2W, Tiles{0}, lane);
      store16h<1>(acc, s.h.xin[0] + HID + 32, s.h.xin[1] + HID + 32, PX, 0, P + OFF_G2B, lane, 8);
    }
    __syncthreads();
    // fusion Linear(168, 256) + ReLU: 16 tiles, two per wavefront
    {
      floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
      gemmh<2, true, XINP, 256>(acc, s.h.xin[0], s.h.xin[1], PX, P + OFF_FUW, Tiles{2 * w}, lane);
      store16h<2>(acc, s.h.xh[0], s.h.xh[1], PXH, 32 * w, P + OFF_FUB, lane, 256);
    }
    __syncthreads();
    // LSTM gates [fused | h] (384) x W (384 x 512) + b.  Wavefront w takes
    // hidden units 16 w .. 16 w + 15 of all four gates (tile t = gate), so
    // each lane holds i, f, g, o of the same (row, unit) and updates the
    // cell in registers.
    {
      floatx4 acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = floatx4{0, 0, 0, 0};
      gemmh<4, true, 384, G4>(acc, s.h.xh[0], s.h.xh[1], PXH, P + OFF_LW,
                     [&](int t) { return 8 * t + w; }, lane);
      {
        const int u = 16 * w + r16;
        const float bi = P[OFF_LB + u], bf = P[OFF_LB + HID + u];
        const float bg = P[OFF_LB + 2 * HID + u], bo = P[OFF_LB + 3 * HID + u];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * q + j, row = hr0 + r;
          const bool mine = 16 * ht + r < ROWS && row < a.batch;
          const float ig = sigm(acc[0][j] + bi), fg = sigm(acc[1][j] + bf);
          const float gg = tanhf(acc[2][j] + bg), og = sigm(acc[3][j] + bo);
          float cp = 0.0f;
          if (mine && !(a.reset && a.reset[row / a.rows_per_env])) cp = a.c[(size_t)row * HID + u];
          const float c2 = fg * cp + ig * gg;
          const float h2 = og * tanhf(c2);
          put_split(s.h.hn[0], s.h.hn[1], r * PHN + u, h2);
          if (mine) {
            a.c[(size_t)row * HID + u] = c2;
            a.h[(size_t)row * HID + u] = h2;
          }
        }
      }
    }
    __syncthreads();
    // heads' hidden layers 128 -> 192 + ReLU: 12 tiles, two per wavefront
    // 0-3 and one per wavefront 4-7
    if (w < 4) {
      floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
      gemmh<2, true, HID, 3 * HEAD>(acc, s.h.hn[0], s.h.hn[1], PHN, P + OFF_HW, Tiles{2 * w}, lane);
      store16h<2>(acc, s.h.hd[0], s.h.hd[1], PHD, 32 * w, P + OFF_HB, lane, 3 * HEAD);
    } else {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, true, HID, 3 * HEAD>(acc, s.h.hn[0], s.h.hn[1], PHN, P + OFF_HW, Tiles{8 + (w - 4)},
                     lane);
      store16h<1>(acc, s.h.hd[0], s.h.hd[1], PHD, 128 + 16 * (w - 4), P + OFF_HB, lane, 3 * HEAD);
    }
    __syncthreads();
    // output layer 192 -> 8 (block diagonal, 16 padded columns): wavefront 0
    if (w == 0) {
      floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
      gemmh<1, true, 3 * HEAD, 16>(acc, s.h.hd[0], s.h.hd[1], PHD, P + OFF_OW, Tiles{0}, lane);
      store16<1>(acc, s.h.lg, LD_LG, 0, P + OFF_OB, false, lane, 16);
    }
    __syncthreads();
    // outputs and masked sampling: one thread per row
    if (tid < 16 && 16 * ht + tid < ROWS && hr0 + tid < a.batch) {
      const int row = hr0 + tid;
      const float* lg = s.h.lg + tid * LD_LG;
      const size_t o = (size_t)row * a.out_stride + a.out_slot;
      if (a.logits_out) {
#pragma unroll
        for (int k = 0; k < 8; ++k) a.logits_out[(size_t)row * 8 + k] = lg[k];
      }
      if (a.value_out) a.value_out[o] = lg[7];
      if (a.sample) {
        const int env = row / a.rows_per_env;
        const int pid = a.rows_per_env == 1 ? a.pid0 : row % a.rows_per_env;
        uint8_t mm[5], bm[2];
#pragma unroll
        for (int k = 0; k < 5; ++k) mm[k] = a.move_mask[(size_t)row * a.mm_row_stride + k];
#pragma unroll
        for (int k = 0; k < 2; ++k) bm[k] = a.bomb_mask[(size_t)row * a.bm_row_stride + k];
        float um, ub;
        if (a.uniforms) {
          um = a.uniforms[(size_t)row * 2 + 0];
          ub = a.uniforms[(size_t)row * 2 + 1];
        } else {
          float u4[4];
          philox_block(a.seed, (uint32_t)env, a.tick, STREAM_POLICY, (uint32_t)((2 * pid) >> 2), u4);
          um = u4[(2 * pid) & 3];
          ub = u4[(2 * pid + 1) & 3];
        }
        float lpm, lpb;
        const int am = sample_masked<5>(lg, mm, um, &lpm);
        const int ab = sample_masked<2>(lg + 5, bm, ub, &lpb);
        if (a.actions) {
          a.actions[o * 2 + 0] = am;
          a.actions[o * 2 + 1] = ab;
        }
        if (a.actions_i8) {
          a.actions_i8[o * 2 + 0] = (int8_t)am;
          a.actions_i8[o * 2 + 1] = (int8_t)ab;
        }
        if (a.logp_out) a.logp_out[o] = lpm + lpb;
      }
    }
  }
}

}  // namespace lstm

extern thread_local char g_err[512];

}  // namespace qqt

extern "C" {

int qqt_lstm_features(const qqt_sim_config* cfg, const qqt_lstm_feat_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!cfg || !a || !a->cells || !a->players || !a->envs || !a->obs || !a->local || !a->rel ||
      !a->glob) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_features: null pointer argument");
    return QQT_E_ARG;
  }
  if (a->n_envs <= 0 || a->p_out < 1 || a->p_out > cfg->n_players || cfg->max_steps <= 0 ||
      cfg->max_hp <= 0 || cfg->max_bombs <= 0 || cfg->fuse <= 0) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_features: bad sizes or config");
    return QQT_E_ARG;
  }
  const int nch = 5 * cfg->n_players + 4;
  if (a->local_stride < (int64_t)a->p_out * nch * 49 || a->rel_stride < (int64_t)a->p_out * 60 ||
      a->glob_stride < (int64_t)a->p_out * 5) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_features: output strides smaller than a row");
    return QQT_E_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  if (cfg->height == 13 && cfg->width == 13 && cfg->n_players == 2) {
    QQT_LAUNCH(QQT_KERNEL_LSTM_FEAT, (lstm::lstm_feat_kernel<13, 13, 2>), dim3(a->n_envs), dim3(64),
               st, *cfg, *a);
  } else {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_features: grid/player combination not compiled");
    return QQT_E_UNSUPPORTED;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "lstm feature launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

int qqt_lstm_act(const qqt_lstm_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!a || !a->local || !a->rel || !a->glob || !a->params || !a->h || !a->c) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_act: null pointer argument");
    return QQT_E_ARG;
  }
  if (a->batch <= 0 || a->c_in <= 0 || a->c_in > lstm::C_MAX || a->rows_per_env < 1 ||
      a->local_stride < (int64_t)a->c_in * 49 || a->rel_stride < 60 || a->glob_stride < 5 ||
      a->out_stride < 1 || a->out_slot < 0 || a->out_slot >= a->out_stride) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_act: bad shape/stride");
    return QQT_E_ARG;
  }
  if (a->sample && (!a->move_mask || !a->bomb_mask)) {
    snprintf(g_err, sizeof(g_err), "qqt_lstm_act: sampling needs masks");
    return QQT_E_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  // 16 or 24 rows per workgroup (one workgroup per CU), whichever needs
  // fewer rounds of the 256 CUs at its cost per workgroup: 24 rows take
  // ~1.8x the time of 16 (1.5x the trunk, a second head tile)
  const int blocks16 = (a->batch + 15) / 16, blocks24 = (a->batch + 23) / 24;
  const int rounds16 = (blocks16 + 255) / 256, rounds24 = (blocks24 + 255) / 256;
  if (rounds24 * 18 < rounds16 * 10)
    QQT_LAUNCH(QQT_KERNEL_LSTM, lstm::lstm_act_kernel<24>, dim3(blocks24), dim3(lstm::NTHR), st, *a);
  else
    QQT_LAUNCH(QQT_KERNEL_LSTM, lstm::lstm_act_kernel<16>, dim3(blocks16), dim3(lstm::NTHR), st, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "lstm act launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
