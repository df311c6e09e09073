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
// of four wavefronts per 16 rows, float32 arithmetic throughout on
// v_mfma_f32_16x16x4_f32 (A: 16 rows x 4 K, B: 4 K x 16 columns; lane l
// supplies A[l%16][l/16] and B[l/16][l%16] and holds D[4(l/16)+j][l%16]).
// * Trunk, one row at a time: the 14 x 7 x 7 window sits in LDS as a zero-
//   bordered 9 x 9 grid per channel; each 3x3 convolution is an implicit GEMM
//   (M = the 49 positions in four tiles, one per wavefront; N = output
//   channels; K = channel x tap) whose A operand is gathered from the grid and
//   whose B operand (the weights, k-major) is staged in LDS for the whole
//   launch.  conv1's output goes to a second zero-bordered grid, conv2's to a
//   7 x 7 plane per channel, and the 2x2 max pool writes the row's 576
//   features into a 16-row tile.
// * Head, the 16 rows together (M = 16): Linear(576,128), the rel and glob
//   MLPs, the fusion layer, the LSTM gates (K = 256 inputs + 128 hidden, N =
//   512, gate order i, f, g, o as torch.nn.LSTM stores them), the cell update,
//   the three heads and the block-diagonal output layer, all from k-major
//   weight blocks read from L2 (each weight once per 16 rows), activations in
//   LDS; then masked sampling, one thread per row.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace lstm {

constexpr int MAX_T = 10, GLOB = 5, K7 = 7, HALF = 3;
constexpr int HID = 128, HEAD = 64;
constexpr int C_MAX = 14;                 // observation channels the packing allows
constexpr int K1 = 128;                   // conv1 K (9 C_MAX = 126, padded)
constexpr int K2 = 288;                   // conv2 K (9 x 32)
constexpr int FEAT = 576;                 // 64 x 3 x 3 pooled features
constexpr int XIN = 168;                  // 128 + 32 + 8 fusion inputs
constexpr int XH = 384;                   // 256 fused + 128 hidden: LSTM inputs
constexpr int G4 = 512;                   // 4 x 128 gates
constexpr int ROWS = 16;                  // rows per workgroup
constexpr int NTHR = 256;

// packed parameter block (floats; built by qqtsim/policy.py pack_lstm), all
// weights k-major [in][out]
constexpr int OFF_C1W = 0, OFF_C1B = 4096, OFF_C2W = 4160, OFF_C2B = 22592;
constexpr int OFF_FCW = 22656, OFF_FCB = 96384, OFF_R1W = 96512, OFF_R1B = 100608;
constexpr int OFF_R2W = 100672, OFF_R2B = 102720, OFF_G1W = 102784, OFF_G1B = 102912;
constexpr int OFF_G2W = 102976, OFF_G2B = 103232, OFF_FUW = 103296, OFF_FUB = 146304;
constexpr int OFF_LW = 146560, OFF_LB = 343168, OFF_HW = 343680, OFF_HB = 368256;
constexpr int OFF_OW = 368448, OFF_OB = 371520, N_PARAMS = 371584;
static_assert(N_PARAMS == QQT_LSTM_PARAMS, "packed block size");

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
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
struct __align__(16) ActLds {
  union {
    struct {                       // trunk: conv weights + one row's planes
      float w1[K1 * 32];
      float w2[K2 * 64];
      float in[C_MAX * 81];        // zero-bordered 9 x 9 per input channel
      float a1[32 * 81];           // conv1 output, zero-bordered
      float a2[64 * 49];           // conv2 output
    } t;
    struct {                       // head: activations of the 16 rows
      float xin[ROWS][XIN];        // fc | rel | glob outputs
      float xh[ROWS][XH];          // fused | previous h
      float g[ROWS][G4];           // LSTM gates
      float hn[ROWS][HID];         // new h
      float hd[ROWS][3 * HEAD];    // heads' hidden layers
      float r1[ROWS][64], g1[ROWS][16];
      float rel[ROWS][64];         // rel inputs (60 used)
      float glb[ROWS][8];          // glob inputs (5 used)
      float lg[ROWS][16];          // outputs
    } h;
  };
  float pooled[ROWS][FEAT];
};

// acc[t] += A (16 rows, LDS, row stride lda) x B (global k-major, row stride
// ldb) over K (a multiple of 4), output column tiles n0 + 16 t.
template <int NT>
__device__ __forceinline__ void gemm16(floatx4 (&acc)[NT], const float* A, int lda, const float* B,
                                       int ldb, int n0, int K, int lane) {
  const int r = lane & 15, q = lane >> 4;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 4) {
    const float av = A[r * lda + k0 + q];
    const float* b = B + (size_t)(k0 + q) * ldb + n0 + r;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mfma4(av, b[16 * t], acc[t]);
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

__global__ __launch_bounds__(NTHR) void lstm_act_kernel(const qqt_lstm_args a) {
  __shared__ ActLds s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row0 = blockIdx.x * ROWS;
  const float* P = a.params;
  const int cin = a.c_in, k1 = 9 * cin;

  // conv weights to LDS; zero the bordered planes once
  for (int i = tid; i < K1 * 32; i += NTHR) s.t.w1[i] = P[OFF_C1W + i];
  for (int i = tid; i < K2 * 64; i += NTHR) s.t.w2[i] = P[OFF_C2W + i];
  for (int i = tid; i < C_MAX * 81; i += NTHR) s.t.in[i] = 0.0f;
  for (int i = tid; i < 32 * 81; i += NTHR) s.t.a1[i] = 0.0f;

  // per-lane gather geometry: wavefront w owns positions 16w .. 16w+15
  const int pos = 16 * w + (lane & 15), q = lane >> 4;
  const bool pv = pos < 49;
  const int poff = pv ? (pos / 7) * 9 + pos % 7 : 0;   // top-left of the 3x3 window in a 9x9 grid
  auto tap = [](int k) { return (k / 9) * 81 + ((k % 9) / 3) * 9 + (k % 3); };

  for (int rr = 0; rr < ROWS; ++rr) {
    const int row = min(row0 + rr, a.batch - 1);        // rows past the batch: computed, dropped
    __syncthreads();                                     // previous row's planes are consumed
    const uint16_t* loc = a.local + (size_t)row * a.local_stride;
    for (int i = tid; i < cin * 49; i += NTHR)
      s.t.in[(i / 49) * 81 + ((i % 49) / 7 + 1) * 9 + (i % 7) + 1] = h2f(loc[i]);
    __syncthreads();
    // conv1: C -> 32; this wavefront's position tile, both channel tiles
    {
      floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
#pragma unroll 4
      for (int k0 = 0; k0 < K1; k0 += 4) {
        const int k = k0 + q;
        const float av = (pv && k < k1) ? s.t.in[poff + tap(k)] : 0.0f;
        acc[0] = mfma4(av, s.t.w1[k * 32 + (lane & 15)], acc[0]);
        acc[1] = mfma4(av, s.t.w1[k * 32 + 16 + (lane & 15)], acc[1]);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int co = 16 * t + (lane & 15);
        const float b = P[OFF_C1B + co];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int p = 16 * w + 4 * q + j;
          if (p < 49) s.t.a1[co * 81 + (p / 7 + 1) * 9 + p % 7 + 1] = fmaxf(acc[t][j] + b, 0.0f);
        }
      }
    }
    __syncthreads();
    // conv2: 32 -> 64
    {
      floatx4 acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = floatx4{0, 0, 0, 0};
#pragma unroll 4
      for (int k0 = 0; k0 < K2; k0 += 4) {
        const int k = k0 + q;
        const float av = pv ? s.t.a1[poff + tap(k)] : 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = mfma4(av, s.t.w2[k * 64 + 16 * t + (lane & 15)], acc[t]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int co = 16 * t + (lane & 15);
        const float b = P[OFF_C2B + co];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int p = 16 * w + 4 * q + j;
          if (p < 49) s.t.a2[co * 49 + p] = fmaxf(acc[t][j] + b, 0.0f);
        }
      }
    }
    __syncthreads();
    // 2x2 max pool (7 -> 3), flattened channel-major like x.view(B, -1)
    for (int i = tid; i < FEAT; i += NTHR) {
      const int c = i / 9, y = (i % 9) / 3, x = i % 3;
      const float* p = s.t.a2 + c * 49 + (2 * y) * 7 + 2 * x;
      s.pooled[rr][i] = fmaxf(fmaxf(p[0], p[1]), fmaxf(p[7], p[8]));
    }
  }
  __syncthreads();   // trunk done: its LDS becomes the head's

  // rel / glob inputs, previous hidden state
  for (int i = tid; i < ROWS * 64; i += NTHR) {
    const int r = i / 64, k = i % 64, row = min(row0 + r, a.batch - 1);
    s.h.rel[r][k] = k < MAX_T * 6 ? h2f(a.rel[(size_t)row * a.rel_stride + k]) : 0.0f;
  }
  for (int i = tid; i < ROWS * 8; i += NTHR) {
    const int r = i / 8, k = i % 8, row = min(row0 + r, a.batch - 1);
    s.h.glb[r][k] = k < GLOB ? h2f(a.glob[(size_t)row * a.glob_stride + k]) : 0.0f;
  }
  for (int i = tid; i < ROWS * HID; i += NTHR) {
    const int r = i / HID, k = i % HID, row = min(row0 + r, a.batch - 1);
    const bool zero = a.reset && a.reset[row / a.rows_per_env];
    s.h.xh[r][256 + k] = zero ? 0.0f : a.h[(size_t)row * HID + k];
  }
  // Linear(576, 128) + ReLU: 8 column tiles, two per wavefront
  {
    floatx4 acc[2] = {floatx4{0, 0, 0, 0}, floatx4{0, 0, 0, 0}};
    gemm16<2>(acc, &s.pooled[0][0], FEAT, P + OFF_FCW, HID, 32 * w, FEAT, lane);
    store16<2>(acc, &s.h.xin[0][0], XIN, 32 * w, P + OFF_FCB, true, lane, HID);
  }
  __syncthreads();
  // rel 60 -> 64 (one tile per wavefront), glob 5 -> 16 (wavefront 0)
  {
    floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
    gemm16<1>(acc, &s.h.rel[0][0], 64, P + OFF_R1W, 64, 16 * w, 64, lane);
    store16<1>(acc, &s.h.r1[0][0], 64, 16 * w, P + OFF_R1B, true, lane, 64);
    if (w == 0) {
      floatx4 ag[1] = {floatx4{0, 0, 0, 0}};
      gemm16<1>(ag, &s.h.glb[0][0], 8, P + OFF_G1W, 16, 0, 8, lane);
      store16<1>(ag, &s.h.g1[0][0], 16, 0, P + OFF_G1B, true, lane, 16);
    }
  }
  __syncthreads();
  // rel 64 -> 32 (wavefronts 0, 1), glob 16 -> 8 (wavefront 2)
  if (w < 2) {
    floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
    gemm16<1>(acc, &s.h.r1[0][0], 64, P + OFF_R2W, 32, 16 * w, 64, lane);
    store16<1>(acc, &s.h.xin[0][HID], XIN, 16 * w, P + OFF_R2B, true, lane, 32);
  } else if (w == 2) {
    floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
    gemm16<1>(acc, &s.h.g1[0][0], 16, P + OFF_G2W, 16, 0, 16, lane);
    store16<1>(acc, &s.h.xin[0][HID + 32], XIN, 0, P + OFF_G2B, true, lane, 8);
  }
  __syncthreads();
  // fusion Linear(168, 256) + ReLU: 16 tiles, four per wavefront
  {
    floatx4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = floatx4{0, 0, 0, 0};
    gemm16<4>(acc, &s.h.xin[0][0], XIN, P + OFF_FUW, 256, 64 * w, XIN, lane);
    store16<4>(acc, &s.h.xh[0][0], XH, 64 * w, P + OFF_FUB, true, lane, 256);
  }
  __syncthreads();
  // LSTM gates: [fused | h] (384) x W (384 x 512) + b: 32 tiles, eight per wavefront
  {
    floatx4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = floatx4{0, 0, 0, 0};
    gemm16<8>(acc, &s.h.xh[0][0], XH, P + OFF_LW, G4, 128 * w, XH, lane);
    store16<8>(acc, &s.h.g[0][0], G4, 128 * w, P + OFF_LB, false, lane, G4);
  }
  __syncthreads();
  // cell update
  for (int i = tid; i < ROWS * HID; i += NTHR) {
    const int r = i / HID, k = i % HID, row = row0 + r;
    const float ig = sigm(s.h.g[r][k]), fg = sigm(s.h.g[r][HID + k]);
    const float gg = tanhf(s.h.g[r][2 * HID + k]), og = sigm(s.h.g[r][3 * HID + k]);
    float cp = 0.0f;
    if (row < a.batch && !(a.reset && a.reset[row / a.rows_per_env])) cp = a.c[(size_t)row * HID + k];
    const float c2 = fg * cp + ig * gg;
    const float h2 = og * tanhf(c2);
    s.h.hn[r][k] = h2;
    if (row < a.batch) {
      a.c[(size_t)row * HID + k] = c2;
      a.h[(size_t)row * HID + k] = h2;
    }
  }
  __syncthreads();
  // heads' hidden layers 128 -> 192 + ReLU: 12 tiles, three per wavefront
  {
    floatx4 acc[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) acc[t] = floatx4{0, 0, 0, 0};
    gemm16<3>(acc, &s.h.hn[0][0], HID, P + OFF_HW, 3 * HEAD, 48 * w, HID, lane);
    store16<3>(acc, &s.h.hd[0][0], 3 * HEAD, 48 * w, P + OFF_HB, true, lane, 3 * HEAD);
  }
  __syncthreads();
  // output layer 192 -> 8 (block diagonal, 16 padded columns): wavefront 0
  if (w == 0) {
    floatx4 acc[1] = {floatx4{0, 0, 0, 0}};
    gemm16<1>(acc, &s.h.hd[0][0], 3 * HEAD, P + OFF_OW, 16, 0, 3 * HEAD, lane);
    store16<1>(acc, &s.h.lg[0][0], 16, 0, P + OFF_OB, false, lane, 16);
  }
  __syncthreads();
  // outputs and masked sampling: one thread per row
  if (tid < ROWS && row0 + tid < a.batch) {
    const int row = row0 + tid;
    const float* lg = s.h.lg[tid];
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
  const int blocks = (a->batch + lstm::ROWS - 1) / lstm::ROWS;
  QQT_LAUNCH(QQT_KERNEL_LSTM, lstm::lstm_act_kernel, dim3(blocks), dim3(lstm::NTHR), st, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "lstm act launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
