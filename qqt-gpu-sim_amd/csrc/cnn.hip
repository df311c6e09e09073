// cnn actor/critic forward + masked factored sampling for gfx950 (the
// reference's ActorCritic(arch="cnn"), train/model.py:79-96, 186-190).
//
// Network per (observation row, player): conv0 3x3 (14 -> 16 channels, the
// player's view permutation applied to the input planes) -> LayerNorm([16,
// 13,13]) -> ReLU -> conv 3x3 16 -> 32 -> LN -> ReLU -> conv 3x3 32 -> 64 ->
// LN -> ReLU -> conv 1x1 64 -> 8 -> LN -> ReLU -> flatten (1352) ->
// Linear(1352,128) -> LN -> ReLU -> Linear(128,128) -> LN -> ReLU -> three
// heads 128 -> 64 -> ReLU -> 5 | 2 | 1.  Every LayerNorm normalises one
// sample over all of its values (eps 1e-5) with an elementwise affine.
//
// Two kernels.  cnn_trunk_kernel: persistent, three workgroups of 4
// wavefronts per CU (one wavefront per SIMD each, at most 168 registers),
// each walking a contiguous range of items (row, player) one item at a
// time, so the workgroups' LayerNorm phases and convolutions overlap.
// cnn_head_kernel: 32 items per workgroup, from the trunk's flattened
// features in the workspace.
//
// Trunk.  Feature maps live in LDS as float16 hi and lo planes (x = hi +
// lo) on a zero-bordered grid 16 positions wide (x = -1 .. 14) with the 32
// channels of a position contiguous (40 halves per position).  The 3x3
// convs are implicit GEMMs on v_mfma_f32_16x16x32_f16 with float32
// accumulation: M = one output row (lane x = position; x >= 13 computed
// from the padding and ignored), N = output channels, K in steps of 32 =
// four 8-channel blocks, so lane l's A operand (8 halves) is one 16-byte LDS
// read of 8 channels at one position and tap, 16 lanes at consecutive
// positions:
//   16 input channels (conv0, conv 16->32): step s, lane group g = l / 16
//     takes combination c = 4 s + g: tap min(c / 2, 8), channels 8 (c % 2)..;
//     combinations 18, 19 carry zero weights;
//   32 input channels (conv 32->64): step s = tap, channels 8 g...
// Each product is hi*hi + hi*lo + lo*hi of the weight and activation planes
// (the observation is exact in float16, so conv0 skips its lo plane), which
// keeps the layer outputs within ~1e-6 relative of float32.  Products are
// taken as weights x activations, so a lane's accumulators are four
// consecutive channels of one position.  B operands come from L2 two K
// steps ahead (packed on the host as [tile][step][lane][8] halves).  The
// per-sample LayerNorm reduces the accumulators across the workgroup (mean,
// then squared deviations) and the rectified, normalised values are written
// over the input planes as hi/lo halves; after conv 32->64 they feed the
// 1x1 conv 64 -> 8 directly (v_mfma_f32_16x16x16_f16 per wavefront's
// 16-channel slice, partial sums added in LDS), whose LayerNorm output goes
// into this item's workspace rows (flattened index c * 169 + p).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "pipeline.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

namespace cnn {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int T = 256, NW = 4;
constexpr int HW = 13, NP = 169, MT = 13;    // position tiles = the 13 output rows
constexpr int PW = 16;                      // padded row: x = -1 .. 14 (lane x of a row tile)
constexpr int PP = 15 * PW + 2;             // padded positions (row tile 12's lane 15 reads 2 past)
constexpr int CS = 40;                      // halves per position (32 channels + 8: bank spread)
constexpr int C0 = 14;
constexpr int HB = 32, HM = HB / 16;        // items per head workgroup, its 16-row M tiles
constexpr int FLAT = 8 * NP;                // 1352
constexpr int KF = 1376;                    // flattened features padded to 43 K steps of 32
constexpr int S0H = KF / 32;                // 43
constexpr int WS_ROW = 2 * KF;              // workspace halves per item (hi and lo planes)
// Workspace layout, per block of HB items: [plane hi, lo][K step 43][item][32
// halves], so that a head workgroup reads one contiguous span, 2 KB per K
// step.  Item i's value k of plane pl is at
//   (i / HB) * HB * WS_ROW + ((pl * S0H + k / 32) * HB + i % HB) * 32 + k % 32.
__device__ __forceinline__ int ws_off(int pl, int k) {
  return (pl * S0H + (k >> 5)) * HB * 32 + (k & 31);   // + (i % HB) * 32 in the item's base
}
constexpr int HID = 128, HS = 130, HYS = 194;
constexpr int S0 = 5, S1 = 5, S2 = 9, S3 = 2;       // 32-deep K steps of the four convolutions
constexpr int L1 = HID / 4;                         // K steps of the float32 head GEMMs
constexpr int BFRAG = 64 * 8;                       // halves of one step's B fragments
#ifndef QQT_CNN_HEAD_D
#define QQT_CNN_HEAD_D 1
#endif
#ifndef QQT_CNN_CONV_D
#define QQT_CNN_CONV_D 1
#endif
constexpr int CONV_D = QQT_CNN_CONV_D;              // steps the convs' B fragments load ahead
constexpr int HEAD_D = QQT_CNN_HEAD_D;              // steps the head's layer-1 operands load ahead
static_assert(WS_ROW * 2 == QQT_CNN_WS_BYTES_PER_ITEM, "workspace row size");

struct __align__(16) Lds {                 // every member a multiple of 16 bytes long
  union {
    uint16_t act[2][PP * CS];               // hi, lo planes [position][channel]
    float part[NW][MT][8][16];              // the 1x1 conv's partial sums [wave][row][out][x]
  };
  float red[2][NW];
  int perm[2][16];                          // view permutations of the two item kinds
};
static_assert(sizeof(uint16_t) * 2 * PP * CS % 16 == 0, "16-byte fragment reads stay aligned");
static_assert(sizeof(float) * NW * MT * 8 * 16 <= sizeof(uint16_t) * 2 * PP * CS,
              "the partial sums fit in the activation planes");
static_assert(3 * sizeof(Lds) <= 160 * 1024, "three trunk workgroups fit in one CU's LDS");

// the head's small weights, staged in LDS: biases, LayerNorm affines and
// the output layer, at these offsets
constexpr int V_S0B = 0, V_S1W = 128, V_S1B = 256, V_S3B = 384, V_S4W = 512, V_S4B = 640,
              V_HB = 768, V_FW = 960, V_FB = 1472, V_N = 1480;

constexpr int PART_N = NW * HM * 8 * 64 * 4;        // layer 1's partial sums: [wave][M tile][N tile][lane][4]
struct __align__(16) HeadLds {
  float hy[HB * HYS];                       // heads' hidden layer; before it the first layer's
  float h2[HB * HS];                        // output h (stride HS, read by the second layer)
  float pad[PART_N - HB * HYS - HB * HS];   // hy .. pad: the partial sums before that
  float lg[HB * 8];
  float v[V_N];
};
static_assert(PART_N > HB * HYS + HB * HS, "the partial sums span hy, h2 and pad");
static_assert(2 * sizeof(HeadLds) <= 160 * 1024, "two head workgroups fit in one CU's LDS");

__device__ __forceinline__ floatx4 mfma(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Workgroup sum through red[slot][wave]: one barrier.  Consecutive calls
// alternate slots, so a slot is rewritten only after a later barrier has
// ordered every read of it.
__device__ __forceinline__ float block_sum(float v, float (*red)[NW], int& slot) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) red[slot][threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += red[slot][i];
  slot ^= 1;
  return s;
}

__device__ __forceinline__ half8 ld8(const uint16_t* p) {
  union { uint4 u; half8 h; } c;
  c.u = *reinterpret_cast<const uint4*>(p);
  return c.h;
}
// Uniform base + unsigned 32-bit byte offset: the form the compiler turns
// into a scalar-base global access (no 64-bit address arithmetic per lane).
template <class T>
__device__ __forceinline__ const T* at(const T* base, uint32_t byte_off) {
  return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}
template <class T>
__device__ __forceinline__ T* at(T* base, uint32_t byte_off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + byte_off);
}

__device__ __forceinline__ half8 bld8(Rsrc r, uint32_t byte_off) { return bld16<half8>(r, byte_off); }

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ floatx4 mfma16k16(half4 a, half4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
struct BFrag { half8 hi, lo; };

// Lane (thread) index the compiler cannot see through: values derived from
// it inside the persistent item loop are recomputed per item instead of
// hoisted out of the loop and held (or spilled) for the whole kernel.
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x & 63;
  asm volatile("" : "+v"(l));
  return l;
}
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// relu of four float32 values, saturated at float16's 65504 (one med3 each),
// split into float16 hi + lo (y = hi + lo to ~2^-22 relative), each plane
// packed two halves per word (v_cvt_pk_f16_f32, round to nearest)
__device__ __forceinline__ void relu_split4(const float (&z)[4], uint2& hi, uint2& lo) {
  float y[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) y[q] = __builtin_amdgcn_fmed3f(z[q], 0.0f, 65504.0f);
  const half2v h01 = {(_Float16)y[0], (_Float16)y[1]}, h23 = {(_Float16)y[2], (_Float16)y[3]};
  const half2v l01 = {(_Float16)(y[0] - (float)h01.x), (_Float16)(y[1] - (float)h01.y)};
  const half2v l23 = {(_Float16)(y[2] - (float)h23.x), (_Float16)(y[3] - (float)h23.y)};
  hi = uint2{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
  lo = uint2{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
}

__device__ __forceinline__ constexpr int tap_off(int tap) { return (tap / 3) * PW + tap % 3; }

// One conv layer for this wavefront (KIND 0: 3x3 over 16 channels, 1: 3x3
// over 32, 2: 1x1 over 64): row tiles min(mt0 + t ms, 12), t < NTL
// (duplicates of row 12 are computed and later ignored), lane x of a tile
// at output position (row, x), x >= 13 computed from the padding and
// ignored; the 16 lanes of a tile read consecutive padded positions, so the
// 16-byte reads are free of bank conflicts.  The products are taken as
// weights x activations, so the accumulators hold the transposed tile:
// value q of lane l is output channel 16 ntile + 4 (l / 16) + q at
// position x = l % 16 of the row; acc[t] = bias +
// sum over steps of A B, three float16 products per step (two without the
// activations' lo plane).  bfrag(s) returns step s's B fragments, loaded
// CONV_D steps ahead (pipeline), and each
// product kind runs over all tiles before the next, so no two consecutive
// MFMAs share an accumulator.
template <int KIND, int STEPS, int NTL, bool ALO, class BF>
__device__ __forceinline__ void conv(const uint16_t* act_hi, const uint16_t* act_lo, BF bfrag,
                                     floatx4 bias, int mt0, int ms, floatx4 (&acc)[NTL]) {
  constexpr int CG = NTL > 8 ? (NTL + 2) / 3 : NTL;
  const int lane = opaque_lane(), i16 = lane & 15, kq = lane >> 4;
  int base[NTL];
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const int pb = min(mt0 + t * ms, MT - 1) * PW + i16;   // padded position of tap (0, 0)
    base[t] = KIND == 0 ? pb * CS + 8 * (kq & 1) : KIND == 1 ? pb * CS + 8 * kq
                        : (pb + PW + 1) * CS + 8 * kq;
    acc[t] = bias;
  }
  pipeline<STEPS, CONV_D>(bfrag, [&](int st, const BFrag& b) {
    int off;
    if constexpr (KIND == 0)
      off = tap_off(min(2 * st + (kq >> 1), 8)) * CS;
    else if constexpr (KIND == 1)
      off = tap_off(st) * CS;
    else
      off = 32 * st;
    // tiles in groups (at most 8; 5 of the 13), so that one group's A
    // fragments are live
#pragma unroll
    for (int t0 = 0; t0 < NTL; t0 += CG) {
      half8 ah[CG], al[CG];
#pragma unroll
      for (int u = 0; u < CG; ++u)
        if (t0 + u < NTL) {
          ah[u] = ld8(act_hi + base[t0 + u] + off);
          if constexpr (ALO) al[u] = ld8(act_lo + base[t0 + u] + off);
        }
#pragma unroll
      for (int u = 0; u < CG; ++u)
        if (t0 + u < NTL) acc[t0 + u] = mfma16(b.hi, ah[u], acc[t0 + u]);
#pragma unroll
      for (int u = 0; u < CG; ++u)
        if (t0 + u < NTL) acc[t0 + u] = mfma16(b.lo, ah[u], acc[t0 + u]);
      if constexpr (ALO) {
#pragma unroll
        for (int u = 0; u < CG; ++u)
          if (t0 + u < NTL) acc[t0 + u] = mfma16(b.hi, al[u], acc[t0 + u]);
      }
    }
  });
}

// LayerNorm statistics over the valid outputs of a layer (lane x < 13,
// channel group kq < cq, row tile < 13); the accumulators are left centred
// (acc - mean).
template <int NTL>
__device__ __forceinline__ void ln_stats(floatx4 (&acc)[NTL], int mt0, int ms, int cq,
                                         float (*red)[NW], int& slot, float inv_count,
                                         float& mean, float& rstd) {
  const int lane = opaque_lane();
  const bool on = (lane & 15) < HW && (lane >> 4) < cq;
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT) {
#pragma unroll
      for (int q = 0; q < 4; ++q) s += acc[t][q];
    }
  mean = block_sum(on ? s : 0.0f, red, slot) * inv_count;
  float v = 0.0f;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[t][q] -= mean;                         // left centred for the write
        v = fmaf(acc[t][q], acc[t][q], v);
      }
    }
  rstd = 1.0f / sqrtf(block_sum(on ? v : 0.0f, red, slot) * inv_count + 1e-5f);
}

// LayerNorm affine tables of this wavefront's row tiles (min(mt0 + t ms,
// 12)), loaded before the statistics so that their latency overlaps the
// reductions.  g / bt: [NT][13][64][4] packed in the accumulator layout.
template <int NTL>
__device__ __forceinline__ void ln_tables(int mt0, int ms, int ntile,
                                          const float* __restrict__ g,
                                          const float* __restrict__ bt, float4 (&gg)[NTL],
                                          float4 (&bb)[NTL]) {
  const uint32_t tl = opaque_lane() * 16u;
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const uint32_t gi = (uint32_t)(ntile * MT + min(mt0 + t * ms, MT - 1)) * 1024u + tl;
    gg[t] = *at(reinterpret_cast<const float4*>(g), gi);
    bb[t] = *at(reinterpret_cast<const float4*>(bt), gi);
  }
}

// relu(LN affine) of this wavefront's centred outputs (lanes x < 13,
// channel groups kq < cq; saturated at 65504): a lane's four values are four consecutive
// channels of one position, one 8-byte store per plane into the activation
// planes, or (fl != nullptr) into the item's workspace block (value
// n * 169 + p of each plane, ws_off).
template <int NTL>
__device__ __forceinline__ void ln_write(const floatx4 (&acc)[NTL], int mt0, int ms, int ntile,
                                         int cq, float rstd,
                                         const float4 (&gg)[NTL], const float4 (&bb)[NTL],
                                         uint16_t* act_hi, uint16_t* act_lo, uint16_t* fl) {
  const int lane = opaque_lane(), x = lane & 15, kq = lane >> 4;
  if (x >= HW || kq >= cq) return;
  const int n0 = 16 * ntile + 4 * kq;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT) {
      const int y = mt0 + t * ms;
      const float gv[4] = {gg[t].x, gg[t].y, gg[t].z, gg[t].w};
      const float bv[4] = {bb[t].x, bb[t].y, bb[t].z, bb[t].w};
      float z[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) z[q] = fmaf(acc[t][q], rstd * gv[q], bv[q]);
      uint2 hi, lo;
      relu_split4(z, hi, lo);
      if (fl) {
        const int f0 = n0 * NP + y * HW + x;
        const uint32_t hw[4] = {hi.x, hi.x >> 16, hi.y, hi.y >> 16};
        const uint32_t lw[4] = {lo.x, lo.x >> 16, lo.y, lo.y >> 16};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          *at(fl, (uint32_t)ws_off(0, f0 + q * NP) * 2u) = (uint16_t)hw[q];
          *at(fl, (uint32_t)ws_off(1, f0 + q * NP) * 2u) = (uint16_t)lw[q];
        }
      } else {
        const int i0 = ((y + 1) * PW + x + 1) * CS + n0;
        *reinterpret_cast<uint2*>(act_hi + i0) = hi;
        *reinterpret_cast<uint2*>(act_lo + i0) = lo;
      }
    }
}

// relu(LN affine) of conv 32->64's row tiles (this wavefront's 16 output
// channels, all 13 rows) taken straight into the 1x1 conv 64->8: a lane's
// four values (channels 4 kq .. + 3 of the block at position x) are the B
// operand of v_mfma_f32_16x16x16_f16, the block's 8 x 16 slice of the 1x1
// weights (w3h + w3l, rows 8..15 zero) the A operand, three products per
// tile (hi*hi + lo*hi + hi*lo); the partial sums of outputs o < 8 go to
// part[w][row][o][x] for the workgroup to add up.
template <int NTL>
__device__ __forceinline__ void ln_conv3(const floatx4 (&acc)[NTL], int ntile, float rstd, const float* __restrict__ g,
                                         const float* __restrict__ bt, half4 w3h, half4 w3l,
                                         float* part) {
  const int lane = opaque_lane(), x = lane & 15, kq = lane >> 4;
  const uint32_t tl = (uint32_t)lane * 16u;
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const uint32_t gi = (uint32_t)(ntile * MT + t) * 1024u + tl;
    const float4 gg = *at(reinterpret_cast<const float4*>(g), gi);
    const float4 bb = *at(reinterpret_cast<const float4*>(bt), gi);
    const float z[4] = {fmaf(acc[t][0], rstd * gg.x, bb.x), fmaf(acc[t][1], rstd * gg.y, bb.y),
                        fmaf(acc[t][2], rstd * gg.z, bb.z), fmaf(acc[t][3], rstd * gg.w, bb.w)};
    uint2 hi, lo;
    relu_split4(z, hi, lo);
    const half4 yh = __builtin_bit_cast(half4, hi), yl = __builtin_bit_cast(half4, lo);
    floatx4 d = {0.0f, 0.0f, 0.0f, 0.0f};
    d = mfma16k16(w3h, yh, d);
    d = mfma16k16(w3l, yh, d);
    d = mfma16k16(w3h, yl, d);
    if (kq < 2) {
#pragma unroll
      for (int q = 0; q < 4; ++q) part[(t * 8 + 4 * kq + q) * 16 + x] = d[q];
    }
  }
}

// A head layer's weight operands for tiles nt0 + i (i < NTW), W packed
// [tile][step][lane] in global memory: loaded ahead of the GEMM.
template <int STEPS, int NTW>
__device__ __forceinline__ void head_weights(const float* __restrict__ w, int nt0,
                                             float (&bw)[NTW][STEPS]) {
  const float* b = w + (size_t)nt0 * STEPS * 64 + (threadIdx.x & 63);
#pragma unroll
  for (int i = 0; i < NTW; ++i)
#pragma unroll
    for (int j = 0; j < STEPS; ++j) bw[i][j] = b[(i * STEPS + j) * 64];
}

// Head GEMM over the HM row tiles: D[m][n] = sum_k A[m * as + k] W[k][n],
// A in LDS, the weight operands in registers (each feeds every row tile).
template <int STEPS, int NTW>
__device__ __forceinline__ void head_gemm(const float* A, int as, const float (&bw)[NTW][STEPS],
                                          floatx4 (&c)[HM][NTW]) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int m = 0; m < HM; ++m)
#pragma unroll
    for (int i = 0; i < NTW; ++i) c[m][i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < STEPS; ++j) {
    float av[HM];
#pragma unroll
    for (int m = 0; m < HM; ++m) av[m] = A[(16 * m + i16) * as + kq + 4 * j];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
      for (int m = 0; m < HM; ++m) c[m][i] = mfma(av[m], bw[i][j], c[m][i]);
  }
}

// D tile -> dst[m * ds + 16 * ntile + i16] for the 16 rows m (+ bias, optional ReLU).
__device__ __forceinline__ void head_store(floatx4 c, float* dst, int ds, int ntile,
                                           const float* __restrict__ bias, bool relu) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
  const int n = 16 * ntile + i16;
  const float bv = bias[n];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float y = c[q] + bv;
    dst[(4 * kq + q) * ds + n] = relu ? fmaxf(y, 0.0f) : y;
  }
}

// LayerNorm(128) + ReLU of rows m < nb of h (stride HS), 16 threads per row.
__device__ __forceinline__ void head_ln(float* h, int nb, const float* __restrict__ g,
                                        const float* __restrict__ bt) {
  const int c = threadIdx.x & 15;
#pragma unroll
  for (int m = threadIdx.x >> 4; m < HB; m += T / 16) {
    float v[8];
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      v[r] = h[m * HS + c + 16 * r];
      s += v[r];
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    const float mean = s * (1.0f / HID);
    float q = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) q += (v[r] - mean) * (v[r] - mean);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
    const float rstd = 1.0f / sqrtf(q * (1.0f / HID) + 1e-5f);
    if (m < nb) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int k = c + 16 * r;
        h[m * HS + k] = fmaxf((v[r] - mean) * rstd * g[k] + bt[k], 0.0f);
      }
    }
  }
}

__global__ __launch_bounds__(T, 3) void cnn_trunk_kernel(const qqt_cnn_args a, int items,
                                                          int per) {
  __shared__ Lds s;
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63, i16 = lane & 15;

  // B operands of the 3x3 convs from global memory step by step (L2 hits:
  // 10, 20 and 72 KB shared by every workgroup); this wavefront's slice of
  // the 1x1 conv (its 16 input channels) in registers
  const int n1 = w & 1, n2 = w;
  // biases of the four output channels 16 tile + 4 (lane / 16) .. + 3
  const int kq4 = 4 * (lane >> 4);
  auto bias4 = [&](const float* b, int tile) {
    const float* const p = b + 16 * tile + kq4;
    return floatx4{p[0], p[1], p[2], p[3]};
  };
  const floatx4 bias0 = bias4(a.c0b, 0), bias1 = bias4(a.c1b, n1), bias2 = bias4(a.c2b, n2);
  const half4 w3h = *at(reinterpret_cast<const half4*>(a.c3w), (uint32_t)(w * 64 + lane) * 8u);
  const half4 w3l = *at(reinterpret_cast<const half4*>(a.c3w_lo), (uint32_t)(w * 64 + lane) * 8u);

  // row tiles per wavefront: conv0 {w + 4i}, i < 4; conv1 {w/2 + 2i},
  // i < 7; conv2 (and its 1x1 slice) all 13
  const int mt1 = w >> 1;

  for (int i = t; i < PP * CS; i += T) s.act[0][i] = s.act[1][i] = 0;
  const uint32_t lb = (uint32_t)lane * 16u;        // this lane's bytes in a step's fragments
  // buffer resources over this wavefront's B slices (STEPS fragments each)
  const Rsrc c1h = rsrc(a.c1w + (size_t)n1 * S1 * BFRAG, S1 * BFRAG * 2);
  const Rsrc c1l = rsrc(a.c1w_lo + (size_t)n1 * S1 * BFRAG, S1 * BFRAG * 2);
  auto breg1 = [&](int j) {
    const uint32_t o = lb + (uint32_t)j * (BFRAG * 2);
    return BFrag{bld8(c1h, o), bld8(c1l, o)};
  };
  const Rsrc c2h = rsrc(a.c2w + (size_t)n2 * S2 * BFRAG, S2 * BFRAG * 2);
  const Rsrc c2l = rsrc(a.c2w_lo + (size_t)n2 * S2 * BFRAG, S2 * BFRAG * 2);
  auto breg2 = [&](int j) {
    const uint32_t o = lb + (uint32_t)j * (BFRAG * 2);
    return BFrag{bld8(c2h, o), bld8(c2l, o)};
  };
  const Rsrc c0h = rsrc(a.c0w, S0 * BFRAG * 2), c0l = rsrc(a.c0w_lo, S0 * BFRAG * 2);
  auto bglob0 = [&](int j) {
    const uint32_t o = lb + (uint32_t)j * (BFRAG * 2);
    return BFrag{bld8(c0h, o), bld8(c0l, o)};
  };

  // Observation staging: thread t < 169 moves position p = t of the item's
  // 14 input planes (plane c is observation channel view_perm[pid][c]): the
  // next item's 14 values are loaded into registers while this item
  // computes, and leave as three 8-byte and one 4-byte LDS store (channels
  // contiguous at the position).  Threads past 169 load position 168 and
  // store nothing.
  if (t < 2 * C0) {
    const int kind = t / C0;
    const int pid = a.npid == 2 ? kind : a.pid0;
    s.perm[kind][t % C0] = a.view_perm[pid * C0 + t % C0];
  }
  __syncthreads();
  uint32_t ov[C0];
  auto fetch = [&](int item) {
    const int row = item / a.npid, kind = a.npid == 2 ? (item & 1) : 0;
    const uint16_t* const ob = a.obs + (size_t)row * a.obs_stride;
    const int pt = min(opaque_tid(), NP - 1);
#pragma unroll
    for (int c = 0; c < C0; ++c) ov[c] = *at(ob, (uint32_t)(s.perm[kind][c] * NP + pt) * 2u);
  };
  auto stage = [&]() {
    const int pt = opaque_tid();
    if (pt < NP) {
      const int y = pt / HW;
      uint16_t* const d = &s.act[0][((y + 1) * PW + (pt - y * HW) + 1) * CS];
      *reinterpret_cast<uint2*>(d) = uint2{ov[0] | ov[1] << 16, ov[2] | ov[3] << 16};
      *reinterpret_cast<uint2*>(d + 4) = uint2{ov[4] | ov[5] << 16, ov[6] | ov[7] << 16};
      *reinterpret_cast<uint2*>(d + 8) = uint2{ov[8] | ov[9] << 16, ov[10] | ov[11] << 16};
      *reinterpret_cast<uint32_t*>(d + 12) = ov[12] | ov[13] << 16;
    }
  };

  int rslot = 0;                                   // reduction slot
  const int start = blockIdx.x * per, end = min(items, start + per);
  if (start < end) fetch(start);
  for (int item = start; item < end; ++item) {
    __syncthreads();                                  // channels 0..13 free
    stage();                                          // exact in float16: hi plane only
    __syncthreads();

    float mean, rstd;
    {
      floatx4 acc[4];
      float4 gg[4], bb[4];
      conv<0, S0, 4, false>(s.act[0], s.act[1], bglob0, bias0, w, 4, acc);
      ln_tables<4>(w, 4, 0, a.ln0w, a.ln0b, gg, bb);
      ln_stats<4>(acc, w, 4, 4, s.red, rslot, 1.0f / (16 * NP), mean, rstd);
      ln_write<4>(acc, w, 4, 0, 4, rstd, gg, bb, s.act[0], s.act[1], nullptr);
    }
    __syncthreads();
    {
      floatx4 acc[7];
      float4 gg[7], bb[7];
      conv<0, S1, 7, true>(s.act[0], s.act[1], breg1, bias1, mt1, 2, acc);
      ln_tables<7>(mt1, 2, n1, a.ln1w, a.ln1b, gg, bb);
      ln_stats<7>(acc, mt1, 2, 4, s.red, rslot, 1.0f / (32 * NP), mean, rstd);
      ln_write<7>(acc, mt1, 2, n1, 4, rstd, gg, bb, s.act[0], s.act[1], nullptr);
    }
    __syncthreads();
    {
      floatx4 acc[MT];
      conv<1, S2, MT, true>(s.act[0], s.act[1], breg2, bias2, 0, 1, acc);
      ln_stats<MT>(acc, 0, 1, 4, s.red, rslot, 1.0f / (64 * NP), mean, rstd);
      // every wavefront is past its conv reads: the planes take the partials
      ln_conv3<MT>(acc, n2, rstd, a.ln2w, a.ln2b, w3h, w3l, &s.part[w][0][0][0]);
    }
    __syncthreads();
    // 1x1 conv outputs (o < 8, 169 positions) = bias + the four partial
    // sums; thread t takes slots t + 256 i = row * 128 + o * 16 + x (x < 13)
    {
      constexpr int NS = (MT * 128 + T - 1) / T;
      const int tt = opaque_tid();
      float v[NS];
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int sl = min(tt + T * i, MT * 128 - 1), o = (sl >> 4) & 7, x = sl & 15;
        const bool ok = tt + T * i < MT * 128 && x < HW;
        const float* const pp = &s.part[0][0][0][0] + sl;
        const float u = pp[0] + pp[MT * 128] + pp[2 * MT * 128] + pp[3 * MT * 128] +
                        *at(a.c3b, (uint32_t)o * 4u);
        v[i] = ok ? u : 0.0f;
        sum += v[i];
      }
      // this thread's LayerNorm affines, then the next item's observation:
      // no load is issued after the fetch before the next item stages it
      // (loads complete in issue order, so a wait for a later load would
      // wait for the fetch as well)
      float lw[NS], lb[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int sl = min(tt + T * i, MT * 128 - 1), y = sl >> 7, o = (sl >> 4) & 7;
        const int k = o * NP + y * HW + min(sl & 15, HW - 1);
        lw[i] = *at(a.ln3w, (uint32_t)k * 4u);
        lb[i] = *at(a.ln3b, (uint32_t)k * 4u);
      }
      fetch(min(item + 1, end - 1));
      mean = block_sum(sum, s.red, rslot) * (1.0f / FLAT);
      // every thread is past its partial-sum reads: zero the bytes they
      // occupied, the next item's padding and unused channel slots
      for (int i = tt; i < (int)(sizeof(s.part) / 16); i += T)
        reinterpret_cast<uint4*>(&s.part[0][0][0][0])[i] = uint4{0u, 0u, 0u, 0u};
      float var = 0.0f;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int sl = tt + T * i;
        const float d = v[i] - mean;
        if (sl < MT * 128 && (sl & 15) < HW) var = fmaf(d, d, var);
      }
      rstd = 1.0f / sqrtf(block_sum(var, s.red, rslot) * (1.0f / FLAT) + 1e-5f);
      uint16_t* const fl = a.workspace + (size_t)(item / HB) * HB * WS_ROW + (item % HB) * 32;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int sl = tt + T * i, y = sl >> 7, o = (sl >> 4) & 7, x = sl & 15;
        if (sl < MT * 128 && x < HW) {
          const int k = o * NP + y * HW + x;              // flattened [8][13][13] index
          const float y = __builtin_amdgcn_fmed3f(fmaf(v[i] - mean, rstd * lw[i], lb[i]), 0.0f, 65504.0f);
          const _Float16 hi = (_Float16)y, lo = (_Float16)(y - (float)hi);
          *at(fl, (uint32_t)ws_off(0, k) * 2u) = __builtin_bit_cast(uint16_t, hi);
          *at(fl, (uint32_t)ws_off(1, k) * 2u) = __builtin_bit_cast(uint16_t, lo);
        }
      }
      if (t < KF - FLAT) fl[ws_off(0, FLAT + t)] = fl[ws_off(1, FLAT + t)] = 0;
    }
  }
}

// Head over items ib .. ib + 31 (rows m of the GEMMs; rows past the batch
// repeat its last item and are not written out).
__global__ __launch_bounds__(T) void cnn_head_kernel(const qqt_cnn_args a, int items) {
  __shared__ HeadLds s;
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63, i16 = lane & 15, kq = lane >> 4;
  const int ib = blockIdx.x * HB, nb = min(HB, items - ib);
  float* const h = s.hy;
  {
    const float* const src[9] = {a.s0b, a.s1w, a.s1b, a.s3b, a.s4w, a.s4b, a.hb, a.fw, a.fb};
    const int off[10] = {V_S0B, V_S1W, V_S1B, V_S3B, V_S4W, V_S4B, V_HB, V_FW, V_FB, V_N};
#pragma unroll
    for (int k = 0; k < 9; ++k)
      for (int i = t; i < off[k + 1] - off[k]; i += T) s.v[off[k] + i] = src[k][i];
  }

  // Linear(1352,128): wavefront w takes K steps KQ w .. KQ w + KQ - 1 (the
  // last wavefront the 10 that remain) for all HM x 8 output tiles, so the
  // workgroup reads its items' features once; the four partial sums meet in
  // LDS and wavefront w finishes output tiles 2w, 2w + 1 of every row tile
  {
    constexpr int KQ = (S0H + NW - 1) / NW;
    const int k0 = KQ * w, kn = min(KQ, S0H - k0);
    const Rsrc ws = rsrc(a.workspace + (size_t)ib * WS_ROW, HB * WS_ROW * 2);
    uint32_t ar[HM];
#pragma unroll
    for (int m = 0; m < HM; ++m) ar[m] = (uint32_t)(min(16 * m + i16, nb - 1) * 32 + 8 * kq) * 2u;
    constexpr uint32_t tile = S0H * BFRAG * 2;       // bytes of one output tile's plane
    const Rsrc bh = rsrc(a.s0h, 8 * tile), bl = rsrc(a.s0l, 8 * tile);
    const uint32_t lb = (uint32_t)lane * 16u;
    struct Frag { half8 ah[HM], al[HM], h[8], l[8]; };
    auto load = [&](int i) {
      const int st = min(k0 + i, S0H - 1);
      Frag f;
#pragma unroll
      for (int m = 0; m < HM; ++m) {
        f.ah[m] = bld8(ws, ar[m] + (uint32_t)st * (HB * 32 * 2));
        f.al[m] = bld8(ws, ar[m] + (uint32_t)(S0H + st) * (HB * 32 * 2));
      }
      const uint32_t o = lb + (uint32_t)st * (BFRAG * 2);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        f.h[n] = bld8(bh, o + n * tile);
        f.l[n] = bld8(bl, o + n * tile);
      }
      return f;
    };
    floatx4 c[HM][8];
#pragma unroll
    for (int m = 0; m < HM; ++m)
#pragma unroll
      for (int n = 0; n < 8; ++n) c[m][n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    pipeline<KQ, HEAD_D>(load, [&](int i, const Frag& f) {
      if (i < kn) {
#pragma unroll
        for (int m = 0; m < HM; ++m)
#pragma unroll
          for (int n = 0; n < 8; ++n) c[m][n] = mfma16(f.ah[m], f.h[n], c[m][n]);
#pragma unroll
        for (int m = 0; m < HM; ++m)
#pragma unroll
          for (int n = 0; n < 8; ++n) c[m][n] = mfma16(f.ah[m], f.l[n], c[m][n]);
#pragma unroll
        for (int m = 0; m < HM; ++m)
#pragma unroll
          for (int n = 0; n < 8; ++n) c[m][n] = mfma16(f.al[m], f.h[n], c[m][n]);
      }
    });
    floatx4* const part = reinterpret_cast<floatx4*>(s.hy);
#pragma unroll
    for (int m = 0; m < HM; ++m)
#pragma unroll
      for (int n = 0; n < 8; ++n) part[((w * HM + m) * 8 + n) * 64 + lane] = c[m][n];
  }
  float w3[2][L1];                                  // Linear(128,128) operands, loaded under the sums
  head_weights<L1, 2>(a.s3p, 2 * w, w3);
  __syncthreads();
  {
    const floatx4* const part = reinterpret_cast<const floatx4*>(s.hy);
    floatx4 c[HM][2];
#pragma unroll
    for (int m = 0; m < HM; ++m)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = 2 * w + j;
        c[m][j] = part[(m * 8 + n) * 64 + lane];
#pragma unroll
        for (int v = 1; v < NW; ++v) c[m][j] += part[((v * HM + m) * 8 + n) * 64 + lane];
      }
    __syncthreads();                                  // every sum read before h overwrites them
#pragma unroll
    for (int m = 0; m < HM; ++m) {
      head_store(c[m][0], h + 16 * m * HS, HS, 2 * w, s.v + V_S0B, false);
      head_store(c[m][1], h + 16 * m * HS, HS, 2 * w + 1, s.v + V_S0B, false);
    }
  }
  __syncthreads();
  head_ln(h, nb, s.v + V_S1W, s.v + V_S1B);
  __syncthreads();
  {
    floatx4 c[HM][2];
    head_gemm<L1, 2>(h, HS, w3, c);
#pragma unroll
    for (int m = 0; m < HM; ++m) {
      head_store(c[m][0], s.h2 + 16 * m * HS, HS, 2 * w, s.v + V_S3B, false);
      head_store(c[m][1], s.h2 + 16 * m * HS, HS, 2 * w + 1, s.v + V_S3B, false);
    }
  }
  float wh[3][L1];                                  // heads' operands, loaded under the LayerNorm
  head_weights<L1, 3>(a.hp, 3 * w, wh);
  __syncthreads();
  head_ln(s.h2, nb, s.v + V_S4W, s.v + V_S4B);
  __syncthreads();
  {
    floatx4 c[HM][3];
    head_gemm<L1, 3>(s.h2, HS, wh, c);
#pragma unroll
    for (int m = 0; m < HM; ++m)
#pragma unroll
      for (int i = 0; i < 3; ++i)
        head_store(c[m][i], s.hy + 16 * m * HYS, HYS, 3 * w + i, s.v + V_HB, true);
  }
  __syncthreads();
  if (t < HB * 8) {                                   // output layer: item m, output o
    const int m = t >> 3, o = t & 7;
    const int base = o < 5 ? 0 : o < 7 ? 64 : 128;
    const float* x = s.hy + m * HYS + base;
    const float* wf = s.v + V_FW + o * 64;
    float acc = 0.0f;
#pragma unroll 8
    for (int k = 0; k < 64; ++k) acc += x[k] * wf[k];
    s.lg[m * 8 + o] = acc + s.v[V_FB + o];
  }
  __syncthreads();
  if (t < nb) {
    const int item = ib + t;
    const int row = item / a.npid, slot = item % a.npid;
    const int pid = a.npid == 2 ? slot : a.pid0;
    float l8[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) l8[k] = s.lg[t * 8 + k];
    const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;
    const int oslot = a.npid == 2 ? slot : a.out_slot;
    const size_t o = (size_t)row * oslots + oslot;
    if (a.logits_out) {
#pragma unroll
      for (int k = 0; k < 8; ++k) a.logits_out[o * 8 + k] = l8[k];
    }
    if (a.value_out) a.value_out[o] = l8[7];
    if (a.sample) {
      uint8_t mm[5], bm[2];
#pragma unroll
      for (int k = 0; k < 5; ++k)
        mm[k] = a.move_mask[(size_t)row * a.mm_row_stride + (size_t)pid * a.mm_pid_stride + k];
#pragma unroll
      for (int k = 0; k < 2; ++k)
        bm[k] = a.bomb_mask[(size_t)row * a.bm_row_stride + (size_t)pid * a.bm_pid_stride + k];
      float um, ub;
      if (a.uniforms) {
        um = a.uniforms[o * 2 + 0];
        ub = a.uniforms[o * 2 + 1];
      } else {
        float u4[4];
        philox_block(a.seed, (uint32_t)row, a.tick, STREAM_POLICY, (uint32_t)((2 * pid) >> 2),
                     u4);
        um = u4[(2 * pid) & 3];
        ub = u4[(2 * pid + 1) & 3];
      }
      float lpm, lpb;
      const int am = sample_masked<5>(l8, mm, um, &lpm);
      const int ab = sample_masked<2>(l8 + 5, bm, ub, &lpb);
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

int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        c <= 0)
      c = 256;
    cus[dev] = c;
  }
  return cus[dev];
}

}  // namespace cnn
}  // namespace qqt

extern "C" {

int qqt_cnn_act(const qqt_cnn_args* a, void* stream) {
  using namespace qqt;
  using namespace qqt::cnn;
  g_err[0] = 0;
  if (!a || !a->obs || !a->view_perm || !a->c0w || !a->c0w_lo || !a->c0b || !a->ln0w ||
      !a->ln0b || !a->c1w || !a->c1w_lo || !a->c1b || !a->ln1w || !a->ln1b || !a->c2w ||
      !a->c2w_lo || !a->c2b || !a->ln2w || !a->ln2b || !a->c3w || !a->c3w_lo || !a->c3b ||
      !a->ln3w || !a->ln3b || !a->s0h || !a->s0l || !a->s0b ||
      !a->s1w || !a->s1b || !a->s3p || !a->s3b || !a->s4w || !a->s4b || !a->hp || !a->hb ||
      !a->fw || !a->fb) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: null pointer argument");
    return QQT_E_ARG;
  }
  if (((uintptr_t)a->ln0w | (uintptr_t)a->ln0b | (uintptr_t)a->ln1w | (uintptr_t)a->ln1b |
       (uintptr_t)a->ln2w | (uintptr_t)a->ln2b | (uintptr_t)a->ln3w | (uintptr_t)a->ln3b |
       (uintptr_t)a->c1w | (uintptr_t)a->c1w_lo | (uintptr_t)a->c2w | (uintptr_t)a->c2w_lo |
       (uintptr_t)a->s0h | (uintptr_t)a->s0l) & 15) {
    snprintf(g_err, sizeof(g_err),
             "qqt_cnn_act: LayerNorm tables, conv and first head weights must be 16-byte aligned");
    return QQT_E_ARG;
  }
  if (a->batch <= 0 || (a->npid != 1 && a->npid != 2) || a->w_players < a->npid ||
      a->w_players > 4 || a->pid0 < 0 || (a->npid == 1 && a->pid0 >= a->w_players) ||
      a->obs_stride < C0 * NP || (int64_t)a->batch * a->npid > INT32_MAX) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: bad batch, players or observation stride");
    return QQT_E_ARG;
  }
  const int oslots = a->out_slots > 0 ? a->out_slots : a->npid;
  if (a->out_slots < 0 || oslots < a->npid || oslots > 4 || a->out_slot < 0 ||
      (a->npid == 1 && a->out_slot >= oslots)) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: bad output slots");
    return QQT_E_ARG;
  }
  if (a->sample && (!a->move_mask || !a->bomb_mask)) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: sampling needs masks");
    return QQT_E_ARG;
  }
  const int items = a->batch * a->npid;
  if (!a->workspace || ((uintptr_t)a->workspace & 15) ||
      a->workspace_bytes < (int64_t)((items + HB - 1) / HB) * HB * QQT_CNN_WS_BYTES_PER_ITEM) {
    snprintf(g_err, sizeof(g_err),
             "qqt_cnn_act: workspace must be 16-byte aligned and hold %d bytes per item "
             "(items rounded up to %d)", QQT_CNN_WS_BYTES_PER_ITEM, HB);
    return QQT_E_ARG;
  }
  const int grid = min(3 * cu_count(), items);     // three resident workgroups per CU
  const int per = (items + grid - 1) / grid;
  hipStream_t st = (hipStream_t)stream;
  QQT_LAUNCH(QQT_KERNEL_CNN, cnn_trunk_kernel, dim3(grid), dim3(T), st, *a, items, per);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) {
    QQT_LAUNCH(QQT_KERNEL_CNN_HEAD, cnn_head_kernel, dim3((items + HB - 1) / HB), dim3(T), st,
               *a, items);
    err = hipGetLastError();
  }
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "cnn launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
