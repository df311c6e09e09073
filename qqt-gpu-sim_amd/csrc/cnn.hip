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
// Persistent kernel: one workgroup (4 wavefronts, one per SIMD, so each
// wavefront may hold 512 registers) per CU walks a contiguous range of items
// (row, player).
//
// Trunk, one item at a time.  Feature maps live in LDS as zero-bordered
// 15 x 15 grids of positions with the channels of a position contiguous
// (72 halves per position), as float16 hi and lo planes (x = hi + lo).
// Convolutions are implicit GEMMs on v_mfma_f32_16x16x32_f16 with float32
// accumulation: M = positions (11 tiles of 16), N = output channels, K in
// steps of 32 = four 8-channel blocks, so lane l's A operand (8 halves) is
// one 16-byte LDS read of 8 channels at one position and tap:
//   16 input channels (conv0, conv 16->32): step s, lane group g = l / 16
//     takes combination c = 4 s + g: tap min(c / 2, 8), channels 8 (c % 2)..;
//     combinations 18, 19 carry zero weights;
//   32 input channels (conv 32->64): step s = tap, channels 8 g..;
//   64 input channels (1x1): step s, channels 8 (4 s + g)...
// Each product is hi*hi + hi*lo + lo*hi of the activation and weight
// planes (the observation is exact in float16, so conv0 skips its lo
// plane), which keeps the layer outputs within ~1e-6 relative of float32.
// The B operands of the 16->32 and 32->64 convs stay in registers for the
// whole kernel (wavefront w owns output tile w % NT of each); those of conv0
// and the 1x1 conv (one output tile, used by every wavefront) sit in LDS; all
// are packed on the host as [tile][step][lane][8] halves.  The accumulators
// are the layer's output: the per-sample LayerNorm reduces them across the
// workgroup (mean, then squared deviations) and the rectified, normalised
// values are written over the input planes as hi/lo halves (after the last
// conv, into this item's row of the float32 flat buffer).
// Head, per batch of up to 15 items: Linear(1352,128), Linear(128,128) and
// the heads' hidden layer are v_mfma_f32_16x16x4_f32 GEMMs with M = the items
// (B streamed from L2 once per batch), LayerNorm(128) by 16 threads per item,
// then the output layer and the masked sampling per item.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

namespace cnn {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int T = 256, NW = 4;
constexpr int HW = 13, NP = 169, MT = 11;
constexpr int PP = 225;                     // padded positions (15 x 15)
constexpr int CS = 72;                      // halves per position (64 channels + 8: bank spread)
constexpr int C0 = 14;
constexpr int SB = 15;                      // items per head batch (<= the 16 MFMA rows)
constexpr int FLAT = 8 * NP;                // 1352
constexpr int FS = 1378;                    // flat row stride (2 mod 32 banks)
constexpr int HID = 128, HS = 130, HYS = 194;
constexpr int S0 = 5, S1 = 5, S2 = 9, S3 = 2;       // 32-deep K steps of the four convolutions
constexpr int L0 = FLAT / 4, L1 = HID / 4;          // K steps of the head GEMMs
constexpr int BFRAG = 64 * 8;                       // halves of one step's B fragments

struct __align__(16) Lds {                 // every member a multiple of 16 bytes long
  uint16_t act[2][PP * CS];                 // hi, lo planes [position][channel]
  uint16_t wc0[2][S0 * BFRAG], wc3[2][S3 * BFRAG];   // conv0 / 1x1 B (hi, lo), all waves
  float flat[SB * FS];                      // trunk outputs; head scratch after GEMM 1
  float red[2][NW];
};
static_assert(sizeof(uint16_t) * 2 * PP * CS % 16 == 0, "16-byte fragment reads stay aligned");
// head scratch inside flat (free once Linear(1352,128) has read it)
constexpr int H_OFF = 0, H2_OFF = SB * HS, HY_OFF = 2 * SB * HS, LG_OFF = 2 * SB * HS + SB * HYS;
static_assert(LG_OFF + 16 * 8 <= SB * FS, "head scratch (16 rows) fits in the flat buffer");

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
__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
struct BFrag { half8 hi, lo; };

__device__ __forceinline__ constexpr int tap_off(int tap) { return (tap / 3) * 15 + tap % 3; }

// One conv layer for this wavefront (KIND 0: 3x3 over 16 channels, 1: 3x3
// over 32, 2: 1x1 over 64): position tiles min(mt0 + t ms, 10), t < NTL
// (duplicates of tile 10 are computed and later ignored); acc[t] = bias +
// sum over steps of A B, three float16 products per step (two without the
// activations' lo plane).  bfrag(s) returns step s's B fragments.
template <int KIND, int STEPS, int NTL, bool ALO, class BF>
__device__ __forceinline__ void conv(const uint16_t* act_hi, const uint16_t* act_lo, BF bfrag,
                                     float bias, int mt0, int ms, floatx4 (&acc)[NTL]) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
  int base[NTL];
#pragma unroll
  for (int t = 0; t < NTL; ++t) {
    const int p = min(16 * min(mt0 + t * ms, MT - 1) + i16, NP - 1);
    const int pb = (p / HW) * 15 + (p % HW);          // padded position of tap (0, 0)
    base[t] = KIND == 0 ? pb * CS + 8 * (kq & 1) : KIND == 1 ? pb * CS + 8 * kq
                        : (pb + 16) * CS + 8 * kq;
    acc[t] = floatx4{bias, bias, bias, bias};
  }
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    int off;
    if constexpr (KIND == 0)
      off = ((kq >> 1) ? tap_off(min(2 * st + 1, 8)) : tap_off(min(2 * st, 8))) * CS;
    else if constexpr (KIND == 1)
      off = tap_off(st) * CS;
    else
      off = 32 * st;
    const BFrag b = bfrag(st);
#pragma unroll
    for (int t = 0; t < NTL; ++t) {
      const half8 ah = ld8(act_hi + base[t] + off);
      acc[t] = mfma16(ah, b.hi, acc[t]);
      acc[t] = mfma16(ah, b.lo, acc[t]);
      if constexpr (ALO) acc[t] = mfma16(ld8(act_lo + base[t] + off), b.hi, acc[t]);
    }
  }
}

// LayerNorm statistics over the valid outputs of a layer (n < cout, p < 169).
template <int NTL>
__device__ __forceinline__ void ln_stats(const floatx4 (&acc)[NTL], int mt0, int ms,
                                         bool nvalid, float (*red)[NW], int& slot,
                                         float inv_count, float& mean, float& rstd) {
  const int kq = (threadIdx.x & 63) >> 4;
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT && nvalid) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (16 * (mt0 + t * ms) + 4 * kq + q < NP) s += acc[t][q];
    }
  mean = block_sum(s, red, slot) * inv_count;
  float v = 0.0f;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT && nvalid) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (16 * (mt0 + t * ms) + 4 * kq + q < NP) {
          const float d = acc[t][q] - mean;
          v += d * d;
        }
    }
  rstd = 1.0f / sqrtf(block_sum(v, red, slot) * inv_count + 1e-5f);
}

// relu(LN affine) of this wavefront's outputs: into the hi/lo activation
// planes, or (flat != nullptr) into flat[n * 169 + p].  g / bt: [NT][11][64][4]
// packed.
template <int NTL>
__device__ __forceinline__ void ln_write(const floatx4 (&acc)[NTL], int mt0, int ms, int ntile,
                                         bool nvalid, float mean, float rstd,
                                         const float* __restrict__ g, const float* __restrict__ bt,
                                         uint16_t* act_hi, uint16_t* act_lo, float* flat) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
  const int n = 16 * ntile + i16;
#pragma unroll
  for (int t = 0; t < NTL; ++t)
    if (mt0 + t * ms < MT && nvalid) {
      const int mt = mt0 + t * ms;
      const size_t gi = ((size_t)(ntile * MT + mt) * 64 + lane) * 4;
      const float4 gg = *reinterpret_cast<const float4*>(g + gi);
      const float4 bb = *reinterpret_cast<const float4*>(bt + gi);
      const float gv[4] = {gg.x, gg.y, gg.z, gg.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p = 16 * mt + 4 * kq + q;
        if (p < NP) {
          const float y = fmaxf((acc[t][q] - mean) * rstd * gv[q] + bv[q], 0.0f);
          if (flat) {
            flat[n * NP + p] = y;
          } else {
            const int i = ((p / HW + 1) * 15 + (p % HW) + 1) * CS + n;
            const __half h = __float2half_rn(y);
            act_hi[i] = __half_as_ushort(h);
            act_lo[i] = __half_as_ushort(__float2half_rn(y - __half2float(h)));
          }
        }
      }
    }
}

// Head GEMM for tiles nt0 + i (i < NTW): D[m][n] = sum_k A[m * as + k] W[k][n],
// A in LDS, W packed [tile][step][lane] in global memory.
template <int STEPS, int NTW>
__device__ __forceinline__ void head_gemm(const float* A, int as, const float* __restrict__ w,
                                          int nt0, floatx4 (&c)[NTW]) {
  const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
  const float* a = A + min(i16, SB - 1) * as + kq;   // rows past the batch repeat its last
  const float* b = w + (size_t)nt0 * STEPS * 64 + lane;
#pragma unroll
  for (int i = 0; i < NTW; ++i) c[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
  for (int j = 0; j < STEPS; ++j) {
    const float av = a[4 * j];
#pragma unroll
    for (int i = 0; i < NTW; ++i) c[i] = mfma(av, b[(i * STEPS + j) * 64], c[i]);
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
  const int m = threadIdx.x >> 4, c = threadIdx.x & 15;
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

__global__ __launch_bounds__(T, 1) void cnn_act_kernel(const qqt_cnn_args a, int items, int per) {
  __shared__ Lds s;
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63, i16 = lane & 15;

  // B operands of the 16->32 and 32->64 convs, resident for the whole kernel
  half8 b1h[S1], b1l[S1], b2h[S2], b2l[S2];
  const int n1 = w & 1, n2 = w;
#pragma unroll
  for (int j = 0; j < S1; ++j) {
    const size_t o = ((size_t)(n1 * S1 + j) * 64 + lane) * 8;
    b1h[j] = ld8(a.c1w + o);
    b1l[j] = ld8(a.c1w_lo + o);
  }
#pragma unroll
  for (int j = 0; j < S2; ++j) {
    const size_t o = ((size_t)(n2 * S2 + j) * 64 + lane) * 8;
    b2h[j] = ld8(a.c2w + o);
    b2l[j] = ld8(a.c2w_lo + o);
  }
  const float bias0 = a.c0b[i16], bias1 = a.c1b[16 * n1 + i16], bias2 = a.c2b[16 * n2 + i16];
  const float bias3 = a.c3b[i16];

  // position tiles per wavefront: conv0 / conv3 {w + 4i}, i < 3; conv1
  // {w/2 + 2i}, i < 6; conv2 all 11
  const int mt1 = w >> 1;

  for (int i = t; i < PP * CS; i += T) s.act[0][i] = s.act[1][i] = 0;
  for (int i = t; i < S0 * BFRAG; i += T) {
    s.wc0[0][i] = a.c0w[i];
    s.wc0[1][i] = a.c0w_lo[i];
  }
  for (int i = t; i < S3 * BFRAG; i += T) {
    s.wc3[0][i] = a.c3w[i];
    s.wc3[1][i] = a.c3w_lo[i];
  }
  auto breg1 = [&](int j) { return BFrag{b1h[j], b1l[j]}; };
  auto breg2 = [&](int j) { return BFrag{b2h[j], b2l[j]}; };
  auto blds0 = [&](int j) {
    return BFrag{ld8(s.wc0[0] + (j * 64 + lane) * 8), ld8(s.wc0[1] + (j * 64 + lane) * 8)};
  };
  auto blds3 = [&](int j) {
    return BFrag{ld8(s.wc3[0] + (j * 64 + lane) * 8), ld8(s.wc3[1] + (j * 64 + lane) * 8)};
  };

  int rslot = 0;                                   // reduction slot
  const int start = blockIdx.x * per, end = min(items, start + per);
  for (int ib = start; ib < end; ib += SB) {
    const int nb = min(SB, end - ib);
    for (int ii = 0; ii < nb; ++ii) {
      const int item = ib + ii;
      const int row = item / a.npid, slot = item % a.npid;
      const int pid = a.npid == 2 ? slot : a.pid0;
      __syncthreads();                                  // channels 0..13 free
      const uint16_t* ob = a.obs + (size_t)row * a.obs_stride;
      const int32_t* perm = a.view_perm + pid * C0;
      for (int i = t; i < C0 * NP; i += T) {          // exact in float16: hi plane only
        const int c = i / NP, p = i - c * NP;
        s.act[0][((p / HW + 1) * 15 + (p % HW) + 1) * CS + c] = ob[perm[c] * NP + p];
      }
      __syncthreads();

      float mean, rstd;
      {
        floatx4 acc[3];
        conv<0, S0, 3, false>(s.act[0], s.act[1], blds0, bias0, w, 4, acc);
        ln_stats<3>(acc, w, 4, true, s.red, rslot, 1.0f / (16 * NP), mean, rstd);
        ln_write<3>(acc, w, 4, 0, true, mean, rstd, a.ln0w, a.ln0b, s.act[0], s.act[1], nullptr);
      }
      __syncthreads();
      {
        floatx4 acc[6];
        conv<0, S1, 6, true>(s.act[0], s.act[1], breg1, bias1, mt1, 2, acc);
        ln_stats<6>(acc, mt1, 2, true, s.red, rslot, 1.0f / (32 * NP), mean, rstd);
        ln_write<6>(acc, mt1, 2, n1, true, mean, rstd, a.ln1w, a.ln1b, s.act[0], s.act[1],
                    nullptr);
      }
      __syncthreads();
      {
        floatx4 acc[MT];
        conv<1, S2, MT, true>(s.act[0], s.act[1], breg2, bias2, 0, 1, acc);
        ln_stats<MT>(acc, 0, 1, true, s.red, rslot, 1.0f / (64 * NP), mean, rstd);
        ln_write<MT>(acc, 0, 1, n2, true, mean, rstd, a.ln2w, a.ln2b, s.act[0], s.act[1],
                     nullptr);
      }
      __syncthreads();
      {
        floatx4 acc[3];
        conv<2, S3, 3, true>(s.act[0], s.act[1], blds3, bias3, w, 4, acc);
        const bool nv = i16 < 8;
        ln_stats<3>(acc, w, 4, nv, s.red, rslot, 1.0f / (8 * NP), mean, rstd);
        ln_write<3>(acc, w, 4, 0, nv, mean, rstd, a.ln3w, a.ln3b, s.act[0], s.act[1],
                    s.flat + ii * FS);
      }
    }
    __syncthreads();

    // ---------------- head over the batch's nb items (rows m of the GEMMs;
    // rows >= nb carry stale values that only reach their own rows)
    float* const h = s.flat + H_OFF;
    float* const h2 = s.flat + H2_OFF;
    float* const hy = s.flat + HY_OFF;
    float* const lg = s.flat + LG_OFF;
    {
      floatx4 c[2];
      head_gemm<L0, 2>(s.flat, FS, a.s0p, 2 * w, c);
      __syncthreads();                                  // flat fully read
      head_store(c[0], h, HS, 2 * w, a.s0b, false);
      head_store(c[1], h, HS, 2 * w + 1, a.s0b, false);
    }
    __syncthreads();
    head_ln(h, nb, a.s1w, a.s1b);
    __syncthreads();
    {
      floatx4 c[2];
      head_gemm<L1, 2>(h, HS, a.s3p, 2 * w, c);
      head_store(c[0], h2, HS, 2 * w, a.s3b, false);
      head_store(c[1], h2, HS, 2 * w + 1, a.s3b, false);
    }
    __syncthreads();
    head_ln(h2, nb, a.s4w, a.s4b);
    __syncthreads();
    {
      floatx4 c[3];
      head_gemm<L1, 3>(h2, HS, a.hp, 3 * w, c);
#pragma unroll
      for (int i = 0; i < 3; ++i) head_store(c[i], hy, HYS, 3 * w + i, a.hb, true);
    }
    __syncthreads();
    if (t < SB * 8) {                                   // output layer: item m, output o
      const int m = t >> 3, o = t & 7;
      const int base = o < 5 ? 0 : o < 7 ? 64 : 128;
      const float* x = hy + m * HYS + base;
      const float* wf = a.fw + o * 64;
      float acc = 0.0f;
#pragma unroll 8
      for (int k = 0; k < 64; ++k) acc += x[k] * wf[k];
      lg[m * 8 + o] = acc + a.fb[o];
    }
    __syncthreads();
    if (t < nb) {
      const int item = ib + t;
      const int row = item / a.npid, slot = item % a.npid;
      const int pid = a.npid == 2 ? slot : a.pid0;
      float l8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) l8[k] = lg[t * 8 + k];
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
      !a->ln3w || !a->ln3b || !a->s0p || !a->s0b ||
      !a->s1w || !a->s1b || !a->s3p || !a->s3b || !a->s4w || !a->s4b || !a->hp || !a->hb ||
      !a->fw || !a->fb) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: null pointer argument");
    return QQT_E_ARG;
  }
  if (((uintptr_t)a->ln0w | (uintptr_t)a->ln0b | (uintptr_t)a->ln1w | (uintptr_t)a->ln1b |
       (uintptr_t)a->ln2w | (uintptr_t)a->ln2b | (uintptr_t)a->ln3w | (uintptr_t)a->ln3b |
       (uintptr_t)a->c1w | (uintptr_t)a->c1w_lo | (uintptr_t)a->c2w | (uintptr_t)a->c2w_lo) & 15) {
    snprintf(g_err, sizeof(g_err),
             "qqt_cnn_act: LayerNorm tables and conv weights must be 16-byte aligned");
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
  const int grid = min(cu_count(), (items + SB - 1) / SB);
  const int per = (items + grid - 1) / grid;
  QQT_LAUNCH(QQT_KERNEL_CNN, cnn_act_kernel, dim3(grid), dim3(T), (hipStream_t)stream, *a,
             items, per);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "cnn launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
