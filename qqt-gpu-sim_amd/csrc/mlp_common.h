// MLP actor/critic pieces shared by the act kernels (mlp.hip, mlp_sparse.hip):
// operand types, the parameter-vector layout in LDS, the float16 hi/lo
// products and LayerNorms of the layers after the first, and the sampler.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // 16 bytes staged global -> LDS

constexpr int HID = 128;           // hidden width
constexpr int HEAD = 64;           // head hidden width
constexpr int NOUT = 8;            // 5 move + 2 bomb + 1 value

constexpr int NTHR = 512;          // 8 wavefronts

// parameter vectors staged in LDS (floats)
constexpr int V_B0 = 0, V_G1 = 128, V_BE1 = 256, V_B1 = 384, V_G2 = 512, V_BE2 = 640;
constexpr int V_BH = 768, V_BF = 960, V_N = 968;

constexpr int W1_HALVES = HID * HID;         // one plane of the layer-2 fragments (32 KB)
constexpr int WH_HALVES = 3 * HEAD * HID;    // one plane of the head-layer fragments (48 KB)
constexpr int WF_HALVES = 16 * 3 * HEAD;     // one plane of the output-layer fragments (6 KB)

struct Frag16 { half8 lo, hi; };   // 16 halves of one lane in one K block

__device__ __forceinline__ half8 as_h8(uint4 v) {
  union { uint4 u; half8 h; } c;
  c.u = v;
  return c.h;
}

__device__ __forceinline__ half8 as_h8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// 32 bytes of a first-layer weight fragment (32-byte aligned in w0).
__device__ __forceinline__ Frag16 load_b(const uint16_t* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  Frag16 f;
  f.lo = as_h8(q[0]);
  f.hi = as_h8(q[1]);
  return f;
}

// d = A B + c; A: weights (16 features x 32 K), B: activations (32 K x 16 rows).
__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// This lane's four values of feature tile t of an LDS parameter vector
// (features 16t + 4q .. +3).
__device__ __forceinline__ floatx4 vec4(const float* v, int t, int q) {
  return *reinterpret_cast<const floatx4*>(v + 16 * t + 4 * q);
}

// y (>= 0) -> element e of the float16 hi/lo fragment pair (y = hi + lo).
__device__ __forceinline__ void split_into(float y, half8& fh, half8& fl, int e) {
  const _Float16 h = (_Float16)y;
  fh[e] = h;
  fl[e] = (_Float16)(y - (float)h);
}

// LayerNorm(128) + ReLU of one 16-row tile in output layout (v[t] = features
// 16t + 4q .. +3 of row lane%16, bias included), then the float16 hi/lo B
// fragments of the next product (K step s = feature tiles 2s, 2s+1).  The
// affine parameters are read before the reductions so their LDS latency
// overlaps them.
__device__ __forceinline__ void ln_relu_split(const floatx4 (&v)[8], const float* gam,
                                              const float* bet, int q, half8 (&fh)[4],
                                              half8 (&fl)[4]) {
  floatx4 g[8], e[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    g[t] = vec4(gam, t, q);
    e[t] = vec4(bet, t, q);
  }
  float p = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) p += v[t][j];
  p += __shfl_xor(p, 16, 64);
  p += __shfl_xor(p, 32, 64);
  const float mean = p * (1.0f / HID);
  float d2 = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = v[t][j] - mean;
      d2 += d * d;
    }
  d2 += __shfl_xor(d2, 16, 64);
  d2 += __shfl_xor(d2, 32, 64);
  const float rstd = 1.0f / sqrtf(d2 * (1.0f / HID) + 1e-5f);
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      split_into(fmaxf((v[t][j] - mean) * rstd * g[t][j] + e[t][j], 0.0f), fh[t >> 1],
                 fl[t >> 1], 4 * (t & 1) + j);
}

// acc[t] += W(tile t) h over KS K steps: weight fragments from the LDS planes
// a_hi, a_lo ([tile][kstep][lane][8]), activation fragments bh, bl in
// registers.  Work goes in chunks of G tiles at one K step; the weight
// fragments of the next chunk are read while the current one multiplies,
// and each product runs over the chunk's G independent accumulators before
// the next product touches them.
template <int NT, int KS>
__device__ __forceinline__ void tail_gemm(floatx4 (&acc)[NT], const uint16_t* a_hi,
                                          const uint16_t* a_lo, const half8 (&bh)[KS],
                                          const half8 (&bl)[KS], int lane) {
  constexpr int G = NT < 4 ? NT : 4;
  static_assert(NT % G == 0, "whole chunks");
  constexpr int NG = NT / G, NC = KS * NG;   // chunk c: K step c / NG, tiles G * (c % NG) ..
  half8 fa[2][2][G];                          // [buffer][plane][tile of the chunk]
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
    for (int g = 0; g < G; ++g) acc[t0 + g] = mfma(f[0][g], bh[s], acc[t0 + g]);
#pragma unroll
    for (int g = 0; g < G; ++g) acc[t0 + g] = mfma(f[0][g], bl[s], acc[t0 + g]);
#pragma unroll
    for (int g = 0; g < G; ++g) acc[t0 + g] = mfma(f[1][g], bh[s], acc[t0 + g]);
  }
}

// sample_masked<5> restricted to the first n entries: entries k >= n get
// probability exactly zero (even when every real entry is masked), so their
// terms add exact zeros to the sums and the draw and log-probability equal
// sample_masked<n>'s.  Lets the move (n = 5) and bomb (n = 2) draws of a row
// run as one instruction stream on two lanes.
__device__ __forceinline__ int sample_masked_n(const float (&logit)[5], const uint8_t (&mask)[5],
                                               int n, float u, float* logp) {
  const float NEG = -3.4028234663852886e38f;
  float ml[5], ex[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) ml[k] = mask[k] && k < n ? logit[k] : NEG;
  float m = ml[0];
#pragma unroll
  for (int k = 1; k < 5; ++k) m = fmaxf(m, ml[k]);
#pragma unroll
  for (int k = 0; k < 5; ++k) ex[k] = k < n ? exp_q(ml[k] - m) : 0.0f;
  float sum = ex[0];
#pragma unroll
  for (int k = 1; k < 5; ++k) sum = sum + ex[k];
  const float t = u * sum;
  float run = 0.0f;
  int count = 0, last = 0;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    run = run + ex[k];
    count += run <= t;
    if (ex[k] > 0.0f) last = k;
  }
  const int a = count >= n ? last : count;
  *logp = (ml[a] - m) - log_q(sum);
  return a;
}

// Sampling inputs of one row, drawn by two lanes of its tail wavefront:
// half 0 (lane r) the move, half 1 (lane r + 16) the bomb.
struct RowSampler {
  bool on;
  uint8_t m[5];
  float u;
};

// Mask and uniform of one half of output row `row` for player pid (Philox
// when the caller passes no uniforms).
__device__ __forceinline__ RowSampler load_sampler(const qqt_mlp_args& a, bool on, int half,
                                                   int row, int pid, int oslots, int oslot) {
  RowSampler r;
  r.on = on;
#pragma unroll
  for (int k = 0; k < 5; ++k) r.m[k] = 0;
  r.u = 0.0f;
  if (on) {
    if (half == 0) {
#pragma unroll
      for (int k = 0; k < 5; ++k)
        r.m[k] = a.move_mask[(size_t)row * a.mm_row_stride + (size_t)pid * a.mm_pid_stride + k];
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        r.m[k] = a.bomb_mask[(size_t)row * a.bm_row_stride + (size_t)pid * a.bm_pid_stride + k];
    }
    const size_t o = (size_t)row * oslots + oslot;
    if (a.uniforms) {
      r.u = a.uniforms[o * 2 + half];
    } else {
      float u4[4];
      philox_block(a.seed, (uint32_t)row, a.tick, STREAM_POLICY, (uint32_t)((2 * pid) >> 2), u4);
      r.u = u4[(2 * pid + half) & 3];
    }
  }
  return r;
}

// The sparse-first-layer act kernel (mlp_sparse.hip): whether an argument
// block qualifies for it, and its launch.
bool mlp_sparse_eligible(const qqt_mlp_args& a);
int mlp_sparse_launch(const qqt_mlp_args& a, hipStream_t st);

}  // namespace qqt
