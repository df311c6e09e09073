// cnn actor/critic forward + masked factored sampling for gfx950 (the
// reference's ActorCritic(arch="cnn"), train/model.py:79-96, 186-190).
//
// Network per player view: conv0 3x3 (C=14 -> 16, the view permutation
// folded into its input channels) -> LayerNorm([16,13,13]) -> ReLU -> conv
// 3x3 16 -> 32 -> LN -> ReLU -> conv 3x3 32 -> 64 -> LN -> ReLU -> conv 1x1
// 64 -> 8 -> LN -> ReLU -> flatten (1352) -> Linear(1352,128) -> LN ->
// ReLU -> Linear(128,128) -> LN -> ReLU -> three heads 128 -> 64 -> ReLU ->
// 5 | 2 | 1.  Every LayerNorm normalises one sample over all of its values
// with an elementwise affine of the same shape.
//
// One workgroup (8 wavefronts) per (observation row, player).  The feature
// maps live in LDS: the conv input as zero-padded 15 x 15 planes [C][225],
// the conv output as [C][176] (169 positions padded to 11 row tiles of 16).
// Each conv is an implicit GEMM on v_mfma_f32_16x16x4_f32 (float32 operands,
// so the trunk is float32 throughout): M = positions (11 tiles), N = output
// channels (16 per tile), K = C_in x taps with k = ci * 9 + 3 dy + dx; lane l
// reads its A element from the padded plane at the position of row l % 16
// shifted by the tap of K row k0 + l / 16, and its B element from the K-major
// weight [K][C_out] in global memory (L2-resident, shared by every
// workgroup).  The per-sample LayerNorms reduce over the workgroup (two
// passes: mean, then squared deviations).  The MLP head runs as
// matrix-vector products on the vector units, four (or two, eight) threads
// per output with a shuffle reduction; sampling as in the mlp kernel.

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

constexpr int T = 512;                 // threads
constexpr int NW = T / 64;             // wavefronts
constexpr int HW = 13, NP = 169, NPT = 176, PL = 225;   // grid, positions, padded
constexpr int C0 = 14, F0 = 16, F1 = 32, F2 = 64, F3 = 8;
constexpr int FLAT = F3 * NP;          // 1352
constexpr int HID = 128, HEAD = 64;

struct __align__(16) Lds {
  float in[F2][PL];                    // padded conv input planes
  float out[F2][NPT];                  // conv output [channel][position]
  float red[NW];
  float h[HID], h2[HID], hy[3 * HEAD], logit[8];
};

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += red[i];
  __syncthreads();
  return s;
}

// out[n][p] = bias[n] + sum_k A[p][k] W[k][n]; A[p][k] = in[ci][pad(p) + tap(k)].
template <int CIN, int COUT, int KS>
__device__ __forceinline__ void conv(const float (*in)[PL], const float* __restrict__ w,
                                     const float* __restrict__ bias, float (*out)[NPT]) {
  constexpr int TAPS = KS * KS, K = CIN * TAPS, KP = (K + 3) & ~3;
  constexpr int NT = (COUT + 15) / 16, MT = NPT / 16;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i16 = lane & 15, kq = lane >> 4;
  for (int tile = wv; tile < MT * NT; tile += NW) {
    const int mt = tile % MT, nt = tile / MT;
    const int p = min(16 * mt + i16, NP - 1);        // A row: position (rows past 168 unused)
    const int pbase = (p / HW) * 15 + (p % HW);      // padded (y, x) of tap (0, 0)
    const int n = 16 * nt + i16;                     // B column: output channel
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int k0 = 0; k0 < KP; k0 += 4) {
      const int k = k0 + kq;
      float av = 0.0f, bv = 0.0f;
      if (k < K) {
        const int ci = k / TAPS, tap = k % TAPS;
        const int off = KS == 3 ? (tap / 3) * 15 + (tap % 3) : 16;   // 1x1: the centre
        av = in[ci][pbase + off];
        if (n < COUT) bv = w[k * COUT + n];
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
    if (n < COUT) {
      const float b = bias[n];
#pragma unroll
      for (int q = 0; q < 4; ++q) out[n][16 * mt + 4 * kq + q] = acc[q] + b;
    }
  }
}

// LayerNorm over out[0..C)[0..169) with elementwise affine gamma/beta [C*169],
// ReLU; results to the padded planes (or, flat, to dst[c*169 + p]).
template <int C>
__device__ __forceinline__ void ln_relu(float (*out)[NPT], const float* __restrict__ gam,
                                        const float* __restrict__ bet, float (*dst)[PL],
                                        float* flat, float* red) {
  float s = 0.0f;
  for (int i = threadIdx.x; i < C * NP; i += T) s += out[i / NP][i % NP];
  const float mean = block_sum(s, red) / (float)(C * NP);
  float q = 0.0f;
  for (int i = threadIdx.x; i < C * NP; i += T) {
    const float d = out[i / NP][i % NP] - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(block_sum(q, red) / (float)(C * NP) + 1e-5f);
  for (int i = threadIdx.x; i < C * NP; i += T) {
    const int c = i / NP, p = i % NP;
    const float y = fmaxf((out[c][p] - mean) * rstd * gam[i] + bet[i], 0.0f);
    if (flat) flat[i] = y;
    else dst[c][(p / HW + 1) * 15 + (p % HW) + 1] = y;
  }
}

// LayerNorm(128) + ReLU of v in place, by the first wavefront (2 values per lane).
__device__ __forceinline__ void ln128(float* v, const float* __restrict__ gam,
                                      const float* __restrict__ bet) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    float a = v[l], b = v[l + 64];
    float s = a + b;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    const float mean = s / (float)HID;
    float q = (a - mean) * (a - mean) + (b - mean) * (b - mean);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) q += __shfl_xor(q, m, 64);
    const float rstd = 1.0f / sqrtf(q / (float)HID + 1e-5f);
    v[l] = fmaxf((a - mean) * rstd * gam[l] + bet[l], 0.0f);
    v[l + 64] = fmaxf((b - mean) * rstd * gam[l + 64] + bet[l + 64], 0.0f);
  }
}

// y[o] = b[o] + sum_k x[k] wt[k][o] for o < NO, with G threads per output
// (a power of two, consecutive lanes) summing k = j, j + G, ...
template <int NI, int NO, int G>
__device__ __forceinline__ void matvec(const float* x, const float* __restrict__ wt,
                                       const float* __restrict__ b, float* y) {
  const int o = threadIdx.x / G, j = threadIdx.x % G;
  float acc = 0.0f;
  if (o < NO)
    for (int k = j; k < NI; k += G) acc += x[k] * wt[k * NO + o];
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (o < NO && j == 0) y[o] = acc + b[o];
}

__global__ __launch_bounds__(T) void cnn_act_kernel(const qqt_cnn_args a) {
  __shared__ Lds s;
  const int row = blockIdx.x / a.npid, slot = blockIdx.x % a.npid;
  const int pid = a.npid == 2 ? slot : a.pid0;
  const int t = threadIdx.x;

  // zero the padded planes, then the observation row into channels 0..13
  for (int i = t; i < F2 * PL; i += T) (&s.in[0][0])[i] = 0.0f;
  __syncthreads();
  const uint16_t* ob = a.obs + (size_t)row * a.obs_stride;
  for (int i = t; i < C0 * NP; i += T) {
    const int c = i / NP, p = i % NP;
    s.in[c][(p / HW + 1) * 15 + (p % HW) + 1] = __half2float(__ushort_as_half(ob[i]));
  }
  __syncthreads();

  conv<C0, F0, 3>(s.in, a.c0w + (size_t)pid * C0 * 9 * F0, a.c0b, s.out);
  __syncthreads();
  ln_relu<F0>(s.out, a.ln0w, a.ln0b, s.in, nullptr, s.red);
  __syncthreads();
  conv<F0, F1, 3>(s.in, a.c1w, a.c1b, s.out);
  __syncthreads();
  ln_relu<F1>(s.out, a.ln1w, a.ln1b, s.in, nullptr, s.red);
  __syncthreads();
  conv<F1, F2, 3>(s.in, a.c2w, a.c2b, s.out);
  __syncthreads();
  ln_relu<F2>(s.out, a.ln2w, a.ln2b, s.in, nullptr, s.red);
  __syncthreads();
  conv<F2, F3, 1>(s.in, a.c3w, a.c3b, s.out);
  __syncthreads();
  float* const flat = &s.in[0][0];                    // the planes are free now
  ln_relu<F3>(s.out, a.ln3w, a.ln3b, s.in, flat, s.red);
  __syncthreads();

  // shared MLP and heads
  matvec<FLAT, HID, 4>(flat, a.s0wt, a.s0b, s.h);
  __syncthreads();
  ln128(s.h, a.s1w, a.s1b);
  __syncthreads();
  matvec<HID, HID, 4>(s.h, a.s3wt, a.s3b, s.h2);
  __syncthreads();
  ln128(s.h2, a.s4w, a.s4b);
  __syncthreads();
  matvec<HID, 3 * HEAD, 2>(s.h2, a.hwt, a.hb, s.hy);
  __syncthreads();
  for (int i = t; i < 3 * HEAD; i += T) s.hy[i] = fmaxf(s.hy[i], 0.0f);
  __syncthreads();
  if (t < 8 * 8) {                                     // outputs: 8 threads each, 8 terms
    const int o = t >> 3, j = t & 7;
    const int base = o < 5 ? 0 : o < 7 ? HEAD : 2 * HEAD;
    float acc = 0.0f;
    for (int k = j; k < HEAD; k += 8) acc += s.hy[base + k] * a.fw[o * HEAD + k];
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if (j == 0) s.logit[o] = acc + a.fb[o];
  }
  __syncthreads();

  if (t == 0) {
    const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;
    const int oslot = a.npid == 2 ? slot : a.out_slot;
    const size_t o = (size_t)row * oslots + oslot;
    if (a.logits_out) {
#pragma unroll
      for (int k = 0; k < 8; ++k) a.logits_out[o * 8 + k] = s.logit[k];
    }
    if (a.value_out) a.value_out[o] = s.logit[7];
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
        philox_block(a.seed, (uint32_t)row, a.tick, STREAM_POLICY, (uint32_t)((2 * pid) >> 2), u4);
        um = u4[(2 * pid) & 3];
        ub = u4[(2 * pid + 1) & 3];
      }
      float lpm, lpb;
      const int am = sample_masked<5>(s.logit, mm, um, &lpm);
      const int ab = sample_masked<2>(s.logit + 5, bm, ub, &lpb);
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

}  // namespace cnn
}  // namespace qqt

extern "C" {

int qqt_cnn_act(const qqt_cnn_args* a, void* stream) {
  using namespace qqt;
  using namespace qqt::cnn;
  g_err[0] = 0;
  if (!a || !a->obs || !a->c0w || !a->c0b || !a->ln0w || !a->ln0b || !a->c1w || !a->c1b ||
      !a->ln1w || !a->ln1b || !a->c2w || !a->c2b || !a->ln2w || !a->ln2b || !a->c3w ||
      !a->c3b || !a->ln3w || !a->ln3b || !a->s0wt || !a->s0b || !a->s1w || !a->s1b ||
      !a->s3wt || !a->s3b || !a->s4w || !a->s4b || !a->hwt || !a->hb || !a->fw || !a->fb) {
    snprintf(g_err, sizeof(g_err), "qqt_cnn_act: null pointer argument");
    return QQT_E_ARG;
  }
  if (a->batch <= 0 || (a->npid != 1 && a->npid != 2) || a->w_players < a->npid ||
      a->w_players > 4 || a->pid0 < 0 || (a->npid == 1 && a->pid0 >= a->w_players) ||
      a->obs_stride < C0 * NP) {
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
  QQT_LAUNCH(QQT_KERNEL_CNN, cnn_act_kernel, dim3(a->batch * a->npid), dim3(T),
             (hipStream_t)stream, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "cnn launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
