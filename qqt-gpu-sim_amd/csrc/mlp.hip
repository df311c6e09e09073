// MLP actor/critic forward + masked factored sampling for gfx950 (MFMA).
//
// Network (train/model.py:121-196, arch "mlp"): obs (B, C*H*W) float16 ->
// Linear(2366,128) -> LayerNorm -> ReLU -> Linear(128,128) -> LayerNorm ->
// ReLU -> three heads Linear(128,64) -> ReLU -> Linear(64, 5 | 2 | 1).
// A player's view permutation is folded into the first-layer weights, so one
// pass over the shared observation serves both players: layer 1 is a single
// (B x 2366) x (2366 x 256) GEMM whose columns are [player 0 | player 1].
//
// Workgroup = 4 wavefronts.  With both players, wavefront w computes rows
// [0, 64) of the tile for player w/2, output columns 64*(w%2) .. +63; with
// one player the four wavefronts cover 128 rows.  Every product runs on
// v_mfma_f32_16x16x32_f16 with float32 accumulation; LayerNorm statistics of
// a row are combined across the two wavefronts holding its 128 columns
// through LDS.  The observation is exact in float16 and the first layer's
// weights are rounded to float16 once; every later layer carries both its
// activations and its weights as float16 hi/lo pairs (x = hi + lo) and sums
// the three products hi*hi + hi*lo + lo*hi, which keeps logits within ~5e-4
// of a float32 forward even for large (orthogonal, gain sqrt 2) weights.  B operands are pre-arranged on the host (qqtsim/policy.py)
// so each lane reads 32 contiguous bytes per 64-deep K block:
//   frag[tile][kblock][lane][16] = W[16*tile + lane%16][64*kblock + 16*(lane/16) + j].
// The matching A fragment is the lane's 16 contiguous halves of its row, so
// the K order inside a block is a permutation shared by A and B.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HID = 128;           // hidden width
constexpr int HEAD = 64;           // head hidden width
constexpr int NOUT = 8;            // 5 move + 2 bomb + 1 value
constexpr int ROWS = 64;           // rows per wavefront pair

struct Frag16 { half8 lo, hi; };   // 16 halves of one lane in one K block

__device__ __forceinline__ half8 as_h8(uint4 v) {
  union { uint4 u; half8 h; } c;
  c.u = v;
  return c.h;
}

// 32 bytes of a B fragment (32-byte aligned in the packed weight buffers).
__device__ __forceinline__ Frag16 load_b(const uint16_t* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  Frag16 f;
  f.lo = as_h8(q[0]);
  f.hi = as_h8(q[1]);
  return f;
}

// 16 halves of an observation row starting at element k (4-byte aligned).
__device__ __forceinline__ Frag16 load_a_global(const uint16_t* row, int k, int kmax) {
  uint32_t v[8];
  const uint32_t* p = reinterpret_cast<const uint32_t*>(row + k);
  if (k + 16 <= kmax) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_nontemporal_load(p + i);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (k + 2 * i + 2 <= kmax) ? p[i] : 0u;
  }
  Frag16 f;
  f.lo = as_h8(make_uint4(v[0], v[1], v[2], v[3]));
  f.hi = as_h8(make_uint4(v[4], v[5], v[6], v[7]));
  return f;
}

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Activations as float16 hi/lo planes: h1 and h2 ([slot][plane][row][128])
// each fill 64 KB; the head hidden layer ([slot][plane][row][192], 96 KB)
// reuses both once every wavefront has finished reading h2.
constexpr int ACT_HALVES = 2 * 2 * ROWS * HID;   // one of h1 / h2
struct __align__(16) MlpLds {
  uint16_t act[2 * ACT_HALVES];
  float logit[2][ROWS][NOUT];
  float stat[2][2][ROWS];            // [slot][half][row] partial row sums
};
__device__ __forceinline__ uint16_t* h_at(uint16_t* base, int slot, int plane, int row, int col) {
  return base + ((slot * 2 + plane) * ROWS + row) * HID + col;
}
__device__ __forceinline__ uint16_t* hy_at(uint16_t* base, int slot, int plane, int row, int col) {
  return base + ((slot * 2 + plane) * ROWS + row) * (3 * HEAD) + col;
}
__device__ __forceinline__ void split_store(uint16_t* hi, uint16_t* lo, float y) {
  const __half h = __float2half_rn(y);
  *hi = __half_as_ushort(h);
  *lo = __half_as_ushort(__float2half_rn(y - __half2float(h)));
}

// Sum over the 16 lanes that share lane/16 (they hold the same rows).
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  return v;
}

// Bias + LayerNorm(128) + ReLU of a 64 x 64 accumulator block (this wave's
// half of one player's columns); writes float16 into dst[row][col].
__device__ __forceinline__ void ln_relu_store(floatx4 (&acc)[4][4], const float* bias,
                                              const float* gamma, const float* beta,
                                              MlpLds& s, int slot, int half, int lane,
                                              uint16_t* dst) {
  const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const float b = bias[64 * half + 16 * ct + r16];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[rt][ct][j] += b;
  }
  float mean[4][4], rstd[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float p = 0.0f;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) p += acc[rt][ct][j];
      p = sum16(p);
      if (r16 == 0) s.stat[slot][half][16 * rt + 4 * q + j] = p;
    }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 16 * rt + 4 * q + j;
      mean[rt][j] = (s.stat[slot][0][row] + s.stat[slot][1][row]) * (1.0f / HID);
    }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float p = 0.0f;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const float d = acc[rt][ct][j] - mean[rt][j];
        p += d * d;
      }
      p = sum16(p);
      if (r16 == 0) s.stat[slot][half][16 * rt + 4 * q + j] = p;
    }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 16 * rt + 4 * q + j;
      const float var = (s.stat[slot][0][row] + s.stat[slot][1][row]) * (1.0f / HID);
      rstd[rt][j] = 1.0f / sqrtf(var + 1e-5f);
    }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int col = 64 * half + 16 * ct + r16;
    const float ga = gamma[col], be = beta[col];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float y = (acc[rt][ct][j] - mean[rt][j]) * rstd[rt][j] * ga + be;
        y = fmaxf(y, 0.0f);
        const int row = 16 * rt + 4 * q + j;
        split_store(h_at(dst, slot, 0, row, col), h_at(dst, slot, 1, row, col), y);
      }
  }
}

// Masked categorical draw by inverse CDF on injected uniforms; same float32
// operation sequence as the host sampler (oracle/policy.py).
template <int K>
__device__ __forceinline__ int sample_masked(const float* logit, const uint8_t* mask, float u,
                                             float* logp) {
  const float NEG = -3.4028234663852886e38f;
  float ml[K], ex[K];
#pragma unroll
  for (int k = 0; k < K; ++k) ml[k] = mask[k] ? logit[k] : NEG;
  float m = ml[0];
#pragma unroll
  for (int k = 1; k < K; ++k) m = fmaxf(m, ml[k]);
#pragma unroll
  for (int k = 0; k < K; ++k) ex[k] = exp_q(ml[k] - m);
  float sum = ex[0];
#pragma unroll
  for (int k = 1; k < K; ++k) sum = sum + ex[k];
  const float t = u * sum;
  float run = 0.0f;
  int count = 0, last = 0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    run = run + ex[k];
    count += run <= t;
    if (ex[k] > 0.0f) last = k;
  }
  const int a = count >= K ? last : count;
  *logp = (ml[a] - m) - log_q(sum);
  return a;
}

__global__ __launch_bounds__(256) void mlp_act_kernel(const qqt_mlp_args a) {
  __shared__ MlpLds s;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int slot = w >> 1, half = w & 1;
  const bool two = a.npid == 2;
  const int pid = two ? slot : a.pid0;
  const int rows_per_block = two ? ROWS : 2 * ROWS;
  const int row0 = blockIdx.x * rows_per_block + (two ? 0 : slot * ROWS);
  const int lslot = slot;  // LDS slot: player slot (two) or row block (one)

  // ---------------- layer 1: (64 rows) x (64 columns of this player), K = 2366
  floatx4 acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* rowp[4];
  bool rowok[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int row = row0 + 16 * rt + r16;
    rowok[rt] = row < a.batch;
    rowp[rt] = a.obs + (size_t)(rowok[rt] ? row : 0) * a.obs_stride;
  }
  const uint16_t* wb = a.w0 + (size_t)((pid * 8 + half * 4) * a.kblocks0) * 64 * 16;
  for (int kb = 0; kb < a.kblocks0; ++kb) {
    const int k = 64 * kb + 16 * q;
    Frag16 af[4], bf[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      af[rt] = rowok[rt] ? load_a_global(rowp[rt], k, a.k0) : Frag16{};
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      bf[ct] = load_b(wb + ((size_t)(ct * a.kblocks0 + kb) * 64 + lane) * 16);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        acc[rt][ct] = mfma(af[rt].lo, bf[ct].lo, acc[rt][ct]);
        acc[rt][ct] = mfma(af[rt].hi, bf[ct].hi, acc[rt][ct]);
      }
  }
  uint16_t* const H1 = s.act;
  uint16_t* const H2 = s.act + ACT_HALVES;
  ln_relu_store(acc, a.b0, a.ln1_w, a.ln1_b, s, lslot, half, lane, H1);
  __syncthreads();

  // ---------------- layer 2: K = 128 from LDS
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    Frag16 ah[4], al[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const uint4* ph = reinterpret_cast<const uint4*>(h_at(H1, lslot, 0, 16 * rt + r16, 64 * kb + 16 * q));
      const uint4* pl = reinterpret_cast<const uint4*>(h_at(H1, lslot, 1, 16 * rt + r16, 64 * kb + 16 * q));
      ah[rt].lo = as_h8(ph[0]); ah[rt].hi = as_h8(ph[1]);
      al[rt].lo = as_h8(pl[0]); al[rt].hi = as_h8(pl[1]);
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const size_t off = ((size_t)((half * 4 + ct) * 2 + kb) * 64 + lane) * 16;
      const Frag16 bh = load_b(a.w1 + off), bl = load_b(a.w1_lo + off);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        acc[rt][ct] = mfma(ah[rt].lo, bh.lo, acc[rt][ct]);
        acc[rt][ct] = mfma(ah[rt].hi, bh.hi, acc[rt][ct]);
        acc[rt][ct] = mfma(ah[rt].lo, bl.lo, acc[rt][ct]);
        acc[rt][ct] = mfma(ah[rt].hi, bl.hi, acc[rt][ct]);
        acc[rt][ct] = mfma(al[rt].lo, bh.lo, acc[rt][ct]);
        acc[rt][ct] = mfma(al[rt].hi, bh.hi, acc[rt][ct]);
      }
    }
  }
  ln_relu_store(acc, a.b1, a.ln2_w, a.ln2_b, s, lslot, half, lane, H2);
  __syncthreads();

  // ---------------- heads, first layer: 192 hidden columns (this wave: 96)
  {
    floatx4 hac[4][6];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 6; ++ct) hac[rt][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      Frag16 ah[4], al[4];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const uint4* ph = reinterpret_cast<const uint4*>(h_at(H2, lslot, 0, 16 * rt + r16, 64 * kb + 16 * q));
        const uint4* pl = reinterpret_cast<const uint4*>(h_at(H2, lslot, 1, 16 * rt + r16, 64 * kb + 16 * q));
        ah[rt].lo = as_h8(ph[0]); ah[rt].hi = as_h8(ph[1]);
        al[rt].lo = as_h8(pl[0]); al[rt].hi = as_h8(pl[1]);
      }
#pragma unroll
      for (int ct = 0; ct < 6; ++ct) {
        const size_t off = ((size_t)((half * 6 + ct) * 2 + kb) * 64 + lane) * 16;
        const Frag16 bh = load_b(a.wh + off), bl = load_b(a.wh_lo + off);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          hac[rt][ct] = mfma(ah[rt].lo, bh.lo, hac[rt][ct]);
          hac[rt][ct] = mfma(ah[rt].hi, bh.hi, hac[rt][ct]);
          hac[rt][ct] = mfma(ah[rt].lo, bl.lo, hac[rt][ct]);
          hac[rt][ct] = mfma(ah[rt].hi, bl.hi, hac[rt][ct]);
          hac[rt][ct] = mfma(al[rt].lo, bh.lo, hac[rt][ct]);
          hac[rt][ct] = mfma(al[rt].hi, bh.hi, hac[rt][ct]);
        }
      }
    }
    __syncthreads();  // every wavefront is done reading h2: the head layer reuses it
#pragma unroll
    for (int ct = 0; ct < 6; ++ct) {
      const int col = 96 * half + 16 * ct + r16;
      const float b = a.bh[col];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 16 * rt + 4 * q + j;
          split_store(hy_at(s.act, lslot, 0, row, col), hy_at(s.act, lslot, 1, row, col),
                      fmaxf(hac[rt][ct][j] + b, 0.0f));
        }
    }
  }
  __syncthreads();

  // ---------------- heads, output layer: 192 -> 8 (block diagonal), MFMA
  {
    floatx4 oac[2] = {floatx4{0.0f, 0.0f, 0.0f, 0.0f}, floatx4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int kb = 0; kb < 3; ++kb) {
      const size_t off = ((size_t)kb * 64 + lane) * 16;
      const Frag16 bh = load_b(a.wf + off), bl = load_b(a.wf_lo + off);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int rt = 2 * half + i;
        const uint4* ph = reinterpret_cast<const uint4*>(hy_at(s.act, lslot, 0, 16 * rt + r16, 64 * kb + 16 * q));
        const uint4* pl = reinterpret_cast<const uint4*>(hy_at(s.act, lslot, 1, 16 * rt + r16, 64 * kb + 16 * q));
        const half8 h0 = as_h8(ph[0]), h1 = as_h8(ph[1]), l0 = as_h8(pl[0]), l1 = as_h8(pl[1]);
        oac[i] = mfma(h0, bh.lo, oac[i]);
        oac[i] = mfma(h1, bh.hi, oac[i]);
        oac[i] = mfma(h0, bl.lo, oac[i]);
        oac[i] = mfma(h1, bl.hi, oac[i]);
        oac[i] = mfma(l0, bh.lo, oac[i]);
        oac[i] = mfma(l1, bh.hi, oac[i]);
      }
    }
    if (r16 < NOUT) {
      const float b = a.bf[r16];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s.logit[lslot][16 * (2 * half + i) + 4 * q + j][r16] = oac[i][j] + b;
    }
  }
  __syncthreads();

  // ---------------- outputs and sampling: one thread per (row, player slot)
  if (threadIdx.x < 2 * ROWS) {
    const int slot2 = threadIdx.x >> 6, rl = threadIdx.x & 63;
    const int pid2 = two ? slot2 : a.pid0;
    const int row = blockIdx.x * rows_per_block + (two ? rl : slot2 * ROWS + rl);
    const int oslot = two ? slot2 : 0;
    if (row < a.batch) {
      const float* lg = s.logit[slot2][rl];
      const size_t o = (size_t)row * a.npid + oslot;
      if (a.logits_out) {
#pragma unroll
        for (int k = 0; k < NOUT; ++k) a.logits_out[o * NOUT + k] = lg[k];
      }
      if (a.value_out) a.value_out[o] = lg[7];
      if (a.sample) {
        uint8_t mm[5], bm[2];
#pragma unroll
        for (int k = 0; k < 5; ++k)
          mm[k] = a.move_mask[(size_t)row * a.mm_row_stride + (size_t)pid2 * a.mm_pid_stride + k];
#pragma unroll
        for (int k = 0; k < 2; ++k)
          bm[k] = a.bomb_mask[(size_t)row * a.bm_row_stride + (size_t)pid2 * a.bm_pid_stride + k];
        float um, ub;
        if (a.uniforms) {
          um = a.uniforms[o * 2 + 0];
          ub = a.uniforms[o * 2 + 1];
        } else {
          float u4[4];
          philox_block(a.seed, (uint32_t)row, a.tick, STREAM_POLICY, (uint32_t)((2 * pid2) >> 2), u4);
          um = u4[(2 * pid2) & 3];
          ub = u4[(2 * pid2 + 1) & 3];
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
  if (a->batch <= 0 || (a->npid != 1 && a->npid != 2) || a->pid0 < 0 || a->pid0 > 3 ||
      a->k0 <= 0 || a->k0 % 2 || a->kblocks0 != (a->k0 + 63) / 64 || a->obs_stride < a->k0 ||
      (a->obs_stride % 2) || (((uintptr_t)a->obs) & 3)) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: bad shape/stride/alignment");
    return QQT_E_ARG;
  }
  if (a->sample && (!a->move_mask || !a->bomb_mask)) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: sampling needs masks");
    return QQT_E_ARG;
  }
  const int rows_per_block = a->npid == 2 ? ROWS : 2 * ROWS;
  const int blocks = (a->batch + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL(mlp_act_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "mlp launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
