// The PPO minibatch loss and its backward through the mlp ActorCritic above
// the first layer (train/ppo.py:401-421 on train/model.py:140-153, 192-196,
// 215-256), fused: from z1 = x W0^T + b0 of each row to the gradient dz1
// that the first layer's weight gradient (csrc/mlp_grad.hip) consumes.
//
// Forward, per row: LayerNorm 1 + ReLU -> Linear(128,128) -> LayerNorm 2 +
// ReLU -> the three heads' Linear(128,64) + ReLU -> move (5), bomb (2) and
// value (1) outputs; masked log-softmax, log-prob of the taken actions,
// entropies.  Loss terms (the reference's, with torch's gradient rules:
// min/max ties split the gradient in halves, clamp passes it at its bounds):
//   ratio = exp(logp - old_logp)
//   pg    = -mean(min(ratio A, clamp(ratio, 1-e, 1+e) A))
//   vf    = 0.5 mean(max((v - R)^2, (old_v + clamp(v - old_v, -e, e) - R)^2))
//   loss  = pg + value_coef vf - entropy_coef mean(H_move + H_bomb)
// Backward, per row, through the heads, LayerNorm 2, Linear(128,128) and
// LayerNorm 1.  Float32 throughout; the four products (K and N of 128 and
// 192) on v_mfma_f32_16x16x4_f32, the 16 rows as one M tile.
//
// One workgroup of 512 threads takes 16 rows; activations live in LDS
// (rows padded by 4 floats against bank conflicts; two workgroups per CU).  Outputs: dz1, and for the weight
// gradients the caller forms as batched products (their reduction runs over
// the whole minibatch): h1, dz2, h2, hy, dhy and the output-layer gradients
// dl; per-workgroup sums of the LayerNorm parameter gradients and of the
// loss statistics.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

namespace ppo {

constexpr int R = 16;        // rows per workgroup
constexpr int T = 512;       // threads: 8 wavefronts (one per column tile of a 128-wide product)
constexpr int TR = 256;      // threads of the row-wise phases (16 per row)
static_assert(R * 8 * 4 == T, "the output layer takes four threads per (row, output)");
constexpr int H = 128;       // hidden width
constexpr int HY = 192;      // three heads x 64
constexpr int HP = H + 4, HYP = HY + 4;   // padded LDS row strides
constexpr float LN_EPS = 1e-5f;

typedef float floatx4 __attribute__((ext_vector_type(4)));

// 48 KB, so three workgroups share a CU.  The LayerNorms keep their inputs
// and per-row statistics, not the normalised values: the backward recomputes
// xh = (z - mean) rstd and the ReLU mask xh gamma + beta > 0 with the
// forward's operations (bit for bit).  Buffers are reused by liveness.
struct __align__(16) Lds {
  float z1[R][HP];    // LayerNorm 1's input, for the whole kernel
  float z2[R][HP];    // LayerNorm 2's input until its backward, then dh1 -> dz1
  float hb[R][HP];    // h1 (stored out after its product), then h2
  float g[R][HP];     // dh2 -> dz2
  float y[R][HYP];    // hy (stored out when the backward starts), then dhy
  float logit[R][8], dl[R][8];
  float mean1[R], rstd1[R], mean2[R], rstd2[R];
  float stat[R][5];
};

// Y[r][n] = sum_k X[r][k] W[k][n] (+ bias[n]) for the 16 rows, X and Y in
// LDS.  W [K][N] comes from global memory as MFMA fragments: value i of lane
// l in group g of column tile t is W[16 g + 4(l/16) + i][16 t + l%16], so a
// lane's four B values of a 16-k group are one 16-byte load, paired with its
// four A values X[l%16][16 g + 4(l/16) .. + 3] (one 16-byte LDS read).  MFMA
// 16x16x4 f32 holds D[4(l/16)+q][l%16] in lane l.  Wavefront w takes column
// tiles w, w+8, ...
template <int K, int N, int LDX, int LDY, bool RELU = false>
__device__ __forceinline__ void gemm(const float (*X)[LDX], const float* __restrict__ W,
                                     const float* __restrict__ bias, float (*Y)[LDY]) {
  constexpr int CT = N / 16, KG = K / 16;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i16 = lane & 15, kq = lane >> 4;
  const float4* F = reinterpret_cast<const float4*>(W);
  for (int ct = w; ct < CT; ct += T / 64) {
    const int col = 16 * ct + i16;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int g = 0; g < KG; ++g) {
      const float4 av = *reinterpret_cast<const float4*>(&X[i16][16 * g + 4 * kq]);
      const float4 bv = F[((size_t)ct * KG + g) * 64 + lane];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
    }
    const float b = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) Y[4 * kq + q][col] = RELU ? fmaxf(acc[q] + b, 0.0f) : acc[q] + b;
  }
}

// Sum over the 16 lanes of one row (threads 16r .. 16r+15).
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, 16);
  return v;
}

// LayerNorm + ReLU of Z[r] into h, keeping the row's mean and rstd; 16
// threads per row, feature c = lane + 16 i.
__device__ __forceinline__ void ln_forward(const float (*Z)[HP], const float* __restrict__ gam,
                                           const float* __restrict__ bet, float (*h)[HP],
                                           float* mean_out, float* rstd_out) {
  const int r = threadIdx.x >> 4, j = threadIdx.x & 15;
  float v[8];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = Z[r][j + 16 * i];
    s += v[i];
  }
  const float mean = sum16(s) / (float)H;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(sum16(q) / (float)H + LN_EPS);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = j + 16 * i;
    const float x = (v[i] - mean) * rstd;
    h[r][c] = fmaxf(x * gam[c] + bet[c], 0.0f);
  }
  if (j == 0) {
    mean_out[r] = mean;
    rstd_out[r] = rstd;
  }
}

// The forward's normalised value of (r, c) and whether its ReLU passed.
__device__ __forceinline__ float ln_xh(const float (*Z)[HP], const float* mean, const float* rstd,
                                       int r, int c) {
  return (Z[r][c] - mean[r]) * rstd[r];
}

// LayerNorm backward with the ReLU after it: dy = G (gradient of the ReLU
// output) where h > 0; dz = rstd (dx - mean(dx) - xh mean(dx xh)), dx =
// dy gamma.  Writes dz over G.
__device__ __forceinline__ void ln_backward(float (*G)[HP], const float (*Z)[HP],
                                            const float* mean, const float* rstd,
                                            const float* __restrict__ gam,
                                            const float* __restrict__ bet) {
  const int r = threadIdx.x >> 4, j = threadIdx.x & 15;
  float dx[8], x[8];
  float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = j + 16 * i;
    x[i] = ln_xh(Z, mean, rstd, r, c);
    const float dy = x[i] * gam[c] + bet[c] > 0.0f ? G[r][c] : 0.0f;
    dx[i] = dy * gam[c];
    s1 += dx[i];
    s2 += dx[i] * x[i];
  }
  const float m1 = sum16(s1) / (float)H, m2 = sum16(s2) / (float)H;
  const float rs = rstd[r];
#pragma unroll
  for (int i = 0; i < 8; ++i) G[r][j + 16 * i] = rs * ((dx[i] - m1) - x[i] * m2);
}

// Per-workgroup sums over the rows of dgamma = dy xh and dbeta = dy, where
// dy = G (before ln_backward overwrote it) masked by h > 0.
// Index of (row r, column c) of an n-column output: row-major, or in
// t_chunk-row chunks stored [chunk][n][t_chunk].
__device__ __forceinline__ size_t out_at(int64_t r, int c, int n, int t_chunk) {
  return t_chunk > 0 ? ((size_t)(r / t_chunk) * n + c) * t_chunk + (size_t)(r % t_chunk)
                     : (size_t)r * n + c;
}

__device__ __forceinline__ void ln_param_sums(const float (*G)[HP], const float (*Z)[HP],
                                              const float* mean, const float* rstd,
                                              const float* __restrict__ gam,
                                              const float* __restrict__ bet, float* out_g,
                                              float* out_b) {
  const int c = threadIdx.x;
  if (c < H) {
    float sg = 0.0f, sb = 0.0f;
    for (int r = 0; r < R; ++r) {
      const float x = ln_xh(Z, mean, rstd, r, c);
      const float dy = x * gam[c] + bet[c] > 0.0f ? G[r][c] : 0.0f;
      sg += dy * x;
      sb += dy;
    }
    out_g[c] = sg;
    out_b[c] = sb;
  }
}

// Masked categorical over K logits: log-softmax (masked entries at the
// float32 minimum, as torch.where(mask, logits, finfo.min)), probabilities,
// entropy H = -sum p log p over the clamped normalised logits.
template <int K>
__device__ __forceinline__ void masked_cat(const float* lg, const uint8_t* mask, float* lp, float* p,
                                           float* ent) {
  const float NEG = -3.4028234663852886e38f;
  float z[K];
  float m = NEG;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    z[k] = mask[k] ? lg[k] : NEG;
    m = fmaxf(m, z[k]);
  }
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) s += expf(z[k] - m);
  const float lse = m + logf(s);
  float h = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    lp[k] = fmaxf(z[k] - lse, NEG);
    p[k] = expf(z[k] - lse);
    h -= lp[k] * p[k];
  }
  *ent = h;
}

__global__ __launch_bounds__(T) void ppo_grad_kernel(const qqt_ppo_args a) {
  __shared__ Lds s;
  const int t = threadIdx.x;
  const int row0 = blockIdx.x * R;
  const int nrows = min(R, a.batch - row0);

  // ---- z1 tile (rows past the batch are zero and masked out of every sum)
  for (int i = t; i < R * H / 4; i += T) {
    const int r = i / (H / 4), c4 = i % (H / 4);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < nrows) v = reinterpret_cast<const float4*>(a.z1 + (size_t)(row0 + r) * H)[c4];
    *reinterpret_cast<float4*>(&s.z1[r][4 * c4]) = v;
  }
  __syncthreads();
  if (t < TR) ln_forward(s.z1, a.ln1_w, a.ln1_b, s.hb, s.mean1, s.rstd1);
  __syncthreads();
  gemm<H, H, HP, HP>(s.hb, a.w1t, a.b1, s.z2);              // z2 = h1 W1^T + b1
  __syncthreads();
  for (int i = t; i < R * H; i += T) {                      // h1 out before h2 takes its place
    const int r = i / H, c = i % H;
    if (r < nrows) a.h1[(size_t)(row0 + r) * H + c] = s.hb[r][c];
  }
  __syncthreads();
  if (t < TR) ln_forward(s.z2, a.ln2_w, a.ln2_b, s.hb, s.mean2, s.rstd2);
  __syncthreads();
  gemm<H, HY, HP, HYP, true>(s.hb, a.wht, a.bh, s.y);       // heads' hidden layers + ReLU
  __syncthreads();
  {                                                           // outputs: 5 move, 2 bomb, value
    // thread t: row t / 32, output (t / 4) % 8, quarter t % 4 of its 64 inputs;
    // the quarters meet by two lane exchanges
    const int r = t >> 5, j = (t >> 2) & 7, part = t & 3;
    const int base = (j < 5 ? 0 : j < 7 ? 64 : 128) + 16 * part;
    const float* wj = a.wf + j * 64 + 16 * part;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) acc += s.y[r][base + k] * wj[k];
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    if (part == 0) s.logit[r][j] = a.bf[j] + acc;
  }
  __syncthreads();

  // ---- loss terms and output gradients, one thread per row
  if (t < R) {
    const int r = t;
    float dl[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float st[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < nrows) {
      const size_t g = (size_t)(row0 + r);                       // minibatch row (outputs)
      const size_t gi = a.row_index                              // its inputs' row
          ? (size_t)min(max(a.row_index[g], (int64_t)0), a.src_rows - 1) : g;
      uint8_t mm[5], bm[2];
#pragma unroll
      for (int k = 0; k < 5; ++k) mm[k] = a.move_mask[gi * 5 + k];
#pragma unroll
      for (int k = 0; k < 2; ++k) bm[k] = a.bomb_mask[gi * 2 + k];
      const int am = (int)a.actions[gi * 2 + 0], ab = (int)a.actions[gi * 2 + 1];
      float lpm[5], pm[5], lpb[2], pb[2], hm, hb;
      masked_cat<5>(&s.logit[r][0], mm, lpm, pm, &hm);
      masked_cat<2>(&s.logit[r][5], bm, lpb, pb, &hb);
      float lpa = 0.0f, lpb_a = 0.0f;                          // select, not index (registers)
#pragma unroll
      for (int k = 0; k < 5; ++k) lpa = k == am ? lpm[k] : lpa;
#pragma unroll
      for (int k = 0; k < 2; ++k) lpb_a = k == ab ? lpb[k] : lpb_a;
      const float logp = lpa + lpb_a;
      const float v = s.logit[r][7];
      const float B = (float)a.batch;
      // policy term
      const float ratio = expf(logp - a.old_logp[gi]);
      const float adv = a.adv[gi];
      const float cr = fminf(fmaxf(ratio, a.ratio_lo), a.ratio_hi);
      const float s1 = ratio * adv, s2 = cr * adv;
      const float w1 = s1 < s2 ? 1.0f : s1 == s2 ? 0.5f : 0.0f;
      const float w2 = 1.0f - w1;
      const float pass = (ratio >= a.ratio_lo && ratio <= a.ratio_hi) ? 1.0f : 0.0f;
      const float gmin = -1.0f / B;                           // d loss / d min_i
      const float glogp = gmin * (w1 * adv + w2 * adv * pass) * ratio;
      // value term
      const float ov = a.old_val[gi], ret = a.ret[gi];
      const float dvc = v - ov;
      const float vc = ov + fminf(fmaxf(dvc, -a.clip_eps), a.clip_eps);
      const float e1 = (v - ret) * (v - ret), e2 = (vc - ret) * (vc - ret);
      const float u1 = e1 > e2 ? 1.0f : e1 == e2 ? 0.5f : 0.0f;
      const float u2 = 1.0f - u1;
      const float vpass = (dvc >= -a.clip_eps && dvc <= a.clip_eps) ? 1.0f : 0.0f;
      const float gmax = a.value_coef * 0.5f / B;             // d loss / d max_i
      dl[7] = gmax * (u1 * 2.0f * (v - ret) + u2 * 2.0f * (vc - ret) * vpass);
      // entropy term
      const float gh = -a.entropy_coef / B;
#pragma unroll
      for (int k = 0; k < 5; ++k)
        if (mm[k]) dl[k] = glogp * ((k == am ? 1.0f : 0.0f) - pm[k]) - gh * pm[k] * (lpm[k] + hm);
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (bm[k]) dl[5 + k] = glogp * ((k == ab ? 1.0f : 0.0f) - pb[k]) - gh * pb[k] * (lpb[k] + hb);
      st[0] = -fminf(s1, s2);
      st[1] = 0.5f * fmaxf(e1, e2);
      st[2] = hm + hb;
      st[3] = a.old_logp[gi] - logp;
      st[4] = fabsf(ratio - 1.0f) > a.clip_eps ? 1.0f : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) a.dl[out_at(g, k, 8, a.t_chunk)] = dl[k];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) s.dl[r][k] = dl[k];
#pragma unroll
    for (int k = 0; k < 5; ++k) s.stat[r][k] = st[k];
  }
  __syncthreads();
  if (t < 5) {
    float sum = 0.0f;
    for (int r = 0; r < R; ++r) sum += s.stat[r][t];
    a.stats_part[(size_t)blockIdx.x * 5 + t] = sum;
  }

  // ---- backward: output layer -> heads' hidden (ReLU); hy goes out first
  for (int i = t; i < R * HY; i += T) {
    const int r = i / HY, c = i % HY;
    const float hyv = s.y[r][c];
    if (r < nrows) a.hy[(size_t)(row0 + r) * HY + c] = hyv;
    const int head = c >> 6, k = c & 63;
    float d = 0.0f;
    if (head == 0) {
#pragma unroll
      for (int j = 0; j < 5; ++j) d += s.dl[r][j] * a.wf[j * 64 + k];
    } else if (head == 1) {
      d = s.dl[r][5] * a.wf[5 * 64 + k] + s.dl[r][6] * a.wf[6 * 64 + k];
    } else {
      d = s.dl[r][7] * a.wf[7 * 64 + k];
    }
    s.y[r][c] = hyv > 0.0f ? d : 0.0f;                       // dhy over hy
  }
  __syncthreads();
  gemm<HY, H, HYP, HP>(s.y, a.wh, nullptr, s.g);            // dh2 = dhy Wh
  __syncthreads();
  if (t < H)
    ln_param_sums(s.g, s.z2, s.mean2, s.rstd2, a.ln2_w, a.ln2_b,
                  a.ln_part + ((size_t)blockIdx.x * 4 + 2) * H,
                  a.ln_part + ((size_t)blockIdx.x * 4 + 3) * H);
  __syncthreads();
  if (t < TR) ln_backward(s.g, s.z2, s.mean2, s.rstd2, a.ln2_w, a.ln2_b);   // s.g = dz2
  __syncthreads();
  gemm<H, H, HP, HP>(s.g, a.w1, nullptr, s.z2);             // dh1 = dz2 W1 (z2 is dead)
  __syncthreads();
  if (t < H)
    ln_param_sums(s.z2, s.z1, s.mean1, s.rstd1, a.ln1_w, a.ln1_b,
                  a.ln_part + ((size_t)blockIdx.x * 4 + 0) * H,
                  a.ln_part + ((size_t)blockIdx.x * 4 + 1) * H);
  __syncthreads();
  if (t < TR) ln_backward(s.z2, s.z1, s.mean1, s.rstd1, a.ln1_w, a.ln1_b);   // s.z2 = dz1
  __syncthreads();

  // ---- row outputs
  for (int i = t; i < R * H; i += T) {
    const int r = i / H, c = i % H;
    if (r < nrows) {
      const size_t o = (size_t)(row0 + r) * H + c;
      a.dz1[o] = s.z2[r][c];
      a.h2[o] = s.hb[r][c];
    }
  }
  // dz2 and dhy in the caller's layout (rows fastest, so chunk-transposed
  // stores are 16 consecutive floats)
  for (int i = t; i < R * H; i += T) {
    const int r = i % R, c = i / R;
    if (r < nrows) a.dz2[out_at(row0 + r, c, H, a.t_chunk)] = s.g[r][c];
  }
  for (int i = t; i < R * HY; i += T) {
    const int r = i % R, c = i / R;
    if (r < nrows) a.dhy[out_at(row0 + r, c, HY, a.t_chunk)] = s.y[r][c];
  }
  // ---- this block's column sums of dz1, dz2, dhy, dl (the bias gradients'
  // partials) and max |dz1| per column (the weight-gradient kernel's scale)
  constexpr int NB = 2 * H + HY + 8;
  if (a.bias_part) {
    for (int c = t; c < NB; c += T) {
      float sum = 0.0f;
      for (int r = 0; r < nrows; ++r)
        sum += c < H ? s.z2[r][c]
                     : c < 2 * H ? s.g[r][c - H] : c < 2 * H + HY ? s.y[r][c - 2 * H]
                                                                : s.dl[r][c - 2 * H - HY];
      a.bias_part[(size_t)blockIdx.x * NB + c] = sum;
    }
  }
  if (a.dz1_absmax_part && t < H) {
    float m = 0.0f;
    for (int r = 0; r < nrows; ++r) m = fmaxf(m, fabsf(s.z2[r][t]));
    a.dz1_absmax_part[(size_t)blockIdx.x * H + t] = m;
  }
}

// One wavefront per destination row: all of the row's loads are issued
// before its stores, 4-byte words coalesced across the lanes.
__global__ __launch_bounds__(256) void gather_rows_kernel(const qqt_gather_args a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.n) return;
  const int64_t src = a.index[row];
  if (src < 0 || src >= a.src_rows) return;
  const uint32_t* s = a.src + src * a.src_stride;
  uint32_t* d = a.dst + (int64_t)row * a.dst_stride;
  constexpr int U = 8;
  for (int w0 = 0; w0 < a.row_words; w0 += 64 * U) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + 64 * u + lane;
      v[u] = w < a.row_words ? s[w] : 0u;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + 64 * u + lane;
      if (w < a.row_words) d[w] = v[u];
    }
  }
}

}  // namespace ppo
}  // namespace qqt

extern "C" {

int qqt_ppo_grad(const qqt_ppo_args* a, void* stream) {
  using namespace qqt;
  using namespace qqt::ppo;
  g_err[0] = 0;
  if (!a || !a->z1 || !a->ln1_w || !a->ln1_b || !a->w1 || !a->w1t || !a->b1 || !a->ln2_w ||
      !a->ln2_b || !a->wh || !a->wht || !a->bh || !a->wf || !a->bf || !a->actions ||
      !a->move_mask || !a->bomb_mask || !a->old_logp || !a->adv || !a->ret || !a->old_val ||
      !a->dz1 || !a->h1 || !a->dz2 || !a->h2 || !a->hy || !a->dhy || !a->dl || !a->ln_part ||
      !a->stats_part) {
    snprintf(g_err, sizeof(g_err), "qqt_ppo_grad: null argument");
    return QQT_E_ARG;
  }
  const uintptr_t al = (uintptr_t)a->z1 | (uintptr_t)a->w1 | (uintptr_t)a->w1t | (uintptr_t)a->b1 |
                       (uintptr_t)a->wh | (uintptr_t)a->wht | (uintptr_t)a->bh;
  if (a->batch <= 0 || (al & 15) || !(a->clip_eps >= 0.0f) || a->t_chunk < 0 ||
      a->t_chunk % R) {
    snprintf(g_err, sizeof(g_err), "qqt_ppo_grad: bad batch, clip or 16-byte alignment");
    return QQT_E_ARG;
  }
  if (a->row_index && (a->src_rows <= 0 || (((uintptr_t)a->row_index) & 7))) {
    snprintf(g_err, sizeof(g_err), "qqt_ppo_grad: row_index needs src_rows > 0 and 8-byte alignment");
    return QQT_E_ARG;
  }
  const int blocks = (a->batch + R - 1) / R;
  QQT_LAUNCH(QQT_KERNEL_PPO, ppo_grad_kernel, dim3(blocks), dim3(T), (hipStream_t)stream, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "ppo grad launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

int qqt_gather_rows(const qqt_gather_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!a || !a->src || !a->dst || !a->index) {
    snprintf(g_err, sizeof(g_err), "qqt_gather_rows: null pointer argument");
    return QQT_E_ARG;
  }
  if (a->n < 0 || a->row_words <= 0 || a->src_rows < 0 || a->src_stride < a->row_words ||
      a->dst_stride < a->row_words) {
    snprintf(g_err, sizeof(g_err), "qqt_gather_rows: bad sizes or strides");
    return QQT_E_ARG;
  }
  if (a->n == 0) return QQT_OK;
  hipLaunchKernelGGL(ppo::gather_rows_kernel, dim3((a->n + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "gather launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
