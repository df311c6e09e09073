// MLP actor/critic forward + masked factored sampling for gfx950 (MFMA).
//
// Network (train/model.py:121-196, arch "mlp"): obs (B, C*H*W) float16 ->
// Linear(2366,128) -> LayerNorm -> ReLU -> Linear(128,128) -> LayerNorm ->
// ReLU -> three heads Linear(128,64) -> ReLU -> Linear(64, 5 | 2 | 1).
// A player's view permutation is folded into the first-layer weights, so a
// player is just a column block of one shared weight buffer.
//
// Workgroup = 8 wavefronts (2 per SIMD) = one 64-row block of one player.
// Both players' workgroups of a row block are dispatched back to back on the
// same XCD (workgroups are dealt to the 8 XCDs round robin), so the second
// read of the observation tile hits that XCD's L2.
//
// Layer 1 (K = 2366) is split over two groups of four wavefronts: group g
// takes K blocks g, g+2, g+4, ...  Each group streams its 64 x 64 observation
// tiles through its own double-buffered, XOR-swizzled LDS tile (loaded PD
// steps ahead into registers); the weight fragments go straight from L2 into
// registers, PD steps ahead.  Wavefront (g, c) owns output columns
// 32c..32c+31.  The two groups' partial sums meet in an fp32 LDS tile, where
// LayerNorm runs row-wise (8 lanes per row, 16 contiguous columns per lane).
// The small layers split rows and columns over all eight wavefronts.
//
// Every product runs on v_mfma_f32_16x16x32_f16 with float32 accumulation.
// The observation is exact in float16 and the first layer's weights are
// rounded to float16 once; every later layer carries both its activations
// and its weights as float16 hi/lo pairs (x = hi + lo) and sums the three
// products hi*hi + hi*lo + lo*hi, which keeps logits within ~5e-4 of a
// float32 forward even for large (orthogonal, gain sqrt 2) weights.  B
// operands are pre-arranged on the host (qqtsim/policy.py) so each lane reads
// 32 contiguous bytes per 64-deep K block:
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
constexpr int ROWS = 64;           // rows per block (a workgroup takes one or two)
constexpr int MLP_TWO_BLOCK_ROWS = 1 << 16;   // forward batches from here use two blocks
constexpr int NTHR = 512;          // 8 wavefronts
constexpr int FST = HID + 4;       // fp32 row stride of the LayerNorm tile (bank spread)
#ifndef QQT_MLP_PD
#define QQT_MLP_PD 2
#endif
constexpr int PD = QQT_MLP_PD;     // K blocks of layer 1 in flight per group (even)
static_assert(PD >= 2 && PD % 2 == 0, "the x tile ring pairs with an LDS double buffer");

// parameter vectors staged in LDS (floats)
constexpr int V_B0 = 0, V_G1 = 128, V_BE1 = 256, V_B1 = 384, V_G2 = 512, V_BE2 = 640;
constexpr int V_BH = 768, V_BF = 960, V_N = 968;

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

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LDS tiles store rows of float16 in 16-byte chunks; chunk c of row r sits at
// chunk position c ^ (r & 7), so the 16 rows of an A fragment read land on
// distinct banks.
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ (row & 7); }

constexpr int XT_HALVES = ROWS * 64;            // one 64 x 64 observation tile (8 KB)
constexpr int H_HALVES = 2 * ROWS * HID;        // hi + lo planes of h1 or h2 (32 KB)
constexpr int HY_HALVES = 2 * ROWS * 3 * HEAD;  // hi + lo planes of the head layer (48 KB)
static_assert(HY_HALVES <= 4 * XT_HALVES + H_HALVES, "head layer reuses the x tiles and h1");
static_assert(HY_HALVES <= 8 * XT_HALVES, "two-block head layer fits in the x tiles alone");
static_assert(ROWS * HID * 2 <= 4 * XT_HALVES, "the second partial tile fits in the x tiles");

constexpr int WF_HALVES = 3 * 64 * 16;          // output layer: 1 column tile x 3 K blocks
constexpr int WF_CHUNKS = 2 * WF_HALVES / 8;    // 16-byte chunks of both planes

// LDS of a workgroup of RB 64-row blocks.  xs_h1 holds the layer-1 x tiles
// (RB x 32 KB), then h1; the tail reuses the x tiles for the second partial
// tile and the head layer.  With RB = 1 the head layer spills over into the
// dead h1 and h2 has its own region; with RB = 2 the x tiles alone hold the
// head layer and h2 reuses h1 (dead once layer 2 has read it).
template <int RB>
struct __align__(16) MlpLds {
  uint16_t xs_h1[RB * 4 * XT_HALVES + H_HALVES];   // x tiles [group][buffer] | h1
  uint16_t h2[RB == 1 ? H_HALVES : 8];
  float f[ROWS][FST];                         // fp32 pre-LayerNorm tile
  float vec[V_N];                             // biases and LayerNorm affine parameters
  float logit[ROWS][NOUT];
  uint16_t wf[2][WF_HALVES];                  // output-layer B fragments, hi and lo planes
};

__device__ __forceinline__ uint16_t* h_at(uint16_t* base, int width, int plane, int row, int col) {
  return base + (plane * ROWS + row) * width + (swz(row, col >> 3) << 3) + (col & 7);
}
__device__ __forceinline__ void split_store(uint16_t* hi, uint16_t* lo, float y) {
  const __half h = __float2half_rn(y);
  *hi = __half_as_ushort(h);
  *lo = __half_as_ushort(__float2half_rn(y - __half2float(h)));
}
// A fragment (16 halves) of row `row`, K block kb, from a swizzled tile.
__device__ __forceinline__ Frag16 read_a(const uint16_t* plane, int width, int row, int kb, int q) {
  const uint16_t* r = plane + row * width;
  const int c = 8 * kb + 2 * q;
  Frag16 f;
  f.lo = as_h8(*reinterpret_cast<const uint4*>(r + (swz(row, c) << 3)));
  f.hi = as_h8(*reinterpret_cast<const uint4*>(r + (swz(row, c + 1) << 3)));
  return f;
}

// Sum over the 8 consecutive lanes that hold one row in the LayerNorm phase.
__device__ __forceinline__ float sum8(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  return v;
}

// fp32 partial-sum tile of layer 1's second K group, kept in the (dead) x
// tiles: 64 rows x 128 floats, float4 j of row r stored at j ^ (r & 31).
__device__ __forceinline__ float* f1_at(uint16_t* xs, int row, int col) {
  float* base = reinterpret_cast<float*>(xs);
  return base + row * HID + ((((col >> 2) ^ (row & 31))) << 2) + (col & 3);
}

// Row-wise bias + LayerNorm(128) + ReLU from the fp32 tile (plus the second
// partial tile f1 when given): thread t owns row t/8; lane j = t%8 of a row
// owns columns 32i + 4j .. +3 (i = 0..3), so for each i the row's 8 lanes
// read 128 contiguous bytes (no bank conflicts); writes float16 hi/lo planes
// of dst as 8-byte stores.
template <class L>
__device__ __forceinline__ void layernorm_rows(L& s, const uint16_t* f1, int vb, int vg,
                                               int vbe, uint16_t* dst) {
  const int t = threadIdx.x, row = t >> 3, j = t & 7;
  float v[16], ga[16], be[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 32 * i + 4 * j;
    const float4 x = *reinterpret_cast<const float4*>(&s.f[row][c]);
    const float4 b = *reinterpret_cast<const float4*>(&s.vec[vb + c]);
    const float4 g = *reinterpret_cast<const float4*>(&s.vec[vg + c]);
    const float4 e = *reinterpret_cast<const float4*>(&s.vec[vbe + c]);
    float4 y = x;
    if (f1) {
      const float4 z = *reinterpret_cast<const float4*>(
          f1_at(const_cast<uint16_t*>(f1), row, c));
      y = make_float4(z.x + x.x, z.y + x.y, z.z + x.z, z.w + x.w);
    }
    v[4 * i + 0] = y.x + b.x;
    v[4 * i + 1] = y.y + b.y;
    v[4 * i + 2] = y.z + b.z;
    v[4 * i + 3] = y.w + b.w;
    ga[4 * i + 0] = g.x; ga[4 * i + 1] = g.y; ga[4 * i + 2] = g.z; ga[4 * i + 3] = g.w;
    be[4 * i + 0] = e.x; be[4 * i + 1] = e.y; be[4 * i + 2] = e.z; be[4 * i + 3] = e.w;
  }
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) p += v[i];
  const float mean = sum8(p) * (1.0f / HID);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(sum8(q) * (1.0f / HID) + 1e-5f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t hi[2], lo[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const int k = 4 * i + e;
      const float y0 = fmaxf((v[k] - mean) * rstd * ga[k] + be[k], 0.0f);
      const float y1 = fmaxf((v[k + 1] - mean) * rstd * ga[k + 1] + be[k + 1], 0.0f);
      const __half h0 = __float2half_rn(y0), h1 = __float2half_rn(y1);
      const __half l0 = __float2half_rn(y0 - __half2float(h0));
      const __half l1 = __float2half_rn(y1 - __half2float(h1));
      hi[e / 2] = (uint32_t)__half_as_ushort(h0) | ((uint32_t)__half_as_ushort(h1) << 16);
      lo[e / 2] = (uint32_t)__half_as_ushort(l0) | ((uint32_t)__half_as_ushort(l1) << 16);
    }
    const int c = 32 * i + 4 * j;                 // 4 halves = half of chunk c/8
    const int off = (swz(row, c >> 3) << 3) + (c & 7);
    *reinterpret_cast<uint2*>(dst + (0 * ROWS + row) * HID + off) = make_uint2(hi[0], hi[1]);
    *reinterpret_cast<uint2*>(dst + (1 * ROWS + row) * HID + off) = make_uint2(lo[0], lo[1]);
  }
}

// hi and lo B fragments of CT column tiles x KB K blocks (tiles tile0..).
template <int CT, int KB>
struct SplitB { Frag16 hi[KB][CT], lo[KB][CT]; };
template <int CT, int KB>
__device__ __forceinline__ void load_split_b(SplitB<CT, KB>& b, const uint16_t* b_hi,
                                             const uint16_t* b_lo, int tile0, int lane) {
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const size_t off = ((size_t)((tile0 + ct) * KB + kb) * 64 + lane) * 16;
      b.hi[kb][ct] = load_b(b_hi + off);
      b.lo[kb][ct] = load_b(b_lo + off);
    }
}

// RT row tiles (rows 16*(rt0+i) + lane%16) x CT column tiles of a hi/lo layer:
// acc += A(hi,lo) * B(hi,lo) over KB K blocks.
template <int RT, int CT, int KB>
__device__ __forceinline__ void split_gemm(floatx4 (&acc)[RT][CT], const uint16_t* a_hi,
                                           const uint16_t* a_lo, int width, int rt0,
                                           const SplitB<CT, KB>& b, int lane) {
  const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    Frag16 ah[RT], al[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      ah[i] = read_a(a_hi, width, 16 * (rt0 + i) + r16, kb, q);
      al[i] = read_a(a_lo, width, 16 * (rt0 + i) + r16, kb, q);
    }
    // the six products of each (row tile, column tile) pair in turn over all
    // pairs: consecutive MFMAs never wait for each other's accumulator
#pragma unroll
    for (int p = 0; p < 6; ++p)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const Frag16& bv = (p == 2 || p == 3) ? b.lo[kb][ct] : b.hi[kb][ct];
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const Frag16& av = p < 4 ? ah[i] : al[i];
          acc[i][ct] = (p & 1) ? mfma(av.hi, bv.hi, acc[i][ct]) : mfma(av.lo, bv.lo, acc[i][ct]);
        }
      }
  }
}

// Sampling inputs of one row (threads < 64 of a row block): masks and the
// two uniforms (move, bomb).
struct RowSampler {
  bool on;
  uint8_t mm[5], bm[2];
  float um, ub;
};

// Masks and uniforms of output row `row` for player pid (Philox when the
// caller passes no uniforms).
__device__ __forceinline__ RowSampler load_sampler(const qqt_mlp_args& a, bool on, int row, int pid,
                                                   int oslots, int oslot) {
  RowSampler r;
  r.on = on;
#pragma unroll
  for (int k = 0; k < 5; ++k) r.mm[k] = 0;
  r.bm[0] = r.bm[1] = 0;
  r.um = r.ub = 0.0f;
  if (on) {
#pragma unroll
    for (int k = 0; k < 5; ++k)
      r.mm[k] = a.move_mask[(size_t)row * a.mm_row_stride + (size_t)pid * a.mm_pid_stride + k];
#pragma unroll
    for (int k = 0; k < 2; ++k)
      r.bm[k] = a.bomb_mask[(size_t)row * a.bm_row_stride + (size_t)pid * a.bm_pid_stride + k];
    const size_t o = (size_t)row * oslots + oslot;
    if (a.uniforms) {
      r.um = a.uniforms[o * 2 + 0];
      r.ub = a.uniforms[o * 2 + 1];
    } else {
      float u4[4];
      philox_block(a.seed, (uint32_t)row, a.tick, STREAM_POLICY, (uint32_t)((2 * pid) >> 2), u4);
      r.um = u4[(2 * pid) & 3];
      r.ub = u4[(2 * pid + 1) & 3];
    }
  }
  return r;
}

// Everything after the first layer for one 64-row block (512 threads):
// bias + LayerNorm 1 (s.f plus the second partial tile f1 when given) +
// ReLU, Linear(128,128), LayerNorm 2 + ReLU, the heads' hidden and output
// layers, then the outputs and the masked sampling, one thread per row.
// w1b holds the layer-2 B fragments, already in flight.  H1, H2 and HY are
// LDS planes; HY may overlay f1 and H1 (both dead by then).
template <class L>
__device__ __forceinline__ void mlp_tail(L& s, const qqt_mlp_args& a, const uint16_t* f1,
                                         uint16_t* H1, uint16_t* H2, uint16_t* HY, int brow0,
                                         int oslots, int oslot, const RowSampler& rs,
                                         const SplitB<2, 2>& w1b) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int cg = w & 3, rh = w >> 2;      // column group, row half of the small layers
  layernorm_rows(s, f1, V_B0, V_G1, V_BE1, H1);
  __syncthreads();

  // ---------------- layer 2: 128 -> 128; wavefront w: rows 32rh.., columns 32cg..
  floatx4 acc2[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc2[i][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  split_gemm<2, 2, 2>(acc2, H1, H1 + ROWS * HID, HID, 2 * rh, w1b, lane);
  SplitB<3, 2> whb;                 // head weights: in flight during LayerNorm 2
  load_split_b(whb, a.wh, a.wh_lo, 3 * cg, lane);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s.f[32 * rh + 16 * i + 4 * q + j][32 * cg + 16 * ct + r16] = acc2[i][ct][j];
  __syncthreads();
  layernorm_rows(s, nullptr, V_B1, V_G2, V_BE2, H2);
  __syncthreads();

  // ---------------- heads, first layer: 128 -> 192; rows 32rh.., columns 48cg..
  {
    floatx4 hac[2][3];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int ct = 0; ct < 3; ++ct) hac[i][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    split_gemm<2, 3, 2>(hac, H2, H2 + ROWS * HID, HID, 2 * rh, whb, lane);
#pragma unroll
    for (int ct = 0; ct < 3; ++ct) {
      const int col = 48 * cg + 16 * ct + r16;
      const float b = s.vec[V_BH + col];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 32 * rh + 16 * i + 4 * q + j;
          split_store(h_at(HY, 3 * HEAD, 0, row, col), h_at(HY, 3 * HEAD, 1, row, col),
                      fmaxf(hac[i][ct][j] + b, 0.0f));
        }
    }
  }
  __syncthreads();

  // ---------------- heads, output layer: 192 -> 8 (block diagonal); wavefronts 0-3: rows 16w..
  if (w < 4) {
    floatx4 oac = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 3; ++kb) {
      const Frag16 bh = load_b(&s.wf[0][(kb * 64 + lane) * 16]);
      const Frag16 bl = load_b(&s.wf[1][(kb * 64 + lane) * 16]);
      const int row = 16 * w + r16;
      const Frag16 ah = read_a(HY, 3 * HEAD, row, kb, q);
      const Frag16 al = read_a(HY + ROWS * 3 * HEAD, 3 * HEAD, row, kb, q);
      oac = mfma(ah.lo, bh.lo, oac);
      oac = mfma(ah.hi, bh.hi, oac);
      oac = mfma(ah.lo, bl.lo, oac);
      oac = mfma(ah.hi, bl.hi, oac);
      oac = mfma(al.lo, bh.lo, oac);
      oac = mfma(al.hi, bh.hi, oac);
    }
    if (r16 < NOUT) {
      const float b = s.vec[V_BF + r16];
#pragma unroll
      for (int j = 0; j < 4; ++j) s.logit[16 * w + 4 * q + j][r16] = oac[j] + b;
    }
  }
  __syncthreads();

  // ---------------- outputs and sampling: one thread per row
  const int orow = brow0 + (int)threadIdx.x;
  if (threadIdx.x < ROWS && orow < a.batch) {
    const float* lg = s.logit[threadIdx.x];
    const size_t o = (size_t)orow * oslots + oslot;
    if (a.logits_out) {
#pragma unroll
      for (int k = 0; k < NOUT; ++k) a.logits_out[o * NOUT + k] = lg[k];
    }
    if (a.value_out) a.value_out[o] = lg[7];
    if (rs.on) {
      float lpm, lpb;
      const int am = sample_masked<5>(lg, rs.mm, rs.um, &lpm);
      const int ab = sample_masked<2>(lg + 5, rs.bm, rs.ub, &lpb);
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

// RB row blocks of 64 per workgroup: RB = 2 halves the W0 bytes each row
// costs (large forward batches, no sampling); the tail runs once per block.
// Z1: the first-layer-only instantiation of the training forward (z1_out).
template <int RB, bool Z1>
__global__ __launch_bounds__(NTHR) void mlp_act_kernel(const qqt_mlp_args a) {
  static_assert(RB == 1 || RB == 2, "one or two row blocks per workgroup");
  constexpr int RT = 4 * RB;               // layer-1 row tiles per wavefront
  constexpr int NX = 8 * RB;               // x load instructions per wavefront and K block
  constexpr int XT = RB * XT_HALVES;       // one x tile of the workgroup
  __shared__ MlpLds<RB> s;
  const int nrb = (a.batch + RB * ROWS - 1) / (RB * ROWS);
  const int xcd = blockIdx.x & 7, seq = blockIdx.x >> 3;
  const int slot = seq % a.npid;
  const int rb = (seq / a.npid) * 8 + xcd;
  if (rb >= nrb) return;                   // padding workgroup (uniform, before any barrier)
  const int pid = a.npid == 2 ? slot : a.pid0;
  const int row0 = rb * RB * ROWS;
  // wavefront index as a scalar: branches and addresses on it stay uniform
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r16 = lane & 15, q = lane >> 4;
  const int kg = w >> 2, cg = w & 3;       // layer-1 K group, column group
  const int oslots = a.out_slots > 0 ? a.out_slots : a.npid;   // output row width (slots)
  const int oslot = a.npid == 2 ? slot : a.out_slot;

  // Parameter vectors: two floats per thread, loaded before the first tiles
  // (vmcnt retires in order) and written to LDS after they are issued.
  auto vec_src = [&](int i) -> const float* {
    return i < V_G1 ? a.b0 + (i - V_B0) : i < V_BE1 ? a.ln1_w + (i - V_G1)
         : i < V_B1 ? a.ln1_b + (i - V_BE1) : i < V_G2 ? a.b1 + (i - V_B1)
         : i < V_BE2 ? a.ln2_w + (i - V_G2) : i < V_BH ? a.ln2_b + (i - V_BE2)
         : i < V_BF ? a.bh + (i - V_BH) : a.bf + (i - V_BF);
  };
  const int vi0 = threadIdx.x, vi1 = threadIdx.x + NTHR;   // vi1 < V_N for the first 456
  const float vv0 = *vec_src(vi0);
  const float vv1 = vi1 < V_N ? *vec_src(vi1) : 0.0f;
  // output-layer weights (both planes, 16-byte chunks t and t + NTHR)
  static_assert(WF_CHUNKS <= 2 * NTHR && WF_CHUNKS > NTHR, "two chunks per thread");
  auto wf_src = [&](int c) {
    const int plane = c / (WF_HALVES / 8), i = c % (WF_HALVES / 8);
    return reinterpret_cast<const uint4*>(plane ? a.wf_lo : a.wf) + i;
  };
  const int wc1 = threadIdx.x + NTHR;
  const uint4 wfv0 = *wf_src(threadIdx.x);
  const uint4 wfv1 = wc1 < WF_CHUNKS ? *wf_src(wc1) : make_uint4(0u, 0u, 0u, 0u);

  // ---------------- layer 1: group kg, K blocks kg, kg+2, ...; columns 32cg..32cg+31
  floatx4 acc[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // x loads: instruction i of wavefront (kg, cg) covers tile rows
  // 16RBcg+2i, 16RBcg+2i+1; lane l reads dword l&31 (two halves) of row
  // 16RBcg+2i+(l>>5).
  const int nkb = a.kblocks0;
  const int dw = lane & 31;
  // row addresses are formed at each load from one base row (clamped to
  // the batch for a ragged last block), not held as NX pointers
  const int xrow0 = row0 + 16 * RB * cg + (lane >> 5);
  const uint32_t* const xbase = reinterpret_cast<const uint32_t*>(a.obs);
  const size_t xstride = (size_t)a.obs_stride / 2;    // dwords per row
  const uint16_t* wb = a.w0 + (size_t)((pid * 8 + 2 * cg) * nkb) * 64 * 16 + lane * 16;
  const size_t wtile = (size_t)nkb * 64 * 16;   // halves between B tiles
  uint16_t* const xt = s.xs_h1 + kg * 2 * XT;   // this group's two x tiles

  // Loads run PD group steps ahead; the tail mask (elements >= k0) is applied
  // when the registers are written to LDS, so no load is waited on early.
  // Lanes past k0 read dword 0 of their row (in bounds).
  auto load_x = [&](int kb, uint32_t (&xr)[NX]) {
    const int k = 64 * kb + 2 * dw;              // first half of this lane's pair
    const int off = k < a.k0 ? (k >> 1) : 0;     // k0 is even: pairs never straddle
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int r = min(xrow0 + 2 * i, a.batch - 1);
      xr[i] = xbase[(size_t)r * xstride + off];   // cached: two workgroups read each row
    }
  };
  auto load_w = [&](int kb, Frag16 (&br)[2]) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) br[ct] = load_b(wb + ct * wtile + (size_t)kb * 64 * 16);
  };
  auto store_x = [&](const uint32_t (&xr)[NX], int buf, int kb) {
    const bool ok = 64 * kb + 2 * dw < a.k0;
    uint32_t* t = reinterpret_cast<uint32_t*>(xt + buf * XT);
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int r = 16 * RB * cg + 2 * i + (lane >> 5);
      t[r * 32 + (swz(r, dw >> 2) << 2) + (dw & 3)] = ok ? xr[i] : 0u;
    }
  };
  auto compute = [&](int buf, const Frag16 (&br)[2]) {
    const uint16_t* t = xt + buf * XT;
    Frag16 af[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) af[rt] = read_a(t, 64, 16 * rt + r16, 0, q);
    // low K halves over every tile pair, then the high halves
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
          acc[rt][ct] = h ? mfma(af[rt].hi, br[ct].hi, acc[rt][ct])
                          : mfma(af[rt].lo, br[ct].lo, acc[rt][ct]);
  };

  // Group step i handles K block 2i + kg.  Register ring of PD steps in
  // flight, LDS double buffer per group, one barrier per step, no branches:
  // prefetch indices are clamped to the last block, and the step count is
  // padded to a multiple of PD with all-zero x tiles (store_x masks every
  // element >= k0), which add exactly zero.
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

  const int srow = row0 + (int)threadIdx.x;          // sampling row of threads < 64
  const RowSampler rs = load_sampler(a, RB == 1 && threadIdx.x < ROWS && srow < a.batch && a.sample,
                                     srow, pid, oslots, oslot);

  s.vec[vi0] = vv0;
  if (vi1 < V_N) s.vec[vi1] = vv1;
  reinterpret_cast<uint4*>(&s.wf[0][0])[threadIdx.x] = wfv0;
  if (wc1 < WF_CHUNKS) reinterpret_cast<uint4*>(&s.wf[0][0])[wc1] = wfv1;
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
    compute(j & 1, br[j]);
    if (j + 1 < PD) store_x(xr[(j + 1) % PD], (j + 1) & 1, kblk(nsteps - PD + j + 1));
    __syncthreads();
  }

  // Combine the two groups' partial sums in the fp32 tile.
  uint16_t* const H1 = s.xs_h1 + RB * 4 * XT_HALVES;
  uint16_t* const H2 = RB == 1 ? s.h2 : H1;
  const int rh = w >> 2;            // row half of the small layers
#pragma unroll
  for (int hb = 0; hb < RB; ++hb) {   // one 64-row block at a time
  const int brow0 = row0 + ROWS * hb;
  SplitB<2, 2> w1b;                 // layer-2 weights: in flight during LayerNorm 1
  load_split_b(w1b, a.w1, a.w1_lo, 2 * cg, lane);
  // The last loop step ended with a barrier, so the x tiles are free.
  // (kg is uniform: one branch around both store loops)
  if (kg == 0) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s.f[16 * rt + 4 * q + j][32 * cg + 16 * ct + r16] = acc[4 * hb + rt][ct][j];
  } else {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *f1_at(s.xs_h1, 16 * rt + 4 * q + j, 32 * cg + 16 * ct + r16) = acc[4 * hb + rt][ct][j];
  }
  __syncthreads();
  if constexpr (Z1) {   // first layer only (the training forward): z1 = (f1 + f) + b0
    const int t = threadIdx.x, row = t >> 3, j = t & 7, orow = brow0 + row;
    if (orow < a.batch) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 32 * i + 4 * j;
        const float4 x = *reinterpret_cast<const float4*>(&s.f[row][c]);
        const float4 z = *reinterpret_cast<const float4*>(f1_at(s.xs_h1, row, c));
        const float4 b = *reinterpret_cast<const float4*>(&s.vec[V_B0 + c]);
        *reinterpret_cast<float4*>(a.z1_out + (size_t)orow * HID + c) =
            make_float4((z.x + x.x) + b.x, (z.y + x.y) + b.y, (z.z + x.z) + b.z,
                        (z.w + x.w) + b.w);
      }
    }
    if (hb + 1 < RB) __syncthreads();   // the next block rewrites both tiles
    continue;
  }
  mlp_tail(s, a, s.xs_h1, H1, H2, s.xs_h1, brow0, oslots, oslot, rs, w1b);
  if (hb + 1 < RB) __syncthreads();   // the next block reuses every tail buffer
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
  if (a->z1_out && (a->npid != 1 || a->sample || (((uintptr_t)a->z1_out) & 15))) {
    snprintf(g_err, sizeof(g_err), "qqt_mlp_act: z1_out needs npid 1, no sampling, 16-byte alignment");
    return QQT_E_ARG;
  }
  // one workgroup per (row block, player); row blocks are dealt to the 8
  // XCDs round robin with both players' workgroups adjacent on one XCD.
  // Large forward batches take two 64-row blocks per workgroup (half the
  // W0 bytes per row); rollouts keep one, for twice the workgroups.
  const bool two = !a->sample && a->batch >= MLP_TWO_BLOCK_ROWS;
  const int rows_wg = (two ? 2 : 1) * ROWS;
  const int nrb = (a->batch + rows_wg - 1) / rows_wg;
  const int blocks = ((nrb + 7) / 8) * 8 * a->npid;
  hipStream_t st = (hipStream_t)stream;
  if (a->z1_out && two)
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<2, true>), dim3(blocks), dim3(NTHR), st, *a);
  else if (a->z1_out)
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<1, true>), dim3(blocks), dim3(NTHR), st, *a);
  else if (two)
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<2, false>), dim3(blocks), dim3(NTHR), st, *a);
  else
    QQT_LAUNCH(QQT_KERNEL_MLP, (mlp_act_kernel<1, false>), dim3(blocks), dim3(NTHR), st, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "mlp launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
