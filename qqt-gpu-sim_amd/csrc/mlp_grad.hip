// First-layer weight gradient of the mlp ActorCritic for the PPO update
// (train/ppo.py:364-437 runs loss.backward() through train/model.py:121-147):
//   dW0[h][k] = sum_b dz1[b][h] * obs[b][k]
// over a minibatch of B observation rows (float16, exact) and the float32
// gradient dz1 of the first layer's output.  This product carries nearly all
// of the backward pass's work and bytes (K = 2366 observation columns per
// row; the later layers are 128 wide).
//
// MFMA v_mfma_f32_16x16x32_f16 with the batch as the contraction index.  The
// observation is exact in float16; dz1 is scaled by a power of two (so its
// largest magnitude is 2^14) and split into float16 hi + lo, two products per
// tile, which keeps the result within ~1e-6 relative of a float32 sum.
//
// Grid: (column tile of 256 observation columns) x (chunk of the batch).  A
// workgroup (8 wavefronts) owns a 128 x 256 fp32 output tile for its chunk
// and walks the chunk 32 rows at a time: each step loads 32 x 256 float16 of
// the observation and 32 x 128 of dz1 into registers one step ahead, writes
// them transposed into LDS (the MFMA operands need the batch index
// contiguous), one barrier per step.  Partial tiles go to a workspace
// [chunk][128][tiles*256]; a second kernel sums the chunks in a fixed order
// (deterministic) and applies the inverse scale.
//
// Algorithmic bytes per row: 2 * k0 (observation) + 512 (dz1, read once per
// column tile: ceil(k0 / 256) times).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

namespace l1g {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HID = 128;          // first-layer outputs
constexpr int NCOL = 256;         // observation columns per workgroup
constexpr int KS = 32;            // batch rows per step (one MFMA K)
constexpr int XS = KS + 8;        // LDS row stride (halves) of the transposed tiles
constexpr int NT = 512;           // threads
constexpr int MAX_CHUNKS = 64;
constexpr int TARGET_WGS = 512;  // two workgroups (80 KB of LDS each) on each of the 256 CUs
constexpr int MIN_CHUNK_ROWS = 2048;

struct __align__(16) Lds {
  uint16_t xt[2][NCOL][XS];       // observation, [column][row]
  uint16_t dt[2][2][HID][XS];     // dz1 hi and lo planes, [hidden][row]
};

__device__ __forceinline__ half8 ld8(const uint16_t* p) {
  union { uint4 u; half8 h; } c;
  c.u = *reinterpret_cast<const uint4*>(p);
  return c.h;
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)__half_as_ushort(__float2half_rn(a)) |
         ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
}

__global__ __launch_bounds__(NT) void l1_grad_kernel(const qqt_l1_grad_args a, int chunk_rows,
                                                     int ws_cols) {
  __shared__ Lds s;
  const int t = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const int col0 = blockIdx.x * NCOL;
  const int r_begin = blockIdx.y * chunk_rows;
  const int r_end = min(r_begin + chunk_rows, a.batch);
  const int steps = (r_end - r_begin + KS - 1) / KS;     // >= 1 (chunks are non-empty)
  const float scale = a.dz_scale ? *a.dz_scale : 1.0f;

  // loader roles: observation dword column xd (columns 2xd, 2xd+1) of rows
  // 8xg..8xg+7; dz1 hidden pair hd (2hd, 2hd+1) of rows 4dg..4dg+3
  const int xd = t & 127, xg = w >> 1;                    // xg = t >> 7, as a scalar
  const int hd = t & 63, dg = t >> 6;
  const bool xcol_ok = col0 + 2 * xd < a.k0;              // k0 is even
  const uint32_t* const xbase = reinterpret_cast<const uint32_t*>(a.obs);
  const size_t xstride = (size_t)a.obs_stride / 2;

  uint32_t xr[8];
  float2 dr[4];
  auto load = [&](int step) {
    const int r0 = r_begin + KS * step;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + 8 * xg + i;
      xr[i] = (r < r_end && xcol_ok) ? xbase[obs_row(a, r) * xstride + (col0 >> 1) + xd] : 0u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + 4 * dg + i;
      dr[i] = r < r_end ? *reinterpret_cast<const float2*>(a.dz1 + (size_t)r * HID + 2 * hd)
                        : make_float2(0.0f, 0.0f);
    }
  };
  auto store = [&](int buf) {
    uint32_t lo4[4], hi4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo4[i] = (xr[2 * i] & 0xFFFFu) | (xr[2 * i + 1] << 16);            // column 2xd
      hi4[i] = (xr[2 * i] >> 16) | (xr[2 * i + 1] & 0xFFFF0000u);        // column 2xd+1
    }
    *reinterpret_cast<uint4*>(&s.xt[buf][2 * xd][8 * xg]) = make_uint4(lo4[0], lo4[1], lo4[2], lo4[3]);
    *reinterpret_cast<uint4*>(&s.xt[buf][2 * xd + 1][8 * xg]) =
        make_uint4(hi4[0], hi4[1], hi4[2], hi4[3]);
    float v0[4], v1[4], l0[4], l1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v0[i] = dr[i].x * scale;
      v1[i] = dr[i].y * scale;
      l0[i] = v0[i] - __half2float(__float2half_rn(v0[i]));
      l1[i] = v1[i] - __half2float(__float2half_rn(v1[i]));
    }
    *reinterpret_cast<uint2*>(&s.dt[buf][0][2 * hd][4 * dg]) =
        make_uint2(pack2(v0[0], v0[1]), pack2(v0[2], v0[3]));
    *reinterpret_cast<uint2*>(&s.dt[buf][0][2 * hd + 1][4 * dg]) =
        make_uint2(pack2(v1[0], v1[1]), pack2(v1[2], v1[3]));
    *reinterpret_cast<uint2*>(&s.dt[buf][1][2 * hd][4 * dg]) =
        make_uint2(pack2(l0[0], l0[1]), pack2(l0[2], l0[3]));
    *reinterpret_cast<uint2*>(&s.dt[buf][1][2 * hd + 1][4 * dg]) =
        make_uint2(pack2(l1[0], l1[1]), pack2(l1[2], l1[3]));
  };

  // wavefront w: hidden rows 32(w&3)..+31 (two m tiles), columns 128(w>>2)..+127
  const int mw = 32 * (w & 3), nw = 128 * (w >> 2);
  const int r16 = lane & 15, kq = 8 * (lane >> 4);
  floatx4 acc[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  load(0);
  store(0);
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    if (step + 1 < steps) load(step + 1);
    half8 ah[2], al[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ah[i] = ld8(&s.dt[buf][0][mw + 16 * i + r16][kq]);
      al[i] = ld8(&s.dt[buf][1][mw + 16 * i + r16][kq]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const half8 b = ld8(&s.xt[buf][nw + 16 * j + r16][kq]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b, acc[i][j], 0, 0, 0);
      }
    }
    if (step + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

  // partial tile -> workspace [chunk][hidden][ws_cols]; lane holds rows
  // 4(lane/16)+q of each m tile at column lane%16 of each n tile
  float* const out = a.workspace + (size_t)blockIdx.y * HID * ws_cols + col0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mw + 16 * i + 4 * (lane >> 4) + q;
        out[(size_t)m * ws_cols + nw + 16 * j + r16] = acc[i][j][q];
      }
}

// dw0[h][k] = (sum over chunks, in chunk order) / scale, k < k0.
__global__ __launch_bounds__(256) void l1_grad_reduce(const qqt_l1_grad_args a, int chunks,
                                                      int ws_cols) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= HID * a.k0) return;
  const int h = i / a.k0, k = i % a.k0;
  const float inv = a.dz_scale ? 1.0f / *a.dz_scale : 1.0f;   // power of two: exact
  float sum = 0.0f;
  for (int c = 0; c < chunks; ++c) sum += a.workspace[((size_t)c * HID + h) * ws_cols + k];
  a.dw0[i] = sum * inv;
}

// Chunks of the batch: rows per chunk a multiple of KS, at least
// MIN_CHUNK_ROWS, and chunks x column tiles at most TARGET_WGS (all
// workgroups resident at once, evenly two per CU) and MAX_CHUNKS.  (A
// 180,224-row minibatch of 2366 columns: 51 chunks x 10 tiles = 510
// workgroups, 374 us; 32 chunks = 320 workgroups left 192 CUs with one
// workgroup and took 526 us; 64 chunks need a second round, 478 us.)
__host__ inline void plan(int batch, int k0, int& chunks, int& chunk_rows) {
  const int tiles = (k0 + NCOL - 1) / NCOL;
  chunks = (batch + MIN_CHUNK_ROWS - 1) / MIN_CHUNK_ROWS;
  if (chunks > TARGET_WGS / tiles) chunks = TARGET_WGS / tiles;
  if (chunks > MAX_CHUNKS) chunks = MAX_CHUNKS;
  if (chunks < 1) chunks = 1;
  chunk_rows = (batch + chunks - 1) / chunks;
  chunk_rows = (chunk_rows + KS - 1) / KS * KS;
  chunks = (batch + chunk_rows - 1) / chunk_rows;
}

}  // namespace l1g

// Scratch of qqt_l1_grad_noalloc: the chunk partials of the largest plan
// (MAX_CHUNKS chunks of 128 x QQT_L1_GRAD_NOALLOC_MAX_K0 columns), one copy
// per GPU, held until the process ends.  Host code never passes this name
// to a kernel (on the host it is only a stand-in for the symbol): it uses
// the device address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float
    l1g_scratch[l1g::MAX_CHUNKS * l1g::HID * QQT_L1_GRAD_NOALLOC_MAX_K0];

namespace l1g {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[MAX_DEVICES] = {};

// The scratch's device address on the current device, looked up once per
// device (with that device current); nullptr with g_err set on failure.
float* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    snprintf(g_err, sizeof(g_err), "qqt_l1_grad_noalloc: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(l1g_scratch));
    if (err != hipSuccess || !p) {
      snprintf(g_err, sizeof(g_err), "qqt_l1_grad_noalloc: hipGetSymbolAddress failed: %s",
               hipGetErrorString(err));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}

}  // namespace l1g
}  // namespace qqt

extern "C" {

int64_t qqt_l1_grad_workspace_floats(int32_t batch, int32_t k0) {
  using namespace qqt::l1g;
  if (batch <= 0 || k0 <= 0) return -1;
  int chunks, rows;
  plan(batch, k0, chunks, rows);
  const int tiles = (k0 + NCOL - 1) / NCOL;
  return (int64_t)chunks * HID * tiles * NCOL;
}

namespace {

// Shape checks shared by both entry points (the workspace is checked by the
// caller of each).
int l1_grad_check(const qqt_l1_grad_args* a, const char* who) {
  using namespace qqt;
  if (!a || !a->obs || !a->dz1 || !a->dw0) {
    snprintf(g_err, sizeof(g_err), "%s: null argument", who);
    return QQT_E_ARG;
  }
  if (a->batch <= 0 || a->k0 <= 0 || (a->k0 & 1) || a->obs_stride < a->k0 ||
      (a->obs_stride & 1) || (((uintptr_t)a->obs) & 3) || (((uintptr_t)a->dz1) & 7)) {
    snprintf(g_err, sizeof(g_err), "%s: bad shape/stride/alignment", who);
    return QQT_E_ARG;
  }
  if (a->row_index && (a->obs_rows <= 0 || (((uintptr_t)a->row_index) & 7))) {
    snprintf(g_err, sizeof(g_err), "%s: row_index needs obs_rows > 0 and 8-byte alignment", who);
    return QQT_E_ARG;
  }
  return QQT_OK;
}

// Both launches over a checked argument block whose workspace holds the
// plan's partials.
int l1_grad_launch(const qqt_l1_grad_args& a, hipStream_t st) {
  using namespace qqt;
  using namespace qqt::l1g;
  int chunks, rows;
  plan(a.batch, a.k0, chunks, rows);
  const int tiles = (a.k0 + NCOL - 1) / NCOL;
  const int ws_cols = tiles * NCOL;
  QQT_LAUNCH(QQT_KERNEL_L1GRAD, l1_grad_kernel, dim3(tiles, chunks), dim3(NT), st, a, rows,
             ws_cols);
  hipError_t err = hipGetLastError();
  if (err == hipSuccess) {
    const int n = HID * a.k0;
    QQT_LAUNCH(QQT_KERNEL_L1GRAD, l1_grad_reduce, dim3((n + 255) / 256), dim3(256), st, a,
               chunks, ws_cols);
    err = hipGetLastError();
  }
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "l1 grad launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // namespace

int qqt_l1_grad(const qqt_l1_grad_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (const int rc = l1_grad_check(a, "qqt_l1_grad")) return rc;
  if (!a->workspace) {
    snprintf(g_err, sizeof(g_err), "qqt_l1_grad: null workspace");
    return QQT_E_ARG;
  }
  if (a->workspace_floats < qqt_l1_grad_workspace_floats(a->batch, a->k0)) {
    snprintf(g_err, sizeof(g_err), "qqt_l1_grad: workspace too small");
    return QQT_E_ARG;
  }
  return l1_grad_launch(*a, (hipStream_t)stream);
}

int qqt_l1_grad_noalloc(const qqt_l1_grad_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (const int rc = l1_grad_check(a, "qqt_l1_grad_noalloc")) return rc;
  if (a->k0 > QQT_L1_GRAD_NOALLOC_MAX_K0) {
    snprintf(g_err, sizeof(g_err),
             "qqt_l1_grad_noalloc: k0 = %d exceeds the static scratch's maximum of %d columns",
             a->k0, QQT_L1_GRAD_NOALLOC_MAX_K0);
    return QQT_E_ARG;
  }
  float* const ptr = l1g::scratch_on_current_device();
  if (!ptr) return QQT_E_LAUNCH;
  qqt_l1_grad_args b = *a;          // the caller's workspace fields are ignored
  b.workspace = ptr;
  b.workspace_floats = (int64_t)l1g::MAX_CHUNKS * l1g::HID * QQT_L1_GRAD_NOALLOC_MAX_K0;
  if (b.workspace_floats < qqt_l1_grad_workspace_floats(b.batch, b.k0)) {
    snprintf(g_err, sizeof(g_err), "qqt_l1_grad_noalloc: plan exceeds the static scratch");
    return QQT_E_ARG;
  }
  return l1_grad_launch(b, (hipStream_t)stream);
}

}  // extern "C"
