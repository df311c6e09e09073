// Shared device helpers: Philox4x32-10, unit uniforms, the sampler's exp/log.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qqt {

// Rows (envs) of one XCD row block.  The act kernel's rollout-sized
// workgroups take this many rows, and the tick and bot kernels deal blocks
// of this many envs to the 8 XCDs the same way (block b: row block
// (b / 8 / workgroups per block) * 8 + b % 8), so an env's state, observation,
// masks and actions stay in the L2 of one XCD from kernel to kernel.  44 rows:
// 5632 envs are 16 blocks per XCD = 704 envs, exactly the tick kernel's one
// round on an XCD's 32 CUs (22 envs each), and 256 act workgroups.
constexpr int XCD_ROWS = 44;

// Envs per wavefront of the STEP tick: two (32 lanes each) up to
// GROUP32_MAX_ENVS envs, four above.  The tick writes the astar bot's reach
// source one blast-cap maximum per wavefront, i.e. per group of that many
// envs.
constexpr int GROUP32_MAX_ENVS = 8192;
__host__ __device__ inline int tick_envs_per_wave(int n_envs) {
  return n_envs <= GROUP32_MAX_ENVS ? 2 : 4;
}

// Philox stream ids (third counter word); the host oracle uses the same ids.
enum : uint32_t {
  STREAM_CRATE = 1, STREAM_RESET_CELL = 2, STREAM_RESET_MISC = 3,
  STREAM_POLICY = 4, STREAM_RANDOM_ACT = 5, STREAM_INJECT_ACT = 6, STREAM_BOT = 7,
  STREAM_RECYCLE = 8, STREAM_BOT_MODE = 9
};

// Philox4x32 with 10 rounds (Salmon et al., SC'11).  c holds the counter on
// entry and the four output words on exit.
__device__ __forceinline__ void philox10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c[0];
    const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]);
    const uint32_t lo1 = 0xCD9E8D57u * c[2];
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]);
    const uint32_t n0 = hi1 ^ c[1] ^ k0;
    const uint32_t n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// 24 random bits -> float in [0, 1), exact.
__device__ __forceinline__ float unit24(uint32_t x) {
  return (float)(x >> 8) * (1.0f / 16777216.0f);
}

// Uniform j of Philox(key=seed, ctr=(env, epoch, stream, j / 4)), word j % 4.
__device__ __forceinline__ float philox_uniform(uint64_t seed, uint32_t env, uint32_t epoch,
                                                uint32_t stream, uint32_t j) {
  uint32_t c[4] = {env, epoch, stream, j >> 2};
  philox10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const uint32_t w = (j & 3) == 0 ? c[0] : (j & 3) == 1 ? c[1] : (j & 3) == 2 ? c[2] : c[3];
  return unit24(w);
}

// Four uniforms of one block.
__device__ __forceinline__ void philox_block(uint64_t seed, uint32_t env, uint32_t epoch,
                                             uint32_t stream, uint32_t block, float u[4]) {
  uint32_t c[4] = {env, epoch, stream, block};
  philox10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  u[0] = unit24(c[0]); u[1] = unit24(c[1]); u[2] = unit24(c[2]); u[3] = unit24(c[3]);
}

// exp(x) for x <= 0 (Cody-Waite reduction, degree-6 Taylor polynomial), 0 below
// -80.  Same float32 operation sequence as the host sampler (no contraction).
__device__ __forceinline__ float exp_q(float x) {
  if (x < -80.0f) return 0.0f;
  const float n = rintf(x * 1.4426950408889634f);
  const float r = (x - n * 0.693145751953125f) - n * 1.428606765330187e-06f;
  float p = 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const float scale = __int_as_float(((int)n + 127) << 23);
  return p * scale;
}

// log(x) for normal x > 0: x = 2^k m, m in [sqrt(1/2), sqrt(2)), 2 atanh series.
__device__ __forceinline__ float log_q(float x) {
  const int bits = __float_as_int(x);
  int k = ((bits >> 23) & 0xFF) - 127;
  float m = __int_as_float((bits & 0x7FFFFF) | (127 << 23));
  if (m >= 1.4142135623730951f) { m = m * 0.5f; k += 1; }
  const float s = __fdiv_rn(m - 1.0f, m + 1.0f);
  const float s2 = s * s;
  float q = 1.0f / 9.0f;
  q = q * s2 + 1.0f / 7.0f;
  q = q * s2 + 1.0f / 5.0f;
  q = q * s2 + 1.0f / 3.0f;
  q = q * s2 + 1.0f;
  const float lm = 2.0f * (s * q);
  return (float)k * 0.6931471805599453f + lm;
}

// Dispatch timing (timing.hip): true, with an event pair, when the next
// launch of kernel kind `kind` (QQT_KERNEL_*) is to be timed.
bool timing_take(int kind, hipEvent_t* e0, hipEvent_t* e1);

// Kernel launch that records a start/stop event pair on the dispatch packet
// itself (hipExtLaunchKernel) when timing is armed.
#define QQT_LAUNCH(kind, kernel, grid, block, stream, ...)                              \
  do {                                                                                  \
    hipEvent_t qqt_e0_, qqt_e1_;                                                        \
    if (::qqt::timing_take((kind), &qqt_e0_, &qqt_e1_))                                 \
      hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, qqt_e0_, qqt_e1_, 0, __VA_ARGS__); \
    else                                                                                \
      hipLaunchKernelGGL(kernel, grid, block, 0, stream, __VA_ARGS__);                  \
  } while (0)

// Sync point of a wavefront that works alone on its own LDS region: one
// wavefront's LDS accesses are performed in program order, so the sync only
// has to keep the compiler from moving memory operations across it
// (wavefront-scope fences, no s_barrier and no wait for the LDS queue).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

// Observation row of batch row r for an argument block with row_index /
// obs_rows fields: row_index[r] clamped into [0, obs_rows) when the caller
// maps the batch onto rows of a larger buffer, else r.
template <class Args>
__device__ __forceinline__ int64_t obs_row(const Args& a, int r) {
  return a.row_index ? min(max(a.row_index[r], (int64_t)0), a.obs_rows - 1) : (int64_t)r;
}

}  // namespace qqt
