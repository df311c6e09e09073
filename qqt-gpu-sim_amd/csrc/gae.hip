// Generalised advantage estimation over a filled rollout buffer (the
// reverse-time scan of compute_gae, train/ppo.py:101-110).
//
// One thread per env walks t = T-1 .. 0.  The scan is sequential in t, so
// the reference's float32 rounding order is kept exactly: every product and
// sum rounds separately (the library is built with -ffp-contract=off), and
// gamma * lam arrives pre-rounded from the double product the reference's
// Python expression forms.  Loads do not depend on the running sum, so each
// block of 32 steps is loaded before its arithmetic.  Algorithmic bytes:
// 4 + 4 + 1 read and 8 written per (step, env); with one thread per env the
// kernel is bound by T / 32 rounds of memory latency, not by bandwidth (it
// runs once per collected rollout).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

constexpr int GAE_THREADS = 64;  // one wavefront per workgroup: the envs spread over more CUs
constexpr int GAE_BLOCK = 32;   // steps whose loads are in flight together

// Steps t1-1 .. t1-B of one env: loads first (indices clamped at 0), then the
// recurrence; steps below 0 (a partial last block) are skipped by predicate.
template <int B>
__device__ __forceinline__ void gae_block(const qqt_gae_args& a, const float* __restrict__ rew,
                                          const float* __restrict__ val,
                                          const uint8_t* __restrict__ done,
                                          float* __restrict__ adv, float* __restrict__ ret,
                                          int t1, float& gae, float& next_val) {
  const size_t ns = (size_t)a.n_envs;
  float r[B], v[B], d[B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const int t = t1 - 1 - i;
    const int tc = t < 0 ? 0 : t;
    r[i] = rew[(size_t)tc * a.step_stride];
    v[i] = val[(size_t)tc * a.step_stride];
    d[i] = (float)done[(size_t)tc * ns];
  }
#pragma unroll
  for (int i = 0; i < B; ++i) {
    const int t = t1 - 1 - i;
    if (t >= 0) {
      const float nt = 1.0f - d[i];
      const float delta = (r[i] + (a.gamma * next_val) * nt) - v[i];
      gae = delta + (a.gamma_lam * nt) * gae;
      adv[(size_t)t * ns] = gae;
      ret[(size_t)t * ns] = gae + v[i];
      next_val = v[i];
    }
  }
}

__global__ __launch_bounds__(GAE_THREADS) void gae_kernel(const qqt_gae_args a) {
  const int n = blockIdx.x * GAE_THREADS + (int)threadIdx.x;
  if (n >= a.n_envs) return;
  const float* __restrict__ rew = a.rew + (size_t)n * a.env_stride;
  const float* __restrict__ val = a.val + (size_t)n * a.env_stride;
  const uint8_t* __restrict__ done = a.done + n;
  float* __restrict__ adv = a.adv + n;
  float* __restrict__ ret = a.ret + n;
  float gae = 0.0f;
  float next_val = a.last_val[n];
  for (int t1 = a.steps; t1 > 0; t1 -= GAE_BLOCK)
    gae_block<GAE_BLOCK>(a, rew, val, done, adv, ret, t1, gae, next_val);
}

}  // namespace qqt

extern "C" {

int qqt_gae(const qqt_gae_args* a, void* stream) {
  using namespace qqt;
  g_err[0] = 0;
  if (!a || !a->rew || !a->val || !a->done || !a->last_val || !a->adv || !a->ret) {
    snprintf(g_err, sizeof(g_err), "qqt_gae: null argument");
    return QQT_E_ARG;
  }
  if (a->steps <= 0 || a->n_envs <= 0 || a->step_stride <= 0 || a->env_stride <= 0) {
    snprintf(g_err, sizeof(g_err), "qqt_gae: steps, n_envs and strides must be positive");
    return QQT_E_ARG;
  }
  QQT_LAUNCH(QQT_KERNEL_GAE, gae_kernel, dim3((a->n_envs + GAE_THREADS - 1) / GAE_THREADS),
             dim3(GAE_THREADS), (hipStream_t)stream, *a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "gae launch failed: %s", hipGetErrorString(err));
    return QQT_E_LAUNCH;
  }
  return QQT_OK;
}

}  // extern "C"
