// Dispatch timing for benchmark harnesses.
//
// Armed launches go through hipExtLaunchKernel with a start/stop event pair,
// so each pair spans exactly one dispatch packet (kernel begin to kernel
// end, the interval a kernel-trace profiler reports), instead of separate
// marker packets whose own latency would be counted.  Pairs come from a
// fixed pool created on the first arm; launches beyond the armed count or
// the pool run untimed.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "qqt_common.h"
#include "qqt_hip.h"

namespace qqt {

extern thread_local char g_err[512];

namespace {

constexpr int POOL = 4096;

struct Timing {
  std::mutex mu;
  bool created = false;
  int armed = 0;   // launches still to be timed
  int used = 0;    // pairs handed out since the last collect
  hipEvent_t start[POOL], stop[POOL];
  int kind[POOL];
};

Timing& timing() {
  static Timing t;
  return t;
}

}  // namespace

bool timing_take(int kind, hipEvent_t* e0, hipEvent_t* e1) {
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  if (t.armed <= 0 || t.used >= POOL) return false;
  --t.armed;
  const int i = t.used++;
  t.kind[i] = kind;
  *e0 = t.start[i];
  *e1 = t.stop[i];
  return true;
}

}  // namespace qqt

extern "C" {

int qqt_timing_arm(int32_t launches) {
  using namespace qqt;
  g_err[0] = 0;
  if (launches < 0 || launches > POOL) {
    snprintf(g_err, sizeof(g_err), "qqt_timing_arm: launches must be in [0, %d]", POOL);
    return QQT_E_ARG;
  }
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  if (!t.created) {
    for (int i = 0; i < POOL; ++i) {
      // no system-scope fence at the events (an L2 writeback that would slow
      // the timed dispatch and the kernel after it): the timestamps alone
      if (hipEventCreateWithFlags(&t.start[i], hipEventDisableSystemFence) != hipSuccess ||
          hipEventCreateWithFlags(&t.stop[i], hipEventDisableSystemFence) != hipSuccess) {
        snprintf(g_err, sizeof(g_err), "qqt_timing_arm: hipEventCreate failed");
        return QQT_E_LAUNCH;
      }
    }
    t.created = true;
  }
  t.armed += launches;
  return QQT_OK;
}

int qqt_timing_collect(double* ms, int32_t* count, int32_t n_kinds) {
  using namespace qqt;
  g_err[0] = 0;
  if (!ms || !count || n_kinds <= 0) {
    snprintf(g_err, sizeof(g_err), "qqt_timing_collect: null output or n_kinds <= 0");
    return QQT_E_ARG;
  }
  for (int k = 0; k < n_kinds; ++k) {
    ms[k] = 0.0;
    count[k] = 0;
  }
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  for (int i = 0; i < t.used; ++i) {
    float e = 0.0f;
    if (hipEventSynchronize(t.stop[i]) != hipSuccess ||
        hipEventElapsedTime(&e, t.start[i], t.stop[i]) != hipSuccess) {
      snprintf(g_err, sizeof(g_err), "qqt_timing_collect: event query failed (%s)",
               hipGetErrorString(hipGetLastError()));
      t.used = 0;
      t.armed = 0;
      return QQT_E_LAUNCH;
    }
    if (t.kind[i] >= 0 && t.kind[i] < n_kinds) {
      ms[t.kind[i]] += (double)e;
      count[t.kind[i]] += 1;
    }
  }
  t.used = 0;
  t.armed = 0;
  return QQT_OK;
}

}  // extern "C"
