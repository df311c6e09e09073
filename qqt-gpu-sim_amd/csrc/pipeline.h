// Software-pipelined operand loads for the MFMA step loops (cnn.hip,
// lstm.hip): 16-byte raw buffer loads and a loop that keeps them in flight.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qqt {

// Buffer resource over `bytes` bytes at p (raw, unswizzled; offsets past the
// end read as zero).  Loads through it are intrinsic calls rather than plain
// loads, which the compiler does not merge across a loop's back edge into a
// load at the top of the iteration that consumes them (what it does to a
// plain load feeding a loop-carried value), so an operand loaded steps ahead
// stays in flight while those steps compute.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at byte offset byte_off, as V (a 16-byte vector type)
template <class V>
__device__ __forceinline__ V bld16(Rsrc r, uint32_t byte_off) {
  static_assert(sizeof(V) == 16, "16-byte loads");
  return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Software-pipelined loop over N steps: step st's operands are load(st),
// issued D steps ahead into a ring of D + 1 buffers, and compute(st, ops)
// consumes them.  The loop is unrolled by the ring's length, so every buffer
// keeps its registers across the back edge (a register copy of an operand
// still in flight would wait for it).  Loads of the last group past step
// N - 1 repeat step N - 1 and are not consumed.
template <int N, int D, class LD, class CP>
__device__ __forceinline__ void pipeline(LD load, CP compute) {
  constexpr int P = D + 1, G = N / P;
  decltype(load(0)) f[P];
#pragma unroll
  for (int i = 0; i < D && i < N; ++i) f[i] = load(i);
#pragma unroll 1
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int st = g * P + j;
      f[(j + D) % P] = load(min(st + D, N - 1));
      compute(st, f[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < N % P; ++j) {
    const int st = G * P + j;
    if (st + D < N) f[(j + D) % P] = load(st + D);
    compute(st, f[j]);
  }
}

}  // namespace qqt
