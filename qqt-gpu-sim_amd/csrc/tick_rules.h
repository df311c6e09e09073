// Cell-word rules shared by the tick kernels: the packed cell word, the
// danger weight, ray walks over the grid and the AABB slide-stop movement
// (sim/move.py:154-231, sim/blast.py:43-317).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qqt {

constexpr uint32_t F_WALL = 1u << 24, F_BRICK = 1u << 25, F_CRATE = 1u << 26, F_REC = 1u << 27;
constexpr uint32_t EMPTY_CELL = 0x0000FF00u;  // fuse 0, owner -1, blast 0, no flags

__device__ __forceinline__ int cw_fuse(uint32_t w) { return (int)(w & 0xFFu); }
__device__ __forceinline__ int cw_owner(uint32_t w) { return (int)(int8_t)((w >> 8) & 0xFFu); }
__device__ __forceinline__ int cw_bb(uint32_t w) { return (int)((w >> 16) & 0xFFu); }
__device__ __forceinline__ uint32_t cw_make(uint32_t flags, int fuse, int owner, int bb) {
  return (flags & 0xFF000000u) | ((uint32_t)fuse & 0xFFu) | (((uint32_t)owner & 0xFFu) << 8) |
         (((uint32_t)bb & 0xFFu) << 16);
}
__device__ __forceinline__ bool cw_solid(uint32_t w) {  // stops flame and players
  return (w & F_BRICK) || cw_fuse(w) > 0;
}
__device__ __forceinline__ int blast_of(uint32_t w, int cfg_blast) {
  const int b = cw_bb(w);
  return b > 0 ? b : cfg_blast;
}

// Danger weight (1 - (f-1)/FUSE)^2 clamped at 0 (sim/blast.py:218-220).
__device__ __forceinline__ float bomb_weight(int f, float fuse_max) {
  const float raw = 1.0f - __fdiv_rn((float)f - 1.0f, fuse_max);
  const float v = raw > 0.0f ? raw : 0.0f;
  return v * v;
}

__device__ __forceinline__ int dir_dr(int d) { return d == 0 ? -1 : (d == 1 ? 1 : 0); }
__device__ __forceinline__ int dir_dc(int d) { return d == 2 ? -1 : (d == 3 ? 1 : 0); }

// Walk up to `len` steps from `src` in direction sgn * d, four cells per LDS
// round trip: the cell words of the next four steps are loaded together
// (out-of-grid steps read as a plain wall), then step(k, x, w) runs for
// k = 1, 2, ... in registers until it returns false.  Most rays end within
// the first four cells.
template <int H, int W, class F>
__device__ __forceinline__ void walk_ray(const uint32_t* cw, int src, int d, int len, int sgn,
                                         F&& step) {
  constexpr int KR = (H > W ? H : W) - 1;   // longest ray inside the grid
  constexpr int CH = 4;
  const int r0 = src / W, c0 = src % W, dr = sgn * dir_dr(d), dc = sgn * dir_dc(d);
  const int n = min(len, KR);
  for (int k0 = 1; k0 <= n; k0 += CH) {
    uint32_t w[CH];
    int x[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int k = k0 + i, rr = r0 + k * dr, cc = c0 + k * dc;
      const bool in = k <= n && rr >= 0 && rr < H && cc >= 0 && cc < W;
      const int xx = in ? rr * W + cc : src;
      const uint32_t v = cw[xx];
      x[i] = xx;
      w[i] = in ? v : F_WALL;
    }
    bool go = true;
#pragma unroll
    for (int i = 0; i < CH; ++i)
      if (go) go = step(k0 + i, x[i], w[i]);
    if (!go) break;
  }
}

// ---------------------------------------------------------------- movement
// One axis of the AABB slide-stop resolution (sim/move.py:154-231).
// `coord`/`delta` are the moved coordinate and displacement on this axis;
// (y, x) is the pre-move centre.  The two probed cells of a lead line lie at
// the box's own extent on the other axis (floor(other -+ r) with other the
// box centre), so the reference's "cell inside the current box" test reduces
// to the lead coordinate lying inside the box's extent on this axis.
template <int H, int W>
__device__ __forceinline__ float resolve_axis(const uint32_t* cw, float coord, float delta,
                                              float y, float x, float rad, bool vertical) {
  const float eps = 1e-4f;
  const float own = vertical ? y : x, other = vertical ? x : y;
  const int lim_own = vertical ? H : W, lim_oth = vertical ? W : H;
  const float sgn = delta > 0.0f ? 1.0f : (delta < 0.0f ? -1.0f : 0.0f);
  const int old_lead = (int)floorf((coord - delta) + sgn * rad);
  const int new_lead = (int)floorf(coord + sgn * rad);
  const int lo = min(old_lead, new_lead), hi = max(old_lead, new_lead);
  const int a0 = (int)floorf(other - rad), a1 = (int)floorf(other + rad);
  const int b0 = (int)floorf(own - rad), b1 = (int)floorf(own + rad);
  const bool span_oob = (a0 < 0) | (a0 >= lim_oth) | (a1 < 0) | (a1 >= lim_oth);
  const int a0c = min(max(a0, 0), lim_oth - 1), a1c = min(max(a1, 0), lim_oth - 1);
  auto hit = [&](int lead) -> bool {
    const int lc = min(max(lead, 0), lim_own - 1);
    const uint32_t w0 = vertical ? cw[lc * W + a0c] : cw[a0c * W + lc];
    const uint32_t w1 = vertical ? cw[lc * W + a1c] : cw[a1c * W + lc];
    const bool blk = (w0 & F_WALL) || cw_solid(w0) || (w1 & F_WALL) || cw_solid(w1);
    const bool inside = (lead >= b0) & (lead <= b1);
    return span_oob | (lead < 0) | (lead >= lim_own) | (blk & !inside);
  };
  const bool hit_lo = hit(lo);
  const bool hit_hi = hi == lo ? hit_lo : hit(hi);
  const bool fwd = sgn > 0.0f;
  const int first_lead = fwd ? hi : lo, second_lead = fwd ? lo : hi;
  const bool fh = fwd ? hit_hi : hit_lo, sh = fwd ? hit_lo : hit_hi;
  const int stop_cell = fh ? first_lead : (sh ? second_lead : 0);
  const float sc = (float)stop_cell;
  const float stop = fwd ? ((sc - rad) - eps) : (((sc + 1.0f) + rad) + eps);
  return (fh | sh) ? stop : coord;
}

}  // namespace qqt
