// gs_strip.h -- the compositors' conservative strip culling.
//
// A 16x16 tile is walked as four strips of four pixel rows; a splat's strip
// mask says which strips may hold a pixel where the splat passes the alpha
// test (p >= plim).  A strip whose bit is clear is skipped, so the mask must
// never clear the bit of a strip with such a pixel.  The function is written
// once for the device (hardware reciprocal and square root) and for a host
// build that tests this property against brute force with those two
// operations perturbed by their error bound (tests/test_strip_mask_cpu.py);
// Ops supplies rcp and sqrt, and the caller defines GS_HD as the function
// qualifiers of its compiler (__device__ __forceinline__ for HIP).
#pragma once

#include <stdint.h>

namespace gs {

// Bit k set unless strip k of the tile at (x0, y0) certainly holds no pixel
// with p >= plim.  The support ellipse q(dx, dy) = a dx^2 + 2b dx dy + c dy^2
// <= tc (tau = -2 ln(thr/o) = -2 ln(2) plim, enlarged to tc = 1.02 tau +
// 1e-3) cut by the tile's slab of pixel-centre columns dx in [dxa, dxb] is
// convex, so its rows form one interval [dy_lo, dy_hi]: a strip is kept iff
// its pixel-centre rows meet it.  On column dx the ellipse spans
//   dy = (-b dx +- sqrt(c tc - det dx^2)) / c,
// whose upper end is concave in dx with its maximum at the top point
// dx_t = -b hy / a (hy = sqrt(a tc / det)) and whose lower end is convex with
// its minimum at -dx_t; clamping those points into the slab gives dy_hi and
// dy_lo.  The margin of tc covers the rounding of p's chain and of the
// reciprocals and square roots here (about 1 ulp each) as long as
// det > 1e-3 a c (|b| < (1 - 5e-4) sqrt(ac)); other conics are never culled.
template <class Ops>
GS_HD uint32_t strip_mask_t(float mx, float my, float a, float b, float c,
                            float plim, int x0, int y0) {
  if (plim > 0.0f) return 0u;  // p <= 0 < plim: invisible everywhere
  const float tau = -1.38629436f * plim;
  const float det = a * c - b * b;
  if (!(a > 0.0f && c > 0.0f && det > 1e-3f * (a * c) && tau < 3.0e38f))
    return 0xFu;
  const float tc = tau * 1.02f + 1e-3f;
  const float inv_c = Ops::rcp(c);
  const float hy = Ops::sqrt(a * tc * Ops::rcp(det));
  const float dx_t = -b * hy * Ops::rcp(a);
  const float dxa = ((float)x0 + 0.5f) - mx, dxb = dxa + 15.0f;
  const float ct = c * tc;
  const float ut = fminf(fmaxf(dx_t, dxa), dxb);
  const float ub = fminf(fmaxf(-dx_t, dxa), dxb);
  const float y_hi = my + (-b * ut + Ops::sqrt(fmaxf(ct - det * ut * ut, 0.0f))) * inv_c;
  const float y_lo = my + (-b * ub - Ops::sqrt(fmaxf(ct - det * ub * ub, 0.0f))) * inv_c;
  uint32_t m = 0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float r0 = (float)(y0 + 4 * k) + 0.5f;  // first and last row centre
    if (y_lo <= r0 + 3.0f && y_hi >= r0) m |= 1u << k;
  }
  return m;
}

}  // namespace gs
