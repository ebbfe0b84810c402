// gs_strip.h -- the compositors' conservative strip culling and the "plain"
// record test.
//
// A 16x16 tile is walked as four strips of four pixel rows; a splat's strip
// mask says which strips may hold a pixel where the splat passes the alpha
// test (p >= plim).  A strip whose bit is clear is skipped, so the mask must
// never clear the bit of a strip with such a pixel.  The per-splat part
// (strip_consts_t, once per splat when its record is packed) and the per-tile
// part (strip_mask_t, once per staged record) are written once for the
// device and for a host build that tests this property against brute force
// with the divisions and square roots perturbed by their error bound
// (tests/test_strip_mask_cpu.py); Ops supplies div and sqrt, and the caller
// defines GS_HD as the function qualifiers of its compiler
// (__device__ __forceinline__ for HIP).
#pragma once

#include <stdint.h>

namespace gs {

// Per-splat constants of the strip test: the support ellipse
// q(dx, dy) = a dx^2 + 2b dx dy + c dy^2 <= tc (tau = -2 ln(thr/o) =
// -2 ln(2) plim, enlarged to tc = 1.02 tau + 1e-3) spans, on column dx,
//   dy = beta dx +- sqrt(gamma - delta dx^2),
//   beta = -b/c, gamma = tc/c, delta = det/c^2 (det = ac - b^2);
// its upper end is concave in dx with its maximum at the top point
// dxt = -b hy / a (hy = sqrt(a tc / det)), its lower end convex with its
// minimum at -dxt.  Two encodings stand outside the formula: a splat that is
// never culled (conics with det <= 1e-3 a c, i.e. |b| >= (1 - 5e-4)
// sqrt(ac), or huge tau) has {0, 0, +inf, 0}, whose span is infinite for
// every finite centre; an invisible one (plim > 0: p <= 0 < plim everywhere)
// has beta = NaN, which fails every comparison of strip_mask_t.  The margin
// of tc covers the rounding of p's chain and of the divisions and square
// roots (about 1 ulp each) for the other conics.
struct StripConsts {
  float dxt, beta, gamma, delta;
};

template <class Ops>
GS_HD StripConsts strip_consts_t(float a, float b, float c, float plim) {
  StripConsts k{0.0f, 0.0f, __builtin_inff(), 0.0f};
  if (plim > 0.0f) {
    k.beta = __builtin_nanf("");
    return k;
  }
  const float tau = -1.38629436f * plim;
  const float det = a * c - b * b;
  if (!(a > 0.0f && c > 0.0f && det > 1e-3f * (a * c) && tau < 3.0e38f))
    return k;
  const float tc = tau * 1.02f + 1e-3f;
  const float hy = Ops::sqrt(Ops::div(a * tc, det));
  k.dxt = Ops::div(-b * hy, a);
  k.beta = Ops::div(-b, c);
  k.gamma = Ops::div(tc, c);
  // (c * c rounded up or overflowing only lowers delta: a wider span)
  k.delta = Ops::div(det, c * c);
  return k;
}

// Bit k set unless strip k of the tile at (x0, y0) certainly holds no pixel
// with p >= plim.  The ellipse cut by the tile's slab of pixel-centre
// columns dx in [dxa, dxb] is convex, so its rows form one interval
// [dy_lo, dy_hi]: clamping the top and bottom points into the slab gives
// them, and a strip is kept iff its pixel-centre rows meet the interval.
// Rows are compared relative to the tile's first row centre y0 + 1/2
// (strip k's rows are 4k .. 4k + 3 there); rounding that difference never
// turns a kept strip into a skipped one, as 4k is exact.
template <class Ops>
GS_HD uint32_t strip_mask_t(const StripConsts& k, float mx, float my, int x0,
                            int y0) {
  const float dxa = ((float)x0 + 0.5f) - mx, dxb = dxa + 15.0f;
  const float ry = my - ((float)y0 + 0.5f);
  const float ut = fminf(fmaxf(k.dxt, dxa), dxb);
  const float ub = fminf(fmaxf(-k.dxt, dxa), dxb);
  const float sh = Ops::sqrt(fmaxf(k.gamma - (k.delta * ut) * ut, 0.0f));
  const float sl = Ops::sqrt(fmaxf(k.gamma - (k.delta * ub) * ub, 0.0f));
  const float y_hi = ry + (k.beta * ut + sh);
  const float y_lo = ry + (k.beta * ub - sl);
  uint32_t m = 0u;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (y_lo <= (float)(4 * s + 3) && y_hi >= (float)(4 * s)) m |= 1u << s;
  }
  return m;
}

// A "plain" splat: for it the compositors' tests e <= 0 and 2^p < max_alpha
// always hold, so they are left out (same results, fewer operations per
// pixel).  A = (-a/2) L, B = (-b) L, C = (-c/2) L as the compositors form
// them (L = log2(e) rounded to float), o the opacity, o_plain =
// plain_opacity_limit(max_alpha).  True when, for every pixel, the computed
// exponent e = fma(fma(C, dy, B dx), dy, (A dx) dx) is <= 0 and 2^p
// (p = fma(t, dy, (A dx) dx + lo)) stays below max_alpha:
//  * -p is the quadratic form a' dx^2 + b' dx dy + c' dy^2 (a' = -A,
//    b' = -B, c' = -C) whose smallest eigenvalue is at least
//    (4a'c' - b'^2) / (4 (a' + c')) >= 2^-18 (a' + c') when 4a'c' - b'^2 >=
//    2^-16 (a' + c')^2.  The chain computes (1 + d5) times c' dy^2 (1 + d2)
//    + b' dx dy (1 + d1)(1 + d2) + a' dx^2 (1 + d3)(1 + d4) (|di| <= 2^-24;
//    the last rounding only scales), which is off the quadratic form by at
//    most 2.0001 2^-24 (a' dx^2 + |b' dx dy| + c' dy^2) <= 3.0002 2^-24
//    (a' + c') (dx^2 + dy^2): the sign of p is never flipped.  Where the
//    inner fma cancels to a subnormal its absolute error, 2^-150 |dy|, is
//    below 2^-78 dy^2 for |dy| >= 2^-25.  The bounds on a', c',
//    |b'| and the centre keep every product of the chain normal and finite
//    (|dx| and |dy| are 0 or at least 2^-25, and at most 2^33, since pixel
//    centres are below 2^31); dx = dy = 0 gives e = +-0, which passes e <= 0;
//  * the unrounded t dy + (A dx) dx is <= 0 by the same bound, and the
//    rounding of (A dx) dx + lo adds at most 2^-24 (|(A dx) dx| + |lo|),
//    where 2^-24 |(A dx) dx| <= 2^-6 of the bound's margin, so p <= lo +
//    2^-23 |lo|.  lo is within 7 2^-24 |lo| of log2(o) (ln within 4 ulp, the
//    rounding of log2(e) and of the product), so 2^p <= o 2^(9 2^-24 |lo|),
//    which for 2^-20 <= o <= o_plain = max_alpha (1 - 2^-16) (|lo| <= 20)
//    and the hardware exp2 (within 1 ulp) stays below max_alpha: the clamp
//    and the gradient gate never act.
// NaN anywhere fails a comparison and leaves the splat on the general path.
GS_HD bool plain_record(float A, float B, float C, float mx, float my,
                        float o, float o_plain) {
  const float a = -A, c = -C, s = a + c;
  return (o >= 0x1p-20f) & (o <= o_plain) & (a >= 0x1p-60f) & (c >= 0x1p-60f) &
         (a <= 0x1p40f) & (c <= 0x1p40f) & (B <= 0x1p40f) & (B >= -0x1p40f) &
         (4.0f * a * c - B * B >= 0x1p-16f * s * s) & (mx <= 0x1p32f) &
         (mx >= -0x1p32f) & (my <= 0x1p32f) & (my >= -0x1p32f);
}

// o_plain of plain_record for a clamp value max_alpha.
GS_HD float plain_opacity_limit(float max_alpha) {
  return max_alpha * (1.0f - 0x1p-16f);
}

}  // namespace gs
