// gs_predicate.h -- splat support / tile-overlap predicate used by binning.
//
// These functions decide which (splat, tile) pairs exist, so their results
// must be reproducible bit for bit by the CPU oracle.  Every operation here
// is an IEEE-754 single-precision +, -, *, /, sqrt, floor, ceil, min, max or
// compare (all correctly rounded on gfx950 with the library's build flags),
// FP contraction is switched off, and the one transcendental (log) is
// computed by gs_logf below from those operations only.
//
// Semantics follow the reference's predicate:
//   alpha_support_params  variants/v8/csrc/metal/gsplat_v8_kernels.metal:77-82
//   snugbox               gsplat_v8_kernels.metal:84-93
//   ellipse_intersects_rect gsplat_v8_kernels.metal:95-119
//   tile rectangle        gsplat_v8_kernels.metal:275-281
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// Natural logarithm for x > 0 by binary range reduction and the atanh series
// (Abramowitz & Stegun 4.1.27: ln m = 2 atanh(s), s = (m-1)/(m+1)), with
// m in [sqrt(1/2), sqrt(2)) so |s| <= 0.1716 and terms through s^11 leave a
// truncation error below 1e-10 relative.  ln 2 is split Cody-Waite style
// (hi has 12 trailing zero bits, so e*hi is exact).  Accuracy is a few ulp;
// what matters is that the result is a fixed function of x built only from
// correctly rounded operations, so host and device agree exactly.
__device__ __forceinline__ float gs_logf(float x) {
#pragma clang fp contract(off)
  if (!(x == x)) return x;                                    // NaN
  if (x <= 0.0f) return (x == 0.0f) ? -__builtin_inff() : __builtin_nanf("");
  if (x == __builtin_inff()) return x;
  uint32_t u = __float_as_uint(x);
  int e = 0;
  if ((u >> 23) == 0u) {                                      // subnormal
    x = x * 8388608.0f;                                       // 2^23, exact
    u = __float_as_uint(x);
    e = -23;
  }
  e += (int)((u >> 23) & 0xffu) - 127;
  float m = __uint_as_float((u & 0x007fffffu) | 0x3f800000u); // [1, 2)
  if (m > 1.41421354f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 0.0909090936f;                 // 1/11
  p = p * z + 0.111111112f;                // 1/9
  p = p * z + 0.142857149f;                // 1/7
  p = p * z + 0.200000003f;                // 1/5
  p = p * z + 0.333333343f;                // 1/3
  p = p * z;
  const float two_s = s + s;
  const float lnm = two_s + two_s * p;
  const float fe = (float)e;
  return fe * 0.693115234f + (fe * 3.19461833e-05f + lnm);
}

// Support of o*exp(-q/2) >= thr:  q <= tau = -2 ln(max(thr / max(o,eps), eps)).
__device__ __forceinline__ bool alpha_support(float opacity, float thr,
                                              float eps, float& tau) {
#pragma clang fp contract(off)
  if (opacity <= thr) return false;
  const float ratio = fmaxf(thr / fmaxf(opacity, eps), eps);
  tau = -2.0f * gs_logf(ratio);
  return __builtin_isfinite(tau) && (tau > 0.0f);
}

// log2(e) rounded to float.  The compositor evaluates the exponent in base 2:
// p = kLog2e * power, alpha = min(max_alpha, o * 2^p).
constexpr float kLog2e = 1.44269502f;

// Base-2 exponent limit of the compositor's alpha test.  The reference's test
// min(max_alpha, o*exp(power)) >= alpha_threshold (eval_alpha,
// gsplat_v8_kernels.metal:121-139) is evaluated as p >= plim with
//   plim = kLog2e * ln(max(alpha_threshold / o, FLT_MIN)),
// which is the same condition up to rounding, but is decided by a fixed
// function of the inputs that the CPU oracle reproduces bit for bit.
// +inf (nothing visible) when o is not positive or max_alpha < threshold;
// -inf (every p <= 0 visible) when the threshold is not positive.
__device__ __forceinline__ float visibility_limit(float opacity, float thr,
                                                  float max_alpha) {
#pragma clang fp contract(off)
  if (!(opacity > 0.0f) || max_alpha < thr) return __builtin_inff();
  if (!(thr > 0.0f)) return -__builtin_inff();
  const float ratio = fmaxf(thr / opacity, 1.17549435e-38f);
  return kLog2e * gs_logf(ratio);
}

// Base-2 logarithm of the opacity, kLog2e * ln(o) by gs_logf (-inf for
// o = 0, NaN for o < 0 or NaN): the compositors evaluate o * 2^p as
// 2^(p + lo) and test visibility as p + lo >= plim + lo.
__device__ __forceinline__ float opacity_log2(float o) {
  return kLog2e * gs_logf(o);
}

__device__ __forceinline__ int clamp_to_int(float v) {
  // Saturating float->int for the bbox corners (NaN -> 0).  Values that
  // matter are small integers already.
  v = fminf(fmaxf(v, -1073741824.0f), 1073741824.0f);
  return (int)v;
}

struct PixBox {
  int x0, y0, x1, y1;  // inclusive pixel bbox; empty if x0 > x1 or y0 > y1
};

__device__ __forceinline__ PixBox snugbox(float mx, float my, float a, float b,
                                          float c, float tau, int width,
                                          int height, float eps) {
#pragma clang fp contract(off)
  const float det = fmaxf(a * c - b * b, eps);
  const float hx = __builtin_sqrtf(fmaxf(tau * c / det, 0.0f));
  const float hy = __builtin_sqrtf(fmaxf(tau * a / det, 0.0f));
  PixBox r;
  r.x0 = max(0, clamp_to_int(floorf(mx - hx - 0.5f)));
  r.x1 = min(width - 1, clamp_to_int(ceilf(mx + hx - 0.5f)));
  r.y0 = max(0, clamp_to_int(floorf(my - hy - 0.5f)));
  r.y1 = min(height - 1, clamp_to_int(ceilf(my + hy - 0.5f)));
  return r;
}

__device__ __forceinline__ float quad_form(float a, float b, float c, float dx,
                                           float dy) {
#pragma clang fp contract(off)
  return a * dx * dx + 2.0f * b * dx * dy + c * dy * dy;
}

// Per-splat constants of the rectangle test: the slopes -(b/c) and -(b/a) of
// the lines where the quadratic is minimal along x = const and y = const.
struct ConicSlopes {
  float kc, ka;
  bool use_c, use_a;
};

__device__ __forceinline__ ConicSlopes conic_slopes(float a, float b,
                                                    float c) {
#pragma clang fp contract(off)
  ConicSlopes s;
  s.use_c = c > 1e-8f;
  s.use_a = a > 1e-8f;
  s.kc = s.use_c ? -(b / c) : 0.0f;
  s.ka = s.use_a ? -(b / a) : 0.0f;
  return s;
}

// Exact minimum of the conic quadratic over the axis-aligned rectangle of
// pixel centres [rx0,rx1]x[ry0,ry1] compared against tau.
__device__ __forceinline__ bool ellipse_hits_rect(float mx, float my, float a,
                                                  float b, float c,
                                                  const ConicSlopes& k,
                                                  float tau, float rx0,
                                                  float ry0, float rx1,
                                                  float ry1) {
#pragma clang fp contract(off)
  if (mx >= rx0 && mx <= rx1 && my >= ry0 && my <= ry1) return true;
  const float dx0 = rx0 - mx, dx1 = rx1 - mx;
  const float dy0 = ry0 - my, dy1 = ry1 - my;
  // The corner nearest the centre first: its quadratic is one of the terms
  // minimised below, so if it is within tau the minimum is too and the
  // answer is already known (the same decision, bit for bit).  Tiles inside
  // a large splat, most of its candidates, end here.
  const float cx = fabsf(dx0) <= fabsf(dx1) ? dx0 : dx1;
  const float cy = fabsf(dy0) <= fabsf(dy1) ? dy0 : dy1;
  if (quad_form(a, b, c, cx, cy) <= tau) return true;
  float q = quad_form(a, b, c, dx0, dy0);
  q = fminf(q, quad_form(a, b, c, dx0, dy1));
  q = fminf(q, quad_form(a, b, c, dx1, dy0));
  q = fminf(q, quad_form(a, b, c, dx1, dy1));
  if (k.use_c) {
    float dy = fminf(fmaxf(k.kc * dx0, dy0), dy1);
    q = fminf(q, quad_form(a, b, c, dx0, dy));
    dy = fminf(fmaxf(k.kc * dx1, dy0), dy1);
    q = fminf(q, quad_form(a, b, c, dx1, dy));
  }
  if (k.use_a) {
    float dx = fminf(fmaxf(k.ka * dy0, dx0), dx1);
    q = fminf(q, quad_form(a, b, c, dx, dy0));
    dx = fminf(fmaxf(k.ka * dy1, dx0), dx1);
    q = fminf(q, quad_form(a, b, c, dx, dy1));
  }
  return q <= tau;
}

// Pixel-centre rectangle of tile (tx, ty), clipped to the image.
__device__ __forceinline__ void tile_rect(int tx, int ty, int width, int height,
                                          float& rx0, float& ry0, float& rx1,
                                          float& ry1) {
#pragma clang fp contract(off)
  rx0 = (float)(tx * 16) + 0.5f;
  rx1 = fminf((float)(width - 1) + 0.5f, (float)(tx * 16 + 15) + 0.5f);
  ry0 = (float)(ty * 16) + 0.5f;
  ry1 = fminf((float)(height - 1) + 0.5f, (float)(ty * 16 + 15) + 0.5f);
}

}  // namespace gs
