// Host build of the compositors' strip culling (fast-mac-gsplat_amd/csrc/
// gs_strip.h) for tests/test_strip_mask_cpu.py: the strip masks of splats on
// a tile, with the divisions and square roots rounded down, to nearest or up
// by twice their error bound, beside the strips that brute force finds
// holding a pixel that passes the compositors' alpha test.
#include <math.h>
#include <stdint.h>

#define GS_HD static inline
#include "../fast-mac-gsplat_amd/csrc/gs_strip.h"

namespace {

// Relative perturbation of the operations: 2^-22 (2 ulp) below, exact, or
// above (the per-splat constants are correctly rounded, the hardware square
// root of the per-tile part is within 1 ulp).
template <int Dir>
struct PerturbedOps {
  static float scale(float v) { return v * (1.0f + (float)Dir * 0x1p-22f); }
  static float div(float x, float y) { return scale(x / y); }
  static float sqrt(float x) { return scale(sqrtf(x)); }
};

template <int Dir>
uint32_t mask_of(float mx, float my, float a, float b, float c, float plim, int x0, int y0) {
  const gs::StripConsts k = gs::strip_consts_t<PerturbedOps<Dir>>(a, b, c, plim);
  return gs::strip_mask_t<PerturbedOps<Dir>>(k, mx, my, x0, y0);
}

// The compositors' exponent chain (composite.hip x_terms / exponents):
// A = (-a/2) L, B = (-b) L, C = (-c/2) L, t = fma(C, dy, B dx),
// e = fma(t, dy, (A dx) dx), p = fma(t, dy, (A dx) dx + lo); a pixel sees the
// splat iff e <= 0 and p >= plim + lo.
bool visible(float mx, float my, float a, float b, float c, float plim, float lo, float px,
             float py) {
  const float L = 1.44269502f;
  const float A = (-0.5f * a) * L, B = (-b) * L, C = (-0.5f * c) * L;
  const float dx = px - mx, dy = py - my;
  const float t = fmaf(C, dy, B * dx);
  const float a0 = (A * dx) * dx;
  const float e = fmaf(t, dy, a0);
  const float p = fmaf(t, dy, a0 + lo);
  return e <= 0.0f && p >= plim + lo;
}

}  // namespace

extern "C" int strip_mask_check(const float* splats, const float* plims, const int32_t* tiles, int n,
                                uint32_t* masks, uint32_t* needed) {
  for (int i = 0; i < n; ++i) {
    const float* s = splats + 6 * i;  // mx, my, a, b, c, lo
    const int x0 = tiles[2 * i], y0 = tiles[2 * i + 1];
    const float mx = s[0], my = s[1], a = s[2], b = s[3], c = s[4], plim = plims[i];
    masks[3 * i + 0] = mask_of<-1>(mx, my, a, b, c, plim, x0, y0);
    masks[3 * i + 1] = mask_of<0>(mx, my, a, b, c, plim, x0, y0);
    masks[3 * i + 2] = mask_of<1>(mx, my, a, b, c, plim, x0, y0);
    uint32_t need = 0;
    for (int k = 0; k < 4; ++k)
      for (int r = 0; r < 4; ++r)
        for (int col = 0; col < 16; ++col)
          if (visible(mx, my, a, b, c, plim, s[5], (float)(x0 + col) + 0.5f,
                      (float)(y0 + 4 * k + r) + 0.5f))
            need |= 1u << k;
    needed[i] = need;
  }
  return 0;
}
