/*
 * tile_oracle.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the
 * reference's batched tile rasterizer, used by tests/ (as the parity checker)
 * and by bench.py's cpu_baseline leg (timed beside the GPU path).  Product
 * code never links, loads or calls it.
 *
 * Reference algorithm restated here (nbardy/fast-mac-gsplat, variants/v8):
 *   depth order      torch.argsort(depths, stable=True) per image
 *                    (torch_gsplat_bridge_v8/rasterize.py:466)
 *   alpha_support    csrc/metal/gsplat_v8_kernels.metal:77-82
 *   snugbox          gsplat_v8_kernels.metal:84-93
 *   ellipse/rect     gsplat_v8_kernels.metal:95-119
 *   tile loop        gsplat_v8_kernels.metal:271-287 (count) / :309-326 (emit)
 *   in-tile order    ascending sorted index (bitonic sort, :141-164)
 *   eval_alpha       gsplat_v8_kernels.metal:121-139
 *   forward + stop   gsplat_v8_kernels.metal:444-475
 *   backward         gsplat_v8_kernels.metal:511-607 (forward replay for
 *                    T_final / end_i, then the reverse gT recurrence)
 *
 * The binning predicate is evaluated in float32 with FP contraction off
 * (build with -ffp-contract=off) and with the logarithm below, so that its
 * results are a fixed function of the inputs: the HIP kernels must reproduce
 * the tile lists bit for bit.  Compositing is float32 like the reference
 * kernels with a fixed rounding chain for the Gaussian exponent and an exact
 * visibility decision (see eval_alpha); it is compared with tolerances, and
 * pixels whose early-stop or gradient-gate decisions fall inside exp's
 * last-ulp window are flagged.  Such a pixel's stop may be forced to another
 * implementation's decision (force_last), which the oracle accepts only when
 * that decision also lies inside the window.
 *
 * Parallel (OpenMP) over fixed chunks of splats and over tiles; every result
 * is independent of the thread count.  Each per-(pixel, splat) gradient
 * contribution is computed in float32 as the reference does; the per-splat
 * sums are accumulated in double in a fixed order (tile by tile), and beside
 * them the backward reports per gradient entry the sums of cancellation-free
 * magnitudes of the contributions (error-bound inputs for the tests).
 *
 * Pinned by (tests/test_oracle_cpu.py): brute-force completeness/tightness of
 * the predicate in double precision, oracle_logf against libm, the dense
 * Torch reference (oracle/dense_reference.py) on small scenes, closed forms,
 * a serial float32 restatement of the backward (tests/test_oracle_bounds_cpu.py)
 * and planted-error checks of the error bounds.
 */
#define _GNU_SOURCE
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int32_t height, width, batch, gpb;
  float alpha_threshold, transmittance_threshold;
  float bg[3];
  float eps, max_alpha;
} oracle_meta;

/* ------------------------------------------------------------------ log */
/* ln(x) by binary range reduction to m in [sqrt(1/2), sqrt(2)) and the atanh
 * series ln m = 2(s + s^3/3 + ... + s^11/11), s = (m-1)/(m+1)
 * (Abramowitz & Stegun 4.1.27), ln 2 split into a 12-trailing-zero-bit high
 * part and a low part (Cody & Waite).  Same constants and operation order as
 * the device predicate, so results agree bit for bit. */
static inline float f_from_u(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t u_from_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_logf(float x) {
  if (!(x == x)) return x;
  if (x <= 0.0f) return (x == 0.0f) ? -INFINITY : NAN;
  if (x == INFINITY) return x;
  uint32_t u = u_from_f(x);
  int e = 0;
  if ((u >> 23) == 0u) {
    x = x * 8388608.0f;
    u = u_from_f(x);
    e = -23;
  }
  e += (int)((u >> 23) & 0xffu) - 127;
  float m = f_from_u((u & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421354f) {
    m = m * 0.5f;
    e += 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 0.0909090936f;
  p = p * z + 0.111111112f;
  p = p * z + 0.142857149f;
  p = p * z + 0.200000003f;
  p = p * z + 0.333333343f;
  p = p * z;
  const float two_s = s + s;
  const float lnm = two_s + two_s * p;
  const float fe = (float)e;
  return fe * 0.693115234f + (fe * 3.19461833e-05f + lnm);
}

/* ------------------------------------------------------------ predicate */
static int alpha_support(float o, float thr, float eps, float* tau) {
  if (o <= thr) return 0;
  const float ratio = fmaxf(thr / fmaxf(o, eps), eps);
  *tau = -2.0f * oracle_logf(ratio);
  return isfinite(*tau) && (*tau > 0.0f);
}

static int sat_int(float v) {
  v = fminf(fmaxf(v, -1073741824.0f), 1073741824.0f);
  return (int)v;
}

static float qform(float a, float b, float c, float dx, float dy) {
  return a * dx * dx + 2.0f * b * dx * dy + c * dy * dy;
}

static int ellipse_rect(float mx, float my, float a, float b, float c, float tau,
                        float rx0, float ry0, float rx1, float ry1) {
  if (mx >= rx0 && mx <= rx1 && my >= ry0 && my <= ry1) return 1;
  const float dx0 = rx0 - mx, dx1 = rx1 - mx, dy0 = ry0 - my, dy1 = ry1 - my;
  float q = INFINITY;
  q = fminf(q, qform(a, b, c, dx0, dy0));
  q = fminf(q, qform(a, b, c, dx0, dy1));
  q = fminf(q, qform(a, b, c, dx1, dy0));
  q = fminf(q, qform(a, b, c, dx1, dy1));
  if (c > 1e-8f) {
    float dy = fminf(fmaxf(-(b / c) * dx0, dy0), dy1);
    q = fminf(q, qform(a, b, c, dx0, dy));
    dy = fminf(fmaxf(-(b / c) * dx1, dy0), dy1);
    q = fminf(q, qform(a, b, c, dx1, dy));
  }
  if (a > 1e-8f) {
    float dx = fminf(fmaxf(-(b / a) * dy0, dx0), dx1);
    q = fminf(q, qform(a, b, c, dx, dy0));
    dx = fminf(fmaxf(-(b / a) * dy1, dx0), dx1);
    q = fminf(q, qform(a, b, c, dx, dy1));
  }
  return q <= tau;
}

/* Visits the tiles hit by one splat in row-major order.  If out != NULL the
 * global tile ids are stored there.  Returns the number of tiles hit. */
static int splat_tiles(const oracle_meta* M, float mx, float my, float a, float b,
                       float c, float o, int batch, int32_t* out) {
  float tau;
  if (!alpha_support(o, M->alpha_threshold, M->eps, &tau)) return 0;
  const float det = fmaxf(a * c - b * b, M->eps);
  const float hx = sqrtf(fmaxf(tau * c / det, 0.0f));
  const float hy = sqrtf(fmaxf(tau * a / det, 0.0f));
  int x0 = sat_int(floorf(mx - hx - 0.5f));
  int x1 = sat_int(ceilf(mx + hx - 0.5f));
  int y0 = sat_int(floorf(my - hy - 0.5f));
  int y1 = sat_int(ceilf(my + hy - 0.5f));
  if (x0 < 0) x0 = 0;
  if (y0 < 0) y0 = 0;
  if (x1 > M->width - 1) x1 = M->width - 1;
  if (y1 > M->height - 1) y1 = M->height - 1;
  if (x0 > x1 || y0 > y1) return 0;
  const int tiles_x = (M->width + 15) / 16, tiles_y = (M->height + 15) / 16;
  const int base = batch * tiles_x * tiles_y;
  int n = 0;
  for (int ty = y0 / 16; ty <= y1 / 16; ++ty) {
    const float ry0 = (float)(ty * 16) + 0.5f;
    const float ry1 = fminf((float)(M->height - 1) + 0.5f, (float)(ty * 16 + 15) + 0.5f);
    for (int tx = x0 / 16; tx <= x1 / 16; ++tx) {
      const float rx0 = (float)(tx * 16) + 0.5f;
      const float rx1 = fminf((float)(M->width - 1) + 0.5f, (float)(tx * 16 + 15) + 0.5f);
      if (ellipse_rect(mx, my, a, b, c, tau, rx0, ry0, rx1, ry1)) {
        if (out) out[n] = base + ty * tiles_x + tx;
        ++n;
      }
    }
  }
  return n;
}

/* ---------------------------------------------------------- depth order */
static int cmp_depth_r(const void* pa, const void* pb, void* ctx) {
  const float* depths = (const float*)ctx;
  const int32_t ia = *(const int32_t*)pa, ib = *(const int32_t*)pb;
  const float a = depths[ia], b = depths[ib];
  const int na = !(a == a), nb = !(b == b);
  if (na != nb) return na ? 1 : -1;   /* NaN sorts last */
  if (!na) {
    if (a < b) return -1;
    if (a > b) return 1;              /* -0.0 == +0.0 */
  }
  return (ia < ib) ? -1 : (ia > ib);  /* stable: original index */
}

/* perm[b*G + r] = original index (within image b) of depth rank r. */
void oracle_depth_order(const float* depths, int32_t B, int32_t G, int32_t* perm) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t b = 0; b < B; ++b) {
    int32_t* p = perm + (int64_t)b * G;
    for (int32_t i = 0; i < G; ++i) p[i] = i;
    qsort_r(p, (size_t)G, sizeof(int32_t), cmp_depth_r, (void*)(depths + (int64_t)b * G));
  }
}

/* ------------------------------------------------------------- binning */
/* Splats are processed in kChunks fixed contiguous gid ranges (independent of
 * the thread count), so per-chunk tile counts give every chunk its own
 * cursors into the tile ranges and the scatter keeps ascending gid order
 * inside every tile. */
enum { kChunks = 256 };

static int64_t num_tiles(const oracle_meta* M) {
  return (int64_t)M->batch * ((M->width + 15) / 16) * ((M->height + 15) / 16);
}

static int64_t tiles_per_image(const oracle_meta* M) {
  return (int64_t)((M->width + 15) / 16) * ((M->height + 15) / 16);
}

static int splat_tiles_of_gid(const oracle_meta* M, const float* means2d,
                              const float* conics, const float* opac,
                              const int32_t* perm, int64_t gid, int32_t* out) {
  const int b = (int)(gid / M->gpb);
  const int64_t o = (int64_t)b * M->gpb + perm[gid];
  return splat_tiles(M, means2d[2 * o], means2d[2 * o + 1], conics[3 * o],
                     conics[3 * o + 1], conics[3 * o + 2], opac[o], b, out);
}

/* chunk_counts [kChunks][T]: tiles hit by each chunk's splats. */
static int32_t* chunk_tile_counts(const oracle_meta* M, const float* means2d,
                                  const float* conics, const float* opac,
                                  const int32_t* perm) {
  const int64_t tiles = num_tiles(M), tpi = tiles_per_image(M);
  const int64_t BG = (int64_t)M->batch * M->gpb;
  int32_t* cc = (int32_t*)calloc((size_t)kChunks * (size_t)(tiles > 0 ? tiles : 1), sizeof(int32_t));
#pragma omp parallel
  {
    int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(tpi > 0 ? tpi : 1));
#pragma omp for schedule(dynamic, 1)
    for (int c = 0; c < kChunks; ++c) {
      int32_t* cnt = cc + (int64_t)c * tiles;
      for (int64_t gid = BG * c / kChunks; gid < BG * (c + 1) / kChunks; ++gid) {
        const int n = splat_tiles_of_gid(M, means2d, conics, opac, perm, gid, tmp);
        for (int k = 0; k < n; ++k) cnt[tmp[k]]++;
      }
    }
    free(tmp);
  }
  return cc;
}

/* Inputs in original order; perm from oracle_depth_order.  Fills
 * tile_counts[T] and tile_offsets[T+1]; returns N. */
int64_t oracle_bin_count(const oracle_meta* M, const float* means2d, const float* conics,
                         const float* opac, const int32_t* perm, int32_t* tile_counts,
                         int32_t* tile_offsets) {
  const int64_t tiles = num_tiles(M);
  int32_t* cc = chunk_tile_counts(M, means2d, conics, opac, perm);
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < tiles; ++t) {
    int32_t s = 0;
    for (int c = 0; c < kChunks; ++c) s += cc[(int64_t)c * tiles + t];
    tile_counts[t] = s;
  }
  free(cc);
  int64_t run = 0;
  for (int64_t t = 0; t < tiles; ++t) {
    tile_offsets[t] = (int32_t)run;
    run += tile_counts[t];
  }
  tile_offsets[tiles] = (int32_t)run;
  return run;
}

/* binned_ids[N]: gids grouped by tile, ascending inside each tile. */
void oracle_bin_fill(const oracle_meta* M, const float* means2d, const float* conics,
                     const float* opac, const int32_t* perm, const int32_t* tile_offsets,
                     int32_t* binned_ids) {
  const int64_t tiles = num_tiles(M), tpi = tiles_per_image(M);
  const int64_t BG = (int64_t)M->batch * M->gpb;
  int32_t* cc = chunk_tile_counts(M, means2d, conics, opac, perm);
  /* cursors: chunk c's first slot in tile t */
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < tiles; ++t) {
    int32_t run = tile_offsets[t];
    for (int c = 0; c < kChunks; ++c) {
      const int32_t n = cc[(int64_t)c * tiles + t];
      cc[(int64_t)c * tiles + t] = run;
      run += n;
    }
  }
#pragma omp parallel
  {
    int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(tpi > 0 ? tpi : 1));
#pragma omp for schedule(dynamic, 1)
    for (int c = 0; c < kChunks; ++c) {
      int32_t* cur = cc + (int64_t)c * tiles;
      for (int64_t gid = BG * c / kChunks; gid < BG * (c + 1) / kChunks; ++gid) {
        const int n = splat_tiles_of_gid(M, means2d, conics, opac, perm, gid, tmp);
        for (int k = 0; k < n; ++k) binned_ids[cur[tmp[k]]++] = (int32_t)gid;
      }
    }
    free(tmp);
  }
  free(cc);
}

/* ---------------------------------------------------------- compositing */
typedef struct {
  float mx, my, a, b, c, o, r, g, bl;
  float plim; /* base-2 exponent limit of the alpha test (oracle_plim) */
  float lo;   /* log2 of the opacity (oracle_opacity_log2) */
  float q;    /* plim + lo: the limit of the exponent with lo folded in */
  int64_t orig;
} splat_t;

#define LOG2E_F 1.44269502f

/* Base-2 exponent at which o * 2^p reaches alpha_threshold:
 * log2(e)_f32 * ln(max(thr / o, FLT_MIN)) with oracle_logf; +inf when nothing
 * can be visible (o <= 0 or max_alpha < thr), -inf when thr <= 0.  The
 * compositor tests p >= plim, which is the reference's
 * min(max_alpha, o*exp(power)) >= alpha_threshold (eval_alpha,
 * gsplat_v8_kernels.metal:121-139) up to rounding; the packed records written
 * by binning carry this exact value. */
float oracle_plim(float o, float thr, float max_alpha) {
  if (!(o > 0.0f) || max_alpha < thr) return INFINITY;
  if (!(thr > 0.0f)) return -INFINITY;
  const float ratio = fmaxf(thr / o, 1.17549435e-38f);
  return LOG2E_F * oracle_logf(ratio);
}

/* log2(e)_f32 * ln(o) with oracle_logf (-inf for o = 0, NaN for o < 0 or
 * NaN): the compositors evaluate o * 2^p as 2^(p + lo); the packed records
 * written by binning carry this exact value. */
float oracle_opacity_log2(float o) { return LOG2E_F * oracle_logf(o); }

/* Depth-ordered splat records (index gid), gathered once. */
static splat_t* gather_splats(const oracle_meta* M, const float* means2d, const float* conics,
                              const float* colors, const float* opac, const int32_t* perm) {
  const int64_t BG = (int64_t)M->batch * M->gpb;
  splat_t* sp = (splat_t*)malloc(sizeof(splat_t) * (size_t)(BG > 0 ? BG : 1));
#pragma omp parallel for schedule(static)
  for (int64_t gid = 0; gid < BG; ++gid) {
    splat_t s;
    const int64_t b = gid / M->gpb;
    const int64_t o = b * M->gpb + perm[gid];
    s.mx = means2d[2 * o]; s.my = means2d[2 * o + 1];
    s.a = conics[3 * o]; s.b = conics[3 * o + 1]; s.c = conics[3 * o + 2];
    s.r = colors[3 * o]; s.g = colors[3 * o + 1]; s.bl = colors[3 * o + 2];
    s.o = opac[o];
    s.plim = oracle_plim(s.o, M->alpha_threshold, M->max_alpha);
    s.lo = oracle_opacity_log2(s.o);
    s.q = s.plim + s.lo;
    s.orig = o;
    sp[gid] = s;
  }
  return sp;
}

/* Reference eval_alpha: visible iff power <= 0 and alpha >= threshold, with
 * power = -0.5*(a dx^2 + 2 b dx dy + c dy^2) and alpha = min(max_alpha,
 * o exp(power)).  Evaluated in base 2 by a fixed chain of roundings,
 *   A = (-a/2) L, B = (-b) L, C = (-c/2) L   (L = log2(e) rounded to float)
 *   t = fma(C, dy, B dx)
 *   e = fma(t, dy, (A dx) dx)            (L power)
 *   p = fma(t, dy, (A dx) dx + lo)       (L power + log2(o))
 * with the visibility decision e <= 0 and p >= q = plim + lo (oracle_plim,
 * oracle_opacity_log2), which the HIP compositor takes bit for bit the same
 * way, and alpha = min(max_alpha, 2^p).  The decision is exact for this
 * base-2 form, not for the reference's own form (below), which rounds power
 * differently and takes exp: the two can disagree where alpha lies within
 * rounding of alpha_threshold, flagged AMB_ALPHA.  2^p is rounded once from
 * double; the hardware exp2 is within 1 ulp, so later decisions that depend
 * on the value of alpha (early stop on T, the max_alpha gradient gate) can
 * differ in their last-ulp window, reported through the ambiguity flags. */
#define AMB_ALPHA 1  /* the reference's form may decide the alpha test otherwise */
#define AMB_STOP 2   /* T within rounding of transmittance_threshold */
#define AMB_GATE 4   /* raw alpha within rounding of max_alpha (gradient gate) */
#define AMB_FORCED_BAD 8 /* a forced stop lies outside the ambiguity window */
#define AMB_ALPHA_FLIP 16 /* ... and does: the two forms' decisions differ */
#define AMB_REL 4e-7f
/* AMB_ALPHA window: the reference's raw alpha within this many float ulps
 * (2^-24 relative) of alpha_threshold.  Its exp is libm's here, torch's in
 * the dense reference and Metal's in the reference kernels (a few ulps
 * apart). */
#define AMB_ALPHA_ULPS 16.0f

static void splat_exponents(const splat_t* s, float dx, float dy, float* e, float* p) {
  const float A = (-0.5f * s->a) * LOG2E_F, B = (-s->b) * LOG2E_F;
  const float C = (-0.5f * s->c) * LOG2E_F;
  const float t = fmaf(C, dy, B * dx);
  const float a0 = (A * dx) * dx;
  *e = fmaf(t, dy, a0);
  *p = fmaf(t, dy, a0 + s->lo);
}

/* The reference's own visibility decision (gsplat_v8_kernels.metal:129-138;
 * the dense Torch reference computes the same expression): float32, left to
 * right, no contraction (this file is built with -ffp-contract=off), exp
 * from libm.  *raw_ref = o exp(power) (0 when power > 0). */
static int ref_form_visible(const oracle_meta* M, const splat_t* s, float dx, float dy, float* raw_ref) {
  const float power = -0.5f * (s->a * dx * dx + 2.0f * s->b * dx * dy + s->c * dy * dy);
  if (power > 0.0f) {
    *raw_ref = 0.0f;
    return 0;
  }
  *raw_ref = s->o * expf(power);
  return fminf(M->max_alpha, *raw_ref) >= M->alpha_threshold;
}

static int eval_alpha(const oracle_meta* M, const splat_t* s, float px, float py,
                      float* alpha, float* raw, float* dx, float* dy, int* amb) {
  *dx = px - s->mx;
  *dy = py - s->my;
  float e, p;
  splat_exponents(s, *dx, *dy, &e, &p);
  const int vis = e <= 0.0f && p >= s->q;
  if (amb) {
    /* Near either threshold of the base-2 form (p - q and e in log2 units):
     * compare with the reference's form.  The two forms' distances to the
     * threshold differ by the rounding of power (a few ulps of m, the sum of
     * the magnitudes of its terms), of lo and plim (ulps of |log2 thr|) and
     * of exp: far below this margin, so no disagreement lies outside it. */
    const float m = 0.5f * (fabsf(s->a) * *dx * *dx + 2.0f * fabsf(s->b * *dx * *dy) + fabsf(s->c) * *dy * *dy);
    const float near = 0x1p-10f + 0x1p-16f * m;
    if (fabsf(p - s->q) <= near || fabsf(e) <= near) {
      float raw_ref;
      const int vis_ref = ref_form_visible(M, s, *dx, *dy, &raw_ref);
      if (vis_ref != vis)
        *amb |= AMB_ALPHA | AMB_ALPHA_FLIP;
      else if (raw_ref > 0.0f &&
               fabsf(raw_ref - M->alpha_threshold) <= AMB_ALPHA_ULPS * 0x1p-24f * M->alpha_threshold)
        *amb |= AMB_ALPHA;
    }
  }
  if (!vis) return 0;
  *raw = (float)exp2((double)p);
  *alpha = fminf(M->max_alpha, *raw);
  if (amb && fabsf(*raw - M->max_alpha) <= AMB_REL * M->max_alpha) *amb |= AMB_GATE;
  return 1;
}

/* Front-to-back walk of one pixel over the n records of its tile (list
 * order).  force < 0: the reference's stop rule (break after the blend that
 * brings T to the threshold); force >= 0: walk exactly the first `force`
 * records (another implementation's local_stop), flagging AMB_FORCED_BAD when
 * that decision is not one the ambiguity window allows.  wsum: sum over the
 * blends of 1 + alpha/(1-alpha), T's first-order relative rounding error in
 * units of 2^-24. */
typedef struct {
  float T, cr, cg, cb;
  int last, amb;
  double wsum;
} pixel_walk;

static void walk_pixel(const oracle_meta* M, const splat_t* sp, int n, float fx, float fy,
                       int force, pixel_walk* w) {
  const float thr = M->transmittance_threshold;
  float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
  int last = 0, amb = 0, last_blend = -1;
  float errT = 0.0f; /* bound on T's relative deviation from exp2 ulps */
  float win = 0.0f;
  double wsum = 0.0;
  const int lim = (force >= 0 && force < n) ? force : n;
  for (int i = 0; i < lim; ++i) {
    last = i + 1; /* iterated while alive (reference :457) */
    float alpha, raw, dx, dy;
    if (!eval_alpha(M, &sp[i], fx, fy, &alpha, &raw, &dx, &dy, &amb)) continue;
    const float wgt = T * alpha;
    cr += wgt * sp[i].r; cg += wgt * sp[i].g; cb += wgt * sp[i].bl;
    T *= (1.0f - alpha);
    errT += 2.4e-7f * alpha / (1.0f - alpha);
    wsum += 1.0 + (double)alpha / (1.0 - (double)alpha);
    last_blend = i;
    win = (errT + 1e-6f) * thr;
    if (fabsf(T - thr) <= win) amb |= AMB_STOP;
    if (T <= thr) {
      if (force < 0) break;
      if (i + 1 < lim && T < thr - win) amb |= AMB_FORCED_BAD; /* surely stopped here */
    }
  }
  if (force >= 0) {
    if (force > n) amb |= AMB_FORCED_BAD;
    else if (force < n && (last_blend != force - 1 || T > thr + win)) amb |= AMB_FORCED_BAD;
    last = force > n ? n : force;
  }
  w->T = T; w->cr = cr; w->cg = cg; w->cb = cb;
  w->last = last; w->amb = amb; w->wsum = wsum;
}

/* Records of tile t in list order (buffer of at least the tile's length). */
static int tile_records(const splat_t* sp, const int32_t* tile_offsets, const int32_t* binned_ids,
                        int64_t t, splat_t** buf, int* cap) {
  const int start = tile_offsets[t], end = tile_offsets[t + 1];
  const int n = end - start;
  if (n > *cap) {
    free(*buf);
    *cap = n;
    *buf = (splat_t*)malloc(sizeof(splat_t) * (size_t)n);
  }
  for (int i = 0; i < n; ++i) (*buf)[i] = sp[binned_ids[start + i]];
  return n;
}

/* out_rgb [B,H,W,3]; out_T [B,H,W]; out_last [B,H,W] = the reference's
 * local_stop (gsplat_v8_kernels.metal:455-467): 1 + index in the tile list of
 * the splat whose blend brought T to the threshold, or the list length if
 * the pixel never stopped (every splat iterated); tile_stop [T] = max last.
 * force_last (NULL, or [B,H,W] with -1 = decide): forced stops, see
 * walk_pixel.  out_amb [B,H,W]: AMB_* bits. */
void oracle_render_forward(const oracle_meta* M, const float* means2d, const float* conics,
                           const float* colors, const float* opac, const int32_t* perm,
                           const int32_t* tile_offsets, const int32_t* binned_ids,
                           const int32_t* force_last, float* out_rgb, float* out_T,
                           int32_t* out_last, int32_t* tile_stop, uint8_t* out_amb) {
  const int tiles_x = (M->width + 15) / 16;
  const int64_t tpi = tiles_per_image(M), tiles = num_tiles(M);
  splat_t* sp = gather_splats(M, means2d, conics, colors, opac, perm);
#pragma omp parallel
  {
    splat_t* buf = NULL;
    int cap = 0;
#pragma omp for schedule(dynamic, 16)
    for (int64_t t = 0; t < tiles; ++t) {
      const int b = (int)(t / tpi), lt = (int)(t % tpi), ty = lt / tiles_x, tx = lt % tiles_x;
      const int n = tile_records(sp, tile_offsets, binned_ids, t, &buf, &cap);
      int tmax = 0;
      for (int py = 0; py < 16; ++py) {
        const int y = ty * 16 + py;
        if (y >= M->height) continue;
        for (int pxi = 0; pxi < 16; ++pxi) {
          const int x = tx * 16 + pxi;
          if (x >= M->width) continue;
          const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
          pixel_walk w;
          walk_pixel(M, buf, n, (float)x + 0.5f, (float)y + 0.5f,
                     force_last ? force_last[pix] : -1, &w);
          out_rgb[3 * pix] = w.cr + w.T * M->bg[0];
          out_rgb[3 * pix + 1] = w.cg + w.T * M->bg[1];
          out_rgb[3 * pix + 2] = w.cb + w.T * M->bg[2];
          if (out_T) out_T[pix] = w.T;
          if (out_last) out_last[pix] = w.last;
          if (out_amb) out_amb[pix] = (uint8_t)w.amb;
          if (w.last > tmax) tmax = w.last;
        }
      }
      if (tile_stop) tile_stop[t] = tmax;
    }
    free(buf);
  }
  free(sp);
}

/* Gradient entries per splat: g_means2d (2), g_conics (3), g_colors (3),
 * g_opacities (1). */
enum { kEnt = 9, kPart = 4 * kEnt };

/* Gradients in ORIGINAL order (overwritten): g_means2d [BG,2], g_conics
 * [BG,3], g_colors [BG,3], g_opac [BG].  Follows the reference's backward:
 * replay the forward per pixel for T_final and end_i (with force_last as in
 * the forward), then walk the list in reverse:
 *   T_prev = T / max(1 - alpha, eps), g_alpha = T_prev (<g,c> - gT),
 *   g_color = g T_prev alpha, g_raw = g_alpha if raw < max_alpha else 0,
 *   g_power = g_raw raw, g_conic = g_power (-dx^2/2, -dx dy, -dy^2/2),
 *   g_mean = g_power (a dx + b dy, b dx + c dy), g_opacity = g_raw raw / o,
 *   gT <- alpha <g,c> + (1 - alpha) gT.
 * Each contribution is a float32 value as in the reference; per splat they
 * are summed in double, tile by tile in tile order, pixel by pixel in pixel
 * order inside a tile.
 *
 * Optional error-bound outputs, float64 [BG, 9] in the entry order
 * (mean x, mean y, conic a, b, c, colour r, g, b, opacity), each a sum over
 * the splat's contributions:
 *   mag    |c| with every difference replaced by the sum of its operands'
 *          magnitudes (|<g,c> - gT| -> |<g,c>| + |gT|, |a dx + b dy| ->
 *          |a dx| + |b dy|): bounds the effect of relative errors in the
 *          operands without cancellation;
 *   chain  kappa |c|, kappa = 8 + the pixel's wsum (T_final's error) + twice
 *          the wsum of the splats after this one (the divisions that rebuilt
 *          T_prev and the gT recurrence): first-order relative error of the
 *          contribution's T_prev and gT in units of 2^-24;
 *   slack  |c| (gate open) of contributions whose gate decision raw <
 *          max_alpha lies within rounding (the other decision is as valid). */
void oracle_render_backward(const oracle_meta* M, const float* means2d, const float* conics,
                            const float* colors, const float* opac, const int32_t* perm,
                            const int32_t* tile_offsets, const int32_t* binned_ids,
                            const int32_t* force_last, const float* grad_rgb,
                            float* g_means2d, float* g_conics, float* g_colors, float* g_opac,
                            double* mag, double* chain, double* slack) {
  const int tiles_x = (M->width + 15) / 16;
  const int64_t tpi = tiles_per_image(M), tiles = num_tiles(M);
  const int64_t BG = (int64_t)M->batch * M->gpb;
  splat_t* sp = gather_splats(M, means2d, conics, colors, opac, perm);
  /* (1) replay: walked length per tile */
  int32_t* walk = (int32_t*)calloc((size_t)(tiles > 0 ? tiles : 1), sizeof(int32_t));
#pragma omp parallel
  {
    splat_t* buf = NULL;
    int cap = 0;
#pragma omp for schedule(dynamic, 16)
    for (int64_t t = 0; t < tiles; ++t) {
      const int b = (int)(t / tpi), lt = (int)(t % tpi), ty = lt / tiles_x, tx = lt % tiles_x;
      const int n = tile_records(sp, tile_offsets, binned_ids, t, &buf, &cap);
      if (n == 0) continue;
      int tmax = 0;
      for (int py = 0; py < 16; ++py) {
        const int y = ty * 16 + py;
        if (y >= M->height) continue;
        for (int pxi = 0; pxi < 16; ++pxi) {
          const int x = tx * 16 + pxi;
          if (x >= M->width) continue;
          const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
          pixel_walk w;
          walk_pixel(M, buf, n, (float)x + 0.5f, (float)y + 0.5f,
                     force_last ? force_last[pix] : -1, &w);
          if (w.last > tmax) tmax = w.last;
        }
      }
      walk[t] = tmax;
    }
    free(buf);
  }
  int64_t* woff = (int64_t*)malloc(sizeof(int64_t) * (size_t)(tiles + 1));
  woff[0] = 0;
  for (int64_t t = 0; t < tiles; ++t) woff[t + 1] = woff[t] + walk[t];
  /* (2) per (tile, walked record) partial sums: kEnt values, magnitudes,
   * chain-weighted magnitudes and gate slack */
  double* part = (double*)calloc((size_t)(woff[tiles] > 0 ? woff[tiles] : 1) * kPart, sizeof(double));
#pragma omp parallel
  {
    splat_t* buf = NULL;
    int cap = 0;
#pragma omp for schedule(dynamic, 16)
    for (int64_t t = 0; t < tiles; ++t) {
      if (walk[t] == 0) continue;
      const int b = (int)(t / tpi), lt = (int)(t % tpi), ty = lt / tiles_x, tx = lt % tiles_x;
      const int n = tile_records(sp, tile_offsets, binned_ids, t, &buf, &cap);
      double* P = part + woff[t] * kPart;
      for (int py = 0; py < 16; ++py) {
        const int y = ty * 16 + py;
        if (y >= M->height) continue;
        for (int pxi = 0; pxi < 16; ++pxi) {
          const int x = tx * 16 + pxi;
          if (x >= M->width) continue;
          const float fx = (float)x + 0.5f, fy = (float)y + 0.5f;
          const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
          const float gr = grad_rgb[3 * pix], gg = grad_rgb[3 * pix + 1], gb = grad_rgb[3 * pix + 2];
          pixel_walk w;
          walk_pixel(M, buf, n, fx, fy, force_last ? force_last[pix] : -1, &w);
          float T_cur = w.T;
          float gT = gr * M->bg[0] + gg * M->bg[1] + gb * M->bg[2];
          double after = 0.0; /* wsum of the splats after the current one */
          for (int li = w.last - 1; li >= 0; --li) {
            const splat_t* s = &buf[li];
            float alpha, raw, dx, dy;
            int amb = 0;
            if (!eval_alpha(M, s, fx, fy, &alpha, &raw, &dx, &dy, &amb)) continue;
            const float T_prev = T_cur / fmaxf(1.0f - alpha, M->eps);
            const float dot_gc = gr * s->r + gg * s->g + gb * s->bl;
            const float g_alpha = T_prev * (dot_gc - gT);
            const float wgt = T_prev * alpha;
            const int open = raw < M->max_alpha;
            const float g_raw = open ? g_alpha : 0.0f;
            const float g_pow = g_raw * raw;
            const float c[kEnt] = {
                g_pow * (s->a * dx + s->b * dy), g_pow * (s->b * dx + s->c * dy),
                g_pow * (-0.5f) * dx * dx, g_pow * (-1.0f) * dx * dy, g_pow * (-0.5f) * dy * dy,
                gr * wgt, gg * wgt, gb * wgt, g_raw * (raw / fmaxf(s->o, M->eps))};
            const double mA = (double)T_prev * (fabs((double)dot_gc) + fabs((double)gT));
            const double mp = mA * raw;
            const double ddx = dx, ddy = dy;
            const double m[kEnt] = {
                mp * (fabs(s->a * ddx) + fabs(s->b * ddy)), mp * (fabs(s->b * ddx) + fabs(s->c * ddy)),
                mp * 0.5 * ddx * ddx, mp * fabs(ddx * ddy), mp * 0.5 * ddy * ddy,
                fabs((double)gr) * wgt, fabs((double)gg) * wgt, fabs((double)gb) * wgt,
                mA * raw / fmax((double)s->o, (double)M->eps)};
            const double kappa = 8.0 + w.wsum + 2.0 * after;
            double* Q = P + (int64_t)li * kPart;
            for (int e = 0; e < kEnt; ++e) {
              /* colour terms do not pass the gate */
              const double me = (open || (e >= 5 && e < 8)) ? m[e] : 0.0;
              Q[e] += c[e];
              Q[kEnt + e] += me;
              Q[2 * kEnt + e] += kappa * me;
              if ((amb & AMB_GATE) && !(e >= 5 && e < 8)) Q[3 * kEnt + e] += m[e];
            }
            gT = alpha * dot_gc + (1.0f - alpha) * gT;
            T_cur = T_prev;
            after += 1.0 + (double)alpha / (1.0 - (double)alpha);
          }
        }
      }
    }
    free(buf);
  }
  /* (3) per-splat sums in tile order */
  double* acc = (double*)calloc((size_t)(BG > 0 ? BG : 1) * kPart, sizeof(double));
  for (int64_t t = 0; t < tiles; ++t) {
    const int start = tile_offsets[t];
    for (int li = 0; li < walk[t]; ++li) {
      const int64_t o = sp[binned_ids[start + li]].orig;
      const double* Q = part + (woff[t] + li) * kPart;
      double* A = acc + o * kPart;
      for (int e = 0; e < kPart; ++e) A[e] += Q[e];
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < BG; ++o) {
    const double* A = acc + o * kPart;
    g_means2d[2 * o] = (float)A[0];
    g_means2d[2 * o + 1] = (float)A[1];
    for (int k = 0; k < 3; ++k) {
      g_conics[3 * o + k] = (float)A[2 + k];
      g_colors[3 * o + k] = (float)A[5 + k];
    }
    g_opac[o] = (float)A[8];
    for (int e = 0; e < kEnt; ++e) {
      if (mag) mag[o * kEnt + e] = A[kEnt + e];
      if (chain) chain[o * kEnt + e] = A[2 * kEnt + e];
      if (slack) slack[o * kEnt + e] = A[3 * kEnt + e];
    }
  }
  free(acc);
  free(part);
  free(woff);
  free(walk);
  free(sp);
}

/* Reference-order single-thread float32 backward (the accumulation of the
 * reference kernels, one float sum per entry in pixel order): the
 * independent restatement the tests compare oracle_render_backward with. */
void oracle_render_backward_serial(const oracle_meta* M, const float* means2d, const float* conics,
                                   const float* colors, const float* opac, const int32_t* perm,
                                   const int32_t* tile_offsets, const int32_t* binned_ids,
                                   const float* grad_rgb, float* g_means2d, float* g_conics,
                                   float* g_colors, float* g_opac) {
  const int tiles_x = (M->width + 15) / 16, tiles_y = (M->height + 15) / 16;
  const int tpi = tiles_x * tiles_y;
  splat_t* sp = gather_splats(M, means2d, conics, colors, opac, perm);
  for (int t = 0; t < M->batch * tpi; ++t) {
    const int b = t / tpi, lt = t % tpi, ty = lt / tiles_x, tx = lt % tiles_x;
    const int start = tile_offsets[t], end = tile_offsets[t + 1];
    if (end == start) continue;
    for (int py = 0; py < 16; ++py) {
      const int y = ty * 16 + py;
      if (y >= M->height) continue;
      for (int pxi = 0; pxi < 16; ++pxi) {
        const int x = tx * 16 + pxi;
        if (x >= M->width) continue;
        const float fx = (float)x + 0.5f, fy = (float)y + 0.5f;
        const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
        const float gr = grad_rgb[3 * pix], gg = grad_rgb[3 * pix + 1], gb = grad_rgb[3 * pix + 2];
        /* replay */
        float T_final = 1.0f;
        int end_i = end - start;
        for (int i = start; i < end; ++i) {
          const splat_t* s = &sp[binned_ids[i]];
          float alpha, raw, dx, dy;
          if (!eval_alpha(M, s, fx, fy, &alpha, &raw, &dx, &dy, NULL)) continue;
          T_final *= (1.0f - alpha);
          if (T_final <= M->transmittance_threshold) { end_i = i - start + 1; break; }
        }
        float T_cur = T_final;
        float gT = gr * M->bg[0] + gg * M->bg[1] + gb * M->bg[2];
        for (int li = end_i - 1; li >= 0; --li) {
          const splat_t* s = &sp[binned_ids[start + li]];
          float alpha, raw, dx, dy;
          if (!eval_alpha(M, s, fx, fy, &alpha, &raw, &dx, &dy, NULL)) continue;
          const float T_prev = T_cur / fmaxf(1.0f - alpha, M->eps);
          const float dot_gc = gr * s->r + gg * s->g + gb * s->bl;
          const float g_alpha = T_prev * (dot_gc - gT);
          const float wgt = T_prev * alpha;
          const float g_raw = (raw < M->max_alpha) ? g_alpha : 0.0f;
          const float g_pow = g_raw * raw;
          const int64_t o = s->orig;
          g_colors[3 * o] += gr * wgt;
          g_colors[3 * o + 1] += gg * wgt;
          g_colors[3 * o + 2] += gb * wgt;
          g_conics[3 * o] += g_pow * (-0.5f) * dx * dx;
          g_conics[3 * o + 1] += g_pow * (-1.0f) * dx * dy;
          g_conics[3 * o + 2] += g_pow * (-0.5f) * dy * dy;
          g_means2d[2 * o] += g_pow * (s->a * dx + s->b * dy);
          g_means2d[2 * o + 1] += g_pow * (s->b * dx + s->c * dy);
          g_opac[o] += g_raw * (raw / fmaxf(s->o, M->eps));
          gT = alpha * dot_gc + (1.0f - alpha) * gT;
          T_cur = T_prev;
        }
      }
    }
  }
  free(sp);
}

/* Threads the parallel functions use (OMP_NUM_THREADS or the core count). */
int oracle_threads(void) { return omp_get_max_threads(); }

/* Sets the thread count of the parallel functions (results do not depend on
 * it; the tests check that). */
void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
