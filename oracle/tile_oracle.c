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
 * last-ulp window are flagged.
 *
 * Pinned by (tests/test_oracle_cpu.py): brute-force completeness/tightness of
 * the predicate in double precision, oracle_logf against libm, the dense
 * Torch reference (oracle/dense_reference.py) on small scenes, and closed
 * forms.
 */
#include <math.h>
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
static const float* g_sort_depths;
static int cmp_depth(const void* pa, const void* pb) {
  const int32_t ia = *(const int32_t*)pa, ib = *(const int32_t*)pb;
  const float a = g_sort_depths[ia], b = g_sort_depths[ib];
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
  for (int32_t b = 0; b < B; ++b) {
    int32_t* p = perm + (int64_t)b * G;
    for (int32_t i = 0; i < G; ++i) p[i] = i;
    g_sort_depths = depths + (int64_t)b * G;
    qsort(p, (size_t)G, sizeof(int32_t), cmp_depth);
  }
}

/* ------------------------------------------------------------- binning */
/* Inputs in original order; perm from oracle_depth_order.  Fills
 * tile_counts[T] and tile_offsets[T+1]; returns N. */
int64_t oracle_bin_count(const oracle_meta* M, const float* means2d, const float* conics,
                         const float* opac, const int32_t* perm, int32_t* tile_counts,
                         int32_t* tile_offsets) {
  const int tiles = M->batch * ((M->width + 15) / 16) * ((M->height + 15) / 16);
  memset(tile_counts, 0, sizeof(int32_t) * (size_t)tiles);
  int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(tiles > 0 ? tiles : 1));
  const int64_t BG = (int64_t)M->batch * M->gpb;
  for (int64_t gid = 0; gid < BG; ++gid) {
    const int b = (int)(gid / M->gpb);
    const int64_t o = (int64_t)b * M->gpb + perm[gid];
    const int n = splat_tiles(M, means2d[2 * o], means2d[2 * o + 1], conics[3 * o],
                              conics[3 * o + 1], conics[3 * o + 2], opac[o], b, tmp);
    for (int k = 0; k < n; ++k) tile_counts[tmp[k]]++;
  }
  free(tmp);
  int64_t run = 0;
  for (int t = 0; t < tiles; ++t) {
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
  const int tiles = M->batch * ((M->width + 15) / 16) * ((M->height + 15) / 16);
  int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)(tiles > 0 ? tiles : 1));
  int32_t* tmp = (int32_t*)malloc(sizeof(int32_t) * (size_t)(tiles > 0 ? tiles : 1));
  memcpy(cursor, tile_offsets, sizeof(int32_t) * (size_t)tiles);
  const int64_t BG = (int64_t)M->batch * M->gpb;
  for (int64_t gid = 0; gid < BG; ++gid) {   /* ascending gid => sorted tiles */
    const int b = (int)(gid / M->gpb);
    const int64_t o = (int64_t)b * M->gpb + perm[gid];
    const int n = splat_tiles(M, means2d[2 * o], means2d[2 * o + 1], conics[3 * o],
                              conics[3 * o + 1], conics[3 * o + 2], opac[o], b, tmp);
    for (int k = 0; k < n; ++k) binned_ids[cursor[tmp[k]]++] = (int32_t)gid;
  }
  free(tmp);
  free(cursor);
}

/* ---------------------------------------------------------- compositing */
typedef struct {
  float mx, my, a, b, c, o, r, g, bl;
  float plim; /* base-2 exponent limit of the alpha test (oracle_plim) */
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

static splat_t load_splat(const oracle_meta* M, const float* means2d, const float* conics,
                          const float* colors, const float* opac, const int32_t* perm,
                          int32_t gid) {
  splat_t s;
  const int b = gid / M->gpb;
  const int64_t o = (int64_t)b * M->gpb + perm[gid];
  s.mx = means2d[2 * o]; s.my = means2d[2 * o + 1];
  s.a = conics[3 * o]; s.b = conics[3 * o + 1]; s.c = conics[3 * o + 2];
  s.r = colors[3 * o]; s.g = colors[3 * o + 1]; s.bl = colors[3 * o + 2];
  s.o = opac[o];
  s.plim = oracle_plim(s.o, M->alpha_threshold, M->max_alpha);
  s.orig = o;
  return s;
}

/* Reference eval_alpha: visible iff power <= 0 and alpha >= threshold, with
 * power = -0.5*(a dx^2 + 2 b dx dy + c dy^2) and alpha = min(max_alpha,
 * o exp(power)).  Evaluated in base 2 by a fixed chain of roundings,
 *   A = (-a/2) L, B = (-b) L, C = (-c/2) L   (L = log2(e) rounded to float)
 *   p = fma(C dy, dy, fma(B dx, dy, (A dx) dx))
 * with the visibility decision p <= 0 and p >= plim (oracle_plim), which the
 * HIP compositor takes bit for bit the same way.  2^p is rounded once from
 * double; the hardware exp2 is within 1 ulp, so later decisions that depend
 * on the value of alpha (early stop on T, the max_alpha gradient gate) can
 * differ in their last-ulp window, reported through the ambiguity flags. */
#define AMB_ALPHA 1 /* unused: the alpha-threshold decision is exact */
#define AMB_STOP 2  /* T within rounding of transmittance_threshold */
#define AMB_GATE 4  /* raw alpha within rounding of max_alpha (gradient gate) */
#define AMB_REL 4e-7f

static float splat_exponent(const splat_t* s, float dx, float dy) {
  const float A = (-0.5f * s->a) * LOG2E_F, B = (-s->b) * LOG2E_F;
  const float C = (-0.5f * s->c) * LOG2E_F;
  return fmaf(C * dy, dy, fmaf(B * dx, dy, (A * dx) * dx));
}

static int eval_alpha(const oracle_meta* M, const splat_t* s, float px, float py,
                      float* alpha, float* raw, float* dx, float* dy, int* amb) {
  *dx = px - s->mx;
  *dy = py - s->my;
  const float p = splat_exponent(s, *dx, *dy);
  if (!(p <= 0.0f && p >= s->plim)) return 0;
  *raw = s->o * (float)exp2((double)p);
  *alpha = fminf(M->max_alpha, *raw);
  if (amb && fabsf(*raw - M->max_alpha) <= AMB_REL * M->max_alpha) *amb |= AMB_GATE;
  return 1;
}

/* out_rgb [B,H,W,3]; out_T [B,H,W]; out_last [B,H,W] = the reference's
 * local_stop (gsplat_v8_kernels.metal:455-467): 1 + index in the tile list of
 * the splat whose blend brought T to the threshold, or the list length if
 * the pixel never stopped (every splat iterated); tile_stop [T] = max last. */
void oracle_render_forward(const oracle_meta* M, const float* means2d, const float* conics,
                           const float* colors, const float* opac, const int32_t* perm,
                           const int32_t* tile_offsets, const int32_t* binned_ids,
                           float* out_rgb, float* out_T, int32_t* out_last,
                           int32_t* tile_stop, uint8_t* out_amb) {
  const int tiles_x = (M->width + 15) / 16, tiles_y = (M->height + 15) / 16;
  const int tpi = tiles_x * tiles_y;
  for (int t = 0; t < M->batch * tpi; ++t) {
    const int b = t / tpi, lt = t % tpi, ty = lt / tiles_x, tx = lt % tiles_x;
    const int start = tile_offsets[t], end = tile_offsets[t + 1];
    int tmax = 0;
    for (int py = 0; py < 16; ++py) {
      const int y = ty * 16 + py;
      if (y >= M->height) continue;
      for (int pxi = 0; pxi < 16; ++pxi) {
        const int x = tx * 16 + pxi;
        if (x >= M->width) continue;
        float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
        int last = 0, amb = 0;
        float errT = 0.0f; /* bound on T's relative deviation from exp2 ulps */
        for (int i = start; i < end; ++i) {
          last = i - start + 1; /* iterated while alive (reference :457) */
          const splat_t s = load_splat(M, means2d, conics, colors, opac, perm, binned_ids[i]);
          float alpha, raw, dx, dy;
          if (!eval_alpha(M, &s, (float)x + 0.5f, (float)y + 0.5f, &alpha, &raw, &dx, &dy, &amb)) continue;
          const float w = T * alpha;
          cr += w * s.r; cg += w * s.g; cb += w * s.bl;
          T *= (1.0f - alpha);
          errT += 2.4e-7f * alpha / (1.0f - alpha);
          if (fabsf(T - M->transmittance_threshold) <= (errT + 1e-6f) * M->transmittance_threshold)
            amb |= AMB_STOP;
          if (T <= M->transmittance_threshold) break;
        }
        const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
        out_rgb[3 * pix] = cr + T * M->bg[0];
        out_rgb[3 * pix + 1] = cg + T * M->bg[1];
        out_rgb[3 * pix + 2] = cb + T * M->bg[2];
        if (out_T) out_T[pix] = T;
        if (out_last) out_last[pix] = last;
        if (out_amb) out_amb[pix] = (uint8_t)amb;
        if (last > tmax) tmax = last;
      }
    }
    if (tile_stop) tile_stop[t] = tmax;
  }
}

/* Gradients (ORIGINAL order, accumulated, caller zeroes): g_means2d [BG,2],
 * g_conics [BG,3], g_colors [BG,3], g_opac [BG].  Follows the reference's
 * backward: replay forward per pixel for T_final and end_i, then walk the
 * list in reverse. */
void oracle_render_backward(const oracle_meta* M, const float* means2d, const float* conics,
                            const float* colors, const float* opac, const int32_t* perm,
                            const int32_t* tile_offsets, const int32_t* binned_ids,
                            const float* grad_rgb, float* g_means2d, float* g_conics,
                            float* g_colors, float* g_opac) {
  const int tiles_x = (M->width + 15) / 16, tiles_y = (M->height + 15) / 16;
  const int tpi = tiles_x * tiles_y;
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
          const splat_t s = load_splat(M, means2d, conics, colors, opac, perm, binned_ids[i]);
          float alpha, raw, dx, dy;
          if (!eval_alpha(M, &s, fx, fy, &alpha, &raw, &dx, &dy, NULL)) continue;
          T_final *= (1.0f - alpha);
          if (T_final <= M->transmittance_threshold) { end_i = i - start + 1; break; }
        }
        float T_cur = T_final;
        float gT = gr * M->bg[0] + gg * M->bg[1] + gb * M->bg[2];
        for (int li = end_i - 1; li >= 0; --li) {
          const splat_t s = load_splat(M, means2d, conics, colors, opac, perm, binned_ids[start + li]);
          float alpha, raw, dx, dy;
          if (!eval_alpha(M, &s, fx, fy, &alpha, &raw, &dx, &dy, NULL)) continue;
          const float T_prev = T_cur / fmaxf(1.0f - alpha, M->eps);
          const float dot_gc = gr * s.r + gg * s.g + gb * s.bl;
          const float g_alpha = T_prev * (dot_gc - gT);
          const float wgt = T_prev * alpha;
          const float g_raw = (raw < M->max_alpha) ? g_alpha : 0.0f;
          const float g_pow = g_raw * raw;
          const int64_t o = s.orig;
          g_colors[3 * o] += gr * wgt;
          g_colors[3 * o + 1] += gg * wgt;
          g_colors[3 * o + 2] += gb * wgt;
          g_conics[3 * o] += g_pow * (-0.5f) * dx * dx;
          g_conics[3 * o + 1] += g_pow * (-1.0f) * dx * dy;
          g_conics[3 * o + 2] += g_pow * (-0.5f) * dy * dy;
          g_means2d[2 * o] += g_pow * (s.a * dx + s.b * dy);
          g_means2d[2 * o + 1] += g_pow * (s.b * dx + s.c * dy);
          g_opac[o] += g_raw * (raw / fmaxf(s.o, M->eps));
          gT = alpha * dot_gc + (1.0f - alpha) * gT;
          T_cur = T_prev;
        }
      }
    }
  }
}

/* Marks (tainted[orig] = 1) every splat whose gradient an ambiguous pixel of
 * `amb` can change: the splats visible at that pixel anywhere in its tile
 * list.  Conservative: a
 * different decision at one splat changes T for the pixel's later splats and
 * the suffix colour seen by its earlier ones, all of which are visible ones. */
void oracle_taint(const oracle_meta* M, const float* means2d, const float* conics,
                  const float* colors, const float* opac, const int32_t* perm,
                  const int32_t* tile_offsets, const int32_t* binned_ids,
                  const uint8_t* amb, uint8_t* tainted) {
  const int tiles_x = (M->width + 15) / 16, tiles_y = (M->height + 15) / 16;
  const int tpi = tiles_x * tiles_y;
  for (int b = 0; b < M->batch; ++b) {
    for (int y = 0; y < M->height; ++y) {
      for (int x = 0; x < M->width; ++x) {
        const int64_t pix = ((int64_t)b * M->height + y) * M->width + x;
        if (!amb[pix]) continue;
        const int t = b * tpi + (y / 16) * tiles_x + (x / 16);
        for (int i = tile_offsets[t]; i < tile_offsets[t + 1]; ++i) {
          const splat_t s = load_splat(M, means2d, conics, colors, opac, perm, binned_ids[i]);
          float alpha, raw, dx, dy;
          if (eval_alpha(M, &s, (float)x + 0.5f, (float)y + 0.5f, &alpha, &raw, &dx, &dy, NULL))
            tainted[s.orig] = 1;
        }
      }
    }
  }
}
