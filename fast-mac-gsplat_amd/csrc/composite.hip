// composite.hip -- per-tile front-to-back compositor (forward) and its
// reverse-order adjoint (backward).
//
// Work decomposition (gfx950): one 64-lane workgroup (= one wavefront) per
// 16x16 tile.  Slot k = 0..3 is the strip of tile rows 4k..4k+3 and lane l
// owns pixel (l%16, 4k + l/16) of every strip, so the four pixels of a lane
// share their x coordinate (and the x-only part of the Gaussian exponent),
// every splat record is read once per wave and reused for four pixels, and no
// barrier spans more than one wavefront.  Splat records of the tile's range
// are staged 64 at a time in LDS (each lane gathers one 48-byte record and
// derives the per-tile constants) and read by all lanes as broadcasts.  A
// strip is skipped (scalar branch on a per-record bit mask) when the
// minimum of the splat's quadratic form over the strip's pixel centres
// exceeds the alpha-support radius by a safety margin, so no pixel that
// could pass the alpha test is ever skipped.
//
// Alpha test (reference eval_alpha, variants/v8/csrc/metal/gsplat_v8_kernels.metal:121-139):
// the exponent is evaluated in base 2, p = log2(e) * power, by the fixed
// rounding chain
//   A = (-a/2)*L, B = (-b)*L, C = (-c/2)*L  (L = log2(e) rounded to float),
//   p = fma(C*dy, dy, fma(B*dx, dy, (A*dx)*dx)),
// and a pixel sees the splat iff p <= 0 and p >= plim, where plim (stored in
// the packed record by binning) is the exponent at which o * 2^p equals the
// alpha threshold.  Both decisions are therefore exact functions of the
// inputs that the CPU oracle reproduces; alpha = min(max_alpha, o * 2^p) with
// the hardware exp2 (within 1 ulp).
//
// Forward (reference tile_fast_forward_state, gsplat_v8_kernels.metal:400-476):
//   C += T*alpha*c; T *= 1-alpha; a pixel stops after the splat that brings
//   T <= transmittance_threshold.  Saves per pixel the final T and last = 1 +
//   index of the last composited splat, and per tile the max of last, so the
//   backward pass needs no forward replay.
// Backward (reference tile_fast_backward_saved, :478-608, and the recurrence
// of docs/v8_critical_theory_notes.md:113-141): walks the tile range in
// reverse from the tile's max(last); T_prev = T/(1-alpha),
//   g_alpha = T_prev (<g,c> - gT), g_color = g T_prev alpha,
//   g_raw = g_alpha if raw < max_alpha, g_power = g_raw raw,
//   g_conic = g_power (-dx^2/2, -dx dy, -dy^2/2),
//   g_mean = g_power (a dx + b dy, b dx + c dy), g_opacity = g_raw exp(power),
//   gT <- gT + alpha (<g,c> - gT).
// Per lane only S0 = sum g_power, S1 = sum g_power dy, S2 = sum g_power dy^2
// (dx is shared by the lane's pixels) and the colour sums are kept (the
// opacity gradient is sum g_raw exp(power) = S0 / o);
// the nine per-splat values are formed from them and reduced across the
// wavefront by a transposed butterfly: two rounds of half-wave register swaps
// (v_permlane32_swap / v_permlane16_swap) fold eight values into two
// registers whose four rows each hold one value, four DPP row steps finish
// them, and lanes 0, 16, 32 and 48 each issue the float atomic for their row
// into the original splat order (the ninth value uses a plain DPP reduction).
#include "gs_internal.h"
#include "gs_predicate.h"

namespace gs {
namespace {

constexpr int kLanes = 64;
constexpr int kPix = 4;
constexpr int kBatch = 64;

struct TileCoord {
  int tile, batch, x0, y0;  // tile origin
  int lx, ly;               // this lane's column and row inside a strip
};

__device__ __forceinline__ TileCoord tile_coord_of(const RasterParams& P,
                                                   int tile) {
  TileCoord c;
  c.tile = tile;
  c.batch = c.tile / P.tiles_per_image;
  const int lt = c.tile - c.batch * P.tiles_per_image;
  const int ty = lt / P.tiles_x;
  const int tx = lt - ty * P.tiles_x;
  c.x0 = tx * 16;
  c.y0 = ty * 16;
  c.lx = threadIdx.x & 15;
  c.ly = threadIdx.x >> 4;
  return c;
}

__device__ __forceinline__ TileCoord tile_coord(const RasterParams& P) {
  return tile_coord_of(P, xcd_remap((int)blockIdx.x, P.num_tiles));
}

__device__ __forceinline__ int slot_y(const TileCoord& c, int k) {
  return c.y0 + 4 * k + c.ly;
}

struct Staged {
  float4 s0[kBatch];  // mx, my, A, B
  float4 s1[kBatch];  // C, opacity, r, g
  float4 s2[kBatch];  // blue, orig index bits, plim, strip mask bits
};

__device__ __forceinline__ float conic_q(float a, float b, float c, float dx,
                                         float dy) {
  return a * dx * dx + 2.0f * b * dx * dy + c * dy * dy;
}

// Bit k set unless strip k of the tile at (x0, y0) certainly holds no pixel
// with p >= plim.  Exact minimum of the conic quadratic q over each strip's
// pixel-centre rectangle (the centre if inside, else the minima along the
// four edges), compared with the support radius tau = -2 ln(thr/o) =
// -2 ln(2) plim enlarged by 2% + 1e-3, which covers the rounding of p's chain
// and of this test as long as det > 1e-3 a c (|b| < (1 - 5e-4) sqrt(ac)).
// Conics outside that range are never culled.
__device__ __forceinline__ uint32_t strip_mask(float mx, float my, float a,
                                               float b, float c, float plim,
                                               int x0, int y0) {
  if (plim > 0.0f) return 0u;  // p <= 0 < plim: invisible everywhere
  const float tau = -1.38629436f * plim;
  const float det = a * c - b * b;
  if (!(a > 0.0f && c > 0.0f && det > 1e-3f * (a * c) && tau < 3.0e38f))
    return 0xFu;
  const float tc = tau * 1.02f + 1e-3f;
  const float dx0 = ((float)x0 + 0.5f) - mx, dx1 = dx0 + 15.0f;
  const float kc = -b / c, ka = -b / a;
  const float ex0 = kc * dx0, ex1 = kc * dx1;  // dy minimising q on x = dx0/dx1
  uint32_t m = 0u;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const float dy0 = ((float)(y0 + 4 * k) + 0.5f) - my, dy1 = dy0 + 3.0f;
    const bool inside = dx0 <= 0.0f && dx1 >= 0.0f && dy0 <= 0.0f && dy1 >= 0.0f;
    float q = conic_q(a, b, c, dx0, fminf(fmaxf(ex0, dy0), dy1));
    q = fminf(q, conic_q(a, b, c, dx1, fminf(fmaxf(ex1, dy0), dy1)));
    q = fminf(q, conic_q(a, b, c, fminf(fmaxf(ka * dy0, dx0), dx1), dy0));
    q = fminf(q, conic_q(a, b, c, fminf(fmaxf(ka * dy1, dx0), dx1), dy1));
    if (inside || q <= tc) m |= 1u << k;
  }
  return m;
}

// Stages records [first, first+n) of the tile range into LDS with the
// base-2 exponent coefficients and the tile's strip mask.
__device__ __forceinline__ void stage_batch(const float4* __restrict__ packed,
                                            const int32_t* __restrict__ binned,
                                            int first, int n,
                                            const TileCoord& tc, Staged& S) {
  const int lane = threadIdx.x;
  if (lane < n) {
    const int gid = binned[first + lane];
    const float4 p0 = packed[3 * gid + 0];
    const float4 p1 = packed[3 * gid + 1];
    const float4 p2 = packed[3 * gid + 2];
    const float a = p0.z, b = p0.w, c = p1.x;
    const uint32_t m = strip_mask(p0.x, p0.y, a, b, c, p2.z, tc.x0, tc.y0);
    float A, B, C;
    {
#pragma clang fp contract(off)
      A = (-0.5f * a) * kLog2e;
      B = (-b) * kLog2e;
      C = (-0.5f * c) * kLog2e;
    }
    S.s0[lane] = make_float4(p0.x, p0.y, A, B);
    S.s1[lane] = make_float4(C, p1.y, p1.z, p1.w);
    S.s2[lane] = make_float4(p2.x, p2.y, p2.z, __uint_as_float(m));
  }
}

// p = fma(C dy, dy, fma(B dx, dy, (A dx) dx)) with the x-only products
// Adxdx = (A dx) dx and Bdx = B dx precomputed; contraction stays off so the
// chain of roundings is exactly the one the CPU oracle evaluates.
__device__ __forceinline__ float splat_exponent(float Adxdx, float Bdx, float C,
                                                float dy) {
#pragma clang fp contract(off)
  return __builtin_fmaf(C * dy, dy, __builtin_fmaf(Bdx, dy, Adxdx));
}

__device__ __forceinline__ void x_terms(float A, float B, float dx,
                                        float& Adxdx, float& Bdx) {
#pragma clang fp contract(off)
  Adxdx = (A * dx) * dx;
  Bdx = B * dx;
}

__device__ __forceinline__ uint32_t uniform_bits(float v) {
  return __builtin_amdgcn_readfirstlane(__float_as_uint(v));
}

// Heavy tiles.  A tile whose range holds more than kHeavyCount pairs gets
// ceil(count / kSegSplats) segment slots.  For each segment k the forward
// records per pixel seg[k] = (colour composited by the segment's splats,
// transmittance at the segment's end); its colour accumulators restart at
// every segment boundary, the completed segments' colour being summed in the
// output pixel.  With those records the backward of segment k needs nothing
// from the later segments' walks: the gT
// of the reverse recurrence at the segment's end is
//   gT_k = (<g, sum_{j>k} colour_j> + <g, bg> T_final) / T_end_k,
// the closed form of gT <- alpha <g,c> + (1 - alpha) gT over the later
// splats.  Segments of a tile whose stop exceeds one segment are then walked
// in parallel, each by its own wavefront, in the same launch as the other
// tiles.
constexpr int kSegSplats = 128;   // multiple of kBatch
constexpr int kHeavyCount = 128;  // >= kSegSplats

struct HeavyState {    // all null: no heavy-tile handling
  int32_t* counter;    // segment slots handed out (zeroed before the forward)
  int32_t* tile_slot;  // [T] first slot of a heavy tile, -1 otherwise
  int32_t* slot_tile;  // [max_slots] tile of each slot
  float4* seg;         // [max_slots][256] (r, g, b, T at the segment's end)
  int max_slots;
};

// Pixel index inside the tile used by the per-pixel heavy-tile buffers.
__device__ __forceinline__ int tile_pixel(int k) {
  return 64 * k + (int)threadIdx.x;
}

// Output pixel of this lane's first strip.  Computed where it is used, from
// an opaque copy of the lane id, so that the compiler does not keep four
// 64-bit pixel addresses live across the compositing loop for the rare
// segment boundaries.
__device__ __forceinline__ float* heavy_out(const RasterParams& P,
                                            const TileCoord& tc,
                                            float* out_rgb) {
  int lane = (int)threadIdx.x;
  asm volatile("" : "+v"(lane));
  const int y = tc.y0 + (lane >> 4);
  const int x = tc.x0 + (lane & 15);
  return out_rgb + 3 * (((int64_t)tc.batch * P.height + y) * P.width + x);
}

__global__ __launch_bounds__(kLanes) void render_fwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, float* __restrict__ out_rgb,
    float* __restrict__ out_T, int32_t* __restrict__ out_last,
    int32_t* __restrict__ out_tile_stop, HeavyState H) {
  __shared__ Staged S;
  const TileCoord tc = tile_coord(P);
  const int x = tc.x0 + tc.lx;
  const float px = (float)x + 0.5f;
  // A pixel is alive while T > transmittance_threshold (< 1, checked on the
  // host); pixels outside the image start at T = 0 and are never written.
  const float t_thr = P.trans_thr;
  const float max_alpha = fminf(P.max_alpha, 1.0f);
  float py[kPix], T[kPix], cr[kPix], cg[kPix], cb[kPix];
  int last[kPix];
  bool valid[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int y = slot_y(tc, k);
    valid[k] = (x < P.width) && (y < P.height);
    py[k] = (float)y + 0.5f;
    T[k] = valid[k] ? 1.0f : 0.0f;
    cr[k] = cg[k] = cb[k] = 0.0f;
    last[k] = 0;
  }
  const int start = tile_offsets[tc.tile];
  const int end = tile_offsets[tc.tile + 1];
  // Heavy tiles sum their colour per segment whether or not the segments are
  // recorded, so the eval and training forwards give identical images.
  const bool heavy = end - start > kHeavyCount;
  int slot = -1;
  if (H.seg != nullptr) {
    if (heavy) {
      const int nseg = (end - start + kSegSplats - 1) / kSegSplats;
      if (threadIdx.x == 0) {
        slot = atomicAdd(H.counter, nseg);
        if (slot + nseg > H.max_slots) slot = -1;  // out of slots: plain tile
      }
      slot = __shfl(slot, 0, 64);
      if (slot >= 0)
        for (int k = threadIdx.x; k < nseg; k += kLanes) H.slot_tile[slot + k] = tc.tile;
    }
    if (threadIdx.x == 0) H.tile_slot[tc.tile] = slot;
  }
  int seg_cur = 0;  // segment of the batch being composited
  for (int base = start; base < end; base += kBatch) {
    const bool any_alive = (T[0] > t_thr) | (T[1] > t_thr) | (T[2] > t_thr) |
                           (T[3] > t_thr);
    if (!__any(any_alive)) break;
    if (heavy && base > start && (base - start) % kSegSplats == 0) {
      // Segment boundary: record the segment and fold its colour into the
      // output pixel, which holds the sum of the completed segments (each
      // lane reads back only what it wrote itself).
      float4* sp = H.seg + (int64_t)(slot + seg_cur) * 256;
      float* o0 = heavy_out(P, tc, out_rgb);
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (slot >= 0) sp[tile_pixel(k)] = make_float4(cr[k], cg[k], cb[k], T[k]);
        if (valid[k]) {
          float* o = o0 + (int64_t)12 * k * P.width;
          if (seg_cur > 0) {
            cr[k] += o[0];
            cg[k] += o[1];
            cb[k] += o[2];
          }
          o[0] = cr[k];
          o[1] = cg[k];
          o[2] = cb[k];
        }
        cr[k] = cg[k] = cb[k] = 0.0f;
      }
      ++seg_cur;
    }
    const int n = min(kBatch, end - base);
    __syncthreads();
    stage_batch(packed, binned, base, n, tc, S);
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 a2 = S.s2[j];
      const uint32_t mask = uniform_bits(a2.w);
      if (mask == 0u) continue;
      const float4 a0 = S.s0[j];
      const float4 a1 = S.s1[j];
      const float plim = a2.z;
      float Adxdx, Bdx;
      x_terms(a0.z, a0.w, px - a0.x, Adxdx, Bdx);
      const int idx1 = base - start + j + 1;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (!((mask >> k) & 1u)) continue;  // scalar branch
        if (T[k] > t_thr) {
          const float p = splat_exponent(Adxdx, Bdx, a1.x, py[k] - a0.y);
          if (p <= 0.0f && p >= plim) {
            const float alpha =
                fminf(max_alpha, a1.y * __builtin_amdgcn_exp2f(p));
            const float w = T[k] * alpha;
            cr[k] += w * a1.z;
            cg[k] += w * a1.w;
            cb[k] += w * a2.x;
            T[k] *= (1.0f - alpha);
            last[k] = idx1;
          }
        }
      }
    }
  }
  if (heavy) {
    // the segment composited last; later segments hold no pixel's last
    float4* sp = H.seg + (int64_t)(slot + seg_cur) * 256;
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
      if (slot >= 0) sp[tile_pixel(k)] = make_float4(cr[k], cg[k], cb[k], T[k]);
      if (valid[k] && seg_cur > 0) {
        const float* o = heavy_out(P, tc, out_rgb) + (int64_t)12 * k * P.width;
        cr[k] += o[0];
        cg[k] += o[1];
        cb[k] += o[2];
      }
    }
  }
  int tile_max = 0;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    if (valid[k]) {
      const int64_t pix =
          ((int64_t)tc.batch * P.height + slot_y(tc, k)) * P.width + x;
      out_rgb[3 * pix + 0] = cr[k] + T[k] * P.bg_r;
      out_rgb[3 * pix + 1] = cg[k] + T[k] * P.bg_g;
      out_rgb[3 * pix + 2] = cb[k] + T[k] * P.bg_b;
      if (out_T) {
        out_T[pix] = T[k];
        out_last[pix] = last[k];
      }
      tile_max = max(tile_max, last[k]);
    }
  }
  if (out_tile_stop) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
      tile_max = max(tile_max, __shfl_xor(tile_max, off, 64));
    if (threadIdx.x == 0) out_tile_stop[tc.tile] = tile_max;
  }
}

// One DPP lane-permute feeding an add: returns the value of `x` from the
// source lane selected by CTRL for lanes of the rows in ROW_MASK, 0 for the
// other rows.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_src(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

// Sum over each 16-lane row, left in every lane of the row: quad_perm
// [1,0,3,2] and [2,3,0,1] reduce quads, row_half_mirror and row_mirror
// combine them.
__device__ __forceinline__ float row_sum_dpp(float x) {
  x += dpp_src<0xB1>(x);
  x += dpp_src<0x4E>(x);
  x += dpp_src<0x141>(x);
  x += dpp_src<0x140>(x);
  return x;
}

// Sum over the 64 lanes, left in every lane of row 3 (lanes 48..63):
// row sums, then row_bcast:15 and row_bcast:31 carry them upward.
__device__ __forceinline__ float wave_sum_row3(float x) {
  x = row_sum_dpp(x);
  x += dpp_src<0x142, 0xA>(x);
  x += dpp_src<0x143, 0xC>(x);
  return x;
}

// Sums of four values over the 64 lanes: returns a register whose row r
// (lanes 16r..16r+15) holds in every lane the total of v[order[r]] with
// order = {0, 2, 1, 3}.  v_permlane32_swap exchanges the upper half of its
// first operand with the lower half of its second, v_permlane16_swap the odd
// rows of the first with the even rows of the second.
__device__ __forceinline__ float wave_sum4(float v0, float v1, float v2,
                                           float v3) {
  const auto s01 = __builtin_amdgcn_permlane32_swap(
      __float_as_uint(v0), __float_as_uint(v1), false, false);
  const auto s23 = __builtin_amdgcn_permlane32_swap(
      __float_as_uint(v2), __float_as_uint(v3), false, false);
  // rows of h01: v0(rows 0+2), v0(1+3), v1(0+2), v1(1+3); h23 likewise
  const float h01 = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);
  const float h23 = __uint_as_float(s23[0]) + __uint_as_float(s23[1]);
  const auto s = __builtin_amdgcn_permlane16_swap(
      __float_as_uint(h01), __float_as_uint(h23), false, false);
  return row_sum_dpp(__uint_as_float(s[0]) + __uint_as_float(s[1]));
}

// Where lanes 0, 16, 32 and 48 (the row heads) send their reduced values.
// Register 1 rows hold {V_mx, V_ca, V_my, V_cb}, register 2 rows
// {V_cc, V_g, V_r, V_b}, and row 3 of register 3 holds S0 (see the backward
// kernel for the values).  A row's destination is base + orig * stride floats.
struct AtomicRole {
  float* base1;
  float* base2;
  bool stride3;  // register 1 target has 3 floats per splat (else 2)
  float scale1, scale2;
};

__device__ __forceinline__ AtomicRole atomic_role(float* g_means2d,
                                                  float* g_conics,
                                                  float* g_colors) {
  // g_mean = -(2/L) V_m since a = -2A/L, b = -B/L, c = -2C/L.
  constexpr float kMeanScale = -2.0f / kLog2e;
  AtomicRole r;
  switch (threadIdx.x >> 4) {
    case 0:
      r.base1 = g_means2d + 0; r.stride3 = false; r.scale1 = kMeanScale;
      r.base2 = g_conics + 2; r.scale2 = -0.5f;
      break;
    case 1:
      r.base1 = g_conics + 0; r.stride3 = true; r.scale1 = -0.5f;
      r.base2 = g_colors + 1; r.scale2 = 1.0f;
      break;
    case 2:
      r.base1 = g_means2d + 1; r.stride3 = false; r.scale1 = kMeanScale;
      r.base2 = g_colors + 0; r.scale2 = 1.0f;
      break;
    default:
      r.base1 = g_conics + 1; r.stride3 = true; r.scale1 = -1.0f;
      r.base2 = g_colors + 2; r.scale2 = 1.0f;
      break;
  }
  return r;
}

// Per-pixel state of the backward walk (4 pixels per lane).
struct BwdPixels {
  float px;
  float py[kPix], Tc[kPix], gr[kPix], gg[kPix], gb[kPix], gT[kPix];
  int lk[kPix];
};

// Loads grad and saved state; T and gT start at final_T and the background
// term.  Pixels outside the image get lk = 0 (never processed).
__device__ __forceinline__ void load_bwd_pixels(
    const RasterParams& P, const TileCoord& tc,
    const float* __restrict__ final_T, const int32_t* __restrict__ last_in,
    const float* __restrict__ grad_rgb, BwdPixels& Q) {
  const int x = tc.x0 + tc.lx;
  Q.px = (float)x + 0.5f;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int y = slot_y(tc, k);
    const bool valid = (x < P.width) && (y < P.height);
    Q.py[k] = (float)y + 0.5f;
    if (valid) {
      const int64_t pix = ((int64_t)tc.batch * P.height + y) * P.width + x;
      Q.gr[k] = grad_rgb[3 * pix + 0];
      Q.gg[k] = grad_rgb[3 * pix + 1];
      Q.gb[k] = grad_rgb[3 * pix + 2];
      Q.Tc[k] = final_T[pix];
      Q.lk[k] = last_in[pix];
    } else {
      Q.gr[k] = Q.gg[k] = Q.gb[k] = 0.0f;
      Q.Tc[k] = 1.0f;
      Q.lk[k] = 0;
    }
    Q.gT[k] = Q.gr[k] * P.bg_r + Q.gg[k] * P.bg_g + Q.gb[k] * P.bg_b;
  }
}

// Reverse walk over the tile-range indices [lo, hi): gradients of every
// splat, reduced across the wavefront and added atomically in original order.
__device__ __forceinline__ void bwd_walk(
    const RasterParams& P, const float4* __restrict__ packed,
    const int32_t* __restrict__ binned, int start, int lo, int hi,
    const TileCoord& tc, Staged& S, BwdPixels& Q, float* __restrict__ g_means2d,
    float* __restrict__ g_conics, float* __restrict__ g_colors,
    float* __restrict__ g_opac) {
  const AtomicRole role = atomic_role(g_means2d, g_conics, g_colors);
  const bool row_head = (threadIdx.x & 15) == 0;
  const float max_alpha = fminf(P.max_alpha, 1.0f);
  // Per-lane partial sums of the current splat; zero between splats.
  float S0 = 0.f, S1 = 0.f, S2 = 0.f;
  float acc_r = 0.f, acc_g = 0.f, acc_b = 0.f;
  for (int cend = hi; cend > lo; cend -= kBatch) {
    const int cstart = max(lo, cend - kBatch);
    const int n = cend - cstart;
    __syncthreads();
    stage_batch(packed, binned, start + cstart, n, tc, S);
    __syncthreads();
    for (int j = n - 1; j >= 0; --j) {
      const float4 a2 = S.s2[j];
      const uint32_t mask = uniform_bits(a2.w);
      if (mask == 0u) continue;
      const int i = cstart + j;
      const float4 a0 = S.s0[j];
      const float4 a1 = S.s1[j];
      const float dx = Q.px - a0.x;
      float Adxdx, Bdx;
      x_terms(a0.z, a0.w, dx, Adxdx, Bdx);
      bool contrib = false;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (!((mask >> k) & 1u)) continue;  // scalar branch
        if (i < Q.lk[k]) {
          const float dy = Q.py[k] - a0.y;
          const float p = splat_exponent(Adxdx, Bdx, a1.x, dy);
          if (p <= 0.0f && p >= a2.z) {
            contrib = true;
            const float e = __builtin_amdgcn_exp2f(p);
            const float raw = a1.y * e;
            const bool open = raw < max_alpha;  // gradient gate
            const float alpha = open ? raw : max_alpha;
            // 1 - alpha >= 1 - max_alpha >= eps (checked on the host), so the
            // reference's max(1 - alpha, eps) is 1 - alpha.
            const float T_prev =
                Q.Tc[k] * __builtin_amdgcn_rcpf(1.0f - alpha);
            const float dot_gc =
                Q.gr[k] * a1.z + Q.gg[k] * a1.w + Q.gb[k] * a2.x;
            const float diff = dot_gc - Q.gT[k];
            const float wgt = T_prev * alpha;
            acc_r += Q.gr[k] * wgt;
            acc_g += Q.gg[k] * wgt;
            acc_b += Q.gb[k] * wgt;
            const float g_pow = open ? (T_prev * diff) * raw : 0.0f;
            const float hdy = g_pow * dy;
            S0 += g_pow;
            S1 += hdy;
            S2 += hdy * dy;
            Q.gT[k] += alpha * diff;
            Q.Tc[k] = T_prev;
          }
        }
      }
      if (__any(contrib)) {
        // Per-lane parts of the splat's gradients (a, b, c = -2A/L, -B/L,
        // -2C/L): g_mean = -(2/L) (V_mx, V_my), g_conic = (-V_ca/2, -V_cb,
        // -V_cc/2) with V_cc = S2, and g_opacity = sum g_raw exp(power) =
        // (sum g_power) / o = S0 / o.
        const float X = dx * S0;             // sum g_power dx
        const float hB = 0.5f * a0.w;
        const float V_mx = a0.z * X + hB * S1;
        const float V_my = hB * X + a1.x * S1;
        const float V_ca = dx * X;           // sum g_power dx^2
        const float V_cb = dx * S1;          // sum g_power dx dy
        const float r3 = wave_sum_row3(S0);
        const float r1 = wave_sum4(V_mx, V_my, V_ca, V_cb);
        const float r2 = wave_sum4(S2, acc_r, acc_g, acc_b);
        S0 = S1 = S2 = 0.f;
        acc_r = acc_g = acc_b = 0.f;
        if (row_head) {
          const uint32_t orig = uniform_bits(a2.y);
          const uint64_t off2 = (uint64_t)orig * 8u;   // bytes, 2 floats
          const uint64_t off3 = (uint64_t)orig * 12u;  // bytes, 3 floats
          float* p1 = reinterpret_cast<float*>(
              reinterpret_cast<char*>(role.base1) + (role.stride3 ? off3 : off2));
          float* p2 = reinterpret_cast<float*>(
              reinterpret_cast<char*>(role.base2) + off3);
          unsafeAtomicAdd(p1, r1 * role.scale1);
          unsafeAtomicAdd(p2, r2 * role.scale2);
          if (threadIdx.x == 48)
            unsafeAtomicAdd(g_opac + orig, r3 * __builtin_amdgcn_rcpf(a1.y));
        }
      }
    }
  }
}

__device__ __forceinline__ bool heavy_backward(const HeavyState& H, int tile,
                                               int nstop) {
  return H.tile_slot != nullptr && H.tile_slot[tile] >= 0 && nstop > kSegSplats;
}

// Decodes segment slot m: tile, segment index k, segment count and the range
// [lo, hi) of tile indices; false if the slot has no backward work.
__device__ __forceinline__ bool seg_item(const RasterParams& P,
                                         const HeavyState& H,
                                         const int32_t* __restrict__ tile_stop,
                                         int m, int& tile, int& slot0, int& k,
                                         int& nseg, int& lo, int& hi) {
  if (H.counter == nullptr || m >= *H.counter || m >= H.max_slots) return false;
  tile = H.slot_tile[m];
  // Only slots handed to a recorded tile are meaningful: check the tile id
  // and that m lies inside that tile's own slot range.
  if (tile < 0 || tile >= P.num_tiles) return false;
  slot0 = H.tile_slot[tile];
  const int nstop = tile_stop[tile];
  if (slot0 < 0 || m < slot0 || nstop <= kSegSplats) return false;
  k = m - slot0;
  nseg = (nstop + kSegSplats - 1) / kSegSplats;
  if (k >= nseg || slot0 > H.max_slots - nseg) return false;
  lo = k * kSegSplats;
  hi = min(lo + kSegSplats, nstop);
  return true;
}

// Work items: blocks [0, seg_blocks) are heavy-tile segment slots (the
// longest walks, dispatched first), the rest are tiles (heavy tiles among
// them return at once).
__global__ __launch_bounds__(kLanes) void render_bwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, const float* __restrict__ final_T,
    const int32_t* __restrict__ last_in, const int32_t* __restrict__ tile_stop,
    const float* __restrict__ grad_rgb, float* __restrict__ g_means2d,
    float* __restrict__ g_conics, float* __restrict__ g_colors,
    float* __restrict__ g_opac, HeavyState H, int seg_blocks) {
  __shared__ Staged S;
  int tile, slot0 = 0, kseg = 0, nseg = 1, lo = 0, hi;
  const int bid = (int)blockIdx.x;
  if (bid < seg_blocks) {
    if (!seg_item(P, H, tile_stop, bid, tile, slot0, kseg, nseg, lo, hi))
      return;
  } else {
    // seg_blocks is a multiple of 8, so the XCD-aware mapping is preserved
    tile = xcd_remap(bid - seg_blocks, P.num_tiles);
    hi = tile_stop[tile];
    if (hi <= 0) return;
    if (heavy_backward(H, tile, hi)) return;  // walked as segments
  }
  const TileCoord tc = tile_coord_of(P, tile);
  BwdPixels Q;
  load_bwd_pixels(P, tc, final_T, last_in, grad_rgb, Q);
  if (kseg < nseg - 1) {
    // Pixels composited past this segment: T and gT at its end from the
    // forward's segment records (Q.gT holds <g, bg>, Q.Tc holds T_final).
    const float4* rec = H.seg + (int64_t)slot0 * 256;
    float cr[kPix], cg[kPix], cb[kPix];
#pragma unroll
    for (int k = 0; k < kPix; ++k) cr[k] = cg[k] = cb[k] = 0.0f;
    for (int j = kseg + 1; j < nseg; ++j) {
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        const float4 v = rec[j * 256 + tile_pixel(k)];
        cr[k] += v.x;
        cg[k] += v.y;
        cb[k] += v.z;
      }
    }
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
      if (Q.lk[k] > hi) {
        const float Te = rec[kseg * 256 + tile_pixel(k)].w;  // > 0: alive
        const float num = Q.gr[k] * cr[k] + Q.gg[k] * cg[k] +
                          Q.gb[k] * cb[k] + Q.gT[k] * Q.Tc[k];
        Q.gT[k] = num / Te;
        Q.Tc[k] = Te;
      }
    }
  }
  bwd_walk(P, packed, binned, tile_offsets[tile], lo, hi, tc, S, Q, g_means2d,
           g_conics, g_colors, g_opac);
}

size_t heavy_max_slots(const RasterParams& P, int64_t n_pairs) {
  // A heavy tile (> kHeavyCount pairs) with c pairs takes ceil(c / kSegSplats)
  // < c / kSegSplats + 1 slots, and there are at most
  // min(T, n_pairs / kHeavyCount) heavy tiles.
  const int64_t tiles = std::min<int64_t>(P.num_tiles, n_pairs / kHeavyCount);
  return (size_t)(n_pairs / kSegSplats + tiles + 1);
}

}  // namespace

size_t render_workspace_bytes(const RasterParams& P, int64_t n_pairs) {
  const size_t slots = heavy_max_slots(P, n_pairs);
  return 256 + align_up((size_t)P.num_tiles * 4, 256) + align_up(slots * 4, 256) +
         align_up(slots * 256 * sizeof(float4), 256);
}

namespace {
HeavyState heavy_state(const RasterParams& P, int64_t n_pairs, void* ws) {
  HeavyState H{};
  if (ws == nullptr) return H;
  const size_t slots = heavy_max_slots(P, n_pairs);
  char* p = static_cast<char*>(ws);
  H.counter = reinterpret_cast<int32_t*>(p);
  p += 256;
  H.tile_slot = reinterpret_cast<int32_t*>(p);
  p += align_up((size_t)P.num_tiles * 4, 256);
  H.slot_tile = reinterpret_cast<int32_t*>(p);
  p += align_up(slots * 4, 256);
  H.seg = reinterpret_cast<float4*>(p);
  H.max_slots = (int)slots;
  return H;
}
}  // namespace

int launch_render_forward(const RasterParams& P, const float* packed,
                          const int32_t* tile_offsets,
                          const int32_t* binned_ids, float* out_rgb,
                          float* out_T, int32_t* out_last,
                          int32_t* out_tile_stop, int64_t n_pairs,
                          void* workspace, hipStream_t stream) {
  if (P.num_tiles == 0) return GSPLAT_OK;
  const HeavyState H = heavy_state(P, n_pairs, workspace);
  if (H.counter != nullptr) {
    const int rc = launch_fill_i32(H.counter, 0, 1, stream);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(render_fwd_kernel, dim3((unsigned)P.num_tiles),
                     dim3(kLanes), 0, stream, P,
                     reinterpret_cast<const float4*>(packed), tile_offsets,
                     binned_ids, out_rgb, out_T, out_last, out_tile_stop, H);
  return check_launch("render_fwd_kernel");
}

int launch_render_backward(const RasterParams& P, const float* packed,
                           const int32_t* tile_offsets,
                           const int32_t* binned_ids, const float* final_T,
                           const int32_t* last, const int32_t* tile_stop,
                           const float* grad_rgb, float* g_means2d,
                           float* g_conics, float* g_colors, float* g_opac,
                           int64_t n_pairs, void* workspace,
                           hipStream_t stream) {
  int rc = launch_zero_grads(g_means2d, g_conics, g_colors, g_opac,
                             P.num_splats, stream);
  if (rc) return rc;
  if (P.num_tiles == 0) return GSPLAT_OK;
  const HeavyState H = heavy_state(P, n_pairs, workspace);
  const float4* pk = reinterpret_cast<const float4*>(packed);
  const int seg_blocks = H.counter ? (H.max_slots + 7) & ~7 : 0;
  hipLaunchKernelGGL(render_bwd_kernel,
                     dim3((unsigned)(seg_blocks + P.num_tiles)), dim3(kLanes),
                     0, stream, P, pk, tile_offsets, binned_ids, final_T, last,
                     tile_stop, grad_rgb, g_means2d, g_conics, g_colors,
                     g_opac, H, seg_blocks);
  return check_launch("render_bwd_kernel");
}

}  // namespace gs
