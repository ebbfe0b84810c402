// composite.hip -- per-tile front-to-back compositor (forward) and its
// reverse-order adjoint (backward).
//
// Work decomposition (gfx950): one 64-lane workgroup (= one wavefront) per
// 16x16 tile.  Slot k = 0..3 of the wave is one 8x8 quadrant of the tile and
// lane l owns pixel (l%8, l/8) of every quadrant, so every splat record is
// read once per wave and reused for four pixels, and no barrier spans more
// than one wavefront.  Splat records of the tile's range are staged 64 at a
// time in LDS (each lane gathers one 48-byte record) and read by all lanes as
// broadcasts.  A quadrant is skipped (wave-uniform branch) when it lies
// outside the splat's bounding box, padded by 1% + 0.01 px so that no pixel
// that could pass the alpha test is ever skipped.
//
// Forward (reference tile_fast_forward_state,
// variants/v8/csrc/metal/gsplat_v8_kernels.metal:400-476):
//   alpha = min(max_alpha, o*exp(power)), visible iff power <= 0 and
//   alpha >= alpha_threshold; C += T*alpha*c; T *= 1-alpha; a pixel stops
//   after the splat that brings T <= transmittance_threshold.  Saves per
//   pixel the final T and last = 1 + index of the last composited splat, and
//   per tile the max of last, so backward needs no forward replay.
// Backward (reference tile_fast_backward_saved, :478-608, and the recurrence
// of docs/v8_critical_theory_notes.md:113-141): walks the tile range in
// reverse from the tile's max(last); T_prev = T/(1-alpha),
//   g_alpha = T_prev (<g,c> - gT), g_color = g T_prev alpha,
//   g_raw = g_alpha if raw < max_alpha, g_power = g_raw raw,
//   g_conic = g_power (-dx^2/2, -dx dy, -dy^2/2),
//   g_mean = g_power (a dx + b dy, b dx + c dy), g_opacity = g_raw exp(power),
//   gT <- gT + alpha (<g,c> - gT).
// Per pixel only the moments g_power*(dx, dy, dx^2, dx*dy, dy^2) are
// accumulated; the conic and mean gradients are formed from their wave sums
// once per splat.  The nine per-splat sums are reduced across the wavefront
// with DPP lane-permute adds (no LDS traffic) and one lane issues nine float
// atomics into the original splat order.
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kLanes = 64;
constexpr int kPix = 4;
constexpr int kBatch = 64;

struct TileCoord {
  int tile, batch, x0, y0;  // tile origin
  int lx, ly;               // this lane's offset inside a quadrant
};

__device__ __forceinline__ TileCoord tile_coord(const RasterParams& P) {
  TileCoord c;
  c.tile = xcd_remap((int)blockIdx.x, P.num_tiles);
  c.batch = c.tile / P.tiles_per_image;
  const int lt = c.tile - c.batch * P.tiles_per_image;
  const int ty = lt / P.tiles_x;
  const int tx = lt - ty * P.tiles_x;
  c.x0 = tx * 16;
  c.y0 = ty * 16;
  c.lx = threadIdx.x & 7;
  c.ly = threadIdx.x >> 3;
  return c;
}

// Pixel of slot (quadrant) k for this lane.
__device__ __forceinline__ int slot_x(const TileCoord& c, int k) {
  return c.x0 + 8 * (k & 1) + c.lx;
}
__device__ __forceinline__ int slot_y(const TileCoord& c, int k) {
  return c.y0 + 8 * (k >> 1) + c.ly;
}

struct Staged {
  float4 s0[kBatch];  // mx, my, A, B
  float4 s1[kBatch];  // C, opacity, r, g
  float4 s2[kBatch];  // blue, orig index bits, -, -
  float4 s3[kBatch];  // xlo, xhi, ylo, yhi
};

// Stages records [first, first+n) of the tile range into LDS with
// A = -a/2, B = -b, C = -c/2 (exact scalings of the conic) and a padded
// bounding box of the pixels where alpha >= alpha_threshold is possible:
// |dx| <= sqrt(tau c / det), |dy| <= sqrt(tau a / det), tau = -2 ln(thr / o).
__device__ __forceinline__ void stage_batch(const RasterParams& P,
                                            const float4* __restrict__ packed,
                                            const int32_t* __restrict__ binned,
                                            int first, int n, Staged& S) {
  const int lane = threadIdx.x;
  if (lane < n) {
    const int gid = binned[first + lane];
    const float4 p0 = packed[3 * gid + 0];
    const float4 p1 = packed[3 * gid + 1];
    const float4 p2 = packed[3 * gid + 2];
    const float a = p0.z, b = p0.w, c = p1.x, o = p1.y;
    const float det = fmaxf(a * c - b * b, 1e-30f);
    const float tau = fmaxf(-2.0f * __logf(P.alpha_thr / o), 0.0f);
    const float hx = __builtin_sqrtf(tau * c / det) * 1.01f + 0.01f;
    const float hy = __builtin_sqrtf(tau * a / det) * 1.01f + 0.01f;
    // No culling when det is not accurate to well under 1% (nearly
    // degenerate conic) or a bound is not finite.
    const bool finite = hx == hx && hy == hy && hx < 3.0e38f &&
                        hy < 3.0e38f && det > 1e-4f * (a * c);
    S.s0[lane] = make_float4(p0.x, p0.y, -0.5f * a, -b);
    S.s1[lane] = make_float4(-0.5f * c, o, p1.z, p1.w);
    S.s2[lane] = p2;
    S.s3[lane] = finite
        ? make_float4(p0.x - hx, p0.x + hx, p0.y - hy, p0.y + hy)
        : make_float4(-3.0e38f, 3.0e38f, -3.0e38f, 3.0e38f);
  }
}

// power = -0.5*(a dx^2 + 2 b dx dy + c dy^2), evaluated as one fixed chain of
// roundings (two explicit FMAs) so that the CPU oracle can reproduce it bit
// for bit; A, B, C as staged above.
__device__ __forceinline__ float splat_power(float A, float B, float C,
                                             float dx, float dy) {
#pragma clang fp contract(off)
  return __builtin_fmaf(C * dy, dy, __builtin_fmaf(B * dx, dy, (A * dx) * dx));
}

// exp(power) as 2^(power * log2(e)) with the float-rounded constant; the
// hardware exp2 is within 1 ulp.
__device__ __forceinline__ float splat_exp(float power) {
#pragma clang fp contract(off)
  return __builtin_amdgcn_exp2f(power * 1.44269502f);
}

// Does quadrant k (pixel centres x0+8(k&1)+0.5 .. +7.5, y0+8(k>>1)+0.5 ..
// +7.5) meet the box b = (xlo, xhi, ylo, yhi)?
__device__ __forceinline__ bool quad_hit(const TileCoord& c, int k,
                                         const float4& b) {
  const float qx = (float)(c.x0 + 8 * (k & 1)) + 0.5f;
  const float qy = (float)(c.y0 + 8 * (k >> 1)) + 0.5f;
  return !(b.y < qx || b.x > qx + 7.0f || b.w < qy || b.z > qy + 7.0f);
}

__global__ __launch_bounds__(kLanes) void render_fwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, float* __restrict__ out_rgb,
    float* __restrict__ out_T, int32_t* __restrict__ out_last,
    int32_t* __restrict__ out_tile_stop) {
  __shared__ Staged S;
  const TileCoord tc = tile_coord(P);
  float px[kPix], py[kPix], T[kPix], cr[kPix], cg[kPix], cb[kPix];
  int last[kPix];
  bool valid[kPix], alive[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int x = slot_x(tc, k), y = slot_y(tc, k);
    valid[k] = (x < P.width) && (y < P.height);
    px[k] = (float)x + 0.5f;
    py[k] = (float)y + 0.5f;
    T[k] = 1.0f;
    cr[k] = cg[k] = cb[k] = 0.0f;
    last[k] = 0;
    alive[k] = valid[k];
  }
  const int start = tile_offsets[tc.tile];
  const int end = tile_offsets[tc.tile + 1];
  for (int base = start; base < end; base += kBatch) {
    const bool any_alive = alive[0] | alive[1] | alive[2] | alive[3];
    if (!__any(any_alive)) break;
    const int n = min(kBatch, end - base);
    __syncthreads();
    stage_batch(P, packed, binned, base, n, S);
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 a0 = S.s0[j];
      const float4 a1 = S.s1[j];
      const float blue = S.s2[j].x;
      const float4 box = S.s3[j];
      const int idx1 = base - start + j + 1;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (!quad_hit(tc, k, box)) continue;  // wave-uniform
        if (alive[k]) {
          const float dx = px[k] - a0.x;
          const float dy = py[k] - a0.y;
          const float power = splat_power(a0.z, a0.w, a1.x, dx, dy);
          if (power <= 0.0f) {
            const float raw = a1.y * splat_exp(power);
            const float alpha = fminf(P.max_alpha, raw);
            if (alpha >= P.alpha_thr) {
              const float w = T[k] * alpha;
              cr[k] += w * a1.z;
              cg[k] += w * a1.w;
              cb[k] += w * blue;
              T[k] *= (1.0f - alpha);
              last[k] = idx1;
              if (T[k] <= P.trans_thr) alive[k] = false;
            }
          }
        }
      }
    }
  }
  int tile_max = 0;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    if (valid[k]) {
      const int64_t pix =
          ((int64_t)tc.batch * P.height + slot_y(tc, k)) * P.width + slot_x(tc, k);
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

// Sum over the 64 lanes (all active), returned as a wave-uniform value:
// quad_perm [1,0,3,2] and [2,3,0,1] reduce quads, row_half_mirror and
// row_mirror reduce 16-lane rows, row_bcast:15 / row_bcast:31 carry row sums
// upward so lane 63 ends with the total.
__device__ __forceinline__ float wave_sum_dpp(float x) {
  x += dpp_src<0xB1>(x);
  x += dpp_src<0x4E>(x);
  x += dpp_src<0x141>(x);
  x += dpp_src<0x140>(x);
  x += dpp_src<0x142, 0xA>(x);
  x += dpp_src<0x143, 0xC>(x);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

__global__ __launch_bounds__(kLanes) void render_bwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, const float* __restrict__ final_T,
    const int32_t* __restrict__ last_in, const int32_t* __restrict__ tile_stop,
    const float* __restrict__ grad_rgb, float* __restrict__ g_means2d,
    float* __restrict__ g_conics, float* __restrict__ g_colors,
    float* __restrict__ g_opac) {
  __shared__ Staged S;
  const TileCoord tc = tile_coord(P);
  const int nstop = tile_stop[tc.tile];
  if (nstop <= 0) return;
  const int start = tile_offsets[tc.tile];
  float px[kPix], py[kPix], Tc[kPix], gr[kPix], gg[kPix], gb[kPix], gT[kPix];
  int lk[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int x = slot_x(tc, k), y = slot_y(tc, k);
    const bool valid = (x < P.width) && (y < P.height);
    px[k] = (float)x + 0.5f;
    py[k] = (float)y + 0.5f;
    if (valid) {
      const int64_t pix = ((int64_t)tc.batch * P.height + y) * P.width + x;
      gr[k] = grad_rgb[3 * pix + 0];
      gg[k] = grad_rgb[3 * pix + 1];
      gb[k] = grad_rgb[3 * pix + 2];
      Tc[k] = final_T[pix];
      lk[k] = last_in[pix];
    } else {
      gr[k] = gg[k] = gb[k] = 0.0f;
      Tc[k] = 1.0f;
      lk[k] = 0;
    }
    gT[k] = gr[k] * P.bg_r + gg[k] * P.bg_g + gb[k] * P.bg_b;
  }
  for (int cend = nstop; cend > 0; cend -= kBatch) {
    const int cstart = max(0, cend - kBatch);
    const int n = cend - cstart;
    __syncthreads();
    stage_batch(P, packed, binned, start + cstart, n, S);
    __syncthreads();
    for (int j = n - 1; j >= 0; --j) {
      const int i = cstart + j;
      const float4 a0 = S.s0[j];
      const float4 a1 = S.s1[j];
      const float2 a2 = make_float2(S.s2[j].x, S.s2[j].y);
      const float4 box = S.s3[j];
      // moments of g_power over this lane's pixels
      float m_x = 0.f, m_y = 0.f, m_xx = 0.f, m_xy = 0.f, m_yy = 0.f;
      float acc_r = 0.f, acc_g = 0.f, acc_bl = 0.f, acc_o = 0.f;
      bool contrib = false;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (!quad_hit(tc, k, box)) continue;  // wave-uniform
        if (i < lk[k]) {
          const float dx = px[k] - a0.x;
          const float dy = py[k] - a0.y;
          const float power = splat_power(a0.z, a0.w, a1.x, dx, dy);
          if (power <= 0.0f) {
            const float e = splat_exp(power);
            const float raw = a1.y * e;
            const float alpha = fminf(P.max_alpha, raw);
            if (alpha >= P.alpha_thr) {
              contrib = true;
              // alpha <= max_alpha < 1, so 1 - alpha > 0
              const float T_prev =
                  Tc[k] * __builtin_amdgcn_rcpf(fmaxf(1.0f - alpha, P.eps));
              const float dot_gc = gr[k] * a1.z + gg[k] * a1.w + gb[k] * a2.x;
              const float diff = dot_gc - gT[k];
              const float wgt = T_prev * alpha;
              acc_r += gr[k] * wgt;
              acc_g += gg[k] * wgt;
              acc_bl += gb[k] * wgt;
              const float g_raw = (raw < P.max_alpha) ? T_prev * diff : 0.0f;
              const float g_pow = g_raw * raw;
              const float hdx = g_pow * dx, hdy = g_pow * dy;
              m_x += hdx;
              m_y += hdy;
              m_xx += hdx * dx;
              m_xy += hdx * dy;
              m_yy += hdy * dy;
              acc_o += g_raw * e;
              gT[k] += alpha * diff;
              Tc[k] = T_prev;
            }
          }
        }
      }
      if (__any(contrib)) {
        m_x = wave_sum_dpp(m_x);
        m_y = wave_sum_dpp(m_y);
        m_xx = wave_sum_dpp(m_xx);
        m_xy = wave_sum_dpp(m_xy);
        m_yy = wave_sum_dpp(m_yy);
        acc_r = wave_sum_dpp(acc_r);
        acc_g = wave_sum_dpp(acc_g);
        acc_bl = wave_sum_dpp(acc_bl);
        acc_o = wave_sum_dpp(acc_o);
        if (threadIdx.x == 0) {
          const int64_t orig = __float_as_int(a2.y);
          // a = -2A, b = -B, c = -2C
          const float a = -2.0f * a0.z, b = -a0.w, c = -2.0f * a1.x;
          unsafeAtomicAdd(&g_means2d[2 * orig + 0], a * m_x + b * m_y);
          unsafeAtomicAdd(&g_means2d[2 * orig + 1], b * m_x + c * m_y);
          unsafeAtomicAdd(&g_conics[3 * orig + 0], -0.5f * m_xx);
          unsafeAtomicAdd(&g_conics[3 * orig + 1], -m_xy);
          unsafeAtomicAdd(&g_conics[3 * orig + 2], -0.5f * m_yy);
          unsafeAtomicAdd(&g_colors[3 * orig + 0], acc_r);
          unsafeAtomicAdd(&g_colors[3 * orig + 1], acc_g);
          unsafeAtomicAdd(&g_colors[3 * orig + 2], acc_bl);
          unsafeAtomicAdd(&g_opac[orig], acc_o);
        }
      }
    }
  }
}

}  // namespace

int launch_render_forward(const RasterParams& P, const float* packed,
                          const int32_t* tile_offsets,
                          const int32_t* binned_ids, float* out_rgb,
                          float* out_T, int32_t* out_last,
                          int32_t* out_tile_stop, hipStream_t stream) {
  if (P.num_tiles == 0) return GSPLAT_OK;
  hipLaunchKernelGGL(render_fwd_kernel, dim3((unsigned)P.num_tiles),
                     dim3(kLanes), 0, stream, P,
                     reinterpret_cast<const float4*>(packed), tile_offsets,
                     binned_ids, out_rgb, out_T, out_last, out_tile_stop);
  return check_launch("render_fwd_kernel");
}

int launch_render_backward(const RasterParams& P, const float* packed,
                           const int32_t* tile_offsets,
                           const int32_t* binned_ids, const float* final_T,
                           const int32_t* last, const int32_t* tile_stop,
                           const float* grad_rgb, float* g_means2d,
                           float* g_conics, float* g_colors, float* g_opac,
                           hipStream_t stream) {
  int rc = launch_zero_grads(g_means2d, g_conics, g_colors, g_opac,
                             P.num_splats, stream);
  if (rc) return rc;
  if (P.num_tiles == 0) return GSPLAT_OK;
  hipLaunchKernelGGL(render_bwd_kernel, dim3((unsigned)P.num_tiles),
                     dim3(kLanes), 0, stream, P,
                     reinterpret_cast<const float4*>(packed), tile_offsets,
                     binned_ids, final_T, last, tile_stop, grad_rgb, g_means2d,
                     g_conics, g_colors, g_opac);
  return check_launch("render_bwd_kernel");
}

}  // namespace gs
