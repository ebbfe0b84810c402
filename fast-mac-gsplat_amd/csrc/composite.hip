// composite.hip -- per-tile front-to-back compositor (forward) and its
// reverse-order adjoint (backward).
//
// Work decomposition (gfx950): one 64-lane workgroup (= one wavefront) per
// 16x16 tile.  Lane l owns the four pixels (x0 + l%16, y0 + l/16 + 4k),
// k = 0..3, so every splat record is read once per wave and reused for four
// pixels, and no workgroup barrier spans more than one wavefront.  Splat
// records of the tile's range are staged 64 at a time in LDS (each lane
// gathers one 48-byte record) and then read by all lanes as broadcasts.
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
//   gT <- alpha <g,c> + (1-alpha) gT.
// The nine per-splat partials are summed across the wavefront with lane
// shuffles and one lane issues nine float atomics into the original order.
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kLanes = 64;
constexpr int kPix = 4;
constexpr int kBatch = 64;

struct TileCoord {
  int tile, batch, x, ybase;
};

__device__ __forceinline__ TileCoord tile_coord(const RasterParams& P) {
  TileCoord c;
  c.tile = xcd_remap((int)blockIdx.x, P.num_tiles);
  c.batch = c.tile / P.tiles_per_image;
  const int lt = c.tile - c.batch * P.tiles_per_image;
  const int ty = lt / P.tiles_x;
  const int tx = lt - ty * P.tiles_x;
  const int lane = threadIdx.x;
  c.x = tx * 16 + (lane & 15);
  c.ybase = ty * 16 + (lane >> 4);
  return c;
}

// Stages records [first, first+n) of the tile range into LDS as
//   s0 = (mx, my, A, B), s1 = (C, opacity, r, g), s2 = (blue, orig, 0, 0)
// with A = -a/2, B = -b, C = -c/2 (exact scalings of the conic).
__device__ __forceinline__ void stage_batch(const float4* __restrict__ packed,
                                            const int32_t* __restrict__ binned,
                                            int first, int n, float4* s0,
                                            float4* s1, float4* s2) {
  const int lane = threadIdx.x;
  if (lane < n) {
    const int gid = binned[first + lane];
    const float4 p0 = packed[3 * gid + 0];
    const float4 p1 = packed[3 * gid + 1];
    const float4 p2 = packed[3 * gid + 2];
    s0[lane] = make_float4(p0.x, p0.y, -0.5f * p0.z, -p0.w);
    s1[lane] = make_float4(-0.5f * p1.x, p1.y, p1.z, p1.w);
    s2[lane] = p2;
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

__global__ __launch_bounds__(kLanes) void render_fwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, float* __restrict__ out_rgb,
    float* __restrict__ out_T, int32_t* __restrict__ out_last,
    int32_t* __restrict__ out_tile_stop) {
  __shared__ float4 s0[kBatch], s1[kBatch], s2[kBatch];
  const TileCoord tc = tile_coord(P);
  const float px = (float)tc.x + 0.5f;
  float py[kPix], T[kPix], cr[kPix], cg[kPix], cb[kPix];
  int last[kPix];
  bool valid[kPix], alive[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int y = tc.ybase + 4 * k;
    valid[k] = (tc.x < P.width) && (y < P.height);
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
    stage_batch(packed, binned, base, n, s0, s1, s2);
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      const float4 a0 = s0[j];   // mx, my, A, B
      const float4 a1 = s1[j];   // C, opacity, r, g
      const float cbl = s2[j].x; // blue
      const float dx = px - a0.x;
      const int idx1 = base - start + j + 1;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (alive[k]) {
          const float dy = py[k] - a0.y;
          const float power = splat_power(a0.z, a0.w, a1.x, dx, dy);
          if (power <= 0.0f) {
            const float raw = a1.y * splat_exp(power);
            const float alpha = fminf(P.max_alpha, raw);
            if (alpha >= P.alpha_thr) {
              const float w = T[k] * alpha;
              cr[k] += w * a1.z;
              cg[k] += w * a1.w;
              cb[k] += w * cbl;
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
          ((int64_t)tc.batch * P.height + (tc.ybase + 4 * k)) * P.width + tc.x;
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ __launch_bounds__(kLanes) void render_bwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, const float* __restrict__ final_T,
    const int32_t* __restrict__ last_in, const int32_t* __restrict__ tile_stop,
    const float* __restrict__ grad_rgb, float* __restrict__ g_means2d,
    float* __restrict__ g_conics, float* __restrict__ g_colors,
    float* __restrict__ g_opac) {
  __shared__ float4 s0[kBatch], s1[kBatch], s2[kBatch];
  const TileCoord tc = tile_coord(P);
  const int nstop = tile_stop[tc.tile];
  if (nstop <= 0) return;
  const int start = tile_offsets[tc.tile];
  const float px = (float)tc.x + 0.5f;
  float py[kPix], Tc[kPix], gr[kPix], gg[kPix], gb[kPix], gT[kPix];
  int lk[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int y = tc.ybase + 4 * k;
    const bool valid = (tc.x < P.width) && (y < P.height);
    py[k] = (float)y + 0.5f;
    if (valid) {
      const int64_t pix = ((int64_t)tc.batch * P.height + y) * P.width + tc.x;
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
    stage_batch(packed, binned, start + cstart, n, s0, s1, s2);
    __syncthreads();
    for (int j = n - 1; j >= 0; --j) {
      const int i = cstart + j;
      const float4 a0 = s0[j];   // mx, my, A, B
      const float4 a1 = s1[j];   // C, opacity, r, g
      const float4 a2 = s2[j];   // blue, orig index bits
      const float dx = px - a0.x;
      float acc_mx = 0.f, acc_my = 0.f, acc_a = 0.f, acc_b = 0.f, acc_c = 0.f;
      float acc_r = 0.f, acc_g = 0.f, acc_bl = 0.f, acc_o = 0.f;
      bool contrib = false;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        if (i < lk[k]) {
          const float dy = py[k] - a0.y;
          const float power = splat_power(a0.z, a0.w, a1.x, dx, dy);
          if (power <= 0.0f) {
            const float e = splat_exp(power);
            const float raw = a1.y * e;
            const float alpha = fminf(P.max_alpha, raw);
            if (alpha >= P.alpha_thr) {
              contrib = true;
              const float T_prev = Tc[k] / fmaxf(1.0f - alpha, P.eps);
              const float dot_gc = gr[k] * a1.z + gg[k] * a1.w + gb[k] * a2.x;
              const float g_alpha = T_prev * (dot_gc - gT[k]);
              const float wgt = T_prev * alpha;
              acc_r += gr[k] * wgt;
              acc_g += gg[k] * wgt;
              acc_bl += gb[k] * wgt;
              const float g_raw = (raw < P.max_alpha) ? g_alpha : 0.0f;
              const float g_pow = g_raw * raw;
              acc_a += g_pow * (-0.5f) * dx * dx;
              acc_b += g_pow * (-1.0f) * dx * dy;
              acc_c += g_pow * (-0.5f) * dy * dy;
              // a = -2A, b = -B, c = -2C
              acc_mx -= g_pow * (2.0f * a0.z * dx + a0.w * dy);
              acc_my -= g_pow * (a0.w * dx + 2.0f * a1.x * dy);
              acc_o += g_raw * e;
              gT[k] = alpha * dot_gc + (1.0f - alpha) * gT[k];
              Tc[k] = T_prev;
            }
          }
        }
      }
      if (__any(contrib)) {
        acc_mx = wave_sum(acc_mx);
        acc_my = wave_sum(acc_my);
        acc_a = wave_sum(acc_a);
        acc_b = wave_sum(acc_b);
        acc_c = wave_sum(acc_c);
        acc_r = wave_sum(acc_r);
        acc_g = wave_sum(acc_g);
        acc_bl = wave_sum(acc_bl);
        acc_o = wave_sum(acc_o);
        if (threadIdx.x == 0) {
          const int64_t orig = __float_as_int(a2.y);
          unsafeAtomicAdd(&g_means2d[2 * orig + 0], acc_mx);
          unsafeAtomicAdd(&g_means2d[2 * orig + 1], acc_my);
          unsafeAtomicAdd(&g_conics[3 * orig + 0], acc_a);
          unsafeAtomicAdd(&g_conics[3 * orig + 1], acc_b);
          unsafeAtomicAdd(&g_conics[3 * orig + 2], acc_c);
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
