// binning.hip -- per-splat tile intersection count, record packing, and
// deterministic (tile, gid) pair emission.
//
// This translation unit is compiled with -ffp-contract=off: the predicate
// results must match the CPU oracle bit for bit.
//
// count_kernel  one thread per splat in the original order: counts the tiles
//   whose pixel-centre rectangle meets the splat's alpha >= threshold ellipse
//   (reference count_tiles, variants/v8/csrc/metal/gsplat_v8_kernels.metal:
//   244-288) and bumps the per-tile pair counters.
// pack_kernel   one thread per depth-sorted splat (gid): writes the packed
//   48-byte record and the exclusive per-gid pair offsets (workgroup scan +
//   decoupled look-back in the same launch).
// emit_kernel   one thread per gid; repeats the same tile walk and writes
//   (tile, gid) at splat_offsets[gid] + k, so pairs land in ascending gid
//   order (reference emit_binned_ids, :290-327, which uses per-tile atomic
//   cursors and therefore needs a later per-tile sort).  The same launch also
//   prepares the pair sort: it zeroes the sort's look-back status and
//   accumulates its per-pass digit histograms from the tile counts.
#include "gs_internal.h"
#include "gs_predicate.h"
#include "lookback.h"

namespace gs {
namespace {

constexpr int kThreads = 256;

struct SplatGeom {
  float mx, my, a, b, c, o;
};

// Walks the tiles of one splat's snug bbox in row-major order and calls
// fn(global_tile, k) for the k-th tile that passes the exact ellipse/rect test.
template <typename Fn>
__device__ __forceinline__ int for_each_hit_tile(const RasterParams& P,
                                                 const SplatGeom& s, int batch,
                                                 Fn&& fn) {
#pragma clang fp contract(off)
  float tau;
  if (!alpha_support(s.o, P.alpha_thr, P.eps, tau)) return 0;
  const PixBox bb =
      snugbox(s.mx, s.my, s.a, s.b, s.c, tau, P.width, P.height, P.eps);
  if (bb.x0 > bb.x1 || bb.y0 > bb.y1) return 0;
  const int tx0 = bb.x0 >> 4, tx1 = bb.x1 >> 4;
  const int ty0 = bb.y0 >> 4, ty1 = bb.y1 >> 4;
  const int tile_base = batch * P.tiles_per_image;
  const ConicSlopes k = conic_slopes(s.a, s.b, s.c);
  int n = 0;
  for (int ty = ty0; ty <= ty1; ++ty) {
    for (int tx = tx0; tx <= tx1; ++tx) {
      float rx0, ry0, rx1, ry1;
      tile_rect(tx, ty, P.width, P.height, rx0, ry0, rx1, ry1);
      if (ellipse_hits_rect(s.mx, s.my, s.a, s.b, s.c, k, tau, rx0, ry0, rx1,
                            ry1)) {
        fn(tile_base + ty * P.tiles_x + tx, n);
        ++n;
      }
    }
  }
  return n;
}

// One thread per splat in the ORIGINAL order: tile-hit count into
// splat_count[orig] and per-tile pair counters (reference count_tiles,
// gsplat_v8_kernels.metal:244-288).  Runs before the depth sort, so the pair
// count N = sum(tile_counts) is known while the sort is still running.
__global__ __launch_bounds__(kThreads) void count_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ opacities,
    int32_t* __restrict__ splat_count, int32_t* __restrict__ tile_counts) {
  const int orig = blockIdx.x * kThreads + threadIdx.x;
  if (orig >= P.num_splats) return;
  SplatGeom s;
  s.mx = means2d[2 * orig + 0];
  s.my = means2d[2 * orig + 1];
  s.a = conics[3 * orig + 0];
  s.b = conics[3 * orig + 1];
  s.c = conics[3 * orig + 2];
  s.o = opacities[orig];
  splat_count[orig] = for_each_hit_tile(P, s, orig / P.gpb, [&](int tile, int) {
    atomicAdd(&tile_counts[tile], 1);
  });
}

// One thread per depth-sorted splat (gid): gathers the attributes of
// orig = perm[gid] into the packed 48-byte record and turns the per-gid
// tile-hit counts into exclusive offsets splat_offsets in the same launch
// (workgroup scan + decoupled look-back).
__global__ __launch_bounds__(kThreads) void pack_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, const uint32_t* __restrict__ perm,
    const int32_t* __restrict__ splat_count, float4* __restrict__ packed,
    int32_t* __restrict__ splat_offsets, uint64_t* scan_status,
    uint32_t* scan_ticket) {
  __shared__ int wsum[kThreads / 64];
  __shared__ int s_prefix;
  const int vb = take_ticket(scan_ticket);
  const int gid = vb * kThreads + threadIdx.x;
  int n = 0;
  if (gid < P.num_splats) {
    const int batch = gid / P.gpb;
    const int orig = batch * P.gpb + (int)perm[gid];
    const float mx = means2d[2 * orig + 0];
    const float my = means2d[2 * orig + 1];
    const float a = conics[3 * orig + 0];
    const float b = conics[3 * orig + 1];
    const float c = conics[3 * orig + 2];
    const float o = opacities[orig];
    const float cr = colors[3 * orig + 0];
    const float cg = colors[3 * orig + 1];
    const float cb = colors[3 * orig + 2];
    n = splat_count[orig];
    packed[3 * gid + 0] = make_float4(mx, my, a, b);
    packed[3 * gid + 1] = make_float4(c, o, cr, cg);
    packed[3 * gid + 2] =
        make_float4(cb, __int_as_float(orig),
                    visibility_limit(o, P.alpha_thr, P.max_alpha), 0.0f);
  }
  // Workgroup exclusive scan of the counts.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = n;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(inc, off, 64);
    if (lane >= off) inc += y;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  int pre = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    pre += (w < wave) ? wsum[w] : 0;
    total += wsum[w];
  }
  if (wave == 0) {
    if (lane == 0)
      status_store(&scan_status[vb], (vb == 0 ? kFlagInc64 : kFlagAgg64) |
                                         (uint64_t)(uint32_t)total);
    uint64_t prefix = 0;
    if (vb > 0) {
      prefix = lookback64_wave(scan_status, vb);
      if (lane == 0)
        status_store(&scan_status[vb], kFlagInc64 | (prefix + (uint32_t)total));
    }
    if (lane == 0) s_prefix = (int)prefix;
  }
  __syncthreads();
  const int off = s_prefix + pre + inc - n;
  if (gid < P.num_splats) splat_offsets[gid] = off;
  if (gid == P.num_splats - 1) splat_offsets[P.num_splats] = off + n;
}

__global__ __launch_bounds__(kThreads) void emit_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ splat_offsets,
    const int32_t* __restrict__ tile_counts, uint32_t* __restrict__ keys,
    uint32_t* __restrict__ vals, int pair_passes, uint32_t* pair_ghist,
    uint32_t* pair_status, int64_t pair_status_words) {
  __shared__ uint32_t h[4][256];
  const int t = threadIdx.x;
  // (1) zero the pair sort's look-back status (grid-stride)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + t; i < pair_status_words;
       i += (int64_t)gridDim.x * kThreads)
    pair_status[i] = 0u;
  // (2) pair-sort digit histograms from this workgroup's slice of tiles
  for (int i = t; i < 4 * 256; i += kThreads) (&h[0][0])[i] = 0u;
  __syncthreads();
  const int per = (P.num_tiles + gridDim.x - 1) / gridDim.x;
  const int t0 = blockIdx.x * per;
  const int t1 = min(P.num_tiles, t0 + per);
  for (int tile = t0 + t; tile < t1; tile += kThreads) {
    const uint32_t c = (uint32_t)tile_counts[tile];
    if (c == 0u) continue;
    for (int p = 0; p < pair_passes; ++p)
      atomicAdd(&h[p][((uint32_t)tile >> (8 * p)) & 255u], c);
  }
  __syncthreads();
  for (int p = 0; p < pair_passes; ++p) {
    const uint32_t c = h[p][t];
    if (c) atomicAdd(&pair_ghist[p * 256 + t], c);
  }
  // (3) pair emission
  const int gid = blockIdx.x * kThreads + t;
  if (gid >= P.num_splats) return;
  const float4 p0 = packed[3 * gid + 0];
  const float4 p1 = packed[3 * gid + 1];
  const SplatGeom s{p0.x, p0.y, p0.z, p0.w, p1.x, p1.y};
  const int batch = gid / P.gpb;
  const int64_t base = splat_offsets[gid];
  for_each_hit_tile(P, s, batch, [&](int tile, int k) {
    keys[base + k] = (uint32_t)tile;
    vals[base + k] = (uint32_t)gid;
  });
}

__global__ void fill_i32_kernel(int32_t* dst, int32_t v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = v;
}

__global__ void fill_f32_kernel(float* dst, float v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = v;
}

// Zeroes two word ranges in one launch (grid-stride).
__global__ void zero2_kernel(uint32_t* a, int64_t na, uint32_t* b, int64_t nb) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
       i < na || i < nb; i += stride) {
    if (i < na) a[i] = 0u;
    if (i < nb) b[i] = 0u;
  }
}

// Zeroes the four per-splat gradient arrays (2n, 3n, 3n, n floats) in one
// launch.
__global__ void zero_grads_kernel(float* g_m, float* g_q, float* g_c,
                                  float* g_o, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 2 * n) g_m[i] = 0.0f;
  if (i < 3 * n) {
    g_q[i] = 0.0f;
    g_c[i] = 0.0f;
  }
  if (i < n) g_o[i] = 0.0f;
}

}  // namespace

int launch_count(const RasterParams& P, const float* means2d,
                 const float* conics, const float* opacities,
                 int32_t* splat_count, int32_t* tile_counts,
                 hipStream_t stream) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(count_kernel, dim3(grid), dim3(kThreads), 0, stream, P,
                     means2d, conics, opacities, splat_count, tile_counts);
  return check_launch("count_kernel");
}

int launch_pack(const RasterParams& P, const float* means2d,
                const float* conics, const float* colors,
                const float* opacities, const uint32_t* perm,
                const int32_t* splat_count, float* packed,
                int32_t* splat_offsets, uint64_t* scan_status,
                uint32_t* scan_ticket, hipStream_t stream) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(kThreads), 0, stream, P,
                     means2d, conics, colors, opacities, perm, splat_count,
                     reinterpret_cast<float4*>(packed), splat_offsets,
                     scan_status, scan_ticket);
  return check_launch("pack_kernel");
}

int count_scan_blocks(const RasterParams& P) {
  return (P.num_splats + kThreads - 1) / kThreads;
}

int launch_emit(const RasterParams& P, const float* packed,
                const int32_t* splat_offsets, const int32_t* tile_counts,
                uint32_t* keys, uint32_t* vals, int pair_passes,
                uint32_t* pair_ghist, uint32_t* pair_status,
                int64_t pair_status_words, hipStream_t stream) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(emit_kernel, dim3(grid), dim3(kThreads), 0, stream, P,
                     reinterpret_cast<const float4*>(packed), splat_offsets,
                     tile_counts, keys, vals, pair_passes, pair_ghist,
                     pair_status, pair_status_words);
  return check_launch("emit_kernel");
}

int launch_zero2(uint32_t* a, int64_t na, uint32_t* b, int64_t nb,
                 hipStream_t stream) {
  const int64_t n = na > nb ? na : nb;
  if (n <= 0) return GSPLAT_OK;
  int64_t grid = (n + 255) / 256;
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(zero2_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     a, na, b, nb);
  return check_launch("zero2_kernel");
}

int launch_fill_i32(int32_t* dst, int32_t value, int64_t n,
                    hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (n + 255) / 256;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)grid), dim3(256), 0,
                     stream, dst, value, n);
  return check_launch("fill_i32_kernel");
}

int launch_zero_grads(float* g_m, float* g_q, float* g_c, float* g_o,
                      int64_t n, hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (3 * n + 255) / 256;
  hipLaunchKernelGGL(zero_grads_kernel, dim3((unsigned)grid), dim3(256), 0,
                     stream, g_m, g_q, g_c, g_o, n);
  return check_launch("zero_grads_kernel");
}

int launch_fill_f32(float* dst, float value, int64_t n, hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (n + 255) / 256;
  hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)grid), dim3(256), 0,
                     stream, dst, value, n);
  return check_launch("fill_f32_kernel");
}

}  // namespace gs
