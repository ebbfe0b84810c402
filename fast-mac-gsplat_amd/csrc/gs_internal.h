// gs_internal.h -- declarations shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gsplat_hip.h"

namespace gs {

// Render parameters passed by value to every raster kernel (the HIP analogue
// of the reference's MetaI32/MetaF32 constant buffers,
// variants/v8/csrc/metal/gsplat_v8_kernels.metal:23-48).
struct RasterParams {
  int height, width;
  int tiles_x, tiles_y;
  int tiles_per_image;
  int num_tiles;  // B * tiles_per_image
  int batch, gpb;  // gaussians per batch
  int num_splats;  // B * G
  float alpha_thr, trans_thr;
  float bg_r, bg_g, bg_b;
  float eps, max_alpha;
};

struct ProjectParams {
  int batch, gpb, num_splats;
  float near_plane;
};

// Error reporting (thread-local message, see gsplat_hip_last_error).
void set_error(const char* fmt, ...);
int check_launch(const char* what);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---- scan (scan.hip)
size_t scan_workspace_bytes(int64_t n);
int exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, void* ws,
                       size_t ws_bytes, hipStream_t stream);

// ---- radix sort (radix_sort.hip)
size_t radix_sort_workspace_bytes(int64_t n_per_segment, int segments);
// key_from_depth: first pass derives keys from float depths (depth_src) and
// values from the in-segment index.
int radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in,
                     const float* depth_src, uint32_t* keys_out,
                     uint32_t* vals_out, int64_t n_per_segment, int segments,
                     int begin_bit, int end_bit, void* ws, size_t ws_bytes,
                     hipStream_t stream);

// ---- binning (binning.hip)
int launch_count_pack(const RasterParams& P, const float* means2d,
                      const float* conics, const float* colors,
                      const float* opacities, const uint32_t* perm,
                      float* packed, int32_t* splat_counts,
                      int32_t* tile_counts, hipStream_t stream);
int launch_emit(const RasterParams& P, const float* packed,
                const int32_t* splat_offsets, uint32_t* keys, uint32_t* vals,
                hipStream_t stream);
int launch_fill_i32(int32_t* dst, int32_t value, int64_t n, hipStream_t stream);
int launch_fill_f32(float* dst, float value, int64_t n, hipStream_t stream);
int launch_zero_grads(float* g_m, float* g_q, float* g_c, float* g_o,
                      int64_t n, hipStream_t stream);

// ---- compositing (composite.hip)
int launch_render_forward(const RasterParams& P, const float* packed,
                          const int32_t* tile_offsets,
                          const int32_t* binned_ids, float* out_rgb,
                          float* out_T, int32_t* out_last,
                          int32_t* out_tile_stop, hipStream_t stream);
int launch_render_backward(const RasterParams& P, const float* packed,
                           const int32_t* tile_offsets,
                           const int32_t* binned_ids, const float* final_T,
                           const int32_t* last, const int32_t* tile_stop,
                           const float* grad_rgb, float* g_means2d,
                           float* g_conics, float* g_colors, float* g_opac,
                           hipStream_t stream);

// ---- projection (project.hip)
int launch_project_forward(const ProjectParams& P, const float* means3d,
                           const float* scales, const float* quats,
                           const float* opacities, const float* c2w,
                           const float* cam, float* out_means2d,
                           float* out_conics, float* out_opac,
                           float* out_depths, hipStream_t stream);
int launch_project_backward(const ProjectParams& P, const float* g_means2d,
                            const float* g_conics, const float* g_opac_out,
                            const float* g_depths, const float* means3d,
                            const float* scales, const float* quats,
                            const float* opacities, const float* c2w,
                            const float* cam, float* g_means3d,
                            float* g_scales, float* g_quats, float* g_opac,
                            float* g_c2w, float* g_cam, hipStream_t stream);

// Maps a linear workgroup id onto a linear work index so that the 8 XCDs of
// an MI355X (which receive workgroups round-robin) each process one
// contiguous range of work items.  Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  return xcd * q + min(xcd, r) + slot;
}

}  // namespace gs
