/*
 * gsplat_hip.h -- C ABI of the MI355X (gfx950) differentiable Gaussian-splat
 * rasterizer.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream (passed as void*).  The caller owns all memory: outputs and
 * workspaces are allocated by the caller (the Python layer uses torch's
 * caching allocator) and sized with the *_workspace_bytes queries.  No entry
 * point allocates, frees or synchronises the stream.
 *
 * All functions return GSPLAT_OK (0) on success.  On failure they return a
 * non-zero status and a thread-local message is available from
 * gsplat_hip_last_error().  Kernel launch errors are checked after every
 * launch.
 *
 * Conventions (shared with the reference's batched API):
 *   B      images in the batch, G splats per image, BG = B*G
 *   tiles  16x16 pixels, tiles_x = ceil(W/16), tiles_y = ceil(H/16),
 *          tile id = b*tiles_y*tiles_x + ty*tiles_x + tx, T = B*tiles_y*tiles_x
 *   "gid"  flat index b*G + r where r is the splat's rank in a stable sort of
 *          image b's depths (ascending, ties by original index); ascending gid
 *          within a tile is front-to-back order.
 *   packed splat record: 16 floats per gid (GSPLAT_RECORD_FLOATS),
 *          {mx, my, a, b}, {c, opacity, r, g}, {b, orig_index | plain << 31,
 *          q, lo}, {dxt, beta, gamma, delta}
 *          with the conic (a,b,c) meaning power = -0.5*(a dx^2 + 2 b dx dy + c dy^2);
 *          lo = log2(e)_f32 * ln(opacity) and q = plim + lo, where plim is
 *          the base-2 exponent limit of the alpha test,
 *          log2(e)_f32 * ln(max(alpha_threshold / opacity, FLT_MIN)), with
 *          ln evaluated by a fixed sequence of correctly rounded float
 *          operations (plim = +inf if opacity <= 0 or max_alpha <
 *          alpha_threshold, -inf if alpha_threshold <= 0; lo = -inf for 0,
 *          NaN for a negative or NaN opacity): the compositors evaluate
 *          opacity * 2^p as 2^(p + lo) and test p + lo >= q.  plain (bit 31
 *          of the orig word) marks a splat whose alpha test never needs the
 *          power <= 0 test or the max_alpha clamp; the last four floats are
 *          the splat's constants of the compositors' strip culling.
 *   sizes  at most 2^24 tiles per image, 2^31 - 1 tiles in the batch and
 *          fewer than 2^40 / 3 pixels in the batch.
 */
#ifndef GSPLAT_HIP_H
#define GSPLAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSPLAT_HIP_ABI_VERSION 15
#define GSPLAT_TILE_SIZE 16
#define GSPLAT_RECORD_FLOATS 16

enum gsplat_status {
  GSPLAT_OK = 0,
  GSPLAT_ERR_INVALID_ARGUMENT = 1,
  GSPLAT_ERR_HIP = 2,
  GSPLAT_ERR_WORKSPACE = 3
};

/* Device status words (the `status` outputs below): 0 when every kernel
 * completed normally.  The scans and sorts obtain earlier workgroups' totals
 * by decoupled look-back; a wait that exceeds its poll budget (a predecessor
 * starved for about a second, e.g. by another process on the GPU) gives up so
 * that every wave terminates, and sets this bit: the outputs of that call are
 * then wrong and must be discarded. */
#define GSPLAT_STATUS_LOOKBACK_TIMEOUT 1

/* Static render parameters.  Mirrors the reference's RasterConfig plus the
 * meta packing of variants/v8/torch_gsplat_bridge_v8/rasterize.py:129-173
 * (eps = 1e-8 and max_alpha = 0.99 are fixed there and passed here). */
typedef struct gsplat_raster_meta {
  int32_t height;
  int32_t width;
  int32_t tile_size;           /* must be 16 */
  int32_t batch;               /* B >= 1 */
  int32_t gaussians_per_batch; /* G >= 1 */
  float alpha_threshold;       /* 1/255 by default */
  float transmittance_threshold; /* 1e-4 by default */
  float background[3];
  float eps;                   /* 1e-8 */
  float max_alpha;             /* 0.99 */
} gsplat_raster_meta;

/* Pinhole projection parameters (variants/v9_project3d_train/
 * torch_gsplat_bridge_v9_project3d_train/rasterize.py:265-285). */
typedef struct gsplat_project_meta {
  int32_t batch;
  int32_t gaussians_per_batch;
  float near_plane;            /* 1e-4 by default */
} gsplat_project_meta;

int gsplat_hip_abi_version(void);
const char* gsplat_hip_last_error(void);

/* Timing of the next compositor launch on the calling thread (one-shot):
 * which = GSPLAT_TIME_FORWARD brackets the next forward (its first kernel
 * through the long-tile continuation when the same call issues it),
 * GSPLAT_TIME_BACKWARD the next backward's compositing kernel alone (not the
 * copy of its gradient records), with the caller's events (hipEvent_t
 * created with timing; both may be NULL to disarm), recorded by the launch
 * itself rather than as separate stream commands.  It has no counterpart in
 * the reference: it is for callers that measure the compositors' kernel
 * time, such as a benchmark's roofline figure. */
#define GSPLAT_TIME_FORWARD 0
#define GSPLAT_TIME_BACKWARD 1
int gsplat_hip_time_next_launch(int which, void* start_event,
                                void* stop_event);

/* Launch trace (instrumentation; no counterpart in the reference: it is for
 * callers that measure every kernel of a step, such as a benchmark's
 * per-stage breakdown).  Arms a process-wide trace of the next n kernel
 * launches of the library (n <= GSPLAT_TRACE_MAX), on any host thread:
 * launch k is bracketed by events[2k] and events[2k+1] (the caller's
 * hipEvent_t, created with timing), which the launch itself records at the
 * kernel's start and end (hipExtLaunchKernelGGL), so their elapsed time is
 * the kernel's.  Launches after the n-th run untraced.  n = 0 disarms.
 * gsplat_hip_trace_count() gives the launches traced since the trace was
 * armed (at most n), gsplat_hip_trace_name(k) the k-th one's kernel name
 * (static storage; NULL for k out of range).  A traced launch costs the
 * stream ~10 us more than an untraced one; do not arm it around a timed
 * region.  Arm and read it while no other thread launches work of the
 * library. */
#define GSPLAT_TRACE_MAX 1024
int gsplat_hip_trace_launches(void* const* events, int n);
int gsplat_hip_trace_count(void);
const char* gsplat_hip_trace_name(int k);

/* ---------------------------------------------------------------- binning
 * Replaces torch.ops.gsplat_metal_v8.bin (variants/v8/csrc/bindings.cpp:201,
 * host side variants/v8/csrc/metal/gsplat_metal.mm:140-204) together with the
 * stable depth argsort + gathers of variants/v8/torch_gsplat_bridge_v8/
 * rasterize.py:465-475 and the per-tile sort (gsplat_v8_kernels.metal:
 * 141-164).  The reference sizes binned_ids with a host read of
 * tile_offsets[-1] (gsplat_metal.mm:188).  Here binning is four calls sharing
 * one workspace:
 *   gsplat_hip_bin_count        per-splat tile-hit counts; writes the pair
 *                               count N;
 *   gsplat_hip_bin_depth_order  stable depth order per image;
 *   gsplat_hip_bin_pack         packed records in depth order, per-splat pair
 *                               offsets (after both calls above);
 *   gsplat_hip_bin_emit         pair emission, the stable sort by tile, and
 *                               the tile ranges/counts from the sorted keys.
 * bin_count and bin_depth_order use disjoint parts of the workspace and may
 * run concurrently on two streams; the caller orders bin_pack after both
 * (e.g. with an event) and bin_emit after bin_pack.  bin_emit reads N on the
 * device and takes the capacity of its buffers from the caller, so no host
 * read of N is needed before the compositors are enqueued: a caller sizes the
 * buffers from an earlier call (or reads N first, as the reference does),
 * copies N to the host asynchronously after bin_count and checks it against
 * the capacity later, binning again with larger buffers if it did not fit. */

/* Bytes of the binning workspace used by all four binning calls. */
size_t gsplat_hip_bin_count_workspace_bytes(const gsplat_raster_meta* meta);

/* Inputs (original order): means2d [BG,2], conics [BG,3], opacities [BG].
 * Output: *pair_count (one int32 in device memory) = N, the number of
 * (tile, splat) pairs, or -1 if N does not fit in int32.  The workspace keeps
 * the per-splat tile-hit counts and the zeroed control state that bin_pack
 * and bin_emit consume: pass the same workspace to them, unmodified. */
int gsplat_hip_bin_count(const gsplat_raster_meta* meta,
                         const float* means2d, const float* conics,
                         const float* opacities, int32_t* pair_count,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* Stable depth order per image (replaces torch.argsort(depths, stable=True),
 * v8 rasterize.py:466): perm int32 [BG], perm[b*G+r] = original index
 * (within image b) of the splat of depth rank r; -0.0 sorts as +0.0, NaNs
 * last.  Input depths [BG] in the original order. */
int gsplat_hip_bin_depth_order(const gsplat_raster_meta* meta,
                               const float* depths, int32_t* perm,
                               void* workspace, size_t workspace_bytes,
                               void* stream);

/* Inputs (original order): means2d [BG,2], conics [BG,3], colors [BG,3],
 * opacities [BG]; perm from bin_depth_order; the workspace after bin_count.
 * Outputs (gathers of v8 rasterize.py:467-475):
 *   packed        float [BG*16] packed records in gid (depth rank) order
 *   splat_offsets int32 [BG+1] exclusive scan of per-gid tile-hit counts */
int gsplat_hip_bin_pack(const gsplat_raster_meta* meta,
                        const float* means2d, const float* conics,
                        const float* colors, const float* opacities,
                        const int32_t* perm, float* packed,
                        int32_t* splat_offsets, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Packed records of splats that are already in depth order (record i from
 * attributes i: gradients of the compositor come back in this same order).
 * Inputs: means2d [BG,2], conics [BG,3], colors [BG,3], opacities [BG];
 * output packed float [BG*16].  The reference's compositor ops take the
 * depth-sorted flat arrays themselves and read them by binned id
 * (torch.ops.gsplat_metal_v8.render_* with the gathers of v8 rasterize.py:
 * 466-475 done by the caller; load_chunk_params in gsplat_v8_kernels.metal):
 * a caller that holds those arrays packs them with this call before
 * gsplat_hip_render_forward / _backward. */
int gsplat_hip_pack_records(const gsplat_raster_meta* meta,
                            const float* means2d, const float* conics,
                            const float* colors, const float* opacities,
                            float* packed, void* stream);

size_t gsplat_hip_bin_emit_workspace_bytes(const gsplat_raster_meta* meta,
                                           int64_t n_pairs);

/* Emits the N (tile, gid) pairs, sorts them by tile with a stable LSD radix
 * sort (8-bit digits) and extracts the tile ranges.  N is read on the device
 * (splat_offsets[BG] as bin_pack wrote it); n_pairs is the capacity of
 * binned_ids and the size the workspace was queried for.  Outputs:
 *   binned_ids    int32 [n_pairs]  first N entries: gids grouped by tile,
 *                              ascending gid (= depth order) inside each tile
 *                              range; the sorted 64-bit key of pair i is
 *                              (tile << 32) | binned_ids[i]
 *   tile_counts   int32 [T]    pairs per tile (may be NULL: not computed)
 *   tile_offsets  int32 [T+1]  tile t's range is [tile_offsets[t],
 *                              tile_offsets[t+1]); tile_offsets[T] = N
 * With n_pairs < N only the first n_pairs pairs in (gid, tile) order are
 * binned (tile_offsets[T] = n_pairs): a consistent but incomplete result that
 * the caller discards and redoes from bin_count with n_pairs >= N.  With
 * N = -1 (overflow) nothing is binned.
 * status (device int32, may be NULL): receives the OR of the GSPLAT_STATUS_*
 * bits of the whole binning (bin_depth_order, bin_pack and this call); when
 * it is not 0 every tile range is empty (tile_offsets all 0).
 * count_workspace is the workspace of bin_count / bin_pack.  Replaces
 * emit_binned_ids (variants/v8/csrc/metal/gsplat_v8_kernels.metal:290-327),
 * the reference's tile_counts/tile_offsets (count_tiles :244-288 + the
 * cumsum of gsplat_metal.mm:183-189) and its per-tile bitonic sort
 * (:141-164, :441-442). */
int gsplat_hip_bin_emit(const gsplat_raster_meta* meta, const float* packed,
                        const int32_t* splat_offsets, int64_t n_pairs,
                        int32_t* binned_ids, int32_t* tile_counts,
                        int32_t* tile_offsets, int32_t* status,
                        void* count_workspace, size_t count_workspace_bytes,
                        void* workspace, size_t workspace_bytes, void* stream);

/* All four binning calls in one: bin_count on count_stream (NULL: `stream`),
 * ordered after the work already enqueued on `stream` through inputs_event,
 * after which count_event is recorded; bin_depth_order on `stream`
 * concurrently; then bin_pack (after count_event) and bin_emit with the pair
 * capacity `capacity` (see bin_emit: n_pairs).  Finally a launch on
 * `stream` reports the binning to host_words (four int32 of page-locked host
 * memory mapped for the device, as hipHostMalloc and torch's pin_memory
 * allocate it; may be NULL): host_words[0] = the pair count N,
 * host_words[1] = the binning's status word (GSPLAT_STATUS_*),
 * host_words[2] = 1 if some tile range is longer than GSPLAT_HANDOFF_PAIRS
 * pairs, else 0, and then host_words[3] = 1.  The call sets host_words[3]
 * to 0 before it launches anything; the device writes it last, with
 * system-scope stores (release order), so a host thread that reads 1 there
 * may read words 0-2 without further synchronisation.  status_event (may be
 * NULL) is recorded on `stream` after the report: waiting for it is the
 * other way to know the words are final.  The events are the
 * caller's (hipEvent_t; inputs_event and count_event are required when
 * count_stream differs from stream).  If a look-back gave up, every tile
 * range is empty (the compositors then read no pair) and the status says
 * so.  Outputs as bin_depth_order (perm), bin_pack (packed, splat_offsets)
 * and bin_emit (binned_ids [capacity], tile_offsets).  One call instead of
 * four keeps the host's per-step launch overhead small; it replaces the same
 * reference steps as the four calls. */
size_t gsplat_hip_bin_workspace_bytes(const gsplat_raster_meta* meta,
                                      int64_t capacity);
int gsplat_hip_bin(const gsplat_raster_meta* meta, const float* means2d,
                   const float* conics, const float* colors,
                   const float* opacities, const float* depths,
                   int64_t capacity, int32_t* perm, float* packed,
                   int32_t* splat_offsets, int32_t* binned_ids,
                   int32_t* tile_offsets, int32_t* host_words,
                   void* workspace, size_t workspace_bytes, void* stream,
                   void* count_stream, void* inputs_event,
                   void* count_event, void* status_event);

/* -------------------------------------------------------------- composite
 * Compositor workspace (optional).  With it the forward continues a tile
 * that still has live pixels after 128 splats with four wavefronts, and,
 * when the state outputs are given, records the tile's 128-splat segments so
 * that the backward given the same workspace walks them in parallel.
 * Without it every tile is walked by one wavefront.  Images are identical
 * either way; gradients differ only in summation order.  The forward
 * overwrites the workspace.  The backward reads the forward's part and
 * accumulates into one 64-byte record per splat, so that the nine atomic
 * additions a tile makes to a splat's gradients go to one cache line
 * (without a workspace they go straight to the four output arrays); the
 * training forward zeroes these records and the backward leaves them zero,
 * so a backward takes a workspace that a training forward with n_pairs > 0
 * has filled (repeated backwards on it are fine).  n_pairs sizes the
 * record area: the pair count N or any capacity >= N (the length of the
 * binned_ids buffer), and the forward and the backward of one binning must
 * receive the same value (the layout follows it; a backward given another
 * n_pairs ignores the records and walks every tile whole).  n_pairs = 0
 * sizes the smaller workspace of the eval forward (state outputs NULL),
 * which records no segments. */
size_t gsplat_hip_render_workspace_bytes(const gsplat_raster_meta* meta,
                                         int64_t n_pairs);

/* Forward compositor.  Replaces render_fast_forward_state / _eval
 * (variants/v8/csrc/bindings.cpp:202-203; kernels gsplat_v8_kernels.metal:
 * 330-476).  out_rgb float [B,H,W,3].  State outputs (all NULL together for
 * the eval path): out_final_T float [B,H,W]
 * transmittance after the last composited splat, out_last int32 [B,H,W] =
 * the reference's per-pixel stop count (local_stop, gsplat_v8_kernels.metal:
 * 455-467): 1 + index (within the tile range) of the splat whose blend
 * brought T to transmittance_threshold, or the tile's pair count if the
 * pixel never stopped, out_tile_stop int32 [T] = max of out_last over the
 * tile's pixels (the reference's stop count). */
int gsplat_hip_render_forward(const gsplat_raster_meta* meta,
                              const float* packed, const int32_t* tile_offsets,
                              const int32_t* binned_ids, float* out_rgb,
                              float* out_final_T, int32_t* out_last,
                              int32_t* out_tile_stop, int64_t n_pairs,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* Tile ranges longer than this many pairs are handed from the forward's
 * one-wavefront walk to a continuation with four wavefronts per tile (with
 * a workspace). */
#define GSPLAT_HANDOFF_PAIRS 128

/* The forward compositor in two parts.  gsplat_hip_render_forward is
 * gsplat_hip_bin_render_forward's forward followed by this call, which
 * continues the tiles that the forward handed off (nothing without a
 * workspace, or when no tile range is longer than GSPLAT_HANDOFF_PAIRS).
 * Same arguments as gsplat_hip_render_forward.  It has no counterpart in
 * the reference: it is for callers that read host_words[2] of the binning
 * and skip it when it is 0. */
int gsplat_hip_render_forward_long(const gsplat_raster_meta* meta,
                                   const float* packed,
                                   const int32_t* tile_offsets,
                                   const int32_t* binned_ids, float* out_rgb,
                                   float* out_final_T, int32_t* out_last,
                                   int32_t* out_tile_stop, int64_t n_pairs,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream);

/* gsplat_hip_bin (arguments up to status_event, with its workspace as
 * bin_workspace) followed by gsplat_hip_render_forward on its outputs with
 * n_pairs = capacity and render_workspace (required, as are host_words),
 * except that the continuation of long tiles is left to
 * gsplat_hip_render_forward_long: call it with the same arguments unless
 * host_words[2] is 0.  The tile-range launch of the binning also zeroes the
 * forward's workspace words, so the forward follows it without a launch of
 * its own for that.  The binning's report (see gsplat_hip_bin) is written
 * by the forward's first workgroup as it starts, so the host can poll
 * host_words[3] and read the words while the forward runs; status_event
 * (may be NULL) is recorded after the forward.  With N above capacity
 * (see gsplat_hip_bin) the image is that of the incomplete binning.
 * out_last is written only for the tiles where a pixel stopped
 * (out_final_T <= transmittance_threshold); the other entries are left as
 * they were, since gsplat_hip_render_backward reads last only where the
 * pixel stopped.  It
 * has no counterpart in the reference (which binds bin and render as two
 * ops): it is the one-call form of both for the per-step path. */
int gsplat_hip_bin_render_forward(
    const gsplat_raster_meta* meta, const float* means2d, const float* conics,
    const float* colors, const float* opacities, const float* depths,
    int64_t capacity, int32_t* perm, float* packed, int32_t* splat_offsets,
    int32_t* binned_ids, int32_t* tile_offsets, int32_t* host_words,
    void* bin_workspace, size_t bin_workspace_bytes, float* out_rgb,
    float* out_final_T, int32_t* out_last, int32_t* out_tile_stop,
    void* render_workspace, size_t render_workspace_bytes, void* stream,
    void* count_stream, void* inputs_event, void* count_event,
    void* status_event);

/* Backward compositor.  Replaces render_fast_backward_saved
 * (variants/v8/csrc/bindings.cpp:204; kernel gsplat_v8_kernels.metal:
 * 478-608) and the unsort of v8 rasterize.py:676-680: gradients are written
 * in the ORIGINAL splat order using the orig_index stored in each packed
 * record; the four gradient arrays are written in full by this call.
 * last is read only for pixels with final_T <= transmittance_threshold
 * (a pixel above it composited its whole tile range).
 * workspace: the forward's (or NULL). */
int gsplat_hip_render_backward(const gsplat_raster_meta* meta,
                               const float* packed,
                               const int32_t* tile_offsets,
                               const int32_t* binned_ids,
                               const float* final_T, const int32_t* last,
                               const int32_t* tile_stop, const float* grad_rgb,
                               float* g_means2d, float* g_conics,
                               float* g_colors, float* g_opacities,
                               int64_t n_pairs, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------- projection
 * Pinhole projection.  Replaces torch.ops.gsplat_metal_v9_project3d_train.
 * project_pinhole_forward / _backward (variants/v9_project3d_train/csrc/
 * bindings.cpp:175-176; kernels gsplat_v9_project3d_train_kernels.metal:
 * 66-174 and 217-501).  means3d [BG,3], scales [BG,3] (linear), quats [BG,4]
 * (r,i,j,k, not normalised), opacities [BG], camera_to_world [B,4,4]
 * row-major, camera_params [B,4] = (fx, fy, cx, cy).  Outputs means2d
 * [BG,2], conics [BG,3], opacities [BG] (0 behind the near plane), depths
 * [BG] (camera z). */
int gsplat_hip_project_forward(const gsplat_project_meta* meta,
                               const float* means3d, const float* scales,
                               const float* quats, const float* opacities,
                               const float* camera_to_world,
                               const float* camera_params,
                               float* out_means2d, float* out_conics,
                               float* out_opacities, float* out_depths,
                               void* stream);

/* Bytes of the workspace of gsplat_hip_project_backward (camera-gradient
 * partial sums, B * ceil(G/256) * 16 floats). */
size_t gsplat_hip_project_backward_workspace_bytes(
    const gsplat_project_meta* meta);

/* Vector-Jacobian product of gsplat_hip_project_forward.  grad_depths may be
 * NULL, meaning a zero depth gradient (the rasterizer's, whose depth gradient
 * is zero).  Per-splat grads are written directly; g_camera_to_world [B,4,4]
 * (last row zero) and
 * g_camera_params [B,4] are overwritten with the camera gradients, summed
 * per workgroup into the workspace and then in a fixed order (no atomics). */
int gsplat_hip_project_backward(const gsplat_project_meta* meta,
                                const float* grad_means2d,
                                const float* grad_conics,
                                const float* grad_opacities,
                                const float* grad_depths,
                                const float* means3d, const float* scales,
                                const float* quats, const float* opacities,
                                const float* camera_to_world,
                                const float* camera_params,
                                float* g_means3d, float* g_scales,
                                float* g_quats, float* g_opacities,
                                float* g_camera_to_world,
                                float* g_camera_params,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/* Allocation-free variant of gsplat_hip_project_backward.  It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, results and kernels as
 * gsplat_hip_project_backward, without the workspace: the camera-gradient
 * partial sums go to a static device array of
 * GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends
 * and looked up on the stream's device at the first call there.  Limit:
 * B * ceil(G / 256) * 64 bytes must fit, i.e. B * ceil(G / 256) <= 16384
 * (B = 1: up to 4,194,304 splats); larger problems return
 * GSPLAT_ERR_INVALID_ARGUMENT.  Every slot of the array that a call reads
 * is written earlier by the same call, so nothing is cleared between calls.
 * All calls on one GPU share the array: calls that overlap on one GPU (on
 * different streams, or from different threads) race and must be ordered
 * by the caller.  Calls no hipMalloc, hipFree or allocating routine. */
#define GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES (1 << 20)
int gsplat_hip_project_backward_noalloc(
    const gsplat_project_meta* meta, const float* grad_means2d,
    const float* grad_conics, const float* grad_opacities,
    const float* grad_depths, const float* means3d, const float* scales,
    const float* quats, const float* opacities, const float* camera_to_world,
    const float* camera_params, float* g_means3d, float* g_scales,
    float* g_quats, float* g_opacities, float* g_camera_to_world,
    float* g_camera_params, void* stream);

/* ------------------------------------------------------------- primitives
 * Device-wide building blocks used by the stages above, exported so they can
 * be tested in isolation.  They have no counterpart in the reference (which
 * uses torch::cumsum, gsplat_metal.mm:183, and an in-threadgroup bitonic
 * sort). */

size_t gsplat_hip_scan_workspace_bytes(int64_t n);
/* out[0..n] = exclusive prefix sum of in[0..n-1]; out[n] = total.  In-place
 * (out == in) is allowed.  status (device int32, may be NULL): 0 or
 * GSPLAT_STATUS_* bits. */
int gsplat_hip_exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n,
                                  int32_t* status, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* Diagnostic (no counterpart in the reference): the scan above with its
 * first `stalled_blocks` 4096-element blocks never scanned, so their
 * look-back statuses are never published, and each look-back wait limited
 * to spin_limit polls.  The block after them gives up waiting, every kernel
 * finishes, and *status receives GSPLAT_STATUS_LOOKBACK_TIMEOUT; out holds
 * prefixes that miss the stalled blocks' totals (elements of the stalled
 * blocks themselves are not written).  It exists to test that a look-back
 * give-up reaches the caller; 0 <= stalled_blocks < ceil(n / 4096). */
int gsplat_hip_debug_stalled_scan(const int32_t* in, int32_t* out, int64_t n,
                                  int32_t stalled_blocks, int32_t spin_limit,
                                  int32_t* status, void* workspace,
                                  size_t workspace_bytes, void* stream);

size_t gsplat_hip_radix_sort_workspace_bytes(int64_t n_per_segment,
                                             int32_t segments);
/* Stable LSD radix sort of (key, value) pairs on key bits
 * [begin_bit, end_bit), 8-bit digits, independently inside each of
 * `segments` contiguous segments of n_per_segment elements.  vals_in may be
 * NULL (values are then the index within the segment); keys_out may be NULL
 * (keys are then not written).  status (device int32, may be NULL): 0 or
 * GSPLAT_STATUS_* bits. */
int gsplat_hip_radix_sort_pairs_u32(const uint32_t* keys_in,
                                    const uint32_t* vals_in,
                                    uint32_t* keys_out, uint32_t* vals_out,
                                    int64_t n_per_segment, int32_t segments,
                                    int32_t begin_bit, int32_t end_bit,
                                    int32_t* status, void* workspace,
                                    size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GSPLAT_HIP_H */
