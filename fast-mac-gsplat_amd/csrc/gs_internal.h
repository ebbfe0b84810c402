// gs_internal.h -- declarations shared by the library's translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gsplat_hip.h"

namespace gs {

// float4 words of one packed splat record (GSPLAT_RECORD_FLOATS floats).
constexpr int kRecordVec4 = GSPLAT_RECORD_FLOATS / 4;
static_assert(GSPLAT_RECORD_FLOATS == 16, "record layout of pack_record");

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

// Order-preserving map of a float depth to uint32 (ascending float order ==
// ascending key).  -0.0 and +0.0 map to the same key (they compare equal in
// torch.argsort); every NaN maps to 0xffc00000, above +inf (torch sorts NaN
// last).
__device__ __forceinline__ uint32_t depth_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (f == 0.0f) u = 0u;
  if (!(f == f)) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- scan (scan.hip)
size_t scan_workspace_bytes(int64_t n);
// ctl_zeroed: the workspace's look-back status and ticket are already zero
// (otherwise they are zeroed by an extra launch).  status_out (device int32,
// may be null): receives 0 or GSPLAT_STATUS_LOOKBACK_TIMEOUT (zeroed by the
// same launch).  first_ticket > 0 (diagnostic only): workgroup tickets start
// there, so the first first_ticket blocks are never scanned and their
// look-back statuses never published; spin_limit bounds each wait.
int exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, void* ws,
                       size_t ws_bytes, hipStream_t stream,
                       bool ctl_zeroed = false, int32_t* status_out = nullptr,
                       int first_ticket = 0, int spin_limit = 1 << 20);

// ---- radix sort (radix_sort.hip)
// Layout of one sort: a control block (global digit histograms, look-back
// status, tickets; must be zero before the sort, except that the histograms
// may be filled by the caller) and ping-pong key/value buffers.
struct RadixPlan {
  int64_t n_seg;
  int segments, nblk, passes, begin_bit, end_bit;
  int rounds;  // 64-element groups per wavefront of a sort workgroup
  int64_t ghist_words, status_words, ticket_words;
  size_t a_keys, a_vals, b_keys, b_vals, buffer_bytes;
};
struct RadixCtl {
  uint32_t* ghist;    // [4][segments][256]
  uint32_t* status;   // [passes][segments][nblk][256]
  uint32_t* tickets;  // [4] (ticket_words = 8: the tickets, then the error
                      // word radix_ctl_at points err at)
  uint32_t* err;      // look-back give-up status (GSPLAT_STATUS_*), zeroed
                      // with the control block
};
RadixPlan radix_plan(int64_t n_seg, int segments, int begin_bit, int end_bit);
size_t radix_ctl_bytes(const RadixPlan& L);
RadixCtl radix_ctl_at(const RadixPlan& L, void* p);
bool radix_size_ok(int64_t n_seg, int segments);
size_t radix_sort_workspace_bytes(int64_t n_per_segment, int segments);
int launch_zero_u32(uint32_t* p, int64_t n, hipStream_t stream);
// Fills C.ghist (zeroed) from the keys, or from float depths when depth_src.
int radix_global_hist(const RadixPlan& L, const RadixCtl& C,
                      const uint32_t* keys, const float* depth_src,
                      hipStream_t stream);
// One onesweep launch per pass.  depth_src: first pass derives keys from
// float depths and values from the in-segment index.  n_dev (one segment
// only): the sort takes the first min(*n_dev, L.n_seg) elements, L.n_seg
// being the capacity of the buffers; the histograms must count exactly those.
int radix_passes(const RadixPlan& L, const RadixCtl& C, void* buffers,
                 const uint32_t* keys_in, const uint32_t* vals_in,
                 const float* depth_src, uint32_t* keys_out,
                 uint32_t* vals_out, hipStream_t stream,
                 const int32_t* n_dev = nullptr);
// The tile-pair sort as two passes over packed words (keys below 2^16,
// values below 2^24: radix_pair_ranges_ok), whose second pass also writes
// tile_offsets[0..num_tiles] (every entry; workgroup 0 writes
// tile_offsets[num_tiles] = n).  Nothing is written for n = 0.  Uses the
// plan's first ping-pong value buffer; ghist holds both passes' counts.
bool radix_pair_ranges_ok(const RadixPlan& L, int64_t num_values);
// Its input is the emit's key_bytes form: key_bytes (the tiles' low bytes)
// and words ((tile >> 8) << 24 | gid).  The control words that
// radix_pair_zero_span returns (*words of them) must be zero before it.
uint32_t* radix_pair_zero_span(const RadixPlan& L, const RadixCtl& C,
                               int64_t* words);
int radix_pair_sort_ranges(const RadixPlan& L, const RadixCtl& C,
                           void* buffers, const uint8_t* key_bytes,
                           const uint32_t* words, uint32_t* vals_out,
                           int32_t* tile_offsets, int num_tiles,
                           hipStream_t stream, const int32_t* n_dev);
// Self-contained sort (zeroes its control block, computes the histograms).
// status_out (device int32, may be null): receives 0 or
// GSPLAT_STATUS_LOOKBACK_TIMEOUT.
int radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in,
                     const float* depth_src, uint32_t* keys_out,
                     uint32_t* vals_out, int64_t n_per_segment, int segments,
                     int begin_bit, int end_bit, void* ws, size_t ws_bytes,
                     hipStream_t stream, int32_t* status_out = nullptr);
// ---- stable depth order of small images (depth_sort.hip)
// Images of at most 131072 splats: run sort in LDS + merge ranks, two
// launches.  buffers: depth_small_bytes(G, batch) bytes.
bool depth_small_ok(int64_t G);
size_t depth_small_bytes(int64_t G, int batch);
int launch_depth_order_small(const float* depths, int32_t* perm, int64_t G,
                             int batch, void* buffers, hipStream_t stream);
// The second of those launches alone (the runs are already in buffers).
int launch_depth_ranks_small(void* buffers, int32_t* perm, int64_t G,
                             int batch, hipStream_t stream);

// ---- binning (binning.hip)
// count: per-splat tile-hit counts (original order) into splat_count, the
// per-workgroup sums into block_sums (count_blocks(P) ints) and their total
// N into *pair_count (-1 if N does not fit in int32); the same launch zeroes
// zero_words[0..n_zero_words).  Requires P.num_splats > 0.
int count_blocks(const RasterParams& P);
// With colors and rec_orig (float [BG*16]) the count also writes each
// splat's packed record in original order with its hit count in the orig
// slot, for launch_pack's rec_orig.  With hit_bits (hit_bits_words(P)
// words) it records each wavefront's first kHitSlab walk steps' hit
// ballots, which launch_emit's original-order walk then reads instead of
// testing those candidates again.
constexpr int kHitSlab = 128;
size_t hit_bits_words(const RasterParams& P);
int launch_count(const RasterParams& P, const float* means2d,
                 const float* conics, const float* opacities,
                 int32_t* splat_count, int32_t* block_sums,
                 int32_t* pair_count, uint32_t* zero_words,
                 int64_t n_zero_words, hipStream_t stream,
                 const float* colors = nullptr, float* rec_orig = nullptr,
                 uint64_t* hit_bits = nullptr);
// count_depth_runs: the count (splat_count, zero_words as above; no block
// sums and no N) and the first launch of the small-image depth order (runs
// into depth_buffers) as one launch.  Requires P.num_splats > 0 and
// depth_small_ok(P.gpb); launch_depth_ranks_small completes the order.
// The pair sort's one-pass histogram counted by the count blocks of
// launch_count_depth_runs (digit (tile >> shift) & 255 of every hit, one
// row of 256 partial counts per count block in parts) and summed into
// ghist[0..255] by an extra workgroup of launch_rank_pack; parts null: not
// counted there.
struct CountHist {
  uint32_t* parts = nullptr;
  int shift = 0;
  int nparts = 0;
  uint32_t* ghist = nullptr;
};
int count_depth_runs_blocks(const RasterParams& P);
int launch_count_depth_runs(const RasterParams& P, const float* means2d,
                            const float* conics, const float* opacities,
                            int32_t* splat_count, uint32_t* zero_words,
                            int64_t n_zero_words, const float* depths,
                            void* depth_buffers, hipStream_t stream,
                            const CountHist& H = CountHist{});
// pack: packed records in gid order and splat_offsets[0..BG] (exclusive scan
// of splat_count[perm]) via a look-back scan whose status
// (count_scan_blocks(P) words) and ticket must be zero.
// err: the give-up status word of the look-back (zero before the launch).
// orig_slot (int32 [BG][2], may be null): per original index {pair offset,
// gid}, for launch_emit's original-order walk.
int launch_pack(const RasterParams& P, const float* means2d,
                const float* conics, const float* colors,
                const float* opacities, const uint32_t* perm,
                const int32_t* splat_count, float* packed,
                int32_t* splat_offsets, uint64_t* scan_status,
                uint32_t* scan_ticket, uint32_t* err, hipStream_t stream,
                const float* rec_orig = nullptr, int32_t* orig_slot = nullptr);
int count_scan_blocks(const RasterParams& P);
// pack_records: the packed records of splats already in depth order
// (record gid from attributes gid, orig = gid).
int launch_pack_records(const RasterParams& P, const float* means2d,
                        const float* conics, const float* colors,
                        const float* opacities, float* packed,
                        hipStream_t stream);
// Words that a launch zeroes on the side (n 32-bit words at p).
struct ZeroSpan {
  uint32_t* p;
  int64_t n;
};

// emit: writes the (tile, gid) pairs into each splat's range, zeroes
// pair_status, and fills pair_ghist ([pair_passes][256], zero on entry) with
// the pair sort's digit histograms (digit p = bits hist_shift + 8p .. +7 of
// the tile), atomically or via per-workgroup partials
// (emit_blocks(P) * 4 * 256 words) and a reduction launch.  Only the first min(N, capacity) pairs are written and counted,
// N = splat_offsets[num_splats] (-1 when N overflowed: nothing is written).
int emit_blocks(const RasterParams& P);
// With scan, the emit scans the per-gid counts itself, each workgroup from
// the sum of block_totals (emit_blocks(P) words: per emit workgroup the sum
// of its gids' counts, as launch_rank_pack adds them) over the workgroups
// before it, and writes splat_offsets[0..BG] there; splat_offsets is then
// not read.
struct EmitScanArgs {
  const int32_t* gid_count;
  int32_t* splat_offsets;
  const uint32_t* block_totals;
};
// With orig (not with scan), the emit walks the splats in original order,
// as the count did: from the count's records (rec_orig, launch_count's),
// the pack's orig_slot and the count's hit_bits (may be null: every
// candidate is tested), writing the same pairs at the same positions.
struct EmitOrigArgs {
  const float* rec_orig;
  const int32_t* orig_slot;
  const uint64_t* hit_bits;
};
int launch_emit(const RasterParams& P, const float* packed,
                const int32_t* splat_offsets, int64_t capacity, uint32_t* keys,
                uint32_t* vals, int pair_passes, uint32_t* hist_partials,
                uint32_t* pair_ghist, uint32_t* pair_status,
                int64_t pair_status_words, hipStream_t stream,
                const EmitScanArgs* scan = nullptr, int hist_shift = 0,
                uint8_t* key_bytes = nullptr,
                const EmitOrigArgs* orig = nullptr);
// Second half of the pair sort when one onesweep pass has ordered the pairs
// by the tile bits above low_bits (a bucket = 2^low_bits consecutive tiles;
// at most 256 buckets): one workgroup per bucket sorts its pairs stably on
// the low bits and writes binned_ids, the bucket's tile_offsets (and
// tile_counts unless NULL), tile_offsets[num_tiles] = min(n, *n_dev), the
// status OR and the long-range flag as launch_tile_ranges does, and zeroes
// the two spans.  bucket_sizes: the pass's digit histogram.  Any bucket size
// is sorted correctly; one of at most kBucketChunk pairs takes one pass.
constexpr int kBucketChunk = 4096;
struct BucketSortArgs {
  const uint32_t* keys;
  const uint32_t* vals;
  const uint32_t* bucket_sizes;
  int64_t n;
  const int32_t* n_dev;
  int num_tiles, low_bits;
  int32_t* tile_offsets;
  int32_t* tile_counts;
  uint32_t* binned_ids;
  const uint32_t* err[3];
  int32_t* status_out;
  int32_t* long_flag;
  ZeroSpan zero[2];
};
int launch_bucket_sort(const BucketSortArgs& A, hipStream_t stream);
// rank_pack: the second launch of the small-image depth order (runs in
// depth_buffers, as launch_count_depth_runs leaves them) with the records
// packed at the ranks: perm, packed, gid_count[gid] = splat_count[orig], and
// each gid's count added to block_totals[gid / gids per emit workgroup]
// (zero before the launch; the pair offsets then come from launch_emit with
// scan).
int launch_rank_pack(const RasterParams& P, const float* means2d,
                     const float* conics, const float* colors,
                     const float* opacities, void* depth_buffers,
                     const int32_t* splat_count, int32_t* perm, float* packed,
                     int32_t* gid_count, uint32_t* block_totals,
                     hipStream_t stream, const CountHist& H = CountHist{});
// Tile ranges longer than this many pairs are walked by the forward's first
// launch only up to here and continued by its second (render_fwd_long).
constexpr int kHandoffPairs = GSPLAT_HANDOFF_PAIRS;


// tile_offsets[0..T] and (unless tile_counts is NULL) tile_counts[0..T)
// from the n sorted tile keys (min(n, *n_dev) of them with n_dev).  With
// status_out, the same launch writes there the OR of the (non-null) give-up
// status words err[0..2] of the binning's look-backs; with long_flag (a
// device word that is zero before the launch, n > 0 only) it sets
// *long_flag to 1 if a tile range is longer than kHandoffPairs.
// zero (may be null): two spans that the same launch zeroes.
int launch_tile_ranges(const uint32_t* sorted_keys, int64_t n, int num_tiles,
                       int32_t* tile_offsets, int32_t* tile_counts,
                       hipStream_t stream, const int32_t* n_dev = nullptr,
                       const uint32_t* err0 = nullptr,
                       const uint32_t* err1 = nullptr,
                       const uint32_t* err2 = nullptr,
                       int32_t* status_out = nullptr,
                       int32_t* long_flag = nullptr,
                       const ZeroSpan* zero = nullptr);
// After radix_pair_sort_ranges: status, emptied ranges on a look-back
// give-up or n = 0, the long-range flag, zero spans and tile_counts (may be
// null), as launch_tile_ranges does from sorted keys.
int launch_ranges_finish(int64_t n, int num_tiles, int32_t* tile_offsets,
                         int32_t* tile_counts, hipStream_t stream,
                         const int32_t* n_dev, const uint32_t* err0,
                         const uint32_t* err1, const uint32_t* err2,
                         int32_t* status_out, int32_t* long_flag,
                         const ZeroSpan* zero);

// The binning's results for the host: device words {N, status, long-range
// flag} copied to pinned host words host[0..2], then host[3] = 1.  Every
// store is a system-scope store, and host[3] is a release store, so a host
// thread that reads host[3] == 1 then reads the final host[0..2] without a
// HIP event or stream synchronisation.
struct HostReport {
  const int32_t* n;
  const int32_t* status;
  const int32_t* long_flag;
  int32_t* host;
};
__device__ inline void write_host_report(const HostReport& R) {
  const int32_t v0 = *R.n, v1 = *R.status, v2 = *R.long_flag;
  __hip_atomic_store(R.host + 0, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(R.host + 1, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(R.host + 2, v2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __hip_atomic_store(R.host + 3, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
// One workgroup that writes the report (when no forward launch carries it).
int launch_host_report(const HostReport& R, hipStream_t stream);
int launch_zero2(uint32_t* a, int64_t na, uint32_t* b, int64_t nb,
                 hipStream_t stream);
int launch_fill_i32(int32_t* dst, int32_t value, int64_t n, hipStream_t stream);
int launch_fill_f32(float* dst, float value, int64_t n, hipStream_t stream);
int launch_zero_grads(float* g_m, float* g_q, float* g_c, float* g_o,
                      int64_t n, hipStream_t stream);

// Per-thread, one-shot timing of the compositors' launches with the
// caller's events (created with timing): kTimeForward brackets the forward
// (render_fwd_kernel, through the long-tile continuation when the same call
// issues it), kTimeBackward render_bwd_kernel alone.  The next such launch
// on the thread takes the pair.
constexpr int kTimeForward = 0;
constexpr int kTimeBackward = 1;
void set_launch_timing(int which, hipEvent_t start, hipEvent_t stop);
void take_launch_timing(int which, hipEvent_t& start, hipEvent_t& stop);

// Launch trace (gsplat_hip_trace_launches): while armed, each kernel launch
// of the library, on any thread, takes the next of the caller's event pairs
// and records its kernel's name; start = stop = null when the trace is not
// armed or is full.
constexpr int kTraceMax = 1024;  // GSPLAT_TRACE_MAX
void trace_take(const char* name, hipEvent_t& start, hipEvent_t& stop);

// Every kernel launch of the library: with the trace's events when the
// trace is armed (hipExtLaunchKernelGGL records them at the kernel's own
// start and end, so they time the kernel alone).  The arguments are
// converted to the kernel's parameter types.
template <typename... KArgs, typename... Args>
inline void launch_traced(const char* name, void (*kernel)(KArgs...),
                          dim3 grid, dim3 block, size_t shmem,
                          hipStream_t stream, Args&&... args) {
  hipEvent_t t0 = nullptr, t1 = nullptr;
  trace_take(name, t0, t1);
  if (t0 != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)shmem, stream, t0, t1,
                          0, static_cast<KArgs>(args)...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream,
                       static_cast<KArgs>(args)...);
}

// ---- compositing (composite.hip)
// workspace (render_workspace_bytes, may be null): heavy-tile segment state,
// written by the forward and read by the backward of the same binning.
size_t render_workspace_bytes(const RasterParams& P, int64_t n_pairs);
// Forward launches.  flags: kForwardPreZeroed (the words of
// render_forward_zero_spans are already zero), kForwardNoLong (the tiles
// handed off are left for launch_render_forward_long, which the caller
// issues unless no tile range is longer than kHandoffPairs),
// kForwardStoppedLast (the one-wavefront kernel stores out_last only for
// the tiles where a pixel stopped, final T <= transmittance threshold: the
// backward reads last only for such pixels, and the other tiles' stores
// were most of 67 MB per launch at 4096x4096).
constexpr int kForwardPreZeroed = 1;
constexpr int kForwardNoLong = 2;
constexpr int kForwardStoppedLast = 4;
// report (may be null): the binning's host report, written by the forward's
// first workgroup as it starts (or by launch_host_report if the forward has
// no workgroup).
int launch_render_forward(const RasterParams& P, const float* packed,
                          const int32_t* tile_offsets,
                          const int32_t* binned_ids, float* out_rgb,
                          float* out_T, int32_t* out_last,
                          int32_t* out_tile_stop, int64_t n_pairs,
                          void* workspace, hipStream_t stream, int flags = 0,
                          const HostReport* report = nullptr);
int launch_render_forward_long(const RasterParams& P, const float* packed,
                               const int32_t* tile_offsets,
                               const int32_t* binned_ids, float* out_rgb,
                               float* out_T, int32_t* out_last,
                               int32_t* out_tile_stop, int64_t n_pairs,
                               void* workspace, hipStream_t stream,
                               hipEvent_t stop = nullptr);
// The workspace words a forward needs zero before it starts (hand-off
// counters; with the state outputs also the backward's gradient records).
void render_forward_zero_spans(const RasterParams& P, int64_t n_pairs,
                               void* workspace, bool training,
                               ZeroSpan out[2]);
int launch_render_backward(const RasterParams& P, const float* packed,
                           const int32_t* tile_offsets,
                           const int32_t* binned_ids, const float* final_T,
                           const int32_t* last, const int32_t* tile_stop,
                           const float* grad_rgb, float* g_means2d,
                           float* g_conics, float* g_colors, float* g_opac,
                           int64_t n_pairs, void* workspace,
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
                            float* g_c2w, float* g_cam, void* workspace,
                            hipStream_t stream);
// Camera-gradient partial sums: B * ceil(G/256) * 16 floats.
size_t project_backward_workspace_bytes(const ProjectParams& P);
// Device address (on the stream's device) of the static scratch array of
// the allocation-free projection backward; looked up once per device.
int project_noalloc_scratch(hipStream_t stream, void** out);

// Maps a linear workgroup id onto a linear work index so that the 8 XCDs of
// an MI355X (which receive workgroups round-robin) each process one
// contiguous range of work items.  Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  return xcd * q + min(xcd, r) + slot;
}

}  // namespace gs
