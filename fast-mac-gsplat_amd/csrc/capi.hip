// capi.hip -- extern "C" entry points declared in include/gsplat_hip.h.
//
// Validation happens here, before any launch; every launch is followed by a
// hipGetLastError check.  Nothing here allocates or synchronises: buffers
// and workspaces belong to the caller and all work is enqueued on the
// caller's stream.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "gs_internal.h"

namespace gs {

namespace {
thread_local char g_err[1024] = "";
// armed launch timing (kTimeForward, kTimeBackward): start, stop
thread_local hipEvent_t g_timing[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
}

void set_launch_timing(int which, hipEvent_t start, hipEvent_t stop) {
  g_timing[which][0] = start;
  g_timing[which][1] = stop;
}

void take_launch_timing(int which, hipEvent_t& start, hipEvent_t& stop) {
  start = g_timing[which][0];
  stop = g_timing[which][1];
  g_timing[which][0] = g_timing[which][1] = nullptr;
}

namespace {
// The launch trace: process-wide, so that launches from any host thread
// (e.g. the autograd engine's device thread) are seen.  Slots are taken
// with one atomic add; g_trace_cap = 0 means disarmed.
hipEvent_t g_trace_ev[2 * kTraceMax];
const char* g_trace_name[kTraceMax];
std::atomic<int> g_trace_next{0};
std::atomic<int> g_trace_cap{0};
}  // namespace

void trace_take(const char* name, hipEvent_t& start, hipEvent_t& stop) {
  start = stop = nullptr;
  const int cap = g_trace_cap.load(std::memory_order_acquire);
  if (cap == 0) return;
  const int k = g_trace_next.fetch_add(1, std::memory_order_relaxed);
  if (k >= cap) return;
  g_trace_name[k] = name;
  start = g_trace_ev[2 * k];
  stop = g_trace_ev[2 * k + 1];
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return GSPLAT_ERR_HIP;
  }
  return GSPLAT_OK;
}

}  // namespace gs

namespace {

using gs::RasterParams;

constexpr int64_t kMaxSplats = int64_t(1) << 28;

int bits_for(int64_t max_value) {
  int b = 0;
  while (b < 32 && (int64_t(1) << b) <= max_value) ++b;
  return b;
}

int make_params(const gsplat_raster_meta* m, RasterParams& P) {
  if (m == nullptr) {
    gs::set_error("meta is NULL");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (m->tile_size != GSPLAT_TILE_SIZE) {
    gs::set_error("tile_size must be %d (got %d)", GSPLAT_TILE_SIZE,
                  m->tile_size);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (m->height <= 0 || m->width <= 0 || m->batch <= 0 ||
      m->gaussians_per_batch <= 0) {
    gs::set_error("height, width, batch and gaussians_per_batch must be > 0");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int64_t tiles_x = (m->width + 15) / 16;
  const int64_t tiles_y = (m->height + 15) / 16;
  const int64_t tpi = tiles_x * tiles_y;
  const int64_t T = tpi * m->batch;
  const int64_t BG = (int64_t)m->batch * m->gaussians_per_batch;
  const int64_t pixels = (int64_t)m->batch * m->height * m->width;
  if (T >= 0x7fffffffLL || tpi > (int64_t(1) << 24) || BG > kMaxSplats ||
      pixels * 3 >= (int64_t(1) << 40)) {
    gs::set_error("problem too large (tiles %lld, splats %lld)", (long long)T,
                  (long long)BG);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  // The compositors rely on 1 - alpha >= 1 - max_alpha >= eps (the
  // reference's max(1 - alpha, eps) guard is then a no-op) and on pixels
  // starting alive (T = 1 > transmittance_threshold).
  if (!(m->eps >= 0.0f && m->max_alpha >= 0.0f && m->max_alpha < 1.0f &&
        1.0f - m->max_alpha >= m->eps)) {
    gs::set_error("max_alpha must lie in [0, 1) with 1 - max_alpha >= eps "
                  "(got %g, eps %g)",
                  (double)m->max_alpha, (double)m->eps);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (!(m->transmittance_threshold >= 0.0f &&
        m->transmittance_threshold < 1.0f)) {
    gs::set_error("transmittance_threshold must lie in [0, 1) (got %g)",
                  (double)m->transmittance_threshold);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  P.height = m->height;
  P.width = m->width;
  P.tiles_x = (int)tiles_x;
  P.tiles_y = (int)tiles_y;
  P.tiles_per_image = (int)tpi;
  P.num_tiles = (int)T;
  P.batch = m->batch;
  P.gpb = m->gaussians_per_batch;
  P.num_splats = (int)BG;
  P.alpha_thr = m->alpha_threshold;
  P.trans_thr = m->transmittance_threshold;
  P.bg_r = m->background[0];
  P.bg_g = m->background[1];
  P.bg_b = m->background[2];
  P.eps = m->eps;
  P.max_alpha = m->max_alpha;
  return GSPLAT_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return GSPLAT_OK;
  (void)hipGetLastError();
  gs::set_error("%s: %s", what, hipGetErrorString(e));
  return GSPLAT_ERR_HIP;
}

int null_check(std::initializer_list<const void*> ptrs, const char* what) {
  for (const void* p : ptrs) {
    if (p == nullptr) {
      gs::set_error("%s: NULL pointer argument", what);
      return GSPLAT_ERR_INVALID_ARGUMENT;
    }
  }
  return GSPLAT_OK;
}

// Binning workspace shared by bin_count, bin_depth_order, bin_pack and
// bin_emit: a control region (the depth sort's control block, zeroed by
// bin_depth_order; then the pack-scan look-back status, its ticket (word 0)
// and give-up status (word 1), and the pair sort's histograms, tickets
// (words 0-3) and give-up status (word 4), zeroed by bin_count), then the
// per-splat tile-hit counts (original order), the count workgroups' sums and
// the depth sort's buffers (the onesweep's ping-pong buffers, or the sorted
// runs and samples of the two-launch sort of small images).  bin_count and
// bin_depth_order touch disjoint parts, so they may run concurrently on two
// streams.
struct CountLayout {
  gs::RadixPlan depth;
  size_t scan_status, scan_ticket, pair_ghist, pair_tickets, ctl_end;
  size_t splat_count, block_sums, gid_count, depth_buffers, rec_orig;
  size_t orig_slot, hit_bits, total;
};

CountLayout count_layout(const RasterParams& P) {
  CountLayout L{};
  L.depth = gs::radix_plan(P.gpb, P.batch, 0, 32);
  size_t off = gs::radix_ctl_bytes(L.depth);
  L.scan_status = off;  // the pack scan's, or the emit scan's in gsplat_hip_bin
  off += gs::align_up((size_t)std::max(gs::count_scan_blocks(P), gs::emit_blocks(P)) *
                          sizeof(uint64_t),
                      256);
  L.scan_ticket = off;
  off += 256;
  L.pair_ghist = off;
  off += 4 * 256 * sizeof(uint32_t);
  L.pair_tickets = off;
  off += 256;
  L.ctl_end = off;
  L.splat_count = off;
  off += gs::align_up((size_t)P.num_splats * sizeof(int32_t), 256);
  L.block_sums = off;
  off += gs::align_up((size_t)gs::count_blocks(P) * sizeof(int32_t), 256);
  L.gid_count = off;  // per-gid counts of gsplat_hip_bin's small-image path
  off += gs::align_up((size_t)P.num_splats * sizeof(int32_t), 256);
  L.depth_buffers = off;
  size_t depth_bytes = L.depth.buffer_bytes;
  if (gs::depth_small_ok(P.gpb))
    depth_bytes = std::max(depth_bytes, gs::depth_small_bytes(P.gpb, P.batch));
  off += gs::align_up(depth_bytes, 256);
  L.rec_orig = off;  // the count's original-order records (gsplat_hip_bin)
  off += gs::align_up((size_t)P.num_splats * GSPLAT_RECORD_FLOATS * sizeof(float),
                      256);
  // gsplat_hip_bin's original-order emit: per splat {pair offset, gid}, and
  // the count's recorded step ballots
  L.orig_slot = off;
  off += gs::align_up((size_t)P.num_splats * 2 * sizeof(int32_t), 256);
  L.hit_bits = off;
  off += gs::align_up(gs::hit_bits_words(P) * sizeof(uint64_t), 256);
  L.total = off;
  return L;
}

// Emit-stage workspace: emitted keys and values, the pair sort's look-back
// status, the emit workgroups' digit histograms, the sorted keys (for the
// tile ranges) and the sort's ping-pong buffers.
struct EmitLayout {
  gs::RadixPlan pairs;
  size_t keys, vals, status, hist, sorted_keys, buffers, total;
};

EmitLayout emit_layout(const RasterParams& P, int64_t n) {
  EmitLayout L{};
  L.pairs = gs::radix_plan(n, 1, 0, bits_for((int64_t)P.num_tiles - 1));
  const size_t vec = gs::align_up((size_t)n * sizeof(uint32_t), 256);
  size_t off = 0;
  L.keys = off;
  off += vec;
  L.vals = off;
  off += vec;
  L.status = off;
  off += gs::align_up((size_t)L.pairs.status_words * sizeof(uint32_t), 256);
  L.hist = off;
  off += gs::align_up((size_t)gs::emit_blocks(P) * 4 * 256 * sizeof(uint32_t), 256);
  L.sorted_keys = off;
  off += vec;
  L.buffers = off;
  off += L.pairs.buffer_bytes;
  L.total = off;
  return L;
}
}  // namespace

extern "C" {

int gsplat_hip_abi_version(void) { return GSPLAT_HIP_ABI_VERSION; }

const char* gsplat_hip_last_error(void) { return gs::g_err; }

size_t gsplat_hip_bin_count_workspace_bytes(const gsplat_raster_meta* meta) {
  RasterParams P;
  if (make_params(meta, P)) return 0;
  return count_layout(P).total;
}

int gsplat_hip_trace_launches(void* const* events, int n) {
  if (n < 0 || n > gs::kTraceMax || (n > 0 && events == nullptr)) {
    gs::set_error("gsplat_hip_trace_launches: n must lie in [0, %d] with "
                  "2n events",
                  gs::kTraceMax);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  gs::g_trace_cap.store(0, std::memory_order_release);
  for (int k = 0; k < 2 * n; ++k) {
    if (events[k] == nullptr) {
      gs::set_error("gsplat_hip_trace_launches: event %d is null", k);
      return GSPLAT_ERR_INVALID_ARGUMENT;
    }
    gs::g_trace_ev[k] = static_cast<hipEvent_t>(events[k]);
  }
  for (int k = 0; k < n; ++k) gs::g_trace_name[k] = nullptr;
  gs::g_trace_next.store(0, std::memory_order_relaxed);
  gs::g_trace_cap.store(n, std::memory_order_release);
  return GSPLAT_OK;
}

int gsplat_hip_trace_count(void) {
  const int cap = gs::g_trace_cap.load(std::memory_order_acquire);
  const int next = gs::g_trace_next.load(std::memory_order_relaxed);
  return next < cap ? next : cap;
}

const char* gsplat_hip_trace_name(int k) {
  if (k < 0 || k >= gsplat_hip_trace_count()) return nullptr;
  return gs::g_trace_name[k];
}

int gsplat_hip_time_next_launch(int which, void* start_event,
                                void* stop_event) {
  if (which != gs::kTimeForward && which != gs::kTimeBackward) {
    gs::set_error("gsplat_hip_time_next_launch: unknown launch %d", which);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  gs::set_launch_timing(which, static_cast<hipEvent_t>(start_event),
                        static_cast<hipEvent_t>(stop_event));
  return GSPLAT_OK;
}

}  // extern "C"

namespace {
// gsplat_hip_bin_count; with colors the count also writes the
// original-order records that bin_pack_impl copies (use_records).  A null
// pair_count skips the total (the one-call binning reports N from the pack
// scan instead, which computes the same value).
int bin_count_impl(const gsplat_raster_meta* meta, const float* means2d,
                   const float* conics, const float* opacities,
                   const float* colors, int32_t* pair_count, void* workspace,
                   size_t workspace_bytes, void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  rc = null_check({means2d, conics, opacities, workspace},
                  "gsplat_hip_bin_count");
  if (rc) return rc;
  const CountLayout L = count_layout(P);
  if (workspace_bytes < L.total) {
    gs::set_error("gsplat_hip_bin_count: workspace too small (%zu < %zu)",
                  workspace_bytes, L.total);
    return GSPLAT_ERR_WORKSPACE;
  }
  if (!gs::radix_size_ok(P.gpb, P.batch)) {
    gs::set_error("gsplat_hip_bin_count: too many splats per image");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(workspace);
  // Per-splat tile-hit counts and their total N; the same launch zeroes the
  // control words of the pack scan and the pair sort.
  const size_t z0 = gs::radix_ctl_bytes(L.depth);
  return gs::launch_count(P, means2d, conics, opacities,
                          reinterpret_cast<int32_t*>(base + L.splat_count),
                          pair_count != nullptr
                              ? reinterpret_cast<int32_t*>(base + L.block_sums)
                              : nullptr,
                          pair_count, reinterpret_cast<uint32_t*>(base + z0),
                          (int64_t)((L.ctl_end - z0) / sizeof(uint32_t)), s,
                          colors,
                          colors != nullptr
                              ? reinterpret_cast<float*>(base + L.rec_orig)
                              : nullptr,
                          colors != nullptr
                              ? reinterpret_cast<uint64_t*>(base + L.hit_bits)
                              : nullptr);
}
}  // namespace

extern "C" {

int gsplat_hip_bin_count(const gsplat_raster_meta* meta, const float* means2d,
                         const float* conics, const float* opacities,
                         int32_t* pair_count, void* workspace,
                         size_t workspace_bytes, void* stream) {
  const int rc = null_check({pair_count}, "gsplat_hip_bin_count");
  if (rc) return rc;
  return bin_count_impl(meta, means2d, conics, opacities, nullptr, pair_count,
                        workspace, workspace_bytes, stream);
}

int gsplat_hip_bin_depth_order(const gsplat_raster_meta* meta,
                               const float* depths, int32_t* perm,
                               void* workspace, size_t workspace_bytes,
                               void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  rc = null_check({depths, perm, workspace}, "gsplat_hip_bin_depth_order");
  if (rc) return rc;
  const CountLayout L = count_layout(P);
  if (workspace_bytes < L.total) {
    gs::set_error("gsplat_hip_bin_depth_order: workspace too small (%zu < %zu)",
                  workspace_bytes, L.total);
    return GSPLAT_ERR_WORKSPACE;
  }
  if (!gs::radix_size_ok(P.gpb, P.batch)) {
    gs::set_error("gsplat_hip_bin_depth_order: too many splats per image");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(workspace);
  // stable depth order per image: small images by run sort + merge ranks
  // (two launches), larger ones by the onesweep LSD over the 32 key bits
  if (gs::depth_small_ok(P.gpb))
    return gs::launch_depth_order_small(depths, perm, P.gpb, P.batch,
                                        base + L.depth_buffers, s);
  const gs::RadixCtl depth_ctl = gs::radix_ctl_at(L.depth, base);
  rc = gs::launch_zero_u32(reinterpret_cast<uint32_t*>(base),
                           (int64_t)(gs::radix_ctl_bytes(L.depth) / sizeof(uint32_t)), s);
  if (!rc) rc = gs::radix_global_hist(L.depth, depth_ctl, nullptr, depths, s);
  if (!rc)
    rc = gs::radix_passes(L.depth, depth_ctl, base + L.depth_buffers, nullptr,
                          nullptr, depths, nullptr,
                          reinterpret_cast<uint32_t*>(perm), s);
  return rc;
}

int gsplat_hip_pack_records(const gsplat_raster_meta* meta,
                            const float* means2d, const float* conics,
                            const float* colors, const float* opacities,
                            float* packed, void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  rc = null_check({means2d, conics, colors, opacities, packed},
                  "gsplat_hip_pack_records");
  if (rc) return rc;
  return gs::launch_pack_records(P, means2d, conics, colors, opacities, packed,
                                 static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {
// gsplat_hip_bin_pack; use_records: copy the count's original-order records
// (bin_count_impl with colors) instead of gathering the attributes, and
// write the original-order emit's offsets and gids.
int bin_pack_impl(const gsplat_raster_meta* meta, const float* means2d,
                  const float* conics, const float* colors,
                  const float* opacities, const int32_t* perm, float* packed,
                  int32_t* splat_offsets, void* workspace,
                  size_t workspace_bytes, void* stream, bool use_records) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  rc = null_check({means2d, conics, colors, opacities, perm, packed,
                   splat_offsets, workspace},
                  "gsplat_hip_bin_pack");
  if (rc) return rc;
  const CountLayout L = count_layout(P);
  if (workspace_bytes < L.total) {
    gs::set_error("gsplat_hip_bin_pack: workspace too small (%zu < %zu)",
                  workspace_bytes, L.total);
    return GSPLAT_ERR_WORKSPACE;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(workspace);
  // packed records in depth order and per-gid pair offsets
  rc = gs::launch_pack(P, means2d, conics, colors, opacities,
                         reinterpret_cast<const uint32_t*>(perm),
                         reinterpret_cast<const int32_t*>(base + L.splat_count),
                         packed, splat_offsets,
                         reinterpret_cast<uint64_t*>(base + L.scan_status),
                         reinterpret_cast<uint32_t*>(base + L.scan_ticket),
                         reinterpret_cast<uint32_t*>(base + L.scan_ticket) + 1,
                         s,
                         use_records
                             ? reinterpret_cast<const float*>(base + L.rec_orig)
                             : nullptr,
                         use_records
                             ? reinterpret_cast<int32_t*>(base + L.orig_slot)
                             : nullptr);
  return rc;
}
}  // namespace

extern "C" {

int gsplat_hip_bin_pack(const gsplat_raster_meta* meta, const float* means2d,
                        const float* conics, const float* colors,
                        const float* opacities, const int32_t* perm,
                        float* packed, int32_t* splat_offsets,
                        void* workspace, size_t workspace_bytes, void* stream) {
  return bin_pack_impl(meta, means2d, conics, colors, opacities, perm, packed,
                       splat_offsets, workspace, workspace_bytes, stream,
                       false);
}

size_t gsplat_hip_bin_emit_workspace_bytes(const gsplat_raster_meta* meta,
                                           int64_t n_pairs) {
  RasterParams P;
  if (make_params(meta, P) || n_pairs < 0) return 0;
  return emit_layout(P, n_pairs).total;
}

}  // extern "C"

namespace {
// bin_emit; with long_flag (a device word that is zero before the call) the
// tile range launch sets it to 1 if a tile range is longer than
// kHandoffPairs.
// The low tile bits of the one-pass-and-bucket form of the pair sort for
// buffers of n_pairs pairs (images of 2^9..2^16 tiles with at most
// kBucketChunk pairs per bucket on average), or -1 for the other forms.
int bucket_low_bits(const RasterParams& P, int64_t n_pairs) {
  const int tile_bits = bits_for((int64_t)P.num_tiles - 1);
  const int low_bits = tile_bits - 8;
  const int64_t buckets =
      low_bits > 0 ? (((int64_t)P.num_tiles + (1 << low_bits) - 1) >> low_bits)
                   : 0;
  return (low_bits >= 1 && tile_bits <= 16 &&
          n_pairs <= buckets * (int64_t)gs::kBucketChunk)
             ? low_bits
             : -1;
}

// hist_counted: the bucket form's histogram is already in the control block
// (counted by the count launch, summed by the rank launch).  orig_walk: the
// count wrote its records and step ballots and the pack the original-order
// offsets (bin_count_impl with colors, bin_pack_impl with use_records), so
// the emit walks in original order and reuses the ballots.
int bin_emit_impl(const gsplat_raster_meta* meta, const float* packed,
                  const int32_t* splat_offsets, int64_t n_pairs,
                  int32_t* binned_ids, int32_t* tile_counts,
                  int32_t* tile_offsets, int32_t* status,
                  void* count_workspace, size_t count_workspace_bytes,
                  void* workspace, size_t workspace_bytes, void* stream,
                  int32_t* long_flag, const gs::ZeroSpan* zero = nullptr,
                  const gs::EmitScanArgs* scan = nullptr,
                  bool hist_counted = false, bool orig_walk = false) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  if (n_pairs < 0 || n_pairs > 0x7fffffffLL) {
    gs::set_error("gsplat_hip_bin_emit: invalid pair count %lld",
                  (long long)n_pairs);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  rc = null_check({tile_offsets}, "gsplat_hip_bin_emit");
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // give-up status words of the binning's look-backs (pack scan, pair sort,
  // and the onesweep depth sort of large images)
  const CountLayout C = count_layout(P);
  char* cbase = static_cast<char*>(count_workspace);
  const uint32_t* err_pack =
      cbase ? reinterpret_cast<const uint32_t*>(cbase + C.scan_ticket) + 1 : nullptr;
  const uint32_t* err_pairs =
      cbase ? reinterpret_cast<const uint32_t*>(cbase + C.pair_tickets) + 4 : nullptr;
  const uint32_t* err_depth =
      (cbase && !gs::depth_small_ok(P.gpb)) ? gs::radix_ctl_at(C.depth, cbase).err : nullptr;
  if (n_pairs == 0 || P.num_splats == 0)
    return gs::launch_tile_ranges(nullptr, 0, P.num_tiles, tile_offsets,
                                  tile_counts, s, nullptr, err_pack, nullptr,
                                  err_depth, status, nullptr, zero);
  rc = null_check({packed, splat_offsets, binned_ids, count_workspace,
                   workspace},
                  "gsplat_hip_bin_emit");
  if (rc) return rc;
  const EmitLayout L = emit_layout(P, n_pairs);
  if (count_workspace_bytes < C.total || workspace_bytes < L.total) {
    gs::set_error("gsplat_hip_bin_emit: workspace too small (%zu < %zu or %zu < %zu)",
                  count_workspace_bytes, C.total, workspace_bytes, L.total);
    return GSPLAT_ERR_WORKSPACE;
  }
  if (!gs::radix_size_ok(n_pairs, 1)) {
    gs::set_error("gsplat_hip_bin_emit: too many pairs");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  char* base = static_cast<char*>(workspace);
  uint32_t* keys = reinterpret_cast<uint32_t*>(base + L.keys);
  uint32_t* vals = reinterpret_cast<uint32_t*>(base + L.vals);
  uint32_t* sorted_keys = reinterpret_cast<uint32_t*>(base + L.sorted_keys);
  const gs::RadixCtl ctl{reinterpret_cast<uint32_t*>(cbase + C.pair_ghist),
                         reinterpret_cast<uint32_t*>(base + L.status),
                         reinterpret_cast<uint32_t*>(cbase + C.pair_tickets),
                         reinterpret_cast<uint32_t*>(cbase + C.pair_tickets) + 4};
  // The pair count N is read on the device (splat_offsets[BG], written by
  // bin_pack); n_pairs is the capacity of the buffers and every stage takes
  // the first min(N, n_pairs) pairs.
  const int32_t* n_dev = splat_offsets + P.num_splats;
  const gs::EmitOrigArgs orig_args{
      reinterpret_cast<const float*>(cbase + C.rec_orig),
      reinterpret_cast<const int32_t*>(cbase + C.orig_slot),
      reinterpret_cast<const uint64_t*>(cbase + C.hit_bits)};
  const gs::EmitOrigArgs* orig =
      orig_walk && scan == nullptr ? &orig_args : nullptr;
  // Images of 2^9..2^16 tiles whose buffers hold at most kBucketChunk pairs
  // per bucket on average: the sort is one onesweep pass on the tile bits
  // above the low ones (bits - 8 of them: 2^(bits-8) tiles per bucket, at
  // most 256 buckets), then a counting sort per bucket that also writes the
  // tile ranges.
  const int tile_bits = bits_for((int64_t)P.num_tiles - 1);
  const int low_bits = bucket_low_bits(P, n_pairs);
  if (low_bits >= 1) {
    const gs::RadixPlan high = gs::radix_plan(n_pairs, 1, low_bits, tile_bits);
    uint32_t* high_vals =
        reinterpret_cast<uint32_t*>(base + L.buffers + L.pairs.a_vals);
    rc = gs::launch_emit(P, packed, splat_offsets, n_pairs, keys, vals,
                         hist_counted ? 0 : 1,
                         reinterpret_cast<uint32_t*>(base + L.hist), ctl.ghist,
                         ctl.status, L.pairs.status_words, s, scan, low_bits,
                         nullptr, orig);
    if (!rc)
      rc = gs::radix_passes(high, ctl, base + L.buffers, keys, vals, nullptr,
                            sorted_keys, high_vals, s, n_dev);
    if (!rc) {
      gs::BucketSortArgs A{};
      A.keys = sorted_keys;
      A.vals = high_vals;
      A.bucket_sizes = ctl.ghist;
      A.n = n_pairs;
      A.n_dev = n_dev;
      A.num_tiles = P.num_tiles;
      A.low_bits = low_bits;
      A.tile_offsets = tile_offsets;
      A.tile_counts = tile_counts;
      A.binned_ids = reinterpret_cast<uint32_t*>(binned_ids);
      A.err[0] = err_pack;
      A.err[1] = err_pairs;
      A.err[2] = err_depth;
      A.status_out = status;
      A.long_flag = long_flag;
      if (zero != nullptr) {
        A.zero[0] = zero[0];
        A.zero[1] = zero[1];
      }
      rc = gs::launch_bucket_sort(A, s);
    }
    return rc;
  }
  // 1. pairs at deterministic per-splat ranges + the sort's histograms;
  // 2-3. tiles below 2^16 and gids below 2^24: the emit writes the pairs as
  // words and low bytes (the sorted keys' buffer holds the bytes) for two
  // passes over packed words, the second of which writes the tile ranges
  // (the emit zeroes the sort's control words that must start at zero)
  if (gs::radix_pair_ranges_ok(L.pairs, P.num_splats)) {
    uint8_t* key_bytes = reinterpret_cast<uint8_t*>(sorted_keys);
    int64_t zero_words = 0;
    uint32_t* zero_span = gs::radix_pair_zero_span(L.pairs, ctl, &zero_words);
    // the emit counts the second pass's digits (the high tile bits) only:
    // the first pass's histogram comes from its block scan
    rc = gs::launch_emit(P, packed, splat_offsets, n_pairs, keys, vals, 1,
                         reinterpret_cast<uint32_t*>(base + L.hist),
                         ctl.ghist + 256, zero_span, zero_words, s, scan, 8,
                         key_bytes, orig);
    if (!rc)
      rc = gs::radix_pair_sort_ranges(
          L.pairs, ctl, base + L.buffers, key_bytes, keys,
          reinterpret_cast<uint32_t*>(binned_ids), tile_offsets, P.num_tiles,
          s, n_dev);
    if (!rc)
      rc = gs::launch_ranges_finish(n_pairs, P.num_tiles, tile_offsets,
                                    tile_counts, s, n_dev, err_pack,
                                    err_pairs, err_depth, status, long_flag,
                                    zero);
    return rc;
  }
  rc = gs::launch_emit(P, packed, splat_offsets, n_pairs, keys, vals,
                       L.pairs.passes,
                       reinterpret_cast<uint32_t*>(base + L.hist), ctl.ghist,
                       ctl.status, L.pairs.status_words, s, scan, 0, nullptr,
                       orig);
  // 2. stable sort by tile
  if (!rc)
    rc = gs::radix_passes(L.pairs, ctl, base + L.buffers, keys, vals, nullptr,
                          sorted_keys, reinterpret_cast<uint32_t*>(binned_ids),
                          s, n_dev);
  // 3. tile ranges and counts from the sorted keys, and the look-back status
  if (!rc)
    rc = gs::launch_tile_ranges(sorted_keys, n_pairs, P.num_tiles,
                                tile_offsets, tile_counts, s, n_dev, err_pack,
                                err_pairs, err_depth, status, long_flag,
                                zero);
  return rc;
}
}  // namespace

extern "C" {

int gsplat_hip_bin_emit(const gsplat_raster_meta* meta, const float* packed,
                        const int32_t* splat_offsets, int64_t n_pairs,
                        int32_t* binned_ids, int32_t* tile_counts,
                        int32_t* tile_offsets, int32_t* status,
                        void* count_workspace, size_t count_workspace_bytes,
                        void* workspace, size_t workspace_bytes,
                        void* stream) {
  return bin_emit_impl(meta, packed, splat_offsets, n_pairs, binned_ids,
                       tile_counts, tile_offsets, status, count_workspace,
                       count_workspace_bytes, workspace, workspace_bytes,
                       stream, nullptr, nullptr);
}

size_t gsplat_hip_bin_workspace_bytes(const gsplat_raster_meta* meta,
                                      int64_t capacity) {
  RasterParams P;
  if (make_params(meta, P) || capacity < 0) return 0;
  return 256 + gs::align_up(count_layout(P).total, 256) +
         emit_layout(P, capacity).total;
}

}  // extern "C"

namespace {
// Largest number of emit workgroups (128 splats each) of the small-image
// one-call binning: 4096 (524,288 splats in the batch), where an emit
// workgroup adds at most 4096 totals (16 per thread).
constexpr int kScanEmitMaxBlocks = 4096;

// gsplat_hip_bin; zero (may be null): two spans that the tile-range launch
// zeroes on the side (or a launch of their own where it does not run).
// With report_out the report of host_words is left to the caller's next
// launch (*report_out says what to copy) and status_event is not recorded;
// otherwise a launch of its own writes it.
int bin_impl(const gsplat_raster_meta* meta, const float* means2d,
             const float* conics, const float* colors, const float* opacities,
             const float* depths, int64_t capacity, int32_t* perm,
             float* packed, int32_t* splat_offsets, int32_t* binned_ids,
             int32_t* tile_offsets, int32_t* host_words, void* workspace,
             size_t workspace_bytes, void* stream, void* count_stream,
             void* inputs_event, void* count_event, void* status_event,
             const gs::ZeroSpan* zero, gs::HostReport* report_out) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  if (capacity < 0 || capacity > 0x7fffffffLL) {
    gs::set_error("gsplat_hip_bin: invalid capacity %lld", (long long)capacity);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  rc = null_check({means2d, conics, colors, opacities, depths, perm, packed,
                   splat_offsets, tile_offsets, workspace},
                  "gsplat_hip_bin");
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStream_t cs = count_stream ? static_cast<hipStream_t>(count_stream) : s;
  if (cs != s && (inputs_event == nullptr || count_event == nullptr)) {
    gs::set_error("gsplat_hip_bin: a count stream needs the events");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const size_t cbytes = gs::align_up(count_layout(P).total, 256);
  const size_t need = gsplat_hip_bin_workspace_bytes(meta, capacity);
  if (workspace_bytes < need) {
    gs::set_error("gsplat_hip_bin: workspace too small (%zu < %zu)",
                  workspace_bytes, need);
    return GSPLAT_ERR_WORKSPACE;
  }
  // host_words[3] turns 1 once host_words[0..2] hold the report
  if (host_words != nullptr) host_words[3] = 0;
  char* base = static_cast<char*>(workspace);
  // (header words: 0 unused, 1 the binning's status)
  int32_t* status_dev = reinterpret_cast<int32_t*>(base) + 1;
  void* cws = base + 256;
  // the long-range flag: a control word of the count workspace, zeroed by
  // the count launch like the pair sort's tickets
  int32_t* long_dev = reinterpret_cast<int32_t*>(
                          static_cast<char*>(cws) + count_layout(P).pair_tickets) +
                      8;
  // the report of host_words, after the tile ranges
  auto report = [&](const int32_t* n_src) -> int {
    const gs::HostReport R{n_src, status_dev, long_dev, host_words};
    int r = GSPLAT_OK;
    if (report_out != nullptr) {
      *report_out = R;
      return r;
    }
    r = gs::launch_host_report(R, s);
    if (!r && status_event != nullptr)
      r = hip_status(hipEventRecord(static_cast<hipEvent_t>(status_event), s),
                     "gsplat_hip_bin: event record");
    return r;
  };
  void* ews = base + 256 + cbytes;
  const size_t ebytes = workspace_bytes - 256 - cbytes;
  hipEvent_t ev_in = static_cast<hipEvent_t>(inputs_event);
  hipEvent_t ev_n = static_cast<hipEvent_t>(count_event);
  // Images of at most 131072 splats whose N goes to host_words: the count
  // and the run step of the depth order share one launch on `stream` (the
  // run step leaves most CUs idle), the rank step packs the records, and the
  // emit scans the pair offsets and writes N, which the tile-range launch
  // reports; the count stream, its events and the sum of the count
  // workgroups are not used.  Each emit workgroup there adds the totals of
  // all workgroups before it, work that grows with the square of their
  // count, so batches of more than kScanEmitMaxBlocks emit workgroups take
  // the look-back path below.
  if (host_words != nullptr && capacity > 0 && P.num_tiles > 0 &&
      P.num_splats > 0 && gs::depth_small_ok(P.gpb) &&
      gs::emit_blocks(P) <= kScanEmitMaxBlocks) {
    const CountLayout C = count_layout(P);
    char* cb = static_cast<char*>(cws);
    const size_t z0 = gs::radix_ctl_bytes(C.depth);
    // The bucket form's histogram is counted by the count blocks, which
    // finish well before the depth run step they share the launch with, and
    // summed by an extra rank workgroup; the emit's workgroups would
    // otherwise add it atomically, all at their end (cfg2: ~5 us of emit).
    gs::CountHist hist;
    const int low_bits = bucket_low_bits(P, capacity);
    if (low_bits >= 1) {
      hist.parts = reinterpret_cast<uint32_t*>(static_cast<char*>(ews) +
                                               emit_layout(P, capacity).hist);
      hist.shift = low_bits;
      hist.nparts = gs::count_depth_runs_blocks(P);
      hist.ghist = reinterpret_cast<uint32_t*>(cb + C.pair_ghist);
    }
    rc = gs::launch_count_depth_runs(
        P, means2d, conics, opacities,
        reinterpret_cast<int32_t*>(cb + C.splat_count),
        reinterpret_cast<uint32_t*>(cb + z0),
        (int64_t)((C.ctl_end - z0) / sizeof(uint32_t)), depths,
        cb + C.depth_buffers, s, hist);
    // ranks with the records packed at them, then the emit scans the pair
    // offsets itself
    int32_t* gid_count = reinterpret_cast<int32_t*>(cb + C.gid_count);
    // per emit workgroup totals (in the zeroed status words of the pack
    // scan, which this path does not run)
    uint32_t* block_totals = reinterpret_cast<uint32_t*>(cb + C.scan_status);
    if (!rc)
      rc = gs::launch_rank_pack(
          P, means2d, conics, colors, opacities, cb + C.depth_buffers,
          reinterpret_cast<const int32_t*>(cb + C.splat_count), perm, packed,
          gid_count, block_totals, s, hist);
    const gs::EmitScanArgs scan{gid_count, splat_offsets, block_totals};
    if (!rc)
      rc = bin_emit_impl(meta, packed, splat_offsets, capacity, binned_ids,
                         nullptr, tile_offsets, status_dev, cws, cbytes, ews,
                         ebytes, s, long_dev, zero, &scan, low_bits >= 1);
    // N is written by the emit's scan
    return rc ? rc : report(splat_offsets + P.num_splats);
  }
  // 1. per-splat hit counts on the count stream (after the caller's work on
  //    `stream`)
  if (cs != s) {
    rc = hip_status(hipEventRecord(ev_in, s), "gsplat_hip_bin: event record");
    if (!rc)
      rc = hip_status(hipStreamWaitEvent(cs, ev_in, 0),
                      "gsplat_hip_bin: stream wait");
    if (rc) return rc;
  }
  rc = bin_count_impl(meta, means2d, conics, opacities, colors, nullptr, cws,
                      cbytes, cs);
  if (!rc && ev_n != nullptr)
    rc = hip_status(hipEventRecord(ev_n, cs), "gsplat_hip_bin: event record");
  if (rc) return rc;
  // 2. stable depth order on `stream`, concurrently with the count
  rc = gsplat_hip_bin_depth_order(meta, depths, perm, cws, cbytes, s);
  if (rc) return rc;
  if (cs != s) {
    rc = hip_status(hipStreamWaitEvent(s, ev_n, 0),
                    "gsplat_hip_bin: stream wait");
    if (rc) return rc;
  }
  // 3. records and offsets, 4. pairs, pair sort, tile ranges and the
  //    look-back status (next to N in the workspace header)
  rc = bin_pack_impl(meta, means2d, conics, colors, opacities, perm, packed,
                     splat_offsets, cws, cbytes, s, true);
  if (rc) return rc;
  rc = bin_emit_impl(meta, packed, splat_offsets, capacity, binned_ids,
                     nullptr, tile_offsets, status_dev, cws, cbytes, ews,
                     ebytes, s, host_words != nullptr ? long_dev : nullptr,
                     zero, nullptr, false, true);
  if (rc || host_words == nullptr) return rc;
  // 5. N (from the pack scan), the status and the long-range flag to the host
  return report(splat_offsets + P.num_splats);
}

}  // namespace

extern "C" {

int gsplat_hip_bin(const gsplat_raster_meta* meta, const float* means2d,
                   const float* conics, const float* colors,
                   const float* opacities, const float* depths,
                   int64_t capacity, int32_t* perm, float* packed,
                   int32_t* splat_offsets, int32_t* binned_ids,
                   int32_t* tile_offsets, int32_t* host_words,
                   void* workspace, size_t workspace_bytes, void* stream,
                   void* count_stream, void* inputs_event,
                   void* count_event, void* status_event) {
  return bin_impl(meta, means2d, conics, colors, opacities, depths, capacity,
                  perm, packed, splat_offsets, binned_ids, tile_offsets,
                  host_words, workspace, workspace_bytes, stream, count_stream,
                  inputs_event, count_event, status_event, nullptr, nullptr);
}

}  // extern "C"

namespace {
// Arguments of the forward entry points (`what` names the entry in errors);
// `in_bin`: the binning's outputs are still to be written by the same call.
int check_forward(const RasterParams& P, const float* packed,
                  const int32_t* tile_offsets, const int32_t* binned_ids,
                  const float* out_rgb, const float* out_final_T,
                  const int32_t* out_last, const int32_t* out_tile_stop,
                  int64_t n_pairs, const void* workspace,
                  size_t workspace_bytes, const char* what) {
  int rc = null_check({packed, tile_offsets, out_rgb}, what);
  if (rc) return rc;
  (void)binned_ids;
  if ((out_final_T == nullptr) != (out_last == nullptr) ||
      (out_final_T == nullptr) != (out_tile_stop == nullptr)) {
    gs::set_error(
        "%s: out_final_T, out_last and out_tile_stop must all be given or all "
        "be NULL",
        what);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (n_pairs < 0) {
    gs::set_error("%s: invalid pair count %lld", what, (long long)n_pairs);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  // the eval forward (no state outputs) records no segments
  const int64_t ws_pairs = out_final_T != nullptr ? n_pairs : 0;
  if (workspace != nullptr &&
      workspace_bytes < gs::render_workspace_bytes(P, ws_pairs)) {
    gs::set_error("%s: workspace too small (%zu < %zu)", what,
                  workspace_bytes, gs::render_workspace_bytes(P, ws_pairs));
    return GSPLAT_ERR_WORKSPACE;
  }
  return GSPLAT_OK;
}
}  // namespace

extern "C" {

int gsplat_hip_render_forward(const gsplat_raster_meta* meta,
                              const float* packed, const int32_t* tile_offsets,
                              const int32_t* binned_ids, float* out_rgb,
                              float* out_final_T, int32_t* out_last,
                              int32_t* out_tile_stop, int64_t n_pairs,
                              void* workspace, size_t workspace_bytes,
                              void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (!rc)
    rc = check_forward(P, packed, tile_offsets, binned_ids, out_rgb,
                       out_final_T, out_last, out_tile_stop, n_pairs,
                       workspace, workspace_bytes, "gsplat_hip_render_forward");
  if (rc) return rc;
  return gs::launch_render_forward(P, packed, tile_offsets, binned_ids, out_rgb,
                                   out_final_T, out_last, out_tile_stop,
                                   n_pairs, workspace,
                                   static_cast<hipStream_t>(stream));
}

int gsplat_hip_render_forward_long(const gsplat_raster_meta* meta,
                                   const float* packed,
                                   const int32_t* tile_offsets,
                                   const int32_t* binned_ids, float* out_rgb,
                                   float* out_final_T, int32_t* out_last,
                                   int32_t* out_tile_stop, int64_t n_pairs,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (!rc)
    rc = check_forward(P, packed, tile_offsets, binned_ids, out_rgb,
                       out_final_T, out_last, out_tile_stop, n_pairs,
                       workspace, workspace_bytes,
                       "gsplat_hip_render_forward_long");
  if (rc) return rc;
  return gs::launch_render_forward_long(
      P, packed, tile_offsets, binned_ids, out_rgb, out_final_T, out_last,
      out_tile_stop, n_pairs, workspace, static_cast<hipStream_t>(stream));
}

int gsplat_hip_bin_render_forward(
    const gsplat_raster_meta* meta, const float* means2d, const float* conics,
    const float* colors, const float* opacities, const float* depths,
    int64_t capacity, int32_t* perm, float* packed, int32_t* splat_offsets,
    int32_t* binned_ids, int32_t* tile_offsets, int32_t* host_words,
    void* bin_workspace, size_t bin_workspace_bytes, float* out_rgb,
    float* out_final_T, int32_t* out_last, int32_t* out_tile_stop,
    void* render_workspace, size_t render_workspace_bytes, void* stream,
    void* count_stream, void* inputs_event, void* count_event,
    void* status_event) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (!rc)
    rc = null_check({host_words, render_workspace},
                    "gsplat_hip_bin_render_forward");
  if (!rc)
    rc = check_forward(P, packed, tile_offsets, binned_ids, out_rgb,
                       out_final_T, out_last, out_tile_stop, capacity,
                       render_workspace, render_workspace_bytes,
                       "gsplat_hip_bin_render_forward");
  if (rc) return rc;
  // The tile-range launch zeroes what the forward needs zero (hand-off
  // counters, gradient records), so the forward follows it directly.
  gs::ZeroSpan zero[2];
  gs::render_forward_zero_spans(P, capacity, render_workspace,
                                out_final_T != nullptr, zero);
  // The forward's first workgroup writes the binning's report to
  // host_words as it starts; status_event follows the forward.
  gs::HostReport report{};
  rc = bin_impl(meta, means2d, conics, colors, opacities, depths, capacity,
                perm, packed, splat_offsets, binned_ids, tile_offsets,
                host_words, bin_workspace, bin_workspace_bytes, stream,
                count_stream, inputs_event, count_event, nullptr, zero,
                &report);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = gs::launch_render_forward(P, packed, tile_offsets, binned_ids, out_rgb,
                                 out_final_T, out_last, out_tile_stop,
                                 capacity, render_workspace, s,
                                 gs::kForwardPreZeroed | gs::kForwardNoLong |
                                     gs::kForwardStoppedLast,
                                 &report);
  if (!rc && status_event != nullptr)
    rc = hip_status(hipEventRecord(static_cast<hipEvent_t>(status_event), s),
                    "gsplat_hip_bin_render_forward: event record");
  return rc;
}

size_t gsplat_hip_render_workspace_bytes(const gsplat_raster_meta* meta,
                                         int64_t n_pairs) {
  RasterParams P;
  if (make_params(meta, P) || n_pairs < 0) return 0;
  return gs::render_workspace_bytes(P, n_pairs);
}

int gsplat_hip_render_backward(const gsplat_raster_meta* meta,
                               const float* packed,
                               const int32_t* tile_offsets,
                               const int32_t* binned_ids,
                               const float* final_T, const int32_t* last,
                               const int32_t* tile_stop, const float* grad_rgb,
                               float* g_means2d, float* g_conics,
                               float* g_colors, float* g_opacities,
                               int64_t n_pairs, void* workspace,
                               size_t workspace_bytes, void* stream) {
  RasterParams P;
  int rc = make_params(meta, P);
  if (rc) return rc;
  rc = null_check({packed, tile_offsets, final_T, last, tile_stop, grad_rgb,
                   g_means2d, g_conics, g_colors, g_opacities},
                  "gsplat_hip_render_backward");
  if (rc) return rc;
  if (n_pairs < 0) {
    gs::set_error("gsplat_hip_render_backward: invalid pair count %lld",
                  (long long)n_pairs);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (workspace != nullptr &&
      workspace_bytes < gs::render_workspace_bytes(P, n_pairs)) {
    gs::set_error("gsplat_hip_render_backward: workspace too small (%zu < %zu)",
                  workspace_bytes, gs::render_workspace_bytes(P, n_pairs));
    return GSPLAT_ERR_WORKSPACE;
  }
  return gs::launch_render_backward(P, packed, tile_offsets, binned_ids,
                                    final_T, last, tile_stop, grad_rgb,
                                    g_means2d, g_conics, g_colors, g_opacities,
                                    n_pairs, workspace,
                                    static_cast<hipStream_t>(stream));
}

static int make_project_params(const gsplat_project_meta* m,
                               gs::ProjectParams& P) {
  if (m == nullptr || m->batch <= 0 || m->gaussians_per_batch <= 0) {
    gs::set_error("project meta: batch and gaussians_per_batch must be > 0");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int64_t BG = (int64_t)m->batch * m->gaussians_per_batch;
  if (BG > kMaxSplats) {
    gs::set_error("project meta: too many splats (%lld)", (long long)BG);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  P.batch = m->batch;
  P.gpb = m->gaussians_per_batch;
  P.num_splats = (int)BG;
  P.near_plane = m->near_plane;
  return GSPLAT_OK;
}

int gsplat_hip_project_forward(const gsplat_project_meta* meta,
                               const float* means3d, const float* scales,
                               const float* quats, const float* opacities,
                               const float* camera_to_world,
                               const float* camera_params, float* out_means2d,
                               float* out_conics, float* out_opacities,
                               float* out_depths, void* stream) {
  gs::ProjectParams P;
  int rc = make_project_params(meta, P);
  if (rc) return rc;
  rc = null_check({means3d, scales, quats, opacities, camera_to_world,
                   camera_params, out_means2d, out_conics, out_opacities,
                   out_depths},
                  "gsplat_hip_project_forward");
  if (rc) return rc;
  return gs::launch_project_forward(P, means3d, scales, quats, opacities,
                                    camera_to_world, camera_params,
                                    out_means2d, out_conics, out_opacities,
                                    out_depths,
                                    static_cast<hipStream_t>(stream));
}

int gsplat_hip_project_backward(
    const gsplat_project_meta* meta, const float* grad_means2d,
    const float* grad_conics, const float* grad_opacities,
    const float* grad_depths, const float* means3d, const float* scales,
    const float* quats, const float* opacities, const float* camera_to_world,
    const float* camera_params, float* g_means3d, float* g_scales,
    float* g_quats, float* g_opacities, float* g_camera_to_world,
    float* g_camera_params, void* workspace, size_t workspace_bytes,
    void* stream) {
  gs::ProjectParams P;
  int rc = make_project_params(meta, P);
  if (rc) return rc;
  // (grad_depths may be null: a zero depth gradient)
  rc = null_check({grad_means2d, grad_conics, grad_opacities, means3d, scales,
                   quats, opacities, camera_to_world, camera_params, g_means3d,
                   g_scales, g_quats, g_opacities, g_camera_to_world,
                   g_camera_params, workspace},
                  "gsplat_hip_project_backward");
  if (rc) return rc;
  if (workspace_bytes < gs::project_backward_workspace_bytes(P)) {
    gs::set_error("gsplat_hip_project_backward: workspace too small (%zu < %zu)",
                  workspace_bytes, gs::project_backward_workspace_bytes(P));
    return GSPLAT_ERR_WORKSPACE;
  }
  return gs::launch_project_backward(
      P, grad_means2d, grad_conics, grad_opacities, grad_depths, means3d,
      scales, quats, opacities, camera_to_world, camera_params, g_means3d,
      g_scales, g_quats, g_opacities, g_camera_to_world, g_camera_params,
      workspace, static_cast<hipStream_t>(stream));
}

int gsplat_hip_project_backward_noalloc(
    const gsplat_project_meta* meta, const float* grad_means2d,
    const float* grad_conics, const float* grad_opacities,
    const float* grad_depths, const float* means3d, const float* scales,
    const float* quats, const float* opacities, const float* camera_to_world,
    const float* camera_params, float* g_means3d, float* g_scales,
    float* g_quats, float* g_opacities, float* g_camera_to_world,
    float* g_camera_params, void* stream) {
  gs::ProjectParams P;
  int rc = make_project_params(meta, P);
  if (rc) return rc;
  rc = null_check({grad_means2d, grad_conics, grad_opacities, means3d, scales,
                   quats, opacities, camera_to_world, camera_params, g_means3d,
                   g_scales, g_quats, g_opacities, g_camera_to_world,
                   g_camera_params},
                  "gsplat_hip_project_backward_noalloc");
  if (rc) return rc;
  const size_t need = gs::project_backward_workspace_bytes(P);
  if (need > GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES) {
    gs::set_error(
        "gsplat_hip_project_backward_noalloc: B * ceil(G/256) * 64 bytes = %zu "
        "exceeds the static scratch of %d bytes (B * ceil(G/256) <= %d); use "
        "gsplat_hip_project_backward with a workspace",
        need, GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES,
        GSPLAT_PROJECT_NOALLOC_SCRATCH_BYTES / 64);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* scratch = nullptr;
  rc = gs::project_noalloc_scratch(s, &scratch);
  if (rc) return rc;
  return gs::launch_project_backward(
      P, grad_means2d, grad_conics, grad_opacities, grad_depths, means3d,
      scales, quats, opacities, camera_to_world, camera_params, g_means3d,
      g_scales, g_quats, g_opacities, g_camera_to_world, g_camera_params,
      scratch, s);
}

size_t gsplat_hip_project_backward_workspace_bytes(
    const gsplat_project_meta* meta) {
  gs::ProjectParams P;
  if (make_project_params(meta, P)) return 0;
  return gs::project_backward_workspace_bytes(P);
}

size_t gsplat_hip_scan_workspace_bytes(int64_t n) {
  return gs::scan_workspace_bytes(n);
}

int gsplat_hip_exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n,
                                  int32_t* status, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (n > 0x7fffffffLL) {
    gs::set_error("exclusive_scan: n too large");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  // An empty input may come with a NULL pointer; out always receives out[0].
  int rc = null_check({n > 0 ? in : out, out}, "gsplat_hip_exclusive_scan_i32");
  if (rc) return rc;
  return gs::exclusive_scan_i32(in, out, n, workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream), false,
                                status);
}

int gsplat_hip_debug_stalled_scan(const int32_t* in, int32_t* out, int64_t n,
                                  int32_t stalled_blocks, int32_t spin_limit,
                                  int32_t* status, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  const int64_t blocks = n <= 0 ? 1 : (n + 4095) / 4096;
  if (n <= 0 || n > 0x7fffffffLL || stalled_blocks < 0 ||
      stalled_blocks >= blocks || spin_limit < 0) {
    gs::set_error("gsplat_hip_debug_stalled_scan: need 0 < n, 0 <= "
                  "stalled_blocks < %lld blocks, spin_limit >= 0",
                  (long long)blocks);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  int rc = null_check({in, out, status}, "gsplat_hip_debug_stalled_scan");
  if (rc) return rc;
  return gs::exclusive_scan_i32(in, out, n, workspace, workspace_bytes,
                                static_cast<hipStream_t>(stream), false,
                                status, stalled_blocks, spin_limit);
}

size_t gsplat_hip_radix_sort_workspace_bytes(int64_t n_per_segment,
                                             int32_t segments) {
  return gs::radix_sort_workspace_bytes(n_per_segment, segments);
}

int gsplat_hip_radix_sort_pairs_u32(const uint32_t* keys_in,
                                    const uint32_t* vals_in,
                                    uint32_t* keys_out, uint32_t* vals_out,
                                    int64_t n_per_segment, int32_t segments,
                                    int32_t begin_bit, int32_t end_bit,
                                    int32_t* status, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return gs::radix_sort_pairs(keys_in, vals_in, nullptr, keys_out, vals_out,
                              n_per_segment, segments, begin_bit, end_bit,
                              workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream), status);
}

}  // extern "C"
