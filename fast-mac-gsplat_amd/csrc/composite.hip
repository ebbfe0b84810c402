// composite.hip -- per-tile front-to-back compositor (forward) and its
// reverse-order adjoint (backward).
//
// Work decomposition (gfx950): one 64-lane workgroup (= one wavefront) per
// 16x16 tile.  Slot k = 0..3 is the strip of tile rows 4k..4k+3 and lane l
// owns pixel (l%16, 4k + l/16) of every strip, so the four pixels of a lane
// share their x coordinate (and the x-only part of the Gaussian exponent),
// every splat record is read once per wave and reused for four pixels, and no
// barrier spans more than one wavefront.  Splat records of the tile's range
// are staged 64 at a time in LDS (each lane gathers one 64-byte record and
// derives the per-tile constants) and read by all lanes as broadcasts.  A
// strip is skipped (scalar branch on a per-record bit mask) when the
// splat's support ellipse, enlarged by a safety margin, spans no row of the
// strip inside the tile's columns, so no pixel that could pass the alpha
// test is ever skipped; the record carries the splat's part of that test
// (gs_strip.h), so a lane only clamps and compares per tile.
//
// Alpha test (reference eval_alpha, variants/v8/csrc/metal/gsplat_v8_kernels.metal:121-139):
// the exponent is evaluated in base 2, by the fixed rounding chain
//   A = (-a/2)*L, B = (-b)*L, C = (-c/2)*L  (L = log2(e) rounded to float),
//   t = fma(C, dy, B*dx),  e = fma(t, dy, (A*dx)*dx)         (L * power),
//   p = fma(t, dy, (A*dx)*dx + lo)                 (L * power + log2(o)),
// where lo = L * ln(o) and plim, the base-2 exponent at which o * 2^power
// equals the alpha threshold, come with the packed record from binning.  A
// pixel sees the splat iff e <= 0 and p >= q = plim + lo.  Both decisions are
// therefore exact functions of the inputs that the CPU oracle reproduces:
// exact for this base-2 form.  The reference's own form, min(max_alpha,
// o*exp(power)) >= threshold with power rounded in another order, decides
// the same way except where alpha lies within a few ulps of the threshold
// (a handful of pixels per 4K image).  alpha = min(max_alpha, 2^p) with the
// hardware exp2 (within 1 ulp).
//
// Forward (reference tile_fast_forward_state, gsplat_v8_kernels.metal:400-476):
//   C += T*alpha*c; T *= 1-alpha; a pixel stops after the splat that brings
//   T <= transmittance_threshold.  Saves per pixel the final T and last, the
//   reference's local_stop (:455-467): 1 + index of the splat that stopped
//   the pixel, or the tile's pair count if it never stops.  The walk records
//   the index of every blend, so a stopped pixel holds that of its stopping
//   splat; pixels still alive at the end get the pair count.  Per tile the
//   max of last (the stop count), so the backward pass needs no forward
//   replay.
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
// wavefront: eight through LDS (each group of eight lanes sums one value's 64
// partials, then three DPP steps; the group's first lane issues the float
// atomic into the original splat order) and the ninth by DPP row steps.
#include <hip/hip_ext.h>

#include "gs_internal.h"
#include "gs_predicate.h"
#define GS_HD __device__ __forceinline__
#include "gs_strip.h"

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

// This lane's index (workgroups of one wavefront), recomputed where it is
// used instead of kept in a register across the walk: the forward's
// register budget spills whatever long-lived value it cannot hold, and each
// wave's spill store and reload went through the caches to HBM (~45 MB more
// writes per launch at 4096^2).
__device__ __forceinline__ int lane_now() {
  int v;
  asm volatile(
      "v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0"
      : "=v"(v));
  return v;
}

// s2 first: the forward reads only its x and z (one ds_read2 whose 8-bit
// dword offsets reach it from the batch's base address without an add).
struct Staged {
  float4 s2[kBatch];  // blue, orig index bits, q, strip mask bits or 1/o
  float4 s0[kBatch];  // mx, my, A, B
  float4 s1[kBatch];  // C, lo, r, g
};

// A value through an empty asm: addresses derived from it are computed
// where they are used, so that the compiler does not keep 64-bit addresses
// for the rare segment boundaries live across the compositing loop.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
// The same for a 64-bit pixel index: the other pixels of a lane are then
// reached by adding multiples of a row stride instead of a full 64-bit
// index computation each.
__device__ __forceinline__ int64_t opaque64(int64_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Strip culling (gs_strip.h) with the hardware square root.
struct HwOps {
  static __device__ __forceinline__ float sqrt(float x) {
    return __builtin_amdgcn_sqrtf(x);
  }
};

// Mask bit of a "plain" record (plain_record of gs_strip.h, flagged by
// binning in bit 31 of the record's orig word): for it the compositors'
// tests e <= 0 and 2^p < max_alpha always hold, so they are left out (same
// results, fewer VALU operations per pixel).  Set only together with a
// strip bit.
constexpr uint32_t kPlainBit = 1u << 4;

// Stages records [first, first+n) of the tile range into LDS with the
// base-2 exponent coefficients and the tile's strip mask (plus kPlainBit).
// Returns this lane's strip mask (0 for lanes past n).  With kMaskInLds the
// mask also goes to s2.w (kernels whose other wavefronts read it); otherwise
// s2.w holds 1 / opacity and the wavefront reads each record's mask from
// the returning lane with readlane.
template <bool kMaskInLds>
__device__ __forceinline__ uint32_t stage_batch(
    const float4* __restrict__ packed, const int32_t* __restrict__ binned,
    int first, int n, const TileCoord& tc, uint32_t max_gid, Staged& S) {
  const int lane = threadIdx.x;
  uint32_t m = 0u;
  if (lane < n) {
    // (clamped: a corrupt pair list cannot make the gather leave the records)
    const uint32_t gid = min((uint32_t)binned[first + lane], max_gid);
    const float4* r = packed + (uint64_t)kRecordVec4 * gid;
    const float4 p0 = r[0];
    const float4 p1 = r[1];
    const float4 p2 = r[2];
    const float4 p3 = r[3];
    // (the tile corner through opaque(): computed here per batch rather than
    // kept live in registers across the walk)
    m = strip_mask_t<HwOps>(StripConsts{p3.x, p3.y, p3.z, p3.w}, p0.x, p0.y,
                            opaque(tc.x0), opaque(tc.y0));
    const uint32_t ob = __float_as_uint(p2.y);
    if (m != 0u && (int32_t)ob < 0) m |= kPlainBit;
    float A, B, C;
    {
#pragma clang fp contract(off)
      A = (-0.5f * p0.z) * kLog2e;
      B = (-p0.w) * kLog2e;
      C = (-0.5f * p1.x) * kLog2e;
    }
    S.s0[lane] = make_float4(p0.x, p0.y, A, B);
    S.s1[lane] = make_float4(C, p2.w, p1.z, p1.w);
    S.s2[lane] = make_float4(
        p2.x, __uint_as_float(ob & 0x7fffffffu), p2.z,
        kMaskInLds ? __uint_as_float(m) : __builtin_amdgcn_rcpf(p1.y));
  }
  return m;
}

// The x-only parts of the exponents, once per splat and lane: a0 = (A dx) dx,
// a = a0 + lo, b = B dx.
struct XTerms {
  float a0, a, b;
};
__device__ __forceinline__ XTerms x_terms(float A, float B, float dx,
                                          float lo) {
#pragma clang fp contract(off)
  XTerms X;
  X.a0 = (A * dx) * dx;
  X.a = X.a0 + lo;
  X.b = B * dx;
  return X;
}

// One pixel's exponents, Horner in dy (after dy two fmas, a third for the
// power <= 0 test): t = fma(C, dy, B dx), p = fma(t, dy, a), e = fma(t, dy,
// a0).  Contraction stays off so the chain of roundings is exactly the one
// the CPU oracle evaluates.
struct Exponents {
  float t, p;
};
__device__ __forceinline__ Exponents exponents(const XTerms& X, float C,
                                               float dy) {
#pragma clang fp contract(off)
  Exponents E;
  E.t = __builtin_fmaf(C, dy, X.b);
  E.p = __builtin_fmaf(E.t, dy, X.a);
  return E;
}
// e <= 0: power <= 0 (the reference's test; always true for plain records)
__device__ __forceinline__ bool power_nonpositive(const Exponents& E,
                                                  const XTerms& X, float dy) {
#pragma clang fp contract(off)
  return __builtin_fmaf(E.t, dy, X.a0) <= 0.0f;
}

__device__ __forceinline__ uint32_t uniform_bits(float v) {
  return __builtin_amdgcn_readfirstlane(__float_as_uint(v));
}

// Maximum of a non-negative int over the 64 lanes, valid in lanes 48..63:
// DPP steps within each 16-lane row (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror), then row_bcast:15 and row_bcast:31 carry the
// row maxima upward (lanes outside a step's rows read 0).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_src_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ int wave_max_row3(int x) {
  x = max(x, dpp_src_i<0xB1>(x));
  x = max(x, dpp_src_i<0x4E>(x));
  x = max(x, dpp_src_i<0x141>(x));
  x = max(x, dpp_src_i<0x140>(x));
  x = max(x, dpp_src_i<0x142, 0xA>(x));
  x = max(x, dpp_src_i<0x143, 0xC>(x));
  return x;
}

// Long tiles.  A tile range is cut into segments of kSegSplats splats and
// colour is summed per segment: at each segment boundary a pixel's colour
// accumulators are added into its output pixel (which holds the sum of the
// completed segments; each lane reads back only what it wrote itself) and
// restart at zero.  The order of the additions depends on the tile range
// alone, so every variant of the forward gives the same image.
//
// With a workspace the forward also
//  * hands a tile that still has live pixels after kHandoff splats to
//    render_fwd_long_kernel, where four wavefronts (one per strip) continue
//    it from the saved state (T in the workspace, last in out_last, the
//    colour sum in the output), so a long tile no longer serialises one
//    wavefront;
//  * with the state outputs (training), records every segment of a tile
//    whose walk crosses a boundary: rec = (colour composited by the segment,
//    T at its end) per pixel, in a slot linked into the tile's chain.
// The backward then walks the segments of a tile whose stop exceeds one
// segment in parallel: the gT of the reverse recurrence at the end of
// segment k is
//   gT_k = (<g, sum_{j>k} colour_j> + <g, bg> T_final) / T_end_k,
// the closed form of gT <- alpha <g,c> + (1 - alpha) gT over the later
// splats, and T at its end is recorded.
constexpr int kSegSplats = 128;     // multiple of kBatch
constexpr int kHandoff = kHandoffPairs;  // multiple of kSegSplats
static_assert(kHandoff % kSegSplats == 0, "hand-off at a segment boundary");
constexpr int kLongStrips = 1;      // strips per wavefront of the long kernel

struct HeavyState {      // all null: every tile is walked whole by one wave
  int32_t* counters;     // [0] slots handed out, [1] tiles handed off
                         // (zeroed by the forward), [2] max_slots of the
                         // forward that recorded segments (-1: none)
  int32_t* tile_slot;    // [T] slot of segment 0, -1: no usable chain
  int32_t* slot_tile;    // [max_slots] tile of each slot
  int32_t* slot_seg;     // [max_slots] segment index of each slot
  int32_t* slot_next;    // [max_slots] slot of the next segment, -1: none
  int32_t* handoff;      // [T] tiles handed to render_fwd_long_kernel
  int32_t* handoff_tail; // [T] their chain's last slot, -2: chain broken
  float* hand_T;         // [T][256] T of each pixel at the hand-off
  float4* rec;           // [max_slots][256] (r, g, b, T at segment end);
                         // null: no records (forward without state)
  float* acc;            // [num_splats][kAccFloats] gradient sums of the
                         // backward (zero outside a backward: the training
                         // forward zeroes them and the backward's unpack
                         // leaves them zero); null with n_pairs = 0
  int max_slots;
};

// One lane per tile: the slot for segment `seg` of `tile`, linked after the
// chain tail `tail` (-1 before segment 0, -2 once broken); -1 if no record
// is kept.  When the workspace is full the chain breaks for good and
// tile_slot is cleared, so the backward walks that tile whole.
__device__ int next_segment(const HeavyState& H, int tile, int seg,
                            int& tail) {
  if (H.rec == nullptr || tail == -2) return -1;
  const int s = atomicAdd(H.counters, 1);
  if (s >= H.max_slots) {
    H.tile_slot[tile] = -1;
    tail = -2;
    return -1;
  }
  H.slot_tile[s] = tile;
  H.slot_seg[s] = seg;
  H.slot_next[s] = -1;
  if (tail < 0)
    H.tile_slot[tile] = s;
  else
    H.slot_next[tail] = s;
  tail = s;
  return s;
}

// Pixel index inside the tile used by the per-pixel segment records.
__device__ __forceinline__ int tile_pixel(int k) {
  return 64 * k + (int)threadIdx.x;
}

// t0 below is the in-tile index (tile_pixel order, 64 strip + lane) of this
// thread's pixel in the first strip it walks; its further strips follow at
// +64 (four rows down).

// Image index of pixel t0 of the tile.
__device__ __forceinline__ int64_t pixel_index(const RasterParams& P,
                                               const TileCoord& tc, int t0) {
  const int t = opaque(t0);
  const int y = tc.y0 + (t >> 4);
  const int x = tc.x0 + (t & 15);
  return ((int64_t)tc.batch * P.height + y) * P.width + x;
}

// Segment record entry of pixel t0 (null if no record is kept).
__device__ __forceinline__ float4* record_at(const HeavyState& H, int slot,
                                             int t0) {
  return slot >= 0 ? H.rec + (int64_t)slot * 256 + opaque(t0) : nullptr;
}

// End of segment `seg` for NP strips per thread: record it in `slot`
// (if >= 0) and fold its colour into the output pixels.
template <int NP>
__device__ __forceinline__ void end_segment(const RasterParams& P,
                                            const TileCoord& tc,
                                            float* out_rgb,
                                            const HeavyState& H, int slot,
                                            int seg, const bool* valid,
                                            float* cr, float* cg, float* cb,
                                            const float* T, int t0) {
  float* o0 = out_rgb + 3 * pixel_index(P, tc, t0);
  float4* r0 = record_at(H, slot, t0);
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    if (r0 != nullptr) r0[64 * k] = make_float4(cr[k], cg[k], cb[k], T[k]);
    if (valid[k]) {
      float* o = o0 + (int64_t)12 * k * P.width;
      if (seg > 0) {
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
}

// Last segment of a walk that crossed a boundary: record it and add the
// completed segments' colour (held in the output pixels) to the
// accumulators.
template <int NP>
__device__ __forceinline__ void last_segment(const RasterParams& P,
                                             const TileCoord& tc,
                                             const float* out_rgb,
                                             const HeavyState& H, int slot,
                                             const bool* valid, float* cr,
                                             float* cg, float* cb,
                                             const float* T, int t0) {
  const float* o0 = out_rgb + 3 * pixel_index(P, tc, t0);
  float4* r0 = record_at(H, slot, t0);
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    if (r0 != nullptr) r0[64 * k] = make_float4(cr[k], cg[k], cb[k], T[k]);
    if (valid[k]) {
      const float* o = o0 + (int64_t)12 * k * P.width;
      cr[k] += o[0];
      cg[k] += o[1];
      cb[k] += o[2];
    }
  }
}

// Front-to-back compositing of splat j of the staged batch into one pixel
// (kPlain: a record with kPlainBit, whose e <= 0 test and clamp never act).
template <bool kPlain>
__device__ __forceinline__ void composite_one(const XTerms& X,
                                              const float4& a1,
                                              const float4& a2, float py,
                                              float my, float t_thr,
                                              float max_alpha, int idx1,
                                              float& T, float& cr, float& cg,
                                              float& cb, int& last) {
  // One combined test (alive and visible): pixels rarely die inside a
  // batch, so guarding the exponent by T would save little and cost a
  // second branch.
  const float dy = py - my;
  const Exponents E = exponents(X, a1.x, dy);
  if ((T > t_thr) & (kPlain || power_nonpositive(E, X, dy)) & (E.p >= a2.z)) {
    // min(max_alpha, 2^p) as one med3: 2^p >= 0, so the lower bound 0 never
    // changes the result.
    const float raw = __builtin_amdgcn_exp2f(E.p);
    const float alpha =
        kPlain ? raw : __builtin_amdgcn_fmed3f(raw, 0.0f, max_alpha);
    const float w = T * alpha;
    cr += w * a1.z;
    cg += w * a1.w;
    cb += w * a2.x;
    T *= (1.0f - alpha);
    last = idx1;
  }
}

// True when every record of the staged batch that reaches a strip carries
// kPlainBit (m: the staging lane's mask), so the batch is composited without
// the e <= 0 test and the max_alpha clamp.
__device__ __forceinline__ bool batch_plain(uint32_t m) {
  return __builtin_amdgcn_ballot_w64((m != 0u) & !(m & kPlainBit)) == 0;
}

// Front-to-back compositing of the n staged records of one batch into the
// lane's kPix pixels (idx1: 1 + tile index of record 0).
template <bool kPlain>
__device__ __forceinline__ void fwd_batch(const Staged& S, uint32_t bmask,
                                          int n, int idx1, float px,
                                          const float* py, float t_thr,
                                          float max_alpha, float* T, float* cr,
                                          float* cg, float* cb, int* last) {
  for (int j = 0; j < n; ++j) {
    const uint32_t mask = __builtin_amdgcn_readlane(bmask, j);
    if (mask == 0u) continue;
    const float4 a2 = S.s2[j];
    const float4 a0 = S.s0[j];
    const float4 a1 = S.s1[j];
    const XTerms xt = x_terms(a0.z, a0.w, px - a0.x, a1.y);
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
      if (!((mask >> k) & 1u)) continue;  // scalar branch
      composite_one<kPlain>(xt, a1, a2, py[k], a0.y, t_thr, max_alpha,
                            idx1 + j, T[k], cr[k], cg[k], cb[k], last[k]);
    }
  }
}

// Eight wavefronts per SIMD (at most 64 VGPRs): the walk is bound by the
// latency of each wavefront's loads and LDS round trips, so more resident
// wavefronts shorten it (7% at 1860 pairs per tile).  all_last: out_last
// for every tile, else only for the tiles where a pixel stopped
// (T <= threshold; the others composited their whole tile range, and the
// backward reads last only where a pixel stopped).
__global__ __launch_bounds__(kLanes) __attribute__((amdgpu_waves_per_eu(8, 8)))
void render_fwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, float* __restrict__ out_rgb,
    float* __restrict__ out_T, int32_t* __restrict__ out_last,
    int32_t* __restrict__ out_tile_stop, HeavyState H, HostReport R,
    bool all_last) {
  __shared__ Staged S;
  // The binning's report reaches the host as the forward starts.
  if (R.host != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    write_host_report(R);
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
  if (H.rec != nullptr && threadIdx.x == 0) H.tile_slot[tc.tile] = -1;
  // The workspace's layout follows n_pairs: the backward uses the segment
  // records only if it was given the same n_pairs (same max_slots).
  if (H.counters != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    H.counters[2] = H.rec != nullptr ? H.max_slots : -1;
  // With a workspace a tile longer than kHandoff is walked here only up to
  // kHandoff, so segment boundaries inside this loop (and records) occur
  // only without a workspace.
  const int walk_end =
      (H.counters != nullptr && end - start > kHandoff) ? start + kHandoff : end;
  int seg_cur = 0;  // segment of the batch being composited
  for (int base = start; base < walk_end; base += kBatch) {
    const bool any_alive = (T[0] > t_thr) | (T[1] > t_thr) | (T[2] > t_thr) |
                           (T[3] > t_thr);
    if (!__any(any_alive)) break;
    if (base > start && (base - start) % kSegSplats == 0) {
      end_segment<kPix>(P, tc, out_rgb, H, -1, seg_cur, valid, cr, cg, cb, T,
                        (int)threadIdx.x);
      ++seg_cur;
    }
    const int n = min(kBatch, end - base);
    __syncthreads();
    const uint32_t bmask =
        stage_batch<false>(packed, binned, base, n, tc,
                           (uint32_t)P.num_splats - 1u, S);
    __syncthreads();
    if (batch_plain(bmask))
      fwd_batch<true>(S, bmask, n, base - start + 1, px, py, t_thr, max_alpha,
                      T, cr, cg, cb, last);
    else
      fwd_batch<false>(S, bmask, n, base - start + 1, px, py, t_thr,
                       max_alpha, T, cr, cg, cb, last);
  }
  if (walk_end < end) {
    const bool any_alive = (T[0] > t_thr) | (T[1] > t_thr) | (T[2] > t_thr) |
                           (T[3] > t_thr);
    if (__any(any_alive)) {
      // Close segment 0 and hand the rest of the tile to the four-wavefront
      // kernel: T to the workspace, last (of the blends so far) to out_last,
      // the colour sum is in the output.
      int tail = -1, slot = -1;  // chain state, meaningful in lane 0
      if (threadIdx.x == 0) slot = next_segment(H, tc.tile, 0, tail);
      slot = __shfl(slot, 0, 64);
      end_segment<kPix>(P, tc, out_rgb, H, slot, 0, valid, cr, cg, cb, T,
                        (int)threadIdx.x);
      int item = 0;
      if (threadIdx.x == 0) item = atomicAdd(H.counters + 1, 1);
      item = __shfl(item, 0, 64);
      const int64_t pix0 = pixel_index(P, tc, (int)threadIdx.x);
      int tile_max = 0;
#pragma unroll
      for (int k = 0; k < kPix; ++k) {
        H.hand_T[(int64_t)item * 256 + tile_pixel(k)] = T[k];
        if (out_last != nullptr && valid[k])
          out_last[pix0 + (int64_t)4 * k * P.width] = last[k];
        tile_max = max(tile_max, last[k]);
      }
      tile_max = wave_max_row3(tile_max);
      if (threadIdx.x == kLanes - 1 && out_tile_stop != nullptr)
        out_tile_stop[tc.tile] = tile_max;
      if (threadIdx.x == 0) {
        H.handoff[item] = tc.tile;
        H.handoff_tail[item] = tail;
      }
      return;
    }
  }
  if (seg_cur > 0)  // (no workspace: nothing recorded)
    last_segment<kPix>(P, tc, out_rgb, H, -1, valid, cr, cg, cb, T,
                       (int)threadIdx.x);
  int tile_max = 0;
  // The lane's pixels are 4 rows apart: one 64-bit index, then increments
  // (the lane's column and row from a fresh lane index).
  const int lane_end = lane_now();
  const int64_t pix0 = opaque64(
      ((int64_t)tc.batch * P.height + tc.y0 + (lane_end >> 4)) * P.width +
      tc.x0 + (lane_end & 15));
  const int64_t strip = (int64_t)4 * P.width;
  // the whole tile's last or none of it (whole 64-byte rows: lines that the
  // neighbouring tile also writes are written back whole)
  bool stop = false;
#pragma unroll
  for (int k = 0; k < kPix; ++k) stop |= valid[k] && !(T[k] > t_thr);
  const bool put_last = all_last || __builtin_amdgcn_ballot_w64(stop) != 0;
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    if (valid[k]) {
      if (T[k] > t_thr) last[k] = end - start;  // never stopped: whole list
      const int64_t pix = pix0 + k * strip;
      // ordinary stores: a tile row's 192 bytes of colour and 64 bytes each of
      // T and last share 128-byte lines with the neighbouring tile's, which the
      // L2 merges before writing back (streaming stores wrote such lines in
      // part, 15% more bytes in all)
      out_rgb[3 * pix + 0] = cr[k] + T[k] * P.bg_r;
      out_rgb[3 * pix + 1] = cg[k] + T[k] * P.bg_g;
      out_rgb[3 * pix + 2] = cb[k] + T[k] * P.bg_b;
      if (out_T) {
        out_T[pix] = T[k];
        if (put_last) out_last[pix] = last[k];
      }
      tile_max = max(tile_max, last[k]);
    }
  }
  if (out_tile_stop) {
    tile_max = wave_max_row3(tile_max);
    if (threadIdx.x == kLanes - 1) out_tile_stop[tc.tile] = tile_max;
  }
}

// The long kernel's walk over the n staged records of one batch for this
// wavefront's kSpW strips (strips s0 .. s0 + kSpW - 1; strip masks in s2.w).
// Software pipelined: record j + 1 is read from LDS while record j is
// composited, so the walk does not wait for LDS on every splat.
template <int kSpW, bool kPlain>
__device__ __forceinline__ void long_batch(const Staged& S, int n, int idx1,
                                           int s0, float px, const float* py,
                                           float t_thr, float max_alpha,
                                           float* T, float* cr, float* cg,
                                           float* cb, int* last) {
  float4 n0 = S.s0[0], n1 = S.s1[0], n2 = S.s2[0];
  for (int j = 0; j < n; ++j) {
    const float4 a0 = n0, a1 = n1, a2 = n2;
    const int jn = min(j + 1, n - 1);
    n0 = S.s0[jn];
    n1 = S.s1[jn];
    n2 = S.s2[jn];
    const uint32_t mask = uniform_bits(a2.w) >> s0;
    if (!(mask & ((1u << kSpW) - 1u))) continue;  // scalar branch
    const XTerms xt = x_terms(a0.z, a0.w, px - a0.x, a1.y);
#pragma unroll
    for (int k = 0; k < kSpW; ++k) {
      if (!((mask >> k) & 1u)) continue;  // scalar branch
      composite_one<kPlain>(xt, a1, a2, py[k], a0.y, t_thr, max_alpha,
                            idx1 + j, T[k], cr[k], cg[k], cb[k], last[k]);
    }
  }
}

// Continuation of the tiles handed off by render_fwd_kernel: a workgroup of
// 4 / kSpW wavefronts per tile, wavefront w walking strips kSpW w ..
// kSpW w + kSpW - 1 (lane l: column l % 16, row 4 strip + l / 16) from the
// saved state with the same per-pixel operations, so the result is bit for
// bit the one-wavefront walk's.  Workgroup b takes hand-off items b,
// b + gridDim.x, ...
template <int kSpW>
__global__ __launch_bounds__(256 / kSpW) void render_fwd_long_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, float* __restrict__ out_rgb,
    float* __restrict__ out_T, int32_t* __restrict__ out_last,
    int32_t* __restrict__ out_tile_stop, HeavyState H) {
  __shared__ Staged S;
  __shared__ int sh_slot;
  __shared__ int sh_plain;  // batch_plain of the staged batch
  const int lane = (int)threadIdx.x & 63;
  const int s0 = __builtin_amdgcn_readfirstlane(((int)threadIdx.x >> 6) * kSpW);
  const int t0 = 64 * s0 + lane;  // in-tile index of the first strip's pixel
  const int n_items = H.counters[1];
  const float t_thr = P.trans_thr;
  const float max_alpha = fminf(P.max_alpha, 1.0f);
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    __syncthreads();  // the previous tile's reads of S and sh_slot are done
    const int tile = H.handoff[item];
    int tail = H.handoff_tail[item];  // used by thread 0
    const TileCoord tc = tile_coord_of(P, tile);
    const int x = tc.x0 + (lane & 15);
    const float px = (float)x + 0.5f;
    float py[kSpW], T[kSpW], cr[kSpW], cg[kSpW], cb[kSpW];
    int last[kSpW];
    bool valid[kSpW];
    int64_t pix[kSpW];
#pragma unroll
    for (int k = 0; k < kSpW; ++k) {
      const int y = tc.y0 + 4 * (s0 + k) + (lane >> 4);
      valid[k] = (x < P.width) && (y < P.height);
      py[k] = (float)y + 0.5f;
      pix[k] = ((int64_t)tc.batch * P.height + y) * P.width + x;
      T[k] = H.hand_T[(int64_t)item * 256 + t0 + 64 * k];
      last[k] = (valid[k] && out_last != nullptr) ? out_last[pix[k]] : 0;
      cr[k] = cg[k] = cb[k] = 0.0f;
    }
    const int start = tile_offsets[tile];
    const int end = tile_offsets[tile + 1];
    int seg_cur = kHandoff / kSegSplats;
    for (int base = start + kHandoff; base < end; base += kBatch) {
      bool alive = false;
#pragma unroll
      for (int k = 0; k < kSpW; ++k) alive |= T[k] > t_thr;
      if (!__syncthreads_or(alive)) break;  // uniform; frees S
      // (the boundary at kHandoff was closed by render_fwd_kernel)
      if (base > start + kHandoff && (base - start) % kSegSplats == 0) {
        if (threadIdx.x == 0) sh_slot = next_segment(H, tile, seg_cur, tail);
        __syncthreads();
        end_segment<kSpW>(P, tc, out_rgb, H, sh_slot, seg_cur, valid, cr, cg,
                          cb, T, t0);
        ++seg_cur;
      }
      const int n = min(kBatch, end - base);
      const uint32_t m =
          stage_batch<true>(packed, binned, base, n, tc,
                            (uint32_t)P.num_splats - 1u, S);
      if (threadIdx.x < kLanes) {  // wavefront 0 staged the batch
        const bool all_plain = batch_plain(m);
        if (threadIdx.x == 0) sh_plain = all_plain;
      }
      __syncthreads();
      const bool plain = sh_plain != 0;
      if (plain)
        long_batch<kSpW, true>(S, n, base - start + 1, s0, px, py, t_thr,
                               max_alpha, T, cr, cg, cb, last);
      else
        long_batch<kSpW, false>(S, n, base - start + 1, s0, px, py, t_thr,
                                max_alpha, T, cr, cg, cb, last);
    }
    __syncthreads();  // sh_slot of the last boundary has been read
    if (threadIdx.x == 0) sh_slot = next_segment(H, tile, seg_cur, tail);
    __syncthreads();
    last_segment<kSpW>(P, tc, out_rgb, H, sh_slot, valid, cr, cg, cb, T, t0);
    int tile_max = 0;
#pragma unroll
    for (int k = 0; k < kSpW; ++k) {
      if (valid[k]) {
        if (T[k] > t_thr) last[k] = end - start;  // never stopped: whole list
        out_rgb[3 * pix[k] + 0] = cr[k] + T[k] * P.bg_r;
        out_rgb[3 * pix[k] + 1] = cg[k] + T[k] * P.bg_g;
        out_rgb[3 * pix[k] + 2] = cb[k] + T[k] * P.bg_b;
        if (out_T != nullptr) {
          out_T[pix[k]] = T[k];
          out_last[pix[k]] = last[k];
        }
        tile_max = max(tile_max, last[k]);
      }
    }
    if (out_tile_stop != nullptr) {
      tile_max = wave_max_row3(tile_max);
      if (lane == kLanes - 1) atomicMax(out_tile_stop + tile, tile_max);
    }
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

// x += x of the lane that the DPP control selects, in one v_add_f32_dpp, for
// the rows of ROW_MASK; the other rows keep x (as x + 0 would).  Written as
// inline assembly because the compiler splits a partial-row-mask update (and
// one it sinks into a branch) into a zero move, a DPP move and an add.  The
// s_nop 1 gives the two wait states a DPP read needs after a VALU write of
// its source, which the compiler does not insert for inline assembly.
#define GS_ADD_DPP(x, CTRL)                                                  \
  asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 " CTRL " bank_mask:0xf" : "+v"(x))

// Sum over the 64 lanes, left in every lane of row 3 (lanes 48..63):
// row sums, then row_bcast:15 and row_bcast:31 carry them upward.
__device__ __forceinline__ float wave_sum_row3(float x) {
  x = row_sum_dpp(x);
  GS_ADD_DPP(x, "row_bcast:15 row_mask:0xa");
  GS_ADD_DPP(x, "row_bcast:31 row_mask:0xc");
  return x;
}

// Sum over each group of eight lanes (8g..8g+7), left in every lane of the
// group.
__device__ __forceinline__ float group8_sum_dpp(float x) {
  x += dpp_src<0xB1>(x);
  x += dpp_src<0x4E>(x);
  GS_ADD_DPP(x, "row_half_mirror row_mask:0xf");
  return x;
}

// Orders this wavefront's LDS stores before its later LDS loads of other
// lanes' data.  The backward's workgroup is one wavefront, so no s_barrier is
// needed: the fences only keep the compiler from moving the accesses and wait
// for the stores.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Gradient reduction of the backward walk.  Per splat each lane holds nine
// partial sums over its pixels.  Eight of them (kGradQ quantities) go through
// LDS: lane l stores quantity q at red[q][l], then the eight lanes of group q
// (lanes 8q..8q+7) each add eight of its 64 values (two 16-byte loads) and
// three DPP steps finish the group's total, which lane 8q adds atomically to
// the splat's gradient.  The ninth, S0, is summed across the wavefront by
// DPP.  LDS accesses issue on their own port, so the reduction costs few
// vector-ALU slots, the compositor's bound.
constexpr int kGradQ = 8;
constexpr int kAccFloats = 16;  // floats per accumulator record (64 bytes)
struct BwdShared {
  Staged S;
  float red[kGradQ * kLanes];
};

// Where the backward adds its gradients (in original splat order): one
// accumulator record of kAccFloats floats per splat, or, without one, the
// four output arrays.  A record holds a splat's nine gradient sums in one
// 64-byte line, {V_mx, V_my, V_ca, V_cb, V_cc, colour r, g, b, g_opacity}
// (the walk's sums before their scales), so the nine atomics a tile adds
// for a splat touch one cache line instead of four or five, at a uniform
// address plus the lane's entry; render_grads_unpack_kernel scales them
// into the output arrays.
struct GradOut {
  float* g_means2d;
  float* g_conics;
  float* g_colors;
  float* g_opac;
  float* acc;  // [num_splats][kAccFloats] or null
};

// Without records, where group q = lane / 8 sends its total: q = 0..7 is
// {V_mx, V_my, V_ca, V_cb, V_cc, colour r, g, b} (see the backward walk),
// added at base + orig * stride bytes after scaling.
struct GradTarget {
  float* base;
  uint32_t stride;
  float scale;
};

// g_mean = -(2/L) V_m since a = -2A/L, b = -B/L, c = -2C/L;
// g_conic = (-V_ca/2, -V_cb, -V_cc/2).
constexpr float kMeanScale = -2.0f / kLog2e;

__device__ __forceinline__ GradTarget grad_target(const GradOut& G) {
  switch (threadIdx.x >> 3) {
    case 0: return {G.g_means2d + 0, 8, kMeanScale};
    case 1: return {G.g_means2d + 1, 8, kMeanScale};
    case 2: return {G.g_conics + 0, 12, -0.5f};
    case 3: return {G.g_conics + 1, 12, -1.0f};
    case 4: return {G.g_conics + 2, 12, -0.5f};
    case 5: return {G.g_colors + 0, 12, 1.0f};
    case 6: return {G.g_colors + 1, 12, 1.0f};
    default: return {G.g_colors + 2, 12, 1.0f};
  }
}

// Where the opacity gradient goes without records (scale 1).
__device__ __forceinline__ GradTarget opac_target(const GradOut& G) {
  return {G.g_opac, 4, 1.0f};
}

// Per-pixel state of the backward walk (4 pixels per lane).
struct BwdPixels {
  float px;
  float py[kPix], Tc[kPix], gr[kPix], gg[kPix], gb[kPix], gT[kPix];
  int lk[kPix];
};

// Loads grad and saved state; T and gT start at final_T and the background
// term.  Pixels outside the image get lk = 0 (never processed).  last is
// read only for the pixels that stopped (T <= threshold), and only by the
// wavefronts that have one: a pixel above the threshold composited its whole
// tile range (lk = 2^31 - 1), and the one-call forward stores last only for
// the pixels that stopped.
__device__ __forceinline__ void load_bwd_pixels(
    const RasterParams& P, const TileCoord& tc,
    const float* __restrict__ final_T, const int32_t* __restrict__ last_in,
    const float* __restrict__ grad_rgb, BwdPixels& Q) {
  const int x = tc.x0 + tc.lx;
  Q.px = (float)x + 0.5f;
  // The lane's pixels are 4 rows apart: one 64-bit index, then increments.
  const int64_t pix0 = opaque64(
      ((int64_t)tc.batch * P.height + slot_y(tc, 0)) * P.width + x);
  const int64_t strip = (int64_t)4 * P.width;
  bool stopped[kPix];
#pragma unroll
  for (int k = 0; k < kPix; ++k) {
    const int y = slot_y(tc, k);
    const bool valid = (x < P.width) && (y < P.height);
    Q.py[k] = (float)y + 0.5f;
    if (valid) {
      const int64_t pix = pix0 + k * strip;
      // streaming loads: each pixel's state is read once
      Q.gr[k] = __builtin_nontemporal_load(grad_rgb + 3 * pix + 0);
      Q.gg[k] = __builtin_nontemporal_load(grad_rgb + 3 * pix + 1);
      Q.gb[k] = __builtin_nontemporal_load(grad_rgb + 3 * pix + 2);
      Q.Tc[k] = __builtin_nontemporal_load(final_T + pix);
    } else {
      Q.gr[k] = Q.gg[k] = Q.gb[k] = 0.0f;
      Q.Tc[k] = 1.0f;
    }
    Q.gT[k] = Q.gr[k] * P.bg_r + Q.gg[k] * P.bg_g + Q.gb[k] * P.bg_b;
    stopped[k] = valid && !(Q.Tc[k] > P.trans_thr);
    Q.lk[k] = valid ? 0x7fffffff : 0;
  }
  bool any = false;
#pragma unroll
  for (int k = 0; k < kPix; ++k) any |= stopped[k];
  if (__builtin_amdgcn_ballot_w64(any) != 0) {
#pragma unroll
    for (int k = 0; k < kPix; ++k)
      if (stopped[k])
        Q.lk[k] = __builtin_nontemporal_load(last_in + pix0 + k * strip);
  }
}

// True when some pixel of the wavefront lies outside the image or stopped
// early in the forward (T <= transmittance threshold).  Otherwise every pixel
// composited every splat visible to it, so a splat at index >= last is
// invisible there and the walk can skip the index test (kCheckLast = false).
__device__ __forceinline__ bool needs_last_test(const RasterParams& P,
                                                const TileCoord& tc,
                                                const BwdPixels& Q) {
  const int x = tc.x0 + tc.lx;
  bool need = false;
#pragma unroll
  for (int k = 0; k < kPix; ++k)
    need |= (x >= P.width) | (slot_y(tc, k) >= P.height) |
            !(Q.Tc[k] > P.trans_thr);
  return __builtin_amdgcn_ballot_w64(need) != 0;
}

// Reverse walk over the n staged records of one batch (tile indices
// cstart .. cstart + n - 1): each pixel undoes the blend of every splat it
// composited in the forward (i < last, tested with kCheckLast) and sees,
// adding its parts of the splat's gradients to the lane's sums, which are
// reduced across the wavefront and added atomically in original order.
// kPlain: every record has kPlainBit, so e <= 0 and the max_alpha gate are
// not tested (they always pass).  kAcc: the totals go to the records at acc,
// else to target and opac.
template <bool kCheckLast, bool kPlain, bool kAcc>
__device__ __forceinline__ void bwd_batch(
    BwdShared& SH, uint32_t bmask, int n, int cstart, float max_alpha,
    float* acc, const GradTarget& target, const GradTarget& opac,
    BwdPixels& Q) {
  const Staged& S = SH.S;
  const int lane = threadIdx.x;
  const bool group_head = (lane & 7) == 0;
  // this lane's eight values of its group's quantity q = lane / 8 in red:
  // 16-byte chunks l and l + 8 of the row (l = lane % 8), so that the eight
  // lanes of a group read 128 consecutive bytes per load.  Rows are 256 bytes
  // apart, one turn of the 64 four-byte LDS banks, so odd groups read their
  // two halves in the other order: each load then spreads over all 64 banks
  // (no bank conflict).  The sum below adds the two halves' sums, which is
  // commutative, so the order does not change the result.
  const int q = lane >> 3;
  const float* red_in0 = SH.red + q * kLanes + (lane & 7) * 4 + (q & 1) * 32;
  const float* red_in1 = SH.red + q * kLanes + (lane & 7) * 4 + (~q & 1) * 32;
  // Per-lane partial sums of the current splat; zero between splats.
  float S0 = 0.f, S1 = 0.f, S2 = 0.f;
  float acc_r = 0.f, acc_g = 0.f, acc_b = 0.f;
  for (int j = n - 1; j >= 0; --j) {
    const uint32_t mask = __builtin_amdgcn_readlane(bmask, j);
    if (mask == 0u) continue;
    const float4 a2 = S.s2[j];
    const int i = cstart + j;
    const float4 a0 = S.s0[j];
    const float4 a1 = S.s1[j];
    const float dx = Q.px - a0.x;
    const XTerms xt = x_terms(a0.z, a0.w, dx, a1.y);
    // lanes with a contribution, from the comparisons' own lane masks
    // (uniform; a ballot of the combined test would be materialised per lane)
    uint64_t hits = 0;
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
      if (!((mask >> k) & 1u)) continue;  // scalar branch
      // one combined test: composited in the forward (i < last) and visible
      const float dy = Q.py[k] - a0.y;
      const Exponents E = exponents(xt, a1.x, dy);
      const bool c_last = (!kCheckLast) | (i < Q.lk[k]);
      const bool c_e = kPlain || power_nonpositive(E, xt, dy);
      const bool c_p = E.p >= a2.z;
      uint64_t hk = __builtin_amdgcn_ballot_w64(c_p);
      if (kCheckLast) hk &= __builtin_amdgcn_ballot_w64(c_last);
      if (!kPlain) hk &= __builtin_amdgcn_ballot_w64(c_e);
      hits |= hk;
      if (c_last & c_e & c_p) {
        const float raw = __builtin_amdgcn_exp2f(E.p);
        const bool open = kPlain || raw < max_alpha;  // gradient gate
        const float alpha = open ? raw : max_alpha;
        // 1 - alpha >= 1 - max_alpha >= eps (checked on the host), so the
        // reference's max(1 - alpha, eps) is 1 - alpha.
        const float T_prev = Q.Tc[k] * __builtin_amdgcn_rcpf(1.0f - alpha);
        const float dot_gc = Q.gr[k] * a1.z + Q.gg[k] * a1.w + Q.gb[k] * a2.x;
        const float diff = dot_gc - Q.gT[k];
        const float wgt = T_prev * alpha;
        acc_r += Q.gr[k] * wgt;
        acc_g += Q.gg[k] * wgt;
        acc_b += Q.gb[k] * wgt;
        // alpha = raw when the gate is open, so T_prev raw = wgt
        const float g_pow = open ? wgt * diff : 0.0f;
        const float hdy = g_pow * dy;
        S0 += g_pow;
        S1 += hdy;
        S2 += hdy * dy;
        Q.gT[k] += alpha * diff;
        Q.Tc[k] = T_prev;
      }
    }
    if (hits != 0) {
      // Per-lane parts of the splat's gradients (a, b, c = -2A/L, -B/L,
      // -2C/L): g_mean = -(2/L) (V_mx, V_my), g_conic = (-V_ca/2, -V_cb,
      // -V_cc/2) with V_cc = S2, and g_opacity = sum g_raw exp(power) =
      // (sum g_power) / o = S0 / o.
      const float X = dx * S0;             // sum g_power dx
      const float hB = 0.5f * a0.w;
      float* red_out = SH.red + lane;
      red_out[0 * kLanes] = a0.z * X + hB * S1;  // V_mx
      red_out[1 * kLanes] = hB * X + a1.x * S1;  // V_my
      red_out[2 * kLanes] = dx * X;              // V_ca = sum g_power dx^2
      red_out[3 * kLanes] = dx * S1;             // V_cb = sum g_power dx dy
      red_out[4 * kLanes] = S2;
      red_out[5 * kLanes] = acc_r;
      red_out[6 * kLanes] = acc_g;
      red_out[7 * kLanes] = acc_b;
      const float r3 = wave_sum_row3(S0);
      S0 = S1 = S2 = 0.f;
      acc_r = acc_g = acc_b = 0.f;
      wave_lds_sync();
      const float4 u = *reinterpret_cast<const float4*>(red_in0);
      const float4 w = *reinterpret_cast<const float4*>(red_in1);
      const float tot = group8_sum_dpp(((u.x + u.y) + (u.z + u.w)) +
                                       ((w.x + w.y) + (w.z + w.w)));
      const uint32_t orig = uniform_bits(a2.y);
      if (kAcc) {
        float* rec = acc + (size_t)orig * kAccFloats;  // uniform
        if (group_head) unsafeAtomicAdd(rec + q, tot);
        if (lane == kLanes - 1) unsafeAtomicAdd(rec + 8, r3 * a2.w);
      } else {
        if (group_head)
          unsafeAtomicAdd(reinterpret_cast<float*>(
                              reinterpret_cast<char*>(target.base) +
                              (uint64_t)orig * target.stride),
                          tot * target.scale);
        if (lane == kLanes - 1)  // a2.w = 1 / opacity
          unsafeAtomicAdd(reinterpret_cast<float*>(
                              reinterpret_cast<char*>(opac.base) +
                              (uint64_t)orig * opac.stride),
                          r3 * a2.w);
      }
      wave_lds_sync();  // loads done before the next splat's stores
    }
  }
}

// Reverse walk over the tile-range indices [lo, hi), one staged batch of 64
// records at a time.
template <bool kCheckLast, bool kAcc>
__device__ __forceinline__ void bwd_walk(
    const RasterParams& P, const float4* __restrict__ packed,
    const int32_t* __restrict__ binned, int start, int lo, int hi,
    const TileCoord& tc, BwdShared& SH, BwdPixels& Q, const GradOut& G) {
  const GradTarget target = kAcc ? GradTarget{} : grad_target(G);
  const GradTarget opac = kAcc ? GradTarget{} : opac_target(G);
  const float max_alpha = fminf(P.max_alpha, 1.0f);
  for (int cend = hi; cend > lo; cend -= kBatch) {
    const int cstart = max(lo, cend - kBatch);
    const int n = cend - cstart;
    __syncthreads();
    const uint32_t bmask =
        stage_batch<false>(packed, binned, start + cstart, n, tc,
                           (uint32_t)P.num_splats - 1u, SH.S);
    __syncthreads();
    if (batch_plain(bmask))
      bwd_batch<kCheckLast, true, kAcc>(SH, bmask, n, cstart, max_alpha,
                                        G.acc, target, opac, Q);
    else
      bwd_batch<kCheckLast, false, kAcc>(SH, bmask, n, cstart, max_alpha,
                                         G.acc, target, opac, Q);
  }
}

// Copies the backward's accumulator records (GradOut) to the four gradient
// arrays with their scales (as grad_target's) and zeroes them: one thread
// per splat.
__global__ __launch_bounds__(256) void render_grads_unpack_kernel(GradOut G,
                                                                  int n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float4* rec = reinterpret_cast<float4*>(G.acc + i * kAccFloats);
  const float4 a = rec[0], b = rec[1];
  const float o = G.acc[i * kAccFloats + 8];
  // leave the record zero for the next backward on this workspace
  rec[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  rec[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  G.acc[i * kAccFloats + 8] = 0.0f;
  G.g_means2d[2 * i + 0] = kMeanScale * a.x;
  G.g_means2d[2 * i + 1] = kMeanScale * a.y;
  G.g_conics[3 * i + 0] = -0.5f * a.z;
  G.g_conics[3 * i + 1] = -a.w;
  G.g_conics[3 * i + 2] = -0.5f * b.x;
  G.g_colors[3 * i + 0] = b.y;
  G.g_colors[3 * i + 1] = b.z;
  G.g_colors[3 * i + 2] = b.w;
  G.g_opac[i] = o;
}

// True when the backward walks this tile as segments: the forward recorded
// them (with the same workspace layout) and the tile's stop exceeds one.
__device__ __forceinline__ bool heavy_backward(const HeavyState& H, int tile,
                                               int nstop) {
  // (the stop first: most tiles need neither of the loads after it)
  if (nstop <= kSegSplats || H.tile_slot == nullptr) return false;
  return H.counters[2] == H.max_slots && H.tile_slot[tile] >= 0;
}

// Decodes segment slot m: tile, segment index k, segment count and the range
// [lo, hi) of tile indices; false if the slot has no backward work.
__device__ __forceinline__ bool seg_item(const RasterParams& P,
                                         const HeavyState& H,
                                         const int32_t* __restrict__ tile_stop,
                                         int m, int& tile, int& k, int& nseg,
                                         int& lo, int& hi) {
  tile = H.slot_tile[m];
  if (tile < 0 || tile >= P.num_tiles) return false;
  const int nstop = tile_stop[tile];
  if (!heavy_backward(H, tile, nstop)) return false;
  k = H.slot_seg[m];
  nseg = (nstop + kSegSplats - 1) / kSegSplats;
  if (k < 0 || k >= nseg) return false;
  lo = k * kSegSplats;
  hi = min(lo + kSegSplats, nstop);
  return true;
}

// Work items: block m < seg_blocks walks segment slot m (the longest walks,
// dispatched first), the other blocks are tiles (tiles walked as segments
// return at once).
// kWaves wavefronts per SIMD at least: 6 (at most 80 VGPRs) for tiles of
// many pairs, whose walk's LDS round trips and atomics need the extra
// wavefronts more than the few spilled set-up values cost, and 7 (72 VGPRs,
// more values spilled) for tiles of few pairs, whose time goes to the
// per-tile set-up and the loads of the pixel state.  kAcc: G has the
// gradient records (the workspace path).
template <int kWaves, bool kAcc>
__global__ __launch_bounds__(kLanes)
__attribute__((amdgpu_waves_per_eu(kWaves, 8))) void render_bwd_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ tile_offsets,
    const int32_t* __restrict__ binned, const float* __restrict__ final_T,
    const int32_t* __restrict__ last_in, const int32_t* __restrict__ tile_stop,
    const float* __restrict__ grad_rgb, GradOut G, HeavyState H,
    int seg_blocks) {
  __shared__ BwdShared SH;
  const int bid = (int)blockIdx.x;
  const bool seg = bid < seg_blocks;
  const int m = bid;
  {
    int tile, kseg = 0, nseg = 1, lo = 0, hi;
    if (seg) {
      if (m >= min(H.counters[0], H.max_slots)) return;
      if (!seg_item(P, H, tile_stop, m, tile, kseg, nseg, lo, hi)) return;
    } else {
      // seg_blocks is a multiple of 8, so the XCD-aware mapping is kept
      tile = xcd_remap(bid - seg_blocks, P.num_tiles);
      hi = tile_stop[tile];
    }
    // the tile's range start and pixel state are loaded before its stop is
    // waited for (an empty tile's loads are wasted: few tiles are empty)
    const int start = tile_offsets[tile];
    const TileCoord tc = tile_coord_of(P, tile);
    BwdPixels Q;
    load_bwd_pixels(P, tc, final_T, last_in, grad_rgb, Q);
    // (a tile walked as segments returns here)
    if (!seg && (hi <= 0 || heavy_backward(H, tile, hi))) return;
    {
      if (kseg < nseg - 1) {
        // Pixels composited past this segment: T and gT at its end from the
        // forward's segment records (Q.gT holds <g, bg>, Q.Tc T_final).
        float cr[kPix], cg[kPix], cb[kPix];
#pragma unroll
        for (int k = 0; k < kPix; ++k) cr[k] = cg[k] = cb[k] = 0.0f;
        const int t = opaque((int)threadIdx.x);
        int sl = H.slot_next[m];
        for (int j = kseg + 1;
             j < nseg && (unsigned)sl < (unsigned)H.max_slots; ++j) {
          const float4* rj = H.rec + (int64_t)sl * 256 + t;
#pragma unroll
          for (int k = 0; k < kPix; ++k) {
            const float4 v = rj[64 * k];
            cr[k] += v.x;
            cg[k] += v.y;
            cb[k] += v.z;
          }
          sl = H.slot_next[sl];
        }
        const float4* rm = H.rec + (int64_t)m * 256 + t;
#pragma unroll
        for (int k = 0; k < kPix; ++k) {
          if (Q.lk[k] > hi) {
            const float Te = rm[64 * k].w;  // > 0: the pixel was alive
            const float num = Q.gr[k] * cr[k] + Q.gg[k] * cg[k] +
                              Q.gb[k] * cb[k] + Q.gT[k] * Q.Tc[k];
            Q.gT[k] = num / Te;
            Q.Tc[k] = Te;
          }
        }
      }
    }
    // Q.Tc holds T_final, or T at the segment's end for pixels alive past it
    // (T_end > T_final > threshold), so the test sees the final state.
    if (needs_last_test(P, tc, Q))
      bwd_walk<true, kAcc>(P, packed, binned, start, lo, hi, tc, SH, Q, G);
    else
      bwd_walk<false, kAcc>(P, packed, binned, start, lo, hi, tc, SH, Q, G);
  }
}

// Segment records kept at most: one per segment of every tile in the worst
// case, capped at T + 1024 (4 KB each: at most 16 B per pixel + 4 MB).
// Tiles that find the records full are walked whole by the backward.
// n_pairs = 0 (the eval forward, which records nothing) gives one slot.
size_t heavy_max_slots(const RasterParams& P, int64_t n_pairs) {
  const int64_t per_seg = n_pairs / kSegSplats;
  const int64_t worst =
      per_seg + std::min<int64_t>(P.num_tiles, per_seg) + 1;
  return (size_t)std::min<int64_t>(worst, (int64_t)P.num_tiles + 1024);
}

}  // namespace

// The backward's accumulator records (absent from the eval workspace).
size_t acc_bytes(const RasterParams& P, int64_t n_pairs) {
  return n_pairs > 0 ? align_up((size_t)P.num_splats * 4 * kAccFloats, 256)
                     : 0;
}

size_t render_workspace_bytes(const RasterParams& P, int64_t n_pairs) {
  const size_t slots = heavy_max_slots(P, n_pairs);
  const size_t T = (size_t)P.num_tiles;
  return 256 + 3 * align_up(T * 4, 256) + align_up(T * 256 * 4, 256) +
         3 * align_up(slots * 4, 256) +
         align_up(slots * 256 * sizeof(float4), 256) + acc_bytes(P, n_pairs);
}

namespace {
HeavyState heavy_state(const RasterParams& P, int64_t n_pairs, void* ws) {
  HeavyState H{};
  if (ws == nullptr) return H;
  const size_t slots = heavy_max_slots(P, n_pairs);
  const size_t T = (size_t)P.num_tiles;
  char* p = static_cast<char*>(ws);
  H.counters = reinterpret_cast<int32_t*>(p);
  p += 256;
  H.acc = n_pairs > 0 ? reinterpret_cast<float*>(p) : nullptr;
  p += acc_bytes(P, n_pairs);
  H.tile_slot = reinterpret_cast<int32_t*>(p);
  p += align_up(T * 4, 256);
  H.handoff = reinterpret_cast<int32_t*>(p);
  p += align_up(T * 4, 256);
  H.handoff_tail = reinterpret_cast<int32_t*>(p);
  p += align_up(T * 4, 256);
  H.hand_T = reinterpret_cast<float*>(p);
  p += align_up(T * 256 * 4, 256);
  H.slot_tile = reinterpret_cast<int32_t*>(p);
  p += align_up(slots * 4, 256);
  H.slot_seg = reinterpret_cast<int32_t*>(p);
  p += align_up(slots * 4, 256);
  H.slot_next = reinterpret_cast<int32_t*>(p);
  p += align_up(slots * 4, 256);
  H.rec = reinterpret_cast<float4*>(p);
  H.max_slots = (int)slots;
  return H;
}
}  // namespace

void render_forward_zero_spans(const RasterParams& P, int64_t n_pairs,
                               void* workspace, bool training,
                               ZeroSpan out[2]) {
  out[0] = out[1] = ZeroSpan{nullptr, 0};
  if (P.num_tiles == 0 || workspace == nullptr) return;
  const HeavyState H = heavy_state(P, training ? n_pairs : 0, workspace);
  out[0] = ZeroSpan{reinterpret_cast<uint32_t*>(H.counters), 2};
  // The training forward also zeroes the backward's gradient records (the
  // backward accumulates into them and its unpack leaves them zero again).
  if (training && H.acc != nullptr)
    out[1] = ZeroSpan{reinterpret_cast<uint32_t*>(H.acc),
                      (int64_t)P.num_splats * kAccFloats};
}

namespace {
HeavyState forward_state(const RasterParams& P, int64_t n_pairs,
                         void* workspace, const float* out_T) {
  // Without the state outputs no segment is recorded: the layout of
  // n_pairs = 0 (no slot area to speak of) fits the eval workspace.
  HeavyState H = heavy_state(P, out_T != nullptr ? n_pairs : 0, workspace);
  if (out_T == nullptr) H.rec = nullptr;  // no backward: hand-off only
  return H;
}
}  // namespace

// A launch with the one-shot timing events start/stop (gsplat_hip_time_next_
// launch; either may be null), else a traced launch.
template <typename... KArgs, typename... Args>
void launch_timed(const char* name, void (*kernel)(KArgs...), dim3 grid,
                  dim3 block, hipStream_t stream, hipEvent_t start,
                  hipEvent_t stop, Args... args) {
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0,
                          static_cast<KArgs>(args)...);
  else
    launch_traced(name, kernel, grid, block, 0, stream, args...);
}

int launch_render_forward(const RasterParams& P, const float* packed,
                          const int32_t* tile_offsets,
                          const int32_t* binned_ids, float* out_rgb,
                          float* out_T, int32_t* out_last,
                          int32_t* out_tile_stop, int64_t n_pairs,
                          void* workspace, hipStream_t stream, int flags,
                          const HostReport* report) {
  hipEvent_t t0 = nullptr, t1 = nullptr;
  take_launch_timing(kTimeForward, t0, t1);
  if (P.num_tiles == 0)
    return report != nullptr ? launch_host_report(*report, stream) : GSPLAT_OK;
  const HeavyState H = forward_state(P, n_pairs, workspace, out_T);
  const float4* pk = reinterpret_cast<const float4*>(packed);
  if (H.counters != nullptr && !(flags & kForwardPreZeroed)) {
    ZeroSpan z[2];
    render_forward_zero_spans(P, n_pairs, workspace, out_T != nullptr, z);
    const int rc = launch_zero2(z[0].p, z[0].n, z[1].p, z[1].n, stream);
    if (rc) return rc;
  }
  // the continuation follows in this call: it ends the timed span
  const bool more = !(flags & kForwardNoLong) && workspace != nullptr;
  launch_timed("render_fwd_kernel", render_fwd_kernel, dim3((unsigned)P.num_tiles), dim3(kLanes),
               stream, t0, more ? nullptr : t1, P, pk, tile_offsets,
               binned_ids, out_rgb, out_T, out_last, out_tile_stop, H,
               report != nullptr ? *report : HostReport{},
               !(flags & kForwardStoppedLast));
  const int rc = check_launch("render_fwd_kernel");
  if (rc || !more) return rc;
  return launch_render_forward_long(P, packed, tile_offsets, binned_ids,
                                    out_rgb, out_T, out_last, out_tile_stop,
                                    n_pairs, workspace, stream, t1);
}

int launch_render_forward_long(const RasterParams& P, const float* packed,
                               const int32_t* tile_offsets,
                               const int32_t* binned_ids, float* out_rgb,
                               float* out_T, int32_t* out_last,
                               int32_t* out_tile_stop, int64_t n_pairs,
                               void* workspace, hipStream_t stream,
                               hipEvent_t stop) {
  if (P.num_tiles == 0 || workspace == nullptr) return GSPLAT_OK;
  const HeavyState H = forward_state(P, n_pairs, workspace, out_T);
  // Workgroups stride over the hand-off list (its length is on the device).
  const unsigned grid = (unsigned)std::min<int64_t>(P.num_tiles, 2048);
  launch_timed("render_fwd_long_kernel", render_fwd_long_kernel<kLongStrips>, dim3(grid),
               dim3(256 / kLongStrips), stream, nullptr, stop, P,
               reinterpret_cast<const float4*>(packed), tile_offsets,
               binned_ids, out_rgb, out_T, out_last, out_tile_stop, H);
  return check_launch("render_fwd_long_kernel");
}

int launch_render_backward(const RasterParams& P, const float* packed,
                           const int32_t* tile_offsets,
                           const int32_t* binned_ids, const float* final_T,
                           const int32_t* last, const int32_t* tile_stop,
                           const float* grad_rgb, float* g_means2d,
                           float* g_conics, float* g_colors, float* g_opac,
                           int64_t n_pairs, void* workspace,
                           hipStream_t stream) {
  const HeavyState H = heavy_state(P, n_pairs, workspace);
  const GradOut G{g_means2d, g_conics, g_colors, g_opac,
                  P.num_tiles > 0 ? H.acc : nullptr};
  // The gradient records come zeroed from the training forward (or from
  // the unpack of an earlier backward); without them the outputs are the
  // accumulators and are zeroed here.
  int rc = G.acc != nullptr
               ? GSPLAT_OK
               : launch_zero_grads(g_means2d, g_conics, g_colors, g_opac,
                                   P.num_splats, stream);
  if (rc) return rc;
  if (P.num_tiles == 0) return GSPLAT_OK;
  const float4* pk = reinterpret_cast<const float4*>(packed);
  // One block per possible slot, rounded to a multiple of 8 (XCD mapping).
  const int seg_blocks = H.counters ? (H.max_slots + 7) & ~7 : 0;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  take_launch_timing(kTimeBackward, t0, t1);
  // (the pair buffer's size stands for the pair count: up to 64 pairs per
  // tile on average the short-tile variant is faster)
  const bool short_tiles = n_pairs <= (int64_t)64 * P.num_tiles;
  launch_timed("render_bwd_kernel",
               G.acc == nullptr ? render_bwd_kernel<6, false>
               : short_tiles    ? render_bwd_kernel<7, true>
                                : render_bwd_kernel<6, true>,
               dim3((unsigned)(seg_blocks + P.num_tiles)), dim3(kLanes),
               stream, t0, t1, P, pk, tile_offsets, binned_ids, final_T, last,
               tile_stop, grad_rgb, G, H, seg_blocks);
  rc = check_launch("render_bwd_kernel");
  if (rc || G.acc == nullptr || P.num_splats <= 0) return rc;
  launch_traced("render_grads_unpack_kernel", render_grads_unpack_kernel,
                dim3((unsigned)((P.num_splats + 255) / 256)), dim3(256), 0,
                stream, G, P.num_splats);
  return check_launch("render_grads_unpack_kernel");
}

}  // namespace gs
