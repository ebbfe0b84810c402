// binning.hip -- per-splat tile-hit counts, record packing, deterministic
// (tile, gid) pair emission and tile-range extraction.
//
// This translation unit is compiled with -ffp-contract=off: the predicate
// results must match the CPU oracle bit for bit.
//
// Tile walk (count_kernel and emit_kernel).  The candidate tiles of a splat
// are the tiles of its snug pixel bbox, row-major; a candidate is a hit when
// the tile's pixel-centre rectangle meets the splat's alpha >= threshold
// ellipse (reference count_tiles / emit_binned_ids,
// variants/v8/csrc/metal/gsplat_v8_kernels.metal:244-327).  A wavefront takes
// kWalkSplats (32) splats, prefix-sums their candidate counts in registers
// and then tests 64 candidates per step whatever splats they belong to (each
// lane finds its candidate's splat from LDS marks of the splats that start
// inside the step, spread by a DPP prefix maximum; see walk_candidates), so a
// splat with thousands of candidate tiles does not serialise one lane.
//
// Staged path (one launch per step, also the separate C-ABI steps):
// count_kernel  original order: per-splat hit counts and per-workgroup sums
//   (sum_kernel turns them into the pair count N).
// pack_kernel   one thread per depth-sorted splat (gid): packed 64-byte
//   record and exclusive per-gid pair offsets (workgroup scan + decoupled
//   look-back in the same launch).
// emit_kernel   gid order: each hit claims a slot in its splat's range
//   [splat_offsets[gid], splat_offsets[gid+1]) and writes (tile, gid); the
//   same launch zeroes the pair sort's look-back status and counts the pair
//   sort's digit histograms per workgroup (reduced by hist_reduce_kernel).
//   Pairs of one splat have distinct tiles and splats occupy consecutive
//   ranges in gid order, so a stable sort by tile yields (tile, gid) order
//   whatever order the slots inside a splat's range were claimed in.
// ranges_kernel / counts_kernel  tile_offsets and tile_counts from the
//   sorted tile keys (the reference reads them from its atomic counters).
//
// Images of at most 131,072 splats whose pair count goes to host memory
// (the per-step path) take fewer launches:
// count_depth_runs_kernel  the count blocks above beside the depth sort's
//   run-sorting blocks, in one launch.
// rank_pack_kernel  the depth sort's rank step, packing each record where
//   its rank lands and adding each gid's hit count to the total of the emit
//   workgroup that holds the gid.
// emit_kernel<true>  scans its gids' counts from the sum of the totals of
//   the workgroups before it (no look-back), then emits as above.
// bucket_sort_kernel  after one onesweep pass on the high tile bits, a
//   counting sort of each bucket of 2^(bits-8) tiles on the low bits that
//   also writes the tile ranges (images of 2^9..2^16 tiles whose pair
//   buffer holds at most 4096 pairs per bucket on average).
// host_report_kernel  the binning's report to host memory where the
//   forward compositor does not write it.
//
// Larger images in one call: count_kernel also keeps each wavefront's first
// kHitSlab step ballots and the splats' records in original order;
// pack_kernel gives each original index its pair offset and gid; and
// emit_kernel<false, true> walks the splats in the count's original order,
// taking the hits of the recorded steps from the ballots instead of testing
// them again.
#include <algorithm>

#include "gs_internal.h"
#include "gs_predicate.h"
#define GS_HD __device__ __forceinline__
#include "gs_strip.h"
#include "depth_runs.h"
#include "lookback.h"

namespace gs {
namespace {

constexpr int kThreads = 256;

struct SplatGeom {
  float mx, my, a, b, c, o;
};

constexpr int kWaves = kThreads / 64;

// Splats per wavefront in the tile walk.  A wavefront's 64 lanes test the
// candidates of kWalkSplats splats together; fewer splats per wavefront
// than lanes gives each launch more wavefronts (the walk is latency bound)
// and a shorter slot search.
constexpr int kWalkSplats = 32;
constexpr int kWalkBlockSplats = kWaves * kWalkSplats;
// Emit launches with at most this many workgroups add their pair-sort
// histograms atomically instead of through hist_reduce_kernel.
constexpr int kDirectHistBlocks = 1024;
// Copies of the emit's digit histograms (see emit_kernel).
constexpr int kHistCopies = 2;

// One wavefront's kWalkSplats splats, staged for the cooperative tile walk.
struct WalkSlots {
  float4 g0[kWalkSplats];  // mx, my, a, b
  float4 g1[kWalkSplats];  // c, tau, kc, ka
  int4 box[kWalkSplats];   // tx0, ty0, tiles per bbox row, first tile of the image
  int4 inner[kWalkSplats]; // the certain hits (inner_tiles): x, y relative to
                           // the box corner, width, height
  int flags[kWalkSplats];  // bit 0: use_c, bit 1: use_a
  int cend[kWalkSplats];   // inclusive prefix sum of candidate counts
  int first[kWalkSplats];  // exclusive prefix sum: the splat's first candidate
  int ni_incl[kWalkSplats];  // inclusive prefix sum of the certain hits
  uint32_t own[64];        // per walk step: splats starting at each position
};

// Inclusive prefix maximum over the wavefront's 64 lanes (DPP: row shifts by
// 1, 2, 4, 8, then the row broadcasts carry rows 0 and 2 into rows 1, 3 and
// row 1 into rows 2, 3).  Lanes without a DPP source see 0, the identity.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF,
                                               false);
}
__device__ __forceinline__ uint32_t wave_prefix_max(uint32_t x) {
  x = max(x, dpp_or_zero<0x111>(x));
  x = max(x, dpp_or_zero<0x112>(x));
  x = max(x, dpp_or_zero<0x114>(x));
  x = max(x, dpp_or_zero<0x118>(x));
  x = max(x, dpp_or_zero<0x142, 0xA>(x));
  x = max(x, dpp_or_zero<0x143, 0xC>(x));
  return x;
}

// k / w for 0 <= k and 1 <= w, both below 2^24: the float quotient is
// within a few units of the truth for such operands, and the remainder
// corrects it exactly.
__device__ __forceinline__ int div_small(int k, int w) {
  int q = (int)((float)k * __builtin_amdgcn_rcpf((float)w));
  int r = k - q * w;
  while (r < 0) {
    --q;
    r += w;
  }
  while (r >= w) {
    ++q;
    r -= w;
  }
  return q;
}

// A 64-bit value of lane l (l uniform).
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Index of this thread's splat in the walk order of count / emit: lanes
// 0..kWalkSplats-1 of each wavefront take consecutive splats.
__device__ __forceinline__ int walk_splat_index() {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return ((int)blockIdx.x * kWaves + wave) * kWalkSplats + lane;
}

// Smallest number of certain hits (inner_tiles) taken out of the walk: the
// emit writes a splat's certain hits with the wavefront's 64 lanes.
constexpr int kMinCertainHits = 64;

// Tiles of the box [tx0, tx1] x [ty0, ty1] that certainly pass
// ellipse_hits_rect: those whose pixel-centre rectangle lies in the
// rectangle |dx| <= u, |dy| <= v around the centre, with u = k s hx,
// v = k s hy, s^2 = tau / (a hx^2 + c hy^2 + 2|b| hx hy) and k = 1 - 2^-10.
// The quadratic q = a dx^2 + 2b dx dy + c dy^2 is convex, so on that
// rectangle it is at most its largest corner value a u^2 + c v^2 + 2|b| u v
// = k^2 s^2 (...) <= tau (1 - 2^-9) (s rounded within a few ulp).  A tile
// there has its centre inside (a hit at once) or its nearest corner inside
// the rectangle, where the predicate's rounded q, whose operands dx, dy are
// each one rounded subtraction (relative error 2^-24) and whose three
// terms sum to at most 2 (a dx^2 + c dy^2) <= 2 tau in magnitude (b^2 < ac),
// exceeds the exact one by less than 16 2^-24 tau: below tau.  The tile
// range is computed from u and v less an absolute margin far above the
// rounding of mx +- u and my +- v.  Returns {x, y relative to (tx0, ty0),
// width, height}, all 0 when there is no such tile or any quantity is not
// finite, or when they are fewer than kMinCertainHits.  hx, hy only shape
// the rectangle (the box's half extents).
__device__ __forceinline__ int4 inner_tiles(float mx, float my, float a,
                                            float b, float c, float tau,
                                            int tx0, int ty0, int tx1,
                                            int ty1) {
#pragma clang fp contract(off)
  const float det = a * c - b * b;
  if (!(a > 0.0f && c > 0.0f && det > 0.0f)) return make_int4(0, 0, 0, 0);
  const float hx = __builtin_sqrtf(tau * c / det);
  const float hy = __builtin_sqrtf(tau * a / det);
  const float den = a * hx * hx + c * hy * hy + 2.0f * fabsf(b) * hx * hy;
  const float sk = __builtin_sqrtf(tau / den) * (1.0f - 0x1p-10f);
  const float margin =
      (fabsf(mx) + fabsf(my) + hx + hy) * 0x1p-20f + 0x1p-20f;
  const float u = sk * hx - margin, v = sk * hy - margin;
  if (!(u > 0.0f && v > 0.0f && u < 0x1p30f && v < 0x1p30f &&
        fabsf(mx) < 0x1p30f && fabsf(my) < 0x1p30f))
    return make_int4(0, 0, 0, 0);
  // tiles t with 16 t + 0.5 >= mx - u and 16 t + 15.5 <= mx + u
  const float fx0 = fmaxf(ceilf((mx - u - 0.5f) * 0.0625f), (float)tx0);
  const float fx1 = fminf(floorf((mx + u - 15.5f) * 0.0625f), (float)tx1);
  const float fy0 = fmaxf(ceilf((my - v - 0.5f) * 0.0625f), (float)ty0);
  const float fy1 = fminf(floorf((my + v - 15.5f) * 0.0625f), (float)ty1);
  if (!(fx0 <= fx1 && fy0 <= fy1)) return make_int4(0, 0, 0, 0);
  const int ix0 = (int)fx0, iy0 = (int)fy0;
  const int iw = (int)fx1 - ix0 + 1, ih = (int)fy1 - iy0 + 1;
  // (fewer tiles are cheaper to walk than to write in a loop of their own)
  if (iw * ih < kMinCertainHits) return make_int4(0, 0, 0, 0);
  return make_int4(ix0 - tx0, iy0 - ty0, iw, ih);
}

// Stages this lane's splat (lanes below kWalkSplats) and returns the
// wavefront's candidate total: the tiles of each splat's box outside its
// certain hits (inner_tiles), whose count goes to n_inner.  Candidate
// counts fit in int32: tiles per image are limited to 2^24 on the host, so
// a wavefront has at most 2^28 candidates.
__device__ __forceinline__ int walk_setup(const RasterParams& P, bool valid,
                                          const SplatGeom& s, int batch,
                                          WalkSlots& W, int& n_inner) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  int ncand = 0;
  int4 box = make_int4(0, 0, 1, 0);
  int4 inner = make_int4(0, 0, 0, 0);
  n_inner = 0;
  float4 g1 = make_float4(s.c, 0.0f, 0.0f, 0.0f);
  int flags = 0;
  float tau;
  if (valid && alpha_support(s.o, P.alpha_thr, P.eps, tau)) {
    const PixBox bb =
        snugbox(s.mx, s.my, s.a, s.b, s.c, tau, P.width, P.height, P.eps);
    if (bb.x0 <= bb.x1 && bb.y0 <= bb.y1) {
      const int tx0 = bb.x0 >> 4, tx1 = bb.x1 >> 4;
      const int ty0 = bb.y0 >> 4, ty1 = bb.y1 >> 4;
      box = make_int4(tx0, ty0, tx1 - tx0 + 1, batch * P.tiles_per_image);
      // (the inscribed rectangle is at most 2/pi of the ellipse's box)
      if (box.z * (ty1 - ty0 + 1) >= 2 * kMinCertainHits) {
        inner =
            inner_tiles(s.mx, s.my, s.a, s.b, s.c, tau, tx0, ty0, tx1, ty1);
        n_inner = inner.z * inner.w;
      }
      ncand = box.z * (ty1 - ty0 + 1) - n_inner;
      const ConicSlopes k = conic_slopes(s.a, s.b, s.c);
      g1 = make_float4(s.c, tau, k.kc, k.ka);
      flags = (k.use_c ? 1 : 0) | (k.use_a ? 2 : 0);
    }
  }
  int inc = ncand, inc_i = n_inner;
#pragma unroll
  for (int off = 1; off < kWalkSplats; off <<= 1) {
    const int y = __shfl_up(inc, off, 64);
    const int yi = __shfl_up(inc_i, off, 64);
    if (lane >= off) {
      inc += y;
      inc_i += yi;
    }
  }
  if (lane < kWalkSplats) {
    W.g0[lane] = make_float4(s.mx, s.my, s.a, s.b);
    W.g1[lane] = g1;
    W.box[lane] = box;
    W.inner[lane] = inner;
    W.flags[lane] = flags;
    W.cend[lane] = inc;
    W.first[lane] = inc - ncand;
    W.ni_incl[lane] = inc_i;
  }
  __builtin_amdgcn_wave_barrier();
  return __shfl(inc, kWalkSplats - 1, 64);
}

// Tests the wavefront's candidates 64 at a time and calls on_hit(slot, tile)
// for every hit (slot = 0..kWalkSplats-1, the splat's lane in walk_setup).
// A candidate's slot is the last splat whose first candidate is at or
// before it (a splat without candidates shares its first index with the
// next one and loses to it): the owner of the step's first candidate is
// counted with a ballot, the splats that start inside the step mark their
// position with an LDS max, and a prefix maximum over the lanes spreads the
// marks -- one LDS round trip per step instead of a binary search.
//
// on_step(hm, hit, sl, tile, c0) is called by every lane once per step, hm
// being the step's ballot of hits (hit, sl and tile: this lane's
// candidate's; sl and tile mean nothing without the hit).  Candidates are enumerated splat by
// splat, so the wavefront's hits arrive in splat order: the hits before a
// position are counted with one running total and a lane-masked popcount,
// without per-splat counters (whose atomics would serialise the lanes of one
// splat on one LDS address).
//
// rec (may be null): the wavefront's recorded ballots (kHitSlab words, step
// k's ballot at rec[k], as count_block records them for the same splats):
// the steps they cover take their hits from there instead of the exact
// test, and steps without a hit are skipped (on_step is not called).
template <typename Fn>
__device__ __forceinline__ void walk_candidates(const RasterParams& P,
                                                WalkSlots& W, int total,
                                                const uint64_t* __restrict__ rec,
                                                Fn&& on_step) {
#pragma clang fp contract(off)
  static_assert(kHitSlab % 64 == 0, "a slab is loaded 64 words at a time");
  const int lane = threadIdx.x & 63;
  const int first = lane < kWalkSplats ? W.first[lane] : 0x7fffffff;
  // (without certain hits in the wavefront every box is walked whole)
  const bool any_inner = W.ni_incl[kWalkSplats - 1] != 0;
  uint64_t chunk = 0ull;  // lane l: the recorded ballot of step 64 (k / 64) + l
  for (int c0 = 0; c0 < total; c0 += 64) {
    const int step = c0 >> 6;
    const bool recorded = rec != nullptr && step < kHitSlab;
    uint64_t hm = 0ull;
    if (recorded) {
      if ((step & 63) == 0) chunk = rec[step + lane];  // < kHitSlab
      hm = readlane64(chunk, step & 63);
      if (hm == 0ull) continue;  // no hit among these candidates
    }
    const int owner0 = __popcll(__ballot(first <= c0)) - 1;  // first[0] = 0
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    W.own[lane] = lane == 0 ? (uint32_t)owner0 : 0u;
    if (first > c0 && first < c0 + 64)
      atomicMax(&W.own[first - c0], (uint32_t)lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int sl = (int)wave_prefix_max(W.own[lane]);
    const int c = c0 + lane;
    bool hit = false;
    int tile = 0;
    if (c < total) {
      // Candidate k of the splat's box less its certain hits (an inner
      // rectangle at (ix, iy), iw x ih, in box coordinates): the rows above
      // it in full, then ih rows of bw - iw tiles, then the rows below in
      // full.
      const int k = c - W.first[sl];
      const int4 bx = W.box[sl];
      int tx, ty;
      if (any_inner) {
        const int4 in = W.inner[sl];
        const int top = bx.z * in.y;
        const int mid_w = bx.z - in.z;
        const int mid = mid_w * in.w;
        const bool in_mid = k >= top && k < top + mid;
        const bool below = k >= top + mid;
        const int kk = below ? k - top - mid : (in_mid ? k - top : k);
        const int w = in_mid ? mid_w : bx.z;
        const int q = div_small(kk, w);
        const int j = kk - q * w;
        tx = bx.x + ((in_mid && j >= in.x) ? j + in.z : j);
        ty = bx.y + q + (below ? in.y + in.w : (in_mid ? in.y : 0));
      } else {
        const int q = div_small(k, bx.z);
        tx = bx.x + (k - q * bx.z);
        ty = bx.y + q;
      }
      if (recorded) {
        hit = ((hm >> lane) & 1ull) != 0ull;
      } else {
        const float4 g0 = W.g0[sl], g1 = W.g1[sl];
        const int fl = W.flags[sl];
        ConicSlopes ks;
        ks.kc = g1.z;
        ks.ka = g1.w;
        ks.use_c = (fl & 1) != 0;
        ks.use_a = (fl & 2) != 0;
        float rx0, ry0, rx1, ry1;
        tile_rect(tx, ty, P.width, P.height, rx0, ry0, rx1, ry1);
        hit = ellipse_hits_rect(g0.x, g0.y, g0.z, g0.w, g1.x, ks, g1.y, rx0,
                                ry0, rx1, ry1);
      }
      tile = bx.w + ty * P.tiles_x + tx;
    }
    if (!recorded) hm = __ballot(hit);
    on_step(hm, hit, sl, tile, c0);
  }
}

// Hits among the lanes below `rel` of a step's hit ballot hm (rel in 0..64).
__device__ __forceinline__ int hits_below(uint64_t hm, int rel) {
  return __popcll(rel >= 64 ? hm : (hm & ((1ull << rel) - 1ull)));
}

// LDS of a count block of kW wavefronts.
template <int kW>
struct CountLds {
  WalkSlots walk[kW];
  int wsum[kW];
};

// Divisions and square roots of the per-splat strip constants: correctly
// rounded (this file is built with -fhip-fp32-correctly-rounded-divide-sqrt).
struct IeeeOps {
  static __device__ __forceinline__ float div(float x, float y) { return x / y; }
  static __device__ __forceinline__ float sqrt(float x) {
    return __builtin_sqrtf(x);
  }
};

// The packed 64-byte record of splat orig:
// {mx, my, a, b}, {c, o, r, g}, {b, slot | plain << 31, q, lo},
// {dxt, beta, gamma, delta}: lo = log2(o), q = plim + lo (the compositors'
// visibility bound on p + lo), plain = plain_record of the compositors'
// exponent coefficients, and the strip-culling constants (gs_strip.h).  The
// slot holds orig in the records of the compositors (pack_record) and the
// splat's tile-hit count in the original-order records of the count.
struct Record {
  float4 v[kRecordVec4];
};
__device__ __forceinline__ Record record_of(
    const RasterParams& P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, int orig, uint32_t slot) {
  const float mx = means2d[2 * orig + 0];
  const float my = means2d[2 * orig + 1];
  const float a = conics[3 * orig + 0];
  const float b = conics[3 * orig + 1];
  const float c = conics[3 * orig + 2];
  const float o = opacities[orig];
  const float cr = colors[3 * orig + 0];
  const float cg = colors[3 * orig + 1];
  const float cb = colors[3 * orig + 2];
  const float plim = visibility_limit(o, P.alpha_thr, P.max_alpha);
  const float lo = opacity_log2(o);
  const bool plain = plain_record(
      (-0.5f * a) * kLog2e, (-b) * kLog2e, (-0.5f * c) * kLog2e, mx, my, o,
      plain_opacity_limit(fminf(P.max_alpha, 1.0f)));
  const StripConsts k = strip_consts_t<IeeeOps>(a, b, c, plim);
  Record r;
  r.v[0] = make_float4(mx, my, a, b);
  r.v[1] = make_float4(c, o, cr, cg);
  r.v[2] = make_float4(cb, __uint_as_float(slot | (plain ? 0x80000000u : 0u)),
                       plim + lo, lo);
  r.v[3] = make_float4(k.dxt, k.beta, k.gamma, k.delta);
  return r;
}

__device__ __forceinline__ void store_record(float4* __restrict__ dst,
                                             int64_t i, const Record& r) {
  float4* d = dst + (int64_t)kRecordVec4 * i;
#pragma unroll
  for (int k = 0; k < kRecordVec4; ++k) d[k] = r.v[k];
}

// The record of splat orig at depth rank gid.
__device__ __forceinline__ void pack_record(
    const RasterParams& P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, float4* __restrict__ packed, int gid,
    int orig) {
  store_record(packed, gid,
               record_of(P, means2d, conics, colors, opacities, orig,
                         (uint32_t)orig));
}

// Count block vb of nvb (kW wavefronts, kWalkSplats splats each), original
// order: splat_count[orig] = tile hits of splat orig and, with block_sums,
// block_sums[vb] = the block's total; with rec_orig also the splat's record
// in original order, its count in the slot (pack_kernel then copies one
// 64-byte record per splat instead of gathering five attribute arrays).
// The blocks also zero zero_words[0..n_zero_words) (grid-stride; read only
// by later launches).  With lds_hist (2 x 257 words of LDS) the block also
// counts its hits' tile digits ((tile >> hist_shift) & 255) and writes them
// to hist_row[0..255]: the pair sort's histogram, in partials that a later
// launch sums (it counts every hit, the emit only those below its capacity:
// the two differ only when the capacity is short, and then the binning is
// redone).  With hit_bits the block records each wavefront's first kHitSlab
// step ballots at hit_bits[w * kHitSlab + step] (w = vb * kW + wavefront:
// the splats' index / kWalkSplats), for an emit that walks the same splats.
template <int kW>
__device__ __forceinline__ void count_block(
    const RasterParams& P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ opacities,
    const float* __restrict__ colors, float4* __restrict__ rec_orig,
    int32_t* __restrict__ splat_count, int32_t* __restrict__ block_sums,
    uint32_t* __restrict__ zero_words, int64_t n_zero_words, int vb, int nvb,
    CountLds<kW>& S, uint32_t* lds_hist = nullptr,
    uint32_t* __restrict__ hist_row = nullptr, int hist_shift = 0,
    uint64_t* __restrict__ hit_bits = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t i = (int64_t)vb * (64 * kW) + threadIdx.x; i < n_zero_words;
       i += (int64_t)nvb * (64 * kW))
    zero_words[i] = 0u;
  if (lds_hist != nullptr) {
    for (int i = threadIdx.x; i < 2 * 257; i += 64 * kW) lds_hist[i] = 0u;
    __syncthreads();
  }
  const int orig = (vb * kW + wave) * kWalkSplats + lane;
  const bool valid = lane < kWalkSplats && orig < P.num_splats;
  const int o = valid ? orig : P.num_splats - 1;
  SplatGeom s;
  s.mx = means2d[2 * o + 0];
  s.my = means2d[2 * o + 1];
  s.a = conics[3 * o + 0];
  s.b = conics[3 * o + 1];
  s.c = conics[3 * o + 2];
  s.o = opacities[o];
  WalkSlots& W = S.walk[wave];
  int n_inner;
  const int total = walk_setup(P, valid, s, o / P.gpb, W, n_inner);
  // Hits before the end of this lane's splat's candidates (lanes below
  // kWalkSplats): the running total of the steps before plus the hits below
  // the end inside its step; a splat's count is the difference to the
  // previous lane's.
  const int my_end = lane < kWalkSplats ? W.cend[lane] : 0;
  int run = 0, hits_to_end = 0;
  // the recorded ballots, one store by the first lane per step (holding
  // them in the lanes until 64 are stored together costs the walk more)
  uint64_t* const rec =
      hit_bits != nullptr ? hit_bits + (int64_t)(vb * kW + wave) * kHitSlab
                          : nullptr;
  walk_candidates(P, W, total, nullptr, [&](uint64_t hm, bool hit, int,
                                            int tile, int c0) {
    const int rel = my_end - c0;
    if (rel > 0 && rel <= 64) hits_to_end = run + hits_below(hm, rel);
    run += __popcll(hm);
    if (rec != nullptr && lane == 0 && (c0 >> 6) < kHitSlab)
      rec[c0 >> 6] = hm;
    if (lds_hist != nullptr && hit)
      atomicAdd(&lds_hist[(lane & 1) * 257 + (((uint32_t)tile >> hist_shift) & 255u)], 1u);
  });
  if (lds_hist != nullptr) {
    // the certain hits: each row of the splat's inner rectangle, cut where
    // the digit changes
    if (lane < kWalkSplats && n_inner > 0) {
      const int4 in = W.inner[lane];
      const int4 bx = W.box[lane];
      for (int r = 0; r < in.w; ++r) {
        uint32_t t0 = (uint32_t)(bx.w + (bx.y + in.y + r) * P.tiles_x + bx.x + in.x);
        const uint32_t t1 = t0 + (uint32_t)in.z;
        while (t0 < t1) {
          const uint32_t seg = min(t1, ((t0 >> hist_shift) + 1u) << hist_shift);
          atomicAdd(&lds_hist[(lane & 1) * 257 + ((t0 >> hist_shift) & 255u)], seg - t0);
          t0 = seg;
        }
      }
    }
    __syncthreads();
    if (threadIdx.x < 256)
      hist_row[threadIdx.x] = lds_hist[threadIdx.x] + lds_hist[257 + threadIdx.x];
  }
  const int prev_end = __shfl_up(hits_to_end, 1, 64);
  const int n =
      valid ? hits_to_end - (lane == 0 ? 0 : prev_end) + n_inner : 0;
  if (valid) splat_count[orig] = n;
  // (the attributes are read again here rather than kept across the walk)
  if (valid && rec_orig != nullptr)
    store_record(rec_orig, orig,
                 record_of(P, means2d, conics, colors, opacities, orig,
                           (uint32_t)n));
  if (block_sums == nullptr) return;
  int v = n;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if (lane == 0) S.wsum[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) t += S.wsum[w];
    block_sums[vb] = t;
  }
}

__global__ __launch_bounds__(kThreads) void count_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ opacities,
    const float* __restrict__ colors, float4* __restrict__ rec_orig,
    int32_t* __restrict__ splat_count, int32_t* __restrict__ block_sums,
    uint32_t* __restrict__ zero_words, int64_t n_zero_words,
    uint64_t* __restrict__ hit_bits) {
  __shared__ CountLds<kWaves> S;
  count_block<kWaves>(P, means2d, conics, opacities, colors, rec_orig,
                      splat_count, block_sums, zero_words, n_zero_words,
                      (int)blockIdx.x, (int)gridDim.x, S, nullptr, nullptr, 0,
                      hit_bits);
}

// The count next to the run step of the small-image depth order, in one
// launch: workgroups below run_blocks sort one depth run each (a few CUs for
// most of the launch), the others are count blocks of kRunWaves wavefronts
// and fill the remaining CUs.  The two parts touch disjoint memory.
union CountRunsLds {
  run_step::RunSortLds runs;
  CountLds<run_step::kRunWaves> count;
};

__global__ __launch_bounds__(run_step::kRunThreads) void count_depth_runs_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ opacities,
    int32_t* __restrict__ splat_count, uint32_t* __restrict__ zero_words,
    int64_t n_zero_words, const float* __restrict__ depths, int runs,
    int run_blocks, run_step::RunBuffers runs_out, CountHist H) {
  __shared__ CountRunsLds S;
  __shared__ uint32_t hist[2 * 257];
  if ((int)blockIdx.x < run_blocks) {
    run_step::run_sort_block(depths, P.gpb, runs, (int)blockIdx.x, runs_out,
                             S.runs);
    return;
  }
  const int vb = (int)blockIdx.x - run_blocks;
  count_block<run_step::kRunWaves>(
      P, means2d, conics, opacities, nullptr, nullptr, splat_count, nullptr,
      zero_words, n_zero_words, vb, (int)gridDim.x - run_blocks, S.count,
      H.parts != nullptr ? hist : nullptr,
      H.parts != nullptr ? H.parts + (int64_t)vb * 256 : nullptr, H.shift);
}

// One workgroup: *pair_count = sum of the n block sums (-1 if it does not fit
// in int32).
__global__ __launch_bounds__(kThreads) void sum_kernel(
    const int32_t* __restrict__ block_sums, int n, int32_t* pair_count) {
  __shared__ long long part[kThreads];
  // eight independent loads in flight per thread
  long long acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = threadIdx.x;
  for (; i + 7 * kThreads < n; i += 8 * kThreads) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += block_sums[i + u * kThreads];
  }
  for (; i < n; i += kThreads) acc[0] += block_sums[i];
  long long v = 0;
#pragma unroll
  for (int u = 0; u < 8; ++u) v += acc[u];
  part[threadIdx.x] = v;
  __syncthreads();
  for (int half = kThreads / 2; half > 0; half >>= 1) {
    if (threadIdx.x < half) part[threadIdx.x] += part[threadIdx.x + half];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const long long total = part[0];
    *pair_count = total > 0x7fffffffLL ? -1 : (int32_t)total;
  }
}

// Rank step of the small-image depth order with the records packed where
// the ranks land: perm[gid] = in-image index, the record of gid and
// gid_count[gid] = splat_count[orig] (the pair offsets are then scanned by
// emit_kernel<true>).
// Emit workgroups whose totals a rank_pack workgroup adds in LDS first (its
// 256 gids are increasing and usually span a few dozen of them).
constexpr int kAggBlocks = 128;

__global__ __launch_bounds__(run_step::kRankBlock) void rank_pack_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, run_step::RunBuffers runs_in,
    int runs, const int32_t* __restrict__ splat_count,
    int32_t* __restrict__ perm, float4* __restrict__ packed,
    int32_t* __restrict__ gid_count, uint32_t* __restrict__ block_totals,
    CountHist H) {
  __shared__ run_step::RankLds S;
  __shared__ uint32_t agg[kAggBlocks];
  __shared__ int agg_first;
  const int t = threadIdx.x;
  if (H.parts != nullptr && blockIdx.x == gridDim.x - 1) {
    // the extra workgroup: the pair sort's histogram from the count blocks'
    // partials (kRankSplit thread groups per digit, then their sums in LDS)
    constexpr int kGroups = run_step::kRankBlock / 256;
    uint32_t* red = reinterpret_cast<uint32_t*>(&S);
    const int d = t & 255, g = t >> 8;
    // (eight independent loads in flight per thread)
    uint32_t acc[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    int r = g;
    for (; r + 7 * kGroups < H.nparts; r += 8 * kGroups) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += H.parts[(int64_t)(r + u * kGroups) * 256 + d];
    }
    for (; r < H.nparts; r += kGroups) acc[0] += H.parts[(int64_t)r * 256 + d];
    uint32_t v = 0u;
#pragma unroll
    for (int u = 0; u < 8; ++u) v += acc[u];
    red[g * 256 + d] = v;
    __syncthreads();
    if (t < 256) {
      uint32_t sum = 0u;
#pragma unroll
      for (int k = 0; k < kGroups; ++k) sum += red[k * 256 + t];
      H.ghist[t] = sum;
    }
    return;
  }
  if (t < kAggBlocks) agg[t] = 0u;  // (rank_block synchronises before use)
  int my_gid = -1, my_n = 0;
  run_step::rank_block(
      runs_in.keys, runs_in.vals, runs_in.samples, P.gpb, runs,
      (int)blockIdx.x, S, [&](int64_t base, int pos, uint32_t v) {
        const int gid = (int)base + pos;
        const int orig = (int)base + (int)v;
        perm[gid] = (int32_t)v;
        pack_record(P, means2d, conics, colors, opacities, packed, gid, orig);
        my_n = splat_count[orig];
        gid_count[gid] = my_n;
        my_gid = gid;
      });
  // Each gid's count goes to its emit workgroup's total (the emit's later
  // workgroups start from these): the chunk's element 0 has its smallest
  // gid, so workgroups first .. first + kAggBlocks - 1 are summed in LDS,
  // any further one directly.
  if (t == 0) agg_first = my_gid / kWalkBlockSplats;
  __syncthreads();
  const int first = agg_first;
  if (my_gid >= 0 && my_n != 0) {
    const int wb = my_gid / kWalkBlockSplats;
    if (wb - first < kAggBlocks)
      atomicAdd(&agg[wb - first], (uint32_t)my_n);
    else
      atomicAdd(&block_totals[wb], (uint32_t)my_n);
  }
  __syncthreads();
  if (t < kAggBlocks && agg[t] != 0u) atomicAdd(&block_totals[first + t], agg[t]);
}

// One thread per depth-sorted splat (gid): gathers the attributes of
// orig = perm[gid] into the packed 64-byte record and turns the per-gid
// tile-hit counts into exclusive offsets splat_offsets in the same launch
// (workgroup scan + decoupled look-back).  splat_offsets[num_splats] = N, or
// -1 when N does not fit in int32 (the offsets are then unusable).  With
// orig_slot also orig_slot[orig] = {offset, gid} (the original-order emit's).
__global__ __launch_bounds__(kThreads) void pack_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, const uint32_t* __restrict__ perm,
    const int32_t* __restrict__ splat_count,
    const float4* __restrict__ rec_orig, float4* __restrict__ packed,
    int32_t* __restrict__ splat_offsets, uint64_t* scan_status,
    uint32_t* scan_ticket, uint32_t* err, int2* __restrict__ orig_slot) {
  __shared__ int wsum[kThreads / 64];
  __shared__ long long s_prefix;
  const int vb = take_ticket(scan_ticket);
  const int gid = vb * kThreads + threadIdx.x;
  int n = 0, orig = 0;
  if (gid < P.num_splats) {
    const int batch = gid / P.gpb;
    // (perm is in [0, G) unless a look-back of the depth sort gave up; the
    // clamp keeps the gathers in bounds then, and the status reports it)
    orig = batch * P.gpb + (int)min(perm[gid], (uint32_t)(P.gpb - 1));
    if (rec_orig != nullptr) {  // the count's record: orig replaces the count
      Record r;
#pragma unroll
      for (int k = 0; k < kRecordVec4; ++k)
        r.v[k] = rec_orig[(int64_t)kRecordVec4 * orig + k];
      const uint32_t slot = __float_as_uint(r.v[2].y);
      n = (int)(slot & 0x7fffffffu);
      r.v[2].y = __uint_as_float((uint32_t)orig | (slot & 0x80000000u));
      store_record(packed, gid, r);
    } else {
      pack_record(P, means2d, conics, colors, opacities, packed, gid, orig);
      n = splat_count[orig];
    }
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
      prefix = lookback64_wave(scan_status, vb, err);
      if (lane == 0)
        status_store(&scan_status[vb], kFlagInc64 | (prefix + (uint32_t)total));
    }
    if (lane == 0) s_prefix = (long long)prefix;
  }
  __syncthreads();
  const long long end = s_prefix + pre + inc;
  if (gid < P.num_splats) {
    splat_offsets[gid] = (int)(end - n);
    if (orig_slot != nullptr) orig_slot[orig] = make_int2((int)(end - n), gid);
  }
  if (gid == P.num_splats - 1)
    splat_offsets[P.num_splats] = end > 0x7fffffffLL ? -1 : (int)end;
}

// The records of splats already in depth order (orig = gid), for callers
// that hold the depth-sorted flat attribute arrays themselves (the
// reference's op roles take those arrays, not packed records).
__global__ __launch_bounds__(kThreads) void pack_records_kernel(
    RasterParams P, const float* __restrict__ means2d,
    const float* __restrict__ conics, const float* __restrict__ colors,
    const float* __restrict__ opacities, float4* __restrict__ packed) {
  const int gid = (int)blockIdx.x * kThreads + (int)threadIdx.x;
  if (gid < P.num_splats)
    pack_record(P, means2d, conics, colors, opacities, packed, gid, gid);
}

// emit_kernel<false, true>: the walk in original order over the count's
// records, with the count's recorded step ballots.
struct EmitOrig {
  const float4* rec;       // the count's original-order records (hit count
                           // in the slot)
  const int2* slot;        // per orig: {pair offset, gid} (pack_kernel)
  const uint64_t* bits;    // the count's step ballots (count_block), or null
};

// emit_kernel<true>: the pair offsets are scanned by the emit itself.
struct EmitScan {
  const int32_t* gid_count;     // per-gid tile-hit counts
  int32_t* splat_offsets;       // written: exclusive offsets; [num_splats] = N
                                // (-1 when N does not fit in int32)
  const uint32_t* block_totals; // per emit workgroup: the sum of its gids'
                                // counts (added by rank_pack_kernel)
};

// One pair: (tile, gid) into keys and vals, or, for the two-pass sort of
// tiles below 2^16 and gids below 2^24 (key_bytes), the word
// (tile >> 8) << 24 | gid into keys and the tile's low byte into key_bytes
// (5 bytes instead of 8).
__device__ __forceinline__ void put_pair(uint32_t* __restrict__ keys,
                                         uint32_t* __restrict__ vals,
                                         uint8_t* __restrict__ key_bytes,
                                         int64_t pos, uint32_t tile,
                                         uint32_t gid) {
  if (key_bytes != nullptr) {
    keys[pos] = ((tile >> 8) << 24) | gid;
    key_bytes[pos] = (uint8_t)tile;
  } else {
    keys[pos] = tile;
    vals[pos] = gid;
  }
}

// Pairs are written (and counted in the histograms) only at positions below
// min(N, capacity): with a capacity below N the output is the first
// `capacity` pairs, consistently.  kScan: each workgroup scans its gids'
// counts, starting from the totals of the workgroups before it (their sum:
// no look-back, no order among workgroups), and writes splat_offsets before
// walking (the offsets, not N, bound the positions then: every pair lies
// below N by construction).  Otherwise splat_offsets (and N in
// splat_offsets[num_splats]) come from pack_kernel.  kOrig (not with kScan):
// the workgroups walk the splats in original order, the count's walk, from
// its records (eo.rec) with its recorded ballots (eo.bits): a splat's pairs
// start at eo.slot[orig].x, its certain hits first, then its walk hits,
// numbered by the wavefront's walk hits of the splats before it (its count
// less its certain hits).
template <bool kScan, bool kOrig>
__global__ __launch_bounds__(kThreads) void emit_kernel(
    RasterParams P, const float4* __restrict__ packed,
    const int32_t* __restrict__ splat_offsets, int64_t capacity,
    uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
    uint8_t* __restrict__ key_bytes, int pair_passes, int hist_shift,
    uint32_t* __restrict__ hist_partials,
    uint32_t* ghist_direct, uint32_t* pair_status, int64_t pair_status_words,
    EmitScan sc, EmitOrig eo) {
  static_assert(!(kScan && kOrig), "one source of offsets");
  __shared__ WalkSlots walk[kWaves];
  __shared__ int base[kWaves][kWalkSplats];
  // kOrig: per splat the first position of its walk hits less the wave's
  // walk hits before it, and its gid
  __shared__ int wbase[kOrig ? kWaves : 1][kWalkSplats];
  __shared__ int wgid[kOrig ? kWaves : 1][kWalkSplats];
  // the pair sort's digit histograms in kHistCopies copies (lane l adds to
  // copy l % kHistCopies; rows 257 words apart, so that one digit's copies
  // lie in different LDS banks): hits of one tile row share the row's
  // digit, and a copy per lane group divides their serialisation
  __shared__ uint32_t h[4][kHistCopies][257];
  __shared__ int wsum[kWaves];
  __shared__ long long wbefore[kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // (1) zero the pair sort's look-back status (grid-stride)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + t; i < pair_status_words;
       i += (int64_t)gridDim.x * kThreads)
    pair_status[i] = 0u;
  for (int i = t; i < 4 * kHistCopies * 257; i += kThreads) (&h[0][0][0])[i] = 0u;
  const int vb = (int)blockIdx.x;
  __syncthreads();
  // (2) pair emission (gid: the splat's index in the walk's order, its
  // original index with kOrig)
  const int gid = (vb * kWaves + wave) * kWalkSplats + lane;
  const bool valid = lane < kWalkSplats && gid < P.num_splats;
  const int g = valid ? gid : P.num_splats - 1;
  const float4* __restrict__ src = kOrig ? eo.rec : packed;
  const float4 p0 = src[kRecordVec4 * (int64_t)g + 0];
  const float4 p1 = src[kRecordVec4 * (int64_t)g + 1];
  const SplatGeom s{p0.x, p0.y, p0.z, p0.w, p1.x, p1.y};
  WalkSlots& W = walk[wave];
  int64_t n_eff;
  int total, n_inner;
  if (kScan) {
    // exclusive offsets of the workgroup's gids: wavefront scans, the
    // workgroup's scan, and the totals of the workgroups before it (loaded
    // first, summed after the walk set-up, which overlaps their latency).
    const int n = valid ? sc.gid_count[gid] : 0;
    long long before = 0;
    for (int j = t; j < vb; j += kThreads) before += sc.block_totals[j];
    int inc = n;
#pragma unroll
    for (int off = 1; off < kWalkSplats; off <<= 1) {
      const int y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (lane == kWalkSplats - 1) wsum[wave] = inc;
    total = walk_setup(P, valid, s, g / P.gpb, W, n_inner);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) before += __shfl_xor(before, off, 64);
    if (lane == 0) wbefore[wave] = before;
    __syncthreads();
    long long pre = 0, wg_before = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      pre += (w < wave) ? wsum[w] : 0;
      wg_before += wbefore[w];
    }
    const long long end = wg_before + pre + inc;
    if (valid) {
      sc.splat_offsets[gid] = (int)(end - n);
      // positions at or above the capacity are not written: clamp there
      base[wave][lane] = (int)min((long long)capacity, end - n);
    }
    // (lanes 32..63 alias the next wavefront's gids: only a valid lane
    // writes)
    if (valid && gid == P.num_splats - 1)
      sc.splat_offsets[P.num_splats] = end > 0x7fffffffLL ? -1 : (int)end;
    n_eff = capacity;
  } else if (kOrig) {
    const int n =
        valid ? (int)(__float_as_uint(src[kRecordVec4 * (int64_t)g + 2].y) &
                      0x7fffffffu)
              : 0;
    const int2 sg = valid ? eo.slot[g] : make_int2(0, 0);
    n_eff = min(capacity, (int64_t)max(splat_offsets[P.num_splats], 0));
    total = walk_setup(P, valid, s, g / P.gpb, W, n_inner);
    // walk hits of the wavefront's splats up to this one
    const int w = n - n_inner;
    int inc = w;
#pragma unroll
    for (int off = 1; off < kWalkSplats; off <<= 1) {
      const int y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (lane < kWalkSplats) {
      base[wave][lane] = sg.x;
      wbase[kOrig ? wave : 0][lane] = sg.x + n_inner - (inc - w);
      wgid[kOrig ? wave : 0][lane] = sg.y;
    }
  } else {
    if (lane < kWalkSplats) base[wave][lane] = splat_offsets[g];
    n_eff = min(capacity, (int64_t)max(splat_offsets[P.num_splats], 0));
    total = walk_setup(P, valid, s, g / P.gpb, W, n_inner);
  }
  const int gid0 = gid - lane;
  // The wavefront's splats own consecutive ranges starting at the first
  // one's offset; each range starts with the splat's certain hits
  // (inner_tiles, written below) and the walk's hits follow, arriving in
  // splat order: a walk hit's position is that offset plus the hits before
  // it (running total + lanes below) plus the certain hits of the splats up
  // to its own.
  const int64_t wave_base = base[wave][0];
  int64_t run = 0;
  const uint64_t* const rec =
      (kOrig && eo.bits != nullptr)
          ? eo.bits + (int64_t)(vb * kWaves + wave) * kHitSlab
          : nullptr;
  walk_candidates(P, W, total, rec, [&](uint64_t hm, bool hit, int sl,
                                        int tile, int) {
    const int64_t pos =
        kOrig ? (hit ? (int64_t)wbase[kOrig ? wave : 0][sl] : 0) + run +
                    hits_below(hm, lane)
              : wave_base + run + hits_below(hm, lane) +
                    (hit ? W.ni_incl[sl] : 0);
    run += __popcll(hm);
    // (pos >= 0 whenever n_eff > 0, unless a look-back of the depth sort
    // gave up and left the original-order offsets unwritten)
    if (hit && pos < n_eff && (!kOrig || pos >= 0)) {
      put_pair(keys, vals, key_bytes, pos, (uint32_t)tile,
               kOrig ? (uint32_t)wgid[kOrig ? wave : 0][sl]
                     : (uint32_t)(gid0 + sl));
      for (int p = 0; p < pair_passes; ++p)
        atomicAdd(&h[p][lane % kHistCopies]
                     [((uint32_t)tile >> (hist_shift + 8 * p)) & 255u],
                  1u);
    }
  });
  // The certain hits of each splat, row by row at the start of its range.
  uint64_t with_inner = __ballot(lane < kWalkSplats && n_inner > 0);
  for (; with_inner != 0ull; with_inner &= with_inner - 1ull) {
    const int sl = (int)__builtin_ctzll(with_inner);
    const int4 in = W.inner[sl];
    const int ni = in.z * in.w;
    const int4 bx = W.box[sl];
    const int64_t off = base[wave][sl];
    const uint32_t sg = kOrig ? (uint32_t)wgid[kOrig ? wave : 0][sl]
                              : (uint32_t)(gid0 + sl);
    for (int i = lane; i < ni; i += 64) {
      const int dy = div_small(i, in.z);
      const int tile = bx.w + (bx.y + in.y + dy) * P.tiles_x +
                       (bx.x + in.x + (i - dy * in.z));
      const int64_t pos = off + i;
      if (pos < n_eff && (!kOrig || pos >= 0)) {
        put_pair(keys, vals, key_bytes, pos, (uint32_t)tile, sg);
        for (int p = 0; p < pair_passes; ++p)
          atomicAdd(&h[p][lane % kHistCopies]
                       [((uint32_t)tile >> (hist_shift + 8 * p)) & 255u],
                    1u);
      }
    }
  }
  // (3) this workgroup's digit histograms for the pair sort: added to the
  // zeroed global histograms (ghist_direct, few workgroups) or stored as
  // hist_partials[(p * 256 + d) * nblk + workgroup] for hist_reduce_kernel
  __syncthreads();
  for (int p = 0; p < pair_passes; ++p) {
    uint32_t c = 0u;
#pragma unroll
    for (int q = 0; q < kHistCopies; ++q) c += h[p][q][t];
    if (ghist_direct != nullptr) {
      if (c) atomicAdd(&ghist_direct[p * 256 + t], c);
    } else {
      hist_partials[((int64_t)p * 256 + t) * gridDim.x + blockIdx.x] = c;
    }
  }
}

// ghist[p][d] = sum over the emit workgroups of their digit-d counts of pass
// p: one workgroup per (p, d) reads that row of partials contiguously.
__global__ __launch_bounds__(kThreads) void hist_reduce_kernel(
    const uint32_t* __restrict__ hist_partials, int nblk,
    uint32_t* __restrict__ ghist) {
  __shared__ uint32_t part[kThreads / 64];
  const uint32_t* row = hist_partials + (int64_t)blockIdx.x * nblk;
  // eight independent loads in flight per thread
  uint32_t acc[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  int b = threadIdx.x;
  for (; b + 7 * kThreads < nblk; b += 8 * kThreads) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += row[b + u * kThreads];
  }
  for (; b < nblk; b += kThreads) acc[0] += row[b];
  uint32_t v = 0u;
#pragma unroll
  for (int u = 0; u < 8; ++u) v += acc[u];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0u;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) t += part[w];
    ghist[blockIdx.x] = t;   // blockIdx.x = p * 256 + d
  }
}

// tile_offsets from the sorted tile keys: index i (0 <= i <= n) is the first
// pair of every tile t with keys[i-1] < t <= keys[i] (keys[-1] = -1,
// keys[n] = num_tiles), so tile_offsets[num_tiles] = n.  With n_dev the key
// count is min(*n_dev, n).  Grid-stride over the indices, kRangeUnroll of
// them per iteration with all their loads issued first (indices clamped into
// [0, n_cap), so the loads need no branch), which keeps a launch over 1e8
// keys to a few thousand workgroups.
constexpr int kRangeUnroll = 4;
constexpr int kRangeMaxBlocks = 2048;
struct StatusWords {
  const uint32_t* err[3];  // give-up status words (null: not used)
  int32_t* out;            // their OR (null: not reported)
  int32_t* long_flag;      // null, or a device word (zero before the
                           // launch) set to 1 if a tile range is longer
                           // than kHandoffPairs
  ZeroSpan zero[2];        // zeroed by the launch on the side
};

__global__ __launch_bounds__(kThreads) void ranges_kernel(
    const uint32_t* __restrict__ sorted_keys, int64_t n_cap,
    const int32_t* __restrict__ n_dev, int num_tiles,
    int32_t* __restrict__ tile_offsets, StatusWords sw) {
  // Every look-back of the binning ran in an earlier launch.  If one gave
  // up, the pairs may hold unwritten entries: every tile is emptied instead
  // (the compositors then read no pair), and the status says why.
  uint32_t e = 0u;
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if (sw.err[k] != nullptr) e |= *sw.err[k];
  if (blockIdx.x == 0 && threadIdx.x == 0 && sw.out != nullptr)
    *sw.out = (int32_t)e;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
#pragma unroll
  for (int z = 0; z < 2; ++z)
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
         i < sw.zero[z].n; i += stride)
      sw.zero[z].p[i] = 0u;
  if (e != 0u) {
    for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
         t <= num_tiles; t += stride)
      tile_offsets[t] = 0;
    return;
  }
  const int64_t n = n_dev ? min(n_cap, (int64_t)max(*n_dev, 0)) : n_cap;
  bool long_range = false;  // a range starting here exceeds kHandoffPairs
  for (int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; i0 <= n;
       i0 += kRangeUnroll * stride) {
    uint32_t kp[kRangeUnroll], kc[kRangeUnroll];
#pragma unroll
    for (int u = 0; u < kRangeUnroll; ++u) {
      const int64_t i = min(i0 + u * stride, n);
      kp[u] = sorted_keys[max(i - 1, (int64_t)0)];
      kc[u] = sorted_keys[max(min(i, n - 1), (int64_t)0)];
    }
#pragma unroll
    for (int u = 0; u < kRangeUnroll; ++u) {
      const int64_t i = i0 + u * stride;
      if (i > n) break;
      const int64_t prev = (i == 0) ? -1 : (int64_t)kp[u];
      const int64_t cur = (i == n) ? (int64_t)num_tiles
                                   : min((int64_t)kc[u], (int64_t)num_tiles);
      for (int64_t t = prev + 1; t <= cur; ++t) tile_offsets[t] = (int32_t)i;
      // tile cur's range starts at i: longer than kHandoffPairs iff its
      // key is still there kHandoffPairs places on
      if (sw.long_flag != nullptr && prev != cur && i + kHandoffPairs < n)
        long_range |= sorted_keys[i + kHandoffPairs] == kc[u];
    }
  }
  if (sw.long_flag != nullptr && __ballot(long_range) != 0ull &&
      (threadIdx.x & 63) == 0)
    *sw.long_flag = 1;
}

// After radix_pair_sort_ranges wrote every tile_offsets entry: the
// binning's status, empty ranges (all zero) when a look-back gave up or no
// pair was emitted, the long-range flag and the zero spans, as ranges_kernel
// does beside its ranges.
__global__ __launch_bounds__(kThreads) void ranges_finish_kernel(
    int64_t n_cap, const int32_t* __restrict__ n_dev, int num_tiles,
    int32_t* __restrict__ tile_offsets, StatusWords sw) {
  uint32_t e = 0u;
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if (sw.err[k] != nullptr) e |= *sw.err[k];
  if (blockIdx.x == 0 && threadIdx.x == 0 && sw.out != nullptr)
    *sw.out = (int32_t)e;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t first = (int64_t)blockIdx.x * kThreads + threadIdx.x;
#pragma unroll
  for (int z = 0; z < 2; ++z)
    for (int64_t i = first; i < sw.zero[z].n; i += stride) sw.zero[z].p[i] = 0u;
  const int64_t n = n_dev ? min(n_cap, (int64_t)max(*n_dev, 0)) : n_cap;
  if (e != 0u || n == 0) {
    for (int64_t t = first; t <= num_tiles; t += stride) tile_offsets[t] = 0;
    return;
  }
  bool long_range = false;
  for (int64_t t = first; t < num_tiles; t += stride)
    long_range |= tile_offsets[t + 1] - tile_offsets[t] > kHandoffPairs;
  if (sw.long_flag != nullptr && __ballot(long_range) != 0ull &&
      (threadIdx.x & 63) == 0)
    *sw.long_flag = 1;
}

__global__ void host_report_kernel(HostReport R) {
  if (threadIdx.x == 0) write_host_report(R);
}

// Bucket counting sort (launch_bucket_sort): one workgroup per bucket of
// 2^low_bits tiles, whose pairs the onesweep pass on the higher tile bits
// left contiguous and in gid order.  A pass takes up to kBucketChunk of the
// bucket's pairs: wavefront w the pairs [w*64*R, (w+1)*64*R) of the pass,
// round r of it the 64 from w*64*R + r*64 (R = kBucketRounds), so that the
// order (pass, wavefront, round, lane) is the pairs' order in the bucket.
// A pair's output index is its digit's start, plus the pairs of that digit
// in earlier passes, in earlier wavefronts of its pass, in the lane's earlier
// rounds and in lower lanes of its round (ballot match): a stable sort.  The
// digit starts are the scan of the digit counts: counted by the single pass
// of a bucket of at most kBucketChunk pairs, else by a counting sweep first.
constexpr int kBucketWaves = 16;
constexpr int kBucketThreads = kBucketWaves * 64;
constexpr int kBucketRounds = kBucketChunk / kBucketThreads;

struct BucketLds {
  uint32_t cnt[kBucketWaves][256];  // per-wavefront digit counts, then the
                                    // digit's output index for the wavefront
  uint32_t run[256];                // digit's next output index (sweeps)
  uint32_t wsum[kBucketWaves];
};

// Exclusive scan of v over threads 0..255 of the workgroup (0 elsewhere);
// every thread calls it (it synchronises the workgroup).
__device__ __forceinline__ uint32_t bucket_digit_scan(uint32_t v,
                                                      BucketLds& S) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(inc, off, 64);
    if (lane >= off) inc += y;
  }
  if (lane == 63 && wave < 4) S.wsum[wave] = inc;
  __syncthreads();
  uint32_t pre = 0u;
#pragma unroll
  for (int w = 0; w < 4; ++w) pre += (w < wave) ? S.wsum[w] : 0u;
  __syncthreads();  // wsum is read before it is written again
  return pre + inc - v;
}

__global__ __launch_bounds__(kBucketThreads) void bucket_sort_kernel(
    BucketSortArgs A) {
  __shared__ BucketLds S;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int b = blockIdx.x;
  const int ndig = 1 << A.low_bits;
  const uint32_t dmask = (uint32_t)ndig - 1u;
  const int tile0 = b << A.low_bits;
  uint32_t e = 0u;
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if (A.err[k] != nullptr) e |= *A.err[k];
  if (b == 0 && t == 0 && A.status_out != nullptr) *A.status_out = (int32_t)e;
  const int64_t n =
      A.n_dev ? min(A.n, (int64_t)max(*A.n_dev, 0)) : A.n;
  // the bucket's first index, the sizes of buckets 0..b-1 (b < 256), summed
  // by every wavefront (no workgroup barrier)
  uint32_t before = 0u, all = 0u;
#pragma unroll
  for (int i = lane; i < 256; i += 64) {
    const uint32_t v = A.bucket_sizes[i];
    before += (i < b) ? v : 0u;
    all += v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    before += __shfl_xor(before, off, 64);
    all += __shfl_xor(all, off, 64);
  }
  const uint32_t base = before;
  // (the sizes add up to n by construction; the clamp keeps every access
  // inside the first n pairs regardless)
  const uint32_t size = (uint32_t)min(
      (int64_t)A.bucket_sizes[b], max((int64_t)0, n - (int64_t)base));
  for (int i = t; i < kBucketWaves * 256; i += kBucketThreads)
    (&S.cnt[0][0])[i] = 0u;
  const int64_t stride = (int64_t)gridDim.x * kBucketThreads;
#pragma unroll
  for (int z = 0; z < 2; ++z)
    for (int64_t i = (int64_t)b * kBucketThreads + t; i < A.zero[z].n;
         i += stride)
      A.zero[z].p[i] = 0u;
  // A look-back of the binning gave up: every tile range is empty (as in
  // ranges_kernel).
  if (e != 0u) {
    for (int d = t; d < ndig; d += kBucketThreads) {
      if (tile0 + d >= A.num_tiles) break;
      A.tile_offsets[tile0 + d] = 0;
      if (A.tile_counts != nullptr) A.tile_counts[tile0 + d] = 0;
    }
    if (b == 0 && t == 0) A.tile_offsets[A.num_tiles] = 0;
    return;
  }
  // the end of the last range: the pairs the buckets hold (n by
  // construction), so that no range reaches past the sorted pairs
  if (b == 0 && t == 0)
    A.tile_offsets[A.num_tiles] = (int32_t)min(n, (int64_t)all);
  // An empty bucket (no pairs, or none left below n): its tiles' ranges are
  // empty and start at the bucket's first index (at most n, so that the
  // offsets stay monotone when the buffers hold fewer pairs than the
  // buckets).  The chunk loop below writes the ranges of the other buckets;
  // it does not run for size 0.  (size is the same for the whole workgroup,
  // so no thread waits at a barrier that the others skip.)
  if (size == 0u) {
    const int32_t start = (int32_t)min((int64_t)base, n);
    for (int d = t; d < ndig; d += kBucketThreads) {
      if (tile0 + d >= A.num_tiles) break;
      A.tile_offsets[tile0 + d] = start;
      if (A.tile_counts != nullptr) A.tile_counts[tile0 + d] = 0;
    }
    return;
  }
  const bool sweep = size > (uint32_t)kBucketChunk;
  bool long_range = false;
  if (sweep) {
    // counting sweep, then the digit starts
    if (t < 256) S.run[t] = 0u;
    __syncthreads();
    for (uint32_t i = t; i < size; i += kBucketThreads)
      atomicAdd(&S.run[A.keys[base + i] & dmask], 1u);
    __syncthreads();
    const uint32_t tot = t < 256 ? S.run[t] : 0u;
    const uint32_t first = base + bucket_digit_scan(tot, S);
    if (t < ndig && tile0 + t < A.num_tiles) {
      A.tile_offsets[tile0 + t] = (int32_t)first;
      if (A.tile_counts != nullptr) A.tile_counts[tile0 + t] = (int32_t)tot;
      long_range = tot > (uint32_t)kHandoffPairs;
    }
    if (t < 256) S.run[t] = first;
    __syncthreads();
  }
  const uint64_t lt = run_step::lanes_below();
  for (uint32_t c0 = 0; c0 < size; c0 += kBucketChunk) {
    uint32_t d[kBucketRounds], v[kBucketRounds], rank[kBucketRounds];
    bool ok[kBucketRounds];
#pragma unroll
    for (int r = 0; r < kBucketRounds; ++r) {
      const uint32_t li =
          c0 + (uint32_t)(wave * 64 * kBucketRounds + r * 64 + lane);
      ok[r] = li < size;
      d[r] = ok[r] ? (A.keys[base + li] & dmask) : 0u;
      v[r] = ok[r] ? A.vals[base + li] : 0u;
    }
    __syncthreads();  // the counts are zero
#pragma unroll
    for (int r = 0; r < kBucketRounds; ++r) {
      const uint64_t peers =
          run_step::same_digit_lanes(d[r]) & __builtin_amdgcn_ballot_w64(ok[r]);
      const uint32_t below = (uint32_t)__popcll(peers & lt);
      // every lane of the digit reads the count, then its lowest lane adds
      // the group's size (one wavefront's LDS accesses take effect in
      // program order)
      const uint32_t old = S.cnt[wave][d[r]];
      __builtin_amdgcn_wave_barrier();
      if (ok[r] && below == 0u)
        S.cnt[wave][d[r]] = old + (uint32_t)__popcll(peers);
      rank[r] = old + below;
    }
    __syncthreads();
    // digit t: its wavefronts' output indices
    uint32_t tot = 0u;
    if (t < 256) {
#pragma unroll
      for (int w = 0; w < kBucketWaves; ++w) tot += S.cnt[w][t];
    }
    uint32_t first;
    if (sweep) {
      first = t < 256 ? S.run[t] : 0u;
    } else {
      first = base + bucket_digit_scan(tot, S);
      if (t < ndig && tile0 + t < A.num_tiles) {
        A.tile_offsets[tile0 + t] = (int32_t)first;
        if (A.tile_counts != nullptr) A.tile_counts[tile0 + t] = (int32_t)tot;
        long_range = tot > (uint32_t)kHandoffPairs;
      }
    }
    if (t < 256) {
      uint32_t o = first;
#pragma unroll
      for (int w = 0; w < kBucketWaves; ++w) {
        const uint32_t c = S.cnt[w][t];
        S.cnt[w][t] = o;
        o += c;
      }
      if (sweep) S.run[t] = o;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kBucketRounds; ++r)
      if (ok[r]) A.binned_ids[S.cnt[wave][d[r]] + rank[r]] = v[r];
    if (c0 + kBucketChunk < size) {
      __syncthreads();  // the indices are read before they are cleared
      for (int i = t; i < kBucketWaves * 256; i += kBucketThreads)
        (&S.cnt[0][0])[i] = 0u;
    }
  }
  if (A.long_flag != nullptr && __ballot(long_range) != 0ull && lane == 0)
    *A.long_flag = 1;
}

__global__ __launch_bounds__(kThreads) void counts_kernel(
    const int32_t* __restrict__ tile_offsets, int num_tiles,
    int32_t* __restrict__ tile_counts) {
  const int t = blockIdx.x * kThreads + threadIdx.x;
  if (t < num_tiles) tile_counts[t] = tile_offsets[t + 1] - tile_offsets[t];
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

int count_blocks(const RasterParams& P) {
  return (P.num_splats + kWalkBlockSplats - 1) / kWalkBlockSplats;
}

size_t hit_bits_words(const RasterParams& P) {
  return (size_t)count_blocks(P) * kWaves * kHitSlab;
}

int launch_count(const RasterParams& P, const float* means2d,
                 const float* conics, const float* opacities,
                 int32_t* splat_count, int32_t* block_sums,
                 int32_t* pair_count, uint32_t* zero_words,
                 int64_t n_zero_words, hipStream_t stream,
                 const float* colors, float* rec_orig, uint64_t* hit_bits) {
  const int nblk = count_blocks(P);
  launch_traced("count_kernel", count_kernel, dim3((unsigned)nblk),
                dim3(kThreads), 0, stream, P, means2d, conics, opacities,
                colors, reinterpret_cast<float4*>(rec_orig), splat_count,
                block_sums, zero_words, n_zero_words, hit_bits);
  int rc = check_launch("count_kernel");
  if (rc || pair_count == nullptr) return rc;
  launch_traced("sum_kernel", sum_kernel, dim3(1), dim3(kThreads), 0, stream,
                block_sums, nblk, pair_count);
  return check_launch("sum_kernel");
}

int count_depth_runs_blocks(const RasterParams& P) {
  constexpr int kSplatsPerBlock = run_step::kRunWaves * kWalkSplats;
  return (P.num_splats + kSplatsPerBlock - 1) / kSplatsPerBlock;
}

int launch_count_depth_runs(const RasterParams& P, const float* means2d,
                            const float* conics, const float* opacities,
                            int32_t* splat_count, uint32_t* zero_words,
                            int64_t n_zero_words, const float* depths,
                            void* depth_buffers, hipStream_t stream,
                            const CountHist& H) {
  if (P.num_splats == 0 || !depth_small_ok(P.gpb)) {
    set_error("count + depth runs: needs 1..131072 splats per image");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int runs = run_step::runs_of(P.gpb);
  const int run_blocks = P.batch * runs;
  const int cblocks = count_depth_runs_blocks(P);
  launch_traced("count_depth_runs_kernel", count_depth_runs_kernel,
                dim3((unsigned)(run_blocks + cblocks)),
                dim3(run_step::kRunThreads), 0, stream, P, means2d, conics,
                opacities, splat_count, zero_words, n_zero_words, depths, runs,
                run_blocks,
                run_step::run_buffers(depth_buffers, P.gpb, P.batch), H);
  return check_launch("count_depth_runs_kernel");
}

int launch_rank_pack(const RasterParams& P, const float* means2d,
                     const float* conics, const float* colors,
                     const float* opacities, void* depth_buffers,
                     const int32_t* splat_count, int32_t* perm, float* packed,
                     int32_t* gid_count, uint32_t* block_totals,
                     hipStream_t stream, const CountHist& H) {
  if (P.num_splats == 0 || !depth_small_ok(P.gpb)) {
    set_error("rank + pack: needs 1..131072 splats per image");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int blocks_per_seg =
      (P.gpb + run_step::kRankElems - 1) / run_step::kRankElems;
  launch_traced("rank_pack_kernel", rank_pack_kernel,
                dim3((unsigned)((int64_t)P.batch * blocks_per_seg +
                                (H.parts != nullptr ? 1 : 0))),
                dim3(run_step::kRankBlock), 0, stream, P, means2d, conics,
                colors, opacities,
                run_step::run_buffers(depth_buffers, P.gpb, P.batch),
                run_step::runs_of(P.gpb), splat_count, perm,
                reinterpret_cast<float4*>(packed), gid_count, block_totals, H);
  return check_launch("rank_pack_kernel");
}

int launch_pack(const RasterParams& P, const float* means2d,
                const float* conics, const float* colors,
                const float* opacities, const uint32_t* perm,
                const int32_t* splat_count, float* packed,
                int32_t* splat_offsets, uint64_t* scan_status,
                uint32_t* scan_ticket, uint32_t* err, hipStream_t stream,
                const float* rec_orig, int32_t* orig_slot) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  launch_traced("pack_kernel", pack_kernel, dim3(grid), dim3(kThreads), 0,
                stream, P, means2d, conics, colors, opacities, perm,
                splat_count, reinterpret_cast<const float4*>(rec_orig),
                reinterpret_cast<float4*>(packed), splat_offsets, scan_status,
                scan_ticket, err, reinterpret_cast<int2*>(orig_slot));
  return check_launch("pack_kernel");
}

int launch_pack_records(const RasterParams& P, const float* means2d,
                        const float* conics, const float* colors,
                        const float* opacities, float* packed,
                        hipStream_t stream) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const unsigned grid = (unsigned)((P.num_splats + kThreads - 1) / kThreads);
  launch_traced("pack_records_kernel", pack_records_kernel, dim3(grid),
                dim3(kThreads), 0, stream, P, means2d, conics, colors,
                opacities, reinterpret_cast<float4*>(packed));
  return check_launch("pack_records_kernel");
}

int count_scan_blocks(const RasterParams& P) {
  return (P.num_splats + kThreads - 1) / kThreads;
}

int emit_blocks(const RasterParams& P) {
  return (P.num_splats + kWalkBlockSplats - 1) / kWalkBlockSplats;
}

int launch_emit(const RasterParams& P, const float* packed,
                const int32_t* splat_offsets, int64_t capacity, uint32_t* keys,
                uint32_t* vals, int pair_passes, uint32_t* hist_partials,
                uint32_t* pair_ghist, uint32_t* pair_status,
                int64_t pair_status_words, hipStream_t stream,
                const EmitScanArgs* scan, int hist_shift,
                uint8_t* key_bytes, const EmitOrigArgs* orig) {
  if (P.num_splats == 0) return GSPLAT_OK;
  const int nblk = emit_blocks(P);
  // Few workgroups add their histograms atomically (pair_ghist is zeroed
  // by count_kernel), which saves the reduction launch; many would contend.
  const bool direct = nblk <= kDirectHistBlocks;
  if (scan != nullptr) {
    const EmitScan sc{scan->gid_count, scan->splat_offsets,
                      scan->block_totals};
    launch_traced("emit_kernel<true>", emit_kernel<true, false>,
                  dim3((unsigned)nblk), dim3(kThreads), 0, stream, P,
                  reinterpret_cast<const float4*>(packed), nullptr, capacity,
                  keys, vals, key_bytes, pair_passes, hist_shift, hist_partials,
                  direct ? pair_ghist : nullptr, pair_status, pair_status_words,
                  sc, EmitOrig{});
  } else if (orig != nullptr) {
    const EmitOrig eo{reinterpret_cast<const float4*>(orig->rec_orig),
                      reinterpret_cast<const int2*>(orig->orig_slot),
                      orig->hit_bits};
    launch_traced("emit_kernel<orig>", emit_kernel<false, true>,
                  dim3((unsigned)nblk), dim3(kThreads), 0, stream, P,
                  reinterpret_cast<const float4*>(packed), splat_offsets,
                  capacity, keys, vals, key_bytes, pair_passes, hist_shift,
                  hist_partials,
                  direct ? pair_ghist : nullptr, pair_status, pair_status_words,
                  EmitScan{}, eo);
  } else {
    launch_traced("emit_kernel<false>", emit_kernel<false, false>,
                  dim3((unsigned)nblk), dim3(kThreads), 0, stream, P,
                  reinterpret_cast<const float4*>(packed), splat_offsets,
                  capacity, keys, vals, key_bytes, pair_passes, hist_shift,
                  hist_partials,
                  direct ? pair_ghist : nullptr, pair_status, pair_status_words,
                  EmitScan{}, EmitOrig{});
  }
  int rc = check_launch("emit_kernel");
  if (rc || pair_passes == 0 || direct) return rc;
  launch_traced("hist_reduce_kernel", hist_reduce_kernel,
                dim3((unsigned)(pair_passes * 256)), dim3(kThreads), 0, stream,
                hist_partials, nblk, pair_ghist);
  return check_launch("hist_reduce_kernel");
}

int launch_tile_ranges(const uint32_t* sorted_keys, int64_t n, int num_tiles,
                       int32_t* tile_offsets, int32_t* tile_counts,
                       hipStream_t stream, const int32_t* n_dev,
                       const uint32_t* err0, const uint32_t* err1,
                       const uint32_t* err2, int32_t* status_out,
                       int32_t* long_flag, const ZeroSpan* zero) {
  int rc = GSPLAT_OK;
  if (zero != nullptr && (num_tiles <= 0 || n == 0))
    rc = launch_zero2(zero[0].p, zero[0].n, zero[1].p, zero[1].n, stream);
  if (rc) return rc;
  if (num_tiles <= 0)
    return status_out ? launch_fill_i32(status_out, 0, 1, stream) : GSPLAT_OK;
  StatusWords sw{{err0, err1, err2}, status_out, long_flag, {}};
  if (zero != nullptr) {
    sw.zero[0] = zero[0];
    sw.zero[1] = zero[1];
  }
  if (n == 0) {
    rc = launch_fill_i32(tile_offsets, 0, (int64_t)num_tiles + 1, stream);
    if (!rc && status_out) rc = launch_fill_i32(status_out, 0, 1, stream);
  } else {
    int64_t grid = (n + 1 + kThreads - 1) / kThreads;
    if (grid > kRangeMaxBlocks) grid = kRangeMaxBlocks;
    launch_traced("ranges_kernel", ranges_kernel, dim3((unsigned)grid),
                  dim3(kThreads), 0, stream, sorted_keys, n, n_dev, num_tiles,
                  tile_offsets, sw);
    rc = check_launch("ranges_kernel");
  }
  if (rc || tile_counts == nullptr) return rc;
  launch_traced("counts_kernel", counts_kernel,
                dim3((unsigned)((num_tiles + kThreads - 1) / kThreads)),
                dim3(kThreads), 0, stream, tile_offsets, num_tiles,
                tile_counts);
  return check_launch("counts_kernel");
}

int launch_ranges_finish(int64_t n, int num_tiles, int32_t* tile_offsets,
                         int32_t* tile_counts, hipStream_t stream,
                         const int32_t* n_dev, const uint32_t* err0,
                         const uint32_t* err1, const uint32_t* err2,
                         int32_t* status_out, int32_t* long_flag,
                         const ZeroSpan* zero) {
  if (num_tiles <= 0 || n == 0)
    return launch_tile_ranges(nullptr, 0, num_tiles, tile_offsets, tile_counts,
                              stream, n_dev, err0, err1, err2, status_out,
                              long_flag, zero);
  StatusWords sw{{err0, err1, err2}, status_out, long_flag, {}};
  if (zero != nullptr) {
    sw.zero[0] = zero[0];
    sw.zero[1] = zero[1];
  }
  // (sized for the zero spans too)
  int64_t work = (int64_t)num_tiles + 1;
  for (int z = 0; z < 2; ++z) work = std::max(work, sw.zero[z].n);
  int64_t grid = (work + kThreads - 1) / kThreads;
  if (grid > kRangeMaxBlocks) grid = kRangeMaxBlocks;
  launch_traced("ranges_finish_kernel", ranges_finish_kernel,
                dim3((unsigned)grid), dim3(kThreads), 0, stream, n, n_dev,
                num_tiles, tile_offsets, sw);
  int rc = check_launch("ranges_finish_kernel");
  if (rc || tile_counts == nullptr) return rc;
  launch_traced("counts_kernel", counts_kernel,
                dim3((unsigned)((num_tiles + kThreads - 1) / kThreads)),
                dim3(kThreads), 0, stream, tile_offsets, num_tiles,
                tile_counts);
  return check_launch("counts_kernel");
}

int launch_bucket_sort(const BucketSortArgs& A, hipStream_t stream) {
  if (A.num_tiles <= 0 || A.low_bits < 1 || A.low_bits > 8) {
    set_error("bucket sort: needs tiles and 1..8 low bits");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int64_t buckets =
      ((int64_t)A.num_tiles + (1 << A.low_bits) - 1) >> A.low_bits;
  if (buckets > 256) {
    set_error("bucket sort: more than 256 buckets");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  launch_traced("bucket_sort_kernel", bucket_sort_kernel,
                dim3((unsigned)buckets), dim3(kBucketThreads), 0, stream, A);
  return check_launch("bucket_sort_kernel");
}

int launch_host_report(const HostReport& R, hipStream_t stream) {
  launch_traced("host_report_kernel", host_report_kernel, dim3(1), dim3(64), 0,
                stream, R);
  return check_launch("host_report_kernel");
}

int launch_zero2(uint32_t* a, int64_t na, uint32_t* b, int64_t nb,
                 hipStream_t stream) {
  const int64_t n = na > nb ? na : nb;
  if (n <= 0) return GSPLAT_OK;
  int64_t grid = (n + 255) / 256;
  if (grid > 4096) grid = 4096;
  launch_traced("zero2_kernel", zero2_kernel, dim3((unsigned)grid), dim3(256),
                0, stream, a, na, b, nb);
  return check_launch("zero2_kernel");
}

int launch_fill_i32(int32_t* dst, int32_t value, int64_t n,
                    hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (n + 255) / 256;
  launch_traced("fill_i32_kernel", fill_i32_kernel, dim3((unsigned)grid),
                dim3(256), 0, stream, dst, value, n);
  return check_launch("fill_i32_kernel");
}

int launch_zero_grads(float* g_m, float* g_q, float* g_c, float* g_o,
                      int64_t n, hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (3 * n + 255) / 256;
  launch_traced("zero_grads_kernel", zero_grads_kernel, dim3((unsigned)grid),
                dim3(256), 0, stream, g_m, g_q, g_c, g_o, n);
  return check_launch("zero_grads_kernel");
}

int launch_fill_f32(float* dst, float value, int64_t n, hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  const int64_t grid = (n + 255) / 256;
  launch_traced("fill_f32_kernel", fill_f32_kernel, dim3((unsigned)grid),
                dim3(256), 0, stream, dst, value, n);
  return check_launch("fill_f32_kernel");
}

}  // namespace gs
