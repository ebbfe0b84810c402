// radix_sort.hip -- stable LSD radix sort of (uint32 key, uint32 value) pairs
// with 8-bit digits, independently inside equal-length segments.
//
// One launch per digit pass ("onesweep"): the global digit histogram of every
// pass is known before the first pass (rs_global_hist_kernel, or supplied by
// the caller), so a workgroup only needs the counts of the workgroups before
// it in its segment, which it gets by decoupled look-back (lookback.h).
//
// Inside a workgroup (256 lanes, 64*kR elements per wavefront) each wavefront
// ranks its consecutive elements 64 at a time: lanes holding the same digit
// are found with eight ballots ("match"), the rank is the popcount of
// matching lower lanes plus the wave's running count of that digit, which the
// digit's lowest lane bumps with one LDS atomic (returning the old count) and
// broadcasts to its peers.  Element order inside a workgroup is
// (wave, round, lane) = input order, which makes the sort stable.  The block
// is then staged in LDS in sorted order and written out so that each digit's
// run is one contiguous, coalesced store.
#include "gs_internal.h"
#include "lookback.h"

namespace gs {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
// Look-back window: predecessor statuses read per round trip (8 measured
// faster than 4, 16, 32 or 64 on 1.2e8-pair sorts).
constexpr int kLookbackWindow = 8;

__device__ __forceinline__ uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63u;
  return (lane == 0u) ? 0ull : (~0ull >> (64u - lane));
}

// Lanes of `active` whose 8-bit digit equals this lane's digit.  Per bit:
// n = the bit sign-extended (0 or ~0), b = the wavefront's ballot of it; the
// lanes that agree with this lane are ~(b ^ n), so m &= ~(b ^ n) is one
// three-input bit operation per 32-bit half (truth table 0x90 for
// src0 & ~(src1 ^ src2) with the operand patterns 0xF0, 0xCC, 0xAA).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t active) {
  uint32_t lo = (uint32_t)active, hi = (uint32_t)(active >> 32);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    uint32_t n = (uint32_t)__builtin_amdgcn_sbfe((int)d, bit, 1);
    // (through an empty asm: the ballot then compares n itself instead of
    // recomputing the bit with a shift)
    asm volatile("" : "+v"(n));
    const uint64_t b = __builtin_amdgcn_ballot_w64(n != 0u);
    lo = __builtin_amdgcn_bitop3_b32(lo, (uint32_t)b, n, 0x90);
    hi = __builtin_amdgcn_bitop3_b32(hi, (uint32_t)(b >> 32), n, 0x90);
  }
  return ((uint64_t)hi << 32) | lo;
}

// match_digit for two rounds at once: the two dependency chains interleave.
__device__ __forceinline__ void match_digit2(uint32_t d0, uint32_t d1,
                                             uint64_t act0, uint64_t act1,
                                             uint64_t& m0, uint64_t& m1) {
  uint32_t lo0 = (uint32_t)act0, hi0 = (uint32_t)(act0 >> 32);
  uint32_t lo1 = (uint32_t)act1, hi1 = (uint32_t)(act1 >> 32);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    uint32_t n0 = (uint32_t)__builtin_amdgcn_sbfe((int)d0, bit, 1);
    uint32_t n1 = (uint32_t)__builtin_amdgcn_sbfe((int)d1, bit, 1);
    asm volatile("" : "+v"(n0), "+v"(n1));
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(n0 != 0u);
    const uint64_t b1 = __builtin_amdgcn_ballot_w64(n1 != 0u);
    lo0 = __builtin_amdgcn_bitop3_b32(lo0, (uint32_t)b0, n0, 0x90);
    hi0 = __builtin_amdgcn_bitop3_b32(hi0, (uint32_t)(b0 >> 32), n0, 0x90);
    lo1 = __builtin_amdgcn_bitop3_b32(lo1, (uint32_t)b1, n1, 0x90);
    hi1 = __builtin_amdgcn_bitop3_b32(hi1, (uint32_t)(b1 >> 32), n1, 0x90);
  }
  m0 = ((uint64_t)hi0 << 32) | lo0;
  m1 = ((uint64_t)hi1 << 32) | lo1;
}

// Element i of the array at base, addressed as a uniform base plus a 32-bit
// byte offset (i * sizeof(T) < 2^32 for every caller: segments hold at most
// 2^29 elements), which loads and stores take as one register.
template <class T>
__device__ __forceinline__ const T& at32(const T* base, uint32_t i) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) +
                                     i * (uint32_t)sizeof(T));
}
template <class T>
__device__ __forceinline__ T& at32(T* base, uint32_t i) {
  return *reinterpret_cast<T*>(reinterpret_cast<char*>(base) +
                               i * (uint32_t)sizeof(T));
}

struct PassArgs {
  const uint32_t* keys_in;   // unused with kDepthKeys
  const uint32_t* vals_in;   // unused without kValsIn (values = in-segment index)
  const float* depth_src;    // keys derived from float depths (kDepthKeys)
  uint32_t* keys_out;        // unused without kKeysOut (last pass)
  uint32_t* vals_out;
  int64_t n_seg;             // elements per segment (a capacity with n_dev)
  const int32_t* n_dev;      // one segment: min(*n_dev, n_seg) elements (or null)
  int nblk;                  // workgroups per segment
  int segments;
  int shift;
  int digit_bits;
  const uint32_t* ghist;     // [segments][256] global digit counts of this pass
  uint32_t* status;          // [segments][nblk][256], zeroed
  uint32_t* err;             // look-back give-up status word
  // The tile-pair sort in two passes (kPackHi, then kPairRanges; one
  // segment): the first pass's global digit counts, and the tile ranges the
  // second pass writes.
  const uint32_t* ghist_a;
  int32_t* tile_offsets;     // [num_tiles + 1]
  int num_tiles;
};

// Kernel variants, chosen on the host, so that the load loops hold no
// data-dependent branches: every load of a lane is in flight before the first
// one is used (a branch between a load and its use makes the compiler wait
// for that load before the next is issued).
//
// The tile-pair sort of tile keys below 2^16 and values (gids) below 2^24 runs
// as two passes that move 4 bytes less per element each:
//  kKeyBytes    (first pass): the keys are the tiles' low bytes (uint8) and
//               the values the words (key >> 8) << 24 | gid, written by the
//               emit in that form; the pass moves the words;
//  kPackHi      (a first pass on 32-bit keys and values instead): writes each
//               element as one word, (key >> 8) << 24 | value, and no key;
//  kPairRanges  (second pass, on those words: digit = word >> 24): writes the
//               values (word & 0xffffff) and the tile ranges.  Its input is
//               ordered by the low key byte, which is the first pass's digit:
//               the elements with low byte below lo are exactly those before
//               position P[lo] (the scan of the first pass's digit counts).
//               So the first pair of tile (hi << 8 | lo) lies at dbase[hi] +
//               (elements of digit hi before position P[lo]), and the
//               workgroup whose block holds position P[lo] knows that count
//               from its look-back prefix and its own elements before P[lo]:
//               it writes tile_offsets[(hi << 8) | lo] for every hi.  Every
//               entry is written once (empty tiles included); P[lo] = n is
//               left to workgroup 0, which also writes tile_offsets[T] = n.
//  kPreCounts   (with either): every block's prefix (the elements of each
//               digit in the blocks before it) is already in its status
//               words, from rs_block_counts_kernel and rs_block_scan_kernel
//               launched before the pass; the pass reads it instead of
//               looking back.  A decoupled look-back serialises the
//               workgroups (each one's prefix waits for a predecessor's,
//               a few memory round trips per window of predecessors), which
//               at 2^23+ elements bounds the pass more than its work does.
enum : int {
  kDepthKeys = 1,
  kValsIn = 2,
  kKeysOut = 4,
  kPackHi = 8,
  kPairRanges = 16,
  kKeyBytes = 32,
  kPreCounts = 64
};

// Exclusive scan of one value per thread over a block of kW wavefronts.
template <int kW = kWaves>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* wsum) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(inc, off, 64);
    if (lane >= off) inc += y;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  uint32_t pre = 0u;
  for (int w = 0; w < wave; ++w) pre += wsum[w];
  __syncthreads();
  return pre + inc - v;
}

// Per-pass global digit histograms: ghist[(p*segments + seg)*256 + d] (zeroed
// by the caller) for passes p = 0..passes-1 with digits at begin_bit + 8p.
// Each thread loads kR keys (clamped indices, no branches) before
// counting any of them.
template <bool kDepth, int kR>
__global__ __launch_bounds__(kThreads) void rs_global_hist_kernel(
    const uint32_t* keys, const float* depth_src, int64_t n_seg, int nblk,
    int segments, int begin_bit, int end_bit, int passes, uint32_t* ghist) {
  __shared__ uint32_t h[4][256];
  const int seg = blockIdx.x / nblk;
  const int blk = blockIdx.x - seg * nblk;
  const int t = threadIdx.x;
  for (int i = t; i < 4 * 256; i += kThreads) (&h[0][0])[i] = 0u;
  const int64_t base = (int64_t)seg * n_seg;
  const int64_t lo = (int64_t)blk * (kThreads * kR);
  uint32_t kv[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t j = min(lo + r * kThreads + t, n_seg - 1);
    kv[r] = kDepth ? __float_as_uint(depth_src[base + j]) : keys[base + j];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (lo + r * kThreads + t < n_seg) {
      const uint32_t key = kDepth ? depth_key(__uint_as_float(kv[r])) : kv[r];
      for (int p = 0; p < passes; ++p) {
        const int sh = begin_bit + 8 * p;
        const int bits = min(8, end_bit - sh);
        atomicAdd(&h[p][(key >> sh) & ((1u << bits) - 1u)], 1u);
      }
    }
  }
  __syncthreads();
  for (int p = 0; p < passes; ++p) {
    const uint32_t c = h[p][t];
    if (c) atomicAdd(&ghist[((int64_t)p * segments + seg) * 256 + t], c);
  }
}

// Ranks the wavefront's kR rounds of 64 elements: rreg[r] = the element's
// rank among the wavefront's elements of its digit | digit << 16 (all ones
// for lanes past the segment's end), counting in wcnt (the wavefront's digit
// counters).  Two rounds at a time: their matches interleave; the count
// updates stay in round order.  kFull: every element of the block is valid
// (no per-round masks).  kPairRanges with boundaries: the digits are also
// kept in input order as bytes at dig8.
template <int kMode, int kR, bool kFull>
__device__ __forceinline__ void rank_rounds(uint32_t (&kreg)[kR],
                                            uint32_t (&vreg)[kR],
                                            uint32_t (&rreg)[kR],
                                            uint32_t* wcnt, uint8_t* dig8,
                                            uint32_t lo, uint32_t n32,
                                            int shift, uint32_t dmask,
                                            bool boundaries) {
  constexpr bool kRanges = (kMode & kPairRanges) != 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t lt = lanemask_lt();
#pragma unroll
  for (int r = 0; r < kR; r += 2) {
    uint32_t d[2];
    bool valid[2];
    uint64_t act[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t j = lo + (uint32_t)((r + u) * 64 + lane);
      valid[u] = kFull || j < n32;
      if (kMode & kDepthKeys) kreg[r + u] = depth_key(__uint_as_float(kreg[r + u]));
      if (kRanges)
        vreg[r + u] = kreg[r + u] & 0xffffffu;
      else if (!(kMode & kValsIn))
        vreg[r + u] = j;
      d[u] = (kreg[r + u] >> shift) & dmask;
      if (kRanges && boundaries && valid[u])
        dig8[wave * (64 * kR) + (r + u) * 64 + lane] = (uint8_t)d[u];
      act[u] = kFull ? ~0ull : __ballot(valid[u]);
    }
    uint64_t peers[2];
    match_digit2(d[0], d[1], act[0], act[1], peers[0], peers[1]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t below = (uint32_t)__popcll(peers[u] & lt);
      // Every lane of the digit reads its count, then the digit's lowest
      // lane adds the group's size: one wavefront's LDS accesses take effect
      // in program order, so all of them see the count before the addition.
      const uint32_t old = wcnt[d[u]];
      __builtin_amdgcn_wave_barrier();  // the read stays before the addition
      if (valid[u] && below == 0u)
        atomicAdd(&wcnt[d[u]], (uint32_t)__popcll(peers[u]));
      rreg[r + u] = valid[u] ? ((old + below) | (d[u] << 16)) : 0xffffffffu;
    }
  }
}

// Blocks per chunk of the block-count scan, and thread groups per digit in
// its workgroups.
constexpr int kScanChunk = 128;
constexpr int kScanQ = 4;

// Digit counts of every block of 256 kBlockRounds elements of a pass
// (kPreCounts): status[b][d] = count, and each count added to its chunk's
// total, chunk_tot[b / kScanChunk][d] (zeroed before).  Keys are bytes
// (kBytes: the tile-pair sort's low tile bytes) or words (digit = (word >>
// shift) & dmask).  One workgroup per block (four blocks per workgroup were
// slower); elements past the count are not counted.
template <bool kBytes, int kBlockRounds>
__global__ __launch_bounds__(kThreads) void rs_block_counts_kernel(
    const uint32_t* keys, int64_t n_cap, const int32_t* n_dev, int shift,
    uint32_t dmask, uint32_t* status, uint32_t* chunk_tot) {
  constexpr int kItems = kThreads * kBlockRounds;
  constexpr int kLoads = kBytes ? kBlockRounds / 4 : kBlockRounds;
  __shared__ uint32_t h[kWaves][256];
  const int t = threadIdx.x, wave = t >> 6;
  const int64_t n = n_dev ? min(n_cap, (int64_t)max(*n_dev, 0)) : n_cap;
  const int blk = blockIdx.x;
  if ((int64_t)blk * kItems >= n) return;
  const uint32_t n32 = (uint32_t)n;
  // word j holds elements (kBytes ? 4 : 1) * j onwards
  const uint32_t words_end = kBytes ? (n32 + 3u) / 4u : n32;
  constexpr uint32_t kBlockWords = kBytes ? kItems / 4 : kItems;
  uint32_t v[kLoads];
#pragma unroll
  for (int r = 0; r < kLoads; ++r)
    v[r] = at32(keys, min((uint32_t)blk * kBlockWords + (uint32_t)(r * kThreads + t),
                          words_end - 1u));
  for (int i = t; i < kWaves * 256; i += kThreads) (&h[0][0])[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kLoads; ++r) {
    const uint32_t w = (uint32_t)blk * kBlockWords + (uint32_t)(r * kThreads + t);
    if (kBytes) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (w * 4u + k < n32) atomicAdd(&h[wave][(v[r] >> (8 * k)) & 255u], 1u);
    } else if (w < n32) {
      atomicAdd(&h[wave][(v[r] >> shift) & dmask], 1u);
    }
  }
  __syncthreads();
  uint32_t c = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) c += h[w][t];
  status[(int64_t)blk * 256 + t] = c;
  if (c != 0u) atomicAdd(&chunk_tot[(int64_t)(blk / kScanChunk) * 256 + t], c);
}

// The counts of rs_block_counts_kernel replaced by their exclusive prefix
// over the blocks, per digit.  Workgroup c (kScanQ groups of 256 threads,
// thread t of a group for digit t) takes chunk c: group q sums the totals of
// every kScanQ-th chunk before it from q on (no order among workgroups) and
// the counts of the chunk's rows q kRows .. q kRows + kRows - 1; the groups
// combine their sums in LDS, then each scans its rows.  The workgroup of the
// last chunk also writes each digit's total to digit_tot[0..255] (the pass's
// global histogram; may be null).
template <int kBlockRounds>
__global__ __launch_bounds__(256 * kScanQ) void rs_block_scan_kernel(
    uint32_t* status, const uint32_t* chunk_tot, int64_t n_cap,
    const int32_t* n_dev, uint32_t* digit_tot) {
  constexpr int64_t kItems = (int64_t)kThreads * kBlockRounds;
  constexpr int kRows = kScanChunk / kScanQ;
  __shared__ uint32_t part[kScanQ][256];
  __shared__ uint32_t before[kScanQ][256];
  const int t = threadIdx.x & 255, q = threadIdx.x >> 8;
  const int64_t n = n_dev ? min(n_cap, (int64_t)max(*n_dev, 0)) : n_cap;
  const int nblk = (int)((n + kItems - 1) / kItems);
  const int c = blockIdx.x;
  const int b0 = c * kScanChunk;
  if (b0 >= nblk) return;
  const int nb = min(kScanChunk, nblk - b0);
  uint32_t v[kRows];
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const int row = q * kRows + k;
    const uint32_t x = status[(int64_t)(b0 + min(row, nb - 1)) * 256 + t];
    v[k] = row < nb ? x : 0u;
  }
  uint32_t pre = 0u;
#pragma unroll 8
  for (int j = q; j < c; j += kScanQ) pre += chunk_tot[(int64_t)j * 256 + t];
  uint32_t sum = 0u;
#pragma unroll
  for (int k = 0; k < kRows; ++k) sum += v[k];
  part[q][t] = sum;
  before[q][t] = pre;
  __syncthreads();
  uint32_t run = 0u;
#pragma unroll
  for (int i = 0; i < kScanQ; ++i) run += before[i][t] + (i < q ? part[i][t] : 0u);
#pragma unroll
  for (int k = 0; k < kRows; ++k) {
    const int row = q * kRows + k;
    if (row < nb) status[(int64_t)(b0 + row) * 256 + t] = run;
    run += v[k];
  }
  // (the last group's run ends at the digit's total)
  if (digit_tot != nullptr && b0 + nb == nblk && q == kScanQ - 1)
    digit_tot[t] = run;
}

// A block of 256 kR elements is ranked by onesweep_waves(kR) wavefronts of
// onesweep_rounds(kR) rounds each: blocks of 8192 elements use eight
// wavefronts of 16 rounds, which halves the registers that hold a lane's
// elements (four wavefronts per SIMD instead of two).
constexpr int onesweep_waves(int rounds) { return rounds == 32 ? 8 : kWaves; }
constexpr int onesweep_rounds(int rounds) { return rounds == 32 ? 16 : rounds; }

template <int kMode, int kBlockRounds>
__global__ __launch_bounds__(64 * onesweep_waves(kBlockRounds))
void rs_onesweep_kernel(PassArgs a) {
  constexpr int kW = onesweep_waves(kBlockRounds);
  constexpr int kR = onesweep_rounds(kBlockRounds);
  constexpr int kT = 64 * kW;
  constexpr int kWaveItems = 64 * kR;
  constexpr int kBlockItems = kW * kWaveItems;
  constexpr bool kRanges = (kMode & kPairRanges) != 0;
  constexpr bool kBytes = (kMode & kKeyBytes) != 0;
  __shared__ uint32_t cnt[kW][256];
  // dstart: digit d's first slot in the block's sorted order; gdelta: the
  // global position of that slot.  (kPairRanges: they are written after the
  // tile ranges and hold P[lo] and the digit counts before it until then.)
  __shared__ uint32_t dstart[256];
  __shared__ uint32_t gdelta[256];
  __shared__ uint32_t wsum[kW];
  // The block in sorted order: keys (one byte each with kKeyBytes; with
  // kPairRanges the key is the word and, before the scatter, the block's
  // digits in input order are kept here, one byte each) and values (none
  // with kPairRanges: the value is the word's low 24 bits).  Sizes are
  // per mode so that more workgroups fit in a CU's LDS.
  __shared__ uint32_t sk[kBytes ? kBlockItems / 4 : kBlockItems];
  __shared__ uint32_t sv[kRanges ? 1 : kBlockItems];
  uint32_t* const pstart = dstart;  // P[lo] (kPairRanges)
  uint32_t* const hist = gdelta;    // digits before P[lo] (kPairRanges)
  uint8_t* const dig8 = reinterpret_cast<uint8_t*>(sk);

  // Block = workgroup index.  A workgroup looks back only at blocks of
  // smaller index, and workgroups are dispatched to the XCDs round-robin by
  // index and, within an XCD, in index order: a block that has not started
  // shares its XCD only with running blocks of smaller index, which do not
  // wait for it, so it starts once one of them ends.  (The bounded waits of
  // the look-back report a give-up instead of hanging should that order
  // ever not hold.)  An atomic ticket per workgroup, the usual way to get an
  // order that holds by construction, delays every workgroup's loads by its
  // round trip: pair passes at 1.2e8 pairs 365 -> 330 and 503 -> 479 us
  // without it.
  const int vb = (int)blockIdx.x;
  const int seg = vb / a.nblk;
  const int blk = vb - seg * a.nblk;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // With the element count on the device, workgroups past it have nothing
  // to do: none of the workgroups before them looks back at them.
  const int64_t n_seg =
      a.n_dev ? min(a.n_seg, (int64_t)max(*a.n_dev, 0)) : a.n_seg;
  if ((int64_t)blk * kBlockItems >= n_seg) return;
  const uint32_t n32 = (uint32_t)n_seg;  // (segments hold at most 2^29)
  for (int i = t; i < kW * 256; i += kT) (&cnt[0][0])[i] = 0u;
  // kPairRanges: does this block hold a position P[lo]?
  const uint32_t blk_lo = (uint32_t)blk * kBlockItems;
  const uint32_t blk_hi = min(n32, blk_lo + kBlockItems);
  bool boundaries = false;
  if (kRanges) {
    const uint32_t pl = block_excl_scan<kW>(t < 256 ? a.ghist_a[t] : 0u, wsum);
    if (t < 256) {
      pstart[t] = pl;
      hist[t] = 0u;
    }
    boundaries = __syncthreads_or(t < 256 && pl >= blk_lo && pl < blk_hi);
  }

  const int64_t seg_base = (int64_t)seg * a.n_seg;
  const uint32_t lo = blk_lo + (uint32_t)(wave * kWaveItems);
  const uint32_t dmask = (1u << a.digit_bits) - 1u;

  // Issue every load of this lane's kR elements before ranking any of them
  // (indices clamped into the segment; lanes past its end are masked out of
  // the ranking below).
  uint32_t kreg[kR], vreg[kR], rreg[kR];
  {
    const uint8_t* kin8 = reinterpret_cast<const uint8_t*>(a.keys_in) + seg_base;
    const uint32_t* kin = a.keys_in + seg_base;
    const float* din = a.depth_src + seg_base;
    const uint32_t* vin = a.vals_in + seg_base;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const uint32_t src = min(lo + (uint32_t)(r * 64 + lane), n32 - 1u);
      if (kBytes)
        kreg[r] = at32(kin8, src);
      else
        kreg[r] = (kMode & kDepthKeys) ? __float_as_uint(at32(din, src))
                                       : at32(kin, src);
      if (kMode & kValsIn) vreg[r] = at32(vin, src);
    }
  }
  // this pass's global digit count of digit t (digit bases below)
  const uint32_t gh = t < 256 ? a.ghist[(int64_t)seg * 256 + t] : 0u;
  constexpr bool kPre = (kMode & kPreCounts) != 0;
  uint32_t* my_status = a.status + ((int64_t)seg * a.nblk + blk) * 256 + t;
  uint32_t tot = 0u, prefix = 0u, dbase = 0u, local = 0u;
  if (kPre) {
    // the block's prefix and count (the next block's prefix, or the
    // digit's total after the last block), while the loads fly
    if (t < 256) {
      prefix = *my_status;
      const uint32_t last = (n32 - 1u) / kBlockItems;
      tot = ((uint32_t)blk < last ? my_status[256] : gh) - prefix;
    }
    dbase = block_excl_scan<kW>(gh, wsum);
    local = block_excl_scan<kW>(tot, wsum);
  }
  __syncthreads();

  if (blk_hi - blk_lo == (uint32_t)kBlockItems)
    rank_rounds<kMode, kR, true>(kreg, vreg, rreg, cnt[wave], dig8, lo, n32,
                                 a.shift, dmask, boundaries);
  else
    rank_rounds<kMode, kR, false>(kreg, vreg, rreg, cnt[wave], dig8, lo, n32,
                                  a.shift, dmask, boundaries);
  __syncthreads();

  // Thread t < 256 owns digit t: its count in the block, and each
  // wavefront's first slot among the block's elements of the digit.
  if (t < 256) {
    uint32_t c[kW];
#pragma unroll
    for (int w = 0; w < kW; ++w) c[w] = cnt[w][t];
    uint32_t run = 0u;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      cnt[w][t] = run;
      run += c[w];
    }
    if (!kPre) {
      tot = run;
      status_store(my_status, (blk == 0 ? kFlagInc32 : kFlagAgg32) | tot);
    }
  }
  if (!kPre) {
    dbase = block_excl_scan<kW>(gh, wsum);
    local = block_excl_scan<kW>(tot, wsum);
    if (blk > 0 && t < 256) {
      prefix = lookback32<kLookbackWindow>(
          a.status + (int64_t)seg * a.nblk * 256 + t, blk, 256, a.err);
      status_store(my_status, kFlagInc32 | (prefix + tot));
    }
  }

  if (kRanges) {
    // Tile ranges at the positions P[lo] inside this block, in increasing
    // order (P is nondecreasing): hist counts the block's digits before the
    // current one, each element added once.  Thread t writes the entry of
    // digit t (hi = t).
    const bool hi_ok = t < (1 << a.digit_bits);
    if (boundaries) {
      // (low bytes without pairs share their position with the next one:
      // hist is brought up to each distinct position once)
      uint32_t q_prev = 0u;
      for (int l = 0; l < 256; ++l) {
        const uint32_t p = pstart[l];
        if (p < blk_lo || p >= blk_hi) continue;  // uniform
        const uint32_t q = p - blk_lo;
        if (q != q_prev) {  // uniform
          __syncthreads();  // the reads of hist at q_prev are done
          for (uint32_t i = q_prev + t; i < q; i += kT)
            atomicAdd(&hist[dig8[i]], 1u);
          q_prev = q;
          __syncthreads();
        }
        const int tile = (t << 8) | l;
        if (hi_ok && tile < a.num_tiles)
          a.tile_offsets[tile] = (int32_t)(dbase + prefix + hist[t]);
      }
    }
    if (blk == 0) {
      // P[lo] = n: every pair of digit hi lies before (hi << 8 | lo)
      for (int l = 0; l < 256; ++l) {
        if (pstart[l] != n32) continue;  // uniform
        const int tile = (t << 8) | l;
        if (hi_ok && tile < a.num_tiles)
          a.tile_offsets[tile] = (int32_t)(dbase + gh);
      }
      if (t == 0) a.tile_offsets[a.num_tiles] = (int32_t)n_seg;
    }
    __syncthreads();  // pstart, hist and the digit bytes are read
  }
  if (t < 256) {
    dstart[t] = local;
    // (modulo 2^32: the positions themselves are below 2^29)
    gdelta[t] = dbase + prefix - local;
  }
  __syncthreads();

#pragma unroll
  for (int r = 0; r < kR; ++r) {
    if (rreg[r] != 0xffffffffu) {
      const uint32_t d = rreg[r] >> 16;
      const uint32_t pos = dstart[d] + cnt[wave][d] + (rreg[r] & 0xffffu);
      if (kBytes)
        dig8[pos] = (uint8_t)d;  // the key byte is the digit
      else
        sk[pos] = kreg[r];
      if (!kRanges) sv[pos] = vreg[r];
    }
  }
  __syncthreads();

  // Unrolled, so that the LDS reads of all kR elements are in flight
  // together.
  const uint32_t count = blk_hi - blk_lo;
  uint32_t* kout = a.keys_out + seg_base;
  uint32_t* vout = a.vals_out + seg_base;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const uint32_t i = (uint32_t)(t + r * kT);
    if (i < count) {
      const uint32_t key = kBytes ? (uint32_t)dig8[i] : sk[i];
      const uint32_t pos = gdelta[(key >> a.shift) & dmask] + i;
      if (pos < n32) {  // (fails only with histograms inconsistent with the keys)
        if (kMode & kKeysOut) at32(kout, pos) = key;
        if (kRanges)
          at32(vout, pos) = key & 0xffffffu;
        else if (kMode & kPackHi)
          at32(vout, pos) = ((key >> 8) << 24) | sv[i];
        else
          at32(vout, pos) = sv[i];
      }
    }
  }
}

// Zero-pass "sort": copy (deriving keys/values when needed).
__global__ void rs_copy_kernel(PassArgs a, int64_t n_total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_total) return;
  const int64_t j = i % a.n_seg;
  if (a.keys_out)
    a.keys_out[i] = a.depth_src ? depth_key(a.depth_src[i]) : a.keys_in[i];
  a.vals_out[i] = a.vals_in ? a.vals_in[i] : (uint32_t)j;
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

// Rounds (64-element groups per wavefront) of one onesweep workgroup: small
// segments use smaller workgroups so that more of them run side by side;
// segments above 2^20 use blocks of 8192 elements (eight wavefronts of 16
// rounds), which halves the look-back chain and doubles the length of each
// digit's coalesced run in the scatter (1.7e6 pairs: 22.5 -> 18.2 us per
// pass; at 2^20 depth keys the 4096-element blocks stay faster).
int radix_rounds(int64_t n_seg) {
  if (n_seg <= (int64_t(1) << 18)) return 4;
  return n_seg <= (int64_t(1) << 20) ? 16 : 32;
}

RadixPlan radix_plan(int64_t n_seg, int segments, int begin_bit, int end_bit) {
  RadixPlan L{};
  L.n_seg = n_seg;
  L.segments = segments;
  L.begin_bit = begin_bit;
  L.end_bit = end_bit;
  L.passes = end_bit > begin_bit ? (end_bit - begin_bit + 7) / 8 : 0;
  L.rounds = radix_rounds(n_seg);
  const int64_t block_items = (int64_t)kThreads * L.rounds;
  L.nblk = (int)((n_seg + block_items - 1) / block_items);
  L.ghist_words = (int64_t)4 * segments * 256;
  // the passes' statuses, then per-chunk digit totals of each pass (the
  // two-pass tile-pair sort's block-count scan)
  const int64_t pw = L.passes > 0 ? L.passes : 1;
  L.status_words = pw * segments * L.nblk * 256 +
                   pw * ((L.nblk + kScanChunk - 1) / kScanChunk) * 256;
  L.ticket_words = 8;  // four pass tickets, the give-up status word, padding
  const int64_t n = n_seg * (int64_t)segments;
  const size_t vec = align_up((size_t)n * sizeof(uint32_t), 256);
  size_t off = 0;
  L.a_keys = L.a_vals = L.b_keys = L.b_vals = 0;
  if (L.passes >= 2) {
    L.a_keys = off; off += vec;
    L.a_vals = off; off += vec;
  }
  if (L.passes >= 3) {
    L.b_keys = off; off += vec;
    L.b_vals = off; off += vec;
  }
  L.buffer_bytes = off;
  return L;
}

size_t radix_ctl_bytes(const RadixPlan& L) {
  return align_up((size_t)(L.ghist_words + L.status_words + L.ticket_words) *
                      sizeof(uint32_t), 256);
}

RadixCtl radix_ctl_at(const RadixPlan& L, void* p) {
  uint32_t* w = static_cast<uint32_t*>(p);
  uint32_t* tickets = w + L.ghist_words + L.status_words;
  return RadixCtl{w, w + L.ghist_words, tickets, tickets + 4};
}

size_t radix_sort_workspace_bytes(int64_t n_per_segment, int segments) {
  if (n_per_segment <= 0 || segments <= 0) return 0;
  const RadixPlan L = radix_plan(n_per_segment, segments, 0, 32);
  return radix_ctl_bytes(L) + L.buffer_bytes;
}

int launch_zero_u32(uint32_t* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return GSPLAT_OK;
  int64_t grid = (n + 255) / 256;
  if (grid > 2048) grid = 2048;
  launch_traced("zero_u32_kernel", zero_u32_kernel, dim3((unsigned)grid),
                dim3(256), 0, stream, p, n);
  return check_launch("zero_u32_kernel");
}

int radix_global_hist(const RadixPlan& L, const RadixCtl& C,
                      const uint32_t* keys, const float* depth_src,
                      hipStream_t stream) {
  if (L.passes == 0 || L.n_seg == 0 || L.segments == 0) return GSPLAT_OK;
  const dim3 grid((unsigned)(L.nblk * (int64_t)L.segments));
#define GS_HIST_LAUNCH(D, R)                                                   \
  launch_traced(depth_src != nullptr ? "rs_global_hist_kernel(depth)"      \
                                     : "rs_global_hist_kernel(keys)",       \
                (rs_global_hist_kernel<D, R>), grid, dim3(kThreads), 0,       \
                stream, keys, depth_src, L.n_seg, L.nblk, L.segments,         \
                L.begin_bit, L.end_bit, L.passes, C.ghist)
  if (L.rounds == 4) {
    if (depth_src) GS_HIST_LAUNCH(true, 4); else GS_HIST_LAUNCH(false, 4);
  } else if (L.rounds == 16) {
    if (depth_src) GS_HIST_LAUNCH(true, 16); else GS_HIST_LAUNCH(false, 16);
  } else {
    if (depth_src) GS_HIST_LAUNCH(true, 32); else GS_HIST_LAUNCH(false, 32);
  }
#undef GS_HIST_LAUNCH
  return check_launch("rs_global_hist_kernel");
}

int radix_passes(const RadixPlan& L, const RadixCtl& C, void* buffers,
                 const uint32_t* keys_in, const uint32_t* vals_in,
                 const float* depth_src, uint32_t* keys_out,
                 uint32_t* vals_out, hipStream_t stream,
                 const int32_t* n_dev) {
  if (L.n_seg == 0 || L.segments == 0) return GSPLAT_OK;
  if (n_dev != nullptr && L.segments != 1) {
    set_error("radix sort: a device element count needs one segment");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  char* base = static_cast<char*>(buffers);
  const int64_t n = L.n_seg * L.segments;
  if (L.passes == 0) {  // copies all L.n_seg elements (in bounds with n_dev)
    PassArgs a{keys_in, vals_in, depth_src, keys_out, vals_out, L.n_seg,
               nullptr, L.nblk, L.segments, 0, 0, nullptr, nullptr, nullptr,
               nullptr};
    launch_traced("rs_copy_kernel", rs_copy_kernel,
                  dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a,
                  n);
    return check_launch("rs_copy_kernel");
  }
  uint32_t* bufk[2] = {reinterpret_cast<uint32_t*>(base + L.a_keys),
                       reinterpret_cast<uint32_t*>(base + L.b_keys)};
  uint32_t* bufv[2] = {reinterpret_cast<uint32_t*>(base + L.a_vals),
                       reinterpret_cast<uint32_t*>(base + L.b_vals)};
  const int64_t status_per_pass = (int64_t)L.segments * L.nblk * 256;
  // trace name: the depth sort (float depth keys) or a sort of given keys
  const char* pass_name = depth_src != nullptr ? "rs_onesweep_kernel(depth)"
                                               : "rs_onesweep_kernel(keys)";
  const uint32_t* cur_k = keys_in;
  const uint32_t* cur_v = vals_in;
  const float* cur_depth = depth_src;
  for (int p = 0; p < L.passes; ++p) {
    const int shift = L.begin_bit + 8 * p;
    const int bits = (L.end_bit - shift) < 8 ? (L.end_bit - shift) : 8;
    const bool last = (p == L.passes - 1);
    uint32_t* out_k = last ? keys_out : bufk[p & 1];
    uint32_t* out_v = last ? vals_out : bufv[p & 1];
    PassArgs a{cur_k, cur_v, cur_depth, out_k, out_v, L.n_seg, n_dev, L.nblk,
               L.segments, shift, bits,
               C.ghist + (int64_t)p * L.segments * 256,
               C.status + p * status_per_pass, C.err};
    const int mode = (cur_depth ? kDepthKeys : 0) | (cur_v ? kValsIn : 0) |
                     (out_k ? kKeysOut : 0);
    const dim3 grid((unsigned)(L.nblk * (int64_t)L.segments));
    switch (mode * 32 + L.rounds) {
#define GS_ONESWEEP_CASE(M, R)                                              \
  case M * 32 + R:                                                          \
    launch_traced(pass_name, (rs_onesweep_kernel<M, R>), grid,               \
                  dim3(64 * onesweep_waves(R)),                             \
                  0, stream, a);                                            \
    break;
#define GS_ONESWEEP_MODE(M) \
  GS_ONESWEEP_CASE(M, 4) GS_ONESWEEP_CASE(M, 16) GS_ONESWEEP_CASE(M, 32)
      GS_ONESWEEP_MODE(0) GS_ONESWEEP_MODE(1) GS_ONESWEEP_MODE(2)
      GS_ONESWEEP_MODE(3) GS_ONESWEEP_MODE(4) GS_ONESWEEP_MODE(5)
      GS_ONESWEEP_MODE(6) GS_ONESWEEP_MODE(7)
#undef GS_ONESWEEP_MODE
#undef GS_ONESWEEP_CASE
      default:
        set_error("radix sort: no kernel for mode %d, %d rounds", mode,
                  L.rounds);
        return GSPLAT_ERR_INVALID_ARGUMENT;
    }
    const int rc = check_launch("rs_onesweep_kernel");
    if (rc) return rc;
    cur_k = out_k;
    cur_v = out_v;
    cur_depth = nullptr;
  }
  return GSPLAT_OK;
}

// Buffers of fewer pairs sort them in two passes of keys and values and
// take the tile ranges from the sorted keys (one launch more): below about
// 2^23 pairs the low-byte ranges are short enough that many of them start in
// one sort block, whose second pass then walks them one after another.
constexpr int64_t kPairRangesMinPairs = int64_t(1) << 23;

uint32_t* radix_pair_zero_span(const RadixPlan& L, const RadixCtl& C,
                               int64_t* words) {
  // the second pass's statuses, then the first pass's chunk totals
  const int64_t nchunks = (L.nblk + kScanChunk - 1) / kScanChunk;
  if (words) *words = (int64_t)L.nblk * 256 + nchunks * 256;
  return C.status + (int64_t)L.nblk * 256;
}

bool radix_pair_ranges_ok(const RadixPlan& L, int64_t num_values) {
  return L.segments == 1 && L.passes == 2 && L.begin_bit == 0 &&
         L.end_bit > 8 && L.end_bit <= 16 && num_values <= (int64_t(1) << 24) &&
         L.n_seg >= kPairRangesMinPairs;
}

int radix_pair_sort_ranges(const RadixPlan& L, const RadixCtl& C,
                           void* buffers, const uint8_t* key_bytes,
                           const uint32_t* words_in, uint32_t* vals_out,
                           int32_t* tile_offsets, int num_tiles,
                           hipStream_t stream, const int32_t* n_dev) {
  if (L.segments != 1 || L.passes != 2 || L.begin_bit != 0 ||
      L.end_bit <= 8 || L.end_bit > 16 || num_tiles > (1 << L.end_bit)) {
    set_error("radix sort: the two-pass tile sort needs 9..16 key bits");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (L.n_seg == 0) return GSPLAT_OK;
  uint32_t* words =
      reinterpret_cast<uint32_t*>(static_cast<char*>(buffers) + L.a_vals);
  const int64_t status_per_pass = (int64_t)L.nblk * 256;
  const dim3 grid((unsigned)L.nblk);
  PassArgs a{reinterpret_cast<const uint32_t*>(key_bytes), words_in, nullptr,
             nullptr, words, L.n_seg, n_dev, L.nblk, 1, 0, 8, C.ghist,
             C.status, C.err, nullptr, nullptr, 0};
  PassArgs b{words, nullptr, nullptr, nullptr, vals_out, L.n_seg, n_dev,
             L.nblk, 1, 24, L.end_bit - 8, C.ghist + 256,
             C.status + status_per_pass, C.err,
             C.ghist, tile_offsets, num_tiles};
  // The first pass takes its block prefixes from a count and a scan of the
  // key bytes (1 B/pair read), and its global histogram (ghist[0..255]) from
  // the scan; the second looks back (its counts would cost a read of the
  // 4-byte words, more than its look-back does), with the histogram of the
  // high tile bits at ghist[256..511] from the emit.
  constexpr int kA = kValsIn | kKeyBytes | kPreCounts;
  constexpr int kB = kPairRanges;
  uint32_t* chunk_a = C.status + 2 * (int64_t)L.nblk * 256;
  const dim3 chunks((unsigned)((L.nblk + kScanChunk - 1) / kScanChunk));
#define GS_PAIR_PASSES(R)                                                    \
  launch_traced("rs_block_counts_kernel(pairs:lo)",                          \
                (rs_block_counts_kernel<true, R>), grid, dim3(kThreads), 0,  \
                stream, a.keys_in, L.n_seg, n_dev, 0, 255u, a.status,        \
                chunk_a);                                                    \
  launch_traced("rs_block_scan_kernel(pairs:lo)", (rs_block_scan_kernel<R>), \
                chunks, dim3(256 * kScanQ), 0, stream, a.status, chunk_a,     \
                L.n_seg, n_dev, C.ghist);                                    \
  launch_traced("rs_onesweep_kernel(pairs:lo)", (rs_onesweep_kernel<kA, R>), \
                grid, dim3(64 * onesweep_waves(R)), 0, stream, a);           \
  launch_traced("rs_onesweep_kernel(pairs:hi)", (rs_onesweep_kernel<kB, R>), \
                grid, dim3(64 * onesweep_waves(R)), 0, stream, b);
  if (L.rounds == 4) {
    GS_PAIR_PASSES(4)
  } else if (L.rounds == 16) {
    GS_PAIR_PASSES(16)
  } else {
    GS_PAIR_PASSES(32)
  }
#undef GS_PAIR_PASSES
  return check_launch("rs_onesweep_kernel(pairs)");
}

bool radix_size_ok(int64_t n_seg, int segments) {
  const int64_t block_items = (int64_t)kThreads * radix_rounds(n_seg);
  const int64_t nblk = (n_seg + block_items - 1) / block_items;
  return nblk * segments <= 0x7fffffffLL && n_seg <= (int64_t(1) << 29) &&
         n_seg * segments <= 0x7fffffffLL;
}

int radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in,
                     const float* depth_src, uint32_t* keys_out,
                     uint32_t* vals_out, int64_t n_seg, int segments,
                     int begin_bit, int end_bit, void* ws, size_t ws_bytes,
                     hipStream_t stream, int32_t* status_out) {
  if (n_seg < 0 || segments < 0 || begin_bit < 0 || end_bit > 32 ||
      (keys_in == nullptr && depth_src == nullptr) || vals_out == nullptr) {
    set_error("radix_sort: invalid arguments");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (n_seg == 0 || segments == 0)
    return status_out ? launch_fill_i32(status_out, 0, 1, stream) : GSPLAT_OK;
  if (!radix_size_ok(n_seg, segments)) {
    set_error("radix_sort: input too large");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const RadixPlan L = radix_plan(n_seg, segments, begin_bit, end_bit);
  const size_t ctl = radix_ctl_bytes(L);
  if (L.passes > 0 && (ws == nullptr || ws_bytes < ctl + L.buffer_bytes)) {
    set_error("radix_sort: workspace too small (%zu < %zu)", ws_bytes,
              ctl + L.buffer_bytes);
    return GSPLAT_ERR_WORKSPACE;
  }
  RadixCtl C = radix_ctl_at(L, ws);
  if (status_out) C.err = reinterpret_cast<uint32_t*>(status_out);
  if (L.passes > 0) {
    int rc = launch_zero2(C.ghist, (int64_t)(ctl / sizeof(uint32_t)),
                          reinterpret_cast<uint32_t*>(status_out),
                          status_out ? 1 : 0, stream);
    if (!rc) rc = radix_global_hist(L, C, keys_in, depth_src, stream);
    if (rc) return rc;
  } else if (status_out) {
    const int rc = launch_fill_i32(status_out, 0, 1, stream);
    if (rc) return rc;
  }
  return radix_passes(L, C, static_cast<char*>(ws) + ctl, keys_in, vals_in,
                      depth_src, keys_out, vals_out, stream);
}

}  // namespace gs
