// depth_runs.h -- the run step of the small-image depth order: one
// workgroup of kRunThreads sorts a run of kRunItems consecutive splats of an
// image by depth key in LDS (stable LSD radix, four 8-bit passes; element
// order (wavefront, round, lane) = index order, ranks from ballot matching)
// and writes the run's sorted keys, its in-image indices and every
// kSampleStride-th sorted key (the run's samples).
//
// Shared by depth_run_sort_kernel (depth_sort.hip) and by the binning launch
// that runs it next to the per-splat tile count (binning.hip): the run step
// occupies one workgroup per run, a few of the 256 CUs, and the count fills
// the rest.
#pragma once

#include "gs_internal.h"

namespace gs {
namespace run_step {

constexpr int kRunItems = 4096;
constexpr int kRunWaves = 16;
constexpr int kRunThreads = 64 * kRunWaves;
constexpr int kRunRounds = kRunItems / kRunThreads;  // 64-element groups per wavefront
constexpr int kSampleStride = 64;
constexpr int kRunSamples = kRunItems / kSampleStride;
constexpr int kMaxRuns = 32;
static_assert(kRunRounds * kRunThreads == kRunItems, "run shape");

struct RunSortLds {
  uint32_t cnt[kRunWaves][256];
  uint32_t dstart[256];
  uint32_t wsum[kRunWaves];
  uint32_t sk[kRunItems];
  uint32_t sv[kRunItems];
};

// Where the run step writes: keys and in-image indices of every image's runs
// (same layout as the depths, [batch][G]) and the samples
// ([batch][runs][kRunSamples]).
struct RunBuffers {
  uint32_t* keys;
  uint32_t* vals;
  uint32_t* samples;
};

inline int runs_of(int64_t G) { return (int)((G + kRunItems - 1) / kRunItems); }

inline RunBuffers run_buffers(void* buffers, int64_t G, int batch) {
  const size_t vec = align_up((size_t)(G * batch) * sizeof(uint32_t), 256);
  char* b = static_cast<char*>(buffers);
  return RunBuffers{reinterpret_cast<uint32_t*>(b),
                    reinterpret_cast<uint32_t*>(b + vec),
                    reinterpret_cast<uint32_t*>(b + 2 * vec)};
}

__device__ __forceinline__ uint64_t lanes_below() {
  const unsigned lane = threadIdx.x & 63u;
  return (lane == 0u) ? 0ull : (~0ull >> (64u - lane));
}

// Lanes whose 8-bit digit equals this lane's digit (every lane is active).
// Per bit: n = the bit sign-extended (0 or ~0), b = the wavefront's ballot
// of it; the lanes that agree with this lane are ~(b ^ n), so m &= ~(b ^ n)
// is one three-input bit operation per 32-bit half (truth table 0x90 for
// src0 & ~(src1 ^ src2) with the operand patterns 0xF0, 0xCC, 0xAA).
__device__ __forceinline__ uint64_t same_digit_lanes(uint32_t d) {
  uint32_t lo = ~0u, hi = ~0u;
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

// Sorts run `block % runs` of image `block / runs` (kRunThreads threads).
__device__ __forceinline__ void run_sort_block(const float* __restrict__ depths,
                                               int G, int runs, int block,
                                               const RunBuffers& out,
                                               RunSortLds& S) {
  const int seg = block / runs;
  const int run = block - seg * runs;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int first = run * kRunItems;
  const int len = min(kRunItems, G - first);
  const int64_t base = (int64_t)seg * G + first;
  // Element q = wave * 256 + 64 * round + lane.  Slots past the run's end
  // get key 0xffffffff, above every depth key (NaN maps to 0xffc00000), so
  // they sort after the run's elements.
  uint32_t k[kRunRounds], v[kRunRounds];
#pragma unroll
  for (int r = 0; r < kRunRounds; ++r) {
    const int q = wave * (64 * kRunRounds) + 64 * r + lane;
    const uint32_t key = depth_key(depths[base + min(q, len - 1)]);
    k[r] = q < len ? key : 0xffffffffu;
    v[r] = (uint32_t)(first + q);
  }
  const uint64_t lt = lanes_below();
  for (int shift = 0; shift < 32; shift += 8) {
    for (int i = t; i < kRunWaves * 256; i += kRunThreads) (&S.cnt[0][0])[i] = 0u;
    __syncthreads();
    uint32_t rank[kRunRounds];
#pragma unroll
    for (int r = 0; r < kRunRounds; ++r) {
      const uint32_t d = (k[r] >> shift) & 255u;
      const uint64_t peers = same_digit_lanes(d);
      const uint32_t below = (uint32_t)__popcll(peers & lt);
      // Every lane of the digit reads its count, then the digit's lowest
      // lane adds the group's size: one wavefront's LDS accesses take effect
      // in program order, so all of them see the count before the addition.
      const uint32_t old = S.cnt[wave][d];
      __builtin_amdgcn_wave_barrier();  // the read stays before the addition
      if (below == 0u) atomicAdd(&S.cnt[wave][d], (uint32_t)__popcll(peers));
      rank[r] = old + below;
    }
    __syncthreads();
    // digit t (threads 0..255): wavefront offsets, then the digit's start
    uint32_t tot = 0u;
    if (t < 256) {
#pragma unroll
      for (int w = 0; w < kRunWaves; ++w) {
        const uint32_t c = S.cnt[w][t];
        S.cnt[w][t] = tot;
        tot += c;
      }
    }
    uint32_t inc = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (lane == 63) S.wsum[wave] = inc;
    __syncthreads();
    if (t < 256) {
      uint32_t pre = 0u;
      for (int w = 0; w < wave; ++w) pre += S.wsum[w];
      S.dstart[t] = pre + inc - tot;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRunRounds; ++r) {
      const uint32_t d = (k[r] >> shift) & 255u;
      const uint32_t pos = S.dstart[d] + S.cnt[wave][d] + rank[r];
      S.sk[pos] = k[r];
      S.sv[pos] = v[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRunRounds; ++r) {
      const int q = wave * (64 * kRunRounds) + 64 * r + lane;
      k[r] = S.sk[q];
      v[r] = S.sv[q];
    }
  }
  const int64_t sbase = ((int64_t)seg * runs + run) * kRunSamples;
#pragma unroll
  for (int r = 0; r < kRunRounds; ++r) {
    const int q = wave * (64 * kRunRounds) + 64 * r + lane;
    if (q < len) {
      out.keys[base + q] = k[r];
      out.vals[base + q] = v[r];
      if (q % kSampleStride == 0) out.samples[sbase + q / kSampleStride] = k[r];
    }
  }
}

// Whether a key x of another run precedes key k in the stable order: keys
// of earlier runs precede when x <= k (below_or_equal), of later runs when
// x < k.
__device__ __forceinline__ bool precedes(uint32_t x, uint32_t k,
                                         bool below_or_equal) {
  return below_or_equal ? (x <= k) : (x < k);
}

// Number of the first n keys of the sorted array a[] (n <= 2^kLog2) that
// precede k: they form a prefix, found by binary search.
template <int kLog2, class Load>
__device__ __forceinline__ int prefix_count(Load a, int n, uint32_t k,
                                            bool below_or_equal) {
  int c = 0;
#pragma unroll
  for (int step = 1 << kLog2; step > 0; step >>= 1)
    if (c + step <= n && precedes(a(c + step - 1), k, below_or_equal))
      c += step;
  return c;
}

// Rank kernel: a workgroup takes 256 consecutive elements of one sorted run,
// four threads per element (thread t: element t % 256, run group t / 256).
// The element's counts in another run o all lie in a window [L, U) of o that
// the run's samples bound: L from the samples that precede the chunk's first
// key, U from those that precede its last key (the chunk's keys ascend).
// The workgroup loads the other runs' windows into LDS in coalesced reads
// (kWinKeys keys at most, about 256 + 128 for runs of like key
// distributions; kLdsRuns runs at a time) and each thread finds its
// element's counts in its runs (o = group + 4 v) by binary searches there
// that advance together; a window longer than kWinKeys is searched in global
// memory.  The four partial ranks are added in LDS.
constexpr int kRankElems = 256;                  // elements per workgroup
constexpr int kRankSplit = 4;                    // threads per element
constexpr int kRankBlock = kRankElems * kRankSplit;
constexpr int kWinKeys = 512;
constexpr int kLdsRuns = 16;  // runs whose windows the LDS holds at once
constexpr int kRunsPerThread = kLdsRuns / kRankSplit;
constexpr int kLoadsPerThread = kLdsRuns * kWinKeys / kRankBlock;
static_assert(kRunItems % kRankElems == 0, "a rank workgroup lies in one run");
static_assert(kMaxRuns % kLdsRuns == 0, "run groups");

struct RankLds {
  uint32_t ss[kMaxRuns * kRunSamples];
  int wlo[kMaxRuns], wlen[kMaxRuns];
  uint32_t kfl[2];
  uint32_t win[kLdsRuns * kWinKeys];
  int part[kRankSplit][kRankElems];
};

// Rank step of workgroup `block` (kRankBlock threads): on_rank(base, pos, v)
// is called once per element, by a thread of group 0, with the image's
// first index base, the element's position pos in the image's stable order
// and its in-image index v.
template <class OnRank>
__device__ __forceinline__ void rank_block(
    const uint32_t* __restrict__ run_keys,
    const uint32_t* __restrict__ run_vals,
    const uint32_t* __restrict__ samples, int G, int runs, int block,
    RankLds& S, OnRank&& on_rank) {
  uint32_t* ss = S.ss;
  int* wlo = S.wlo;
  int* wlen = S.wlen;
  uint32_t* kfl = S.kfl;
  uint32_t* win = S.win;
  auto& part = S.part;
  const int t = threadIdx.x;
  const int el = t % kRankElems, grp = t / kRankElems;
  const int blocks_per_seg = (G + kRankElems - 1) / kRankElems;
  const int seg = block / blocks_per_seg;
  const int e0 = (block - seg * blocks_per_seg) * kRankElems;
  const int e = e0 + el;
  const int64_t base = (int64_t)seg * G;
  const int r = e0 / kRunItems;  // the chunk's run
  for (int i = t; i < runs * kRunSamples; i += kRankBlock)
    ss[i] = samples[(int64_t)seg * runs * kRunSamples + i];
  const int ec = min(e, G - 1);
  const uint32_t key = run_keys[base + ec];
  if (t == 0) kfl[0] = key;
  if (grp == 0 && e == min(e0 + kRankElems, G) - 1) kfl[1] = key;
  __syncthreads();
  if (t < runs) {
    const int o = t;
    int L = 0, U = 0;
    if (o != r) {
      const int len = min(kRunItems, G - o * kRunItems);
      const int ns = (len + kSampleStride - 1) / kSampleStride;
      const bool le = o < r;
      const uint32_t* so = ss + o * kRunSamples;
      auto ld = [so](int i) { return so[i]; };
      const int wf = prefix_count<6>(ld, ns, kfl[0], le);
      const int wl = prefix_count<6>(ld, ns, kfl[1], le);
      L = wf == 0 ? 0 : kSampleStride * (wf - 1) + 1;
      U = wl == 0 ? 0 : min(kSampleStride * wl, len);
      U = max(U, L);
    }
    wlo[o] = L;
    wlen[o] = U - L;
  }
  __syncthreads();
  int rank = grp == 0 ? e - r * kRunItems : 0;
  for (int l0 = 0; l0 < runs; l0 += kLdsRuns) {
    if (l0 > 0) __syncthreads();  // searches of the previous runs done
    // Windows of runs l0 .. l0 + kLdsRuns - 1 into LDS: every load in
    // flight before the first store (loads at clamped, in-run positions).
    uint32_t x[kLoadsPerThread];
#pragma unroll
    for (int k = 0; k < kLoadsPerThread; ++k) {
      const int f = t + kRankBlock * k;
      const int o = min(l0 + f / kWinKeys, runs - 1);
      const int len = min(kRunItems, G - o * kRunItems);
      const int n = min(wlen[o], kWinKeys);
      const int i = min(f % kWinKeys, max(n - 1, 0));
      x[k] = run_keys[base + (int64_t)o * kRunItems + min(wlo[o] + i, len - 1)];
    }
#pragma unroll
    for (int k = 0; k < kLoadsPerThread; ++k) {
      const int f = t + kRankBlock * k;
      const int o = l0 + f / kWinKeys;
      if (o < runs && f % kWinKeys < min(wlen[o], kWinKeys)) win[f] = x[k];
    }
    __syncthreads();
    // This thread's runs o = l0 + grp + kRankSplit v: binary searches that
    // advance together (n = 0 for runs not searched here).
    int c[kRunsPerThread], n[kRunsPerThread];
#pragma unroll
    for (int v = 0; v < kRunsPerThread; ++v) {
      const int o = l0 + grp + kRankSplit * v;
      c[v] = 0;
      n[v] = (o < runs && o != r && wlen[o] <= kWinKeys) ? wlen[o] : 0;
    }
#pragma unroll
    for (int step = kWinKeys; step > 0; step >>= 1) {
#pragma unroll
      for (int v = 0; v < kRunsPerThread; ++v) {
        const int u = grp + kRankSplit * v;  // run l0 + u
        const uint32_t x =
            win[u * kWinKeys + min(c[v] + step - 1, kWinKeys - 1)];
        if (c[v] + step <= n[v] && precedes(x, key, l0 + u < r)) c[v] += step;
      }
    }
#pragma unroll
    for (int v = 0; v < kRunsPerThread; ++v) {
      const int o = l0 + grp + kRankSplit * v;
      if (o < runs && o != r) {
        if (wlen[o] > kWinKeys) {  // rare: the window is searched in place
          const uint32_t* w =
              run_keys + base + (int64_t)o * kRunItems + wlo[o];
          c[v] = prefix_count<12>([w](int i) { return w[i]; }, wlen[o], key,
                                  o < r);
        }
        rank += wlo[o] + c[v];
      }
    }
  }
  part[grp][el] = rank;
  __syncthreads();
  if (grp == 0 && e < G) {
    const int pos = part[0][el] + part[1][el] + part[2][el] + part[3][el];
    on_rank(base, pos, run_vals[base + e]);
  }
}


}  // namespace run_step
}  // namespace gs
