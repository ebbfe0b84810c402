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

}  // namespace run_step
}  // namespace gs
