// depth_sort.hip -- stable depth order of images of at most
// kMaxRuns * kRunItems = 131072 splats in two launches (the per-image depth argsort of the reference,
// variants/v8/torch_gsplat_bridge_v8/rasterize.py:466).
//
// Larger images use the onesweep radix sort (radix_sort.hip), whose four
// passes each pay a look-back chain and a kernel launch; at 64K splats
// those latencies, not bandwidth, set its time.  Here:
//
//   depth_run_sort_kernel  one workgroup per run of kRunItems consecutive
//     splats of an image: a stable LSD radix sort of the run in LDS (four
//     8-bit passes over the depth keys; element order (wavefront, round,
//     lane) = index order, ranks from ballot matching as in the onesweep
//     kernel), then the sorted keys and in-image indices of the run and
//     every kSampleStride-th sorted key (the run's samples).
//   depth_run_rank_kernel  a workgroup per 256 consecutive elements of a
//     sorted run, four threads per element: an element's position in the
//     image's order is its position in its own run plus, for every other
//     run of the image, the number of that run's keys that precede it (keys
//     < k for later runs, keys <= k for earlier runs, so equal keys keep
//     index order).  The run's samples bound those counts, for the whole
//     chunk, to a window of the other run (about 256 + 128 keys), which the
//     workgroup loads into LDS; each thread binary-searches its element's
//     counts in a quarter of the runs there and the four partial positions
//     are added.  perm[rank] = in-image index.
//
// No atomics, look-back or control words: nothing needs zeroing and the two
// launches are independent of earlier calls.
#include "depth_runs.h"

namespace gs {
using namespace run_step;
namespace {

__global__ __launch_bounds__(kRunThreads) void depth_run_sort_kernel(
    const float* __restrict__ depths, int G, int runs, RunBuffers out) {
  __shared__ RunSortLds S;
  run_sort_block(depths, G, runs, (int)blockIdx.x, out, S);
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

__global__ __launch_bounds__(kRankBlock) void depth_run_rank_kernel(
    const uint32_t* __restrict__ run_keys,
    const uint32_t* __restrict__ run_vals,
    const uint32_t* __restrict__ samples, int G, int runs,
    int32_t* __restrict__ perm) {
  __shared__ uint32_t ss[kMaxRuns * kRunSamples];
  __shared__ int wlo[kMaxRuns], wlen[kMaxRuns];
  __shared__ uint32_t kfl[2];
  __shared__ uint32_t win[kLdsRuns * kWinKeys];
  __shared__ int part[kRankSplit][kRankElems];
  const int t = threadIdx.x;
  const int el = t % kRankElems, grp = t / kRankElems;
  const int blocks_per_seg = (G + kRankElems - 1) / kRankElems;
  const int seg = blockIdx.x / blocks_per_seg;
  const int e0 = (blockIdx.x - seg * blocks_per_seg) * kRankElems;
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
    perm[base + pos] = (int32_t)run_vals[base + e];
  }
}

}  // namespace

bool depth_small_ok(int64_t G) {
  return G >= 1 && G <= (int64_t)kMaxRuns * kRunItems;
}

size_t depth_small_bytes(int64_t G, int batch) {
  const size_t vec = align_up((size_t)(G * batch) * sizeof(uint32_t), 256);
  return 2 * vec + align_up((size_t)batch * runs_of(G) * kRunSamples *
                                sizeof(uint32_t), 256);
}

int launch_depth_ranks_small(void* buffers, int32_t* perm, int64_t G,
                             int batch, hipStream_t stream) {
  if (!depth_small_ok(G) || batch < 1) {
    set_error("depth order: %lld splats per image exceed the two-launch sort",
              (long long)G);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const RunBuffers b = run_buffers(buffers, G, batch);
  const int blocks_per_seg = (int)((G + kRankElems - 1) / kRankElems);
  hipLaunchKernelGGL(depth_run_rank_kernel,
                     dim3((unsigned)((int64_t)batch * blocks_per_seg)),
                     dim3(kRankBlock), 0, stream, b.keys, b.vals, b.samples,
                     (int)G, runs_of(G), perm);
  return check_launch("depth_run_rank_kernel");
}

int launch_depth_order_small(const float* depths, int32_t* perm, int64_t G,
                             int batch, void* buffers, hipStream_t stream) {
  if (!depth_small_ok(G) || batch < 1) {
    set_error("depth order: %lld splats per image exceed the two-launch sort",
              (long long)G);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int runs = runs_of(G);
  hipLaunchKernelGGL(depth_run_sort_kernel, dim3((unsigned)(batch * runs)),
                     dim3(kRunThreads), 0, stream, depths, (int)G, runs,
                     run_buffers(buffers, G, batch));
  const int rc = check_launch("depth_run_sort_kernel");
  if (rc) return rc;
  return launch_depth_ranks_small(buffers, perm, G, batch, stream);
}

}  // namespace gs
