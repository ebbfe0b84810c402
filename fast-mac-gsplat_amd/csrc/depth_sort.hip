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

__global__ __launch_bounds__(kRankBlock) void depth_run_rank_kernel(
    const uint32_t* __restrict__ run_keys,
    const uint32_t* __restrict__ run_vals,
    const uint32_t* __restrict__ samples, int G, int runs,
    int32_t* __restrict__ perm) {
  __shared__ RankLds S;
  rank_block(run_keys, run_vals, samples, G, runs, (int)blockIdx.x, S,
             [&](int64_t base, int pos, uint32_t v) {
               perm[base + pos] = (int32_t)v;
             });
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
  launch_traced("depth_run_rank_kernel", depth_run_rank_kernel,
                dim3((unsigned)((int64_t)batch * blocks_per_seg)),
                dim3(kRankBlock), 0, stream, b.keys, b.vals, b.samples, (int)G,
                runs_of(G), perm);
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
  launch_traced("depth_run_sort_kernel", depth_run_sort_kernel,
                dim3((unsigned)(batch * runs)), dim3(kRunThreads), 0, stream,
                depths, (int)G, runs, run_buffers(buffers, G, batch));
  const int rc = check_launch("depth_run_sort_kernel");
  if (rc) return rc;
  return launch_depth_ranks_small(buffers, perm, G, batch, stream);
}

}  // namespace gs
