// scan.hip -- device-wide exclusive prefix sum over int32.
//
// Small inputs (<= kSingleMax) use one 1024-thread workgroup that walks the
// array in 8192-element chunks with a running carry (one launch).  Larger
// inputs use reduce-then-scan: per-chunk sums, a single-workgroup scan of the
// chunk sums, and a rescan of each chunk with its carry (three launches, no
// inter-workgroup waiting).
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kThreads = 1024;
constexpr int kItems = 8;
constexpr int kChunk = kThreads * kItems;   // 8192
constexpr int64_t kSingleMax = 1 << 18;

__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

// Exclusive scan of one value per thread across the 1024-thread block.
// Returns the exclusive prefix; *total receives the block sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* wave_sums,
                                                    int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inc = wave_inclusive_scan(v, lane);
  if (lane == 63) wave_sums[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const int w = (lane < kThreads / 64) ? wave_sums[lane] : 0;
    const int winc = wave_inclusive_scan(w, lane);
    if (lane < kThreads / 64) wave_sums[lane] = winc - w;   // exclusive
    if (lane == kThreads / 64 - 1) wave_sums[kThreads / 64] = winc;
  }
  __syncthreads();
  const int r = wave_sums[wave] + inc - v;
  *total = wave_sums[kThreads / 64];
  __syncthreads();
  return r;
}

// Scans chunk [base, base+kChunk) of `in` into `out` with the given carry.
// Returns the chunk's sum.
__device__ __forceinline__ int scan_chunk(const int32_t* in, int32_t* out,
                                          int64_t n, int64_t base, int carry,
                                          int* sh, int* wave_sums) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + (int64_t)i * kThreads + t;
    sh[i * kThreads + t] = (idx < n) ? in[idx] : 0;
  }
  __syncthreads();
  int vals[kItems];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    vals[i] = sh[t * kItems + i];
    sum += vals[i];
  }
  int total;
  int run = block_exclusive_scan(sum, wave_sums, &total) + carry;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    sh[t * kItems + i] = run;
    run += vals[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + (int64_t)i * kThreads + t;
    if (idx < n) out[idx] = sh[i * kThreads + t];
  }
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kThreads) void scan_single_kernel(
    const int32_t* in, int32_t* out, int64_t n) {
  __shared__ int sh[kChunk];
  __shared__ int wave_sums[kThreads / 64 + 1];
  int carry = 0;
  for (int64_t base = 0; base < n; base += kChunk) {
    carry += scan_chunk(in, out, n, base, carry, sh, wave_sums);
  }
  if (threadIdx.x == 0) out[n] = carry;
}

__global__ __launch_bounds__(kThreads) void chunk_sum_kernel(
    const int32_t* in, int64_t n, int32_t* partial) {
  __shared__ int wave_sums[kThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  int s = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int64_t idx = base + (int64_t)i * kThreads + threadIdx.x;
    if (idx < n) s += in[idx];
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) wave_sums[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < kThreads / 64; ++w) t += wave_sums[w];
    partial[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(kThreads) void chunk_rescan_kernel(
    const int32_t* in, int32_t* out, int64_t n, const int32_t* partial,
    int64_t nb) {
  __shared__ int sh[kChunk];
  __shared__ int wave_sums[kThreads / 64 + 1];
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  scan_chunk(in, out, n, base, partial[blockIdx.x], sh, wave_sums);
  if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = partial[nb];
}

}  // namespace

size_t scan_workspace_bytes(int64_t n) {
  if (n <= kSingleMax) return 0;
  const int64_t nb = (n + kChunk - 1) / kChunk;
  return align_up((size_t)(nb + 1) * sizeof(int32_t), 256);
}

int exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  if (n < 0) {
    set_error("exclusive_scan: negative length");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (n <= kSingleMax) {
    hipLaunchKernelGGL(scan_single_kernel, dim3(1), dim3(kThreads), 0, stream,
                       in, out, n);
    return check_launch("scan_single_kernel");
  }
  const int64_t nb = (n + kChunk - 1) / kChunk;
  if (ws == nullptr || ws_bytes < scan_workspace_bytes(n)) {
    set_error("exclusive_scan: workspace too small (%zu < %zu)", ws_bytes,
              scan_workspace_bytes(n));
    return GSPLAT_ERR_WORKSPACE;
  }
  if (nb > 0x7fffffff) {
    set_error("exclusive_scan: input too large");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  int32_t* partial = static_cast<int32_t*>(ws);
  hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)nb), dim3(kThreads), 0,
                     stream, in, n, partial);
  int rc = check_launch("chunk_sum_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(scan_single_kernel, dim3(1), dim3(kThreads), 0, stream,
                     partial, partial, nb);
  rc = check_launch("scan_single_kernel(partials)");
  if (rc) return rc;
  hipLaunchKernelGGL(chunk_rescan_kernel, dim3((unsigned)nb), dim3(kThreads),
                     0, stream, in, out, n, partial, nb);
  return check_launch("chunk_rescan_kernel");
}

}  // namespace gs
