// scan.hip -- device-wide exclusive prefix sum over int32 in one launch.
//
// Workgroups of 256 lanes each scan 4096 consecutive elements (coalesced
// loads into LDS, 16 consecutive elements per lane, a workgroup scan of the
// lane sums) and obtain the total of all earlier workgroups by decoupled
// look-back (lookback.h).  The look-back status (one 64-bit word per
// workgroup), the ticket and the give-up status word live in the caller's
// workspace and must be zero; exclusive_scan_i32 zeroes them unless told
// they already are.  A workgroup whose ticket is past the last block exits
// at once (only the stalled-predecessor diagnostic hands out such tickets).
#include "gs_internal.h"
#include "lookback.h"

namespace gs {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 16;
constexpr int kChunk = kThreads * kItems;   // 4096
constexpr int kPadded = kChunk + kChunk / 16;

__device__ __forceinline__ int pad(int j) { return j + (j >> 4); }

__global__ __launch_bounds__(kThreads) void scan_lookback_kernel(
    const int32_t* in, int32_t* out, int64_t n, uint64_t* status,
    uint32_t* ticket, uint32_t* err, int spin_limit) {
  __shared__ int sh[kPadded];
  __shared__ int wsum[kThreads / 64];
  __shared__ int64_t s_prefix;
  const int vb = take_ticket(ticket);
  if ((int64_t)vb * kChunk >= n && vb > 0) return;  // past the last block
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t base = (int64_t)vb * kChunk;
  // All loads in flight before any is used: clamped indices, no branches
  // between a load and its use (n == 0 loads nothing).
  int ld[kItems];
  if (n > 0) {
#pragma unroll
    for (int i = 0; i < kItems; ++i)
      ld[i] = in[min(base + i * kThreads + t, n - 1)];
  }
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int j = i * kThreads + t;
    sh[pad(j)] = (base + j < n) ? ld[i] : 0;
  }
  __syncthreads();
  int v[kItems];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    v[k] = sh[pad(t * kItems + k)];
    sum += v[k];
  }
  int inc = sum;
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
      status_store(&status[vb], (vb == 0 ? kFlagInc64 : kFlagAgg64) |
                                    (uint64_t)(uint32_t)total);
    uint64_t prefix = 0ull;
    if (vb > 0) {
      prefix = lookback64_wave(status, vb, err, spin_limit);
      if (lane == 0)
        status_store(&status[vb], kFlagInc64 | (prefix + (uint32_t)total));
    }
    if (lane == 0) s_prefix = (int64_t)prefix;
  }
  __syncthreads();
  int run = (int)s_prefix + pre + inc - sum;
#pragma unroll
  for (int k = 0; k < kItems; ++k) {
    sh[pad(t * kItems + k)] = run;
    run += v[k];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int j = i * kThreads + t;
    if (base + j < n) out[base + j] = sh[pad(j)];
  }
  // The workgroup holding element n-1 (the only one, for n == 0) writes the
  // total.
  const bool holds_last = (n == 0) ? (vb == 0) : (base < n && n <= base + kChunk);
  if (t == kThreads - 1 && holds_last) out[n] = (int)s_prefix + total;
}

}  // namespace

int64_t scan_blocks(int64_t n) { return n <= 0 ? 1 : (n + kChunk - 1) / kChunk; }

// Look-back status words, then 256 bytes for the ticket (word 0) and the
// give-up status (word 1).
size_t scan_workspace_bytes(int64_t n) {
  return align_up((size_t)scan_blocks(n) * sizeof(uint64_t) + 256, 256);
}

int exclusive_scan_i32(const int32_t* in, int32_t* out, int64_t n, void* ws,
                       size_t ws_bytes, hipStream_t stream, bool ctl_zeroed,
                       int32_t* status_out, int first_ticket, int spin_limit) {
  if (n < 0 || n > 0x7fffffffLL) {
    set_error("exclusive_scan: invalid length %lld", (long long)n);
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (ws == nullptr || ws_bytes < scan_workspace_bytes(n)) {
    set_error("exclusive_scan: workspace too small (%zu < %zu)", ws_bytes,
              scan_workspace_bytes(n));
    return GSPLAT_ERR_WORKSPACE;
  }
  const int64_t nb = scan_blocks(n);
  uint64_t* status = static_cast<uint64_t*>(ws);
  uint32_t* ticket = reinterpret_cast<uint32_t*>(status + nb);
  uint32_t* err = status_out ? reinterpret_cast<uint32_t*>(status_out) : ticket + 1;
  if (!ctl_zeroed) {
    const int rc = launch_zero2(static_cast<uint32_t*>(ws),
                                (int64_t)(scan_workspace_bytes(n) / 4),
                                reinterpret_cast<uint32_t*>(status_out),
                                status_out ? 1 : 0, stream);
    if (rc) return rc;
  }
  if (first_ticket > 0) {
    const int rc = launch_fill_i32(reinterpret_cast<int32_t*>(ticket),
                                   first_ticket, 1, stream);
    if (rc) return rc;
  }
  launch_traced("scan_lookback_kernel", scan_lookback_kernel,
                dim3((unsigned)nb), dim3(kThreads), 0, stream, in, out, n,
                status, ticket, err, spin_limit);
  return check_launch("scan_lookback_kernel");
}

}  // namespace gs
