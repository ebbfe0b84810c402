// lookback.h -- decoupled look-back: a workgroup obtains the exclusive prefix
// of per-workgroup totals without a separate scan launch.
//
// Workgroups are ordered by a ticket (atomic counter) taken when they start,
// so that a workgroup only ever waits for workgroups with smaller tickets,
// which are already running (the scans), or by their index (radix_sort.hip,
// where the dispatch order gives the same property and the ticket's round
// trip was measured to cost more).  A workgroup publishes its own total
// (flag AGG) before it looks back, then its inclusive prefix (flag INC).
// Payload and flag share one word, so relaxed device-scope atomics suffice.
// Predecessor statuses are read several at a time (independent loads) so the
// walk costs one memory round trip per window rather than per predecessor.
// Waits are bounded:
// after spin_limit polls (kMaxSpins unless a caller passes less) the wait
// gives up, ORs GSPLAT_STATUS_LOOKBACK_TIMEOUT into the caller's status word
// and returns the partial prefix.  Every wave therefore terminates, and the
// status word (which the host reads back) says that the results are wrong.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gsplat_hip.h"

namespace gs {

constexpr uint32_t kFlagAgg32 = 1u << 30;
constexpr uint32_t kFlagInc32 = 2u << 30;
constexpr uint32_t kVal32 = (1u << 30) - 1u;
constexpr uint64_t kFlagAgg64 = 1ull << 62;
constexpr uint64_t kFlagInc64 = 2ull << 62;
constexpr uint64_t kVal64 = (1ull << 62) - 1ull;
constexpr int kMaxSpins = 1 << 20;

__device__ __forceinline__ void report_giveup(uint32_t* err) {
  if (err != nullptr) atomicOr(err, (uint32_t)GSPLAT_STATUS_LOOKBACK_TIMEOUT);
}

__device__ __forceinline__ uint32_t status_load(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void status_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t status_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void status_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix of slot `blk` from the 32-bit statuses of slots
// blk-1, blk-2, ... stored `stride` words apart; one thread, windows of W.
template <int W>
__device__ __forceinline__ uint32_t lookback32(const uint32_t* status, int blk,
                                              int stride, uint32_t* err,
                                              int spin_limit = kMaxSpins) {
  uint32_t prefix = 0u;
  int b = blk - 1;
  int spins = 0;
  while (b >= 0) {
    // Clamped indices and a select after the load keep the W loads
    // independent (no branch between a load and its use).
    uint32_t s[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
      s[k] = status_load(status + (int64_t)max(b - k, 0) * stride);
#pragma unroll
    for (int k = 0; k < W; ++k)
      if (b - k < 0) s[k] = kFlagInc32;
    int consumed = 0;
    bool done = false, wait = false;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      if (done || wait) continue;
      const uint32_t flag = s[k] & ~kVal32;
      if (flag == 0u) {
        wait = true;
        continue;
      }
      prefix += s[k] & kVal32;
      ++consumed;
      if (flag == kFlagInc32) done = true;
    }
    if (done) break;
    b -= consumed;
    if (wait) {
      if (++spins > spin_limit) {
        report_giveup(err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return prefix;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Exclusive prefix of slot `blk` from 64-bit statuses status[0..blk-1],
// computed by one whole wavefront (64 predecessors per round trip).  Every
// lane of the calling wave must call it; all lanes receive the result.
__device__ __forceinline__ uint64_t lookback64_wave(const uint64_t* status,
                                                    int blk, uint32_t* err,
                                                    int spin_limit = kMaxSpins) {
  const int lane = threadIdx.x & 63;
  uint64_t prefix = 0ull;
  int b = blk - 1;
  int spins = 0;
  while (b >= 0) {
    const int idx = b - lane;
    const uint64_t s = (idx >= 0) ? status_load(status + idx) : kFlagInc64;
    const uint64_t flag = s & ~kVal64;
    const uint64_t inc_mask = __ballot(flag == kFlagInc64);
    const uint64_t not_ready = __ballot(flag == 0ull);
    const int first_inc = inc_mask ? (__ffsll((long long)inc_mask) - 1) : 64;
    const uint64_t need =
        first_inc >= 63 ? ~0ull : ((2ull << first_inc) - 1ull);
    if (not_ready & need) {
      if (++spins > spin_limit) {
        if ((threadIdx.x & 63) == 0) report_giveup(err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      continue;
    }
    prefix += wave_sum_u64(lane <= first_inc ? (s & kVal64) : 0ull);
    if (first_inc < 64) break;
    b -= 64;
  }
  return prefix;
}

// Ticket = order in which workgroups of this launch started.
__device__ __forceinline__ int take_ticket(uint32_t* counter) {
  __shared__ int s_ticket;
  if (threadIdx.x == 0) s_ticket = (int)atomicAdd(counter, 1u);
  __syncthreads();
  return s_ticket;
}

}  // namespace gs
