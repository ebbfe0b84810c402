// radix_sort.hip -- stable LSD radix sort of (uint32 key, uint32 value) pairs
// with 8-bit digits, independently inside equal-length segments.
//
// Each pass is three launches with no inter-workgroup waiting:
//   1. rs_hist_kernel    per 4096-element block, digit counts
//                        -> hist[(segment*256 + digit)*nblk + block]
//   2. exclusive scan of hist (flattened), which yields for every
//      (segment, digit, block) the absolute output position of that block's
//      first element with that digit (segments are contiguous and equal, so
//      the flattened scan already includes segment*n)
//   3. rs_scatter_kernel recomputes stable in-block ranks, stages the block
//      in LDS in sorted order and writes it out so that each digit's run is a
//      contiguous, coalesced store.
//
// In-block ranking is wave-level: every wave owns 1024 consecutive elements
// and walks them 64 at a time; lanes holding the same digit are found with
// eight ballots ("match"), the rank is the popcount of matching lower lanes,
// and one leader lane per digit bumps the wave's running count.  Order
// inside a block is (wave, round, lane), which is input order, so the sort
// is stable.
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRounds = 16;
constexpr int kWaveItems = 64 * kRounds;           // 1024
constexpr int kBlockItems = kWaves * kWaveItems;   // 4096

// Order-preserving map of a float depth to uint32 (ascending float order ==
// ascending key).  -0.0 and +0.0 map to the same key (they compare equal in
// torch.argsort); every NaN maps above +inf (torch sorts NaN last).
__device__ __forceinline__ uint32_t depth_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (f == 0.0f) u = 0u;
  if (!(f == f)) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63u;
  return (lane == 0u) ? 0ull : (~0ull >> (64u - lane));
}

// Lanes of `active` whose digit equals this lane's digit.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t active,
                                                int digit_bits) {
  uint64_t m = active;
  for (int bit = 0; bit < digit_bits; ++bit) {
    const bool p = (d >> bit) & 1u;
    const uint64_t b = __ballot(p);
    m &= p ? b : ~b;
  }
  return m;
}

struct PassArgs {
  const uint32_t* keys_in;   // nullptr when depth_src is used
  const uint32_t* vals_in;   // nullptr -> in-segment index
  const float* depth_src;    // nullptr unless first pass of a depth sort
  uint32_t* keys_out;        // nullptr -> keys not written (last pass)
  uint32_t* vals_out;
  int64_t n_seg;
  int nblk;                  // blocks per segment
  int shift;
  int digit_bits;
};

__device__ __forceinline__ uint32_t load_key(const PassArgs& a, int64_t idx) {
  return a.depth_src ? depth_key(a.depth_src[idx]) : a.keys_in[idx];
}

__global__ __launch_bounds__(kThreads) void rs_hist_kernel(PassArgs a,
                                                           uint32_t* hist) {
  __shared__ uint32_t cnt[kWaves][256];
  const int seg = blockIdx.x / a.nblk;
  const int blk = blockIdx.x - seg * a.nblk;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int i = t; i < kWaves * 256; i += kThreads) (&cnt[0][0])[i] = 0u;
  __syncthreads();
  const int64_t seg_base = (int64_t)seg * a.n_seg;
  const int64_t lo = (int64_t)blk * kBlockItems + (int64_t)wave * kWaveItems;
  const uint32_t dmask = (1u << a.digit_bits) - 1u;
  for (int r = 0; r < kRounds; ++r) {
    const int64_t j = lo + r * 64 + lane;
    const bool valid = j < a.n_seg;
    const uint64_t act = __ballot(valid);
    if (act == 0ull) break;
    const uint32_t key = valid ? load_key(a, seg_base + j) : 0u;
    const uint32_t d = (key >> a.shift) & dmask;
    const uint64_t peers = match_digit(d, act, a.digit_bits);
    if (valid && (peers & lanemask_lt()) == 0ull)
      cnt[wave][d] += (uint32_t)__popcll(peers);
    // Other lanes read these counters next round: keep LDS ops in order.
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  const uint32_t total = cnt[0][t] + cnt[1][t] + cnt[2][t] + cnt[3][t];
  hist[((int64_t)seg * 256 + t) * a.nblk + blk] = total;
}

__global__ __launch_bounds__(kThreads) void rs_scatter_kernel(
    PassArgs a, const uint32_t* __restrict__ offs) {
  __shared__ uint32_t cnt[kWaves][256];
  __shared__ uint32_t dstart[256];
  __shared__ uint32_t gbase[256];
  __shared__ uint32_t wsum[kWaves];
  __shared__ uint32_t sk[kBlockItems];
  __shared__ uint32_t sv[kBlockItems];

  const int seg = blockIdx.x / a.nblk;
  const int blk = blockIdx.x - seg * a.nblk;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  for (int i = t; i < kWaves * 256; i += kThreads) (&cnt[0][0])[i] = 0u;
  __syncthreads();

  const int64_t seg_base = (int64_t)seg * a.n_seg;
  const int64_t lo = (int64_t)blk * kBlockItems + (int64_t)wave * kWaveItems;
  const uint32_t dmask = (1u << a.digit_bits) - 1u;
  uint32_t kreg[kRounds], vreg[kRounds], rreg[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int64_t j = lo + r * 64 + lane;
    const bool valid = j < a.n_seg;
    const uint64_t act = __ballot(valid);
    rreg[r] = 0xffffffffu;
    kreg[r] = 0u;
    vreg[r] = 0u;
    if (act != 0ull) {
      const uint32_t key = valid ? load_key(a, seg_base + j) : 0u;
      const uint32_t val =
          valid ? (a.vals_in ? a.vals_in[seg_base + j] : (uint32_t)j) : 0u;
      const uint32_t d = (key >> a.shift) & dmask;
      const uint64_t peers = match_digit(d, act, a.digit_bits);
      const uint32_t below = (uint32_t)__popcll(peers & lanemask_lt());
      const uint32_t old = valid ? cnt[wave][d] : 0u;
      if (valid && below == 0u) cnt[wave][d] = old + (uint32_t)__popcll(peers);
      __builtin_amdgcn_wave_barrier();
      if (valid) {
        kreg[r] = key;
        vreg[r] = val;
        rreg[r] = (old + below) | (d << 16);
      }
    }
  }
  __syncthreads();

  // Thread t owns digit t: exclusive prefix across waves, block-local digit
  // start (exclusive scan over digits) and the global base for this block.
  {
    const uint32_t c0 = cnt[0][t], c1 = cnt[1][t], c2 = cnt[2][t],
                   c3 = cnt[3][t];
    const uint32_t tot = c0 + c1 + c2 + c3;
    cnt[0][t] = 0u;
    cnt[1][t] = c0;
    cnt[2][t] = c0 + c1;
    cnt[3][t] = c0 + c1 + c2;
    uint32_t inc = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    uint32_t wprefix = 0u;
    for (int w = 0; w < wave; ++w) wprefix += wsum[w];
    dstart[t] = wprefix + inc - tot;
    gbase[t] = offs[((int64_t)seg * 256 + t) * a.nblk + blk];
  }
  __syncthreads();

#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (rreg[r] != 0xffffffffu) {
      const uint32_t d = rreg[r] >> 16;
      const uint32_t pos = dstart[d] + cnt[wave][d] + (rreg[r] & 0xffffu);
      sk[pos] = kreg[r];
      sv[pos] = vreg[r];
    }
  }
  __syncthreads();

  const int64_t remain = a.n_seg - (int64_t)blk * kBlockItems;
  const int count = remain < kBlockItems ? (int)remain : kBlockItems;
  for (int i = t; i < count; i += kThreads) {
    const uint32_t key = sk[i];
    const uint32_t d = (key >> a.shift) & dmask;
    const int64_t dst = (int64_t)gbase[d] + (int64_t)(i - (int)dstart[d]);
    if (a.keys_out) a.keys_out[dst] = key;
    a.vals_out[dst] = sv[i];
  }
}

// Zero-pass "sort": copy (deriving keys/values when needed).
__global__ void rs_copy_kernel(PassArgs a, int64_t n_total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_total) return;
  const int64_t j = i % a.n_seg;
  if (a.keys_out) a.keys_out[i] = load_key(a, i);
  a.vals_out[i] = a.vals_in ? a.vals_in[i] : (uint32_t)j;
}

struct WsLayout {
  size_t a_keys, a_vals, b_keys, b_vals, hist, scan, total;
};

WsLayout layout(int64_t n_seg, int segments, int passes) {
  const int64_t n = n_seg * (int64_t)segments;
  const int64_t nblk = (n_seg + kBlockItems - 1) / kBlockItems;
  const int64_t entries = (int64_t)segments * 256 * nblk;
  WsLayout L{};
  size_t off = 0;
  const size_t vec = align_up((size_t)n * sizeof(uint32_t), 256);
  if (passes >= 2) {
    L.a_keys = off; off += vec;
    L.a_vals = off; off += vec;
  }
  if (passes >= 3) {
    L.b_keys = off; off += vec;
    L.b_vals = off; off += vec;
  }
  L.hist = off;
  off += align_up((size_t)(entries + 1) * sizeof(uint32_t), 256);
  L.scan = off;
  off += scan_workspace_bytes(entries);
  L.total = off;
  return L;
}

int num_passes(int begin_bit, int end_bit) {
  return end_bit > begin_bit ? (end_bit - begin_bit + 7) / 8 : 0;
}

}  // namespace

size_t radix_sort_workspace_bytes(int64_t n_per_segment, int segments) {
  // Worst case: 4 passes over 32 bits.
  if (n_per_segment <= 0 || segments <= 0) return 0;
  return layout(n_per_segment, segments, 4).total;
}

int radix_sort_pairs(const uint32_t* keys_in, const uint32_t* vals_in,
                     const float* depth_src, uint32_t* keys_out,
                     uint32_t* vals_out, int64_t n_seg, int segments,
                     int begin_bit, int end_bit, void* ws, size_t ws_bytes,
                     hipStream_t stream) {
  if (n_seg < 0 || segments < 0 || begin_bit < 0 || end_bit > 32 ||
      (keys_in == nullptr && depth_src == nullptr) || vals_out == nullptr) {
    set_error("radix_sort: invalid arguments");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  if (n_seg == 0 || segments == 0) return GSPLAT_OK;
  const int64_t nblk = (n_seg + kBlockItems - 1) / kBlockItems;
  if (nblk * segments > 0x7fffffffLL || n_seg * segments > 0x7fffffffLL) {
    set_error("radix_sort: input too large");
    return GSPLAT_ERR_INVALID_ARGUMENT;
  }
  const int passes = num_passes(begin_bit, end_bit);
  const int64_t n = n_seg * segments;
  if (passes == 0) {
    PassArgs a{keys_in, vals_in, depth_src, keys_out, vals_out, n_seg, (int)nblk,
               0, 0};
    const int64_t grid = (n + 255) / 256;
    hipLaunchKernelGGL(rs_copy_kernel, dim3((unsigned)grid), dim3(256), 0,
                       stream, a, n);
    return check_launch("rs_copy_kernel");
  }
  const WsLayout L = layout(n_seg, segments, passes);
  if (ws == nullptr || ws_bytes < L.total) {
    set_error("radix_sort: workspace too small (%zu < %zu)", ws_bytes, L.total);
    return GSPLAT_ERR_WORKSPACE;
  }
  char* base = static_cast<char*>(ws);
  uint32_t* bufk[2] = {reinterpret_cast<uint32_t*>(base + L.a_keys),
                       reinterpret_cast<uint32_t*>(base + L.b_keys)};
  uint32_t* bufv[2] = {reinterpret_cast<uint32_t*>(base + L.a_vals),
                       reinterpret_cast<uint32_t*>(base + L.b_vals)};
  uint32_t* hist = reinterpret_cast<uint32_t*>(base + L.hist);
  void* scan_ws = base + L.scan;
  const int64_t entries = (int64_t)segments * 256 * nblk;
  const unsigned grid = (unsigned)(nblk * segments);

  const uint32_t* cur_k = keys_in;
  const uint32_t* cur_v = vals_in;
  const float* cur_depth = depth_src;
  for (int p = 0; p < passes; ++p) {
    const int shift = begin_bit + 8 * p;
    const int bits = (end_bit - shift) < 8 ? (end_bit - shift) : 8;
    const bool last = (p == passes - 1);
    uint32_t* out_k = last ? keys_out : bufk[p & 1];
    uint32_t* out_v = last ? vals_out : bufv[p & 1];
    PassArgs a{cur_k, cur_v, cur_depth, out_k, out_v, n_seg, (int)nblk, shift,
               bits};
    hipLaunchKernelGGL(rs_hist_kernel, dim3(grid), dim3(kThreads), 0, stream,
                       a, hist);
    int rc = check_launch("rs_hist_kernel");
    if (rc) return rc;
    rc = exclusive_scan_i32(reinterpret_cast<const int32_t*>(hist),
                            reinterpret_cast<int32_t*>(hist), entries, scan_ws,
                            scan_workspace_bytes(entries), stream);
    if (rc) return rc;
    hipLaunchKernelGGL(rs_scatter_kernel, dim3(grid), dim3(kThreads), 0,
                       stream, a, hist);
    rc = check_launch("rs_scatter_kernel");
    if (rc) return rc;
    cur_k = out_k;
    cur_v = out_v;
    cur_depth = nullptr;
  }
  return GSPLAT_OK;
}

}  // namespace gs
