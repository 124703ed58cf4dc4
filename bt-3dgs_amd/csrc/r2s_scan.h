// Device-wide exclusive prefix sum (reduce -> scan partials -> downsweep).
//
// 256-thread blocks, 4096 items per block taken as 16 chunks of 256: item
// k * 256 + t of a block belongs to thread t, so every load and store of a
// wave covers 64 consecutive items.  The partial sums of all blocks are
// scanned by one 1024-thread block, so a scan of n items needs
// ceil(n / 4096) partials of workspace.  Deterministic: the same input always
// produces the same output.
#pragma once

#include "r2s_common.h"

namespace r2s {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

inline int64_t scan_partials_count(int64_t n) { return ceil_div(n, kScanTile); }

// Exclusive scan across the block; `total` receives the block sum.
// `lds` needs blockDim.x / 64 entries.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T *lds, T &total) {
  const uint32_t w = threadIdx.x / 64, l = threadIdx.x % 64, nw = blockDim.x / 64;
  const T incl = wave_inclusive_scan(v);
  if (l == 63) lds[w] = incl;
  __syncthreads();
  T off = 0, tot = 0;
  for (uint32_t k = 0; k < nw; ++k) {
    const T s = lds[k];
    if (k < w) off += s;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return off + incl - v;
}

template <typename Tin, typename Tout>
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const Tin *__restrict__ in,
                                                                   int64_t n,
                                                                   Tout *__restrict__ partials) {
  __shared__ Tout lds[kScanThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x;
  // Loads clamped in bounds and masked after, so all of them issue at once.
  Tin v[kScanItems];
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) v[k] = in[min(base + k * kScanThreads, n - 1)];
  Tout s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k)
    if (base + k * kScanThreads < n) s += static_cast<Tout>(v[k]);
  Tout total;
  block_exclusive_scan(s, lds, total);
  if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Single block of 1024 threads: exclusive scan of the partials in place and
// the grand total (if `total` is not null).
template <typename Tout>
__global__ __launch_bounds__(1024) void scan_partials_kernel(Tout *__restrict__ partials,
                                                             int64_t nb,
                                                             Tout *__restrict__ total) {
  __shared__ Tout lds[16];
  Tout running = 0;
  for (int64_t start = 0; start < nb; start += 1024) {
    const int64_t i = start + threadIdx.x;
    const Tout v = (i < nb) ? partials[i] : static_cast<Tout>(0);
    Tout chunk;
    const Tout ex = block_exclusive_scan(v, lds, chunk);
    if (i < nb) partials[i] = running + ex;
    running += chunk;
  }
  if (threadIdx.x == 0 && total != nullptr) *total = running;
}

// Per chunk: a wave scan; then one scan over the 64 (chunk, wave) totals in
// item order gives each chunk-wave its offset within the block.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kScanThreads) void scan_down_kernel(const Tin *__restrict__ in,
                                                                 int64_t n,
                                                                 const Tout *__restrict__ partials,
                                                                 Tout *__restrict__ out) {
  static_assert(kScanItems * (kScanThreads / 64) == 64, "one wave scans the chunk totals");
  __shared__ Tout s_tot[64];
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x;
  Tout v[kScanItems], incl[kScanItems];
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k * kScanThreads;
    const Tin x = in[min(i, n - 1)];
    v[k] = i < n ? static_cast<Tout>(x) : static_cast<Tout>(0);
  }
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    incl[k] = wave_inclusive_scan(v[k]);
    if (lane == 63) s_tot[k * (kScanThreads / 64) + w] = incl[k];
  }
  __syncthreads();
  if (w == 0) {  // each lane reads, then overwrites, its own entry
    const Tout t = s_tot[lane];
    s_tot[lane] = wave_inclusive_scan(t) - t;
  }
  __syncthreads();
  const Tout p = partials[blockIdx.x];
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k * kScanThreads;
    if (i < n) out[i] = p + s_tot[k * (kScanThreads / 64) + w] + incl[k] - v[k];
  }
}

// out[i] = sum_{j<i} in[j] for i < n; *total = sum of all (if not null).
// `partials` must hold scan_partials_count(n) elements.
template <typename Tin, typename Tout>
int device_exclusive_scan(const Tin *in, int64_t n, Tout *out, Tout *total, Tout *partials,
                          hipStream_t stream, const char *what) {
  const int64_t nb = scan_partials_count(n);
  if (nb > 0) {
    scan_reduce_kernel<Tin, Tout><<<dim3(static_cast<uint32_t>(nb)), dim3(kScanThreads), 0, stream>>>(
        in, n, partials);
  }
  scan_partials_kernel<Tout><<<dim3(1), dim3(1024), 0, stream>>>(partials, nb, total);
  if (nb > 0) {
    scan_down_kernel<Tin, Tout><<<dim3(static_cast<uint32_t>(nb)), dim3(kScanThreads), 0, stream>>>(
        in, n, partials, out);
  }
  return check_launch(what);
}

template <typename T>
__global__ __launch_bounds__(256) void fill_kernel(T *__restrict__ p, int64_t n, T v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

template <typename T>
int device_fill(T *p, int64_t n, T v, hipStream_t stream, const char *what) {
  if (n <= 0) return R2S_OK;
  fill_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(n, 256))), dim3(256), 0, stream>>>(p, n, v);
  return check_launch(what);
}

}  // namespace r2s
