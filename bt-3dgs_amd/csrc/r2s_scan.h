// Device-wide exclusive prefix sum: block sums, then a downsweep.
//
// 256-thread blocks, 4096 items per block taken as 16 chunks of 256: item
// k * 256 + t of a block belongs to thread t, so every load and store of a
// wave covers 64 consecutive items.  Up to kScanDirectBlocks blocks, block b
// of the downsweep adds up the b block sums before it itself (from L2; two
// launches in all), which costs less than scanning them.  Above that the
// per-block reads would grow as the square of the block count, so the
// block sums are first scanned by the same routine (one level down, out of
// place) and each block reads its own offset.  Deterministic: the same
// input always produces the same output.
#pragma once

#include "r2s_common.h"

namespace r2s {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

constexpr int64_t kScanDirectBlocks = 1024;

// Workspace elements of a scan of n items: the block sums, and above
// kScanDirectBlocks blocks also their scan and its own workspace.
inline int64_t scan_partials_count(int64_t n) {
  const int64_t nb = ceil_div(n, kScanTile);
  return nb > kScanDirectBlocks ? 2 * nb + scan_partials_count(nb) : nb;
}

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

// Per chunk: a wave scan; then one scan over the 64 (chunk, wave) totals in
// item order gives each chunk-wave its offset within the block.  The block's
// own offset is the sum of the partials of the blocks before it; the last
// block also writes the grand total (if `total` is not null).
// kScanned: partials[b] already holds block b's offset (the scanned block
// sums); otherwise the block sums them.
template <typename Tin, typename Tout, bool kScanned>
__global__ __launch_bounds__(kScanThreads) void scan_down_kernel(const Tin *__restrict__ in,
                                                                 int64_t n,
                                                                 const Tout *__restrict__ partials,
                                                                 Tout *__restrict__ out,
                                                                 Tout *__restrict__ total) {
  static_assert(kScanItems * (kScanThreads / 64) == 64, "one wave scans the chunk totals");
  __shared__ Tout s_tot[64];
  __shared__ Tout s_pre[kScanThreads / 64];
  __shared__ Tout s_block;
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
    const Tout it = wave_inclusive_scan(t);
    s_tot[lane] = it - t;
    if (lane == 63) s_block = it;
  }
  Tout p = 0;
  if constexpr (kScanned) {
    p = partials[blockIdx.x];
    __syncthreads();
  } else {
    // Sum of the earlier blocks' partials: strided over the threads, then
    // wave sums and one fixed-order pass over the waves.
    Tout pre = 0;
    for (uint32_t b = threadIdx.x; b < blockIdx.x; b += kScanThreads) pre += partials[b];
    pre = wave_sum(pre);
    if (lane == 0) s_pre[w] = pre;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kScanThreads / 64; ++k) p += s_pre[k];
  }
  if (threadIdx.x == 0 && total != nullptr && blockIdx.x == gridDim.x - 1) *total = p + s_block;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k * kScanThreads;
    if (i < n) out[i] = p + s_tot[k * (kScanThreads / 64) + w] + incl[k] - v[k];
  }
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

template <typename Tin, typename Tout>
int device_exclusive_scan(const Tin *in, int64_t n, Tout *out, Tout *total, Tout *partials,
                          hipStream_t stream, const char *what);

// The downsweep of device_exclusive_scan, for a caller whose kernel already
// stored the block sums (partials[b] = the sum of items [b kScanTile,
// (b + 1) kScanTile), as scan_reduce_kernel does).  n > 0.
template <typename Tin, typename Tout>
int device_exclusive_scan_from_sums(const Tin *in, int64_t n, Tout *out, Tout *total,
                                    Tout *partials, hipStream_t stream, const char *what) {
  const int64_t nb = ceil_div(n, kScanTile);
  const dim3 grid(static_cast<uint32_t>(nb)), block(kScanThreads);
  if (nb <= kScanDirectBlocks) {
    scan_down_kernel<Tin, Tout, false><<<grid, block, 0, stream>>>(in, n, partials, out, total);
    return check_launch(what);
  }
  // Block offsets: the scan of the nb block sums into partials[nb, 2 nb).
  R2S_RETURN_IF(check_launch(what));
  R2S_RETURN_IF((device_exclusive_scan<Tout, Tout>(partials, nb, partials + nb, nullptr,
                                                   partials + 2 * nb, stream, what)));
  scan_down_kernel<Tin, Tout, true><<<grid, block, 0, stream>>>(in, n, partials + nb, out, total);
  return check_launch(what);
}

// out[i] = sum_{j<i} in[j] for i < n; *total = sum of all (if not null).
// `partials` must hold scan_partials_count(n) elements.
template <typename Tin, typename Tout>
int device_exclusive_scan(const Tin *in, int64_t n, Tout *out, Tout *total, Tout *partials,
                          hipStream_t stream, const char *what) {
  const int64_t nb = ceil_div(n, kScanTile);
  if (nb <= 0) {
    if (total != nullptr) return device_fill<Tout>(total, 1, static_cast<Tout>(0), stream, what);
    return R2S_OK;
  }
  scan_reduce_kernel<Tin, Tout><<<dim3(static_cast<uint32_t>(nb)), dim3(kScanThreads), 0,
                                  stream>>>(in, n, partials);
  R2S_RETURN_IF(check_launch(what));
  return device_exclusive_scan_from_sums<Tin, Tout>(in, n, out, total, partials, stream, what);
}

}  // namespace r2s
