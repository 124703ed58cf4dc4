// Per-record partial rows and their per-Gaussian reduction.
//
// The backward kernels walk records in tile order, where every record of a
// Gaussian lands in a different tile.  Adding each record's partials to the
// Gaussian's gradient with device-scope float atomics runs at about 21 G
// atomics/s on MI355X (measured for scattered fp32 adds), which dominates the
// backward passes.  Instead a kernel stores each record's partials as one
// 16-value row of a workspace at the record's emission index; in emission
// order the records of one Gaussian are consecutive, so a streaming pass sums
// each Gaussian's rows with a segmented wave reduction and writes the sums
// once -- plain read-modify-writes, and atomics only for a Gaussian whose
// rows span two waves.  The result does not depend on scheduling.
#pragma once

#include "r2s_common.h"

namespace r2s {

constexpr int kRowStride = 16;  // values per row: 64 bytes (float) / 128 (double)

template <typename T, int NV>
__device__ __forceinline__ void store_row(T *__restrict__ rows, int64_t e, const T (&v)[NV]) {
  static_assert(NV <= kRowStride, "row too long");
  T *dst = rows + e * kRowStride;
#pragma unroll
  for (int c = 0; c < NV; ++c) dst[c] = v[c];
}

// Destination of row value c: ptr[c][g * stride[c]].
template <typename T, int NV>
struct RowTargets {
  T *ptr[NV];
  int stride[NV];
};

template <typename T, int NV>
__global__ __launch_bounds__(256) void row_reduce_kernel(const T *__restrict__ rows,
                                                         const int32_t *__restrict__ emit_ids,
                                                         int64_t n, int64_t n_items,
                                                         RowTargets<T, NV> tg) {
  const int64_t eb = static_cast<int64_t>(blockIdx.x) * 256 + 64 * wave_index();
  if (eb >= n) return;  // uniform per wave
  const uint32_t lane = lane_id();
  const int64_t e = eb + lane;
  const bool in = e < n;
  const int64_t g = in ? static_cast<int64_t>(emit_ids[e]) : -1;
  const int32_t seg = (g >= 0 && g < n_items) ? static_cast<int32_t>(g)
                                               : -1 - static_cast<int32_t>(lane);
  const WaveSegments segs(seg);
  const int32_t seg_prev = __shfl_up(seg, 1, 64);
  const bool head = seg >= 0 && (lane == 0 || seg_prev != seg);
  // Does the Gaussian of lane 0 / lane 63 continue in the previous / next wave?
  const int32_t before = (eb > 0) ? emit_ids[eb - 1] : -1;
  const int32_t after = (eb + 64 < n) ? emit_ids[eb + 64] : -1;
  const int32_t seg_last = __shfl(seg, 63, 64);
  const bool shared = (lane == 0 && before == seg) || (seg == seg_last && after == seg);
  T v[NV];
  const T *src = rows + (in ? e : 0) * kRowStride;
#pragma unroll
  for (int c = 0; c < NV; ++c) v[c] = in ? src[c] : static_cast<T>(0);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const T s = segs.suffix_sum(v[c]);
    if (head) segment_store(tg.ptr[c], g * tg.stride[c], s, shared);
  }
}

template <typename T, int NV>
void launch_row_reduce(const T *rows, const int32_t *emit_ids, int64_t n, int64_t n_items,
                       const RowTargets<T, NV> &tg, hipStream_t stream) {
  row_reduce_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n, 256))), dim3(256), 0,
                             stream>>>(rows, emit_ids, n, n_items, tg);
}

}  // namespace r2s
