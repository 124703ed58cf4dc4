// Per-record partial rows and their per-Gaussian reduction.
//
// The backward kernels walk records in tile order, where every record of a
// Gaussian lands in a different tile.  Adding each record's partials to the
// Gaussian's gradient with device-scope float atomics runs at about 21 G
// atomics/s on MI355X (measured for scattered fp32 adds), which dominates the
// backward passes.  Instead a kernel stores each record's partials as one
// 12-value row of a workspace at the record's emission index; in emission
// order the records of one Gaussian are consecutive, so a streaming pass sums
// each Gaussian's rows with a segmented wave reduction and writes the sums
// once with plain stores.  The result does not depend on scheduling.
#pragma once

#include "r2s_common.h"

namespace r2s {

// Values per row: 48 bytes (float) / 96 (double), three 16-byte vectors; the
// rasterizer stores 9 partials, the voxelizer 10.
constexpr int kRowStride = 12;

template <typename T>
struct Quad;
template <>
struct Quad<float> {
  using type = float4;  // 16 bytes
  static constexpr int n = 4;
};
template <>
struct Quad<double> {
  using type = double2;  // 16 bytes
  static constexpr int n = 2;
};

// Rows start at multiples of 48 (float) / 96 (double) bytes from a
// 16-byte-aligned workspace, so they are written and read as 16-byte vectors.
template <typename T, int NV>
__device__ __forceinline__ void store_row(T *__restrict__ rows, int64_t e, const T (&v)[NV]) {
  static_assert(NV <= kRowStride, "row too long");
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n, nq = (NV + kq - 1) / kq;
  T pad[nq * kq];
#pragma unroll
  for (int c = 0; c < nq * kq; ++c) pad[c] = c < NV ? v[c] : static_cast<T>(0);
  Q *dst = reinterpret_cast<Q *>(rows + e * kRowStride);
#pragma unroll
  for (int q = 0; q < nq; ++q) dst[q] = *reinterpret_cast<const Q *>(pad + q * kq);
}

template <typename T, int NV>
__device__ __forceinline__ void load_row(const T *__restrict__ rows, int64_t e, T (&v)[NV]) {
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n, nq = (NV + kq - 1) / kq;
  T pad[nq * kq];
  const Q *src = reinterpret_cast<const Q *>(rows + e * kRowStride);
#pragma unroll
  for (int q = 0; q < nq; ++q) *reinterpret_cast<Q *>(pad + q * kq) = src[q];
#pragma unroll
  for (int c = 0; c < NV; ++c) v[c] = pad[c];
}

// The upstream-gradient segment of one tile / brick row: vv[k] = row[k] for
// k < n, 0 beyond (and everywhere when !in).  kVec: 16-byte loads, valid
// when the row pointer is 16-byte aligned and n, ts are multiples of the
// vector width (vec_rows_ok), so a vector is either wholly inside or outside.
template <typename T, int R, bool kVec>
__device__ __forceinline__ void load_grad_row(const T *__restrict__ row, bool in, int n, int ts,
                                              T (&vv)[R]) {
  if (kVec) {
    using Q = typename Quad<T>::type;
    constexpr int kq = Quad<T>::n;
#pragma unroll
    for (int q = 0; q < R / kq; ++q) {
      Q x;
      if (q * kq < ts && in && q * kq < n) {
        x = *reinterpret_cast<const Q *>(row + q * kq);
      } else {
        T *z = reinterpret_cast<T *>(&x);
#pragma unroll
        for (int c = 0; c < kq; ++c) z[c] = 0;
      }
      *reinterpret_cast<Q *>(vv + q * kq) = x;
    }
  } else {
#pragma unroll
    for (int k = 0; k < R; ++k) vv[k] = (k < ts && in && k < n) ? row[k] : static_cast<T>(0);
  }
}

// Whether every row segment of a [.., width] array cut into ts-wide tiles
// starts on a 16-byte boundary.
template <typename T>
inline bool vec_rows_ok(const T *base, uint32_t width, uint32_t ts) {
  constexpr uint32_t kq = Quad<T>::n;
  return reinterpret_cast<uintptr_t>(base) % 16 == 0 && width % kq == 0 && ts % kq == 0;
}

// Destination of row value c: ptr[c][g * stride[c]].
template <typename T, int NV>
struct RowTargets {
  T *ptr[NV];
  int stride[NV];
};

// One wave per 64 consecutive rows (emission order).  Each Gaussian is
// written by the wave holding its first row: a Gaussian continuing past the
// wave's last lane has its remaining rows gathered by this wave (64 ids at a
// time); a Gaussian that started in an earlier wave is skipped.  Plain
// stores, no atomics: outputs must be zero on entry, and the per-Gaussian
// summation order is fixed.
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
  const int32_t before = (eb > 0) ? emit_ids[eb - 1] : -1;
  const int32_t seg_first = __shfl(seg, 0, 64);
  const int32_t seg_last = __shfl(seg, 63, 64);
  // First lane of each segment, unless the segment began in an earlier wave.
  const bool head = seg >= 0 && (lane == 0 ? before != seg : seg_prev != seg);
  T v[NV];
  load_row(rows, in ? e : 0, v);
  if (!in) {
#pragma unroll
    for (int c = 0; c < NV; ++c) v[c] = 0;
  }
#pragma unroll
  for (int c = 0; c < NV; ++c) v[c] = segs.suffix_sum(v[c]);
  // Rows of the last segment beyond this wave (uniform branch and loop).
  const bool tail_owned = seg_last >= 0 && !(seg_first == seg_last && before == seg_last);
  if (tail_owned && eb + 64 < n && emit_ids[eb + 64] == seg_last) {
    T t[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) t[c] = 0;
    for (int64_t base = eb + 64; base < n; base += 64) {
      const int64_t e2 = base + lane;
      const bool take = e2 < n && emit_ids[e2] == seg_last;
      if (take) {
        T w[NV];
        load_row(rows, e2, w);
#pragma unroll
        for (int c = 0; c < NV; ++c) t[c] += w[c];
      }
      if (!(base + 63 < n && __shfl(static_cast<int>(take), 63, 64))) break;
    }
#pragma unroll
    for (int c = 0; c < NV; ++c) t[c] = wave_sum(t[c]);
    if (seg == seg_last) {
#pragma unroll
      for (int c = 0; c < NV; ++c) v[c] += t[c];
    }
  }
  if (!head) return;
#pragma unroll
  for (int c = 0; c < NV; ++c) tg.ptr[c][g * tg.stride[c]] = v[c];
}

template <typename T, int NV>
void launch_row_reduce(const T *rows, const int32_t *emit_ids, int64_t n, int64_t n_items,
                       const RowTargets<T, NV> &tg, hipStream_t stream) {
  row_reduce_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n, 256))), dim3(256), 0,
                             stream>>>(rows, emit_ids, n, n_items, tg);
}

}  // namespace r2s
