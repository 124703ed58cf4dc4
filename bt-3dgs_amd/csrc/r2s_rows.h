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

// Zeroes ids [lo, hi) of every target: each lane its first kOwnZeros ids
// itself (gaps are mostly short), the rest of long ranges one lane's range
// after another, all 64 lanes storing consecutive ids.
constexpr int kOwnZeros = 8;

template <typename T, int NV>
__device__ __forceinline__ void zero_id_ranges(int64_t lo, int64_t hi, const RowTargets<T, NV> &tg) {
  const int64_t own = min(hi, lo + kOwnZeros);
  for (int64_t k = lo; k < own; ++k) {
#pragma unroll
    for (int c = 0; c < NV; ++c) tg.ptr[c][k * tg.stride[c]] = static_cast<T>(0);
  }
  lo = own > lo ? own : lo;
  uint64_t pending = ballot(hi > lo);
  while (pending != 0) {
    const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(pending));
    pending &= pending - 1;
    const int64_t a = readlane_i64(lo, src), b = readlane_i64(hi, src);
    for (int64_t k = a + lane_id(); k < b; k += 64) {
#pragma unroll
      for (int c = 0; c < NV; ++c) tg.ptr[c][k * tg.stride[c]] = static_cast<T>(0);
    }
  }
}

// Rounds of 64 rows per wave: the rows of all rounds are loaded up front,
// and a Gaussian crossing from one round into the next carries its sum in
// registers; only one crossing the wave's last row gathers rows of the next
// wave.
constexpr int kReduceRounds = 4;
constexpr int kReduceWaveRows = 64 * kReduceRounds;

// One wave per kReduceWaveRows consecutive rows (emission order).  Each
// Gaussian is written by the wave holding its first row: a Gaussian
// continuing past the wave's last row has its remaining rows gathered by
// this wave (64 ids at a time); a Gaussian that started in an earlier wave
// is skipped.  Plain stores, no atomics, and the per-Gaussian summation
// order is fixed.  Emission order is ascending in the id, so the ids
// strictly between two consecutive records' ids have no records: the first
// row of each Gaussian zeroes the ids between it and the previous record,
// and the wave holding the last record zeroes the ids after it.  Every
// output is written; none needs zeroing beforehand.
template <typename T, int NV>
__global__ __launch_bounds__(256) void row_reduce_kernel(const T *__restrict__ rows,
                                                         const int32_t *__restrict__ emit_ids,
                                                         int64_t n, int64_t n_items,
                                                         RowTargets<T, NV> tg) {
  constexpr int R = kReduceRounds;
  const int64_t eb = (static_cast<int64_t>(blockIdx.x) * 4 + wave_index()) * kReduceWaveRows;
  if (eb >= n) return;  // uniform per wave
  const uint32_t lane = lane_id();
  // Segment id per row: the Gaussian, or a negative value unique to the row
  // slot for rows past the end (or with an id out of range).
  int32_t seg[R];
  T v[R][NV];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t e = eb + r * 64 + lane;
    const bool in = e < n;
    const int64_t g = in ? static_cast<int64_t>(emit_ids[e]) : -1;
    seg[r] = (g >= 0 && g < n_items) ? static_cast<int32_t>(g)
                                     : -1 - static_cast<int32_t>(r * 64 + lane);
    load_row(rows, in ? e : 0, v[r]);
    if (!in) {
#pragma unroll
      for (int c = 0; c < NV; ++c) v[r][c] = 0;
    }
  }
  const int32_t before = (eb > 0) ? emit_ids[eb - 1] : -1;
  const int32_t seg_first = __shfl(seg[0], 0, 64);
  const int32_t seg_last = __shfl(seg[R - 1], 63, 64);
  // Rows of the last segment beyond this wave (uniform branch and loop).
  T carry[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) carry[c] = 0;
  int32_t carry_seg = -1 - kReduceWaveRows;  // matches no row slot
  const bool tail_owned = seg_last >= 0 && !(seg_first == seg_last && before == seg_last);
  const int64_t past = eb + kReduceWaveRows;
  if (tail_owned && past < n && emit_ids[past] == seg_last) {
    for (int64_t base = past; base < n; base += 64) {
      const int64_t e2 = base + lane;
      const bool take = e2 < n && emit_ids[e2] == seg_last;
      if (take) {
        T w[NV];
        load_row(rows, e2, w);
#pragma unroll
        for (int c = 0; c < NV; ++c) carry[c] += w[c];
      }
      if (!(base + 63 < n && __shfl(static_cast<int>(take), 63, 64))) break;
    }
#pragma unroll
    for (int c = 0; c < NV; ++c) carry[c] = wave_sum(carry[c]);
    carry_seg = seg_last;
  }
  // Rounds last to first: each round's suffix sums plus the carry of the
  // segment continuing into the next round; the sum at lane 0 carries on.
  const bool last_wave = past >= n;
#pragma unroll
  for (int r = R - 1; r >= 0; --r) {
    const WaveSegments segs(seg[r]);
    T x[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      x[c] = segs.suffix_sum(v[r][c]);
      if (seg[r] == carry_seg) x[c] += carry[c];
    }
    const int32_t seg_prev = __shfl_up(seg[r], 1, 64);
    const int32_t prev_last = r > 0 ? __shfl(seg[r > 0 ? r - 1 : 0], 63, 64) : before;
    const int32_t p = lane == 0 ? prev_last : seg_prev;
    // First row of each Gaussian, unless it began in an earlier wave.
    const bool head = seg[r] >= 0 && p != seg[r];
#pragma unroll
    for (int c = 0; c < NV; ++c) carry[c] = __shfl(x[c], 0, 64);
    carry_seg = __shfl(seg[r], 0, 64);
    // Ids without records before this Gaussian's id.
    int64_t z_lo = 0, z_hi = 0;
    if (head) {
      z_lo = static_cast<int64_t>(p) + 1;
      z_hi = seg[r];
    }
    zero_id_ranges(z_lo, z_hi, tg);
    if (head) {
      const int64_t g = seg[r];
#pragma unroll
      for (int c = 0; c < NV; ++c) tg.ptr[c][g * tg.stride[c]] = x[c];
    }
  }
  if (last_wave) {  // uniform: this wave holds the last record
    const int64_t last = emit_ids[n - 1];
    const bool take = lane == 0 && last >= 0 && last < n_items;
    zero_id_ranges<T, NV>(take ? last + 1 : 0, take ? n_items : 0, tg);
  }
}

template <typename T, int NV>
void launch_row_reduce(const T *rows, const int32_t *emit_ids, int64_t n, int64_t n_items,
                       const RowTargets<T, NV> &tg, hipStream_t stream) {
  row_reduce_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n, 4 * kReduceWaveRows))),
                             dim3(256), 0, stream>>>(rows, emit_ids, n, n_items, tg);
}

}  // namespace r2s
