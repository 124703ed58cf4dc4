// Per-record partial rows and their per-Gaussian reduction.
//
// The backward kernels walk records in tile order, where every record of a
// Gaussian lands in a different tile.  Adding each record's partials to the
// Gaussian's gradient with device-scope float atomics runs at about 21 G
// atomics/s on MI355X (measured for scattered fp32 adds), which dominates the
// backward passes.  Instead a kernel stores each record's partials as one
// row of a workspace at the record's emission index; in emission
// order the records of one Gaussian are consecutive, so a streaming pass sums
// each Gaussian's rows with a segmented wave reduction and writes the sums
// once with plain stores.  The result does not depend on scheduling.
#pragma once

#include "r2s_common.h"

namespace r2s {

// Slots per row: a row of up to 8 values takes 8 (32 bytes in float, one
// 32-byte sector, so a row written at a scattered index costs one sector), a
// longer one its value count rounded up to even (the voxelizer's 10 values:
// 40 bytes in float, five 8-byte vectors).  Rows are written at scattered
// indices, and fewer bytes per row beat sector-aligned rows there: measured
// on the voxelizer's rows pass, 48-byte rows were 4 % slower than 40-byte
// ones and 64-byte rows 9 %.  The rasterizer stores 8 values (6 without
// absolute gradients).
template <int NV>
constexpr int row_stride() {
  return NV <= 8 ? 8 : (NV + 1) / 2 * 2;
}

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

template <typename T>
struct Pair;
template <>
struct Pair<float> {
  using type = float2;  // 8 bytes
  static constexpr int n = 2;
};
template <>
struct Pair<double> {
  using type = double;  // 8 bytes
  static constexpr int n = 1;
};

// Rows start at multiples of the row size from a 16-byte-aligned workspace,
// so they are written and read as 16-byte vectors when the row size is a
// multiple of 16 bytes, else as 8-byte vectors (an even slot count makes
// every row size a multiple of 8 bytes).
template <typename T, int NV>
struct RowVec {
  static constexpr bool kWide = (row_stride<NV>() * sizeof(T)) % 16 == 0;
  using type = typename std::conditional<kWide, typename Quad<T>::type,
                                         typename Pair<T>::type>::type;
  static constexpr int n = kWide ? Quad<T>::n : Pair<T>::n;
};

template <typename T, int NV>
__device__ __forceinline__ void store_row(T *__restrict__ rows, int64_t e, const T (&v)[NV]) {
  static_assert(NV <= 12, "row too long");
  using Q = typename RowVec<T, NV>::type;
  constexpr int kq = RowVec<T, NV>::n, nq = (NV + kq - 1) / kq;
  T pad[nq * kq];
#pragma unroll
  for (int c = 0; c < nq * kq; ++c) pad[c] = c < NV ? v[c] : static_cast<T>(0);
  Q *dst = reinterpret_cast<Q *>(rows + e * row_stride<NV>());
#pragma unroll
  for (int q = 0; q < nq; ++q) dst[q] = *reinterpret_cast<const Q *>(pad + q * kq);
}

template <typename T, int NV>
__device__ __forceinline__ void load_row(const T *__restrict__ rows, int64_t e, T (&v)[NV]) {
  using Q = typename RowVec<T, NV>::type;
  constexpr int kq = RowVec<T, NV>::n, nq = (NV + kq - 1) / kq;
  T pad[nq * kq];
  const Q *src = reinterpret_cast<const Q *>(rows + e * row_stride<NV>());
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

// Destinations of row value c for Gaussian g: ptr[c][g * stride[c]], times
// scale[c][g] when scale[c] is set; and, when ptr2[c] is set, also
// ptr2[c][g] = value * scale2[c][g] (one sum feeding two gradients, as the
// rasterizer's opacity and mu partials do).
template <typename T, int NV>
struct RowTargets {
  T *ptr[NV];
  int stride[NV];
  const T *scale[NV];
  T *ptr2[NV];
  const T *scale2[NV];
};

// Every output array of a RowTargets as (pointer, stride) entries: the
// ptr[c] columns, then the ptr2[c] columns (stride 1).
template <typename T, int NV>
struct TargetList {
  T *ptr[2 * NV];
  int stride[2 * NV];
  int n;
};

template <typename T, int NV>
inline TargetList<T, NV> target_list(const RowTargets<T, NV> &tg) {
  TargetList<T, NV> tl{};
  for (int c = 0; c < NV; ++c) {
    tl.ptr[tl.n] = tg.ptr[c];
    tl.stride[tl.n++] = tg.stride[c];
  }
  for (int c = 0; c < NV; ++c)
    if (tg.ptr2[c] != nullptr) {
      tl.ptr[tl.n] = tg.ptr2[c];
      tl.stride[tl.n++] = 1;
    }
  return tl;
}

// Zeroes every target over ids [0, n_items): blockIdx.y is the entry.
template <typename T, int NV>
__global__ __launch_bounds__(256) void zero_targets_kernel(TargetList<T, NV> tl, int64_t n_items) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (k < n_items) tl.ptr[blockIdx.y][k * tl.stride[blockIdx.y]] = static_cast<T>(0);
}

// The arrays under a target list: each is covered by `stride` entries at
// base, base + 1, ..., so zeroing the arrays contiguously zeroes every
// target.  Zeroing them with 16-byte stores instead of one strided 4-byte
// store per target halves the fill's time.
template <typename T, int NV>
struct FillArrays {
  T *ptr[2 * NV];
  int64_t len[2 * NV];
};

template <typename T, int NV>
__global__ __launch_bounds__(256) void fill_arrays_kernel(FillArrays<T, NV> fa) {
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n;
  T *p = fa.ptr[blockIdx.y];
  const int64_t len = fa.len[blockIdx.y];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nq = len / kq;
  if (i < nq) {
    Q z;
    T *zp = reinterpret_cast<T *>(&z);
#pragma unroll
    for (int c = 0; c < kq; ++c) zp[c] = static_cast<T>(0);
    reinterpret_cast<Q *>(p)[i] = z;
  } else if (i < nq + (len - nq * kq)) {
    p[nq * kq + (i - nq)] = static_cast<T>(0);
  }
}

// Splits a target list into its arrays: an entry starts an array unless an
// entry of the same stride sits one element before it.  False when an array
// is not 16-byte aligned (then the strided zeroing is used).
template <typename T, int NV>
inline bool target_arrays(const TargetList<T, NV> &tl, int64_t n_items, FillArrays<T, NV> &fa,
                          int &n_arrays) {
  n_arrays = 0;
  for (int c = 0; c < tl.n; ++c) {
    bool start = true;
    for (int d = 0; d < tl.n; ++d)
      if (tl.stride[d] == tl.stride[c] && tl.ptr[d] + 1 == tl.ptr[c]) start = false;
    if (!start) continue;
    if (reinterpret_cast<uintptr_t>(tl.ptr[c]) % 16 != 0) return false;
    fa.ptr[n_arrays] = tl.ptr[c];
    fa.len[n_arrays] = static_cast<int64_t>(tl.stride[c]) * n_items;
    ++n_arrays;
  }
  return true;
}

// Rows per wave of the reduction: 64 lanes x 4 consecutive rows.
constexpr int kReduceRowsPerLane = 4;
constexpr int kReduceWaveRows = 64 * kReduceRowsPerLane;

// The transpose goes through LDS in two phases of 128 rows (load rounds 0-1
// to lanes 0-31, then rounds 2-3 to lanes 32-63), which halves the staging
// buffer: the kernel waits on memory, and the smaller buffer lets twice as
// many waves be resident.  LDS slot of phase-row q (0..127): lane l of the
// half reads rows 4l .. 4l+3 from slots k*32 + ((l + 8k) mod 32), and lane l
// of load round r writes row 64r + l; with the rotation by 8k both the
// writes and the reads of each half-wave hit 32 different banks.
constexpr int kReduceStage = kReduceWaveRows / 2;
__device__ __forceinline__ uint32_t reduce_slot(uint32_t q) {
  return (q & 3u) * 32u + (((q >> 2) + 8u * (q & 3u)) & 31u);
}

// One wave per kReduceWaveRows consecutive rows (emission order), read with
// coalesced loads and transposed through LDS so that each lane holds four
// consecutive rows.  A lane sums the runs of equal ids among its rows in
// registers; one segmented suffix sum over the lanes (keyed by the id of
// each lane's first row) then completes the runs that cross lanes.  Each
// Gaussian is written by the wave holding its first row: a Gaussian
// continuing past the wave's last row has its remaining rows gathered by
// this wave (64 ids at a time); a Gaussian that started in an earlier wave
// is skipped.  Plain stores, no atomics, and the per-Gaussian summation
// order is fixed.  launch_row_reduce zeroes the targets first, so ids
// without records (more than half of them at a heavily culled view) read
// zero.
template <typename T, int NV>
__global__ __launch_bounds__(256) void row_reduce_kernel(const T *__restrict__ rows,
                                                         const int32_t *__restrict__ emit_ids,
                                                         int64_t n, int64_t n_items,
                                                         RowTargets<T, NV> tg) {
  constexpr int K = kReduceRowsPerLane;
  __shared__ T s_val[4][NV][kReduceStage];
  __shared__ int32_t s_seg[4][kReduceStage];
  const uint32_t w = wave_index(), lane = lane_id();
  const int64_t eb = (static_cast<int64_t>(blockIdx.x) * 4 + w) * kReduceWaveRows;
  if (eb >= n) return;  // uniform per wave; the waves share no barrier below
  // Segment id per row: the Gaussian, or a negative value unique to the row
  // slot for rows past the end (or with an id out of range).
  int32_t sr[K];
  T vr[K][NV];
  // The id just before the wave's rows, and the first 64 rows after them
  // with their ids (the last Gaussian nearly always continues there, and
  // the tail gather below starts from them), loaded with the wave's rows:
  // each would otherwise be one more memory round trip of the wave.
  const int64_t past = eb + kReduceWaveRows;
  const int32_t before = (eb > 0) ? emit_ids[eb - 1] : -1;
  const int64_t t_e = past + lane;
  const int32_t t_id = t_e < n ? emit_ids[t_e] : -1;
  T t_row[NV];
  load_row(rows, t_e < n ? t_e : eb, t_row);
#pragma unroll
  for (int r = 0; r < K; ++r) {
    const uint32_t q = 64u * r + lane;
    const int64_t e = eb + q;
    const bool in = e < n;
    const int64_t g = in ? static_cast<int64_t>(emit_ids[e]) : -1;
    sr[r] = (g >= 0 && g < n_items) ? static_cast<int32_t>(g) : -1 - static_cast<int32_t>(q);
    load_row(rows, in ? e : 0, vr[r]);
    if (!in) {
#pragma unroll
      for (int c = 0; c < NV; ++c) vr[r][c] = 0;
    }
  }
  int32_t g[K];
  T v[K][NV];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t slot = reduce_slot(64u * r + lane);
      s_seg[w][slot] = sr[2 * h + r];
#pragma unroll
      for (int c = 0; c < NV; ++c) s_val[w][c][slot] = vr[2 * h + r][c];
    }
    // The wave's LDS operations complete in order, so its own lanes' writes
    // are visible to the reads below (and the reads precede the next
    // phase's writes); keep the compiler from moving them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if ((lane >> 5) == static_cast<uint32_t>(h)) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const uint32_t slot = reduce_slot(K * (lane & 31u) + k);
        g[k] = s_seg[w][slot];
#pragma unroll
        for (int c = 0; c < NV; ++c) v[k][c] = s_val[w][c][slot];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const int32_t seg_first = __shfl(g[0], 0, 64);
  const int32_t seg_last = __shfl(g[K - 1], 63, 64);
  // In-lane run sums, last row first: acc[k] = rows k .. the end of k's run
  // among the lane's rows.
  T acc[K][NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) acc[K - 1][c] = v[K - 1][c];
#pragma unroll
  for (int k = K - 2; k >= 0; --k) {
    const bool same = g[k + 1] == g[k];
#pragma unroll
    for (int c = 0; c < NV; ++c) acc[k][c] = v[k][c] + (same ? acc[k + 1][c] : static_cast<T>(0));
  }
  // Rows of the last segment beyond this wave (uniform branch and loop),
  // added to that segment's runs in lane 63.
  const bool tail_owned = seg_last >= 0 && !(seg_first == seg_last && before == seg_last);
  const int32_t after = __shfl(t_id, 0, 64);
  if (tail_owned && past < n && after == seg_last) {
    T carry[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) carry[c] = 0;
    // The prefetched 64 rows, then K x 64 rows a round with their ids loaded
    // together, so a long tail (a Gaussian over hundreds of tiles) takes a
    // K-th of the memory round trips.  Each lane adds its rows in increasing
    // order either way.
    const bool take0 = t_e < n && t_id == seg_last;
    if (take0) {
#pragma unroll
      for (int c = 0; c < NV; ++c) carry[c] += t_row[c];
    }
    bool more = past + 63 < n && __shfl(static_cast<int>(take0), 63, 64);
    for (int64_t base = past + 64; more && base < n; base += kReduceWaveRows) {  // uniform
      int32_t id2[K];
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int64_t e2 = base + 64 * r + lane;
        id2[r] = e2 < n ? emit_ids[e2] : -1;
      }
      bool take = false;
#pragma unroll
      for (int r = 0; r < K; ++r) {
        const int64_t e2 = base + 64 * r + lane;
        take = e2 < n && id2[r] == seg_last;
        if (take) {
          T wv[NV];
          load_row(rows, e2, wv);
#pragma unroll
          for (int c = 0; c < NV; ++c) carry[c] += wv[c];
        }
      }
      more = base + kReduceWaveRows - 1 < n && __shfl(static_cast<int>(take), 63, 64);
    }
#pragma unroll
    for (int c = 0; c < NV; ++c) carry[c] = wave_sum(carry[c]);
    if (lane == 63) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (g[k] == seg_last) {
#pragma unroll
          for (int c = 0; c < NV; ++c) acc[k][c] += carry[c];
        }
      }
    }
  }
  // Runs crossing lanes: the suffix sums of each lane's first run over the
  // following lanes with the same first id (a lane whose first run does not
  // fill it ends the segment there, as ids ascend).
  const WaveSegments segs(g[0]);
  T lead[NV], next[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    lead[c] = segs.suffix_sum(acc[0][c]);
    next[c] = __shfl_down(lead[c], 1, 64);
  }
  // Shuffles with every lane active (a source lane must take part).
  const int32_t next_first_all = __shfl_down(g[0], 1, 64);
  const int32_t next_first = lane < 63 ? next_first_all : -1;
  const int32_t prev_last = __shfl_up(g[K - 1], 1, 64);
  bool head[K];
  uint32_t n_heads = 0;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int32_t p = k > 0 ? g[k - 1] : (lane == 0 ? before : prev_last);
    head[k] = g[k] >= 0 && p != g[k];
    n_heads += head[k] ? 1u : 0u;
    // The Gaussian's total (kept in acc[k]): its run in this lane, and, when
    // that run reaches the lane's end, the following lanes' share.
    const bool onward = g[K - 1] == g[k] && next_first == g[k];
#pragma unroll
    for (int c = 0; c < NV; ++c)
      acc[k][c] = k == 0 ? lead[c] : acc[k][c] + (onward ? next[c] : static_cast<T>(0));
  }
  // Stored in place, the heads (scattered over the lanes and their four rows)
  // would take 4 NV store instructions with a few active lanes each.  The
  // wave numbers its heads in row order (= Gaussian order), stages each
  // head's id and totals in the transpose buffers (free now), and stores
  // them with consecutive heads on consecutive lanes, kReduceStage heads a
  // round (one round unless the wave's 256 rows hold more Gaussians).
  const uint32_t incl = wave_inclusive_scan(n_heads);
  const uint32_t h_total = readlane_u32(incl, 63);
#pragma unroll 1
  for (uint32_t r0 = 0; r0 < h_total; r0 += kReduceStage) {  // uniform
    uint32_t h = incl - n_heads;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (head[k] && h >= r0 && h < r0 + kReduceStage) {
        const uint32_t slot = h - r0;
        s_seg[w][slot] = g[k];
#pragma unroll
        for (int c = 0; c < NV; ++c) s_val[w][c][slot] = acc[k][c];
      }
      h += head[k] ? 1u : 0u;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t cnt = min(h_total - r0, static_cast<uint32_t>(kReduceStage));
    for (uint32_t q = lane; q < cnt; q += 64) {
      const int64_t gi = s_seg[w][q];
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const T v = s_val[w][c][q];
        tg.ptr[c][gi * tg.stride[c]] = tg.scale[c] != nullptr ? v * tg.scale[c][gi] : v;
        if (tg.ptr2[c] != nullptr) tg.ptr2[c][gi] = v * tg.scale2[c][gi];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Stores every target: zeros (unless the caller stored them already:
// zeroed), then each Gaussian's sum over its rows.
template <typename T, int NV>
void launch_row_reduce(const T *rows, const int32_t *emit_ids, int64_t n, int64_t n_items,
                       const RowTargets<T, NV> &tg, hipStream_t stream, bool zeroed = false) {
  if (n_items <= 0) return;
  if (zeroed) {
    if (n > 0)
      row_reduce_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n, 4 * kReduceWaveRows))),
                                 dim3(256), 0, stream>>>(rows, emit_ids, n, n_items, tg);
    return;
  }
  const TargetList<T, NV> tl = target_list(tg);
  FillArrays<T, NV> fa;
  int n_arrays = 0;
  if (target_arrays(tl, n_items, fa, n_arrays)) {
    int64_t longest = 0;
    for (int a = 0; a < n_arrays; ++a) longest = fa.len[a] > longest ? fa.len[a] : longest;
    const int64_t threads = ceil_div(longest, Quad<T>::n) + Quad<T>::n;
    fill_arrays_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(threads, 256)),
                                     static_cast<uint32_t>(n_arrays)),
                                dim3(256), 0, stream>>>(fa);
  } else {
    zero_targets_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n_items, 256)),
                                      static_cast<uint32_t>(tl.n)),
                                 dim3(256), 0, stream>>>(tl, n_items);
  }
  if (n <= 0) return;
  row_reduce_kernel<T, NV><<<dim3(static_cast<uint32_t>(ceil_div(n, 4 * kReduceWaveRows))),
                             dim3(256), 0, stream>>>(rows, emit_ids, n, n_items, tg);
}

}  // namespace r2s
