// Tile binning: which Gaussians touch which 2D tile / 3D brick, as a list
// sorted by (tile key, record id) plus per-tile lower-bound offsets.
//
//   count   one thread per record: the clamped tile rectangle/box and its
//           area (r2splat/cuda/csrc/IsectTilesKernel.cu:57-113,
//           IsectTiles3DKernel.cu:49-104), then an int64 exclusive scan.
//   emit    wave-cooperative: the 64 records of a wave are expanded one after
//           another by all 64 lanes, so a Gaussian covering thousands of
//           tiles costs ceil(tiles/64) coalesced store rounds instead of a
//           serial per-thread loop.  Emission order is the reference's
//           (record id, then rows / z-y-x), keys are 32-bit.
//   sort    stable LSD radix sort on bits [0, end_bit), 8-bit digits.  Per
//           pass: LDS digit histogram per 4096-item tile, device scan of the
//           digit-major histogram table, stable scatter with per-wave ranks
//           from ballot-based digit matching (no per-item atomics).  The last
//           pass widens keys to int64 on the way out.
//   offsets lower_bound of every key in the sorted list (binary search).
//
// Because emission is in ascending record id and every pass is stable, the
// output is the lexicographic (key, id) order -- identical to the
// reference's CUB sort of the same records.
#pragma clang fp contract(off)

#include <utility>

#include "r2s_common.h"
#include "r2s_scan.h"

namespace r2s {
namespace {

// ------------------------------------------------------------ geometry ---

// IsectTilesKernel.cu:30-40: non-finite or <= 0 -> 0, >= upper -> upper.
template <typename T>
__device__ __forceinline__ uint32_t clamp_tile_bound(T v, uint32_t upper) {
  if (!isfinite(v) || v <= static_cast<T>(0)) return 0u;
  if (v >= static_cast<T>(upper)) return upper;
  return static_cast<uint32_t>(v);
}

// Saturating float -> uint32 (the CUDA conversion used by the 3D bounds).
template <typename T>
__device__ __forceinline__ uint32_t sat_u32(T v) {
  if (!(v > static_cast<T>(0))) return 0u;  // NaN and non-positive
  if (v >= static_cast<T>(4294967295.0)) return 0xffffffffu;
  return static_cast<uint32_t>(v);
}

struct Rect {
  uint32_t x0, x1, y0, y1;
};

// Tile rectangle [x0,x1) x [y0,y1) and its area (0 = emits nothing).
template <typename T>
__device__ __forceinline__ uint32_t rect_2d(const T *__restrict__ means2d,
                                            const int32_t *__restrict__ radii, int rect,
                                            int64_t idx, uint32_t ts, uint32_t tw, uint32_t th,
                                            Rect &r) {
  r = {0, 0, 0, 0};
  const T rx = static_cast<T>(rect ? radii[2 * idx] : radii[idx]);
  const T ry = static_cast<T>(rect ? radii[2 * idx + 1] : radii[idx]);
  if (rx <= static_cast<T>(0) || ry <= static_cast<T>(0)) return 0;
  const T mx = means2d[2 * idx], my = means2d[2 * idx + 1];
  if (!isfinite(mx) || !isfinite(my)) return 0;
  const T tsf = static_cast<T>(ts);
  const T trx = rx / tsf, tyr = ry / tsf, tx = mx / tsf, ty = my / tsf;
  r.x0 = clamp_tile_bound(floor(tx - trx), tw);
  r.y0 = clamp_tile_bound(floor(ty - tyr), th);
  r.x1 = clamp_tile_bound(ceil(tx + trx), tw);
  r.y1 = clamp_tile_bound(ceil(ty + tyr), th);
  if (r.x1 <= r.x0 || r.y1 <= r.y0) return 0;
  return (r.y1 - r.y0) * (r.x1 - r.x0);
}

struct Box {
  uint32_t lo[3], hi[3];  // (dim2, dim1, dim0)
};

template <typename T>
__device__ __forceinline__ uint32_t box_3d(const T *__restrict__ means3d,
                                           const int32_t *__restrict__ radii, int64_t idx,
                                           uint32_t ts, const uint32_t n[3], Box &b) {
#pragma unroll
  for (int a = 0; a < 3; ++a) b.lo[a] = b.hi[a] = 0;
  const T r0 = static_cast<T>(radii[3 * idx]), r1 = static_cast<T>(radii[3 * idx + 1]),
          r2 = static_cast<T>(radii[3 * idx + 2]);
  if (r0 <= static_cast<T>(0) || r1 <= static_cast<T>(0) || r2 <= static_cast<T>(0)) return 0;
  const T tsf = static_cast<T>(ts);
  const T rr[3] = {r0, r1, r2};
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const T c = means3d[3 * idx + a] / tsf;
    const T rt = rr[a] / tsf;
    b.lo[a] = min(sat_u32(floor(c - rt)), n[a]);
    b.hi[a] = min(sat_u32(ceil(c + rt)), n[a]);
  }
  return (b.hi[2] - b.lo[2]) * (b.hi[1] - b.lo[1]) * (b.hi[0] - b.lo[0]);
}

// --------------------------------------------------------------- count ---

template <typename T>
__global__ __launch_bounds__(256) void count_2d_kernel(const T *__restrict__ means2d,
                                                       const int32_t *__restrict__ radii,
                                                       int rect, int64_t M, uint32_t ts,
                                                       uint32_t tw, uint32_t th,
                                                       int32_t *__restrict__ counts) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= M) return;
  Rect r;
  counts[idx] = static_cast<int32_t>(rect_2d(means2d, radii, rect, idx, ts, tw, th, r));
}

template <typename T>
__global__ __launch_bounds__(256) void count_3d_kernel(const T *__restrict__ means3d,
                                                       const int32_t *__restrict__ radii,
                                                       int64_t N, uint32_t ts, uint32_t n2,
                                                       uint32_t n1, uint32_t n0,
                                                       int32_t *__restrict__ counts) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= N) return;
  const uint32_t n[3] = {n2, n1, n0};
  Box b;
  counts[idx] = static_cast<int32_t>(box_3d(means3d, radii, idx, ts, n, b));
}

// ---------------------------------------------------------------- emit ---

// Lane (of the calling wave) owning output t of a wave whose lanes emit
// excl[j] .. excl[j] + cnt[j] - 1: the largest j with excl[j] <= t (a lane
// with cnt > 0, as zero-count lanes share the excl of the next lane).
__device__ __forceinline__ uint32_t owner_lane(uint32_t excl, uint32_t t) {
  uint32_t lo = 0;
#pragma unroll
  for (uint32_t step = 32; step > 0; step >>= 1) {
    const uint32_t cand = lo + step;
    const uint32_t e = static_cast<uint32_t>(__shfl(static_cast<int>(excl), static_cast<int>(cand & 63u), 64));
    if (cand < 64u && e <= t) lo = cand;
  }
  return lo;
}

// Writes one record: key, payload(s) and, for the emission-order arrays,
// the flat id.
__device__ __forceinline__ void put_record(uint32_t *__restrict__ keys, uint32_t *__restrict__ vals,
                                           uint32_t *__restrict__ vals2,
                                           int32_t *__restrict__ emit_ids, int64_t e,
                                           uint32_t key, uint32_t gid) {
  keys[e] = key;
  if (emit_ids != nullptr) {
    vals[e] = static_cast<uint32_t>(e);
    vals2[e] = gid;
    emit_ids[e] = static_cast<int32_t>(gid);
  } else {
    vals[e] = gid;
  }
}

// A wave's 64 consecutive items emit one contiguous range of records
// (offsets is the exclusive scan of the counts); the range is spread over
// the lanes 64 records at a time, so every store instruction writes 64
// consecutive records.  Tiles of one item are row-major in its rectangle.
template <typename T>
__global__ __launch_bounds__(256) void emit_2d_kernel(
    const T *__restrict__ means2d, const int32_t *__restrict__ radii, int rect, int64_t M,
    int64_t N, uint32_t ts, uint32_t tw, uint32_t th, const int64_t *__restrict__ offsets,
    uint32_t *__restrict__ keys, uint32_t *__restrict__ vals, uint32_t *__restrict__ vals2,
    int32_t *__restrict__ emit_ids) {
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * 256 + 64 * wave_index();
  if (wave_first >= M) return;  // uniform per wave
  const int64_t idx = wave_first + lane_id();
  Rect r = {0, 0, 0, 0};
  uint32_t cnt = 0;
  if (idx < M) cnt = rect_2d(means2d, radii, rect, idx, ts, tw, th, r);
  const uint32_t incl = wave_inclusive_scan(cnt);
  const uint32_t excl = incl - cnt;
  const uint32_t total = readlane_u32(incl, 63);
  const int64_t base = offsets[wave_first];
  const uint32_t width = r.x1 - r.x0;
  const uint32_t n_tiles = tw * th;
  // Uniform loop: every lane takes part in the shuffles (a lane past the end
  // works on the last record and stores nothing).
  for (uint32_t t0 = 0; t0 < total; t0 += 64) {
    const uint32_t t = min(t0 + lane_id(), total - 1);
    const uint32_t j = owner_lane(excl, t);
    const int jj = static_cast<int>(j);
    const uint32_t k = t - static_cast<uint32_t>(__shfl(static_cast<int>(excl), jj, 64));
    const uint32_t wj = static_cast<uint32_t>(__shfl(static_cast<int>(width), jj, 64));
    const uint32_t x0 = static_cast<uint32_t>(__shfl(static_cast<int>(r.x0), jj, 64));
    const uint32_t y0 = static_cast<uint32_t>(__shfl(static_cast<int>(r.y0), jj, 64));
    const uint32_t row = k / wj, col = k - row * wj;
    const int64_t gid = wave_first + j;
    const uint32_t key = static_cast<uint32_t>(gid / N) * n_tiles + (y0 + row) * tw + (x0 + col);
    if (t0 + lane_id() < total)
      put_record(keys, vals, vals2, emit_ids, base + t, key, static_cast<uint32_t>(gid));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void emit_3d_kernel(
    const T *__restrict__ means3d, const int32_t *__restrict__ radii, int64_t N, uint32_t ts,
    uint32_t n2, uint32_t n1, uint32_t n0, const int64_t *__restrict__ offsets,
    uint32_t *__restrict__ keys, uint32_t *__restrict__ vals, uint32_t *__restrict__ vals2,
    int32_t *__restrict__ emit_ids) {
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * 256 + 64 * wave_index();
  if (wave_first >= N) return;  // uniform per wave
  const int64_t idx = wave_first + lane_id();
  const uint32_t n[3] = {n2, n1, n0};
  Box b;
  uint32_t cnt = 0;
  if (idx < N) {
    cnt = box_3d(means3d, radii, idx, ts, n, b);
  } else {
#pragma unroll
    for (int a = 0; a < 3; ++a) b.lo[a] = b.hi[a] = 0;
  }
  const uint32_t incl = wave_inclusive_scan(cnt);
  const uint32_t excl = incl - cnt;
  const uint32_t total = readlane_u32(incl, 63);
  const int64_t base = offsets[wave_first];
  const uint32_t e2 = b.hi[0] - b.lo[0], e1 = b.hi[1] - b.lo[1];
  // Uniform loop: every lane takes part in the shuffles (a lane past the end
  // works on the last record and stores nothing).
  for (uint32_t t0 = 0; t0 < total; t0 += 64) {
    const uint32_t t = min(t0 + lane_id(), total - 1);
    const uint32_t j = owner_lane(excl, t);
    const int jj = static_cast<int>(j);
    const uint32_t k = t - static_cast<uint32_t>(__shfl(static_cast<int>(excl), jj, 64));
    const uint32_t e2j = static_cast<uint32_t>(__shfl(static_cast<int>(e2), jj, 64));
    const uint32_t e1j = static_cast<uint32_t>(__shfl(static_cast<int>(e1), jj, 64));
    const uint32_t l2 = static_cast<uint32_t>(__shfl(static_cast<int>(b.lo[0]), jj, 64));
    const uint32_t l1 = static_cast<uint32_t>(__shfl(static_cast<int>(b.lo[1]), jj, 64));
    const uint32_t l0 = static_cast<uint32_t>(__shfl(static_cast<int>(b.lo[2]), jj, 64));
    const uint32_t plane = e2j * e1j;
    const uint32_t tz = k / plane, rem = k - tz * plane;
    const uint32_t ty = rem / e2j, tx = rem - ty * e2j;
    const uint32_t key = (l0 + tz) * (n1 * n2) + (l1 + ty) * n2 + (l2 + tx);
    if (t0 + lane_id() < total)
      put_record(keys, vals, vals2, emit_ids, base + t, key, static_cast<uint32_t>(wave_first + j));
  }
}

// ---------------------------------------------------------- radix sort ---

constexpr int kSortThreads = 256;                       // 4 waves
constexpr int kSortRounds = 16;                         // 64-item rounds per wave
constexpr int kSortWaveItems = 64 * kSortRounds;        // 1024
constexpr int kSortTile = 4 * kSortWaveItems;           // 4096 items per block
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;

__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint32_t *__restrict__ keys,
                                                                  int64_t n, uint32_t shift,
                                                                  uint32_t mask,
                                                                  uint32_t *__restrict__ hist,
                                                                  uint32_t nblocks) {
  __shared__ uint32_t h[kRadix];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += kSortThreads) {
    const int64_t k = base + i;
    if (k < n) atomicAdd(&h[(keys[k] >> shift) & mask], 1u);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = h[threadIdx.x];
}

// One block sorts its kSortTile items by digit in LDS (stable: waves in
// order, rounds in order, lanes by ballot rank), then writes them out in
// block-local digit order, so each digit's items leave as one contiguous run
// of the destination (coalesced writes).  kTwo: a second payload (the flat
// id while the first is the emission index) travels with the key; the final
// pass then writes vals_out32 = second payload and src_out = first.
template <bool kFinal, bool kTwo>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t *__restrict__ keys_in, const uint32_t *__restrict__ vals_in,
    const uint32_t *__restrict__ vals2_in, int64_t n, uint32_t shift, uint32_t bits,
    const uint32_t *__restrict__ digit_offsets, uint32_t nblocks, uint32_t *__restrict__ keys_out,
    uint32_t *__restrict__ vals_out, uint32_t *__restrict__ vals2_out,
    int64_t *__restrict__ keys_out64, int32_t *__restrict__ vals_out32,
    int32_t *__restrict__ src_out) {
  __shared__ uint32_t cnt[4][kRadix];
  __shared__ uint32_t wbase[4][kRadix];
  __shared__ uint32_t dbase[kRadix];   // block-local start of each digit
  __shared__ uint32_t gbase[kRadix];   // global start of this block's run of each digit
  __shared__ uint32_t wsum[4];
  __shared__ uint32_t s_key[kSortTile];
  __shared__ uint32_t s_val[kSortTile];
  __shared__ uint32_t s_val2[kTwo ? kSortTile : 1];
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (int k = threadIdx.x; k < 4 * kRadix; k += kSortThreads) (&cnt[0][0])[k] = 0;
  __syncthreads();
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t block_first = static_cast<int64_t>(blockIdx.x) * kSortTile;
  const int64_t first = block_first + w * kSortWaveItems;
  const uint64_t lt = lanemask_lt();
  uint32_t key[kSortRounds], val[kSortRounds], val2[kSortRounds], rank[kSortRounds];
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    const bool valid = i < n;
    key[r] = valid ? keys_in[i] : 0u;
    val[r] = valid ? vals_in[i] : 0u;
    val2[r] = (kTwo && valid) ? vals2_in[i] : 0u;
    const uint32_t d = (key[r] >> shift) & mask;
    // Lanes holding the same digit: intersect the ballots of every digit bit.
    uint64_t peers = ballot(valid);
    for (uint32_t b = 0; b < bits; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bal = ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    uint32_t c = 0;
    if (valid) c = cnt[w][d];
    rank[r] = c + static_cast<uint32_t>(__popcll(peers & lt));
    // The highest lane of each digit group advances that digit's counter.
    if (valid && lane == 63u - static_cast<uint32_t>(__clzll(peers)))
      cnt[w][d] = c + static_cast<uint32_t>(__popcll(peers));
  }
  __syncthreads();
  {
    // Per digit: wave offsets, block total, then the exclusive scan of the
    // totals over digits (one digit per thread, 4 waves of 64).
    const uint32_t d = threadIdx.x;
    uint32_t tot = 0;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      wbase[ww][d] = tot;
      tot += cnt[ww][d];
    }
    const uint32_t incl = wave_inclusive_scan(tot);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t ww = 0; ww < w; ++ww) before += wsum[ww];
    dbase[d] = before + incl - tot;
    gbase[d] = digit_offsets[static_cast<int64_t>(d) * nblocks + blockIdx.x];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    if (i < n) {
      const uint32_t d = (key[r] >> shift) & mask;
      const uint32_t lp = dbase[d] + wbase[w][d] + rank[r];
      s_key[lp] = key[r];
      s_val[lp] = val[r];
      if (kTwo) s_val2[lp] = val2[r];
    }
  }
  __syncthreads();
  const int count = static_cast<int>(min(static_cast<int64_t>(kSortTile), n - block_first));
  for (int lp = threadIdx.x; lp < count; lp += kSortThreads) {
    const uint32_t k = s_key[lp], v = s_val[lp];
    const uint32_t d = (k >> shift) & mask;
    const int64_t dest = static_cast<int64_t>(gbase[d]) + (lp - static_cast<int>(dbase[d]));
    if (kFinal) {
      keys_out64[dest] = static_cast<int64_t>(k);
      if (kTwo) {
        vals_out32[dest] = static_cast<int32_t>(s_val2[lp]);
        src_out[dest] = static_cast<int32_t>(v);
      } else {
        vals_out32[dest] = static_cast<int32_t>(v);
      }
    } else {
      keys_out[dest] = k;
      vals_out[dest] = v;
      if (kTwo) vals2_out[dest] = s_val2[lp];
    }
  }
}

// ------------------------------------------------------------- offsets ---

__global__ __launch_bounds__(256) void offset_encode_kernel(const int64_t *__restrict__ ids,
                                                            int64_t n, int64_t n_keys,
                                                            int32_t *__restrict__ out) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (k >= n_keys) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ids[mid] < k)
      lo = mid + 1;
    else
      hi = mid;
  }
  out[k] = static_cast<int32_t>(lo);
}

// ----------------------------------------------------------- workspace ---

struct SortSpace {
  uint32_t *ka, *va, *wa, *kb, *vb, *wb, *hist, *hist_scan, *partials;
  int64_t nblocks, n_hist;
};

SortSpace carve_sort(Carver &cv, int64_t n) {
  SortSpace s;
  s.nblocks = ceil_div(n, kSortTile);
  s.n_hist = s.nblocks * kRadix;
  s.ka = cv.take<uint32_t>(n);
  s.va = cv.take<uint32_t>(n);
  s.wa = cv.take<uint32_t>(n);
  s.kb = cv.take<uint32_t>(n);
  s.vb = cv.take<uint32_t>(n);
  s.wb = cv.take<uint32_t>(n);
  s.hist = cv.take<uint32_t>(s.n_hist);
  s.hist_scan = cv.take<uint32_t>(s.n_hist);
  s.partials = cv.take<uint32_t>(scan_partials_count(s.n_hist));
  return s;
}

int64_t count_space_bytes(int64_t n_items) {
  Carver cv(nullptr);
  cv.take<int64_t>(scan_partials_count(n_items));
  return static_cast<int64_t>(cv.used);
}

int64_t sort_space_bytes(int64_t n) {
  Carver cv(nullptr);
  carve_sort(cv, n);
  return static_cast<int64_t>(cv.used);
}

// Sorts the emitted records held in s.ka / s.va (/ s.wa) into the final
// outputs; passes ping-pong between the a and b buffers.  two: s.va holds
// emission indices and s.wa flat ids; the final pass writes vals32 = flat id
// and src = emission index.  The key bits are split evenly over the passes
// (e.g. 6 + 5 for 11 bits): fewer digits per pass give longer runs per digit
// and block, hence better coalesced writes.
int radix_sort(SortSpace &s, int64_t n, uint32_t end_bit, int64_t *keys64, int32_t *vals32,
               bool two, int32_t *src, hipStream_t stream) {
  const uint32_t passes = (end_bit + kRadixBits - 1) / kRadixBits;
  const uint32_t pbits = (end_bit + passes - 1) / passes;
  uint32_t *kin = s.ka, *vin = s.va, *win = s.wa, *kout = s.kb, *vout = s.vb, *wout = s.wb;
  const uint32_t nb = static_cast<uint32_t>(s.nblocks);
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t shift = p * pbits;
    const uint32_t bits = min(pbits, end_bit - shift);
    const uint32_t mask = (1u << bits) - 1u;
    radix_hist_kernel<<<dim3(nb), dim3(kSortThreads), 0, stream>>>(kin, n, shift, mask, s.hist, nb);
    R2S_RETURN_IF(device_exclusive_scan<uint32_t, uint32_t>(s.hist, s.n_hist, s.hist_scan,
                                                            nullptr, s.partials, stream,
                                                            "isect sort scan"));
    const bool last = p == passes - 1;
#define R2S_SCATTER(FINAL, TWO)                                                                 \
  radix_scatter_kernel<FINAL, TWO><<<dim3(nb), dim3(kSortThreads), 0, stream>>>(               \
      kin, vin, win, n, shift, bits, s.hist_scan, nb, kout, vout, wout, keys64, vals32, src)
    if (last) {
      if (two)
        R2S_SCATTER(true, true);
      else
        R2S_SCATTER(true, false);
    } else {
      if (two)
        R2S_SCATTER(false, true);
      else
        R2S_SCATTER(false, false);
      std::swap(kin, kout);
      std::swap(vin, vout);
      std::swap(win, wout);
    }
#undef R2S_SCATTER
    R2S_RETURN_IF(check_launch("isect sort pass"));
  }
  return R2S_OK;
}

// ---------------------------------------------------------------- host ---

int check_workspace(void *ws, size_t have, int64_t need, const char *name) {
  if (need > 0 && (ws == nullptr || static_cast<int64_t>(have) < need)) {
    set_error("%s: workspace of %zu bytes, %lld required", name, have, (long long)need);
    return R2S_EWORKSPACE;
  }
  return R2S_OK;
}

template <typename T>
int count_2d_impl(const T *means2d, const int32_t *radii, int rect, int64_t C, int64_t N,
                  uint32_t ts, uint32_t tw, uint32_t th, int32_t *counts, int64_t *offsets,
                  void *ws, size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles";
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size C=%lld N=%lld", name,
              (long long)C, (long long)N);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_REQUIRE(static_cast<uint64_t>(C) * tw * th <= 0xffffffffull,
              "%s: C * n_tiles exceeds 32 bits", name);
  R2S_REQUIRE(offsets != nullptr, "%s: null offsets", name);
  const int64_t M = C * N;
  hipStream_t stream = as_stream(st);
  if (M == 0) return device_fill<int64_t>(offsets, 1, 0, stream, name);
  R2S_REQUIRE(means2d && radii && counts, "%s: null pointer", name);
  R2S_RETURN_IF(check_workspace(ws, ws_bytes, count_space_bytes(M), name));
  Carver cv(ws);
  int64_t *partials = cv.take<int64_t>(scan_partials_count(M));
  count_2d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(M, 256))), dim3(256), 0, stream>>>(
      means2d, radii, rect, M, ts, tw, th, counts);
  R2S_RETURN_IF(check_launch(name));
  return device_exclusive_scan<int32_t, int64_t>(counts, M, offsets, offsets + M, partials,
                                                 stream, name);
}

template <typename T>
int count_3d_impl(const T *means3d, const int32_t *radii, int64_t N, uint32_t ts, uint32_t n2,
                  uint32_t n1, uint32_t n0, int32_t *counts, int64_t *offsets, void *ws,
                  size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles_3d";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size N=%lld", name, (long long)N);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * n1 * n0 <= 0xffffffffull,
              "%s: n_tiles exceeds 32 bits", name);
  R2S_REQUIRE(offsets != nullptr, "%s: null offsets", name);
  hipStream_t stream = as_stream(st);
  if (N == 0) return device_fill<int64_t>(offsets, 1, 0, stream, name);
  R2S_REQUIRE(means3d && radii && counts, "%s: null pointer", name);
  R2S_RETURN_IF(check_workspace(ws, ws_bytes, count_space_bytes(N), name));
  Carver cv(ws);
  int64_t *partials = cv.take<int64_t>(scan_partials_count(N));
  count_3d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0, stream>>>(
      means3d, radii, N, ts, n2, n1, n0, counts);
  R2S_RETURN_IF(check_launch(name));
  return device_exclusive_scan<int32_t, int64_t>(counts, N, offsets, offsets + N, partials,
                                                 stream, name);
}

int check_sort_args(int64_t n_isects, uint32_t end_bit, int64_t n_keys, void *ws,
                    size_t ws_bytes, int64_t *keys, int32_t *vals, const char *name) {
  R2S_REQUIRE(n_isects >= 0, "%s: negative n_isects", name);
  if (n_isects > kInt32Max) {
    set_error("%s: %lld intersections exceed the int32 offset range", name,
              (long long)n_isects);
    return R2S_ERANGE;
  }
  R2S_REQUIRE(end_bit >= 1 && end_bit <= 32, "%s: end_bit %u out of range", name, end_bit);
  R2S_REQUIRE(n_keys <= (1ll << end_bit), "%s: end_bit %u too small for %lld keys", name,
              end_bit, (long long)n_keys);
  if (n_isects == 0) return R2S_OK;
  R2S_REQUIRE(keys && vals, "%s: null output", name);
  return check_workspace(ws, ws_bytes, sort_space_bytes(n_isects), name);
}

template <typename T>
int emit_sort_2d_impl(const T *means2d, const int32_t *radii, int rect, int64_t C, int64_t N,
                      uint32_t ts, uint32_t tw, uint32_t th, const int64_t *offsets,
                      int64_t n_isects, uint32_t end_bit, int64_t *keys, int32_t *vals,
                      int32_t *emit_ids, int32_t *isect_src, void *ws, size_t ws_bytes,
                      r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles";
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size", name);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_RETURN_IF(check_sort_args(n_isects, end_bit, C * tw * th, ws, ws_bytes, keys, vals, name));
  if (n_isects == 0) return R2S_OK;
  R2S_REQUIRE(means2d && radii && offsets, "%s: null pointer", name);
  hipStream_t stream = as_stream(st);
  Carver cv(ws);
  SortSpace s = carve_sort(cv, n_isects);
  R2S_REQUIRE((emit_ids == nullptr) == (isect_src == nullptr),
              "%s: emit_ids and isect_src must be given together", name);
  const int64_t M = C * N;
  emit_2d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(M, 256))), dim3(256), 0, stream>>>(
      means2d, radii, rect, M, N, ts, tw, th, offsets, s.ka, s.va, s.wa, emit_ids);
  R2S_RETURN_IF(check_launch(name));
  return radix_sort(s, n_isects, end_bit, keys, vals, emit_ids != nullptr, isect_src, stream);
}

template <typename T>
int emit_sort_3d_impl(const T *means3d, const int32_t *radii, int64_t N, uint32_t ts,
                      uint32_t n2, uint32_t n1, uint32_t n0, const int64_t *offsets,
                      int64_t n_isects, uint32_t end_bit, int64_t *keys, int32_t *vals,
                      int32_t *emit_ids, int32_t *isect_src, void *ws, size_t ws_bytes,
                      r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles_3d";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size", name);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_RETURN_IF(check_sort_args(n_isects, end_bit, static_cast<int64_t>(n2) * n1 * n0, ws,
                                ws_bytes, keys, vals, name));
  if (n_isects == 0) return R2S_OK;
  R2S_REQUIRE(means3d && radii && offsets, "%s: null pointer", name);
  hipStream_t stream = as_stream(st);
  Carver cv(ws);
  SortSpace s = carve_sort(cv, n_isects);
  R2S_REQUIRE((emit_ids == nullptr) == (isect_src == nullptr),
              "%s: emit_ids and isect_src must be given together", name);
  emit_3d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0, stream>>>(
      means3d, radii, N, ts, n2, n1, n0, offsets, s.ka, s.va, s.wa, emit_ids);
  R2S_RETURN_IF(check_launch(name));
  return radix_sort(s, n_isects, end_bit, keys, vals, emit_ids != nullptr, isect_src, stream);
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_isect_workspace_bytes(int64_t n_items, int64_t n_isects, uint32_t end_bit) {
  (void)end_bit;
  const int64_t a = n_items > 0 ? r2s::count_space_bytes(n_items) : 0;
  const int64_t b = n_isects > 0 ? r2s::sort_space_bytes(n_isects) : 0;
  return a > b ? a : b;
}

#define R2S_BIN_API(SUF, T)                                                                   \
  int r2s_isect_count_2d_##SUF(const T *means2d, const int32_t *radii, int rect, int64_t C,   \
                               int64_t N, uint32_t ts, uint32_t tw, uint32_t th,              \
                               int32_t *counts, int64_t *offsets, void *ws, size_t ws_bytes,  \
                               r2s_stream_t st) {                                             \
    return r2s::count_2d_impl<T>(means2d, radii, rect, C, N, ts, tw, th, counts, offsets, ws, \
                                 ws_bytes, st);                                               \
  }                                                                                           \
  int r2s_isect_emit_sort_2d_##SUF(const T *means2d, const int32_t *radii, int rect,          \
                                   int64_t C, int64_t N, uint32_t ts, uint32_t tw,            \
                                   uint32_t th, const int64_t *offsets, int64_t n_isects,     \
                                   uint32_t end_bit, int64_t *keys, int32_t *vals,            \
                                   int32_t *emit_ids, int32_t *isect_src, void *ws,          \
                                   size_t ws_bytes, r2s_stream_t st) {                        \
    return r2s::emit_sort_2d_impl<T>(means2d, radii, rect, C, N, ts, tw, th, offsets,         \
                                     n_isects, end_bit, keys, vals, emit_ids, isect_src, ws,  \
                                     ws_bytes, st);                                           \
  }                                                                                           \
  int r2s_isect_count_3d_##SUF(const T *means3d, const int32_t *radii, int64_t N,            \
                               uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,            \
                               int32_t *counts, int64_t *offsets, void *ws, size_t ws_bytes,  \
                               r2s_stream_t st) {                                             \
    return r2s::count_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, counts, offsets, ws,      \
                                 ws_bytes, st);                                               \
  }                                                                                           \
  int r2s_isect_emit_sort_3d_##SUF(const T *means3d, const int32_t *radii, int64_t N,        \
                                   uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,        \
                                   const int64_t *offsets, int64_t n_isects,                  \
                                   uint32_t end_bit, int64_t *keys, int32_t *vals,            \
                                   int32_t *emit_ids, int32_t *isect_src, void *ws,          \
                                   size_t ws_bytes, r2s_stream_t st) {                        \
    return r2s::emit_sort_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, offsets, n_isects,    \
                                     end_bit, keys, vals, emit_ids, isect_src, ws, ws_bytes,  \
                                     st);                                                     \
  }

R2S_BIN_API(f32, float)
R2S_BIN_API(f64, double)

#undef R2S_BIN_API

int r2s_isect_offset_encode(const int64_t *ids, int64_t n_isects, int64_t n_keys,
                            int32_t *out, r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n_isects >= 0 && n_keys >= 0, "isect_offset_encode: negative size");
  if (n_keys == 0) return R2S_OK;
  R2S_REQUIRE(out != nullptr, "isect_offset_encode: null output");
  hipStream_t stream = r2s::as_stream(st);
  if (n_isects == 0) return r2s::device_fill<int32_t>(out, n_keys, 0, stream, "isect_offset_encode");
  R2S_REQUIRE(ids != nullptr, "isect_offset_encode: null isect_ids");
  r2s::offset_encode_kernel<<<dim3(static_cast<uint32_t>(r2s::ceil_div(n_keys, 256))), dim3(256), 0,
                              stream>>>(ids, n_isects, n_keys, out);
  return r2s::check_launch("isect_offset_encode");
}

}  // extern "C"
