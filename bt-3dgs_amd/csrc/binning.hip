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
//   sort    stable LSD radix sort on the bits that hold every key below
//           n_keys, in the fewest passes of at most 11-bit digits (one pass
//           for up to 2048 tiles).  Per pass: LDS digit histogram per
//           4096-item tile, device scan of the digit-major histogram table,
//           stable scatter with per-wave ranks from ballot-based digit
//           matching (no per-item atomics).  The first pass takes the
//           emission index from the item's position; the last widens keys
//           to int64 on the way out.
//   offsets lower_bound of every key in the sorted list (binary search).
//
// Because emission is in ascending record id and every pass is stable, the
// output is the lexicographic (key, id) order -- identical to the
// reference's CUB sort of the same records.
#pragma clang fp contract(off)

#include <type_traits>
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

// Brick box of Gaussian idx, restricted to the brick layers z0 <= b0 < z1
// (dim0; the whole grid is z0 = 0, z1 = n0).
template <typename T>
__device__ __forceinline__ uint32_t box_3d(const T *__restrict__ means3d,
                                           const int32_t *__restrict__ radii, int64_t idx,
                                           uint32_t ts, const uint32_t n[3], uint32_t z0,
                                           uint32_t z1, Box &b) {
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
  b.lo[2] = max(b.lo[2], z0);
  b.hi[2] = min(b.hi[2], z1);
  if (b.hi[2] <= b.lo[2]) {
    b.lo[2] = b.hi[2] = z0;
    return 0;
  }
  return (b.hi[2] - b.lo[2]) * (b.hi[1] - b.lo[1]) * (b.hi[0] - b.lo[0]);
}

// --------------------------------------------------------------- count ---
//
// The count kernels cover the scan's tiles (r2s_scan.h: kScanTile items per
// block) and store each block's count sum into the scan's block sums, so the
// exclusive scan of the counts needs only its downsweep (one launch fewer).
// kCountThreads threads per block (item k kCountThreads + t to thread t):
// enough waves in flight to hide the gathers' latency.
constexpr int kCountThreads = 1024;
constexpr int kCountItems = kScanTile / kCountThreads;

template <typename T>
__global__ __launch_bounds__(kCountThreads) void count_2d_kernel(
    const T *__restrict__ means2d, const int32_t *__restrict__ radii, int rect, int64_t M,
    uint32_t ts, uint32_t tw, uint32_t th, int32_t *__restrict__ counts,
    int64_t *__restrict__ block_sums) {
  __shared__ int64_t lds[kCountThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x;
  int64_t s = 0;
#pragma unroll
  for (int k = 0; k < kCountItems; ++k) {
    const int64_t idx = base + k * kCountThreads;
    if (idx < M) {
      Rect r;
      const uint32_t c = rect_2d(means2d, radii, rect, idx, ts, tw, th, r);
      counts[idx] = static_cast<int32_t>(c);
      s += c;
    }
  }
  int64_t total;
  block_exclusive_scan(s, lds, total);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

template <typename T>
__global__ __launch_bounds__(kCountThreads) void count_3d_kernel(
    const T *__restrict__ means3d, const int32_t *__restrict__ radii, int64_t N, uint32_t ts,
    uint32_t n2, uint32_t n1, uint32_t n0, uint32_t z0, uint32_t z1,
    int32_t *__restrict__ counts, int64_t *__restrict__ block_sums) {
  __shared__ int64_t lds[kCountThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x;
  const uint32_t n[3] = {n2, n1, n0};
  int64_t s = 0;
#pragma unroll
  for (int k = 0; k < kCountItems; ++k) {
    const int64_t idx = base + k * kCountThreads;
    if (idx < N) {
      Box b;
      const uint32_t c = box_3d(means3d, radii, idx, ts, n, z0, z1, b);
      counts[idx] = static_cast<int32_t>(c);
      s += c;
    }
  }
  int64_t total;
  block_exclusive_scan(s, lds, total);
  if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// Records per brick layer: each Gaussian's box adds its (dim2, dim1) area to
// the layers [lo2, hi2) of a difference array diff[0..n0] (diff[lo2] += a,
// diff[hi2] -= a), summed in LDS per block when n0 < kLayerBins.
constexpr uint32_t kLayerBins = 1024;

template <typename T>
__global__ __launch_bounds__(256) void layer_diff_3d_kernel(const T *__restrict__ means3d,
                                                            const int32_t *__restrict__ radii,
                                                            int64_t N, uint32_t ts, uint32_t n2,
                                                            uint32_t n1, uint32_t n0,
                                                            unsigned long long *__restrict__ diff) {
  __shared__ unsigned long long s_bins[kLayerBins];
  const bool lds = n0 < kLayerBins;
  if (lds) {
    for (uint32_t k = threadIdx.x; k <= n0; k += 256) s_bins[k] = 0ull;
    __syncthreads();
  }
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx < N) {
    const uint32_t n[3] = {n2, n1, n0};
    Box b;
    if (box_3d(means3d, radii, idx, ts, n, 0u, n0, b) > 0) {
      const unsigned long long area =
          static_cast<unsigned long long>(b.hi[1] - b.lo[1]) * (b.hi[0] - b.lo[0]);
      unsigned long long *bins = lds ? s_bins : diff;
      atomicAdd(bins + b.lo[2], area);
      atomicAdd(bins + b.hi[2], ~area + 1ull);  // two's complement: -area
    }
  }
  if (lds) {
    __syncthreads();
    for (uint32_t k = threadIdx.x; k <= n0; k += 256)
      if (s_bins[k] != 0ull) atomicAdd(diff + k, s_bins[k]);
  }
}

// counts[z] = diff[0] + ... + diff[z] for z < n0 (one thread: n0 is the
// number of brick layers).
__global__ void layer_prefix_kernel(const unsigned long long *__restrict__ diff, uint32_t n0,
                                    int64_t *__restrict__ counts) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  unsigned long long run = 0ull;
  for (uint32_t z = 0; z < n0; ++z) {
    run += diff[z];
    counts[z] = static_cast<int64_t>(run);
  }
}

// ---------------------------------------------------------------- emit ---

// Inclusive prefix maximum over the lanes of a wave: DPP row shifts by 1,
// 2, 4, 8 within each row of 16 lanes, then the row broadcasts of lanes 15
// and 31 (VALU only, no LDS round trip).  -1 is the identity (every value
// is >= -1).
__device__ __forceinline__ int wave_prefix_max(int v) {
  v = max(v, dpp_take<0x111, 0xf>(v, -1));  // row_shr:1
  v = max(v, dpp_take<0x112, 0xf>(v, -1));  // row_shr:2
  v = max(v, dpp_take<0x114, 0xf>(v, -1));  // row_shr:4
  v = max(v, dpp_take<0x118, 0xf>(v, -1));  // row_shr:8
  v = max(v, dpp_take<0x142, 0xa>(v, -1));  // row_bcast:15
  v = max(v, dpp_take<0x143, 0xc>(v, -1));  // row_bcast:31
  return v;
}

// Owners of one round of a wave's emission: the lanes emit excl[j] ..
// excl[j] + cnt[j] - 1, and output t0 + lane belongs to the largest j with
// cnt[j] > 0 and excl[j] <= t0 + lane.  Each lane whose run starts inside the
// round (`starts`, at rel = excl - t0) marks its start in `own` (tagged with
// the round, so older marks read as absent), a prefix maximum over the lanes
// carries each mark forward, and `carry` (the owner of the previous round's
// last output) covers outputs before the round's first start.  Returns the
// owner and updates carry (uniform).
__device__ __forceinline__ int round_owner(uint32_t *own, bool starts, uint32_t rel,
                                           uint32_t round, int &carry) {
  const uint32_t lane = lane_id();
  if (starts) own[rel] = (round << 6) | lane;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t m = own[lane];
  const int mark = (m >> 6) == round ? static_cast<int>(m & 63u) : -1;
  const int o = max(wave_prefix_max(mark), carry);
  carry = __builtin_amdgcn_readlane(o, 63);
  return max(o, 0);
}

// Lane 63's copy of v, in every lane.
__device__ __forceinline__ uint32_t from_lane63(uint32_t v) { return readlane_u32(v, 63); }
__device__ __forceinline__ double from_lane63(double v) {
  return __longlong_as_double(readlane_i64(__double_as_longlong(v), 63));
}

// q = n / d and n - q d for d >= 1 from a double reciprocal of d: one
// multiply instead of an integer division.  The product is within 2^-20 of
// n / d for n < 2^32 (two roundings of 2^-53), so the truncated quotient is
// at most one off, and the remainder corrects it.
__device__ __forceinline__ uint32_t div_rcp(uint32_t n, uint32_t d, double rcp, uint32_t &rem) {
  uint32_t q = static_cast<uint32_t>(static_cast<double>(n) * rcp);
  int64_t r = static_cast<int64_t>(n) - static_cast<int64_t>(q) * d;
  if (r < 0) {
    --q;
    r += d;
  } else if (r >= static_cast<int64_t>(d)) {
    ++q;
    r -= d;
  }
  rem = static_cast<uint32_t>(r);
  return q;
}

// Writes emitted record e: its key and its flat id (the emission-order id
// array the two-pass backward reads, or the sort's own copy).
__device__ __forceinline__ void put_record(uint32_t *__restrict__ keys, uint32_t *__restrict__ gids,
                                           int64_t e, uint32_t key, uint32_t gid) {
  keys[e] = key;
  gids[e] = gid;
}

// A wave's 64 consecutive items emit one contiguous range of records
// (offsets is the exclusive scan of the counts); the range is spread over
// the lanes 64 records at a time, so every store instruction writes 64
// consecutive records.  Tiles of one item are row-major in its rectangle.
template <typename T>
__global__ __launch_bounds__(256) void emit_2d_kernel(
    const T *__restrict__ means2d, const int32_t *__restrict__ radii, int rect, int64_t M,
    int64_t N, uint32_t ts, uint32_t tw, uint32_t th, const int64_t *__restrict__ offsets,
    int64_t cap, uint32_t *__restrict__ keys, uint32_t *__restrict__ gids) {
  __shared__ uint32_t s_own[4][64];
  __shared__ uint4 s_item[4][64];  // excl, width, first key
  __shared__ double s_rcp[4][64];  // 1 / width
  const uint32_t w = wave_index(), lane = lane_id();
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * 256 + 64 * w;
  if (wave_first >= M || offsets[M] > cap) return;  // uniform per wave
  const int64_t idx = wave_first + lane;
  Rect r = {0, 0, 0, 0};
  uint32_t cnt = 0;
  if (idx < M) cnt = rect_2d(means2d, radii, rect, idx, ts, tw, th, r);
  const uint32_t incl = wave_inclusive_scan(cnt);
  const uint32_t excl = incl - cnt;
  const uint32_t total = readlane_u32(incl, 63);
  const int64_t base = offsets[wave_first];
  // Per item once: the key of its rectangle's first tile and 1 / width, so
  // that a record costs a multiply instead of two integer divisions.
  const uint32_t width = max(r.x1 - r.x0, 1u);
  const uint32_t kb = idx < M ? static_cast<uint32_t>(idx / N) * (tw * th) + r.y0 * tw + r.x0 : 0u;
  s_item[w][lane] = make_uint4(excl, width, kb, 0u);
  s_rcp[w][lane] = 1.0 / static_cast<double>(width);
  s_own[w][lane] = 0xffffffffu;  // no round's tag
  int carry = -1, o = 0;
  uint4 it = s_item[w][lane];
  double rc = s_rcp[w][lane];
  for (uint32_t t0 = 0, round = 0; t0 < total; t0 += 64, ++round) {
    const uint32_t rel = excl - t0;  // wraps for runs starting before the round
    const bool starts = cnt > 0u && rel < 64u;
    if (ballot(starts) == 0ull) {
      // The round lies inside the run holding the previous round's last
      // output (never the first round: its first output starts a run).
      o = carry;
      it = make_uint4(from_lane63(it.x), from_lane63(it.y), from_lane63(it.z), 0u);
      rc = from_lane63(rc);
    } else {
      o = round_owner(s_own[w], starts, rel, round, carry);
      it = s_item[w][o];
      rc = s_rcp[w][o];
    }
    const uint32_t t = t0 + lane;
    uint32_t col;
    const uint32_t row = div_rcp(t - it.x, it.y, rc, col);
    if (t < total)
      put_record(keys, gids, base + t, it.z + row * tw + col, static_cast<uint32_t>(wave_first + o));
  }
}

// Keys are relative to the window's first layer: (b0 - z0) n1 n2 + b1 n2 + b2.
template <typename T>
__global__ __launch_bounds__(256) void emit_3d_kernel(
    const T *__restrict__ means3d, const int32_t *__restrict__ radii, int64_t N, uint32_t ts,
    uint32_t n2, uint32_t n1, uint32_t n0, uint32_t z0, uint32_t z1,
    const int64_t *__restrict__ offsets, int64_t cap, uint32_t *__restrict__ keys,
    uint32_t *__restrict__ gids) {
  __shared__ uint32_t s_own[4][64];
  __shared__ uint4 s_item[4][64];     // excl, extent along dim2, plane, first key
  __shared__ double2 s_rcp[4][64];    // 1 / plane, 1 / extent along dim2
  const uint32_t w = wave_index(), lane = lane_id();
  const int64_t wave_first = static_cast<int64_t>(blockIdx.x) * 256 + 64 * w;
  if (wave_first >= N || offsets[N] > cap) return;  // uniform per wave
  const int64_t idx = wave_first + lane;
  const uint32_t n[3] = {n2, n1, n0};
  Box b;
  uint32_t cnt = 0;
  if (idx < N) {
    cnt = box_3d(means3d, radii, idx, ts, n, z0, z1, b);
  } else {
#pragma unroll
    for (int a = 0; a < 3; ++a) b.lo[a] = b.hi[a] = 0;
  }
  const uint32_t incl = wave_inclusive_scan(cnt);
  const uint32_t excl = incl - cnt;
  const uint32_t total = readlane_u32(incl, 63);
  const int64_t base = offsets[wave_first];
  // Per item once: the key of its box's first brick and the reciprocals of
  // its extents, so that a record costs two multiplies instead of two
  // integer divisions.
  const uint32_t e2 = max(b.hi[0] - b.lo[0], 1u), e1 = max(b.hi[1] - b.lo[1], 1u);
  const uint32_t plane = e2 * e1;
  s_item[w][lane] = make_uint4(excl, e2, plane, (b.lo[2] - z0) * (n1 * n2) + b.lo[1] * n2 + b.lo[0]);
  s_rcp[w][lane] = make_double2(1.0 / static_cast<double>(plane), 1.0 / static_cast<double>(e2));
  s_own[w][lane] = 0xffffffffu;  // no round's tag
  int carry = -1, o = 0;
  uint4 it = s_item[w][lane];
  double2 rc = s_rcp[w][lane];
  for (uint32_t t0 = 0, round = 0; t0 < total; t0 += 64, ++round) {
    const uint32_t rel = excl - t0;  // wraps for runs starting before the round
    const bool starts = cnt > 0u && rel < 64u;
    if (ballot(starts) == 0ull) {
      // The round lies inside the run holding the previous round's last
      // output (never the first round: its first output starts a run).
      o = carry;
      it = make_uint4(from_lane63(it.x), from_lane63(it.y), from_lane63(it.z),
                      from_lane63(it.w));
      rc = make_double2(from_lane63(rc.x), from_lane63(rc.y));
    } else {
      o = round_owner(s_own[w], starts, rel, round, carry);
      it = s_item[w][o];
      rc = s_rcp[w][o];
    }
    const uint32_t t = t0 + lane;
    uint32_t rem, tx;
    const uint32_t tz = div_rcp(t - it.x, it.z, rc.x, rem);
    const uint32_t ty = div_rcp(rem, it.y, rc.y, tx);
    if (t < total)
      put_record(keys, gids, base + t, it.w + tz * (n1 * n2) + ty * n2 + tx,
                 static_cast<uint32_t>(wave_first + o));
  }
}

// ---------------------------------------------------------- radix sort ---

constexpr int kSortThreads = 256;                       // 4 waves
constexpr int kSortRounds = 16;                         // 64-item rounds per wave
constexpr int kSortWaveItems = 64 * kSortRounds;        // 1024
constexpr int kSortTile = 4 * kSortWaveItems;           // 4096 items per block
constexpr int kMaxPassBits = 11;                        // up to 2048 digits per pass
constexpr int kMaxDigits = 1 << kMaxPassBits;

// The sort kernels are sized for `cap` items and read the actual count n
// from the device (the emission scan's total); with n > cap they write
// nothing, so a caller may launch them before it knows n.

// Digit histogram of one 4096-item tile, written digit-major:
// hist[d * nblocks + tile] (zero rows for tiles past n).  Tiles are
// XCD-contiguous (xcd_swizzle), so the blocks writing neighbouring words of
// a digit's row share an L2.
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint32_t *__restrict__ keys,
                                                                  const int64_t *__restrict__ n_dev,
                                                                  int64_t cap, uint32_t shift,
                                                                  uint32_t digits,
                                                                  uint32_t *__restrict__ hist,
                                                                  uint32_t nblocks) {
  __shared__ uint32_t h[kMaxDigits];
  const int64_t n = *n_dev;
  if (n <= 0 || n > cap) return;
  const uint32_t tile = xcd_swizzle(blockIdx.x, nblocks);
  for (uint32_t d = threadIdx.x; d < digits; d += kSortThreads) h[d] = 0;
  __syncthreads();
  const uint32_t mask = digits - 1u;
  const int64_t base = static_cast<int64_t>(tile) * kSortTile + threadIdx.x;
  // All loads first (clamped in bounds), then the LDS counts.
  uint32_t key[kSortRounds];
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) key[r] = keys[min(base + r * kSortThreads, n - 1)];
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r)
    if (base + r * kSortThreads < n) atomicAdd(&h[(key[r] >> shift) & mask], 1u);
  __syncthreads();
  for (uint32_t d = threadIdx.x; d < digits; d += kSortThreads)
    hist[static_cast<int64_t>(d) * nblocks + tile] = h[d];
}

// One block sorts its kSortTile items by digit in LDS (stable: waves in
// order, rounds in order, lanes by ballot rank), then writes them out in
// block-local digit order, so each digit's items leave as one contiguous run
// of the destination.  Each item carries its key, its flat id (gid) and,
// with kTwo, its emission index e.  kFirst: the input is the emission-order
// array itself, so e is the input index and only keys and gids are read.
// kFinal: writes keys_out64 / vals_out32 = gid / src_out = e; with
// keys_out64 null (a caller keeping only the tile offsets) the keys go to
// keys_out when it is given (for a later offset search) and nowhere else.
// The LDS footprint follows the sort: digit tables for 2^kDBits digits,
// keys staged as 16 bits when every key fits (kKey16), and in a single-pass
// sort the emission index staged as its 16-bit block-local position.  At
// config 4 (one 10-bit pass) and config 3 (two passes of 8 and 7 bits over
// 15-bit keys) that leaves room for three blocks per CU instead of two.
template <bool kFirst, bool kFinal, bool kTwo, int kDBits, bool kKey16>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint32_t *__restrict__ keys_in, const uint32_t *__restrict__ e_in,
    const uint32_t *__restrict__ gid_in, const int64_t *__restrict__ n_dev, int64_t cap,
    uint32_t shift, uint32_t bits,
    const uint32_t *__restrict__ digit_offsets, uint32_t nblocks, uint32_t *__restrict__ keys_out,
    uint32_t *__restrict__ e_out, uint32_t *__restrict__ gid_out,
    int64_t *__restrict__ keys_out64, int32_t *__restrict__ vals_out32,
    int32_t *__restrict__ src_out, int32_t *__restrict__ tile_offsets, uint32_t n_keys) {
  static_assert(kDBits >= 8 && kDBits <= kMaxPassBits, "digit tables of 256 to 2048");
  constexpr int kD = 1 << kDBits;
  constexpr int kDPT = kD / kSortThreads;  // digits per thread in the scan
  constexpr bool kLocalE = kFirst && kFinal;
  using KeyS = typename std::conditional<kKey16, uint16_t, uint32_t>::type;
  using ES = typename std::conditional<kLocalE, uint16_t, uint32_t>::type;
  // Per-wave digit counters, then (in place) each wave's start within the
  // digit's block-local run; at most 1024 items per wave, so 16 bits hold them.
  __shared__ uint16_t cnt[4][kD];
  __shared__ uint16_t dbase[kD];  // block-local start of each digit (<= 4096)
  __shared__ uint32_t gbase[kD];  // global start of this block's run of each digit
  __shared__ uint32_t wsum[kSortThreads / 64];
  __shared__ KeyS s_key[kSortTile];
  __shared__ uint32_t s_gid[kSortTile];
  __shared__ ES s_e[kTwo ? kSortTile : 1];
  const uint32_t digits = 1u << bits, mask = digits - 1u;
  const uint32_t tile = xcd_swizzle(blockIdx.x, nblocks);
  const int64_t n = *n_dev;
  const int64_t block_first = static_cast<int64_t>(tile) * kSortTile;
  if (n > cap) return;  // uniform per block
  if (block_first >= n) {
    // Block 0 has no records only when there are none at all (a capacity
    // guessed before the count was known): then every key starts at 0.
    if (kFinal && tile_offsets != nullptr && tile == 0)
      for (uint32_t d = threadIdx.x; d < n_keys; d += kSortThreads) tile_offsets[d] = 0;
    return;
  }
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (uint32_t k = threadIdx.x; k < 4 * digits; k += kSortThreads)
    cnt[k / digits][k % digits] = 0;
  __syncthreads();
  const int64_t first = block_first + w * kSortWaveItems;
  const uint64_t lt = lanemask_lt();
  uint32_t key[kSortRounds], gid[kSortRounds], ev[kSortRounds], rank[kSortRounds];
  // All loads first (clamped in bounds: a block's last wave may run past n),
  // so their latencies overlap; then the ranking rounds.  Thread t owns
  // digits [t*dk, t*dk + dk) in the scan below; their global run starts do
  // not depend on the ranking, so they load here too.
  const uint32_t dk = (digits + kSortThreads - 1) / kSortThreads;
  const uint32_t d0 = threadIdx.x * dk;
  uint32_t gb[kDPT];
#pragma unroll
  for (uint32_t j = 0; j < kDPT; ++j) {
    const uint32_t d = min(d0 + j, digits - 1u);
    gb[j] = digit_offsets[static_cast<int64_t>(d) * nblocks + tile];
  }
  // A single pass over the whole key (the caller passes tile_offsets only
  // then): block 0's run starts are the numbers of records with a smaller
  // key, i.e. each key's first index in the sorted list.
  if (kFinal && tile_offsets != nullptr && tile == 0) {
#pragma unroll
    for (uint32_t j = 0; j < kDPT; ++j) {
      const uint32_t d = d0 + j;
      if (j < dk && d < n_keys) tile_offsets[d] = static_cast<int32_t>(gb[j]);
    }
  }
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    const int64_t ic = min(i, n - 1);
    key[r] = keys_in[ic];
    gid[r] = gid_in[ic];
    if (kTwo) ev[r] = kFirst ? static_cast<uint32_t>(i) : e_in[ic];
  }
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    const bool valid = i < n;
    const uint32_t d = (key[r] >> shift) & mask;
    // Lanes holding the same digit: those whose bits agree with the lane's in
    // every ballot.  Per bit, ballot ^ (the lane's bit copied to all 64)
    // marks the lanes that differ there; the union over the bits is the
    // complement of the peers.  The loop runs over the table's kDBits bits,
    // unrolled: bits at or above `bits` are zero in every lane's digit, so
    // they mark no lane.
    uint64_t differ = 0;
#pragma unroll
    for (uint32_t b = 0; b < static_cast<uint32_t>(kDBits); ++b) {
      const uint32_t x = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int32_t>(d), b, 1));
      const uint64_t m = ballot(x != 0u);  // x: 0 or all ones
      differ |= m ^ ((static_cast<uint64_t>(x) << 32) | x);
    }
    const uint64_t peers = ballot(valid) & ~differ;
    uint32_t c = 0;
    if (valid) c = cnt[w][d];
    rank[r] = c + static_cast<uint32_t>(__popcll(peers & lt));
    // The highest lane of each digit group advances that digit's counter.
    if (valid && lane == 63u - static_cast<uint32_t>(__clzll(peers)))
      cnt[w][d] = static_cast<uint16_t>(c + static_cast<uint32_t>(__popcll(peers)));
  }
  __syncthreads();
  {
    // Per owned digit the waves' starts and the block total, then an
    // exclusive scan of the totals over digits.
    const uint32_t k = dk;
    uint32_t tot[kDPT];
    uint32_t mine = 0;
#pragma unroll
    for (uint32_t j = 0; j < kDPT; ++j) {
      tot[j] = 0;
      const uint32_t d = d0 + j;
      if (j < k && d < digits) {
        uint32_t run = 0;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
          const uint32_t c = cnt[ww][d];
          cnt[ww][d] = static_cast<uint16_t>(run);
          run += c;
        }
        tot[j] = run;
        mine += run;
      }
    }
    uint32_t block_total;
    uint32_t run = block_exclusive_scan(mine, wsum, block_total);
#pragma unroll
    for (uint32_t j = 0; j < kDPT; ++j) {
      const uint32_t d = d0 + j;
      if (j < k && d < digits) {
        dbase[d] = static_cast<uint16_t>(run);
        run += tot[j];
        gbase[d] = gb[j];
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSortRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    if (i < n) {
      const uint32_t d = (key[r] >> shift) & mask;
      const uint32_t lp = dbase[d] + cnt[w][d] + rank[r];
      s_key[lp] = static_cast<KeyS>(key[r]);
      s_gid[lp] = gid[r];
      if (kTwo) s_e[lp] = static_cast<ES>(kLocalE ? ev[r] - block_first : ev[r]);
    }
  }
  __syncthreads();
  const int count = static_cast<int>(min(static_cast<int64_t>(kSortTile), n - block_first));
  for (int lp = threadIdx.x; lp < count; lp += kSortThreads) {
    const uint32_t k = s_key[lp];
    const uint32_t d = (k >> shift) & mask;
    const int64_t dest = static_cast<int64_t>(gbase[d]) + (lp - static_cast<int>(dbase[d]));
    if (kFinal) {
      if (keys_out64 != nullptr)
        keys_out64[dest] = static_cast<int64_t>(k);
      else if (keys_out != nullptr)
        keys_out[dest] = k;
      vals_out32[dest] = static_cast<int32_t>(s_gid[lp]);
      if (kTwo)
        src_out[dest] = static_cast<int32_t>(kLocalE ? block_first + s_e[lp] : s_e[lp]);
    } else {
      keys_out[dest] = k;
      gid_out[dest] = s_gid[lp];
      if (kTwo) e_out[dest] = s_e[lp];
    }
  }
}

// ------------------------------------------------------------- offsets ---

// n_dev: the record count on the device, at most n (else nothing is
// written); null: n records.  K: the sorted keys' type (int64 isect_ids, or
// the sort's 32-bit keys).
template <typename K>
__global__ __launch_bounds__(256) void offset_encode_kernel(const K *__restrict__ ids, int64_t n,
                                                            int64_t n_keys,
                                                            int32_t *__restrict__ out,
                                                            const int64_t *__restrict__ n_dev) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (k >= n_keys) return;
  const int64_t nn = n_dev != nullptr ? *n_dev : n;
  if (nn > n) return;
  int64_t lo = 0, hi = nn;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(ids[mid]) < k)
      lo = mid + 1;
    else
      hi = mid;
  }
  out[k] = static_cast<int32_t>(lo);
}

// The inverse: each of the n sorted records' key from the keys' first
// indices (offsets[0] = 0), the last key whose first index is at most the
// record's.  Empty keys share their successor's first index, so a record
// never lands on one.
__global__ __launch_bounds__(256) void keys_from_offsets_kernel(const int32_t *__restrict__ offsets,
                                                                int64_t n_keys, int64_t n,
                                                                int64_t *__restrict__ keys) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= n) return;
  int64_t lo = 0, hi = n_keys;  // offsets[lo] <= r; offsets[hi] > r (offsets[n_keys] = n)
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(offsets[mid]) <= r)
      lo = mid;
    else
      hi = mid;
  }
  keys[r] = lo;
}

// ----------------------------------------------------------- workspace ---

// Workspace of the sort.  Emission writes keys to k0 and flat ids to gid0
// (the caller's emit_ids array, or g0).  Pass p reads one set and writes the
// other: (k0, gid0) -> (k1, e1, g1) -> (k0, e0, g0) -> ...; the final pass
// writes the outputs instead.
struct SortSpace {
  uint32_t *k0, *e0, *g0, *k1, *e1, *g1, *hist, *hist_scan, *partials;
  const uint32_t *gid0;
  int64_t nblocks, n_hist;
};

// Passes and digit width for keys of `key_bits` bits: the fewest passes of
// at most kMaxPassBits bits, split evenly (e.g. 8 + 7 for 15 bits).  Fewer
// passes move the records fewer times; the scatter keeps each digit's items
// of a block together, so even 1024 digits leave in short contiguous runs.
inline uint32_t sort_passes(uint32_t key_bits) {
  return key_bits == 0 ? 1u : (key_bits + kMaxPassBits - 1) / kMaxPassBits;
}

// Sized for any key width up to end_bit: the passes never exceed
// sort_passes(end_bit), and a pass's digits never exceed
// 2^min(end_bit, kMaxPassBits).
SortSpace carve_sort(Carver &cv, int64_t n, uint32_t end_bit) {
  SortSpace s{};
  const uint32_t passes = sort_passes(end_bit);
  const uint32_t max_digits = 1u << min(end_bit, static_cast<uint32_t>(kMaxPassBits));
  s.nblocks = ceil_div(n, kSortTile);
  s.n_hist = s.nblocks * max_digits;
  s.k0 = cv.take<uint32_t>(n);
  s.g0 = cv.take<uint32_t>(n);
  if (passes > 1) {
    s.k1 = cv.take<uint32_t>(n);
    s.e1 = cv.take<uint32_t>(n);
    s.g1 = cv.take<uint32_t>(n);
    s.e0 = cv.take<uint32_t>(n);
  }
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

int64_t sort_space_bytes(int64_t n, uint32_t end_bit) {
  Carver cv(nullptr);
  carve_sort(cv, n, end_bit);
  return static_cast<int64_t>(cv.used);
}

// Number of bits that hold every key below n_keys.
inline uint32_t key_bits_for(int64_t n_keys) {
  uint32_t b = 0;
  while (b < 32 && (1ll << b) < n_keys) ++b;
  return b;
}

// Launches the scatter instantiation for one pass: digit tables of 256,
// 1024 (a single pass) or 2048 digits, 16-bit key staging when the keys fit.
template <bool kFirst, bool kFinal, bool kTwo>
int launch_scatter_sized(uint32_t bits, bool key16, const uint32_t *kin, const uint32_t *ein,
                         const uint32_t *gin, const int64_t *n_dev, int64_t cap, uint32_t shift,
                         const uint32_t *digit_offsets, uint32_t nb, uint32_t *kout,
                         uint32_t *eout, uint32_t *gout, int64_t *keys64, int32_t *vals32,
                         int32_t *src, int32_t *tile_offsets, uint32_t n_keys,
                         hipStream_t stream) {
#define R2S_SCATTER_SIZED(DB, K16)                                                              \
  radix_scatter_kernel<kFirst, kFinal, kTwo, DB, K16><<<dim3(nb), dim3(kSortThreads), 0,      \
                                                       stream>>>(                             \
      kin, ein, gin, n_dev, cap, shift, bits, digit_offsets, nb, kout, eout, gout, keys64,     \
      vals32, src, tile_offsets, n_keys)
  if (bits <= 8 && key16)
    R2S_SCATTER_SIZED(8, true);
  else if (kFirst && kFinal && bits <= 10 && key16)
    R2S_SCATTER_SIZED(10, true);
  else
    R2S_SCATTER_SIZED(kMaxPassBits, false);
#undef R2S_SCATTER_SIZED
  return check_launch("isect sort pass");
}

int launch_scatter(bool first, bool last, bool two, uint32_t bits, bool key16,
                   const uint32_t *kin, const uint32_t *ein, const uint32_t *gin,
                   const int64_t *n_dev, int64_t cap, uint32_t shift,
                   const uint32_t *digit_offsets, uint32_t nb, uint32_t *kout, uint32_t *eout,
                   uint32_t *gout, int64_t *keys64, int32_t *vals32, int32_t *src,
                   int32_t *tile_offsets, uint32_t n_keys, hipStream_t stream) {
#define R2S_SCATTER_PASS(F, L, T)                                                                \
  return launch_scatter_sized<F, L, T>(bits, key16, kin, ein, gin, n_dev, cap, shift,           \
                                       digit_offsets, nb, kout, eout, gout, keys64, vals32, src, \
                                       tile_offsets, n_keys, stream)
  if (first && last) {
    if (two) R2S_SCATTER_PASS(true, true, true);
    R2S_SCATTER_PASS(true, true, false);
  }
  if (first) {
    if (two) R2S_SCATTER_PASS(true, false, true);
    R2S_SCATTER_PASS(true, false, false);
  }
  if (last) {
    if (two) R2S_SCATTER_PASS(false, true, true);
    R2S_SCATTER_PASS(false, true, false);
  }
  if (two) R2S_SCATTER_PASS(false, false, true);
  R2S_SCATTER_PASS(false, false, false);
#undef R2S_SCATTER_PASS
}

// Sorts the emitted records (s.k0, s.gid0) into the final outputs: *n_dev
// records, at most cap (the size s was carved for).  two: the emission
// index travels too and the final pass writes it to src.  tile_offsets
// (optional): each of the n_keys keys' first index in the sorted list, as
// offset_encode_kernel computes it -- taken from a single pass's digit
// offsets when one pass covers the key, else searched in the sorted keys.
// keys64 may be null when tile_offsets is given: a single pass then writes
// no keys, and the last of several passes leaves 32-bit keys in the
// workspace for the search.
int radix_sort(SortSpace &s, const int64_t *n_dev, int64_t cap, uint32_t key_bits,
               int64_t *keys64, int32_t *vals32, bool two, int32_t *src,
               int32_t *tile_offsets, int64_t n_keys, hipStream_t stream) {
  const uint32_t passes = sort_passes(key_bits);
  const uint32_t pbits = max(1u, (key_bits + passes - 1) / passes);
  const uint32_t nb = static_cast<uint32_t>(s.nblocks);
  const uint32_t *kin = s.k0, *ein = nullptr, *gin = s.gid0;
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t shift = p * pbits;
    const uint32_t bits = key_bits == 0 ? 1u : min(pbits, key_bits - shift);
    const uint32_t digits = 1u << bits;
    const int64_t n_hist = static_cast<int64_t>(nb) * digits;
    radix_hist_kernel<<<dim3(nb), dim3(kSortThreads), 0, stream>>>(kin, n_dev, cap, shift,
                                                                   digits, s.hist, nb);
    R2S_RETURN_IF(device_exclusive_scan<uint32_t, uint32_t>(s.hist, n_hist, s.hist_scan, nullptr,
                                                            s.partials, stream,
                                                            "isect sort scan"));
    const bool first = p == 0, last = p == passes - 1;
    uint32_t *kout = (p % 2 == 0) ? s.k1 : s.k0;
    if (last && keys64 == nullptr && passes == 1) kout = nullptr;
    uint32_t *eout = (p % 2 == 0) ? s.e1 : s.e0;
    uint32_t *gout = (p % 2 == 0) ? s.g1 : s.g0;
    R2S_RETURN_IF(launch_scatter(first, last, two, bits, key_bits <= 16, kin, ein, gin, n_dev,
                                 cap, shift, s.hist_scan, nb, kout, eout, gout, keys64, vals32,
                                 src, passes == 1 ? tile_offsets : nullptr,
                                 static_cast<uint32_t>(n_keys), stream));
    kin = kout;
    ein = eout;
    gin = gout;
  }
  if (tile_offsets != nullptr && passes > 1) {
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_keys, 256)));
    if (keys64 != nullptr)
      offset_encode_kernel<int64_t><<<grid, dim3(256), 0, stream>>>(keys64, cap, n_keys,
                                                                     tile_offsets, n_dev);
    else
      offset_encode_kernel<uint32_t><<<grid, dim3(256), 0, stream>>>(kin, cap, n_keys,
                                                                      tile_offsets, n_dev);
    return check_launch("isect offsets");
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
  count_2d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(M, kScanTile))), dim3(kCountThreads),
                      0, stream>>>(means2d, radii, rect, M, ts, tw, th, counts, partials);
  R2S_RETURN_IF(check_launch(name));
  return device_exclusive_scan_from_sums<int32_t, int64_t>(counts, M, offsets, offsets + M,
                                                           partials, stream, name);
}

template <typename T>
int count_3d_impl(const T *means3d, const int32_t *radii, int64_t N, uint32_t ts, uint32_t n2,
                  uint32_t n1, uint32_t n0, uint32_t z0, uint32_t z1, int32_t *counts,
                  int64_t *offsets, void *ws, size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles_3d";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size N=%lld", name, (long long)N);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * n1 * n0 <= 0xffffffffull,
              "%s: n_tiles exceeds 32 bits", name);
  R2S_REQUIRE(z0 <= z1 && z1 <= n0, "%s: brick layers [%u, %u) outside [0, %u)", name, z0,
              z1, n0);
  R2S_REQUIRE(offsets != nullptr, "%s: null offsets", name);
  hipStream_t stream = as_stream(st);
  if (N == 0) return device_fill<int64_t>(offsets, 1, 0, stream, name);
  R2S_REQUIRE(means3d && radii && counts, "%s: null pointer", name);
  R2S_RETURN_IF(check_workspace(ws, ws_bytes, count_space_bytes(N), name));
  Carver cv(ws);
  int64_t *partials = cv.take<int64_t>(scan_partials_count(N));
  count_3d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, kScanTile))), dim3(kCountThreads),
                      0, stream>>>(means3d, radii, N, ts, n2, n1, n0, z0, z1, counts, partials);
  R2S_RETURN_IF(check_launch(name));
  return device_exclusive_scan_from_sums<int32_t, int64_t>(counts, N, offsets, offsets + N,
                                                           partials, stream, name);
}

int check_sort_args(int64_t n_isects, uint32_t end_bit, int64_t n_keys, void *ws,
                    size_t ws_bytes, int64_t *keys, int32_t *vals, const int32_t *tile_offsets,
                    const char *name) {
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
  R2S_REQUIRE(vals, "%s: null flatten_ids", name);
  R2S_REQUIRE(keys || tile_offsets, "%s: null isect_ids without tile_offsets", name);
  return check_workspace(ws, ws_bytes, sort_space_bytes(n_isects, end_bit), name);
}

template <typename T>
int emit_sort_2d_impl(const T *means2d, const int32_t *radii, int rect, int64_t C, int64_t N,
                      uint32_t ts, uint32_t tw, uint32_t th, const int64_t *offsets,
                      int64_t n_isects, uint32_t end_bit, int64_t *keys, int32_t *vals,
                      int32_t *emit_ids, int32_t *isect_src, int32_t *tile_offsets, void *ws,
                      size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles";
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size", name);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_RETURN_IF(check_sort_args(n_isects, end_bit, C * tw * th, ws, ws_bytes, keys, vals,
                                tile_offsets, name));
  const int64_t n_keys = C * tw * th;
  if (n_isects == 0)
    return tile_offsets == nullptr || n_keys == 0
               ? R2S_OK
               : device_fill<int32_t>(tile_offsets, n_keys, 0, as_stream(st), name);
  R2S_REQUIRE(means2d && radii && offsets, "%s: null pointer", name);
  hipStream_t stream = as_stream(st);
  Carver cv(ws);
  SortSpace s = carve_sort(cv, n_isects, end_bit);
  R2S_REQUIRE((emit_ids == nullptr) == (isect_src == nullptr),
              "%s: emit_ids and isect_src must be given together", name);
  uint32_t *gids = emit_ids != nullptr ? reinterpret_cast<uint32_t *>(emit_ids) : s.g0;
  s.gid0 = gids;
  const int64_t M = C * N;
  emit_2d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(M, 256))), dim3(256), 0, stream>>>(
      means2d, radii, rect, M, N, ts, tw, th, offsets, n_isects, s.k0, gids);
  R2S_RETURN_IF(check_launch(name));
  return radix_sort(s, offsets + M, n_isects, key_bits_for(n_keys), keys, vals,
                    emit_ids != nullptr, isect_src, tile_offsets, n_keys, stream);
}

template <typename T>
int emit_sort_3d_impl(const T *means3d, const int32_t *radii, int64_t N, uint32_t ts,
                      uint32_t n2, uint32_t n1, uint32_t n0, uint32_t z0, uint32_t z1,
                      const int64_t *offsets, int64_t n_isects, uint32_t end_bit, int64_t *keys,
                      int32_t *vals, int32_t *emit_ids, int32_t *isect_src,
                      int32_t *tile_offsets, void *ws, size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles_3d";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size", name);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_REQUIRE(z0 <= z1 && z1 <= n0, "%s: brick layers [%u, %u) outside [0, %u)", name, z0,
              z1, n0);
  const int64_t n_keys = static_cast<int64_t>(n2) * n1 * (z1 - z0);
  R2S_RETURN_IF(check_sort_args(n_isects, end_bit, n_keys, ws, ws_bytes, keys, vals,
                                tile_offsets, name));
  if (n_isects == 0)
    return tile_offsets == nullptr || n_keys == 0
               ? R2S_OK
               : device_fill<int32_t>(tile_offsets, n_keys, 0, as_stream(st), name);
  R2S_REQUIRE(means3d && radii && offsets, "%s: null pointer", name);
  hipStream_t stream = as_stream(st);
  Carver cv(ws);
  SortSpace s = carve_sort(cv, n_isects, end_bit);
  R2S_REQUIRE((emit_ids == nullptr) == (isect_src == nullptr),
              "%s: emit_ids and isect_src must be given together", name);
  uint32_t *gids = emit_ids != nullptr ? reinterpret_cast<uint32_t *>(emit_ids) : s.g0;
  s.gid0 = gids;
  emit_3d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0, stream>>>(
      means3d, radii, N, ts, n2, n1, n0, z0, z1, offsets, n_isects, s.k0, gids);
  R2S_RETURN_IF(check_launch(name));
  return radix_sort(s, offsets + N, n_isects, key_bits_for(n_keys), keys, vals,
                    emit_ids != nullptr, isect_src, tile_offsets, n_keys, stream);
}

template <typename T>
int layer_counts_3d_impl(const T *means3d, const int32_t *radii, int64_t N, uint32_t ts,
                         uint32_t n2, uint32_t n1, uint32_t n0, int64_t *counts, void *ws,
                         size_t ws_bytes, r2s_stream_t st) {
  clear_error();
  const char *name = "isect_tiles_3d (layer counts)";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size N=%lld", name, (long long)N);
  R2S_REQUIRE(ts > 0, "%s: tile_size must be positive", name);
  R2S_REQUIRE(n0 >= 1 && static_cast<uint64_t>(n2) * n1 * n0 <= 0xffffffffull,
              "%s: bad brick grid", name);
  R2S_REQUIRE(counts != nullptr, "%s: null counts", name);
  hipStream_t stream = as_stream(st);
  if (N == 0) return device_fill<int64_t>(counts, n0, 0, stream, name);
  R2S_REQUIRE(means3d && radii, "%s: null pointer", name);
  R2S_RETURN_IF(check_workspace(ws, ws_bytes, (static_cast<int64_t>(n0) + 1) * 8, name));
  auto *diff = static_cast<unsigned long long *>(ws);
  R2S_RETURN_IF(device_fill<int64_t>(reinterpret_cast<int64_t *>(diff), n0 + 1, 0, stream,
                                     name));
  layer_diff_3d_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0,
                            stream>>>(means3d, radii, N, ts, n2, n1, n0, diff);
  R2S_RETURN_IF(check_launch(name));
  layer_prefix_kernel<<<dim3(1), dim3(1), 0, stream>>>(diff, n0, counts);
  return check_launch(name);
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_isect_workspace_bytes(int64_t n_items, int64_t n_isects, uint32_t end_bit) {
  const int64_t a = n_items > 0 ? r2s::count_space_bytes(n_items) : 0;
  const int64_t b = n_isects > 0 ? r2s::sort_space_bytes(n_isects, end_bit) : 0;
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
                                   int32_t *emit_ids, int32_t *isect_src,                     \
                                   int32_t *tile_offsets, void *ws, size_t ws_bytes,          \
                                   r2s_stream_t st) {                                         \
    return r2s::emit_sort_2d_impl<T>(means2d, radii, rect, C, N, ts, tw, th, offsets,         \
                                     n_isects, end_bit, keys, vals, emit_ids, isect_src,      \
                                     tile_offsets, ws, ws_bytes, st);                         \
  }                                                                                           \
  int r2s_isect_count_3d_##SUF(const T *means3d, const int32_t *radii, int64_t N,            \
                               uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,            \
                               int32_t *counts, int64_t *offsets, void *ws, size_t ws_bytes,  \
                               r2s_stream_t st) {                                             \
    return r2s::count_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, 0u, n0, counts, offsets,  \
                                 ws, ws_bytes, st);                                           \
  }                                                                                           \
  int r2s_isect_emit_sort_3d_##SUF(const T *means3d, const int32_t *radii, int64_t N,        \
                                   uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,        \
                                   const int64_t *offsets, int64_t n_isects,                  \
                                   uint32_t end_bit, int64_t *keys, int32_t *vals,            \
                                   int32_t *emit_ids, int32_t *isect_src,                     \
                                   int32_t *tile_offsets, void *ws, size_t ws_bytes,          \
                                   r2s_stream_t st) {                                         \
    return r2s::emit_sort_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, 0u, n0,               \
                                     offsets, n_isects, end_bit, keys, vals, emit_ids,        \
                                     isect_src, tile_offsets, ws, ws_bytes, st);              \
  }                                                                                           \
  int r2s_isect_layer_counts_3d_##SUF(const T *means3d, const int32_t *radii, int64_t N,     \
                                      uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,     \
                                      int64_t *counts, void *ws, size_t ws_bytes,             \
                                      r2s_stream_t st) {                                      \
    return r2s::layer_counts_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, counts, ws,        \
                                        ws_bytes, st);                                        \
  }                                                                                           \
  int r2s_isect_count_3d_slab_##SUF(const T *means3d, const int32_t *radii, int64_t N,       \
                                    uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,       \
                                    uint32_t z0, uint32_t z1, int32_t *counts,                \
                                    int64_t *offsets, void *ws, size_t ws_bytes,              \
                                    r2s_stream_t st) {                                        \
    return r2s::count_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, z0, z1, counts, offsets,  \
                                 ws, ws_bytes, st);                                           \
  }                                                                                           \
  int r2s_isect_emit_sort_3d_slab_##SUF(                                                      \
      const T *means3d, const int32_t *radii, int64_t N, uint32_t ts, uint32_t n2,            \
      uint32_t n1, uint32_t n0, uint32_t z0, uint32_t z1, const int64_t *offsets,             \
      int64_t n_isects, uint32_t end_bit, int64_t *keys, int32_t *vals, int32_t *emit_ids,    \
      int32_t *isect_src, int32_t *tile_offsets, void *ws, size_t ws_bytes, r2s_stream_t st) { \
    return r2s::emit_sort_3d_impl<T>(means3d, radii, N, ts, n2, n1, n0, z0, z1, offsets,      \
                                     n_isects, end_bit, keys, vals, emit_ids, isect_src,      \
                                     tile_offsets, ws, ws_bytes, st);                         \
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
  r2s::offset_encode_kernel<int64_t>
      <<<dim3(static_cast<uint32_t>(r2s::ceil_div(n_keys, 256))), dim3(256), 0, stream>>>(
          ids, n_isects, n_keys, out, nullptr);
  return r2s::check_launch("isect_offset_encode");
}

int r2s_isect_keys_from_offsets(const int32_t *tile_offsets, int64_t n_keys, int64_t n_isects,
                                int64_t *isect_ids, r2s_stream_t st) {
  r2s::clear_error();
  const char *name = "isect_keys_from_offsets";
  R2S_REQUIRE(n_isects >= 0 && n_keys >= 0, "%s: negative size", name);
  if (n_isects == 0) return R2S_OK;
  if (n_isects > r2s::kInt32Max) {
    r2s::set_error("%s: %lld records exceed the int32 offset range", name, (long long)n_isects);
    return R2S_ERANGE;
  }
  R2S_REQUIRE(n_keys >= 1, "%s: records without keys", name);
  R2S_REQUIRE(tile_offsets != nullptr && isect_ids != nullptr, "%s: null pointer", name);
  r2s::keys_from_offsets_kernel<<<dim3(static_cast<uint32_t>(r2s::ceil_div(n_isects, 256))),
                                  dim3(256), 0, r2s::as_stream(st)>>>(tile_offsets, n_keys,
                                                                      n_isects, isect_ids);
  return r2s::check_launch(name);
}

}  // extern "C"
