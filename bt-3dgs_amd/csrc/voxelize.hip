// Brick-tiled voxelizer: volume = per voxel sum over its brick's Gaussian
// list of opacity * exp(-sigma), sigma = 1/2 d^T conic d, skipping sigma < 0
// and |alpha| < 1e-6 (r2splat/cuda/csrc/VoxelizeToVoxelsFwd.cu:69-221), and
// its VJP (VoxelizeToVoxelsBwd.cu:71-441).
//
// sigma is evaluated along x-rows of a brick: with dy, dz fixed per row,
//   sigma log2(e) = (h0 dx + B) dx + C,  h0 = p00 log2(e) / 2,
// two FMAs per voxel and one v_exp_f32 for exp(-sigma) = 2^-(sigma log2 e).
//
// Forward: one workgroup per brick; each thread owns R consecutive voxels of
// one x-row (R = ts for ts = 8, 16; R = 1 otherwise) and sums the brick's list
// in list order, as the reference does, so the result is deterministic.
// Records are staged in LDS in batches with their conics pre-scaled and read
// as broadcasts.
//
// Backward: one lane per record of the sorted list, so a wave takes 64
// consecutive records (nearly always of one brick) and the work is balanced
// whatever the list lengths.  All lanes walk the brick-local rows together,
// skipping every slice and row that no lane's alpha-test ellipsoid reaches
// (r2s_cull.h, wave ballots); a lane loads the upstream-gradient row of its
// own brick (lanes of one brick share the cache lines).  Per row a lane accumulates
// the moments s_k = sum(w dx^k), k = 0..2, of w = v exp(-sigma) over passing
// voxels, and per record the ten sums
//   T_k = sum s_k,  Y0 = sum dy s0, Z0 = sum dz s0, Y1 = sum dy s1,
//   Z1 = sum dz s1, YY = sum dy^2 s0, YZ = sum dy dz s0, ZZ = sum dz^2 s0,
// from which the ten partials follow.  They go out through float atomics
// (one-pass form) or as the record's row of a table that r2s_rows.h reduces
// per Gaussian (two-pass form).  The two reference backward variants (per
// voxel, per Gaussian) compute the same sums and share this kernel.
#include "r2s_common.h"
#include "r2s_cull.h"
#include "r2s_rows.h"
#include "r2s_scan.h"

namespace r2s {
namespace {

constexpr double kThr3 = 1e-6;
constexpr int kBwdThreads = 256;
constexpr uint32_t kFwdBatch = 256;

template <typename T>
struct Vec;
template <>
struct Vec<float> {
  using v2 = float2;
  using v4 = float4;
};
template <>
struct Vec<double> {
  using v2 = double2;
  using v4 = double4;
};

struct Brick {
  int oi, oj, ok;  // origin (dim0, dim1, dim2)
  int ni, nj, nk;  // extent inside the volume
};

__device__ __forceinline__ Brick brick_of(uint32_t key, uint32_t n2, uint32_t n1, uint32_t ts,
                                          uint32_t D2, uint32_t D1, uint32_t D0) {
  const uint32_t b0 = key / (n1 * n2), rem = key - b0 * (n1 * n2);
  const uint32_t b1 = rem / n2, b2 = rem - b1 * n2;
  Brick b;
  b.oi = static_cast<int>(b0 * ts);
  b.oj = static_cast<int>(b1 * ts);
  b.ok = static_cast<int>(b2 * ts);
  b.ni = static_cast<int>(min(ts, D0 - b0 * ts));
  b.nj = static_cast<int>(min(ts, D1 - b1 * ts));
  b.nk = static_cast<int>(min(ts, D2 - b2 * ts));
  return b;
}

// Pre-scaled conic: sigma log2(e) = (h0 dx + h1 dy + h2 dz) dx
//                                  + (h3 dy + h4 dz) dy + h5 dz^2.
template <typename T>
__device__ __forceinline__ void scaled_conic(const T q[6], T h[6]) {
  const T l = static_cast<T>(kLog2e), hl = static_cast<T>(0.5 * kLog2e);
  h[0] = hl * q[0];
  h[1] = l * q[1];
  h[2] = l * q[2];
  h[3] = hl * q[3];
  h[4] = l * q[4];
  h[5] = hl * q[5];
}

template <typename T, int R>
__global__ __launch_bounds__(1024) void voxel_fwd_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int32_t *__restrict__ flatten_ids,
    int64_t n_isects, uint32_t n_keys, uint32_t koff, int64_t N, uint32_t D2, uint32_t D1,
    uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, T *__restrict__ volume) {
  using V4 = typename Vec<T>::v4;
  extern __shared__ double smem_raw[];
  const uint32_t nt = blockDim.x;
  const uint32_t nb = min(nt, kFwdBatch);  // records staged per batch
  // Per staged record: {mx, my, mz, o}, {h0, h1, h2, h3}, {h4, h5, limit bits, 0}.
  V4 *s_rec = reinterpret_cast<V4 *>(smem_raw);

  const uint32_t key = xcd_swizzle(blockIdx.x, n_keys);  // in the lists (koff: the grid's)
  const Brick b = brick_of(key + koff, n2, n1, ts, D2, D1, D0);
  const uint32_t tid = threadIdx.x;
  const uint32_t per_row = ts / R;
  const int lk0 = static_cast<int>((tid % per_row) * R);
  const int lj = static_cast<int>((tid / per_row) % ts);
  const int li = static_cast<int>(tid / (per_row * ts));
  const T half = static_cast<T>(0.5);
  const T py = static_cast<T>(b.oj + lj) + half;
  const T pz = static_cast<T>(b.oi + li) + half;
  const T px0 = static_cast<T>(b.ok + lk0) + half;

  const int64_t start = tile_offsets[key];
  const int64_t end = (key == n_keys - 1) ? n_isects : static_cast<int64_t>(tile_offsets[key + 1]);
  T acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0;
  for (int64_t base = start; base < end; base += nb) {
    __syncthreads();
    const int64_t idx = base + tid;
    if (tid < nb && idx < end) {
      int64_t g = flatten_ids[idx];
      V4 mo, h0, h1;
      if (g >= 0 && g < N) {
        T q[6], h[6];
#pragma unroll
        for (int c = 0; c < 6; ++c) q[c] = conics[6 * g + c];
        scaled_conic(q, h);
        mo.x = means3d[3 * g];
        mo.y = means3d[3 * g + 1];
        mo.z = means3d[3 * g + 2];
        mo.w = opac[g];
        h0.x = h[0];
        h0.y = h[1];
        h0.z = h[2];
        h0.w = h[3];
        h1.x = h[4];
        h1.y = h[5];
        // The alpha test's limit on the bits of sl (alpha_limit), kept in h1.z.
        bool fin = isfinite(mo.x) && isfinite(mo.y) && isfinite(mo.z);
#pragma unroll
        for (int c = 0; c < 6; ++c) fin = fin && isfinite(h[c]);
        h1.z = limit_as_value(alpha_limit(mo.w, fin, kThr3));
      } else {  // never passes
        mo.x = mo.y = mo.z = mo.w = 0;
        h0.x = h0.y = h0.z = h0.w = 0;
        h1.x = h1.y = 0;
        h1.z = limit_as_value(static_cast<typename Bits<T>::type>(0));
      }
      h1.w = 0;
      s_rec[3 * tid] = mo;
      s_rec[3 * tid + 1] = h0;
      s_rec[3 * tid + 2] = h1;
    }
    __syncthreads();
    const int cnt = static_cast<int>(min(static_cast<int64_t>(nb), end - base));
    for (int t = 0; t < cnt; ++t) {
      const V4 mo = s_rec[3 * t];
      const V4 h0 = s_rec[3 * t + 1];
      const V4 h1 = s_rec[3 * t + 2];
      const typename Bits<T>::type lim = bits_of(h1.z);
      const T dy = py - mo.y, dz = pz - mo.z;
      const T B = h0.y * dy + h0.z * dz;
      const T C = (h0.w * dy + h1.x * dz) * dy + h1.y * dz * dz;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const T dx = (px0 + static_cast<T>(r)) - mo.x;
        const T sl = (h0.x * dx + B) * dx + C;
        add_passing(sl, lim, mo.w, acc[r]);
      }
    }
  }
  if (li < b.ni && lj < b.nj) {
    T *out = volume + static_cast<int64_t>(b.oi + li) * D1 * D2 +
             static_cast<int64_t>(b.oj + lj) * D2 + (b.ok + lk0);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (lk0 + r < b.nk) out[r] = acc[r];
  }
}

// One backward record in registers.
template <typename T>
struct BwdRecord {
  bool live;     // a valid record whose voxels can pass the alpha test
  T m[3], q[6], h[6], o;
  typename Bits<T>::type lim;  // the alpha test on the bits of sl (alpha_limit)
  Cull3<T> cu;
  int i0, i1;    // slice range (all slices when !cu.ok)
};

// A record's geometry, opacity and alpha limit; every slice of the brick in
// range (no culling).
template <typename T>
__device__ __forceinline__ void load_bwd_record_plain(const T *__restrict__ means3d,
                                                      const T *__restrict__ conics,
                                                      const T *__restrict__ opac, int64_t g,
                                                      int64_t N, bool in_list, const Brick &b,
                                                      BwdRecord<T> &rec) {
  rec.live = in_list && g >= 0 && g < N;
  rec.o = rec.live ? opac[g] : static_cast<T>(0);
  // |alpha| <= |o| for sigma >= 0: nothing passes (non-finite o stays live).
  if (fabs(rec.o) < static_cast<T>(kThr3)) rec.live = false;
  rec.cu.ok = false;
  if (!rec.live) {
    rec.o = 0;
    rec.lim = 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) rec.m[c] = 0;
#pragma unroll
    for (int c = 0; c < 6; ++c) rec.q[c] = rec.h[c] = 0;
    rec.i0 = 0;
    rec.i1 = -1;
    return;
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) rec.m[c] = means3d[3 * g + c];
#pragma unroll
  for (int c = 0; c < 6; ++c) rec.q[c] = conics[6 * g + c];
  scaled_conic(rec.q, rec.h);
  bool fin = true;
#pragma unroll
  for (int c = 0; c < 3; ++c) fin = fin && isfinite(rec.m[c]);
#pragma unroll
  for (int c = 0; c < 6; ++c) fin = fin && isfinite(rec.h[c]);
  rec.lim = alpha_limit(rec.o, fin, kThr3);
  rec.i0 = b.oi;
  rec.i1 = b.oi + b.ni - 1;
}

// As load_bwd_record_plain, with the culling setup and the slice range of
// the record's alpha-test ellipsoid (a record reaching no slice is dead).
template <typename T>
__device__ __forceinline__ void load_bwd_record(const T *__restrict__ means3d,
                                                const T *__restrict__ conics,
                                                const T *__restrict__ opac, int64_t g, int64_t N,
                                                bool in_list, const Brick &b, BwdRecord<T> &rec) {
  load_bwd_record_plain(means3d, conics, opac, g, N, in_list, b, rec);
  if (!rec.live) return;
  rec.cu = cull3_setup(rec.q, fabs(rec.o), kThr3);
  if (rec.cu.ok &&
      !index_range<T>(rec.m[2], -rec.cu.hz, rec.cu.hz, b.oi, b.oi + b.ni - 1, rec.i0, rec.i1))
    rec.live = false;
}

// Moments of one brick row for one record: s0 = sum w, s1 = sum w dx,
// s2 = sum w dx^2 over the row's passing voxels (w = v exp(-sigma)).  vv
// holds the row's upstream gradient (zero beyond the volume).  kGuard: also
// exclude columns k >= nk explicitly -- needed only for records whose sigma
// may be NaN (non-finite geometry passes the alpha test there), for which
// v = 0 would not make w = 0.
template <typename T, int R, bool kExact, bool kGuard>
__device__ __forceinline__ void voxel_row(const BwdRecord<T> &rec, const T (&vv)[R], T dx0,
                                          int nk, int nts, T B, T C, T &s0, T &s1, T &s2) {
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (!kExact && k >= nts) break;
    const T dx = dx0 + static_cast<T>(k);
    const T sl = (rec.h[0] * dx + B) * dx + C;
    const T e = neg_exp2(sl);
    bool skip = !alpha_pass(sl, rec.lim);
    if (kGuard) skip = skip || k >= nk;
    const T p = vv[k] * e;  // unconditional, not a branch around the load and exp
    const T w = skip ? static_cast<T>(0) : p;
    s0 += w;
    const T wx = w * dx;
    s1 += wx;
    s2 += wx * dx;
  }
}

// Slice range of one record's brick rows: rows j0..j1 of slice dz whose
// voxels (columns dx0 .. dx0 + nk - 1 as offsets from the mean) the
// ellipsoid reaches; empty (j1 < j0) when none.  In the slice, the reached
// part of the ellipse is its intersection with the brick's x-band, a convex
// set, so its rows are one range: the top is the top of the vertical chord
// at the band point nearest the ellipse's topmost point (chord tops are a
// concave function of x), the bottom likewise; every term is a completed
// square, so nothing cancels.  The band is widened by kCullMargin and the
// rows are taken with index_range's margin.
template <typename T>
__device__ __forceinline__ void slice_rows(const BwdRecord<T> &rec, const Brick &b, bool in_slice,
                                           T dz, T dx0, int &j0, int &j1) {
  j0 = b.oj;
  j1 = b.oj + b.nj - 1;
  if (!in_slice) {
    j1 = j0 - 1;
    return;
  }
  if (!rec.cu.ok) return;  // every row
  const Cull3<T> &c = rec.cu;
  const T half = static_cast<T>(0.5), two = static_cast<T>(2);
  const T m = static_cast<T>(kCullMargin);
  const T bud = c.s - half * c.c3 * dz * dz;
  const T ye = -c.ky * dz;
  const T xe = -(c.kx * ye + c.kz * dz);
  const T hy = cull_sqrt(fmax(two * bud * c.inv_a2, static_cast<T>(0)));
  const T ulo = (dx0 - m) - xe;
  const T uhi = (dx0 + static_cast<T>(b.nk - 1) + m) - xe;
  // Topmost point of the ellipse at u = -kx hy, bottommost at +kx hy.
  const T ut = fmin(fmax(-c.kx * hy, ulo), uhi);
  const T ub = fmin(fmax(c.kx * hy, ulo), uhi);
  const T rt = bud - half * c.e11 * ut * ut;
  const T rb = bud - half * c.e11 * ub * ub;
  if (!(bud >= static_cast<T>(0)) || !(rt >= static_cast<T>(0))) {
    j1 = j0 - 1;  // the slice, or the band, misses the ellipse
    return;
  }
  const T top = ye + (cull_sqrt(two * rt * c.inv_p11) - c.r11 * ut);
  const T bot = ye - (cull_sqrt(fmax(two * rb * c.inv_p11, static_cast<T>(0))) + c.r11 * ub);
  if (!index_range<T>(rec.m[1], bot, top, b.oj, b.oj + b.nj - 1, j0, j1)) j1 = j0 - 1;
}

// The rows of a brick of size 8 that one record reaches, as a 64-bit mask:
// bit 8 * slice + row (brick-local).
template <typename T>
__device__ __forceinline__ uint64_t reach_mask(const BwdRecord<T> &rec, const Brick &b, T dx0) {
  const T half = static_cast<T>(0.5);
  uint64_t reach = 0;
#pragma unroll 1
  for (int li = 0; li < 8; ++li) {
    const int i = b.oi + li;
    const bool in_slice = rec.live && li < b.ni && i >= rec.i0 && i <= rec.i1;
    const T dz = (static_cast<T>(i) + half) - rec.m[2];
    int j0, j1;
    slice_rows(rec, b, in_slice, dz, dx0, j0, j1);
    const uint32_t c = j1 >= j0 ? static_cast<uint32_t>(j1 - j0 + 1) : 0u;  // rows j0 - oj ..
    const uint32_t run = c >= 8u ? 0xFFu : ((1u << c) - 1u);
    reach |= static_cast<uint64_t>((run << ((j0 - b.oj) & 7)) & 0xFFu) << (8 * li);
  }
  return reach;
}

// Forward at brick size 8 with culled rows.  S waves per brick; lane =
// x-row (slice lane / 8, row lane % 8), its 8 voxels in registers.  Wave w
// takes the batches of 64 records w, w + S, w + 2S, ... of the brick's list.
// Per batch, each lane loads one record and the rows it reaches
// (reach_mask); a 64 x 64 bit transpose hands each row's lane the set of
// batch records that reach that row; each lane then walks its own set in
// list order, so a record costs a row only where it can pass the alpha
// test, and the rows a record does not reach would only add exact zeros.
// With S = 1 every voxel sums its records in list order (the volume equals
// voxel_fwd_kernel's bit for bit); with S > 1 (long lists: the host picks S
// from the mean list length) the S partial bricks are added in wave order
// through LDS, a fixed order.  reach_out (optional): each record's reach
// mask, stored at its list position for a backward over the same lists.
template <typename T, int S>
__global__ __launch_bounds__(64 * S) void voxel_fwd_reach_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int32_t *__restrict__ flatten_ids,
    int64_t n_isects, uint32_t n_keys, uint32_t koff, int64_t N, uint32_t D2, uint32_t D1,
    uint32_t D0, uint32_t n2, uint32_t n1, T *__restrict__ volume,
    uint64_t *__restrict__ reach_out) {
  constexpr int R = 8;
  using V4 = typename Vec<T>::v4;
  // Per staged record {my, mz, o, h0}, {h1, h2, h3, h4}, {h5, limit bits,
  // 0, 0} and its eight column offsets dx_k = (x_k + 1/2) - mx, the same for
  // every row of the brick: five vector reads per use; the 20-word stride
  // spreads 8 consecutive records over all banks.
  __shared__ V4 s_rec[S][64][5];
  __shared__ T s_part[S > 1 ? S - 1 : 1][R][64];
  const uint32_t key = xcd_swizzle(blockIdx.x, n_keys);  // in the lists (koff: the grid's)
  const Brick b = brick_of(key + koff, n2, n1, R, D2, D1, D0);
  const int lane = static_cast<int>(lane_id());
  const int w = S > 1 ? static_cast<int>(wave_index()) : 0;
  const int li = lane >> 3, lj = lane & 7;
  const T half = static_cast<T>(0.5);
  const T py = static_cast<T>(b.oj + lj) + half;
  const T pz = static_cast<T>(b.oi + li) + half;
  const T px0 = static_cast<T>(b.ok) + half;
  const int64_t start = tile_offsets[key];
  const int64_t end = (key == n_keys - 1) ? n_isects : static_cast<int64_t>(tile_offsets[key + 1]);
  T acc[R];
#pragma unroll
  for (int k = 0; k < R; ++k) acc[k] = 0;
  for (int64_t base = start + 64 * w; base < end; base += 64 * S) {
    const int64_t idx = base + lane;
    const bool in = idx < end;
    const int64_t g = in ? static_cast<int64_t>(flatten_ids[idx]) : -1;
    BwdRecord<T> rec;
    load_bwd_record(means3d, conics, opac, g, N, in, b, rec);
    const uint64_t reach = rec.live ? reach_mask(rec, b, px0 - rec.m[0]) : 0ull;
    if (reach_out != nullptr && in) reach_out[idx] = reach;
    V4 a, hq, hr, d0, d1;
    a.x = rec.m[1];
    a.y = rec.m[2];
    a.z = rec.o;
    a.w = rec.h[0];
    hq.x = rec.h[1];
    hq.y = rec.h[2];
    hq.z = rec.h[3];
    hq.w = rec.h[4];
    hr.x = rec.h[5];
    hr.y = limit_as_value(rec.lim);
    hr.z = 0;
    hr.w = 0;
    // The column offsets from the voxel centres x_k + 1/2 = px0 + k (exact),
    // computed once per record instead of once per walked row.
    T dxs[R];
#pragma unroll
    for (int k = 0; k < R; ++k) dxs[k] = (px0 + static_cast<T>(k)) - rec.m[0];
    d0.x = dxs[0];
    d0.y = dxs[1];
    d0.z = dxs[2];
    d0.w = dxs[3];
    d1.x = dxs[4];
    d1.y = dxs[5];
    d1.z = dxs[6];
    d1.w = dxs[7];
    // The wave's LDS operations complete in order: the fences keep the
    // compiler from moving this batch's writes above the previous batch's
    // reads, or the reads below above the writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    s_rec[w][lane][0] = a;
    s_rec[w][lane][1] = hq;
    s_rec[w][lane][2] = hr;
    s_rec[w][lane][3] = d0;
    s_rec[w][lane][4] = d1;
    // Bit t of lane r's set: batch record t reaches row r.
    uint64_t mine = transpose_bits64(reach, static_cast<uint32_t>(lane));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    while (mine != 0ull) {
      const int t = static_cast<int>(__builtin_ctzll(mine));
      mine &= mine - 1ull;
      const V4 qa = s_rec[w][t][0], qh = s_rec[w][t][1], qr = s_rec[w][t][2];
      const V4 q0 = s_rec[w][t][3], q1 = s_rec[w][t][4];
      const T dxs[R] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      const typename Bits<T>::type lim = bits_of(qr.y);
      const T dy = py - qa.x, dz = pz - qa.y;
      const T B = qh.x * dy + qh.y * dz;
      const T C = (qh.z * dy + qh.w * dz) * dy + qr.x * dz * dz;
#pragma unroll
      for (int k = 0; k < R; ++k) {
        const T dx = dxs[k];
        const T sl = (qa.w * dx + B) * dx + C;
        add_passing(sl, lim, qa.z, acc[k]);
      }
    }
  }
  if constexpr (S > 1) {
    // Waves 1 .. S-1 hand their partial bricks to wave 0, which adds them in
    // wave order.
    if (w > 0) {
#pragma unroll
      for (int k = 0; k < R; ++k) s_part[w - 1][k][lane] = acc[k];
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int ww = 0; ww < S - 1; ++ww) {
#pragma unroll
      for (int k = 0; k < R; ++k) acc[k] += s_part[ww][k][lane];
    }
  }
  if (li < b.ni && lj < b.nj) {
    T *out = volume + static_cast<int64_t>(b.oi + li) * D1 * D2 +
             static_cast<int64_t>(b.oj + lj) * D2 + b.ok;
#pragma unroll
    for (int k = 0; k < R; ++k)
      if (k < b.nk) out[k] = acc[k];
  }
}

// The whole brick of one record when every brick of the wave lies inside
// the volume (no column guard).  The column offsets dx_k are the same on
// every row and the column sums W_k = sum over rows of w accumulate per
// column, so T0, T1, T2 follow from W_k once per record and each voxel adds
// three sums (W_k, s0, s1) instead of four.  Rows the record does not reach
// test against a zero limit (every voxel fails), so the upstream
// gradient is loaded without masks.
// kReach: the slices' row ranges come from `reach` (bit 8 * slice + row of
// the reached rows, as voxel_bwd_chunk_kernel computes them) instead of
// slice_rows.
template <typename T, int R, bool kReach = false>
__device__ __forceinline__ void voxel_brick_full(const BwdRecord<T> &rec, const Brick &b,
                                                 const T *__restrict__ v_vol, int64_t plane,
                                                 uint32_t D2, T dx0, T &T0, T &T1, T &T2, T &Y0,
                                                 T &Z0, T &Y1, T &Z1, T &YY, T &YZ, T &ZZ,
                                                 uint64_t reach = 0) {
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n;
  T dxk[R], wk[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    dxk[k] = dx0 + static_cast<T>(k);
    wk[k] = 0;
  }
  const T half = static_cast<T>(0.5);
#pragma unroll 1
  for (int li = 0; li < R; ++li) {
    const int i = b.oi + li;
    const bool in_slice = rec.live && i >= rec.i0 && i <= rec.i1;
    if (ballot(in_slice) == 0) continue;
    const T dz = (static_cast<T>(i) + half) - rec.m[2];
    int j0, j1;
    if constexpr (kReach) {
      const uint32_t byte = static_cast<uint32_t>(reach >> (8 * li)) & 0xFFu;
      j0 = b.oj + static_cast<int>(__builtin_ctz(byte | 0x100u));
      j1 = j0 + __popc(byte) - 1;
    } else {
      slice_rows(rec, b, in_slice, dz, dx0, j0, j1);
    }
    const T h4dz = rec.h[4] * dz, h5dzz = rec.h[5] * dz * dz, Bz = rec.h[2] * dz;
    const T *__restrict__ vslice = v_vol + static_cast<int64_t>(i) * plane + b.ok;
#pragma unroll 1
    for (int lj = 0; lj < R; ++lj) {
      const int j = b.oj + lj;
      const bool in_row = j >= j0 && j <= j1;
      if (ballot(in_row) == 0) continue;
      const T dy = (static_cast<T>(j) + half) - rec.m[1];
      const T B = fma(rec.h[1], dy, Bz);
      const T C = fma(fma(rec.h[3], dy, h4dz), dy, h5dzz);
      const typename Bits<T>::type lim = in_row ? rec.lim : 0;
      const T *__restrict__ vrow = vslice + static_cast<int64_t>(j) * D2;
      T vv[R];
#pragma unroll
      for (int q = 0; q < R / kq; ++q)
        *reinterpret_cast<Q *>(vv + q * kq) = *reinterpret_cast<const Q *>(vrow + q * kq);
      T s0 = 0, s1 = 0;
#pragma unroll
      for (int k = 0; k < R; ++k) {
        // Explicit FMAs keep the row-invariant products of dx_k from being
        // hoisted into extra registers.
        const T dx = dxk[k];
        const T sl = fma(fma(rec.h[0], dx, B), dx, C);
        const T e = neg_exp2(sl);
        const T p = vv[k] * e;  // unconditional, not a branch around the load and exp
        const T w = alpha_pass(sl, lim) ? p : static_cast<T>(0);
        wk[k] += w;
        s0 += w;
        s1 = fma(w, dx, s1);
      }
      const T dys0 = dy * s0, dzs0 = dz * s0;
      Y0 += dys0;
      Z0 += dzs0;
      YY += dy * dys0;
      YZ += dz * dys0;
      ZZ += dz * dzs0;
      Y1 += dy * s1;
      Z1 += dz * s1;
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const T wx = wk[k] * dxk[k];
    T0 += wk[k];
    T1 += wx;
    T2 += wx * dxk[k];
  }
}

// Records in brick order (tile_offsets, flatten_ids; isect_ids optional),
// one lane per record.  kRows = false: each record's ten partials go out
// through global atomics.  kRows = true: they are stored as the row
// isect_src[r] of `rows` (see r2s_rows.h), zeros included.  kExact: the
// brick size equals R (loops fully unrolled); otherwise ts <= R at run time.
template <typename T, int R, bool kExact, bool kRows>
__global__ __launch_bounds__(kBwdThreads) void voxel_bwd_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int64_t *__restrict__ isect_ids,
    const int32_t *__restrict__ flatten_ids, const int32_t *__restrict__ isect_src,
    int64_t n_isects, uint32_t n_keys, uint32_t koff, int64_t N, const T *__restrict__ v_vol,
    uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, bool vec,
    T *__restrict__ v_means, T *__restrict__ v_conics, T *__restrict__ v_opac,
    T *__restrict__ rows) {
  // Consecutive blocks (neighbouring tiles, which share Gaussians) on one XCD.
  const int64_t rb =
      static_cast<int64_t>(xcd_swizzle(blockIdx.x, gridDim.x)) * kBwdThreads + 64 * wave_index();
  if (rb >= n_isects) return;  // uniform per wave
  const int64_t r = rb + lane_id();
  const bool in_list = r < n_isects;
  const int nts = kExact ? R : static_cast<int>(ts);
  uint32_t key;
  bool key_ok = in_list;
  // Issued with the key's load, not after its check (one memory round trip
  // fewer before the record's own loads).
  const int32_t fid = in_list ? flatten_ids[r] : -1;
  if (isect_ids != nullptr) {
    const int64_t k = in_list ? isect_ids[r] : 0;
    key_ok = key_ok && k >= 0 && k < static_cast<int64_t>(n_keys);
    key = key_ok ? static_cast<uint32_t>(k) : 0u;
  } else {
    key = wave_record_key(tile_offsets, n_keys, n_isects, rb, r);
  }
  const int64_t g = key_ok ? static_cast<int64_t>(fid) : -1;
  const Brick b = brick_of(key + koff, n2, n1, static_cast<uint32_t>(nts), D2, D1, D0);
  BwdRecord<T> rec;
  load_bwd_record(means3d, conics, opac, g, N, key_ok, b, rec);
  const T half = static_cast<T>(0.5);
  const T dx0 = (static_cast<T>(b.ok) + half) - rec.m[0];
  const int64_t plane = static_cast<int64_t>(D1) * D2;
  // Columns past the volume matter only for records whose sigma may be
  // non-finite (uniform over the wave).
  const bool guard = ballot(rec.live && !rec.cu.ok && b.nk < nts) != 0;
  T T0 = 0, T1 = 0, T2 = 0, Y0 = 0, Z0 = 0, Y1 = 0, Z1 = 0, YY = 0, YZ = 0, ZZ = 0;
  bool full = false;
  if constexpr (kExact && R % Quad<T>::n == 0)
    full = vec && ballot(b.ni < nts || b.nj < nts || b.nk < nts) == 0;
  if (full && ballot(rec.live) != 0) {
    voxel_brick_full<T, R>(rec, b, v_vol, plane, D2, dx0, T0, T1, T2, Y0, Z0, Y1, Z1, YY, YZ, ZZ);
  } else if (ballot(rec.live) != 0) {
    // Rolled loops: unrolled, the slices and rows multiply the registers.
#pragma unroll 1
    for (int li = 0; li < R; ++li) {
      if (!kExact && li >= nts) break;
      const int i = b.oi + li;
      const bool in_slice = rec.live && i >= rec.i0 && i <= rec.i1;
      if (ballot(in_slice) == 0) continue;
      const T dz = (static_cast<T>(i) + half) - rec.m[2];
      // Rows of this slice the lane's ellipsoid can reach.
      int j0, j1;
      slice_rows(rec, b, in_slice, dz, dx0, j0, j1);
      const T h4dz = rec.h[4] * dz, h5dzz = rec.h[5] * dz * dz, Bz = rec.h[2] * dz;
#pragma unroll 1
      for (int lj = 0; lj < R; ++lj) {
        if (!kExact && lj >= nts) break;
        const int j = b.oj + lj;
        const bool in_row = j >= j0 && j <= j1;
        if (ballot(in_row) == 0) continue;
        const T dy = (static_cast<T>(j) + half) - rec.m[1];
        const T B = rec.h[1] * dy + Bz;
        const T C = (rec.h[3] * dy + h4dz) * dy + h5dzz;
        const T *__restrict__ vrow =
            v_vol +
            (in_row ? static_cast<int64_t>(i) * plane + static_cast<int64_t>(j) * D2 : 0) + b.ok;
        T vv[R];
        if (vec)
          load_grad_row<T, R, true>(vrow, in_row, b.nk, nts, vv);
        else
          load_grad_row<T, R, false>(vrow, in_row, b.nk, nts, vv);
        T s0 = 0, s1 = 0, s2 = 0;
        if (guard)
          voxel_row<T, R, kExact, true>(rec, vv, dx0, b.nk, nts, B, C, s0, s1, s2);
        else
          voxel_row<T, R, kExact, false>(rec, vv, dx0, b.nk, nts, B, C, s0, s1, s2);
        T0 += s0;
        T1 += s1;
        T2 += s2;
        const T dys0 = dy * s0, dzs0 = dz * s0;
        Y0 += dys0;
        Z0 += dzs0;
        YY += dy * dys0;
        YZ += dz * dys0;
        ZZ += dz * dzs0;
        Y1 += dy * s1;
        Z1 += dz * s1;
      }
    }
  }
  if (!key_ok) return;
  // Per-voxel terms of VoxelizeToVoxelsBwd.cu:409-421 summed over the brick
  // (zero for dead records).
  const T o = rec.o;
  const T *q = rec.q;
  const T gx = o * (q[0] * T1 + q[1] * Y0 + q[2] * Z0);
  const T gy = o * (q[3] * Y0 + q[4] * Z0 + q[1] * T1);
  const T gz = o * (q[5] * Z0 + q[4] * Y0 + q[2] * T1);
  const T g0 = -half * o * T2, g1 = -o * Y1, g2 = -o * Z1;
  const T g3 = -half * o * YY, g4 = -o * YZ, g5 = -half * o * ZZ;
  const T go = T0;
  if (kRows) {
    const T v[10] = {gx, gy, gz, g0, g1, g2, g3, g4, g5, go};
    store_row(rows, isect_src[r], v);
    return;
  }
  if (!rec.live) return;
  if (gx == 0 && gy == 0 && gz == 0 && g0 == 0 && g1 == 0 && g2 == 0 && g3 == 0 && g4 == 0 &&
      g5 == 0 && go == 0)
    return;
  atomic_add(v_means + 3 * g, gx);
  atomic_add(v_means + 3 * g + 1, gy);
  atomic_add(v_means + 3 * g + 2, gz);
  atomic_add(v_conics + 6 * g, g0);
  atomic_add(v_conics + 6 * g + 1, g1);
  atomic_add(v_conics + 6 * g + 2, g2);
  atomic_add(v_conics + 6 * g + 3, g3);
  atomic_add(v_conics + 6 * g + 4, g4);
  atomic_add(v_conics + 6 * g + 5, g5);
  atomic_add(v_opac + g, go);
}

// ------------------------------------------- chunked backward (rows) ---
//
// A wave of 64 records walks the union of its lanes' reached rows, which is
// nearly always every row of the brick, while one record's culled
// ellipsoid reaches about 57 % of them at config 3.  This form lists, per
// wave, the (record, slice, row) items the records reach -- slice by slice,
// row by row, as slice_rows gives them -- and hands them out in chunks of up
// to kChunkRows consecutive items of one record, one chunk per lane and
// round, so lanes spend their steps on reached rows.  The full chunks come
// first, ordered by (chunk index within the record, record), then each
// record's short last chunk, longest first; a round takes as many steps as
// its first (longest) chunk.  Within a round each record appears at most
// once per chunk index, and the chunk sums are added to the record's LDS
// accumulators one chunk index at a time in increasing order, so each
// record's chunks add in index order and the result does not depend on
// scheduling.  Every brick must lie inside
// the volume with 16-byte gradient rows, the gradient volume must span at
// most 2^32 bytes and a slice fewer than 2^24 (the caller checks).

constexpr int kChunkRows = 8;
constexpr int kChunkWaves = 4;
// A chunked item costs about 1.3 times a row of the dense walk (indexing,
// the walk, the chunk sums), so a wave whose records reach more than this
// many of their 64 x 64 (record, row) pairs takes the dense walk instead
// (large footprints, e.g. the binary-tree model on a 128^3 volume).
constexpr int kDenseItems = 3072;

template <typename T>
struct ChunkRecord {
  T c[3];  // the brick's first voxel centre minus the mean (x, y, z)
  T h[6];
  typename Bits<T>::type lim;  // 0 for dead records
  uint32_t brick0;             // byte offset of the brick's first voxel in v_vol
};

// Chunks of one chunked wave: its records reach at most kDenseItems rows, in
// chunks of up to kChunkRows, at most one short chunk per record.
constexpr int kMaxChunks = kDenseItems / kChunkRows + 64;

// kGiven: each record's reach mask comes from `reach` (stored by the forward
// over the same lists, voxel_fwd_reach_kernel) instead of the culling
// setup and the per-slice row ranges.
template <typename T, bool kGiven>
__global__ __launch_bounds__(64 * kChunkWaves) void voxel_bwd_chunk_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int64_t *__restrict__ isect_ids,
    const int32_t *__restrict__ flatten_ids, const int32_t *__restrict__ isect_src,
    int64_t n_isects, uint32_t n_keys, uint32_t koff, int64_t N, const T *__restrict__ v_vol,
    uint32_t D2, uint32_t D1, uint32_t D0, uint32_t n2, uint32_t n1, T *__restrict__ rows,
    const uint64_t *__restrict__ reach) {
  constexpr int R = kChunkRows;
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n;
  __shared__ WordMajor<ChunkRecord<T>, 64> s_rec[kChunkWaves];
  __shared__ uint64_t s_rows[kChunkWaves][64];  // reached rows: bit 8 * slice + row
  __shared__ T s_acc[kChunkWaves][10][64];
  // Chunk entries: record lane | first row << 6 | chunk index << 12.
  __shared__ uint16_t s_chunk[kChunkWaves][kMaxChunks];
  const uint32_t w = wave_index(), lane = lane_id();
  const int64_t rb = static_cast<int64_t>(xcd_swizzle(blockIdx.x, gridDim.x)) *
                         (64 * kChunkWaves) + 64 * static_cast<int64_t>(w);
  if (rb >= n_isects) return;  // uniform per wave; the waves share no barrier
  const int64_t r = rb + lane;
  const bool in_list = r < n_isects;
  uint32_t key;
  bool key_ok = in_list;
  // Issued with the key's load, not after its check (one memory round trip
  // fewer before the record's own loads).
  const int32_t fid = in_list ? flatten_ids[r] : -1;
  const uint64_t reach_r = kGiven && in_list ? reach[r] : 0ull;
  if (isect_ids != nullptr) {
    const int64_t k = in_list ? isect_ids[r] : 0;
    key_ok = key_ok && k >= 0 && k < static_cast<int64_t>(n_keys);
    key = key_ok ? static_cast<uint32_t>(k) : 0u;
  } else {
    key = wave_record_key(tile_offsets, n_keys, n_isects, rb, r);
  }
  const int64_t g = key_ok ? static_cast<int64_t>(fid) : -1;
  const Brick b = brick_of(key + koff, n2, n1, R, D2, D1, D0);
  BwdRecord<T> rec;
  if constexpr (kGiven)
    load_bwd_record_plain(means3d, conics, opac, g, N, key_ok, b, rec);
  else
    load_bwd_record(means3d, conics, opac, g, N, key_ok, b, rec);
  const T half = static_cast<T>(0.5);
  const uint32_t plane = D1 * D2;  // the caller checks D2 D1 D0 sizeof(T) <= 2^32
  const uint32_t plane_b = plane * static_cast<uint32_t>(sizeof(T)),
                 row_b = D2 * static_cast<uint32_t>(sizeof(T));
  const T dx0 = (static_cast<T>(b.ok) + half) - rec.m[0];

  // The record's reached rows; the items are its set bits in increasing order.
  uint64_t reached;
  if constexpr (kGiven)
    reached = key_ok && rec.live ? reach_r : 0ull;
  else
    reached = reach_mask(rec, b, dx0);
  const int n_items = __popcll(reached);
  if (wave_sum(n_items) > kDenseItems) {  // uniform per wave
    T T0 = 0, T1 = 0, T2 = 0, Y0 = 0, Z0 = 0, Y1 = 0, Z1 = 0, YY = 0, YZ = 0, ZZ = 0;
    if (ballot(rec.live) != 0)
      voxel_brick_full<T, R, true>(rec, b, v_vol, static_cast<int64_t>(plane), D2, dx0, T0, T1,
                                   T2, Y0, Z0, Y1, Z1, YY, YZ, ZZ, reached);
    if (!key_ok) return;
    const T o = rec.o;
    const T *qc = rec.q;
    const T v[10] = {o * (qc[0] * T1 + qc[1] * Y0 + qc[2] * Z0),
                     o * (qc[3] * Y0 + qc[4] * Z0 + qc[1] * T1),
                     o * (qc[5] * Z0 + qc[4] * Y0 + qc[2] * T1),
                     -half * o * T2,
                     -o * Y1,
                     -o * Z1,
                     -half * o * YY,
                     -o * YZ,
                     -half * o * ZZ,
                     T0};
    store_row(rows, isect_src[r], v);
    return;
  }
  {
    ChunkRecord<T> cr;
    cr.c[0] = dx0;
    cr.c[1] = (static_cast<T>(b.oj) + half) - rec.m[1];
    cr.c[2] = (static_cast<T>(b.oi) + half) - rec.m[2];
#pragma unroll
    for (int c = 0; c < 6; ++c) cr.h[c] = rec.h[c];
    cr.lim = rec.live ? rec.lim : 0;
    // Below 2^32: the caller checks D2 D1 D0 sizeof(T) <= 2^32.
    cr.brick0 = (static_cast<uint32_t>(b.oi) * plane + static_cast<uint32_t>(b.oj) * D2 +
                 static_cast<uint32_t>(b.ok)) * static_cast<uint32_t>(sizeof(T));
    s_rec[w].store(static_cast<int>(lane), cr);
    s_rows[w][lane] = reached;
#pragma unroll
    for (int c = 0; c < 10; ++c) s_acc[w][c][lane] = 0;
  }
  // Chunk list: the full chunks in (chunk index, record) order, then each
  // record's short last chunk, longest first, so that the rounds of short
  // chunks take as many steps as their longest.  Each record's chunks keep
  // increasing chunk indices.  Byte li of pref: the reached rows of the
  // slices before li (0..56).
  uint64_t pref = 0;
  {
    uint32_t run = 0;
#pragma unroll
    for (int li = 0; li < R; ++li) {
      pref |= static_cast<uint64_t>(run) << (8 * li);
      run += static_cast<uint32_t>(__popc(static_cast<uint32_t>(reached >> (8 * li)) & 0xFFu));
    }
  }
  // The chunk's first row, the t-th set bit (t = 8 q): its slice li is the
  // last whose byte of pref is <= t, found for all eight bytes at once (each
  // byte | 0x80, minus t + 1, keeps its high bit exactly when the byte
  // exceeds t); within a slice the reached rows are contiguous.
  auto entry = [&](uint32_t q) {
    const uint32_t t = q * static_cast<uint32_t>(R);
    constexpr uint64_t kHigh = 0x8080808080808080ull, kOnes = 0x0101010101010101ull;
    const uint64_t above = ((pref | kHigh) - static_cast<uint64_t>(t + 1u) * kOnes) & kHigh;
    const int li = 7 - __popcll(above);
    const uint32_t byte = static_cast<uint32_t>(reached >> (8 * li)) & 0xFFu;
    const uint32_t before = static_cast<uint32_t>(pref >> (8 * li)) & 0xFFu;
    const uint32_t first =
        8u * static_cast<uint32_t>(li) + __builtin_ctz(byte | 0x100u) + (t - before);
    return static_cast<uint16_t>(lane | (first << 6) | (q << 12));
  };
  const int n_full = n_items / R, tail = n_items - n_full * R;
  uint32_t n_list = 0;
  const uint64_t lt = lanemask_lt();
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const bool has = n_full > q;
    const uint64_t m = ballot(has);
    if (has)
      s_chunk[w][n_list + static_cast<uint32_t>(__popcll(m & lt))] =
          entry(static_cast<uint32_t>(q));
    n_list += static_cast<uint32_t>(__popcll(m));
  }
#pragma unroll
  for (int len = R - 1; len > 0; --len) {
    const bool has = tail == len;
    const uint64_t m = ballot(has);
    if (has)
      s_chunk[w][n_list + static_cast<uint32_t>(__popcll(m & lt))] =
          entry(static_cast<uint32_t>(n_full));
    n_list += static_cast<uint32_t>(__popcll(m));
  }
  // The wave's LDS operations complete in order, so its own lanes' writes
  // are visible to the reads below; keep the compiler from moving them.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll 1
  for (uint32_t cb = 0; cb < n_list; cb += 64) {
    const uint32_t ci = cb + lane;
    const bool act = ci < n_list;
    const uint32_t ent = act ? static_cast<uint32_t>(s_chunk[w][ci]) : 0u;
    const uint32_t rl = ent & 63u, pos = (ent >> 6) & 63u, q = ent >> 12;
    const ChunkRecord<T> cr = s_rec[w].load(static_cast<int>(rl));
    const uint64_t rows_m = s_rows[w][rl];
    const int n_here =
        act ? min(R, __popcll(rows_m) - static_cast<int>(q) * R) : 0;
    // The record's rows from the chunk's first on: the chunk's items are
    // its n_here lowest set bits.
    uint64_t rest = act ? rows_m & (~0ull << pos) : 0ull;
    T dxk[R], wk[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      dxk[k] = cr.c[0] + static_cast<T>(k);
      wk[k] = 0;
    }
    T Y0 = 0, Z0 = 0, Y1 = 0, Z1 = 0, YY = 0, YZ = 0, ZZ = 0;
    // The round's longest chunk is its first (lane 0 is always active).
    const int steps = __builtin_amdgcn_readfirstlane(n_here);
#pragma unroll 1
    for (int st = 0; st < steps; ++st) {
      const bool item = st < n_here;
      // The next row (bit 63 when none is left: a step without an item
      // still reads a row of the record's own brick, which lies inside the
      // volume, and tests against a zero limit).
      const uint32_t p = static_cast<uint32_t>(__builtin_ctzll(rest | (1ull << 63)));
      rest &= rest - 1ull;
      const uint32_t li = p >> 3, lj = p & 7u;
      // The row centre's offsets from the mean as the columns' (dxk): the
      // brick corner's offset plus the row's index in the brick.
      const T dz = static_cast<T>(li) + cr.c[2];
      const T dy = static_cast<T>(lj) + cr.c[1];
      const T B = fma(cr.h[1], dy, cr.h[2] * dz);
      const T C = fma(fma(cr.h[3], dy, cr.h[4] * dz), dy, cr.h[5] * dz * dz);
      const typename Bits<T>::type lim = item ? cr.lim : 0;
      // 32-bit byte offsets: li, lj < 8 and plane_b = D1 D2 sizeof(T) < 2^24
      // (the caller checks), so two full-rate 24-bit multiply-adds per row.
      uint32_t off = __umul24(lj, row_b) + cr.brick0;
      asm volatile("" : "+v"(off));  // two multiply-adds, not two products and a sum
      off += __umul24(li, plane_b);
      const T *__restrict__ vrow =
          reinterpret_cast<const T *>(reinterpret_cast<const char *>(v_vol) + off);
      T vv[R];
#pragma unroll
      for (int c = 0; c < R / kq; ++c)
        *reinterpret_cast<Q *>(vv + c * kq) = *reinterpret_cast<const Q *>(vrow + c * kq);
      T s0 = 0, s1 = 0;
#pragma unroll
      for (int k = 0; k < R; ++k) {
        const T dx = dxk[k];
        const T slv = fma(fma(cr.h[0], dx, B), dx, C);
        // A failing voxel adds an exact zero whatever its upstream gradient
        // (a non-finite one included), as when the voxel is skipped.  The
        // product is formed unconditionally: as an operand of the
        // conditional it would become a branch around its load and exp.
        const T p = vv[k] * neg_exp2(slv);
        const T wv = alpha_pass(slv, lim) ? p : static_cast<T>(0);
        wk[k] += wv;
        s0 += wv;
        s1 = fma(wv, dx, s1);
      }
      const T dys0 = dy * s0, dzs0 = dz * s0;
      Y0 += dys0;
      Z0 += dzs0;
      YY = fma(dy, dys0, YY);
      YZ = fma(dz, dys0, YZ);
      ZZ = fma(dz, dzs0, ZZ);
      Y1 = fma(dy, s1, Y1);
      Z1 = fma(dz, s1, Z1);
    }
    T t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const T wx = wk[k] * dxk[k];
      t0 += wk[k];
      t1 += wx;
      t2 += wx * dxk[k];
    }
    const T sums[10] = {t0, t1, t2, Y0, Z0, Y1, Z1, YY, YZ, ZZ};
    // One chunk index at a time, in increasing order: the records of one
    // index are distinct, and each record's chunks are added in index order.
    uint32_t qmask = 0;
#pragma unroll
    for (int b = 0; b < R; ++b)
      if (ballot(act && q == static_cast<uint32_t>(b)) != 0) qmask |= 1u << b;
#pragma unroll 1
    for (uint32_t mq = qmask; mq != 0u; mq &= mq - 1u) {
      const uint32_t qq = static_cast<uint32_t>(__builtin_ctz(mq));
      if (act && q == qq) {
#pragma unroll
        for (int c = 0; c < 10; ++c) s_acc[w][c][rl] += sums[c];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  if (!key_ok) return;
  T a[10];
#pragma unroll
  for (int c = 0; c < 10; ++c) a[c] = s_acc[w][c][lane];
  const T T0 = a[0], T1 = a[1], T2 = a[2], Y0 = a[3], Z0 = a[4], Y1 = a[5], Z1 = a[6],
          YY = a[7], YZ = a[8], ZZ = a[9];
  // Per-voxel terms of VoxelizeToVoxelsBwd.cu:409-421 summed over the brick,
  // as in voxel_bwd_kernel.
  const T o = rec.o;
  const T *qc = rec.q;
  const T v[10] = {o * (qc[0] * T1 + qc[1] * Y0 + qc[2] * Z0),
                   o * (qc[3] * Y0 + qc[4] * Z0 + qc[1] * T1),
                   o * (qc[5] * Z0 + qc[4] * Y0 + qc[2] * T1),
                   -half * o * T2,
                   -o * Y1,
                   -o * Z1,
                   -half * o * YY,
                   -o * YZ,
                   -half * o * ZZ,
                   T0};
  store_row(rows, isect_src[r], v);
}

// n0 brick layers of lists from layer z0 on (the whole grid: z0 = 0 and
// n0 ts >= D0; a z-slab: z0 + n0 layers within the grid).
int check_voxel_args(int64_t n_isects, int64_t N, uint32_t D2, uint32_t D1, uint32_t D0,
                     uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0, const char *name,
                     uint32_t z0 = 0, bool slab = false) {
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size N=%lld", name, (long long)N);
  // ts <= 10 first: ts^3 in 32 bits wraps for ts >= 1626.
  R2S_REQUIRE(ts > 0 && ts <= 10 && ts * ts * ts <= 1024,
              "%s: tile_size must be positive with tile_size**3 <= 1024", name);
  R2S_REQUIRE(n_isects >= 0 && n_isects <= kInt32Max, "%s: bad n_isects", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * ts >= D2 && static_cast<uint64_t>(n1) * ts >= D1 &&
                  (slab || static_cast<uint64_t>(n0) * ts >= D0),
              "%s: brick grid does not cover the volume", name);
  R2S_REQUIRE(!slab || (static_cast<uint64_t>(z0) + n0) * ts < static_cast<uint64_t>(D0) + ts,
              "%s: brick layers [%u, %u) outside the volume", name, z0, z0 + n0);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * ts <= 0x7fffffffull &&
                  static_cast<uint64_t>(n1) * ts <= 0x7fffffffull &&
                  static_cast<uint64_t>(n0) * ts <= 0x7fffffffull,
              "%s: brick grid too large", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * n1 * (static_cast<uint64_t>(z0) + n0) <=
                  0x7fffffffull,
              "%s: too many bricks", name);
  return R2S_OK;
}

template <typename T, int R>
void launch_voxel_fwd(const T *means3d, const T *conics, const T *opac,
                      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,
                      uint32_t n_keys, uint32_t koff, int64_t N, uint32_t D2, uint32_t D1,
                      uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, T *volume,
                      hipStream_t stream) {
  const uint32_t nt = ts * ts * (ts / R);
  const size_t smem =
      min(nt, kFwdBatch) * (3 * sizeof(typename Vec<T>::v4));
  voxel_fwd_kernel<T, R><<<dim3(n_keys), dim3(nt), smem, stream>>>(
      means3d, conics, opac, tile_offsets, flatten_ids, n_isects, n_keys, koff, N, D2, D1, D0, ts,
      n2, n1, volume);
}

// slab: the lists are those of brick layers [z0, z0 + n0) (keys relative to
// layer z0) and only that z-range of the whole volume is written.
template <typename T>
int voxel_fwd_impl(const T *means3d, const T *conics, const T *opac,
                   const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,
                   int64_t N, uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2,
                   uint32_t n1, uint32_t n0, T *volume, r2s_stream_t st, uint32_t z0 = 0,
                   bool slab = false, uint64_t *reach = nullptr) {
  clear_error();
  const char *name = "voxelize_to_voxels_fwd";
  R2S_RETURN_IF(check_voxel_args(n_isects, N, D2, D1, D0, ts, n2, n1, n0, name, z0, slab));
  R2S_REQUIRE(reach == nullptr || ts == 8, "%s: reach masks need tile_size 8", name);
  // Voxel slices [i0, i1) of the layers' z-range.
  const int64_t i0 = static_cast<int64_t>(z0) * ts;
  const int64_t i1 = slab ? std::min<int64_t>(static_cast<int64_t>(z0 + n0) * ts, D0) : D0;
  const int64_t plane = static_cast<int64_t>(D2) * D1;
  const int64_t n_vox = plane * (i1 - i0);
  if (n_vox <= 0) return R2S_OK;
  R2S_REQUIRE(volume != nullptr, "%s: null volume", name);
  hipStream_t stream = as_stream(st);
  if (N == 0 || n_isects == 0)
    return device_fill<T>(volume + i0 * plane, n_vox, static_cast<T>(0), stream, name);
  R2S_REQUIRE(means3d && conics && opac && tile_offsets && flatten_ids, "%s: null pointer", name);
  const uint32_t n_keys = n2 * n1 * n0, koff = z0 * n1 * n2;
  if (ts == 8) {
    // Waves per brick from the mean list length: one up to 192 records (3
    // batches), then 2, then 4 from 384, so that long lists (large
    // footprints, few bricks) are shared out.
    const int64_t per_brick = n_isects / n_keys;
    const dim3 grid(n_keys);
#define R2S_VOXEL_FWD_REACH(S)                                                                  \
  voxel_fwd_reach_kernel<T, S><<<grid, dim3(64 * S), 0, stream>>>(                              \
      means3d, conics, opac, tile_offsets, flatten_ids, n_isects, n_keys, koff, N, D2, D1, D0,  \
      n2, n1, volume, reach)
    if (per_brick < 192)
      R2S_VOXEL_FWD_REACH(1);
    else if (per_brick < 384)
      R2S_VOXEL_FWD_REACH(2);
    else
      R2S_VOXEL_FWD_REACH(4);
#undef R2S_VOXEL_FWD_REACH
  } else if (ts == 16)
    launch_voxel_fwd<T, 16>(means3d, conics, opac, tile_offsets, flatten_ids, n_isects, n_keys,
                            koff, N, D2, D1, D0, ts, n2, n1, volume, stream);
  else
    launch_voxel_fwd<T, 1>(means3d, conics, opac, tile_offsets, flatten_ids, n_isects, n_keys,
                           koff, N, D2, D1, D0, ts, n2, n1, volume, stream);
  return check_launch(name);
}

template <typename T, int R, bool kExact>
void launch_voxel_bwd(const T *means3d, const T *conics, const T *opac,
                      const int32_t *tile_offsets, const int64_t *isect_ids,
                      const int32_t *flatten_ids, const int32_t *isect_src, int64_t n_isects,
                      uint32_t n_keys, uint32_t koff, int64_t N, const T *v_vol, uint32_t D2,
                      uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, bool vec,
                      T *v_means, T *v_conics, T *v_opac, T *rows, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(ceil_div(n_isects, kBwdThreads)));
  if (rows != nullptr)
    voxel_bwd_kernel<T, R, kExact, true><<<grid, dim3(kBwdThreads), 0, stream>>>(
        means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects, n_keys,
        koff, N, v_vol, D2, D1, D0, ts, n2, n1, vec, v_means, v_conics, v_opac, rows);
  else
    voxel_bwd_kernel<T, R, kExact, false><<<grid, dim3(kBwdThreads), 0, stream>>>(
        means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects, n_keys,
        koff, N, v_vol, D2, D1, D0, ts, n2, n1, vec, v_means, v_conics, v_opac, rows);
}

int64_t voxel_rows_bytes(int64_t n_isects, int dtype_bytes) {
  return n_isects * row_stride<10>() * static_cast<int64_t>(dtype_bytes);
}

// Second pass of the two-pass backward: per-Gaussian sums of the rows.
template <typename T>
int voxel_reduce_impl(const T *rows, const int32_t *emit_ids, int64_t n_isects, int64_t N,
                      T *v_means, T *v_conics, T *v_opac, r2s_stream_t st) {
  const char *name = "voxelize_to_voxels_bwd (row reduction)";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max && n_isects >= 0 && n_isects <= kInt32Max,
              "%s: bad size", name);
  if (N == 0) return R2S_OK;
  R2S_REQUIRE(v_means && v_conics && v_opac, "%s: null output", name);
  R2S_REQUIRE(n_isects == 0 || (rows && emit_ids), "%s: null pointer", name);
  R2S_REQUIRE(reinterpret_cast<uintptr_t>(rows) % 16 == 0, "%s: rows not 16-byte aligned", name);
  RowTargets<T, 10> tg = {{v_means, v_means + 1, v_means + 2, v_conics, v_conics + 1,
                           v_conics + 2, v_conics + 3, v_conics + 4, v_conics + 5, v_opac},
                          {3, 3, 3, 6, 6, 6, 6, 6, 6, 1}};
  launch_row_reduce(rows, emit_ids, n_isects, N, tg, as_stream(st));
  return check_launch(name);
}

// two_pass: emit_ids / isect_src / ws give the two-pass form (r2s_rows.h);
// rows_only stops after the first pass (the rows are left in ws).
template <typename T>
int voxel_bwd_impl(const T *means3d, const T *conics, const T *opac,
                   const int32_t *tile_offsets, const int64_t *isect_ids,
                   const int32_t *flatten_ids, const int32_t *emit_ids,
                   const int32_t *isect_src, int64_t n_isects, const T *v_vol, int64_t N,
                   uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,
                   uint32_t n0, T *v_means, T *v_conics, T *v_opac, void *ws, size_t ws_bytes,
                   bool two_pass, r2s_stream_t st, bool rows_only = false, uint32_t z0 = 0,
                   bool slab = false, const uint64_t *reach = nullptr) {
  clear_error();
  const char *name = two_pass   ? "voxelize_to_voxels_bwd (two-pass)"
                     : isect_ids ? "voxelize_to_voxels_bwd_per_gaussian"
                                 : "voxelize_to_voxels_bwd";
  R2S_RETURN_IF(check_voxel_args(n_isects, N, D2, D1, D0, ts, n2, n1, n0, name, z0, slab));
  R2S_REQUIRE(reach == nullptr || ts == 8, "%s: reach masks need tile_size 8", name);
  if (N == 0) return R2S_OK;
  const int64_t n_vox = static_cast<int64_t>(D2) * D1 * D0;
  if (n_isects == 0 || n_vox == 0) {  // the two-pass form still stores its (zero) outputs
    if (!two_pass || rows_only) return R2S_OK;
    return voxel_reduce_impl<T>(nullptr, nullptr, 0, N, v_means, v_conics, v_opac, st);
  }
  R2S_REQUIRE(tile_offsets && flatten_ids, "%s: null brick lists", name);
  R2S_REQUIRE(means3d && conics && opac && v_vol, "%s: null pointer", name);
  R2S_REQUIRE(rows_only || (v_means && v_conics && v_opac), "%s: null output", name);
  T *rows = nullptr;
  if (two_pass) {
    R2S_REQUIRE(isect_src && (rows_only || emit_ids), "%s: null emit_ids / isect_src", name);
    const int64_t need = voxel_rows_bytes(n_isects, sizeof(T));
    if (ws == nullptr || static_cast<int64_t>(ws_bytes) < need) {
      set_error("%s: workspace of %zu bytes, %lld required", name, ws_bytes, (long long)need);
      return R2S_EWORKSPACE;
    }
    R2S_REQUIRE(reinterpret_cast<uintptr_t>(ws) % 16 == 0, "%s: workspace not 16-byte aligned",
                name);
    rows = static_cast<T *>(ws);
  }
  const uint32_t n_keys = n2 * n1 * n0, koff = z0 * n1 * n2;
  hipStream_t stream = as_stream(st);
  // 16-byte loads of gradient rows when every row segment starts aligned.
  const bool vec = vec_rows_ok<T>(v_vol, D2, ts);
#define R2S_VOXEL_BWD_R(RR, EXACT)                                                             \
  launch_voxel_bwd<T, RR, EXACT>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids,  \
                                 isect_src, n_isects, n_keys, koff, N, v_vol, D2, D1, D0, ts,  \
                                 n2, n1, vec, v_means, v_conics, v_opac, rows, stream)
  // The chunked walk addresses the gradient with 32-bit byte offsets and
  // 24-bit plane and row strides.
  const int64_t elem = static_cast<int64_t>(sizeof(T));
  if (ts == 8 && rows != nullptr && vec && D2 % 8 == 0 && D1 % 8 == 0 && D0 % 8 == 0 &&
      n_vox * elem <= (int64_t{1} << 32) &&
      static_cast<int64_t>(D1) * D2 * elem < (int64_t{1} << 24)) {
    const dim3 grid(static_cast<uint32_t>(ceil_div(n_isects, 64 * kChunkWaves)));
    if (reach != nullptr)
      voxel_bwd_chunk_kernel<T, true><<<grid, dim3(64 * kChunkWaves), 0, stream>>>(
          means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects,
          n_keys, koff, N, v_vol, D2, D1, D0, n2, n1, rows, reach);
    else
      voxel_bwd_chunk_kernel<T, false><<<grid, dim3(64 * kChunkWaves), 0, stream>>>(
          means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects,
          n_keys, koff, N, v_vol, D2, D1, D0, n2, n1, rows, nullptr);
  } else if (ts == 8)
    R2S_VOXEL_BWD_R(8, true);
  else if (ts == 4)
    R2S_VOXEL_BWD_R(4, true);
  else if (ts < 4)
    R2S_VOXEL_BWD_R(4, false);
  else if (ts < 8)
    R2S_VOXEL_BWD_R(8, false);
  else
    R2S_VOXEL_BWD_R(16, false);
#undef R2S_VOXEL_BWD_R
  R2S_RETURN_IF(check_launch(name));
  if (!two_pass || rows_only) return R2S_OK;
  return voxel_reduce_impl<T>(rows, emit_ids, n_isects, N, v_means, v_conics, v_opac, st);
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_voxelize_bwd_workspace_bytes(int64_t n_isects, int dtype_bytes) {
  if (n_isects <= 0 || (dtype_bytes != 4 && dtype_bytes != 8)) return 0;
  return r2s::voxel_rows_bytes(n_isects, dtype_bytes);
}

#define R2S_VOXEL_API(SUF, T)                                                                  \
  int r2s_voxelize_fwd_##SUF(const T *means3d, const T *conics, const T *opac,                 \
                             const int32_t *tile_offsets, const int32_t *flatten_ids,          \
                             int64_t n_isects, int64_t N, uint32_t D2, uint32_t D1,            \
                             uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,  \
                             T *volume, r2s_stream_t st) {                                     \
    return r2s::voxel_fwd_impl<T>(means3d, conics, opac, tile_offsets, flatten_ids, n_isects,  \
                                  N, D2, D1, D0, ts, n2, n1, n0, volume, st);                  \
  }                                                                                            \
  int r2s_voxelize_bwd_##SUF(const T *means3d, const T *conics, const T *opac,                 \
                             const int32_t *tile_offsets, const int64_t *isect_ids,            \
                             const int32_t *flatten_ids, int64_t n_isects, const T *v_vol,     \
                             int64_t N, uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts,    \
                             uint32_t n2, uint32_t n1, uint32_t n0, T *v_means, T *v_conics,   \
                             T *v_opac, r2s_stream_t st) {                                     \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  nullptr, nullptr, n_isects, v_vol, N, D2, D1, D0, ts, n2,    \
                                  n1, n0, v_means, v_conics, v_opac, nullptr, 0, false, st);   \
  }                                                                                            \
  int r2s_voxelize_bwd_emit_##SUF(                                                             \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *emit_ids,           \
      const int32_t *isect_src, int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2,      \
      uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,            \
      T *v_means, T *v_conics, T *v_opac, void *ws, size_t ws_bytes, r2s_stream_t st) {        \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  emit_ids, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2, \
                                  n1, n0, v_means, v_conics, v_opac, ws, ws_bytes, true, st);  \
  }                                                                                            \
  int r2s_voxelize_fwd_reach_##SUF(const T *means3d, const T *conics, const T *opac,           \
                                   const int32_t *tile_offsets, const int32_t *flatten_ids,    \
                                   int64_t n_isects, int64_t N, uint32_t D2, uint32_t D1,      \
                                   uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,         \
                                   uint32_t n0, T *volume, uint64_t *reach, r2s_stream_t st) { \
    return r2s::voxel_fwd_impl<T>(means3d, conics, opac, tile_offsets, flatten_ids, n_isects,  \
                                  N, D2, D1, D0, ts, n2, n1, n0, volume, st, 0, false, reach); \
  }                                                                                            \
  int r2s_voxelize_bwd_emit_reach_##SUF(                                                       \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *emit_ids,           \
      const int32_t *isect_src, int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2,      \
      uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0,            \
      const uint64_t *reach, T *v_means, T *v_conics, T *v_opac, void *ws, size_t ws_bytes,    \
      r2s_stream_t st) {                                                                       \
    if (reach == nullptr) {                                                                    \
      r2s::clear_error();                                                                      \
      r2s::set_error("voxelize_to_voxels_bwd (two-pass): null reach masks");                   \
      return R2S_EINVAL;                                                                       \
    }                                                                                          \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  emit_ids, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2, \
                                  n1, n0, v_means, v_conics, v_opac, ws, ws_bytes, true, st,   \
                                  false, 0, false, reach);                                     \
  }                                                                                            \
  int r2s_voxelize_fwd_slab_##SUF(const T *means3d, const T *conics, const T *opac,            \
                                  const int32_t *tile_offsets, const int32_t *flatten_ids,     \
                                  int64_t n_isects, int64_t N, uint32_t D2, uint32_t D1,       \
                                  uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,          \
                                  uint32_t z0, uint32_t nz, T *volume, r2s_stream_t st) {      \
    return r2s::voxel_fwd_impl<T>(means3d, conics, opac, tile_offsets, flatten_ids, n_isects,  \
                                  N, D2, D1, D0, ts, n2, n1, nz, volume, st, z0, true);        \
  }                                                                                            \
  int r2s_voxelize_bwd_emit_slab_##SUF(                                                        \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *emit_ids,           \
      const int32_t *isect_src, int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2,      \
      uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, uint32_t z0,            \
      uint32_t nz, T *v_means, T *v_conics, T *v_opac, void *ws, size_t ws_bytes,              \
      r2s_stream_t st) {                                                                       \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  emit_ids, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2, \
                                  n1, nz, v_means, v_conics, v_opac, ws, ws_bytes, true, st,   \
                                  false, z0, true);                                            \
  }

#define R2S_VOXEL_STAGE_API(SUF, T)                                                            \
  int r2s_voxelize_bwd_rows_##SUF(                                                             \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *isect_src,          \
      int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2, uint32_t D1, uint32_t D0,      \
      uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0, void *rows, size_t rows_bytes,       \
      r2s_stream_t st) {                                                                       \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  nullptr, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2,  \
                                  n1, n0, nullptr, nullptr, nullptr, rows, rows_bytes, true,   \
                                  st, true);                                                   \
  }                                                                                            \
  int r2s_voxelize_bwd_rows_reach_##SUF(                                                       \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *isect_src,          \
      int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2, uint32_t D1, uint32_t D0,      \
      uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0, const uint64_t *reach, void *rows,   \
      size_t rows_bytes, r2s_stream_t st) {                                                    \
    if (reach == nullptr) {                                                                    \
      r2s::clear_error();                                                                      \
      r2s::set_error("voxelize_to_voxels_bwd (two-pass): null reach masks");                   \
      return R2S_EINVAL;                                                                       \
    }                                                                                          \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  nullptr, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2,  \
                                  n1, n0, nullptr, nullptr, nullptr, rows, rows_bytes, true,   \
                                  st, true, 0, false, reach);                                  \
  }                                                                                            \
  int r2s_voxelize_bwd_rows_slab_##SUF(                                                        \
      const T *means3d, const T *conics, const T *opac, const int32_t *tile_offsets,           \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *isect_src,          \
      int64_t n_isects, const T *v_vol, int64_t N, uint32_t D2, uint32_t D1, uint32_t D0,      \
      uint32_t ts, uint32_t n2, uint32_t n1, uint32_t z0, uint32_t nz, void *rows,             \
      size_t rows_bytes, r2s_stream_t st) {                                                    \
    return r2s::voxel_bwd_impl<T>(means3d, conics, opac, tile_offsets, isect_ids, flatten_ids, \
                                  nullptr, isect_src, n_isects, v_vol, N, D2, D1, D0, ts, n2,  \
                                  n1, nz, nullptr, nullptr, nullptr, rows, rows_bytes, true,   \
                                  st, true, z0, true);                                         \
  }                                                                                            \
  int r2s_voxelize_bwd_reduce_##SUF(const T *rows, const int32_t *emit_ids, int64_t n_isects,  \
                                    int64_t N, T *v_means, T *v_conics, T *v_opac,             \
                                    r2s_stream_t st) {                                         \
    r2s::clear_error();                                                                        \
    return r2s::voxel_reduce_impl<T>(rows, emit_ids, n_isects, N, v_means, v_conics, v_opac,   \
                                     st);                                                      \
  }

R2S_VOXEL_STAGE_API(f32, float)
R2S_VOXEL_STAGE_API(f64, double)

#undef R2S_VOXEL_STAGE_API

R2S_VOXEL_API(f32, float)
R2S_VOXEL_API(f64, double)

#undef R2S_VOXEL_API

}  // extern "C"
