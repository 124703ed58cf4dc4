// X-ray line-integral rasterizer: image = sum over each tile's Gaussian list
// of opacity * mu * exp(-sigma), sigma = 1/2 d^T conic d, skipping sigma < 0
// and |alpha| < 1e-5 (r2splat/cuda/csrc/RasterizeToPixelsFwd.cu:57-186), and
// its VJP (RasterizeToPixelsBwd.cu:77-480).
//
// Forward (raster_fwd_rows_kernel, tile sizes 8/16/32): blocks of eight
// waves per (view, tile), or per share of a heavy tile's list; the list is
// staged through LDS in batches of 512 pre-scaled records, and a lane sums a
// whole tile row of up to 16 pixels for the records of its group.  Partial
// tiles are added in a fixed order.  Other tile sizes use raster_fwd_kernel
// (one pixel per thread).
//
// Backward (raster_bwd_kernel): one lane per record in list order.  A lane
// walks its tile row by row (rows no lane of the wave can reach are skipped)
// and accumulates the moments sum(w), sum(w dx), sum(w dx^2), sum(w dy),
// sum(w dx dy), sum(w dy^2) of w = v exp(-sigma) over passing pixels, plus
// the per-pixel absolute mean gradients; the nine partials follow once per
// record.  They go out through float atomics (one-pass form) or as the
// record's row of a table that r2s_rows.h reduces per Gaussian (two-pass
// form).  With absolute gradients at tile size 16, raster_bwd_split_kernel
// partitions each block's records so that records whose (P d) keeps one
// sign over the tile run the cheaper |w|-moment form.  The two reference
// backward variants (per pixel, per Gaussian) compute the same sums and
// share these kernels.
#include "r2s_common.h"
#include "r2s_cull.h"
#include "r2s_payload.h"
#include "r2s_rows.h"
#include "r2s_scan.h"

#include <mutex>

// Partial tiles of r2s_rasterize_fwd_noalloc_*: a device array that each GPU
// holds from the library's load to the end of the process.  Host code never
// passes its name to a kernel (on the host it is a stand-in, not a device
// address): it uses the address hipGetSymbolAddress returns for the current
// device.
static __device__ __align__(256) unsigned char scratch[R2S_RASTER_SCRATCH_BYTES];

namespace r2s {
namespace {

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

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
__device__ __forceinline__ double fast_exp(double x) { return exp(x); }

constexpr int kBwdThreads = 256;
// Pixels of a row evaluated together: an unrolled 8-pixel body in a rolled
// loop keeps the kernel at 62 VGPRs (8 waves per SIMD) without spills.
constexpr int kChunk = 8;

template <typename T>
__global__ __launch_bounds__(1024) void raster_fwd_kernel(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, const int32_t *__restrict__ tile_offsets,
    const int32_t *__restrict__ flatten_ids, int64_t n_isects, uint32_t n_keys, uint32_t W,
    uint32_t H, uint32_t ts, uint32_t tw, uint32_t th, T *__restrict__ image) {
  using V2 = typename Vec<T>::v2;
  using V4 = typename Vec<T>::v4;
  extern __shared__ double smem_raw[];
  const uint32_t bs = ts * ts;
  V2 *s_xy = reinterpret_cast<V2 *>(smem_raw);
  V4 *s_q = reinterpret_cast<V4 *>(s_xy + bs + (bs & 1u));  // keep V4 16/32-byte aligned

  const uint32_t key = xcd_swizzle(blockIdx.x, n_keys);
  const uint32_t n_tiles = tw * th;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const uint32_t tr = threadIdx.x;
  const uint32_t ly = tr / ts, lx = tr - ly * ts;
  const uint32_t i = ty * ts + ly, j = tx * ts + lx;
  const bool inside = (i < H) && (j < W);
  const T px = static_cast<T>(j) + static_cast<T>(0.5);
  const T py = static_cast<T>(i) + static_cast<T>(0.5);

  const int64_t start = tile_offsets[key];
  const int64_t end = (key == n_keys - 1) ? n_isects : static_cast<int64_t>(tile_offsets[key + 1]);
  const T thr = static_cast<T>(kThr2);
  T acc = 0;
  for (int64_t b = start; b < end; b += bs) {
    __syncthreads();
    const int64_t idx = b + tr;
    if (idx < end) {
      const int64_t g = flatten_ids[idx];
      const V2 xy = *reinterpret_cast<const V2 *>(means2d + 2 * g);
      s_xy[tr] = xy;
      V4 q;
      q.x = conics[3 * g];
      q.y = conics[3 * g + 1];
      q.z = conics[3 * g + 2];
      q.w = opac[g] * mus[g];
      s_q[tr] = q;
    }
    __syncthreads();
    const int cnt = static_cast<int>(min(static_cast<int64_t>(bs), end - b));
    if (inside) {
#pragma unroll 4
      for (int k = 0; k < cnt; ++k) {
        const V2 xy = s_xy[k];
        const V4 q = s_q[k];
        const T dx = px - xy.x, dy = py - xy.y;
        const T sigma = static_cast<T>(0.5) * (q.x * dx * dx + q.z * dy * dy) + q.y * dx * dy;
        const T alpha = q.w * fast_exp(-sigma);
        const bool skip = (sigma < static_cast<T>(0)) || (fabs(alpha) < thr);
        acc += skip ? static_cast<T>(0) : alpha;
      }
    }
  }
  if (inside) image[static_cast<int64_t>(cam) * H * W + static_cast<int64_t>(i) * W + j] = acc;
}

// Forward for tile sizes 8, 16 and 32: kFwdWaves waves per (view, tile).
// A lane covers R = min(TS, 16) consecutive pixels of one tile row, so a
// record's row terms (dy, b dy, c dy^2) are computed once for R pixels; the
// TS^2 / R lanes covering the tile for one record form a group, and the
// 64 / (TS^2 / R) groups of a wave take different records of each LDS batch
// (4 per wave at TS = 16).  sigma log2(e) = (h_a dx + h_b dy) dx + h_c dy^2
// with pre-scaled coefficients, and the alpha test (sigma >= 0,
// |o mu e| >= 1e-5) is one unsigned compare of sl's bits against a limit
// staged per record (alpha_limit), so a pixel costs two FMAs, one
// v_exp_f32, one compare, a select and the accumulating FMA.  At the end
// each wave adds its groups' partial tiles across lanes and the block adds
// its waves' in order: a fixed order, so the result is deterministic (the
// per-pixel order differs from a plain list-order sum only by rounding).
constexpr int kFwdWaves = 8;
constexpr int kFwdBatch = 64 * kFwdWaves;

// One staged forward record: {x, y, h_a, h_b} and {h_c, o mu, limit bits, 0}.
template <typename T>
struct FwdRecord {
  typename Vec<T>::v4 p, q;
};

// Blocks per (view, tile) of the forward: tiles carry different record counts
// (max/mean 1.4 at config 4) and all of them are resident at once, so one
// block per tile leaves the heaviest tiles running alone at the end.  With
// `splits` blocks per tile, each sums an equal share of the tile's records
// into its own partial tile, and fwd_combine_kernel adds the partials in a
// fixed order (deterministic).
inline uint32_t fwd_splits(int64_t n_keys, int64_t n_isects) {
  if (n_keys <= 0) return 1;
  const int64_t per_tile = n_isects / n_keys;
  const int64_t s = per_tile / 1024;
  return static_cast<uint32_t>(s < 1 ? 1 : (s > 8 ? 8 : s));
}

// kPacked: each record's mean, conic and o mu come from the packed
// per-(view, Gaussian) payload (raster_pack_kernel: 32 bytes in float, one
// sector) instead of four arrays; the staged values, and so the image, are
// the same bit for bit.
template <typename T, int TS, bool kPacked>
__global__ __launch_bounds__(kFwdBatch) void raster_fwd_rows_kernel(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, const int32_t *__restrict__ tile_offsets,
    const int32_t *__restrict__ flatten_ids, int64_t n_isects, uint32_t n_keys, int64_t n_items,
    uint32_t W, uint32_t H, uint32_t tw, uint32_t th, uint32_t splits, T *__restrict__ image,
    T *__restrict__ partial, const T *__restrict__ payload) {
  using V2 = typename Vec<T>::v2;
  using V4 = typename Vec<T>::v4;
  constexpr int R = TS < 16 ? TS : 16;  // pixels per lane (a tile row, at most 16)
  constexpr int NL = TS * TS / R;        // lanes covering the tile for one record
  constexpr int G = 64 / NL;             // records in flight per wave
  constexpr int LPR = TS / R;            // lanes per tile row
  constexpr int NP = kFwdWaves * G;      // records in flight per block
  static_assert(G * NL == 64 && LPR * R == TS, "unsupported tile size");
  // Tile sizes up to 16: a lane covers a whole tile row, so all lanes use
  // the same column offsets dx_c = (x_c + 1/2) - mx of a record; they are
  // staged with it (TS values at a stride of TS + 4, which spreads a round's
  // records over the banks) instead of formed per lane and record.  The
  // batch is halved then, which keeps four blocks per CU.
  constexpr bool kStageDx = TS <= 16;
  constexpr int kBatch = kStageDx ? kFwdBatch / 2 : kFwdBatch;
  constexpr int kDxStride = TS + 4;
  // G - 1 records of padding after the batch: the record loop's last round
  // reads up to G - 1 entries past the batch's end.  Entries past the end
  // hold dead records (zero limit, which no pixel passes).
  __shared__ FwdRecord<T> s_rec[kBatch + G];
  __shared__ __align__(16) T s_dx[kStageDx ? (kBatch + G) * kDxStride : 1];
  __shared__ T s_part[kFwdWaves][TS * TS];

  // The splits of one tile are consecutive logical blocks (same XCD).
  const uint32_t lb = xcd_swizzle(blockIdx.x, gridDim.x);
  const uint32_t key = lb / splits, split = lb - key * splits;
  const uint32_t n_tiles = tw * th;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = static_cast<int>(wave_index()), lane = static_cast<int>(lane_id());
  const int gl = lane % NL;
  const int ly = gl / LPR, lx0 = (gl % LPR) * R;
  const T half = static_cast<T>(0.5);
  const T py = static_cast<T>(static_cast<int>(ty) * TS + ly) + half;
  const T px0 = static_cast<T>(static_cast<int>(tx) * TS + lx0) + half;
  const T l = static_cast<T>(kLog2e), hl = static_cast<T>(0.5 * kLog2e);

  const int64_t t0 = tile_offsets[key];
  const int64_t t1 = (key == n_keys - 1) ? n_isects : static_cast<int64_t>(tile_offsets[key + 1]);
  const int64_t start = t0 + (t1 - t0) * split / splits;
  const int64_t end = t0 + (t1 - t0) * (split + 1) / splits;
  T acc[R], pxk[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    acc[q] = 0;
    // The lane's pixel centres, kept in registers across the record loop
    // (otherwise some are recomputed per record).
    pxk[q] = px0 + static_cast<T>(q);
    if (!kStageDx) asm volatile("" : "+v"(pxk[q]));
  }
  const int wave_first = wave * G;  // uniform: the record loop below is a scalar loop
  const int group = lane / NL;
  if (tid < G) {
    FwdRecord<T> dead;
    dead.p.x = dead.p.y = dead.p.z = dead.p.w = 0;
    dead.q.x = dead.q.y = dead.q.w = 0;
    dead.q.z = limit_as_value(static_cast<typename Bits<T>::type>(0));
    s_rec[kBatch + tid] = dead;
    if (kStageDx) {
#pragma unroll
      for (int c = 0; c < TS; ++c) s_dx[(kBatch + tid) * kDxStride + c] = 0;
    }
  }
  // The tile's first pixel centre; x_c + 1/2 = px_tile + c exactly.
  const T px_tile = static_cast<T>(static_cast<int>(tx) * TS) + half;
  for (int64_t base = start; base < end; base += kBatch) {
    __syncthreads();
    const int64_t idx = base + tid;
    if (tid < kBatch) {
      const int64_t g = idx < end ? static_cast<int64_t>(flatten_ids[idx]) : -1;
      FwdRecord<T> rec;
      V4 &p = rec.p, &q = rec.q;
      if (g >= 0 && g < n_items) {
        if (kPacked) {
          // Payload: {x, y, a, b} {c, o mu, limit, hy}.
          const V4 *src = reinterpret_cast<const V4 *>(payload + kPayloadValues * g);
          const V4 a = src[0], b = src[1];
          p.x = a.x;
          p.y = a.y;
          p.z = hl * a.z;
          p.w = l * a.w;
          q.x = hl * b.x;
          q.y = b.y;
          q.z = b.z;  // alpha_limit(o mu, finite unscaled geometry)
        } else {
          const V2 xy = *reinterpret_cast<const V2 *>(means2d + 2 * g);
          p.x = xy.x;
          p.y = xy.y;
          p.z = hl * conics[3 * g];
          p.w = l * conics[3 * g + 1];
          q.x = hl * conics[3 * g + 2];
          q.y = opac[g] * mus[g];
        }
        // The alpha test's limit on the bits of sl (alpha_limit), kept in q.z.
        // Packed: finite scaled geometry implies finite unscaled geometry, so
        // the payload's limit is alpha_limit's value, and non-finite scaled
        // geometry gives the sign-bit limit either way (no log2 here).
        const bool fin = isfinite(p.x) && isfinite(p.y) && isfinite(p.z) && isfinite(p.w) &&
                         isfinite(q.x);
        if (kPacked)
          q.z = fin ? q.z : limit_as_value(Bits<T>::kSign);
        else
          q.z = limit_as_value(alpha_limit(q.y, fin, kThr2));
      } else {  // never passes
        p.x = p.y = p.z = p.w = 0;
        q.x = q.y = 0;
        q.z = limit_as_value(static_cast<typename Bits<T>::type>(0));
      }
      q.w = 0;
      s_rec[tid] = rec;
      if (kStageDx) {
        // The walking lanes' px_k - mx (px_k = px_tile + k for every lane),
        // with the one rounding they would give it.
#pragma unroll
        for (int c = 0; c < TS; c += 4) {
          V4 d;
          d.x = (px_tile + static_cast<T>(c)) - p.x;
          d.y = (px_tile + static_cast<T>(c + 1)) - p.x;
          d.z = (px_tile + static_cast<T>(c + 2)) - p.x;
          d.w = (px_tile + static_cast<T>(c + 3)) - p.x;
          *reinterpret_cast<V4 *>(s_dx + tid * kDxStride + c) = d;
        }
      }
    }
    __syncthreads();
    const int cnt = static_cast<int>(min(static_cast<int64_t>(kBatch), end - base));
    for (int jb = wave_first; jb < cnt; jb += NP) {
      // A group past the batch's end reads a dead record.
      const V4 p = s_rec[jb + group].p;
      const V4 q = s_rec[jb + group].q;
      T dxs[R];
      if (kStageDx) {
#pragma unroll
        for (int c = 0; c < R; c += 4)
          *reinterpret_cast<V4 *>(dxs + c) =
              *reinterpret_cast<const V4 *>(s_dx + (jb + group) * kDxStride + c);
      }
      const typename Bits<T>::type lim = bits_of(q.z);
      const T dy = py - p.y;
      const T B = p.w * dy, C = q.x * dy * dy;
      // dx as the reference forms it (pixel centre minus mean, one rounding):
      // a quadratic in the column offset instead would cancel badly where
      // sigma is small but the offset's terms are large (sub-pixel
      // footprints far along the row).
#pragma unroll
      for (int k = 0; k < R; ++k) {
        const T dx = kStageDx ? dxs[k] : pxk[k] - p.x;
        const T sl = (p.z * dx + B) * dx + C;
        add_passing(sl, lim, q.y, acc[k]);
      }
    }
  }
  // The wave's G groups cover the same pixels: their partial tiles are added
  // across lanes first (group g + 1 onto g, pairs of groups, ...; a fixed
  // order), so the block stages one partial tile per wave.
#pragma unroll
  for (int off = NL; off < 64; off *= 2) {
#pragma unroll
    for (int k = 0; k < R; ++k) acc[k] += __shfl_xor(acc[k], off, 64);
  }
  if (lane < NL) {
#pragma unroll
    for (int k = 0; k < R; ++k) s_part[wave][ly * TS + lx0 + k] = acc[k];
  }
  __syncthreads();
  for (int pix = tid; pix < TS * TS; pix += kFwdBatch) {
    T sum = s_part[0][pix];
#pragma unroll
    for (int w = 1; w < kFwdWaves; ++w) sum += s_part[w][pix];
    if (splits > 1) {
      partial[(static_cast<int64_t>(key) * splits + split) * (TS * TS) + pix] = sum;
      continue;
    }
    const int i = static_cast<int>(ty) * TS + pix / TS, j = static_cast<int>(tx) * TS + pix % TS;
    if (i < static_cast<int>(H) && j < static_cast<int>(W))
      image[static_cast<int64_t>(cam) * H * W + static_cast<int64_t>(i) * W + j] = sum;
  }
}

// image = sum over the splits of each tile's partial tiles, in split order.
template <typename T, int TS>
__global__ __launch_bounds__(TS * TS) void fwd_combine_kernel(const T *__restrict__ partial,
                                                              uint32_t splits, uint32_t W,
                                                              uint32_t H, uint32_t tw,
                                                              uint32_t th, T *__restrict__ image) {
  const uint32_t key = blockIdx.x, pix = threadIdx.x;
  const uint32_t n_tiles = tw * th;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const T *p = partial + static_cast<int64_t>(key) * splits * (TS * TS) + pix;
  T sum = p[0];
  for (uint32_t s = 1; s < splits; ++s) sum += p[s * (TS * TS)];
  const uint32_t i = ty * TS + pix / TS, j = tx * TS + pix % TS;
  if (i < H && j < W) image[static_cast<int64_t>(cam) * H * W + static_cast<int64_t>(i) * W + j] = sum;
}

// One backward record in registers.
template <typename T>
struct RasterRecord {
  bool live;          // a valid record whose pixels can pass the alpha test
  T mx, my, a, b, c, o, mu, om;
  T ha, hb, hc;       // a/2, b, c/2 pre-scaled by log2(e)
  typename Bits<T>::type lim;  // the alpha test on the bits of sl (alpha_limit)
  int i0, i1;         // rows the alpha-test ellipse reaches (all rows when not PD)
  bool pd;            // conic positive definite and finite (sigma finite, >= 0 up to rounding)
};

template <typename T>
__device__ __forceinline__ void load_raster_record(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, int64_t g, int64_t n_items, bool in_list, int oy, int y1,
    RasterRecord<T> &rec) {
  rec.live = in_list && g >= 0 && g < n_items;
  rec.o = rec.live ? opac[g] : static_cast<T>(0);
  rec.mu = rec.live ? mus[g] : static_cast<T>(0);
  rec.om = rec.o * rec.mu;
  // |alpha| <= |o mu| for sigma >= 0: nothing passes (non-finite stays live).
  if (fabs(rec.om) < static_cast<T>(kThr2)) rec.live = false;
  if (!rec.live) {
    rec.o = rec.mu = rec.om = 0;
    rec.mx = rec.my = rec.a = rec.b = rec.c = rec.ha = rec.hb = rec.hc = 0;
    rec.lim = 0;
    rec.i0 = 0;
    rec.i1 = -1;
    rec.pd = true;
    return;
  }
  rec.mx = means2d[2 * g];
  rec.my = means2d[2 * g + 1];
  rec.a = conics[3 * g];
  rec.b = conics[3 * g + 1];
  rec.c = conics[3 * g + 2];
  rec.ha = static_cast<T>(0.5 * kLog2e) * rec.a;
  rec.hb = static_cast<T>(kLog2e) * rec.b;
  rec.hc = static_cast<T>(0.5 * kLog2e) * rec.c;
  rec.lim = alpha_limit(rec.om, isfinite(rec.mx) && isfinite(rec.my) && isfinite(rec.a) &&
                                   isfinite(rec.b) && isfinite(rec.c),
                        kThr2);
  const Cull2<T> cu = cull2_setup(rec.a, rec.b, rec.c, fabs(rec.om), kThr2);
  rec.pd = cu.ok;
  rec.i0 = oy;
  rec.i1 = y1;
  if (cu.ok && !index_range<T>(rec.my, -cu.hy, cu.hy, oy, y1, rec.i0, rec.i1)) rec.live = false;
}

// Per-(view, Gaussian) payload of the packed forward and of the two-pass
// backward: what their record loads need, packed as kPayloadValues values of
// T (32 bytes in float) -- mean, conic, o mu, the alpha limit's bits and the
// culling half-height hy (negative when the conic is not positive definite)
// -- so that a record's gather touches one sector instead of four arrays'
// lines, and the per-record culling setup runs once per Gaussian.  The rows
// need no o or mu apart from o mu: the reduction forms the opacity and mu
// partials from T0.  The fused projection (r2s_project_pack_fwd_*) writes
// the same payload (store_payload) from its own results.

// With z_xy non-null it also stores zeros into the backward's outputs
// (v_xy_abs may be null), which the reduction then overwrites for every pair
// with records -- one launch fewer than a separate fill.
template <typename T>
__global__ __launch_bounds__(256) void raster_pack_kernel(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, int64_t n_items, T *__restrict__ payload, T *__restrict__ z_xy,
    T *__restrict__ z_abs, T *__restrict__ z_conic, T *__restrict__ z_opac,
    T *__restrict__ z_mu) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= n_items) return;
  if (z_xy != nullptr) store_raster_zeros(g, z_xy, z_abs, z_conic, z_opac, z_mu);
  store_payload(payload, g, means2d[2 * g], means2d[2 * g + 1], conics[3 * g],
                conics[3 * g + 1], conics[3 * g + 2], opac[g] * mus[g]);
}

// load_raster_record from the packed payload (o and mu are left zero).
template <typename T>
__device__ __forceinline__ void load_raster_record_packed(const T *__restrict__ payload,
                                                          int64_t g, int64_t n_items, bool in_list,
                                                          int oy, int y1, RasterRecord<T> &rec) {
  using V4 = typename Vec<T>::v4;
  rec.live = in_list && g >= 0 && g < n_items;
  V4 p0, p1;
  if (rec.live) {
    const V4 *src = reinterpret_cast<const V4 *>(payload + kPayloadValues * g);
    p0 = src[0];
    p1 = src[1];
  } else {
    p0.x = p0.y = p0.z = p0.w = 0;
    p1.x = p1.y = p1.z = p1.w = 0;
  }
  rec.o = rec.mu = 0;
  rec.om = p1.y;
  // |alpha| <= |o mu| for sigma >= 0: nothing passes (non-finite stays live).
  if (fabs(rec.om) < static_cast<T>(kThr2)) rec.live = false;
  if (!rec.live) {
    rec.om = 0;
    rec.mx = rec.my = rec.a = rec.b = rec.c = rec.ha = rec.hb = rec.hc = 0;
    rec.lim = 0;
    rec.i0 = 0;
    rec.i1 = -1;
    rec.pd = true;
    return;
  }
  rec.mx = p0.x;
  rec.my = p0.y;
  rec.a = p0.z;
  rec.b = p0.w;
  rec.c = p1.x;
  rec.ha = static_cast<T>(0.5 * kLog2e) * rec.a;
  rec.hb = static_cast<T>(kLog2e) * rec.b;
  rec.hc = static_cast<T>(0.5 * kLog2e) * rec.c;
  rec.lim = bits_of(p1.z);
  rec.pd = p1.w >= static_cast<T>(0);
  rec.i0 = oy;
  rec.i1 = y1;
  if (rec.pd && !index_range<T>(rec.my, -p1.w, p1.w, oy, y1, rec.i0, rec.i1)) rec.live = false;
}

// Moments of one tile row for one record: s0 = sum w, s1 = sum w dx,
// s2 = sum w dx^2 over the row's passing pixels (w = v exp(-sigma)), and
// px, py = sums of |w (P d)_x|, |w (P d)_y|.  vv holds the row's upstream
// gradient (zero beyond the image).  kGuard: also exclude columns k >= nx
// explicitly -- needed only for records whose sigma may be NaN (non-finite
// geometry passes the alpha test there), for which v = 0 would not make
// w = 0.
template <typename T, int R, bool kExact, bool kAbs, bool kGuard>
__device__ __forceinline__ void raster_row(const RasterRecord<T> &rec, const T (&vv)[R], int k0,
                                           T dx0, int nx, int nts, T B, T C, T bdy, T cdy,
                                           T &s0, T &s1, T &s2, T &px, T &py) {
#pragma unroll
  for (int kk = 0; kk < R; ++kk) {
    const int k = k0 + kk;
    if (!kExact && k >= nts) break;
    const T dx = dx0 + static_cast<T>(k);
    const T sl = (rec.ha * dx + B) * dx + C;
    const T e = neg_exp2(sl);
    bool skip = !alpha_pass(sl, rec.lim);
    if (kGuard) skip = skip || k >= nx;
    const T p = vv[kk] * e;  // unconditional, not a branch around the load and exp
    const T w = skip ? static_cast<T>(0) : p;
    s0 += w;
    const T wx = w * dx;
    s1 += wx;
    s2 += wx * dx;
    if (kAbs) {  // |w t| = |w| |t|: one FMA with source modifiers
      px = fma(fabs(w), fabs(rec.a * dx + bdy), px);
      py = fma(fabs(w), fabs(rec.b * dx + cdy), py);
    }
  }
}

// The whole tile of one record when every tile of the wave lies inside the
// image (no column guard).  The column offsets dx_k are the same on every
// row, so they are kept in registers, and the column sums W_k = sum over
// rows of w accumulate per column: T0, T1, T2 then follow from W_k once per
// record, which leaves three accumulations per pixel (W_k, s0, s1) instead
// of four.  Rows outside the record's reach test against a zero limit
// (every pixel fails), so the upstream gradient is loaded without masks.
template <typename T, int R, bool kAbs>
__device__ __forceinline__ void raster_tile_full(const RasterRecord<T> &rec,
                                                 const T *__restrict__ vimg, uint32_t W, int ox,
                                                 int oy, T dx0, T &T0, T &T1, T &T2, T &Y0, T &Y1,
                                                 T &YY, T &PX, T &PY) {
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
  for (int ly = 0; ly < R; ++ly) {
    const int i = oy + ly;
    const bool in_row = rec.live && i >= rec.i0 && i <= rec.i1;
    if (ballot(in_row) == 0) continue;
    const T dy = (static_cast<T>(i) + half) - rec.my;
    const T B = rec.hb * dy, C = rec.hc * dy * dy;
    const T bdy = rec.b * dy, cdy = rec.c * dy;
    const typename Bits<T>::type lim = in_row ? rec.lim : 0;
    const T *__restrict__ vrow = vimg + static_cast<int64_t>(in_row ? i : oy) * W + ox;
    T s0 = 0, s1 = 0, px = 0, py = 0;
#pragma unroll
    for (int h = 0; h < R; h += kChunk) {
      T vv[kChunk];
#pragma unroll
      for (int q = 0; q < kChunk / kq; ++q)
        *reinterpret_cast<Q *>(vv + q * kq) = *reinterpret_cast<const Q *>(vrow + h + q * kq);
#pragma unroll
      for (int kk = 0; kk < kChunk; ++kk) {
        // Explicit FMAs: written as products plus sums, the products of the
        // row-invariant dx_k would be hoisted out of the row loop into 48
        // more registers for no saving.
        const T dx = dxk[h + kk];
        const T sl = fma(fma(rec.ha, dx, B), dx, C);
        const T e = neg_exp2(sl);
        // The product is formed unconditionally: as an operand of the
        // conditional it would become a branch around its load and exp.
        const T p = vv[kk] * e;
        const T w = alpha_pass(sl, lim) ? p : static_cast<T>(0);
        wk[h + kk] += w;
        s0 += w;
        s1 = fma(w, dx, s1);
        if (kAbs) {
          px = fma(fabs(w), fabs(fma(rec.a, dx, bdy)), px);
          py = fma(fabs(w), fabs(fma(rec.b, dx, cdy)), py);
        }
      }
    }
    Y0 += dy * s0;
    YY += dy * (dy * s0);
    Y1 += dy * s1;
    if (kAbs) {
      PX += px;
      PY += py;
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

// Sums over one record's tile: T_k = sum w dx^k (k = 0, 1, 2), Y0 = sum w dy,
// Y1 = sum w dx dy, YY = sum w dy^2; PX, PY = sums of the per-pixel absolute
// mean gradients |w (P d)_x|, |w (P d)_y|.
template <typename T>
struct TileSums {
  T T0, T1, T2, Y0, Y1, YY, PX, PY;
};

// The sums of one record (one lane) over its tile: the whole-tile form when
// every tile of the wave lies inside the image, else row by row with masked
// loads.  Wave-uniform branches only.
template <typename T, int R, bool kExact, bool kAbs>
__device__ __forceinline__ TileSums<T> raster_record_sums(const RasterRecord<T> &rec,
                                                          const T *__restrict__ vimg, uint32_t W,
                                                          int ox, int oy, int nx, int nts,
                                                          bool vec, T dx0) {
  const T half = static_cast<T>(0.5);
  TileSums<T> s = {0, 0, 0, 0, 0, 0, 0, 0};
  // Columns past the image matter only for records whose sigma may be
  // non-finite (uniform over the wave).
  const bool guard = ballot(rec.live && !rec.pd && nx < nts) != 0;
  bool full = false;
  if constexpr (kExact && R <= 16 && R % kChunk == 0) full = vec && ballot(nx < nts) == 0;
  if (full && ballot(rec.live) != 0) {
    raster_tile_full<T, R, kAbs>(rec, vimg, W, ox, oy, dx0, s.T0, s.T1, s.T2, s.Y0, s.Y1, s.YY,
                                 s.PX, s.PY);
  } else if (ballot(rec.live) != 0) {
    for (int ly = 0; ly < R; ++ly) {
      if (!kExact && ly >= nts) break;
      const int i = oy + ly;
      const bool in_row = rec.live && i >= rec.i0 && i <= rec.i1;
      if (ballot(in_row) == 0) continue;
      const T dy = (static_cast<T>(i) + half) - rec.my;
      const T B = rec.hb * dy, C = rec.hc * dy * dy;
      const T bdy = rec.b * dy, cdy = rec.c * dy;
      const T *__restrict__ vrow = vimg + static_cast<int64_t>(in_row ? i : 0) * W + ox;
      T s0 = 0, s1 = 0, s2 = 0, px = 0, py = 0;
      constexpr int CH = R < kChunk ? R : kChunk;
#pragma unroll 1
      for (int k0 = 0; k0 < R; k0 += CH) {
        if (!kExact && k0 >= nts) break;
        T vv[CH];
        if (vec)
          load_grad_row<T, CH, true>(vrow + k0, in_row, nx - k0, nts - k0, vv);
        else
          load_grad_row<T, CH, false>(vrow + k0, in_row, nx - k0, nts - k0, vv);
        if (guard)
          raster_row<T, CH, kExact, kAbs, true>(rec, vv, k0, dx0, nx, nts, B, C, bdy, cdy, s0,
                                                s1, s2, px, py);
        else
          raster_row<T, CH, kExact, kAbs, false>(rec, vv, k0, dx0, nx, nts, B, C, bdy, cdy, s0,
                                                 s1, s2, px, py);
      }
      s.T0 += s0;
      s.T1 += s1;
      s.T2 += s2;
      const T dys0 = dy * s0;
      s.Y0 += dys0;
      s.YY += dy * dys0;
      s.Y1 += dy * s1;
      if (kAbs) {
        s.PX += px;
        s.PY += py;
      }
    }
  }
  return s;
}

// Per-pixel terms of RasterizeToPixelsBwd.cu summed over the tile, with
// v_sigma = -v alpha, d sigma / d mean = -(P d) and
// d sigma / d conic = (dx^2 / 2, dx dy, dy^2 / 2): the nine partials of one
// record (zero for dead records), in row order
// {v_xy.x, v_xy.y, v_conic.a, v_conic.b, v_conic.c, v_opac, v_mu, v_xy_abs.x, v_xy_abs.y}.
template <typename T, bool kAbs>
__device__ __forceinline__ void raster_partials(const RasterRecord<T> &rec, const TileSums<T> &s,
                                                T (&v)[9]) {
  const T half = static_cast<T>(0.5);
  const T om = rec.om;
  v[0] = om * (rec.a * s.T1 + rec.b * s.Y0);
  v[1] = om * (rec.c * s.Y0 + rec.b * s.T1);
  v[2] = -half * om * s.T2;
  v[3] = -om * s.Y1;
  v[4] = -half * om * s.YY;
  v[5] = rec.mu * s.T0;
  v[6] = rec.o * s.T0;
  v[7] = kAbs ? fabs(om) * s.PX : static_cast<T>(0);
  v[8] = kAbs ? fabs(om) * s.PY : static_cast<T>(0);
}

// Records in tile order (tile_offsets, flatten_ids; isect_ids optional), one
// lane per record.  kRows = false: each record's nine partials go out
// through global atomics.  kRows = true: they are stored as the row
// isect_src[r] of `rows` (see r2s_rows.h), zeros included.  kExact: the tile
// size equals R (loops fully unrolled); otherwise ts <= R at run time.
template <typename T, int R, bool kExact, bool kAbs, bool kRows>
__global__ __launch_bounds__(kBwdThreads) void raster_bwd_kernel(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, const int32_t *__restrict__ tile_offsets,
    const int64_t *__restrict__ isect_ids, const int32_t *__restrict__ flatten_ids,
    const int32_t *__restrict__ isect_src, int64_t n_isects, uint32_t n_keys, int64_t n_items,
    const T *__restrict__ v_image, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw,
    uint32_t th, bool vec, T *__restrict__ v_xy_abs, T *__restrict__ v_xy,
    T *__restrict__ v_conic, T *__restrict__ v_opac, T *__restrict__ v_mu,
    T *__restrict__ rows, const T *__restrict__ payload) {
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
  const uint32_t n_tiles = tw * th;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const int ox = static_cast<int>(tx) * nts, oy = static_cast<int>(ty) * nts;
  const int nx = min(nts, static_cast<int>(W) - ox);
  const int ny = min(nts, static_cast<int>(H) - oy);
  const T *__restrict__ vimg = v_image + static_cast<int64_t>(cam) * H * W;
  RasterRecord<T> rec;
  if (kRows)
    load_raster_record_packed(payload, g, n_items, key_ok, oy, oy + ny - 1, rec);
  else
    load_raster_record(means2d, conics, opac, mus, g, n_items, key_ok, oy, oy + ny - 1, rec);
  const T dx0 = (static_cast<T>(ox) + static_cast<T>(0.5)) - rec.mx;
  const TileSums<T> s =
      raster_record_sums<T, R, kExact, kAbs>(rec, vimg, W, ox, oy, nx, nts, vec, dx0);
  if (!key_ok) return;
  T v[9];
  raster_partials<T, kAbs>(rec, s, v);
  if (kRows) {
    // The opacity and mu partials are mu T0 and o T0: the row keeps T0 and
    // the reduction scales its sum.
    if (kAbs) {
      const T r8[8] = {v[0], v[1], v[2], v[3], v[4], s.T0, v[7], v[8]};
      store_row(rows, isect_src[r], r8);
    } else {
      const T r6[6] = {v[0], v[1], v[2], v[3], v[4], s.T0};
      store_row(rows, isect_src[r], r6);
    }
    return;
  }
  if (!rec.live) return;
  bool any = false;
#pragma unroll
  for (int c = 0; c < 9; ++c) any = any || v[c] != 0;
  if (!any) return;  // nothing to add
  atomic_add(v_xy + 2 * g, v[0]);
  atomic_add(v_xy + 2 * g + 1, v[1]);
  if (kAbs) {
    atomic_add(v_xy_abs + 2 * g, v[7]);
    atomic_add(v_xy_abs + 2 * g + 1, v[8]);
  }
  atomic_add(v_conic + 3 * g, v[2]);
  atomic_add(v_conic + 3 * g + 1, v[3]);
  atomic_add(v_conic + 3 * g + 2, v[4]);
  atomic_add(v_opac + g, v[5]);
  atomic_add(v_mu + g, v[6]);
}

// ------------------------------------------- sign-split backward (rows) ---
//
// When (P d)_x = a dx + b dy keeps one sign over a record's tile,
// sum |w| |(P d)_x| = |a sum |w| dx + b sum |w| dy|: the absolute mean
// gradient costs two accumulations per pixel (|w| and |w| dx per row) instead
// of two FMAs and two absolute-value FMAs; likewise (P d)_y = b dx + c dy.
// Waves are SIMD, so the cheaper form pays only where all 64 records of a
// wave qualify: each block of kSplitThreads records is partitioned in LDS
// (stable), qualifying whole-tile records first, and the waves then take
// the records of their new slots.  Each record's row goes to isect_src[r]
// whichever lane computed it, so the partition does not change the output.

constexpr int kSplitThreads = 256;
// A tile qualifies when min |p dx + q dy| over its pixel centres is at least
// this fraction of max(|p| |dx|) + max(|q| |dy|), which bounds the
// cancellation in |p sum |w| dx + q sum |w| dy| to a factor of 64.
constexpr double kSignMargin = 1.0 / 64.0;

template <typename T>
__device__ __forceinline__ bool one_sign(T p, T q, T dxa, T dxb, T dya, T dyb) {
  const T t0 = fma(p, dxa, q * dya), t1 = fma(p, dxb, q * dya);
  const T t2 = fma(p, dxa, q * dyb), t3 = fma(p, dxb, q * dyb);
  const T lo = fmin(fmin(t0, t1), fmin(t2, t3)), hi = fmax(fmax(t0, t1), fmax(t2, t3));
  const T scale = fabs(p) * fmax(fabs(dxa), fabs(dxb)) + fabs(q) * fmax(fabs(dya), fabs(dyb));
  const T m = static_cast<T>(kSignMargin) * scale;
  return lo >= m || hi <= -m;  // false for NaN
}

// raster_tile_full for a record whose (P d)_x and (P d)_y keep one sign over
// the tile: per row s0 = sum w, s1 = sum w dx, a0 = sum |w|, a1 = sum |w| dx,
// column sums W_k of w; then PX = |a A1 + b AY|, PY = |b A1 + c AY| with
// A1 = sum |w| dx and AY = sum |w| dy over the tile.
template <typename T, int R>
__device__ __forceinline__ TileSums<T> raster_tile_signed(const RasterRecord<T> &rec,
                                                          const T *__restrict__ vimg, uint32_t W,
                                                          int ox, int oy, T dx0) {
  using Q = typename Quad<T>::type;
  constexpr int kq = Quad<T>::n;
  TileSums<T> s = {0, 0, 0, 0, 0, 0, 0, 0};
  T dxk[R], wk[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    dxk[k] = dx0 + static_cast<T>(k);
    wk[k] = 0;
  }
  T A1 = 0, AY = 0;
  const T half = static_cast<T>(0.5);
#pragma unroll 1
  for (int ly = 0; ly < R; ++ly) {
    const int i = oy + ly;
    const bool in_row = rec.live && i >= rec.i0 && i <= rec.i1;
    if (ballot(in_row) == 0) continue;
    const T dy = (static_cast<T>(i) + half) - rec.my;
    const T B = rec.hb * dy, C = rec.hc * dy * dy;
    const typename Bits<T>::type lim = in_row ? rec.lim : 0;
    const T *__restrict__ vrow = vimg + static_cast<int64_t>(i) * W + ox;
    T s0 = 0, s1 = 0, a0 = 0, a1 = 0;
#pragma unroll
    for (int h = 0; h < R; h += kChunk) {
      T vv[kChunk];
#pragma unroll
      for (int q = 0; q < kChunk / kq; ++q)
        *reinterpret_cast<Q *>(vv + q * kq) = *reinterpret_cast<const Q *>(vrow + h + q * kq);
#pragma unroll
      for (int kk = 0; kk < kChunk; ++kk) {
        const T dx = dxk[h + kk];
        const T sl = fma(fma(rec.ha, dx, B), dx, C);
        const T e = neg_exp2(sl);
        // The product is formed unconditionally: as an operand of the
        // conditional it would become a branch around its load and exp.
        const T p = vv[kk] * e;
        const T w = alpha_pass(sl, lim) ? p : static_cast<T>(0);
        wk[h + kk] += w;
        s0 += w;
        s1 = fma(w, dx, s1);
        a0 += fabs(w);
        a1 = fma(fabs(w), dx, a1);
      }
    }
    s.Y0 += dy * s0;
    s.YY += dy * (dy * s0);
    s.Y1 += dy * s1;
    AY = fma(dy, a0, AY);
    A1 += a1;
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const T wx = wk[k] * dxk[k];
    s.T0 += wk[k];
    s.T1 += wx;
    s.T2 += wx * dxk[k];
  }
  s.PX = fabs(fma(rec.a, A1, rec.b * AY));
  s.PY = fabs(fma(rec.b, A1, rec.c * AY));
  return s;
}

// What the partition moves through LDS per record: the fields of a
// RasterRecord loaded from the packed payload that the rows pass reads (o
// and mu stay zero there; the log2(e)-scaled conic is recomputed), ten words
// in float instead of sixteen, so more blocks fit a CU.
template <typename T>
struct SplitRecord {
  T mx, my, a, b, c, om;
  typename Bits<T>::type lim;
  int i0, i1;
  uint32_t flags;  // 1: live, 2: pd
};

template <typename T>
__device__ __forceinline__ SplitRecord<T> split_record(const RasterRecord<T> &r) {
  SplitRecord<T> s;
  s.mx = r.mx;
  s.my = r.my;
  s.a = r.a;
  s.b = r.b;
  s.c = r.c;
  s.om = r.om;
  s.lim = r.lim;
  s.i0 = r.i0;
  s.i1 = r.i1;
  s.flags = (r.live ? 1u : 0u) | (r.pd ? 2u : 0u);
  return s;
}

// The record as load_raster_record_packed forms it (same expressions).
template <typename T>
__device__ __forceinline__ RasterRecord<T> raster_record(const SplitRecord<T> &s) {
  RasterRecord<T> r;
  r.live = (s.flags & 1u) != 0;
  r.pd = (s.flags & 2u) != 0;
  r.mx = s.mx;
  r.my = s.my;
  r.a = s.a;
  r.b = s.b;
  r.c = s.c;
  r.o = r.mu = 0;
  r.om = s.om;
  r.ha = static_cast<T>(0.5 * kLog2e) * r.a;
  r.hb = static_cast<T>(kLog2e) * r.b;
  r.hc = static_cast<T>(0.5 * kLog2e) * r.c;
  r.lim = s.lim;
  r.i0 = s.i0;
  r.i1 = s.i1;
  return r;
}

// The two-pass (rows) backward with absolute gradients at tile size 16 over
// an image whose rows allow 16-byte loads.
template <typename T>
__global__ __launch_bounds__(kSplitThreads) void raster_bwd_split_kernel(
    const T *__restrict__ payload, const int32_t *__restrict__ tile_offsets,
    const int64_t *__restrict__ isect_ids, const int32_t *__restrict__ flatten_ids,
    const int32_t *__restrict__ isect_src, int64_t n_isects, uint32_t n_keys, int64_t n_items,
    const T *__restrict__ v_image, uint32_t W, uint32_t H, uint32_t tw, uint32_t th,
    T *__restrict__ rows) {
  constexpr int R = 16;
  constexpr int kWaves = kSplitThreads / 64;
  __shared__ WordMajor<SplitRecord<T>, kSplitThreads> s_rec;
  __shared__ int32_t s_r[kSplitThreads];
  __shared__ uint32_t s_key[kSplitThreads];
  __shared__ uint32_t s_count[kWaves];
  const uint32_t wave = wave_index(), lane = lane_id();
  const int64_t rb = static_cast<int64_t>(xcd_swizzle(blockIdx.x, gridDim.x)) * kSplitThreads +
                     64 * static_cast<int64_t>(wave);
  const int64_t r = rb + lane;
  bool in_list = r < n_isects;
  const uint32_t n_tiles = tw * th;
  const T half = static_cast<T>(0.5);
  // Load and classify each record in list order.  A record whose key is out
  // of range gets no row, as in raster_bwd_kernel.
  uint32_t key = 0;
  // Issued with the key's load, not after its check (one memory round trip
  // fewer before the record's own loads).
  const int32_t fid = in_list ? flatten_ids[r] : -1;
  if (rb < n_isects) {  // uniform per wave
    if (isect_ids != nullptr) {
      const int64_t k = in_list ? isect_ids[r] : 0;
      in_list = in_list && k >= 0 && k < static_cast<int64_t>(n_keys);
      key = in_list ? static_cast<uint32_t>(k) : 0u;
    } else {
      key = wave_record_key(tile_offsets, n_keys, n_isects, rb, r);
    }
  }
  const int64_t g = in_list ? static_cast<int64_t>(fid) : -1;
  bool fast = false;
  RasterRecord<T> rec;
  {
    const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
    const uint32_t ty = t / tw, tx = t - ty * tw;
    const int ox = static_cast<int>(tx) * R, oy = static_cast<int>(ty) * R;
    const int ny = min(R, static_cast<int>(H) - oy);
    load_raster_record_packed(payload, g, n_items, in_list, oy, oy + ny - 1, rec);
    if (in_list && ox + R <= static_cast<int>(W) && ny == R) {
      const T dxa = (static_cast<T>(ox) + half) - rec.mx;
      const T dya = (static_cast<T>(oy) + half) - rec.my;
      const T dxb = dxa + static_cast<T>(R - 1), dyb = dya + static_cast<T>(R - 1);
      fast = one_sign(rec.a, rec.b, dxa, dxb, dya, dyb) &&
             one_sign(rec.b, rec.c, dxa, dxb, dya, dyb);
    }
  }
  // Stable partition of the block, qualifying records first; each record
  // moves with its loaded state.
  const uint64_t fm = ballot(fast);
  if (lane == 0) s_count[wave] = static_cast<uint32_t>(__popcll(fm));
  __syncthreads();
  uint32_t before = 0, n_fast = 0;
#pragma unroll
  for (uint32_t w = 0; w < kWaves; ++w) {
    const uint32_t c = s_count[w];
    before += w < wave ? c : 0u;
    n_fast += c;
  }
  const uint32_t fast_lt = before + static_cast<uint32_t>(__popcll(fm & lanemask_lt()));
  const uint32_t slot = fast ? fast_lt : n_fast + (threadIdx.x - fast_lt);
  s_r[slot] = in_list ? static_cast<int32_t>(r) : -1;
  s_key[slot] = key;
  s_rec.store(static_cast<int>(slot), split_record(rec));
  __syncthreads();
  const int32_t rr = s_r[threadIdx.x];
  const bool valid = rr >= 0;
  if (ballot(valid) == 0) return;  // uniform per wave; no barrier follows
  key = s_key[threadIdx.x];
  rec = raster_record(s_rec.load(static_cast<int>(threadIdx.x)));
  const bool wave_fast = (wave + 1) * 64 <= n_fast;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const int ox = static_cast<int>(tx) * R, oy = static_cast<int>(ty) * R;
  const int nx = min(R, static_cast<int>(W) - ox);
  const T *__restrict__ vimg = v_image + static_cast<int64_t>(cam) * H * W;
  const T dx0 = (static_cast<T>(ox) + half) - rec.mx;
  TileSums<T> s;
  if (wave_fast)
    s = raster_tile_signed<T, R>(rec, vimg, W, ox, oy, dx0);
  else
    s = raster_record_sums<T, R, true, true>(rec, vimg, W, ox, oy, nx, R, true, dx0);
  if (!valid) return;
  T v[9];
  raster_partials<T, true>(rec, s, v);
  const T r8[8] = {v[0], v[1], v[2], v[3], v[4], s.T0, v[7], v[8]};
  store_row(rows, isect_src[rr], r8);
}

int check_raster_args(int64_t n_isects, int64_t C, int64_t N, uint32_t W, uint32_t H,
                      uint32_t ts, uint32_t tw, uint32_t th, const char *name) {
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size C=%lld N=%lld", name,
              (long long)C, (long long)N);
  // ts <= 32 first: ts * ts in 32 bits wraps for ts >= 65536.
  R2S_REQUIRE(ts > 0 && ts <= 32 && ts * ts <= 1024,
              "%s: tile_size must be positive with tile_size**2 <= 1024", name);
  R2S_REQUIRE(n_isects >= 0 && n_isects <= kInt32Max, "%s: bad n_isects %lld", name,
              (long long)n_isects);
  R2S_REQUIRE(static_cast<uint64_t>(tw) * ts >= W && static_cast<uint64_t>(th) * ts >= H,
              "%s: tile grid %ux%u of size %u does not cover %ux%u", name, tw, th, ts, W, H);
  R2S_REQUIRE(static_cast<uint64_t>(C) * tw * th <= 0xffffffffull, "%s: too many tiles", name);
  return R2S_OK;
}

// payload != null: the records' data come from the packed payload
// (raster_pack_kernel) and means2d .. mus are not read; tile sizes 8, 16, 32.
template <typename T>
int raster_fwd_impl(const T *means2d, const T *conics, const T *opac, const T *mus,
                    const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,
                    int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw,
                    uint32_t th, T *image, void *ws, size_t ws_bytes, r2s_stream_t st,
                    const T *payload = nullptr) {
  clear_error();
  const char *name = payload != nullptr ? "rasterize_to_pixels_fwd (packed)"
                                        : "rasterize_to_pixels_fwd";
  R2S_RETURN_IF(check_raster_args(n_isects, C, N, W, H, ts, tw, th, name));
  R2S_REQUIRE(payload == nullptr || ts == 8 || ts == 16 || ts == 32,
              "%s: tile_size %u; the packed forward takes 8, 16 or 32", name, ts);
  R2S_REQUIRE(payload == nullptr || reinterpret_cast<uintptr_t>(payload) % 16 == 0,
              "%s: payload not 16-byte aligned", name);
  hipStream_t stream = as_stream(st);
  const int64_t n_pix = C * static_cast<int64_t>(W) * H;
  if (n_pix == 0) return R2S_OK;
  R2S_REQUIRE(image != nullptr, "%s: null image", name);
  if (N == 0 || n_isects == 0) return device_fill<T>(image, n_pix, static_cast<T>(0), stream, name);
  R2S_REQUIRE((payload != nullptr || (means2d && conics && opac && mus)) && tile_offsets &&
                  flatten_ids,
              "%s: null pointer", name);
  const uint32_t n_keys = static_cast<uint32_t>(C) * tw * th;
  uint32_t splits = 1;
  T *partial = nullptr;
  if (ts == 8 || ts == 16 || ts == 32) {
    splits = fwd_splits(n_keys, n_isects);
    if (splits > 1) {
      const size_t need = static_cast<size_t>(n_keys) * splits * ts * ts * sizeof(T);
      if (ws == nullptr || ws_bytes < need) {
        set_error("%s: workspace of %zu bytes, %zu required", name, ws_bytes, need);
        return R2S_EWORKSPACE;
      }
      partial = static_cast<T *>(ws);
    }
  }
  R2S_REQUIRE(static_cast<uint64_t>(n_keys) * splits <= 0x7fffffffull, "%s: too many tiles",
              name);
#define R2S_RASTER_FWD_ROWS(TS)                                                                  \
  if (payload != nullptr)                                                                        \
    raster_fwd_rows_kernel<T, TS, true><<<dim3(n_keys * splits), dim3(kFwdBatch), 0, stream>>>( \
        nullptr, nullptr, nullptr, nullptr, tile_offsets, flatten_ids, n_isects, n_keys, C * N,  \
        W, H, tw, th, splits, image, partial, payload);                                          \
  else                                                                                           \
    raster_fwd_rows_kernel<T, TS, false><<<dim3(n_keys * splits), dim3(kFwdBatch), 0, stream>>>( \
        means2d, conics, opac, mus, tile_offsets, flatten_ids, n_isects, n_keys, C * N, W, H,    \
        tw, th, splits, image, partial, nullptr);                                                \
  if (splits > 1)                                                                                \
  fwd_combine_kernel<T, TS><<<dim3(n_keys), dim3(TS * TS), 0, stream>>>(partial, splits, W, H,   \
                                                                        tw, th, image)
  if (ts == 16) {
    R2S_RASTER_FWD_ROWS(16);
  } else if (ts == 8) {
    R2S_RASTER_FWD_ROWS(8);
  } else if (ts == 32) {
    R2S_RASTER_FWD_ROWS(32);
  } else {
    const uint32_t bs = ts * ts;
    const size_t smem =
        (bs + (bs & 1u)) * sizeof(typename Vec<T>::v2) + bs * sizeof(typename Vec<T>::v4);
    raster_fwd_kernel<T><<<dim3(n_keys), dim3(bs), smem, stream>>>(
        means2d, conics, opac, mus, tile_offsets, flatten_ids, n_isects, n_keys, W, H, ts, tw,
        th, image);
  }
#undef R2S_RASTER_FWD_ROWS
  return check_launch(name);
}

template <typename T, int R, bool kExact>
void launch_raster_bwd(const T *means2d, const T *conics, const T *opac, const T *mus,
                       const int32_t *tile_offsets, const int64_t *isect_ids,
                       const int32_t *flatten_ids, const int32_t *isect_src, int64_t n_isects,
                       uint32_t n_keys, int64_t n_items, const T *v_image, uint32_t W,
                       uint32_t H, uint32_t ts, uint32_t tw, uint32_t th, bool vec, T *v_xy_abs,
                       T *v_xy, T *v_conic, T *v_opac, T *v_mu, T *rows, const T *payload,
                       bool absgrad, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(ceil_div(n_isects, kBwdThreads)));
  const dim3 block(kBwdThreads);
#define R2S_RASTER_BWD_LAUNCH(ABS, ROWS)                                                         \
  raster_bwd_kernel<T, R, kExact, ABS, ROWS><<<grid, block, 0, stream>>>(                      \
      means2d, conics, opac, mus, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects,     \
      n_keys, n_items, v_image, W, H, ts, tw, th, vec, v_xy_abs, v_xy, v_conic, v_opac, v_mu,    \
      rows, payload)
  if (v_xy_abs != nullptr || (rows != nullptr && absgrad)) {
    if (rows != nullptr)
      R2S_RASTER_BWD_LAUNCH(true, true);
    else
      R2S_RASTER_BWD_LAUNCH(true, false);
  } else {
    if (rows != nullptr)
      R2S_RASTER_BWD_LAUNCH(false, true);
    else
      R2S_RASTER_BWD_LAUNCH(false, false);
  }
#undef R2S_RASTER_BWD_LAUNCH
}

// Rows of the raster backward: v_xy (2), v_conic (3), T0 = sum of v e^-sigma
// over the passing pixels, and, with absolute gradients, v_xy_abs (2).
constexpr int kRasterRowValues = 8;

int64_t raster_rows_bytes(int64_t n_isects, int dtype_bytes) {
  return n_isects * row_stride<kRasterRowValues>() * static_cast<int64_t>(dtype_bytes);
}

// Workspace of the two-pass backward: the rows, then the packed payload of
// the n_items (view, Gaussian) pairs.
int64_t raster_bwd_ws_bytes(int64_t n_isects, int64_t n_items, int dtype_bytes) {
  return raster_rows_bytes(n_isects, dtype_bytes) +
         n_items * kPayloadValues * static_cast<int64_t>(dtype_bytes);
}

// Second pass of the two-pass backward: per-Gaussian sums of the rows, with
// v_opac = mu sum(T0) and v_mu = o sum(T0).
// zeroed: the outputs hold zeros already (raster_pack_kernel stored them).
template <typename T>
int raster_reduce_impl(const T *rows, const int32_t *emit_ids, int64_t n_isects, int64_t C,
                       int64_t N, const T *opac, const T *mus, T *v_xy_abs, T *v_xy,
                       T *v_conic, T *v_opac, T *v_mu, r2s_stream_t st, bool zeroed = false) {
  const char *name = "rasterize_to_pixels_bwd (row reduction)";
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max && n_isects >= 0 && n_isects <= kInt32Max,
              "%s: bad size", name);
  if (C * N == 0) return R2S_OK;
  R2S_REQUIRE(v_xy && v_conic && v_opac && v_mu, "%s: null output", name);
  R2S_REQUIRE(n_isects == 0 || (rows && emit_ids && opac && mus), "%s: null pointer", name);
  R2S_REQUIRE(reinterpret_cast<uintptr_t>(rows) % 16 == 0, "%s: rows not 16-byte aligned", name);
  hipStream_t stream = as_stream(st);
  if (v_xy_abs != nullptr) {
    RowTargets<T, 8> tg = {{v_xy, v_xy + 1, v_conic, v_conic + 1, v_conic + 2, v_opac, v_xy_abs,
                            v_xy_abs + 1},
                           {2, 2, 3, 3, 3, 1, 2, 2},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, mus, nullptr, nullptr},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, v_mu, nullptr, nullptr},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, opac, nullptr, nullptr}};
    launch_row_reduce(rows, emit_ids, n_isects, C * N, tg, stream, zeroed);
  } else {
    RowTargets<T, 6> tg = {{v_xy, v_xy + 1, v_conic, v_conic + 1, v_conic + 2, v_opac},
                           {2, 2, 3, 3, 3, 1},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, mus},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, v_mu},
                           {nullptr, nullptr, nullptr, nullptr, nullptr, opac}};
    launch_row_reduce(rows, emit_ids, n_isects, C * N, tg, stream, zeroed);
  }
  return check_launch(name);
}

// two_pass: emit_ids / isect_src / ws give the two-pass form (r2s_rows.h);
// rows_only stops after the first pass (the rows are left in ws).
// given_payload (two-pass only): the packed payload was written by
// r2s_rasterize_pack_* already, ws holds only the rows, and means2d / conics
// are not read; zeroed: the outputs hold zeros already (that pack launch
// stored them).
template <typename T>
int raster_bwd_impl(const T *means2d, const T *conics, const T *opac, const T *mus,
                    const int32_t *tile_offsets, const int64_t *isect_ids,
                    const int32_t *flatten_ids, const int32_t *emit_ids,
                    const int32_t *isect_src, int64_t n_isects, const T *v_image, int64_t C,
                    int64_t N, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th,
                    T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac, T *v_mu, void *ws,
                    size_t ws_bytes, bool two_pass, r2s_stream_t st, bool rows_only = false,
                    bool absgrad = true, const T *given_payload = nullptr, bool zeroed = false) {
  clear_error();
  const char *name = given_payload ? "rasterize_to_pixels_bwd (two-pass, packed)"
                     : two_pass    ? "rasterize_to_pixels_bwd (two-pass)"
                     : isect_ids   ? "rasterize_to_pixels_bwd_per_gaussian"
                                   : "rasterize_to_pixels_bwd";
  R2S_RETURN_IF(check_raster_args(n_isects, C, N, W, H, ts, tw, th, name));
  R2S_REQUIRE(given_payload == nullptr || two_pass, "%s: a given payload needs the two-pass form",
              name);
  R2S_REQUIRE(given_payload == nullptr || reinterpret_cast<uintptr_t>(given_payload) % 16 == 0,
              "%s: payload not 16-byte aligned", name);
  if (C * N == 0) return R2S_OK;
  if (n_isects == 0) {  // the two-pass form still stores its (zero) outputs
    if (!two_pass || rows_only) return R2S_OK;
    return raster_reduce_impl<T>(nullptr, nullptr, 0, C, N, opac, mus, v_xy_abs, v_xy,
                                 v_conic, v_opac, v_mu, st, zeroed);
  }
  R2S_REQUIRE(tile_offsets && flatten_ids, "%s: null tile lists", name);
  R2S_REQUIRE((given_payload != nullptr || (means2d && conics && opac && mus)) &&
                  (rows_only || (opac && mus)) && v_image,
              "%s: null pointer", name);
  R2S_REQUIRE(rows_only || (v_xy && v_conic && v_opac && v_mu), "%s: null output", name);
  T *rows = nullptr, *payload = nullptr;
  if (two_pass) {
    R2S_REQUIRE(isect_src && (rows_only || emit_ids), "%s: null emit_ids / isect_src", name);
    const int64_t need = given_payload != nullptr ? raster_rows_bytes(n_isects, sizeof(T))
                                                  : raster_bwd_ws_bytes(n_isects, C * N, sizeof(T));
    if (ws == nullptr || static_cast<int64_t>(ws_bytes) < need) {
      set_error("%s: workspace of %zu bytes, %lld required", name, ws_bytes, (long long)need);
      return R2S_EWORKSPACE;
    }
    R2S_REQUIRE(reinterpret_cast<uintptr_t>(ws) % 16 == 0, "%s: workspace not 16-byte aligned",
                name);
    rows = static_cast<T *>(ws);
    payload = rows + n_isects * row_stride<kRasterRowValues>();
  }
  const uint32_t n_keys = static_cast<uint32_t>(C) * tw * th;
  hipStream_t stream = as_stream(st);
  // The full two-pass call zeroes its outputs in the pack launch.
  const bool zero_in_pack = given_payload != nullptr ? zeroed : two_pass && !rows_only;
  if (given_payload != nullptr)
    payload = const_cast<T *>(given_payload);
  else if (two_pass)
    raster_pack_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(C * N, 256))), dim3(256), 0,
                            stream>>>(means2d, conics, opac, mus, C * N, payload,
                                      zero_in_pack ? v_xy : nullptr, v_xy_abs, v_conic, v_opac,
                                      v_mu);
  // 16-byte loads of gradient rows when every row segment starts aligned.
  const bool vec = vec_rows_ok<T>(v_image, W, ts);
#define R2S_RASTER_BWD_R(RR, EXACT)                                                              \
  launch_raster_bwd<T, RR, EXACT>(means2d, conics, opac, mus, tile_offsets, isect_ids,           \
                                  flatten_ids, isect_src, n_isects, n_keys, C * N, v_image, W,   \
                                  H, ts, tw, th, vec, v_xy_abs, v_xy, v_conic, v_opac, v_mu,     \
                                  rows, payload, absgrad, stream)
  const bool with_abs = v_xy_abs != nullptr || (rows != nullptr && absgrad);
  if (ts == 16 && vec && rows != nullptr && with_abs)
    raster_bwd_split_kernel<T>
        <<<dim3(static_cast<uint32_t>(ceil_div(n_isects, kSplitThreads))), dim3(kSplitThreads),
           0, stream>>>(payload, tile_offsets, isect_ids, flatten_ids, isect_src, n_isects,
                        n_keys, C * N, v_image, W, H, tw, th, rows);
  else if (ts == 16)
    R2S_RASTER_BWD_R(16, true);
  else if (ts == 8)
    R2S_RASTER_BWD_R(8, true);
  else if (ts < 8)
    R2S_RASTER_BWD_R(8, false);
  else if (ts < 16)
    R2S_RASTER_BWD_R(16, false);
  else
    R2S_RASTER_BWD_R(32, false);
#undef R2S_RASTER_BWD_R
  R2S_RETURN_IF(check_launch(name));
  if (!two_pass || rows_only) return R2S_OK;
  return raster_reduce_impl<T>(rows, emit_ids, n_isects, C, N, opac, mus, v_xy_abs, v_xy,
                               v_conic, v_opac, v_mu, st, zero_in_pack);
}

// The packed payload of the C N (view, Gaussian) pairs (raster_pack_kernel),
// and with v_xy non-null zeros in the two-pass backward's outputs (v_xy_abs
// may be null).
template <typename T>
int raster_pack_impl(const T *means2d, const T *conics, const T *opac, const T *mus, int64_t C,
                     int64_t N, T *payload, T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac, T *v_mu,
                     r2s_stream_t st) {
  clear_error();
  const char *name = "rasterize_pack";
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size C=%lld N=%lld", name,
              (long long)C, (long long)N);
  if (C * N == 0) return R2S_OK;
  R2S_REQUIRE(means2d && conics && opac && mus && payload, "%s: null pointer", name);
  R2S_REQUIRE(reinterpret_cast<uintptr_t>(payload) % 16 == 0, "%s: payload not 16-byte aligned",
              name);
  R2S_REQUIRE(v_xy == nullptr || (v_conic && v_opac && v_mu),
              "%s: zero targets need v_means2d, v_conics, v_opacities and v_mus", name);
  raster_pack_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(C * N, 256))), dim3(256), 0,
                          as_stream(st)>>>(means2d, conics, opac, mus, C * N, payload, v_xy,
                                           v_xy_abs, v_conic, v_opac, v_mu);
  return check_launch(name);
}

// Device address of `scratch` on the current device, looked up once per
// device and cached (each GPU holds its own copy at its own address).  A
// hipDeviceReset() would leave the cached address stale; the header states
// that the entry point is not to be called on a device after one.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void **out, hipStream_t stream, const char *name) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", name, hipGetErrorString(err));
    return R2S_EHIP;
  }
  R2S_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond %d", name, dev, kMaxDevices);
  if (stream != nullptr) {
    // The kernels run on the stream's device; the address must be that one's.
    hipDevice_t sdev = -1;
    err = hipStreamGetDevice(stream, &sdev);
    if (err != hipSuccess) {
      set_error("%s: hipStreamGetDevice failed: %s", name, hipGetErrorString(err));
      return R2S_EHIP;
    }
    R2S_REQUIRE(sdev == dev, "%s: the stream belongs to device %d, the current device is %d",
                name, static_cast<int>(sdev), dev);
  }
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                hipGetErrorString(err));
      return R2S_EHIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return R2S_OK;
}

// raster_fwd_impl with the split partial tiles in `scratch` instead of a
// caller's workspace.  Every partial tile is written in full before
// fwd_combine_kernel reads it, so nothing needs clearing between calls.
template <typename T>
int raster_fwd_noalloc_impl(const T *means2d, const T *conics, const T *opac, const T *mus,
                            const int32_t *tile_offsets, const int32_t *flatten_ids,
                            int64_t n_isects, int64_t C, int64_t N, uint32_t W, uint32_t H,
                            uint32_t ts, uint32_t tw, uint32_t th, T *image, r2s_stream_t st) {
  clear_error();
  const char *name = "rasterize_to_pixels_fwd_noalloc";
  R2S_RETURN_IF(check_raster_args(n_isects, C, N, W, H, ts, tw, th, name));
  void *ws = nullptr;
  size_t need = 0;
  if (C * static_cast<int64_t>(W) * H > 0 && N > 0 && n_isects > 0 &&
      (ts == 8 || ts == 16 || ts == 32)) {
    const int64_t n_keys = C * static_cast<int64_t>(tw) * th;
    const uint32_t splits = fwd_splits(n_keys, n_isects);
    if (splits > 1) {
      need = static_cast<size_t>(n_keys) * splits * ts * ts * sizeof(T);
      if (need > static_cast<size_t>(R2S_RASTER_SCRATCH_BYTES)) {
        set_error("%s: %lld tiles split %u ways need %zu bytes of partial tiles; the static "
                  "scratch holds %zu (use r2s_rasterize_fwd_* with a workspace)",
                  name, (long long)n_keys, splits, need,
                  static_cast<size_t>(R2S_RASTER_SCRATCH_BYTES));
        return R2S_ERANGE;
      }
      R2S_RETURN_IF(scratch_address(&ws, as_stream(st), name));
    }
  }
  return raster_fwd_impl<T>(means2d, conics, opac, mus, tile_offsets, flatten_ids, n_isects, C,
                            N, W, H, ts, tw, th, image, ws, need, st);
}

}  // namespace
}  // namespace r2s

extern "C" {

#define R2S_RASTER_NOALLOC_API(SUF, T)                                                        \
  int r2s_rasterize_fwd_noalloc_##SUF(const T *means2d, const T *conics, const T *opac,        \
                                      const T *mus, const int32_t *tile_offsets,               \
                                      const int32_t *flatten_ids, int64_t n_isects, int64_t C, \
                                      int64_t N, uint32_t W, uint32_t H, uint32_t ts,          \
                                      uint32_t tw, uint32_t th, T *image, r2s_stream_t st) {   \
    return r2s::raster_fwd_noalloc_impl<T>(means2d, conics, opac, mus, tile_offsets,          \
                                           flatten_ids, n_isects, C, N, W, H, ts, tw, th,     \
                                           image, st);                                        \
  }

R2S_RASTER_NOALLOC_API(f32, float)
R2S_RASTER_NOALLOC_API(f64, double)

#undef R2S_RASTER_NOALLOC_API

int64_t r2s_rasterize_bwd_workspace_bytes(int64_t n_isects, int64_t n_items, int dtype_bytes) {
  if (n_isects <= 0 || n_items < 0 || (dtype_bytes != 4 && dtype_bytes != 8)) return 0;
  return r2s::raster_bwd_ws_bytes(n_isects, n_items, dtype_bytes);
}

int64_t r2s_rasterize_workspace_bytes(int64_t n_keys, int64_t n_isects, uint32_t tile_size,
                                      int dtype_bytes) {
  if (n_keys <= 0 || (tile_size != 8 && tile_size != 16 && tile_size != 32)) return 0;
  const uint32_t splits = r2s::fwd_splits(n_keys, n_isects);
  if (splits <= 1) return 0;
  return n_keys * splits * static_cast<int64_t>(tile_size) * tile_size * dtype_bytes;
}

#define R2S_RASTER_API(SUF, T)                                                                \
  int r2s_rasterize_fwd_##SUF(const T *means2d, const T *conics, const T *opac, const T *mus, \
                              const int32_t *tile_offsets, const int32_t *flatten_ids,        \
                              int64_t n_isects, int64_t C, int64_t N, uint32_t W, uint32_t H, \
                              uint32_t ts, uint32_t tw, uint32_t th, T *image, void *ws,      \
                              size_t ws_bytes, r2s_stream_t st) {                             \
    return r2s::raster_fwd_impl<T>(means2d, conics, opac, mus, tile_offsets, flatten_ids,     \
                                   n_isects, C, N, W, H, ts, tw, th, image, ws, ws_bytes, st);\
  }                                                                                           \
  int r2s_rasterize_bwd_##SUF(const T *means2d, const T *conics, const T *opac, const T *mus, \
                              const int32_t *tile_offsets, const int64_t *isect_ids,          \
                              const int32_t *flatten_ids, int64_t n_isects, const T *v_image, \
                              int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts,      \
                              uint32_t tw, uint32_t th, T *v_xy_abs, T *v_xy, T *v_conic,     \
                              T *v_opac, T *v_mu, r2s_stream_t st) {                          \
    return r2s::raster_bwd_impl<T>(means2d, conics, opac, mus, tile_offsets, isect_ids,       \
                                   flatten_ids, nullptr, nullptr, n_isects, v_image, C, N, W, \
                                   H, ts, tw, th, v_xy_abs, v_xy, v_conic, v_opac, v_mu,      \
                                   nullptr, 0, false, st);                                    \
  }                                                                                           \
  int r2s_rasterize_bwd_emit_##SUF(                                                           \
      const T *means2d, const T *conics, const T *opac, const T *mus,                         \
      const int32_t *tile_offsets, const int64_t *isect_ids, const int32_t *flatten_ids,      \
      const int32_t *emit_ids, const int32_t *isect_src, int64_t n_isects, const T *v_image,  \
      int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th,    \
      T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac, T *v_mu, void *ws, size_t ws_bytes,        \
      r2s_stream_t st) {                                                                      \
    return r2s::raster_bwd_impl<T>(means2d, conics, opac, mus, tile_offsets, isect_ids,       \
                                   flatten_ids, emit_ids, isect_src, n_isects, v_image, C, N, \
                                   W, H, ts, tw, th, v_xy_abs, v_xy, v_conic, v_opac, v_mu,   \
                                   ws, ws_bytes, true, st, false, v_xy_abs != nullptr);       \
  }

#define R2S_RASTER_STAGE_API(SUF, T)                                                          \
  int r2s_rasterize_bwd_rows_##SUF(                                                           \
      const T *means2d, const T *conics, const T *opac, const T *mus,                         \
      const int32_t *tile_offsets, const int64_t *isect_ids, const int32_t *flatten_ids,      \
      const int32_t *isect_src, int64_t n_isects, const T *v_image, int64_t C, int64_t N,     \
      uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th, int absgrad, void *rows, \
      size_t rows_bytes, r2s_stream_t st) {                                                   \
    return r2s::raster_bwd_impl<T>(means2d, conics, opac, mus, tile_offsets, isect_ids,       \
                                   flatten_ids, nullptr, isect_src, n_isects, v_image, C, N,  \
                                   W, H, ts, tw, th, nullptr, nullptr, nullptr, nullptr,      \
                                   nullptr, rows, rows_bytes, true, st, true, absgrad != 0);  \
  }                                                                                           \
  int r2s_rasterize_bwd_reduce_##SUF(const T *rows, const int32_t *emit_ids, int64_t n_isects, \
                                     int64_t C, int64_t N, const T *opac, const T *mus,       \
                                     T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac, T *v_mu,    \
                                     r2s_stream_t st) {                                       \
    r2s::clear_error();                                                                       \
    return r2s::raster_reduce_impl<T>(rows, emit_ids, n_isects, C, N, opac, mus, v_xy_abs,    \
                                      v_xy, v_conic, v_opac, v_mu, st);                       \
  }

R2S_RASTER_STAGE_API(f32, float)
R2S_RASTER_STAGE_API(f64, double)

#undef R2S_RASTER_STAGE_API

int64_t r2s_rasterize_payload_bytes(int64_t n_items, int dtype_bytes) {
  if (n_items <= 0 || (dtype_bytes != 4 && dtype_bytes != 8)) return 0;
  return n_items * r2s::kPayloadValues * static_cast<int64_t>(dtype_bytes);
}

#define R2S_RASTER_PACKED_API(SUF, T)                                                         \
  int r2s_rasterize_pack_##SUF(const T *means2d, const T *conics, const T *opac,              \
                               const T *mus, int64_t C, int64_t N, T *payload, T *v_xy_abs,   \
                               T *v_xy, T *v_conic, T *v_opac, T *v_mu, r2s_stream_t st) {    \
    return r2s::raster_pack_impl<T>(means2d, conics, opac, mus, C, N, payload, v_xy_abs,      \
                                    v_xy, v_conic, v_opac, v_mu, st);                         \
  }                                                                                           \
  int r2s_rasterize_fwd_packed_##SUF(const T *payload, const int32_t *tile_offsets,           \
                                     const int32_t *flatten_ids, int64_t n_isects, int64_t C, \
                                     int64_t N, uint32_t W, uint32_t H, uint32_t ts,          \
                                     uint32_t tw, uint32_t th, T *image, void *ws,            \
                                     size_t ws_bytes, r2s_stream_t st) {                      \
    return r2s::raster_fwd_impl<T>(nullptr, nullptr, nullptr, nullptr, tile_offsets,         \
                                   flatten_ids, n_isects, C, N, W, H, ts, tw, th, image, ws,  \
                                   ws_bytes, st, payload);                                    \
  }                                                                                           \
  int r2s_rasterize_bwd_packed_##SUF(                                                         \
      const T *payload, const T *opac, const T *mus, const int32_t *tile_offsets,             \
      const int64_t *isect_ids, const int32_t *flatten_ids, const int32_t *emit_ids,          \
      const int32_t *isect_src, int64_t n_isects, const T *v_image, int64_t C, int64_t N,     \
      uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th, T *v_xy_abs, T *v_xy,    \
      T *v_conic, T *v_opac, T *v_mu, int zeroed, void *ws, size_t ws_bytes,                  \
      r2s_stream_t st) {                                                                      \
    return r2s::raster_bwd_impl<T>(nullptr, nullptr, opac, mus, tile_offsets, isect_ids,      \
                                   flatten_ids, emit_ids, isect_src, n_isects, v_image, C, N, \
                                   W, H, ts, tw, th, v_xy_abs, v_xy, v_conic, v_opac, v_mu,   \
                                   ws, ws_bytes, true, st, false, v_xy_abs != nullptr,        \
                                   payload, zeroed != 0);                                     \
  }                                                                                           \
  int r2s_rasterize_bwd_rows_packed_##SUF(                                                    \
      const T *payload, const int32_t *tile_offsets, const int64_t *isect_ids,                \
      const int32_t *flatten_ids, const int32_t *isect_src, int64_t n_isects,                 \
      const T *v_image, int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts,            \
      uint32_t tw, uint32_t th, int absgrad, void *rows, size_t rows_bytes,                   \
      r2s_stream_t st) {                                                                      \
    return r2s::raster_bwd_impl<T>(nullptr, nullptr, nullptr, nullptr, tile_offsets,         \
                                   isect_ids, flatten_ids, nullptr, isect_src, n_isects,      \
                                   v_image, C, N, W, H, ts, tw, th, nullptr, nullptr,         \
                                   nullptr, nullptr, nullptr, rows, rows_bytes, true, st,     \
                                   true, absgrad != 0, payload);                              \
  }

R2S_RASTER_PACKED_API(f32, float)
R2S_RASTER_PACKED_API(f64, double)

#undef R2S_RASTER_PACKED_API

R2S_RASTER_API(f32, float)
R2S_RASTER_API(f64, double)

#undef R2S_RASTER_API

}  // extern "C"
