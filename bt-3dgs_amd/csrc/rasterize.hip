// X-ray line-integral rasterizer: image = sum over each tile's Gaussian list
// of opacity * mu * exp(-sigma), sigma = 1/2 d^T conic d, skipping sigma < 0
// and |alpha| < 1e-5 (r2splat/cuda/csrc/RasterizeToPixelsFwd.cu:57-186), and
// its VJP (RasterizeToPixelsBwd.cu:77-480).
//
// Forward: one workgroup per (camera, tile), one pixel per thread; the
// tile's list is staged through LDS in batches of ts^2 Gaussians
// ({mean} and {conic, opacity*mu} as 8- and 16-byte vectors, read by every
// lane as an LDS broadcast).  Each pixel sums in list order, as the
// reference does.  Workgroups are XCD-swizzled so neighbouring tiles, which
// share most of their Gaussians, run on the same L2.
//
// Backward: one lane per intersection record.  The lane walks the ts^2
// pixels of its record's tile and accumulates the nine partials of that
// Gaussian in registers -- no cross-lane reduction -- then issues one
// hardware float atomic per partial.  Records of one tile are adjacent, so
// the upstream-gradient loads of a wave hit the same cache lines.  The tile
// of a record comes from isect_ids (per-Gaussian mode) or from a binary
// search of tile_offsets (pixel mode); both modes compute the same sums.
#include "r2s_common.h"
#include "r2s_scan.h"

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
  const T thr = static_cast<T>(1e-5);
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

// Key of record r from the offsets: the last k with tile_offsets[k] <= r.
__device__ __forceinline__ uint32_t key_of_record(const int32_t *__restrict__ offsets,
                                                  uint32_t n_keys, int64_t r) {
  uint32_t lo = 0, hi = n_keys;  // invariant: offsets[lo] <= r < offsets[hi] (hi virtual)
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(offsets[mid]) <= r)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

template <typename T>
__global__ __launch_bounds__(256) void raster_bwd_kernel(
    const T *__restrict__ means2d, const T *__restrict__ conics, const T *__restrict__ opac,
    const T *__restrict__ mus, const int32_t *__restrict__ tile_offsets,
    const int64_t *__restrict__ isect_ids, const int32_t *__restrict__ flatten_ids,
    int64_t n_isects, uint32_t n_keys, int64_t n_items, const T *__restrict__ v_image,
    uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th, T *__restrict__ v_xy_abs,
    T *__restrict__ v_xy, T *__restrict__ v_conic, T *__restrict__ v_opac,
    T *__restrict__ v_mu) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= n_isects) return;
  uint32_t key;
  if (isect_ids != nullptr) {
    const int64_t k = isect_ids[r];
    if (k < 0 || k >= static_cast<int64_t>(n_keys)) return;
    key = static_cast<uint32_t>(k);
  } else {
    key = key_of_record(tile_offsets, n_keys, r);
  }
  const int64_t g = flatten_ids[r];
  if (g < 0 || g >= n_items) return;
  const uint32_t n_tiles = tw * th;
  const uint32_t cam = key / n_tiles, t = key - cam * n_tiles;
  const uint32_t ty = t / tw, tx = t - ty * tw;
  const uint32_t ox = tx * ts, oy = ty * ts;
  const T *__restrict__ vimg = v_image + static_cast<int64_t>(cam) * H * W;

  const T mx = means2d[2 * g], my = means2d[2 * g + 1];
  const T a = conics[3 * g], b = conics[3 * g + 1], c = conics[3 * g + 2];
  const T o = opac[g], mu = mus[g];
  const T om = o * mu;
  const T thr = static_cast<T>(1e-5), half = static_cast<T>(0.5);
  // Pixel centres are exact in T: (ox + lx) + 0.5 == (ox + 0.5) + lx.
  const T fx0 = static_cast<T>(ox) + half, fy0 = static_cast<T>(oy) + half;

  T ax = 0, ay = 0, aax = 0, aay = 0, ca = 0, cb = 0, cc = 0, ao = 0, am = 0;
  for (uint32_t ly = 0; ly < ts; ++ly) {
    const uint32_t i = oy + ly;
    if (i >= H) break;
    const T dy = (fy0 + static_cast<T>(ly)) - my;
    const T *__restrict__ vrow = vimg + static_cast<int64_t>(i) * W;
#pragma unroll 4
    for (uint32_t lx = 0; lx < ts; ++lx) {
      const uint32_t jx = ox + lx;
      if (jx >= W) break;
      const T dx = (fx0 + static_cast<T>(lx)) - mx;
      const T sigma = half * (a * dx * dx + c * dy * dy) + b * dx * dy;
      const T vis_raw = fast_exp(-sigma);
      const T alpha_raw = om * vis_raw;
      const bool valid = !((sigma < static_cast<T>(0)) || (fabs(alpha_raw) < thr));
      const T vis = valid ? vis_raw : static_cast<T>(0);
      const T alpha = valid ? alpha_raw : static_cast<T>(0);
      const T v = vrow[jx];
      const T v_sigma = -v * alpha;
      const T gx = -v_sigma * (a * dx + b * dy);
      const T gy = -v_sigma * (c * dy + b * dx);
      ax += gx;
      ay += gy;
      aax += fabs(gx);
      aay += fabs(gy);
      ca += v_sigma * half * dx * dx;
      cb += v_sigma * dx * dy;
      cc += v_sigma * half * dy * dy;
      ao += v * mu * vis;
      am += v * o * vis;
    }
  }
  if (ax == 0 && ay == 0 && aax == 0 && aay == 0 && ca == 0 && cb == 0 && cc == 0 && ao == 0 &&
      am == 0)
    return;  // nothing to add
  atomic_add(v_xy + 2 * g, ax);
  atomic_add(v_xy + 2 * g + 1, ay);
  if (v_xy_abs != nullptr) {
    atomic_add(v_xy_abs + 2 * g, aax);
    atomic_add(v_xy_abs + 2 * g + 1, aay);
  }
  atomic_add(v_conic + 3 * g, ca);
  atomic_add(v_conic + 3 * g + 1, cb);
  atomic_add(v_conic + 3 * g + 2, cc);
  atomic_add(v_opac + g, ao);
  atomic_add(v_mu + g, am);
}

int check_raster_args(int64_t n_isects, int64_t C, int64_t N, uint32_t W, uint32_t H,
                      uint32_t ts, uint32_t tw, uint32_t th, const char *name) {
  R2S_REQUIRE(C >= 0 && N >= 0 && C * N <= kInt32Max, "%s: bad size C=%lld N=%lld", name,
              (long long)C, (long long)N);
  R2S_REQUIRE(ts > 0 && ts * ts <= 1024, "%s: tile_size must be positive with tile_size**2 <= 1024",
              name);
  R2S_REQUIRE(n_isects >= 0 && n_isects <= kInt32Max, "%s: bad n_isects %lld", name,
              (long long)n_isects);
  R2S_REQUIRE(static_cast<uint64_t>(tw) * ts >= W && static_cast<uint64_t>(th) * ts >= H,
              "%s: tile grid %ux%u of size %u does not cover %ux%u", name, tw, th, ts, W, H);
  R2S_REQUIRE(static_cast<uint64_t>(C) * tw * th <= 0xffffffffull, "%s: too many tiles", name);
  return R2S_OK;
}

template <typename T>
int raster_fwd_impl(const T *means2d, const T *conics, const T *opac, const T *mus,
                    const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,
                    int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw,
                    uint32_t th, T *image, r2s_stream_t st) {
  clear_error();
  const char *name = "rasterize_to_pixels_fwd";
  R2S_RETURN_IF(check_raster_args(n_isects, C, N, W, H, ts, tw, th, name));
  hipStream_t stream = as_stream(st);
  const int64_t n_pix = C * static_cast<int64_t>(W) * H;
  if (n_pix == 0) return R2S_OK;
  R2S_REQUIRE(image != nullptr, "%s: null image", name);
  if (N == 0 || n_isects == 0) return device_fill<T>(image, n_pix, static_cast<T>(0), stream, name);
  R2S_REQUIRE(means2d && conics && opac && mus && tile_offsets && flatten_ids,
              "%s: null pointer", name);
  const uint32_t n_keys = static_cast<uint32_t>(C) * tw * th;
  const uint32_t bs = ts * ts;
  const size_t smem = (bs + (bs & 1u)) * sizeof(typename Vec<T>::v2) + bs * sizeof(typename Vec<T>::v4);
  raster_fwd_kernel<T><<<dim3(n_keys), dim3(bs), smem, stream>>>(
      means2d, conics, opac, mus, tile_offsets, flatten_ids, n_isects, n_keys, W, H, ts, tw, th,
      image);
  return check_launch(name);
}

template <typename T>
int raster_bwd_impl(const T *means2d, const T *conics, const T *opac, const T *mus,
                    const int32_t *tile_offsets, const int64_t *isect_ids,
                    const int32_t *flatten_ids, int64_t n_isects, const T *v_image, int64_t C,
                    int64_t N, uint32_t W, uint32_t H, uint32_t ts, uint32_t tw, uint32_t th,
                    T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac, T *v_mu, r2s_stream_t st) {
  clear_error();
  const char *name = isect_ids ? "rasterize_to_pixels_bwd_per_gaussian" : "rasterize_to_pixels_bwd";
  R2S_RETURN_IF(check_raster_args(n_isects, C, N, W, H, ts, tw, th, name));
  if (C * N == 0 || n_isects == 0) return R2S_OK;
  R2S_REQUIRE(means2d && conics && opac && mus && tile_offsets && flatten_ids && v_image &&
                  v_xy && v_conic && v_opac && v_mu,
              "%s: null pointer", name);
  const uint32_t n_keys = static_cast<uint32_t>(C) * tw * th;
  raster_bwd_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(n_isects, 256))), dim3(256), 0,
                         as_stream(st)>>>(means2d, conics, opac, mus, tile_offsets, isect_ids,
                                          flatten_ids, n_isects, n_keys, C * N, v_image, W, H,
                                          ts, tw, th, v_xy_abs, v_xy, v_conic, v_opac, v_mu);
  return check_launch(name);
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_rasterize_workspace_bytes(int64_t n_keys, int64_t n_isects, uint32_t tile_size,
                                      int dtype_bytes) {
  (void)n_keys;
  (void)n_isects;
  (void)tile_size;
  (void)dtype_bytes;
  return 0;
}

#define R2S_RASTER_API(SUF, T)                                                                \
  int r2s_rasterize_fwd_##SUF(const T *means2d, const T *conics, const T *opac, const T *mus, \
                              const int32_t *tile_offsets, const int32_t *flatten_ids,        \
                              int64_t n_isects, int64_t C, int64_t N, uint32_t W, uint32_t H, \
                              uint32_t ts, uint32_t tw, uint32_t th, T *image, void *ws,      \
                              size_t ws_bytes, r2s_stream_t st) {                             \
    (void)ws;                                                                                 \
    (void)ws_bytes;                                                                           \
    return r2s::raster_fwd_impl<T>(means2d, conics, opac, mus, tile_offsets, flatten_ids,     \
                                   n_isects, C, N, W, H, ts, tw, th, image, st);              \
  }                                                                                           \
  int r2s_rasterize_bwd_##SUF(const T *means2d, const T *conics, const T *opac, const T *mus, \
                              const int32_t *tile_offsets, const int64_t *isect_ids,          \
                              const int32_t *flatten_ids, int64_t n_isects, const T *v_image, \
                              int64_t C, int64_t N, uint32_t W, uint32_t H, uint32_t ts,      \
                              uint32_t tw, uint32_t th, T *v_xy_abs, T *v_xy, T *v_conic,     \
                              T *v_opac, T *v_mu, r2s_stream_t st) {                          \
    return r2s::raster_bwd_impl<T>(means2d, conics, opac, mus, tile_offsets, isect_ids,       \
                                   flatten_ids, n_isects, v_image, C, N, W, H, ts, tw, th,    \
                                   v_xy_abs, v_xy, v_conic, v_opac, v_mu, st);                \
  }

R2S_RASTER_API(f32, float)
R2S_RASTER_API(f64, double)

#undef R2S_RASTER_API

}  // extern "C"
