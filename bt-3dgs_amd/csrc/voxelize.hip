// Brick-tiled voxelizer: volume = per voxel sum over its brick's Gaussian
// list of opacity * exp(-sigma), sigma = 1/2 d^T conic d, skipping sigma < 0
// and |alpha| < 1e-6 (r2splat/cuda/csrc/VoxelizeToVoxelsFwd.cu:69-221), and
// its VJP (VoxelizeToVoxelsBwd.cu:71-441).
//
// Forward: one workgroup per brick, one voxel per thread with the lane index
// running along dim2 (the contiguous axis) so stores are coalesced -- the
// reference maps threadIdx.x to dim0.  Gaussians are staged in LDS in
// batches ({mean, opacity}, {c00..c11}, {c12, c22}), read as broadcasts;
// each voxel sums in list order.
//
// Backward: one lane per intersection record walking the ts^3 voxels of its
// brick with the ten partials in registers, then ten hardware float atomics.
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
__global__ __launch_bounds__(1024) void voxel_fwd_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int32_t *__restrict__ flatten_ids,
    int64_t n_isects, uint32_t n_keys, uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts,
    uint32_t n2, uint32_t n1, T *__restrict__ volume) {
  using V2 = typename Vec<T>::v2;
  using V4 = typename Vec<T>::v4;
  extern __shared__ double smem_raw[];
  const uint32_t bs = ts * ts * ts;
  V4 *s_mo = reinterpret_cast<V4 *>(smem_raw);
  V4 *s_c0 = s_mo + bs;
  V2 *s_c1 = reinterpret_cast<V2 *>(s_c0 + bs);

  const uint32_t key = xcd_swizzle(blockIdx.x, n_keys);
  const uint32_t b0 = key / (n1 * n2), rem = key - b0 * (n1 * n2);
  const uint32_t b1 = rem / n2, b2 = rem - b1 * n2;
  const uint32_t tr = threadIdx.x;
  const uint32_t lk = tr % ts, lj = (tr / ts) % ts, li = tr / (ts * ts);
  const uint32_t i = b0 * ts + li, j = b1 * ts + lj, k = b2 * ts + lk;
  const bool inside = (i < D0) && (j < D1) && (k < D2);
  const T px = static_cast<T>(k) + static_cast<T>(0.5);
  const T py = static_cast<T>(j) + static_cast<T>(0.5);
  const T pz = static_cast<T>(i) + static_cast<T>(0.5);

  const int64_t start = tile_offsets[key];
  const int64_t end = (key == n_keys - 1) ? n_isects : static_cast<int64_t>(tile_offsets[key + 1]);
  const T thr = static_cast<T>(1e-6), half = static_cast<T>(0.5);
  T acc = 0;
  for (int64_t b = start; b < end; b += bs) {
    __syncthreads();
    const int64_t idx = b + tr;
    if (idx < end) {
      const int64_t g = flatten_ids[idx];
      V4 mo;
      mo.x = means3d[3 * g];
      mo.y = means3d[3 * g + 1];
      mo.z = means3d[3 * g + 2];
      mo.w = opac[g];
      s_mo[tr] = mo;
      const T *q = conics + 6 * g;
      V4 c0;
      c0.x = q[0];
      c0.y = q[1];
      c0.z = q[2];
      c0.w = q[3];
      s_c0[tr] = c0;
      V2 c1;
      c1.x = q[4];
      c1.y = q[5];
      s_c1[tr] = c1;
    }
    __syncthreads();
    const int cnt = static_cast<int>(min(static_cast<int64_t>(bs), end - b));
    if (inside) {
#pragma unroll 2
      for (int t = 0; t < cnt; ++t) {
        const V4 mo = s_mo[t];
        const V4 c0 = s_c0[t];
        const V2 c1 = s_c1[t];
        const T dx = px - mo.x, dy = py - mo.y, dz = pz - mo.z;
        const T sigma = half * (c0.x * dx * dx + c0.w * dy * dy + c1.y * dz * dz) +
                        c0.y * dx * dy + c0.z * dx * dz + c1.x * dy * dz;
        const T alpha = mo.w * fast_exp(-sigma);
        const bool skip = (sigma < static_cast<T>(0)) || (fabs(alpha) < thr);
        acc += skip ? static_cast<T>(0) : alpha;
      }
    }
  }
  if (inside)
    volume[static_cast<int64_t>(i) * D1 * D2 + static_cast<int64_t>(j) * D2 + k] = acc;
}

__device__ __forceinline__ uint32_t key_of_record(const int32_t *__restrict__ offsets,
                                                  uint32_t n_keys, int64_t r) {
  uint32_t lo = 0, hi = n_keys;
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
__global__ __launch_bounds__(256) void voxel_bwd_kernel(
    const T *__restrict__ means3d, const T *__restrict__ conics, const T *__restrict__ opac,
    const int32_t *__restrict__ tile_offsets, const int64_t *__restrict__ isect_ids,
    const int32_t *__restrict__ flatten_ids, int64_t n_isects, uint32_t n_keys, int64_t N,
    const T *__restrict__ v_vol, uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts,
    uint32_t n2, uint32_t n1, T *__restrict__ v_means, T *__restrict__ v_conics,
    T *__restrict__ v_opac) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= n_isects) return;
  uint32_t key;
  if (isect_ids != nullptr) {
    const int64_t kk = isect_ids[r];
    if (kk < 0 || kk >= static_cast<int64_t>(n_keys)) return;
    key = static_cast<uint32_t>(kk);
  } else {
    key = key_of_record(tile_offsets, n_keys, r);
  }
  const int64_t g = flatten_ids[r];
  if (g < 0 || g >= N) return;
  const uint32_t b0 = key / (n1 * n2), rem = key - b0 * (n1 * n2);
  const uint32_t b1 = rem / n2, b2 = rem - b1 * n2;
  const uint32_t oi = b0 * ts, oj = b1 * ts, ok = b2 * ts;
  const T mx = means3d[3 * g], my = means3d[3 * g + 1], mz = means3d[3 * g + 2];
  const T *q = conics + 6 * g;
  const T a = q[0], p = q[1], qq = q[2], bb = q[3], rr = q[4], cz = q[5];
  const T o = opac[g];
  const T half = static_cast<T>(0.5), thr = static_cast<T>(1e-6);
  const T fx0 = static_cast<T>(ok) + half, fy0 = static_cast<T>(oj) + half,
          fz0 = static_cast<T>(oi) + half;
  T gx = 0, gy = 0, gz = 0, g0 = 0, g1 = 0, g2 = 0, g3 = 0, g4 = 0, g5 = 0, go = 0;
  for (uint32_t li = 0; li < ts; ++li) {
    const uint32_t i = oi + li;
    if (i >= D0) break;
    const T d3 = (fz0 + static_cast<T>(li)) - mz;
    for (uint32_t lj = 0; lj < ts; ++lj) {
      const uint32_t j = oj + lj;
      if (j >= D1) break;
      const T d2 = (fy0 + static_cast<T>(lj)) - my;
      const T *__restrict__ vrow =
          v_vol + static_cast<int64_t>(i) * D1 * D2 + static_cast<int64_t>(j) * D2;
#pragma unroll 4
      for (uint32_t lk = 0; lk < ts; ++lk) {
        const uint32_t kx = ok + lk;
        if (kx >= D2) break;
        const T d1 = (fx0 + static_cast<T>(lk)) - mx;
        const T sigma = half * (a * d1 * d1 + bb * d2 * d2 + cz * d3 * d3) + p * d1 * d2 +
                        qq * d1 * d3 + rr * d2 * d3;
        const T vis_raw = fast_exp(-sigma);
        const bool valid = !((sigma < static_cast<T>(0)) || (fabs(o * vis_raw) < thr));
        const T vis = valid ? vis_raw : static_cast<T>(0);
        const T v = vrow[kx];
        const T v_sigma = -v * o * vis;
        const T oI = o * vis;
        go += v * vis;
        g0 += v_sigma * half * d1 * d1;
        g1 += v_sigma * d1 * d2;
        g2 += v_sigma * d1 * d3;
        g3 += v_sigma * half * d2 * d2;
        g4 += v_sigma * d2 * d3;
        g5 += v_sigma * half * d3 * d3;
        gx += v * oI * (a * d1 + p * d2 + qq * d3);
        gy += v * oI * (bb * d2 + p * d1 + rr * d3);
        gz += v * oI * (cz * d3 + qq * d1 + rr * d2);
      }
    }
  }
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

int check_voxel_args(int64_t n_isects, int64_t N, uint32_t D2, uint32_t D1, uint32_t D0,
                     uint32_t ts, uint32_t n2, uint32_t n1, uint32_t n0, const char *name) {
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size N=%lld", name, (long long)N);
  R2S_REQUIRE(ts > 0 && ts * ts * ts <= 1024,
              "%s: tile_size must be positive with tile_size**3 <= 1024", name);
  R2S_REQUIRE(n_isects >= 0 && n_isects <= kInt32Max, "%s: bad n_isects", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * ts >= D2 && static_cast<uint64_t>(n1) * ts >= D1 &&
                  static_cast<uint64_t>(n0) * ts >= D0,
              "%s: brick grid does not cover the volume", name);
  R2S_REQUIRE(static_cast<uint64_t>(n2) * n1 * n0 <= 0xffffffffull, "%s: too many bricks", name);
  return R2S_OK;
}

template <typename T>
int voxel_fwd_impl(const T *means3d, const T *conics, const T *opac,
                   const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,
                   int64_t N, uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2,
                   uint32_t n1, uint32_t n0, T *volume, r2s_stream_t st) {
  clear_error();
  const char *name = "voxelize_to_voxels_fwd";
  R2S_RETURN_IF(check_voxel_args(n_isects, N, D2, D1, D0, ts, n2, n1, n0, name));
  const int64_t n_vox = static_cast<int64_t>(D2) * D1 * D0;
  if (n_vox == 0) return R2S_OK;
  R2S_REQUIRE(volume != nullptr, "%s: null volume", name);
  hipStream_t stream = as_stream(st);
  if (N == 0 || n_isects == 0) return device_fill<T>(volume, n_vox, static_cast<T>(0), stream, name);
  R2S_REQUIRE(means3d && conics && opac && tile_offsets && flatten_ids, "%s: null pointer", name);
  const uint32_t n_keys = n2 * n1 * n0;
  const uint32_t bs = ts * ts * ts;
  const size_t smem = 2 * bs * sizeof(typename Vec<T>::v4) + bs * sizeof(typename Vec<T>::v2);
  voxel_fwd_kernel<T><<<dim3(n_keys), dim3(bs), smem, stream>>>(
      means3d, conics, opac, tile_offsets, flatten_ids, n_isects, n_keys, D2, D1, D0, ts, n2, n1,
      volume);
  return check_launch(name);
}

template <typename T>
int voxel_bwd_impl(const T *means3d, const T *conics, const T *opac,
                   const int32_t *tile_offsets, const int64_t *isect_ids,
                   const int32_t *flatten_ids, int64_t n_isects, const T *v_vol, int64_t N,
                   uint32_t D2, uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,
                   uint32_t n0, T *v_means, T *v_conics, T *v_opac, r2s_stream_t st) {
  clear_error();
  const char *name = isect_ids ? "voxelize_to_voxels_bwd_per_gaussian" : "voxelize_to_voxels_bwd";
  R2S_RETURN_IF(check_voxel_args(n_isects, N, D2, D1, D0, ts, n2, n1, n0, name));
  if (N == 0 || n_isects == 0) return R2S_OK;
  R2S_REQUIRE(means3d && conics && opac && tile_offsets && flatten_ids && v_vol && v_means &&
                  v_conics && v_opac,
              "%s: null pointer", name);
  const uint32_t n_keys = n2 * n1 * n0;
  voxel_bwd_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(n_isects, 256))), dim3(256), 0,
                        as_stream(st)>>>(means3d, conics, opac, tile_offsets, isect_ids,
                                         flatten_ids, n_isects, n_keys, N, v_vol, D2, D1, D0, ts,
                                         n2, n1, v_means, v_conics, v_opac);
  return check_launch(name);
}

}  // namespace
}  // namespace r2s

extern "C" {

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
                                  n_isects, v_vol, N, D2, D1, D0, ts, n2, n1, n0, v_means,     \
                                  v_conics, v_opac, st);                                       \
  }

R2S_VOXEL_API(f32, float)
R2S_VOXEL_API(f64, double)

#undef R2S_VOXEL_API

}  // extern "C"
