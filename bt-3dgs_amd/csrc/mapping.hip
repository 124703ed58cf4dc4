// World -> voxel mapping of Gaussians and its VJP.
//
// Forward: r = (dim2/range_x, dim1/range_y, dim0/range_z);
// means3d = (p - center) r + dim/2; Sigma_v = diag(r) Sigma diag(r) + eps I;
// conic = Sigma_v^-1 by cofactors (|det| < 1e-12 -> zeros, radii 0);
// radii = ceil(clip sqrt(Sigma_v_kk)).  Backward: v_means = v_means3d r,
// v_Sigma_v = -P V_upper P gathered onto the six packed entries.
//
// Expression order follows r2splat/cuda/csrc/WorldToVolumeMappingFwd.cu:55-189
// and WorldToVolumeMappingBwd.cu:83-198 with contraction off (bit-
// reproducible against an IEEE restatement).  One thread per Gaussian.
#pragma clang fp contract(off)

#include "r2s_common.h"

namespace r2s {
namespace {

template <typename T>
__device__ __forceinline__ bool invert_sym3x3(T a00, T a01, T a02, T a11, T a12, T a22, T o[6]) {
  const T c00 = a11 * a22 - a12 * a12;
  const T c01 = a02 * a12 - a01 * a22;
  const T c02 = a01 * a12 - a02 * a11;
  const T c11 = a00 * a22 - a02 * a02;
  const T c12 = a01 * a02 - a00 * a12;
  const T c22 = a00 * a11 - a01 * a01;
  const T det = a00 * c00 + a01 * c01 + a02 * c02;
  if (fabs(det) < static_cast<T>(1e-12)) {
#pragma unroll
    for (int k = 0; k < 6; ++k) o[k] = 0;
    return false;
  }
  const T inv = static_cast<T>(1) / det;
  o[0] = c00 * inv;
  o[1] = c01 * inv;
  o[2] = c02 * inv;
  o[3] = c11 * inv;
  o[4] = c12 * inv;
  o[5] = c22 * inv;
  return true;
}

template <typename T>
struct VolumeFrame {
  T r0, r1, r2;  // voxels per world unit along x (dim2), y (dim1), z (dim0)
};

template <typename T>
__device__ __forceinline__ VolumeFrame<T> volume_frame(const T *__restrict__ ranges, uint32_t d2,
                                                       uint32_t d1, uint32_t d0) {
  VolumeFrame<T> f;
  f.r0 = static_cast<T>(d2) / ranges[0];
  f.r1 = static_cast<T>(d1) / ranges[1];
  f.r2 = static_cast<T>(d0) / ranges[2];
  return f;
}

template <typename T>
__global__ __launch_bounds__(256) void mapping_fwd_kernel(
    const T *__restrict__ means, const T *__restrict__ covars, const T *__restrict__ ranges,
    const T *__restrict__ centers, uint32_t d2, uint32_t d1, uint32_t d0, T eps, T clip,
    T *__restrict__ means3d, T *__restrict__ conics, int32_t *__restrict__ radii, int64_t N) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const VolumeFrame<T> f = volume_frame(ranges, d2, d1, d0);
  const T half = static_cast<T>(0.5);
  means3d[3 * i] = (means[3 * i] - centers[0]) * f.r0 + static_cast<T>(d2) * half;
  means3d[3 * i + 1] = (means[3 * i + 1] - centers[1]) * f.r1 + static_cast<T>(d1) * half;
  means3d[3 * i + 2] = (means[3 * i + 2] - centers[2]) * f.r2 + static_cast<T>(d0) * half;
  const T *s = covars + 6 * i;
  T Sv00 = f.r0 * f.r0 * s[0];
  const T Sv01 = f.r0 * f.r1 * s[1];
  const T Sv02 = f.r0 * f.r2 * s[2];
  T Sv11 = f.r1 * f.r1 * s[3];
  const T Sv12 = f.r1 * f.r2 * s[4];
  T Sv22 = f.r2 * f.r2 * s[5];
  Sv00 += eps;
  Sv11 += eps;
  Sv22 += eps;
  T P[6];
  const bool ok = invert_sym3x3(Sv00, Sv01, Sv02, Sv11, Sv12, Sv22, P);
#pragma unroll
  for (int k = 0; k < 6; ++k) conics[6 * i + k] = P[k];
  int32_t rad[3] = {0, 0, 0};
  if (ok) {
    const T rx = ceil(clip * sqrt(fmax(static_cast<T>(0), Sv00)));
    const T ry = ceil(clip * sqrt(fmax(static_cast<T>(0), Sv11)));
    const T rz = ceil(clip * sqrt(fmax(static_cast<T>(0), Sv22)));
    if (isfinite(rx) && isfinite(ry) && isfinite(rz) && rx > static_cast<T>(0) &&
        ry > static_cast<T>(0) && rz > static_cast<T>(0)) {
      rad[0] = static_cast<int32_t>(rx);
      rad[1] = static_cast<int32_t>(ry);
      rad[2] = static_cast<int32_t>(rz);
    }
  }
  radii[3 * i] = rad[0];
  radii[3 * i + 1] = rad[1];
  radii[3 * i + 2] = rad[2];
}

template <typename T>
__global__ __launch_bounds__(256) void mapping_bwd_kernel(
    const T *__restrict__ covars, const T *__restrict__ ranges, uint32_t d2, uint32_t d1,
    uint32_t d0, T eps, const T *__restrict__ v_means3d, const T *__restrict__ v_conics,
    T *__restrict__ v_means, T *__restrict__ v_covars, int64_t N) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const VolumeFrame<T> f = volume_frame(ranges, d2, d1, d0);
  const T r0 = f.r0, r1 = f.r1, r2 = f.r2;
  v_means[3 * i] = v_means3d[3 * i] * r0;
  v_means[3 * i + 1] = v_means3d[3 * i + 1] * r1;
  v_means[3 * i + 2] = v_means3d[3 * i + 2] * r2;
  const T *s = covars + 6 * i;
  const T Sv00 = r0 * r0 * s[0] + eps;
  const T Sv01 = r0 * r1 * s[1];
  const T Sv02 = r0 * r2 * s[2];
  const T Sv11 = r1 * r1 * s[3] + eps;
  const T Sv12 = r1 * r2 * s[4];
  const T Sv22 = r2 * r2 * s[5] + eps;
  T P[6];
  T *vc_out = v_covars + 6 * i;
  if (!invert_sym3x3(Sv00, Sv01, Sv02, Sv11, Sv12, Sv22, P)) {
#pragma unroll
    for (int k = 0; k < 6; ++k) vc_out[k] = 0;
    return;
  }
  const T P00 = P[0], P01 = P[1], P02 = P[2], P11 = P[3], P12 = P[4], P22 = P[5];
  const T *vc = v_conics + 6 * i;
  const T vc00 = vc[0], vc01 = vc[1], vc02 = vc[2], vc11 = vc[3], vc12 = vc[4], vc22 = vc[5];
  // T = V_upper P
  const T T00 = vc00 * P00 + vc01 * P01 + vc02 * P02;
  const T T01 = vc00 * P01 + vc01 * P11 + vc02 * P12;
  const T T02 = vc00 * P02 + vc01 * P12 + vc02 * P22;
  const T T10 = vc11 * P01 + vc12 * P02;
  const T T11 = vc11 * P11 + vc12 * P12;
  const T T12 = vc11 * P12 + vc12 * P22;
  const T T20 = vc22 * P02;
  const T T21 = vc22 * P12;
  const T T22 = vc22 * P22;
  // v_Sv = -P T
  const T vS00 = -(P00 * T00 + P01 * T10 + P02 * T20);
  const T vS01 = -(P00 * T01 + P01 * T11 + P02 * T21);
  const T vS02 = -(P00 * T02 + P01 * T12 + P02 * T22);
  const T vS10 = -(P01 * T00 + P11 * T10 + P12 * T20);
  const T vS11 = -(P01 * T01 + P11 * T11 + P12 * T21);
  const T vS12 = -(P01 * T02 + P11 * T12 + P12 * T22);
  const T vS20 = -(P02 * T00 + P12 * T10 + P22 * T20);
  const T vS21 = -(P02 * T01 + P12 * T11 + P22 * T21);
  const T vS22 = -(P02 * T02 + P12 * T12 + P22 * T22);
  vc_out[0] = vS00 * r0 * r0;
  vc_out[1] = (vS01 + vS10) * r0 * r1;
  vc_out[2] = (vS02 + vS20) * r0 * r2;
  vc_out[3] = vS11 * r1 * r1;
  vc_out[4] = (vS12 + vS21) * r1 * r2;
  vc_out[5] = vS22 * r2 * r2;
}

template <typename T>
int mapping_fwd_impl(const T *means, const T *covars, const T *ranges, const T *centers,
                     uint32_t d2, uint32_t d1, uint32_t d0, double eps, double clip, T *means3d,
                     T *conics, int32_t *radii, int64_t N, r2s_stream_t st) {
  clear_error();
  const char *name = "world_to_volume_mapping_fwd";
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size %lld", name, (long long)N);
  if (N == 0) return R2S_OK;
  R2S_REQUIRE(means && covars && ranges && centers && means3d && conics && radii,
              "%s: null pointer", name);
  mapping_fwd_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0,
                          as_stream(st)>>>(means, covars, ranges, centers, d2, d1, d0,
                                           static_cast<T>(eps), static_cast<T>(clip), means3d,
                                           conics, radii, N);
  return check_launch(name);
}

template <typename T>
int mapping_bwd_impl(const T *means, const T *covars, const T *ranges, const T *centers,
                     uint32_t d2, uint32_t d1, uint32_t d0, double eps, const T *v_means3d,
                     const T *v_conics, T *v_means, T *v_covars, int64_t N, r2s_stream_t st) {
  clear_error();
  const char *name = "world_to_volume_mapping_bwd";
  (void)means;
  (void)centers;
  R2S_REQUIRE(N >= 0 && N <= kInt32Max, "%s: bad size %lld", name, (long long)N);
  if (N == 0) return R2S_OK;
  R2S_REQUIRE(covars && ranges && v_means3d && v_conics && v_means && v_covars,
              "%s: null pointer", name);
  mapping_bwd_kernel<T><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0,
                          as_stream(st)>>>(covars, ranges, d2, d1, d0, static_cast<T>(eps),
                                           v_means3d, v_conics, v_means, v_covars, N);
  return check_launch(name);
}

}  // namespace
}  // namespace r2s

extern "C" {

#define R2S_MAP_API(SUF, T)                                                                    \
  int r2s_world_to_volume_mapping_fwd_##SUF(const T *means, const T *covars, const T *ranges,  \
                                            const T *centers, uint32_t d2, uint32_t d1,        \
                                            uint32_t d0, double eps, double clip, T *means3d,  \
                                            T *conics, int32_t *radii, int64_t N,              \
                                            r2s_stream_t st) {                                 \
    return r2s::mapping_fwd_impl<T>(means, covars, ranges, centers, d2, d1, d0, eps, clip,     \
                                    means3d, conics, radii, N, st);                            \
  }                                                                                            \
  int r2s_world_to_volume_mapping_bwd_##SUF(const T *means, const T *covars, const T *ranges,  \
                                            const T *centers, uint32_t d2, uint32_t d1,        \
                                            uint32_t d0, double eps, const T *v_means3d,       \
                                            const T *v_conics, T *v_means, T *v_covars,        \
                                            int64_t N, r2s_stream_t st) {                      \
    return r2s::mapping_bwd_impl<T>(means, covars, ranges, centers, d2, d1, d0, eps,           \
                                    v_means3d, v_conics, v_means, v_covars, N, st);            \
  }

R2S_MAP_API(f32, float)
R2S_MAP_API(f64, double)

#undef R2S_MAP_API

}  // extern "C"
