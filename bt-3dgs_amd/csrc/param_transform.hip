// Parameter transform: (quaternion, raw scale) -> packed 3D covariance, its
// VJP, and the fused "prepare" pass that also applies softplus to the raw
// opacities.  One thread per Gaussian; HBM-streaming (44 B in, 32 B out per
// Gaussian for the fused forward).
//
// Expression order follows r2splat/cuda/csrc/ParameterTransformFwd.cu:53-129
// and ParameterTransformBwd.cu:66-245 term by term, with FMA contraction off,
// so results differ from an IEEE restatement only through exp().
#pragma clang fp contract(off)

#include "r2s_param.h"

namespace r2s {
namespace {

template <typename T>
__device__ __forceinline__ void covariance_of(const QuatFrame<T> &f, const T s[3], T out[6]) {
  const T s0 = s[0] * s[0], s1 = s[1] * s[1], s2 = s[2] * s[2];
  const auto &R = f.R;
  out[0] = R[0][0] * R[0][0] * s0 + R[0][1] * R[0][1] * s1 + R[0][2] * R[0][2] * s2;
  out[1] = R[0][0] * R[1][0] * s0 + R[0][1] * R[1][1] * s1 + R[0][2] * R[1][2] * s2;
  out[2] = R[0][0] * R[2][0] * s0 + R[0][1] * R[2][1] * s1 + R[0][2] * R[2][2] * s2;
  out[3] = R[1][0] * R[1][0] * s0 + R[1][1] * R[1][1] * s1 + R[1][2] * R[1][2] * s2;
  out[4] = R[1][0] * R[2][0] * s0 + R[1][1] * R[2][1] * s1 + R[1][2] * R[2][2] * s2;
  out[5] = R[2][0] * R[2][0] * s0 + R[2][1] * R[2][1] * s1 + R[2][2] * R[2][2] * s2;
}

template <typename T>
__global__ __launch_bounds__(256) void prepare_kernel(
    const T *__restrict__ quats, const T *__restrict__ raw_scales,
    const T *__restrict__ raw_opac, T smin, T smax, T *__restrict__ covars,
    T *__restrict__ max_scales, T *__restrict__ opac_out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const QuatFrame<T> f = quat_frame(quats + 4 * i);
  const T range = smax - smin;
  T s[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) s[k] = sigmoid(raw_scales[3 * i + k]) * range + smin;
  max_scales[i] = fmax(s[0], fmax(s[1], s[2]));
  T c[6];
  covariance_of(f, s, c);
#pragma unroll
  for (int k = 0; k < 6; ++k) covars[6 * i + k] = c[k];
  if (opac_out != nullptr) opac_out[i] = softplus(raw_opac[i]);
}

template <typename T>
__global__ __launch_bounds__(256) void param_bwd_kernel(
    const T *__restrict__ quats, const T *__restrict__ raw_scales, T smin, T smax,
    const T *__restrict__ v_covars, T *__restrict__ v_quats, T *__restrict__ v_raw,
    int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  T vc[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) vc[k] = v_covars[6 * i + k];
  param_bwd_one(quats + 4 * i, raw_scales + 3 * i, smin, smax, vc, v_quats + 4 * i,
                v_raw + 3 * i);
}

// v_raw = (sum_c v_opac_cn[c, i] + v_opac_3d[i]) * sigmoid(raw[i]).
template <typename T>
__global__ __launch_bounds__(256) void opacity_bwd_kernel(
    const T *__restrict__ raw, const T *__restrict__ v_cn, const T *__restrict__ v_3d,
    T *__restrict__ v_raw, int64_t C, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  T v = 0;
  if (v_cn != nullptr)
    for (int64_t c = 0; c < C; ++c) v += v_cn[c * n + i];
  if (v_3d != nullptr) v += v_3d[i];
  v_raw[i] = v * sigmoid(raw[i]);
}

template <typename T>
int prepare_impl(const T *quats, const T *raw_scales, const T *raw_opac, double smin,
                 double smax, T *covars, T *max_scales, T *opac, int64_t n,
                 r2s_stream_t stream, const char *name) {
  clear_error();
  R2S_REQUIRE(n >= 0, "%s: negative size %lld", name, (long long)n);
  if (n == 0) return R2S_OK;
  R2S_REQUIRE(quats && raw_scales && covars && max_scales, "%s: null pointer", name);
  R2S_REQUIRE(opac == nullptr || raw_opac != nullptr, "%s: null raw_opacities", name);
  const int64_t blocks = ceil_div(n, 256);
  prepare_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      quats, raw_scales, raw_opac, static_cast<T>(smin), static_cast<T>(smax), covars,
      max_scales, opac, n);
  return check_launch(name);
}

template <typename T>
int param_bwd_impl(const T *quats, const T *raw_scales, double smin, double smax,
                   const T *v_covars, T *v_quats, T *v_raw, int64_t n,
                   r2s_stream_t stream) {
  clear_error();
  R2S_REQUIRE(n >= 0, "parameter_transform_bwd: negative size");
  if (n == 0) return R2S_OK;
  R2S_REQUIRE(quats && raw_scales && v_covars && v_quats && v_raw,
              "parameter_transform_bwd: null pointer");
  const int64_t blocks = ceil_div(n, 256);
  param_bwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      quats, raw_scales, static_cast<T>(smin), static_cast<T>(smax), v_covars, v_quats,
      v_raw, n);
  return check_launch("parameter_transform_bwd");
}

template <typename T>
int opacity_bwd_impl(const T *raw, const T *v_cn, const T *v_3d, T *v_raw, int64_t C,
                     int64_t n, r2s_stream_t stream) {
  clear_error();
  R2S_REQUIRE(n >= 0 && C >= 0, "opacity_bwd: negative size");
  if (n == 0) return R2S_OK;
  R2S_REQUIRE(raw && v_raw, "opacity_bwd: null pointer");
  const int64_t blocks = ceil_div(n, 256);
  opacity_bwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      raw, v_cn, v_3d, v_raw, C, n);
  return check_launch("opacity_bwd");
}

}  // namespace
}  // namespace r2s

extern "C" {

int r2s_parameter_transform_fwd_f32(const float *q, const float *s, double smin, double smax,
                                    float *cov, float *ms, int64_t n, r2s_stream_t st) {
  return r2s::prepare_impl<float>(q, s, nullptr, smin, smax, cov, ms, nullptr, n, st,
                                  "parameter_transform_fwd");
}
int r2s_parameter_transform_fwd_f64(const double *q, const double *s, double smin,
                                    double smax, double *cov, double *ms, int64_t n,
                                    r2s_stream_t st) {
  return r2s::prepare_impl<double>(q, s, nullptr, smin, smax, cov, ms, nullptr, n, st,
                                   "parameter_transform_fwd");
}
int r2s_parameter_transform_bwd_f32(const float *q, const float *s, double smin, double smax,
                                    const float *vc, float *vq, float *vs, int64_t n,
                                    r2s_stream_t st) {
  return r2s::param_bwd_impl<float>(q, s, smin, smax, vc, vq, vs, n, st);
}
int r2s_parameter_transform_bwd_f64(const double *q, const double *s, double smin,
                                    double smax, const double *vc, double *vq, double *vs,
                                    int64_t n, r2s_stream_t st) {
  return r2s::param_bwd_impl<double>(q, s, smin, smax, vc, vq, vs, n, st);
}
int r2s_prepare_gaussians_f32(const float *q, const float *s, const float *o, double smin,
                              double smax, float *cov, float *ms, float *op, int64_t n,
                              r2s_stream_t st) {
  return r2s::prepare_impl<float>(q, s, o, smin, smax, cov, ms, op, n, st, "prepare_gaussians");
}
int r2s_prepare_gaussians_f64(const double *q, const double *s, const double *o, double smin,
                              double smax, double *cov, double *ms, double *op, int64_t n,
                              r2s_stream_t st) {
  return r2s::prepare_impl<double>(q, s, o, smin, smax, cov, ms, op, n, st,
                                   "prepare_gaussians");
}
int r2s_opacity_bwd_f32(const float *raw, const float *v_cn, const float *v_3d, float *v_raw,
                        int64_t C, int64_t n, r2s_stream_t st) {
  return r2s::opacity_bwd_impl<float>(raw, v_cn, v_3d, v_raw, C, n, st);
}
int r2s_opacity_bwd_f64(const double *raw, const double *v_cn, const double *v_3d,
                        double *v_raw, int64_t C, int64_t n, r2s_stream_t st) {
  return r2s::opacity_bwd_impl<double>(raw, v_cn, v_3d, v_raw, C, n, st);
}

}  // extern "C"
