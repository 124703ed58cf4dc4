// Per-Gaussian parameter transform pieces shared by param_transform.hip and
// the fused explicit backward tail in projection.hip: the normalised
// quaternion frame, the logistic functions, and the VJP of
// (quaternion, raw scale) -> packed covariance for one Gaussian.
//
// Expression order follows r2splat/cuda/csrc/ParameterTransformFwd.cu:53-129
// and ParameterTransformBwd.cu:66-245 term by term; every file that includes
// this header compiles it with FMA contraction off, as the restatement in the
// oracle does.
#pragma once
#pragma clang fp contract(off)

#include "r2s_common.h"

namespace r2s {

template <typename T>
struct QuatFrame {
  T w, x, y, z;       // normalised quaternion
  T R[3][3];          // rotation, row-major
  T qnorm, inv_qnorm;
};

template <typename T>
__device__ __forceinline__ QuatFrame<T> quat_frame(const T *__restrict__ q) {
  QuatFrame<T> f;
  const T rw = q[0], rx = q[1], ry = q[2], rz = q[3];
  f.qnorm = sqrt(rw * rw + rx * rx + ry * ry + rz * rz);
  const T qdenom = fmax(f.qnorm, static_cast<T>(1e-12));
  f.inv_qnorm = static_cast<T>(1) / qdenom;
  f.w = rw * f.inv_qnorm;
  f.x = rx * f.inv_qnorm;
  f.y = ry * f.inv_qnorm;
  f.z = rz * f.inv_qnorm;
  const T x2 = f.x * f.x, y2 = f.y * f.y, z2 = f.z * f.z;
  const T xy = f.x * f.y, xz = f.x * f.z, yz = f.y * f.z;
  const T wx = f.w * f.x, wy = f.w * f.y, wz = f.w * f.z;
  const T one = 1, two = 2;
  f.R[0][0] = one - two * (y2 + z2);
  f.R[0][1] = two * (xy - wz);
  f.R[0][2] = two * (xz + wy);
  f.R[1][0] = two * (xy + wz);
  f.R[1][1] = one - two * (x2 + z2);
  f.R[1][2] = two * (yz - wx);
  f.R[2][0] = two * (xz - wy);
  f.R[2][1] = two * (yz + wx);
  f.R[2][2] = one - two * (x2 + y2);
  return f;
}

template <typename T>
__device__ __forceinline__ T sigmoid(T v) {
  return static_cast<T>(1) / (static_cast<T>(1) + exp(-v));
}

// torch.nn.functional.softplus with beta = 1, threshold = 20.
template <typename T>
__device__ __forceinline__ T softplus(T v) {
  return v > static_cast<T>(20) ? v : log1p(exp(v));
}

// VJP of one Gaussian's covariance (ParameterTransformBwd.cu:66-245): the
// packed upstream gradient vc[6] -> v_quat[4] (through the normalisation)
// and v_raw[3] (through the bounded sigmoid scale activation).
template <typename T>
__device__ __forceinline__ void param_bwd_one(const T *__restrict__ quat,
                                              const T *__restrict__ raw_scale, T smin, T smax,
                                              const T vc[6], T *__restrict__ vq,
                                              T *__restrict__ v_raw) {
  const QuatFrame<T> f = quat_frame(quat);
  const T range = smax - smin;
  T s[3], sig[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    sig[k] = sigmoid(raw_scale[k]);
    s[k] = sig[k] * range + smin;
  }
  const T half = static_cast<T>(0.5), two = static_cast<T>(2);
  // Symmetric upstream gradient with halved off-diagonals.
  const T v0 = vc[0], v1 = vc[1] * half, v2 = vc[2] * half;
  const T v3 = vc[3], v4 = vc[4] * half, v5 = vc[5];
  const T V[3][3] = {{v0, v1, v2}, {v1, v3, v4}, {v2, v4, v5}};
  const auto &R = f.R;
  T vM[3][3], vR[3][3];
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const T inner = V[r][0] * R[0][c] + V[r][1] * R[1][c] + V[r][2] * R[2][c];
      vM[r][c] = two * inner * s[c];
      vR[r][c] = two * inner * s[c] * s[c];
    }
  const T w = f.w, x = f.x, y = f.y, z = f.z;
  const T m2 = static_cast<T>(-2);
  const T vw = two * (x * (vR[2][1] - vR[1][2]) + y * (vR[0][2] - vR[2][0]) +
                      z * (vR[1][0] - vR[0][1]));
  const T vx = two * (m2 * x * (vR[1][1] + vR[2][2]) + y * (vR[0][1] + vR[1][0]) +
                      z * (vR[0][2] + vR[2][0]) + w * (vR[2][1] - vR[1][2]));
  const T vy = two * (x * (vR[0][1] + vR[1][0]) + m2 * y * (vR[0][0] + vR[2][2]) +
                      z * (vR[1][2] + vR[2][1]) + w * (vR[0][2] - vR[2][0]));
  const T vz = two * (x * (vR[0][2] + vR[2][0]) + y * (vR[1][2] + vR[2][1]) +
                      m2 * z * (vR[0][0] + vR[1][1]) + w * (vR[1][0] - vR[0][1]));
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const T vs = R[0][c] * vM[0][c] + R[1][c] * vM[1][c] + R[2][c] * vM[2][c];
    v_raw[c] = vs * sig[c] * (static_cast<T>(1) - sig[c]) * range;
  }
  const T inv = f.inv_qnorm;
  if (f.qnorm > static_cast<T>(1e-12)) {
    const T dot = w * vw + x * vx + y * vy + z * vz;
    vq[0] = (vw - w * dot) * inv;
    vq[1] = (vx - x * dot) * inv;
    vq[2] = (vy - y * dot) * inv;
    vq[3] = (vz - z * dot) * inv;
  } else {
    vq[0] = vw * inv;
    vq[1] = vx * inv;
    vq[2] = vy * inv;
    vq[3] = vz * inv;
  }
}

}  // namespace r2s
