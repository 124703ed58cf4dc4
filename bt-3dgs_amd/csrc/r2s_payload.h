// The rasterizer's packed per-(view, Gaussian) payload, written by
// raster_pack_kernel and by the fused projection (project_fwd_kernel), read
// by the packed forward and the two-pass backward as one 32-byte load (in
// float) per record instead of four arrays' lines.
#pragma once

#include "r2s_common.h"
#include "r2s_cull.h"

namespace r2s {

// The rasterizer's alpha threshold: a pair contributes when |alpha| >= kThr2.
constexpr double kThr2 = 1e-5;
// Values per (view, Gaussian) of the payload.
constexpr int kPayloadValues = 8;

template <typename T>
struct PayloadVec;
template <>
struct PayloadVec<float> {
  using type = float4;
};
template <>
struct PayloadVec<double> {
  using type = double4;
};

// Item idx of the payload: {x, y, a, b} {c, o mu, limit bits, hy} -- the
// mean, the conic, o mu, alpha_limit's bits for them and the culling
// half-height hy (-1 when the conic is not positive definite).  The payload
// is 16-byte aligned (the callers check).
template <typename T>
__device__ __forceinline__ void store_payload(T *__restrict__ payload, int64_t idx, T mx, T my,
                                              T a, T b, T c, T om) {
  using V4 = typename PayloadVec<T>::type;
  V4 p0, p1;
  p0.x = mx;
  p0.y = my;
  p0.z = a;
  p0.w = b;
  p1.x = c;
  p1.y = om;
  const bool fin = isfinite(mx) && isfinite(my) && isfinite(a) && isfinite(b) && isfinite(c);
  p1.z = limit_as_value(alpha_limit(om, fin, kThr2));
  const Cull2<T> cu = cull2_setup(a, b, c, fabs(om), kThr2);
  p1.w = cu.ok ? cu.hy : static_cast<T>(-1);
  V4 *dst = reinterpret_cast<V4 *>(payload + kPayloadValues * idx);
  dst[0] = p0;
  dst[1] = p1;
}

// Zeros of item idx in the raster backward's outputs (v_xy_abs may be null),
// which its reduction overwrites for every item with records.
template <typename T>
__device__ __forceinline__ void store_raster_zeros(int64_t idx, T *__restrict__ v_xy,
                                                   T *__restrict__ v_xy_abs,
                                                   T *__restrict__ v_conic, T *__restrict__ v_opac,
                                                   T *__restrict__ v_mu) {
  const T z = static_cast<T>(0);
  v_xy[2 * idx] = v_xy[2 * idx + 1] = z;
  if (v_xy_abs != nullptr) v_xy_abs[2 * idx] = v_xy_abs[2 * idx + 1] = z;
  v_conic[3 * idx] = v_conic[3 * idx + 1] = v_conic[3 * idx + 2] = z;
  v_opac[idx] = z;
  v_mu[idx] = z;
}

}  // namespace r2s
