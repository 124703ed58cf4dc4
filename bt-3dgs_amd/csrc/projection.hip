// Cone-beam projection of 3D Gaussians to the detector, the line-integral
// normaliser mu, and their VJPs.
//
// Forward (per camera, Gaussian): camera transform, perspective mean, FOV-
// clamped Jacobian J with the ray row, cov2d = J R Sigma R^T J^T (packed
// upper-triangular 3x3), tile radii; then conic = inverse of the blurred 2x2
// block and mu = sqrt(2 pi det3 / det2).  Backward: the VJP of both, summed
// over cameras by one thread per Gaussian (no atomics, no zero-init).
//
// Expression order follows r2splat/cuda/csrc/WorldToImageProjectionFwd.cu,
// WorldToImageProjectionBwd.cu, ConicsMuFwd.cu and ConicsMuBwd.cu term by
// term with contraction off; with IEEE division and square root the float32
// outputs are reproducible bit-for-bit by an IEEE CPU restatement.
// The rasterizer's payload writer, included before the pragma below so that
// it is compiled as in the rasterizer (the fused projection writes the same
// bits as raster_pack_kernel).
#include "r2s_payload.h"

#pragma clang fp contract(off)

#include "r2s_common.h"
#include "r2s_param.h"

namespace r2s {
namespace {

template <typename T>
struct Camera {
  T R[3][3];
  T t[3];
  T fx, fy, cx, cy;
  T lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg;
};

template <typename T>
__device__ __forceinline__ Camera<T> load_camera(const T *__restrict__ vm,
                                                 const T *__restrict__ K, uint32_t width,
                                                 uint32_t height) {
  Camera<T> c;
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int k = 0; k < 3; ++k) c.R[r][k] = vm[4 * r + k];
    c.t[r] = vm[4 * r + 3];
  }
  c.fx = K[0];
  c.fy = K[4];
  c.cx = K[2];
  c.cy = K[5];
  const T W = static_cast<T>(width), H = static_cast<T>(height);
  const T tan_fovx = static_cast<T>(0.5) * W / c.fx;
  const T tan_fovy = static_cast<T>(0.5) * H / c.fy;
  c.lim_x_pos = (W - c.cx) / c.fx + static_cast<T>(0.3) * tan_fovx;
  c.lim_x_neg = c.cx / c.fx + static_cast<T>(0.3) * tan_fovx;
  c.lim_y_pos = (H - c.cy) / c.fy + static_cast<T>(0.3) * tan_fovy;
  c.lim_y_neg = c.cy / c.fy + static_cast<T>(0.3) * tan_fovy;
  return c;
}

// Sigma_c = R Sigma R^T (packed: 00, 01, 02, 11, 12, 22).
template <typename T>
__device__ __forceinline__ void camera_covariance(const Camera<T> &c, const T s[6], T Sc[6]) {
  const T S[3][3] = {{s[0], s[1], s[2]}, {s[1], s[3], s[4]}, {s[2], s[4], s[5]}};
  T M[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      M[i][j] = S[i][0] * c.R[j][0] + S[i][1] * c.R[j][1] + S[i][2] * c.R[j][2];
  const int ii[6] = {0, 0, 0, 1, 1, 2}, jj[6] = {0, 1, 2, 1, 2, 2};
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const int i = ii[k], j = jj[k];
    Sc[k] = c.R[i][0] * M[0][j] + c.R[i][1] * M[1][j] + c.R[i][2] * M[2][j];
  }
}

template <typename T>
struct ProjOut {
  T mx, my;
  T cov[6];
  int32_t rx, ry;
};

// WorldToImageProjectionFwd.cu:118-283 for one (camera, Gaussian).
template <typename T>
__device__ __forceinline__ ProjOut<T> project_one(const Camera<T> &c, const T p[3],
                                                  const T s[6], uint32_t width,
                                                  uint32_t height, T eps, T clip) {
  ProjOut<T> o;
  const T x = c.R[0][0] * p[0] + c.R[0][1] * p[1] + c.R[0][2] * p[2] + c.t[0];
  const T y = c.R[1][0] * p[0] + c.R[1][1] * p[1] + c.R[1][2] * p[2] + c.t[1];
  const T z = c.R[2][0] * p[0] + c.R[2][1] * p[1] + c.R[2][2] * p[2] + c.t[2];
  if (z <= static_cast<T>(0.01)) {
    o.mx = o.my = 0;
#pragma unroll
    for (int k = 0; k < 6; ++k) o.cov[k] = 0;
    o.rx = o.ry = 0;
    return o;
  }
  const T rz = static_cast<T>(1) / z;
  const T rz2 = rz * rz;
  o.mx = c.fx * x * rz + c.cx;
  o.my = c.fy * y * rz + c.cy;
  const T tx = z * fmin(c.lim_x_pos, fmax(-c.lim_x_neg, x * rz));
  const T ty = z * fmin(c.lim_y_pos, fmax(-c.lim_y_neg, y * rz));
  const T l = sqrt(tx * tx + ty * ty + z * z);
  const T rl = static_cast<T>(1) / l;
  const T J00 = c.fx * rz, J02 = -c.fx * tx * rz2;
  const T J11 = c.fy * rz, J12 = -c.fy * ty * rz2;
  const T J20 = tx * rl, J21 = ty * rl, J22 = z * rl;
  T Sc[6];
  camera_covariance(c, s, Sc);
  const T Sc00 = Sc[0], Sc01 = Sc[1], Sc02 = Sc[2], Sc11 = Sc[3], Sc12 = Sc[4], Sc22 = Sc[5];
  // N = Sigma_c J^T, C2 = J N (J01 = J10 = 0).
  const T N00 = Sc00 * J00 + Sc02 * J02;
  const T N01 = Sc01 * J11 + Sc02 * J12;
  const T N02 = Sc00 * J20 + Sc01 * J21 + Sc02 * J22;
  const T N11 = Sc11 * J11 + Sc12 * J12;
  const T N12 = Sc01 * J20 + Sc11 * J21 + Sc12 * J22;
  const T N20 = Sc02 * J00 + Sc22 * J02;
  const T N21 = Sc12 * J11 + Sc22 * J12;
  const T N22 = Sc02 * J20 + Sc12 * J21 + Sc22 * J22;
  o.cov[0] = J00 * N00 + J02 * N20;
  o.cov[1] = J00 * N01 + J02 * N21;
  o.cov[2] = J00 * N02 + J02 * N22;
  o.cov[3] = J11 * N11 + J12 * N21;
  o.cov[4] = J11 * N12 + J12 * N22;
  o.cov[5] = J20 * N02 + J21 * N12 + J22 * N22;
  // Axis-aligned tile radii of the blurred 2x2 block.
  o.rx = o.ry = 0;
  const T a_blur = o.cov[0] + eps;
  const T d_blur = o.cov[3] + eps;
  const T det_blur = a_blur * d_blur - o.cov[1] * o.cov[1];
  if (det_blur <= static_cast<T>(0)) return o;
  const T radius_x = ceil(clip * sqrt(fmax(static_cast<T>(0), a_blur)));
  const T radius_y = ceil(clip * sqrt(fmax(static_cast<T>(0), d_blur)));
  if (!isfinite(radius_x) || !isfinite(radius_y) || radius_x <= static_cast<T>(0) ||
      radius_y <= static_cast<T>(0))
    return o;
  if (o.mx + radius_x <= static_cast<T>(0) || o.mx - radius_x >= static_cast<T>(width) ||
      o.my + radius_y <= static_cast<T>(0) || o.my - radius_y >= static_cast<T>(height))
    return o;
  o.rx = static_cast<int32_t>(radius_x);
  o.ry = static_cast<int32_t>(radius_y);
  return o;
}

// ConicsMuFwd.cu:46-99 for one packed cov2d.
template <typename T>
__device__ __forceinline__ void conic_mu_one(const T cov[6], T eps, T conic[3], T &mu) {
  const T a = cov[0], b = cov[1], c = cov[2], d = cov[3], e = cov[4], f = cov[5];
  const T ab = a + eps, db = d + eps, fb = f + eps;
  const T D2b = ab * db - b * b;
  const T D3b = ab * db * fb - ab * e * e - b * b * fb + static_cast<T>(2) * b * c * e - c * c * db;
  if (D2b <= static_cast<T>(1e-9)) {
    conic[0] = conic[1] = conic[2] = 0;
    mu = 0;
    return;
  }
  const T inv = static_cast<T>(1) / D2b;
  conic[0] = db * inv;
  conic[1] = -b * inv;
  conic[2] = ab * inv;
  const T ratio = D3b * inv;
  mu = ratio > static_cast<T>(0) ? sqrt(static_cast<T>(2.0 * M_PI) * ratio) : static_cast<T>(0);
}

// ConicsMuBwd.cu:63-169 for one element -> v_cov[6].
template <typename T>
__device__ __forceinline__ void conic_mu_bwd_one(const T cov[6], T eps, const T conic[3], T mu,
                                                 const T vcon[3], T vmu, T g[6]) {
  const T u11 = conic[0], u12 = conic[1], u22 = conic[2];
  if (u11 == static_cast<T>(0) && u12 == static_cast<T>(0) && u22 == static_cast<T>(0)) {
#pragma unroll
    for (int k = 0; k < 6; ++k) g[k] = 0;
    return;
  }
  const T two = 2;
  g[0] = -(vcon[0] * u11 * u11 + vcon[1] * u11 * u12 + vcon[2] * u12 * u12);
  g[1] = -(vcon[0] * two * u11 * u12 + vcon[1] * (u11 * u22 + u12 * u12) +
           vcon[2] * two * u12 * u22);
  g[2] = 0;
  g[3] = -(vcon[0] * u12 * u12 + vcon[1] * u12 * u22 + vcon[2] * u22 * u22);
  g[4] = 0;
  g[5] = 0;
  if (mu > static_cast<T>(0)) {
    const T ab = cov[0] + eps, b = cov[1], c = cov[2];
    const T db = cov[3] + eps, e = cov[4], fb = cov[5] + eps;
    const T D3b = ab * db * fb - ab * e * e - b * b * fb + two * b * c * e - c * c * db;
    if (D3b > static_cast<T>(1e-9)) {
      const T inv = static_cast<T>(1) / D3b;
      const T q00 = (db * fb - e * e) * inv;
      const T q01 = (c * e - b * fb) * inv;
      const T q02 = (b * e - c * db) * inv;
      const T q11 = (ab * fb - c * c) * inv;
      const T q12 = (b * c - ab * e) * inv;
      const T q22 = (ab * db - b * b) * inv;
      const T h = static_cast<T>(0.5) * mu * vmu;
      g[0] += h * (q00 - u11);
      g[1] += h * (two * q01 - two * u12);
      g[2] += h * (two * q02);
      g[3] += h * (q11 - u22);
      g[4] += h * (two * q12);
      g[5] += h * q22;
    }
  }
}

// WorldToImageProjectionBwd.cu:116-545 for one (camera, Gaussian); adds the
// world-space gradients into vp[3] and vs[6].
template <typename T>
__device__ __forceinline__ void project_bwd_one(const Camera<T> &c, const T p[3], const T s[6],
                                                T vm2x, T vm2y, const T vcov[6], T vp[3],
                                                T vs[6]) {
  const T x = c.R[0][0] * p[0] + c.R[0][1] * p[1] + c.R[0][2] * p[2] + c.t[0];
  const T y = c.R[1][0] * p[0] + c.R[1][1] * p[1] + c.R[1][2] * p[2] + c.t[1];
  const T z = c.R[2][0] * p[0] + c.R[2][1] * p[1] + c.R[2][2] * p[2] + c.t[2];
  if (z <= static_cast<T>(0.01)) return;
  const T fx = c.fx, fy = c.fy;
  const T rz = static_cast<T>(1) / z;
  const T rz2 = rz * rz;
  const T rz3 = rz2 * rz;
  const T xrz = x * rz, yrz = y * rz;
  const T tx = z * fmin(c.lim_x_pos, fmax(-c.lim_x_neg, xrz));
  const T ty = z * fmin(c.lim_y_pos, fmax(-c.lim_y_neg, yrz));
  const bool x_cl = (xrz > c.lim_x_pos) || (xrz < -c.lim_x_neg);
  const bool y_cl = (yrz > c.lim_y_pos) || (yrz < -c.lim_y_neg);
  const T l = sqrt(tx * tx + ty * ty + z * z);
  const T rl = static_cast<T>(1) / l;
  const T rl2 = rl * rl;
  const T J00 = fx * rz, J02 = -fx * tx * rz2;
  const T J11 = fy * rz, J12 = -fy * ty * rz2;
  const T J20 = tx * rl, J21 = ty * rl, J22 = z * rl;
  T Sc[6];
  camera_covariance(c, s, Sc);
  const T Sc00 = Sc[0], Sc01 = Sc[1], Sc02 = Sc[2], Sc11 = Sc[3], Sc12 = Sc[4], Sc22 = Sc[5];
  const T va = vcov[0], vb = vcov[1], vc = vcov[2], vd = vcov[3], ve = vcov[4], vf = vcov[5];

  // Mean path.
  T v_pc_x = fx * rz * vm2x;
  T v_pc_y = fy * rz * vm2y;
  T v_pc_z = -(fx * x * rz2 * vm2x + fy * y * rz2 * vm2y);

  // Sigma path: v_Sigma_c = J^T G_upper J, then R^T (.) R, symmetric gather.
  const T T00 = va * J00 + vc * J20;
  const T T01 = vb * J11 + vc * J21;
  const T T02 = va * J02 + vb * J12 + vc * J22;
  const T T10 = ve * J20;
  const T T11 = vd * J11 + ve * J21;
  const T T12 = vd * J12 + ve * J22;
  const T T20 = vf * J20;
  const T T21 = vf * J21;
  const T T22 = vf * J22;
  const T vSc[3][3] = {
      {J00 * T00 + J20 * T20, J00 * T01 + J20 * T21, J00 * T02 + J20 * T22},
      {J11 * T10 + J21 * T20, J11 * T11 + J21 * T21, J11 * T12 + J21 * T22},
      {J02 * T00 + J12 * T10 + J22 * T20, J02 * T01 + J12 * T11 + J22 * T21,
       J02 * T02 + J12 * T12 + J22 * T22}};
  T Q[3][3], vS[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      Q[i][j] = vSc[i][0] * c.R[0][j] + vSc[i][1] * c.R[1][j] + vSc[i][2] * c.R[2][j];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      vS[i][j] = c.R[0][i] * Q[0][j] + c.R[1][i] * Q[1][j] + c.R[2][i] * Q[2][j];
  vs[0] += vS[0][0];
  vs[1] += vS[0][1] + vS[1][0];
  vs[2] += vS[0][2] + vS[2][0];
  vs[3] += vS[1][1];
  vs[4] += vS[1][2] + vS[2][1];
  vs[5] += vS[2][2];

  // Jacobian path: v_J = (G + G^T) J Sigma_c.
  const T two = 2;
  const T G[3][3] = {{two * va, vb, vc}, {vb, two * vd, ve}, {vc, ve, two * vf}};
  const T U[3][3] = {
      {J00 * Sc00 + J02 * Sc02, J00 * Sc01 + J02 * Sc12, J00 * Sc02 + J02 * Sc22},
      {J11 * Sc01 + J12 * Sc02, J11 * Sc11 + J12 * Sc12, J11 * Sc12 + J12 * Sc22},
      {J20 * Sc00 + J21 * Sc01 + J22 * Sc02, J20 * Sc01 + J21 * Sc11 + J22 * Sc12,
       J20 * Sc02 + J21 * Sc12 + J22 * Sc22}};
  T vJ[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      vJ[i][j] = G[i][0] * U[0][j] + G[i][1] * U[1][j] + G[i][2] * U[2][j];

  v_pc_z += -fx * rz2 * vJ[0][0];
  v_pc_z += -fy * rz2 * vJ[1][1];
  v_pc_z += rl * vJ[2][2];
  if (!x_cl) v_pc_x += -fx * rz2 * vJ[0][2];
  v_pc_z += two * fx * tx * rz3 * vJ[0][2];
  if (!y_cl) v_pc_y += -fy * rz2 * vJ[1][2];
  v_pc_z += two * fy * ty * rz3 * vJ[1][2];
  if (!x_cl) v_pc_x += rl * vJ[2][0];
  if (!y_cl) v_pc_y += rl * vJ[2][1];
  const T v_l = -tx * rl2 * vJ[2][0] - ty * rl2 * vJ[2][1] - z * rl2 * vJ[2][2];
  if (!x_cl) v_pc_x += v_l * tx * rl;
  if (!y_cl) v_pc_y += v_l * ty * rl;
  v_pc_z += v_l * z * rl;
  if (x_cl) {
    v_pc_z += v_l * tx * rl * (tx / z);
    v_pc_z += (tx / z) * rl * vJ[2][0];
  }
  if (y_cl) {
    v_pc_z += v_l * ty * rl * (ty / z);
    v_pc_z += (ty / z) * rl * vJ[2][1];
  }
  if (x_cl) v_pc_z += -fx * (tx / z) * rz2 * vJ[0][2];
  if (y_cl) v_pc_z += -fy * (ty / z) * rz2 * vJ[1][2];

  vp[0] += c.R[0][0] * v_pc_x + c.R[1][0] * v_pc_y + c.R[2][0] * v_pc_z;
  vp[1] += c.R[0][1] * v_pc_x + c.R[1][1] * v_pc_y + c.R[2][1] * v_pc_z;
  vp[2] += c.R[0][2] * v_pc_x + c.R[1][2] * v_pc_y + c.R[2][2] * v_pc_z;
}

// ---------------------------------------------------------------- kernels --

// Projection forward; optionally fused with conics/mu and the opacity
// broadcast (conics == nullptr selects the plain operator), and then with the
// rasterizer's packed payload (payload != nullptr: what raster_pack_kernel
// writes from these outputs) and the zeros of the raster backward's outputs
// (z_xy != nullptr).
template <typename T>
__global__ __launch_bounds__(256) void project_fwd_kernel(
    const T *__restrict__ means, const T *__restrict__ covars, const T *__restrict__ opac,
    const T *__restrict__ viewmats, const T *__restrict__ Ks, uint32_t width, uint32_t height,
    T eps, T eps_conic, T clip, T *__restrict__ means2d, T *__restrict__ cov2d,
    int32_t *__restrict__ radii, T *__restrict__ conics, T *__restrict__ mus,
    T *__restrict__ opac_cn, int64_t C, int64_t N, T *__restrict__ payload,
    T *__restrict__ z_xy, T *__restrict__ z_abs, T *__restrict__ z_conic,
    T *__restrict__ z_opac, T *__restrict__ z_mu) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= C * N) return;
  const int64_t cam = idx / N, g = idx - cam * N;
  const Camera<T> cm = load_camera(viewmats + 16 * cam, Ks + 9 * cam, width, height);
  const T p[3] = {means[3 * g], means[3 * g + 1], means[3 * g + 2]};
  T s[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) s[k] = covars[6 * g + k];
  const ProjOut<T> o = project_one(cm, p, s, width, height, eps, clip);
  means2d[2 * idx] = o.mx;
  means2d[2 * idx + 1] = o.my;
#pragma unroll
  for (int k = 0; k < 6; ++k) cov2d[6 * idx + k] = o.cov[k];
  radii[2 * idx] = o.rx;
  radii[2 * idx + 1] = o.ry;
  if (conics != nullptr) {
    T con[3], mu;
    conic_mu_one(o.cov, eps_conic, con, mu);
    conics[3 * idx] = con[0];
    conics[3 * idx + 1] = con[1];
    conics[3 * idx + 2] = con[2];
    mus[idx] = mu;
    const T o_g = opac[g];
    opac_cn[idx] = o_g;
    if (payload != nullptr) {
      if (z_xy != nullptr) store_raster_zeros(idx, z_xy, z_abs, z_conic, z_opac, z_mu);
      store_payload(payload, idx, o.mx, o.my, con[0], con[1], con[2], o_g * mu);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void conics_mu_fwd_kernel(const T *__restrict__ cov2d, T eps,
                                                            T *__restrict__ conics,
                                                            T *__restrict__ mus, int64_t total) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  T cov[6], con[3], mu;
#pragma unroll
  for (int k = 0; k < 6; ++k) cov[k] = cov2d[6 * idx + k];
  conic_mu_one(cov, eps, con, mu);
  conics[3 * idx] = con[0];
  conics[3 * idx + 1] = con[1];
  conics[3 * idx + 2] = con[2];
  mus[idx] = mu;
}

template <typename T>
__global__ __launch_bounds__(256) void conics_mu_bwd_kernel(
    const T *__restrict__ cov2d, T eps, const T *__restrict__ conics, const T *__restrict__ mus,
    const T *__restrict__ v_conics, const T *__restrict__ v_mus, T *__restrict__ v_cov2d,
    int64_t total) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  T cov[6], con[3], vcon[3], g[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) cov[k] = cov2d[6 * idx + k];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    con[k] = conics[3 * idx + k];
    vcon[k] = v_conics[3 * idx + k];
  }
  conic_mu_bwd_one(cov, eps, con, mus[idx], vcon, v_mus[idx], g);
#pragma unroll
  for (int k = 0; k < 6; ++k) v_cov2d[6 * idx + k] = g[k];
}

// One thread per Gaussian, cameras summed in order.  With conics != nullptr
// the conics/mu VJP is applied first (fused path); otherwise v_cov2d is read.
template <typename T>
__global__ __launch_bounds__(256) void project_bwd_kernel(
    const T *__restrict__ means, const T *__restrict__ covars, const T *__restrict__ viewmats,
    const T *__restrict__ Ks, uint32_t width, uint32_t height, T eps,
    const T *__restrict__ cov2d, const T *__restrict__ conics, const T *__restrict__ mus,
    const T *__restrict__ v_means2d, const T *__restrict__ v_cov2d,
    const T *__restrict__ v_conics, const T *__restrict__ v_mus, T *__restrict__ v_means,
    T *__restrict__ v_covars, int64_t C, int64_t N) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= N) return;
  const T p[3] = {means[3 * g], means[3 * g + 1], means[3 * g + 2]};
  T s[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) s[k] = covars[6 * g + k];
  T vp[3] = {0, 0, 0}, vs[6] = {0, 0, 0, 0, 0, 0};
  for (int64_t cam = 0; cam < C; ++cam) {
    const int64_t idx = cam * N + g;
    const Camera<T> cm = load_camera(viewmats + 16 * cam, Ks + 9 * cam, width, height);
    T vcov[6];
    if (conics != nullptr) {
      T cov[6], con[3], vcon[3];
#pragma unroll
      for (int k = 0; k < 6; ++k) cov[k] = cov2d[6 * idx + k];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        con[k] = conics[3 * idx + k];
        vcon[k] = v_conics[3 * idx + k];
      }
      conic_mu_bwd_one(cov, eps, con, mus[idx], vcon, v_mus[idx], vcov);
    } else {
#pragma unroll
      for (int k = 0; k < 6; ++k) vcov[k] = v_cov2d[6 * idx + k];
    }
    project_bwd_one(cm, p, s, v_means2d[2 * idx], v_means2d[2 * idx + 1], vcov, vp, vs);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) v_means[3 * g + k] = vp[k];
#pragma unroll
  for (int k = 0; k < 6; ++k) v_covars[6 * g + k] = vs[k];
}

// The end of the explicit backward (r2splat.ops) in one pass per Gaussian:
// the projection VJP summed over the views as project_bwd_kernel computes it
// (conics / mu path), plus the volume pass's world-space gradients when
// given (image + volume, the order in which a running sum of the two adds
// them), stored as v_means; then the covariance gradient's
// parameter-transform VJP (param_bwd_one, as param_bwd_kernel) and the
// opacity VJP (as opacity_bwd_kernel) straight from registers.  The same
// expressions in the same order, so the outputs are bit-identical to the
// three kernels run in turn, without the v_covars round trip and two
// launches.
template <typename T>
struct TailArgs {
  const T *means, *covars, *viewmats, *Ks;
  uint32_t width, height;
  T eps;
  const T *cov2d, *conics, *mus, *v_means2d, *v_conics, *v_mus;
  const T *add_means, *add_covars;  // both or neither
  const T *quats, *raw_scales;
  T smin, smax;
  const T *raw_opac, *v_opac_cn, *v_opac_3d;  // v_opac_3d may be null
  T *v_means, *v_quats, *v_raw_scales, *v_raw_opac;
  int64_t C, N;
};

template <typename T>
__global__ __launch_bounds__(256) void explicit_tail_kernel(TailArgs<T> a) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= a.N) return;
  const T p[3] = {a.means[3 * g], a.means[3 * g + 1], a.means[3 * g + 2]};
  T s[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) s[k] = a.covars[6 * g + k];
  T vp[3] = {0, 0, 0}, vs[6] = {0, 0, 0, 0, 0, 0};
  for (int64_t cam = 0; cam < a.C; ++cam) {
    const int64_t idx = cam * a.N + g;
    const Camera<T> cm = load_camera(a.viewmats + 16 * cam, a.Ks + 9 * cam, a.width, a.height);
    T cov[6], con[3], vcon[3], vcov[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) cov[k] = a.cov2d[6 * idx + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      con[k] = a.conics[3 * idx + k];
      vcon[k] = a.v_conics[3 * idx + k];
    }
    conic_mu_bwd_one(cov, a.eps, con, a.mus[idx], vcon, a.v_mus[idx], vcov);
    project_bwd_one(cm, p, s, a.v_means2d[2 * idx], a.v_means2d[2 * idx + 1], vcov, vp, vs);
  }
  if (a.add_means != nullptr) {
#pragma unroll
    for (int k = 0; k < 3; ++k) vp[k] = vp[k] + a.add_means[3 * g + k];
#pragma unroll
    for (int k = 0; k < 6; ++k) vs[k] = vs[k] + a.add_covars[6 * g + k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) a.v_means[3 * g + k] = vp[k];
  param_bwd_one(a.quats + 4 * g, a.raw_scales + 3 * g, a.smin, a.smax, vs, a.v_quats + 4 * g,
                a.v_raw_scales + 3 * g);
  T v = 0;
  for (int64_t c = 0; c < a.C; ++c) v += a.v_opac_cn[c * a.N + g];
  if (a.v_opac_3d != nullptr) v += a.v_opac_3d[g];
  a.v_raw_opac[g] = v * sigmoid(a.raw_opac[g]);
}

// ------------------------------------------------------------ host side --

int check_sizes(int64_t C, int64_t N, const char *name) {
  R2S_REQUIRE(C >= 0 && N >= 0, "%s: negative size", name);
  R2S_REQUIRE(C * N <= kInt32Max, "%s: C*N = %lld exceeds the int32 index range", name,
              (long long)(C * N));
  return R2S_OK;
}

template <typename T>
int project_fwd_impl(const T *means, const T *covars, const T *opac, const T *viewmats,
                     const T *Ks, uint32_t width, uint32_t height, double eps2d, float clip,
                     T *means2d, T *cov2d, int32_t *radii, T *conics, T *mus, T *opac_cn,
                     int64_t C, int64_t N, r2s_stream_t stream, const char *name,
                     T *payload = nullptr, T *v_xy_abs = nullptr, T *v_xy = nullptr,
                     T *v_conic = nullptr, T *v_opac = nullptr, T *v_mu = nullptr) {
  clear_error();
  R2S_RETURN_IF(check_sizes(C, N, name));
  R2S_REQUIRE(clip > 0.0f, "radius_clip must be positive, got %g", (double)clip);
  R2S_REQUIRE(payload == nullptr || reinterpret_cast<uintptr_t>(payload) % 16 == 0,
              "%s: payload not 16-byte aligned", name);
  R2S_REQUIRE(v_xy == nullptr || (v_conic && v_opac && v_mu),
              "%s: zero targets need v_means2d, v_conics, v_opacities and v_mus", name);
  if (C * N == 0) return R2S_OK;
  R2S_REQUIRE(means && covars && viewmats && Ks && means2d && cov2d && radii,
              "%s: null pointer", name);
  R2S_REQUIRE(conics == nullptr || (mus && opac && opac_cn), "%s: null pointer", name);
  R2S_REQUIRE(payload == nullptr || conics != nullptr, "%s: null conics", name);
  const int64_t blocks = ceil_div(C * N, 256);
  project_fwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      means, covars, opac, viewmats, Ks, width, height,
      static_cast<T>(static_cast<float>(eps2d)), static_cast<T>(eps2d), static_cast<T>(clip),
      means2d, cov2d, radii, conics, mus, opac_cn, C, N, payload, payload ? v_xy : nullptr,
      v_xy_abs, v_conic, v_opac, v_mu);
  return check_launch(name);
}

template <typename T>
int project_bwd_impl(const T *means, const T *covars, const T *viewmats, const T *Ks,
                     uint32_t width, uint32_t height, double eps2d, const T *cov2d,
                     const T *conics, const T *mus, const T *v_means2d, const T *v_cov2d,
                     const T *v_conics, const T *v_mus, T *v_means, T *v_covars, int64_t C,
                     int64_t N, r2s_stream_t stream, const char *name) {
  clear_error();
  R2S_RETURN_IF(check_sizes(C, N, name));
  if (N == 0) return R2S_OK;
  R2S_REQUIRE(means && covars && v_means && v_covars, "%s: null pointer", name);
  R2S_REQUIRE(C == 0 || (viewmats && Ks && v_means2d), "%s: null pointer", name);
  R2S_REQUIRE(C == 0 || conics != nullptr || v_cov2d != nullptr, "%s: null pointer", name);
  R2S_REQUIRE(conics == nullptr || (cov2d && mus && v_conics && v_mus), "%s: null pointer",
              name);
  const int64_t blocks = ceil_div(N, 256);
  project_bwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      means, covars, viewmats, Ks, width, height, static_cast<T>(eps2d), cov2d, conics, mus,
      v_means2d, v_cov2d, v_conics, v_mus, v_means, v_covars, C, N);
  return check_launch(name);
}

template <typename T>
int explicit_tail_impl(TailArgs<T> a, double eps2d, double smin, double smax,
                       r2s_stream_t stream) {
  clear_error();
  const char *name = "explicit_backward_tail";
  R2S_RETURN_IF(check_sizes(a.C, a.N, name));
  R2S_REQUIRE(a.C >= 1, "%s: needs at least one view", name);
  if (a.N == 0) return R2S_OK;
  R2S_REQUIRE(a.means && a.covars && a.viewmats && a.Ks && a.cov2d && a.conics && a.mus &&
                  a.v_means2d && a.v_conics && a.v_mus,
              "%s: null projection input", name);
  R2S_REQUIRE((a.add_means == nullptr) == (a.add_covars == nullptr),
              "%s: add_means and add_covars must be given together", name);
  R2S_REQUIRE(a.quats && a.raw_scales && a.raw_opac && a.v_opac_cn, "%s: null parameter input",
              name);
  R2S_REQUIRE(a.v_means && a.v_quats && a.v_raw_scales && a.v_raw_opac, "%s: null output",
              name);
  a.eps = static_cast<T>(eps2d);
  a.smin = static_cast<T>(smin);
  a.smax = static_cast<T>(smax);
  const int64_t blocks = ceil_div(a.N, 256);
  explicit_tail_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                            as_stream(stream)>>>(a);
  return check_launch(name);
}

template <typename T>
int conics_fwd_impl(const T *cov2d, double eps, T *conics, T *mus, int64_t total,
                    r2s_stream_t stream) {
  clear_error();
  R2S_REQUIRE(total >= 0 && total <= kInt32Max, "conics_mu_fwd: bad size %lld",
              (long long)total);
  if (total == 0) return R2S_OK;
  R2S_REQUIRE(cov2d && conics && mus, "conics_mu_fwd: null pointer");
  const int64_t blocks = ceil_div(total, 256);
  conics_mu_fwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      cov2d, static_cast<T>(eps), conics, mus, total);
  return check_launch("conics_mu_fwd");
}

template <typename T>
int conics_bwd_impl(const T *cov2d, double eps, const T *conics, const T *mus,
                    const T *v_conics, const T *v_mus, T *v_cov2d, int64_t total,
                    r2s_stream_t stream) {
  clear_error();
  R2S_REQUIRE(total >= 0 && total <= kInt32Max, "conics_mu_bwd: bad size %lld",
              (long long)total);
  if (total == 0) return R2S_OK;
  R2S_REQUIRE(cov2d && conics && mus && v_conics && v_mus && v_cov2d,
              "conics_mu_bwd: null pointer");
  const int64_t blocks = ceil_div(total, 256);
  conics_mu_bwd_kernel<T><<<dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, as_stream(stream)>>>(
      cov2d, static_cast<T>(eps), conics, mus, v_conics, v_mus, v_cov2d, total);
  return check_launch("conics_mu_bwd");
}

}  // namespace
}  // namespace r2s

extern "C" {

#define R2S_PROJ_API(SUF, T)                                                                  \
  int r2s_world_to_image_projection_fwd_##SUF(                                                \
      const T *means, const T *covars, const T *viewmats, const T *Ks, uint32_t width,        \
      uint32_t height, float eps2d, float clip, T *means2d, T *cov2d, int32_t *radii,         \
      int64_t C, int64_t N, r2s_stream_t st) {                                                \
    return r2s::project_fwd_impl<T>(means, covars, nullptr, viewmats, Ks, width, height,      \
                                    eps2d, clip, means2d, cov2d, radii, nullptr, nullptr,     \
                                    nullptr, C, N, st, "world_to_image_projection_fwd");      \
  }                                                                                           \
  int r2s_project_gaussians_fwd_##SUF(                                                        \
      const T *means, const T *covars, const T *opac, const T *viewmats, const T *Ks,         \
      uint32_t width, uint32_t height, double eps2d, float clip, T *means2d, T *cov2d,        \
      int32_t *radii, T *conics, T *mus, T *opac_cn, int64_t C, int64_t N, r2s_stream_t st) { \
    if (conics == nullptr) {                                                                  \
      r2s::set_error("project_gaussians_fwd: null conics");                                  \
      return R2S_EINVAL;                                                                      \
    }                                                                                         \
    return r2s::project_fwd_impl<T>(means, covars, opac, viewmats, Ks, width, height, eps2d,  \
                                    clip, means2d, cov2d, radii, conics, mus, opac_cn, C, N,  \
                                    st, "project_gaussians_fwd");                             \
  }                                                                                           \
  int r2s_project_pack_fwd_##SUF(                                                             \
      const T *means, const T *covars, const T *opac, const T *viewmats, const T *Ks,         \
      uint32_t width, uint32_t height, double eps2d, float clip, T *means2d, T *cov2d,        \
      int32_t *radii, T *conics, T *mus, T *opac_cn, T *payload, T *v_xy_abs, T *v_xy,        \
      T *v_conic, T *v_opac, T *v_mu, int64_t C, int64_t N, r2s_stream_t st) {                \
    if (conics == nullptr || payload == nullptr) {                                            \
      r2s::set_error("project_pack_fwd: null conics or payload");                            \
      return R2S_EINVAL;                                                                      \
    }                                                                                         \
    return r2s::project_fwd_impl<T>(means, covars, opac, viewmats, Ks, width, height, eps2d,  \
                                    clip, means2d, cov2d, radii, conics, mus, opac_cn, C, N,  \
                                    st, "project_pack_fwd", payload, v_xy_abs, v_xy,          \
                                    v_conic, v_opac, v_mu);                                   \
  }                                                                                           \
  int r2s_world_to_image_projection_bwd_##SUF(                                                \
      const T *means, const T *covars, const T *viewmats, const T *Ks, uint32_t width,        \
      uint32_t height, const T *v_means2d, const T *v_cov2d, T *v_means, T *v_covars,         \
      int64_t C, int64_t N, r2s_stream_t st) {                                                \
    return r2s::project_bwd_impl<T>(means, covars, viewmats, Ks, width, height, 0.0, nullptr, \
                                    nullptr, nullptr, v_means2d, v_cov2d, nullptr, nullptr,   \
                                    v_means, v_covars, C, N, st,                              \
                                    "world_to_image_projection_bwd");                         \
  }                                                                                           \
  int r2s_project_gaussians_bwd_##SUF(                                                        \
      const T *means, const T *covars, const T *viewmats, const T *Ks, uint32_t width,        \
      uint32_t height, double eps2d, const T *cov2d, const T *conics, const T *mus,           \
      const T *v_means2d, const T *v_conics, const T *v_mus, T *v_means, T *v_covars,         \
      int64_t C, int64_t N, r2s_stream_t st) {                                                \
    if (conics == nullptr) {                                                                  \
      r2s::set_error("project_gaussians_bwd: null conics");                                  \
      return R2S_EINVAL;                                                                      \
    }                                                                                         \
    return r2s::project_bwd_impl<T>(means, covars, viewmats, Ks, width, height, eps2d, cov2d, \
                                    conics, mus, v_means2d, nullptr, v_conics, v_mus,         \
                                    v_means, v_covars, C, N, st, "project_gaussians_bwd");    \
  }                                                                                           \
  int r2s_conics_mu_fwd_##SUF(const T *cov2d, double eps, T *conics, T *mus, int64_t total,   \
                              r2s_stream_t st) {                                              \
    return r2s::conics_fwd_impl<T>(cov2d, eps, conics, mus, total, st);                       \
  }                                                                                           \
  int r2s_conics_mu_bwd_##SUF(const T *cov2d, double eps, const T *conics, const T *mus,      \
                              const T *v_conics, const T *v_mus, T *v_cov2d, int64_t total,   \
                              r2s_stream_t st) {                                              \
    return r2s::conics_bwd_impl<T>(cov2d, eps, conics, mus, v_conics, v_mus, v_cov2d, total,  \
                                   st);                                                       \
  }                                                                                           \
  int r2s_explicit_backward_tail_##SUF(                                                       \
      const T *means, const T *covars, const T *viewmats, const T *Ks, uint32_t width,        \
      uint32_t height, double eps2d, const T *cov2d, const T *conics, const T *mus,           \
      const T *v_means2d, const T *v_conics, const T *v_mus, const T *add_means,              \
      const T *add_covars, const T *quats, const T *raw_scales, double smin, double smax,     \
      const T *raw_opac, const T *v_opac_cn, const T *v_opac_3d, T *v_means, T *v_quats,      \
      T *v_raw_scales, T *v_raw_opac, int64_t C, int64_t N, r2s_stream_t st) {                \
    r2s::TailArgs<T> a{means,      covars,     viewmats,  Ks,        width,       height,      \
                       T(0),       cov2d,      conics,    mus,       v_means2d,   v_conics,    \
                       v_mus,      add_means,  add_covars, quats,    raw_scales,  T(0),        \
                       T(0),       raw_opac,   v_opac_cn, v_opac_3d, v_means,     v_quats,     \
                       v_raw_scales, v_raw_opac, C,       N};                                 \
    return r2s::explicit_tail_impl<T>(a, eps2d, smin, smax, st);                              \
  }

R2S_PROJ_API(f32, float)
R2S_PROJ_API(f64, double)

#undef R2S_PROJ_API

}  // extern "C"
