// Analytic culling of Gaussian footprints for the rasterizer and voxelizer.
//
// A (pixel|voxel, Gaussian) pair contributes only if alpha = w exp(-sigma)
// passes |alpha| >= thr with sigma >= 0, where sigma = 1/2 d^T P d.  For a
// positive-definite P that can only happen inside the ellipsoid
// sigma <= s*, s* = ln(|w| / thr).  These helpers walk that ellipsoid as
// slices -> rows -> a segment along the contiguous axis, using the
// completed-square forms
//   2D: sigma = 1/2 a (x - xc(y))^2 + 1/2 (det / a) y^2,      xc = -(b / a) y
//   3D: sigma = 1/2 p00 (x - xc(y, z))^2 + 1/2 a2 (y - yc(z))^2 + 1/2 c3 z^2
// (a2, c3 Schur complements), whose terms are all non-negative, so the
// remaining budget s - (terms so far) carries no cancellation error.  Every
// range is conservative:
//   * s* is enlarged by a relative 1e-3 and an absolute 1e-3;
//   * every interval end is widened by kCullMargin (0.125) pixel/voxel.
// Elements inside a range are still evaluated with the per-element test, so
// culling only removes elements that cannot pass it.  Determinants and Schur
// complements are computed in double.
#pragma once

#include "r2s_common.h"

namespace r2s {

constexpr double kCullMargin = 0.125;
constexpr double kLog2e = 1.4426950408889634074;

// 2^-x: one v_exp_f32 for float (the kernels pre-scale sigma by log2(e), so
// exp(-sigma) = 2^-(sigma log2 e)); the library exp2 for double.
__device__ __forceinline__ float neg_exp2(float x) { return __builtin_amdgcn_exp2f(-x); }
__device__ __forceinline__ double neg_exp2(double x) { return exp2(-x); }

// The per-element alpha test -- sigma >= 0 and |w| exp(-sigma) >= thr, with
// sl = sigma log2(e) -- as one unsigned compare of sl's bit pattern.
// Non-negative values order like their patterns, and every negative value
// (and -0, -inf, a negative NaN) has a larger pattern than any non-negative
// one, so with sl* = log2(|w| / thr) >= 0:
//   sl in [+0, sl*]  <=>  bits(sl) < bits(sl*) + 1.
// Limits by record:
//   * |w| < thr: 0, nothing passes (|alpha| <= |w| for sigma >= 0);
//   * non-finite geometry or a NaN w: the sign bit, so every sl >= +0, +inf
//     and a positive NaN pass -- their alpha is 0 or non-finite, which the
//     reference does not skip either -- and sl < 0 fails, as there.
// It differs from testing exp(-sigma) against thr / |w| only for elements
// whose alpha is within a few ulp of thr.
template <typename T>
struct Bits;
template <>
struct Bits<float> {
  using type = uint32_t;
  static constexpr uint32_t kSign = 0x80000000u;
};
template <>
struct Bits<double> {
  using type = uint64_t;
  static constexpr uint64_t kSign = 0x8000000000000000ull;
};

__device__ __forceinline__ uint32_t bits_of(float x) { return __float_as_uint(x); }
__device__ __forceinline__ uint64_t bits_of(double x) {
  return static_cast<uint64_t>(__double_as_longlong(x));
}

template <typename T>
__device__ __forceinline__ typename Bits<T>::type alpha_limit(T w, bool finite_geometry,
                                                              double thr) {
  const T aw = fabs(w);
  if (aw != aw || !finite_geometry) return Bits<T>::kSign;
  if (!(aw >= static_cast<T>(thr))) return 0;
  // log2(|w| / thr) >= 0 (+inf for an infinite w).
  const T sl_max = fmax(log2(aw) - static_cast<T>(log2(thr)), static_cast<T>(0));
  return bits_of(sl_max) + 1;
}

template <typename T>
__device__ __forceinline__ bool alpha_pass(T sl, typename Bits<T>::type limit) {
  return bits_of(sl) < limit;
}

// acc += w 2^-sl where the alpha test passes.  As a branch, not a select:
// the scheduling barrier in it cannot be speculated, so the compiler keeps
// the branch, and the test masks the FMA through EXEC with two scalar
// instructions instead of a vector select (one vector instruction fewer per
// pixel / voxel, and no wait on the compare's VCC); the barrier emits no
// code, so no skip branch is added around the one FMA either.  The exp is
// formed before the branch (the asm statement on it keeps it there), so the
// compare and the mask cover its latency.  A failing pair adds nothing,
// where the select added w * 0: the same sum for a finite w, and for a
// non-finite one no NaN from a pair the reference skips.
template <typename T>
__device__ __forceinline__ void add_passing(T sl, typename Bits<T>::type limit, T w, T &acc) {
  T e = neg_exp2(sl);
  asm volatile("" : "+v"(e));
  if (alpha_pass(sl, limit)) {
    __builtin_amdgcn_sched_barrier(0);
    acc = fma(w, e, acc);
  }
}

// Bits of a limit kept in a T slot (forward records stage it in LDS).
__device__ __forceinline__ float limit_as_value(uint32_t b) { return __uint_as_float(b); }
__device__ __forceinline__ double limit_as_value(uint64_t b) {
  return __longlong_as_double(static_cast<long long>(b));
}

// Keys of the records of a wave: `rb` is the wave's first record (uniform),
// `r` the lane's; the key of record r is the last k with offsets[k] <= r
// (offsets[0] = 0, non-decreasing).  One uniform binary search for rb, then a
// uniform walk over the next few keys' first indices; a window holding more
// boundaries than that (empty keys share their successor's first index, so
// a run of them is many boundaries at one index) finishes with a per-lane
// binary search above the walk's last key.
__device__ __forceinline__ uint32_t wave_record_key(const int32_t *__restrict__ offsets,
                                                    uint32_t n_keys, int64_t n_isects, int64_t rb,
                                                    int64_t r) {
  constexpr uint32_t kWalk = 4;
  uint32_t lo = 0, hi = n_keys;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(offsets[mid]) <= rb)
      lo = mid;
    else
      hi = mid;
  }
  const int64_t r_last = min(rb + 63, n_isects - 1);
  uint32_t key = lo;
  uint32_t k = lo + 1;
  for (uint32_t step = 0; step < kWalk; ++step, ++k) {
    if (k >= n_keys) return key;
    const int64_t bnd = offsets[k];
    if (bnd > r_last) return key;
    if (r >= bnd) key = k;
  }
  // offsets[key] <= r: the last such key at or above it.
  uint32_t a = key, b = n_keys;
  while (b - a > 1) {
    const uint32_t mid = (a + b) >> 1;
    if (static_cast<int64_t>(offsets[mid]) <= r)
      a = mid;
    else
      b = mid;
  }
  return a;
}

// Square root for culling bounds: the hardware v_sqrt_f32 (about 1 ulp),
// far inside the margins, instead of the correctly rounded expansion.
__device__ __forceinline__ float cull_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ double cull_sqrt(double x) { return sqrt(x); }

// Enlarged ln(|w| / thr); the float log is ample against the 1e-3 slack.
__device__ __forceinline__ float sigma_bound(float w_abs, double thr) {
  return (logf(w_abs) - static_cast<float>(log(thr))) * (1.0f + 1e-3f) + 1e-3f;
}
__device__ __forceinline__ double sigma_bound(double w_abs, double thr) {
  return log(w_abs / thr) * (1.0 + 1e-3) + 1e-3;
}

// Integer indices j with (j + 0.5) in [c + lo, c + hi], clamped to [j0, j1].
// Returns false when empty.  Inputs may be non-finite (empty or clamped).
template <typename T>
__device__ __forceinline__ bool index_range(T c, T lo, T hi, int j0, int j1, int &a, int &b) {
  const T flo = ceil(c + lo - static_cast<T>(0.5 + kCullMargin));
  const T fhi = floor(c + hi - static_cast<T>(0.5 - kCullMargin));
  const T cl = fmax(flo, static_cast<T>(j0));
  const T ch = fmin(fhi, static_cast<T>(j1));
  if (!(cl <= ch)) return false;
  a = static_cast<int>(cl);
  b = static_cast<int>(ch);
  return true;
}

// Indices j of [j0, j1] with (j + 0.5 - c - centre)^2 <= 2 budget / p, i.e.
// the segment where 1/2 p (u - centre)^2 <= budget.
template <typename T>
__device__ __forceinline__ bool budget_range(T c, T centre, T budget, T inv_p, int j0, int j1,
                                             int &a, int &b) {
  if (!(budget >= static_cast<T>(0))) return false;
  const T h = sqrt(static_cast<T>(2) * budget * inv_p);
  return index_range<T>(c, centre - h, centre + h, j0, j1, a, b);
}

// 2D footprint of conic (a, b, c) = P for weight |w|.
template <typename T>
struct Cull2 {
  bool ok;   // positive definite and finite: the analytic ranges apply
  T s;       // sigma bound
  T hy;      // half extent along y
  T inv_a;   // 1 / a
  T bx;      // x centre per unit y: xc = -bx y  (b / a)
  T c2;      // det / a: row minimum 1/2 c2 y^2
};

template <typename T>
__device__ __forceinline__ Cull2<T> cull2_setup(T a, T b, T c, T w_abs, double thr) {
  Cull2<T> r;
  const double da = a, db = b, dc = c;
  const double det = da * dc - db * db;
  r.ok = (da > 0.0) && (det > 0.0) && isfinite(det) && isfinite(da) &&
         isfinite(static_cast<double>(w_abs));
  r.s = r.hy = r.inv_a = r.bx = r.c2 = 0;
  if (r.ok) {
    const double s = static_cast<double>(sigma_bound(w_abs, thr));
    r.s = static_cast<T>(s);
    r.hy = static_cast<T>(s > 0.0 ? sqrt(2.0 * s * da / det) : 0.0);
    r.inv_a = static_cast<T>(1.0 / da);
    r.bx = static_cast<T>(db / da);
    r.c2 = static_cast<T>(det / da);
  }
  return r;
}

// 3D footprint of the packed conic q = (p00, p01, p02, p11, p12, p22), axis 0
// of the conic = x (contiguous), 1 = y, 2 = z.
template <typename T>
struct Cull3 {
  bool ok;
  T s;
  T hz;          // half extent along z
  T inv_p;       // 1 / p00
  T a2, inv_a2;  // p11 - p01^2 / p00 and its inverse
  T ky;          // y centre per unit z: yc = -ky z
  T c3;          // det / (p00 a2): slice minimum 1/2 c3 z^2
  // The slice ellipse 1/2 p00 (x - xc)^2 + 1/2 a2 (y - yc)^2 <= budget, with
  // xc = -(kx y + kz z), as vertical chords: at x = xe + u (xe its centre)
  //   1/2 p11 (y - ye + r11 u)^2 + 1/2 e11 u^2 <= budget.
  T kx, kz;      // p01 / p00, p02 / p00
  T r11;         // p01 / p11
  T e11;         // (p00 p11 - p01^2) / p11
  T inv_p11;     // 1 / p11
};

template <typename T>
__device__ __forceinline__ Cull3<T> cull3_setup(const T q[6], T w_abs, double thr) {
  Cull3<T> r;
  const double p00 = q[0], p01 = q[1], p02 = q[2], p11 = q[3], p12 = q[4], p22 = q[5];
  const double m2 = p00 * p11 - p01 * p01;
  const double det = p00 * (p11 * p22 - p12 * p12) - p01 * (p01 * p22 - p12 * p02) +
                     p02 * (p01 * p12 - p11 * p02);
  r.ok = (p00 > 0.0) && (m2 > 0.0) && (det > 0.0) && isfinite(det) && isfinite(m2) &&
         isfinite(static_cast<double>(w_abs));
  r.s = r.hz = r.inv_p = r.a2 = r.inv_a2 = r.ky = r.c3 = 0;
  r.kx = r.kz = r.r11 = r.e11 = r.inv_p11 = 0;
  if (r.ok) {
    // Four reciprocals serve every quotient (a few ulp of double, far
    // inside the margins); the differences of products stay in double.
    const double ip00 = 1.0 / p00, im2 = 1.0 / m2, ip11 = 1.0 / p11, idet = 1.0 / det;
    const double s = static_cast<double>(sigma_bound(w_abs, thr));
    const double a2 = m2 * ip00;
    const double k1 = p12 - p01 * p02 * ip00;
    r.s = static_cast<T>(s);
    r.hz = static_cast<T>(s > 0.0 ? sqrt(2.0 * s * m2 * idet) : 0.0);
    r.inv_p = static_cast<T>(ip00);
    r.a2 = static_cast<T>(a2);
    r.inv_a2 = static_cast<T>(p00 * im2);
    r.ky = static_cast<T>(k1 * p00 * im2);
    r.c3 = static_cast<T>(det * im2);
    r.kx = static_cast<T>(p01 * ip00);
    r.kz = static_cast<T>(p02 * ip00);
    r.r11 = static_cast<T>(p01 * ip11);  // p11 > 0 follows from m2 > 0, p00 > 0
    r.e11 = static_cast<T>(m2 * ip11);
    r.inv_p11 = static_cast<T>(ip11);
  }
  return r;
}

}  // namespace r2s
