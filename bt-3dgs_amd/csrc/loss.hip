// Losses of the binary-tree trainer that feed the Gaussian backward: the
// projection loss L1 + (1 - SSIM) + masked edge L1 over rendered projections
// (producing v_image), and the volume TV regulariser (producing v_volume).
//
// src/utils/loss.py:106-172 (BinaryTreeLossComputer) with ssim2d of
// src/utils/metric.py:36-54: 11x11 Gaussian window (sigma 1.5), zero
// padding, c1 = 0.01^2, c2 = 0.03^2, means over all pixels.  The reference
// runs five 2-D convolutions and some twenty element-wise kernels forward
// and about as many again in autograd's backward; here
//
//   ssim_fwd_kernel   one 32x32 tile per block: the two images (and their
//                     halo) in LDS, a separable horizontal pass of the five
//                     moments (x, y, x^2, y^2, xy) into LDS, the vertical
//                     pass, the SSIM map and its partial derivatives A, B, C
//                     (w.r.t. mu_x, E[x^2], E[xy]) written for the backward,
//                     and per-block sums of S, |x - y| and m |x - e|;
//   loss_reduce_kernel the block sums in a fixed order (deterministic);
//   ssim_bwd_kernel   the adjoint: separable passes over A, B, C and the
//                     gradient  d/dx = s_l1 sgn(x - y) / n
//                              - s_ssim (G*A + 2 x G*B + y G*C) / n
//                              + s_edge m sgn(x - e) / n,
//                     with the three upstream scales read from device memory.
//
// Everything is float32, as the reference computes.  The separable window
// g_i g_j equals the reference's outer-product window up to one rounding.
#include <algorithm>
#include <cmath>

#include "r2s_common.h"
#include "r2s_scan.h"

namespace r2s {
namespace {

constexpr int kTile = 32;                  // output tile edge
constexpr int kMaxRadius = 7;              // windows up to 15 x 15
constexpr int kSpan = kTile + 2 * kMaxRadius;
constexpr int kLossThreads = 256;
constexpr int kPerThread = kTile * kTile / kLossThreads;

struct Window {
  float g[2 * kMaxRadius + 1];
  int r;
};

__device__ __forceinline__ float sgn(float v) {
  return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
}

// Loads the tile's (kTile + 2r)^2 halo region of `n_maps` maps (zero outside
// the image) into s[map][row * span + col].
template <int kMaps>
__device__ __forceinline__ void load_halo(const float *const (&src)[kMaps], int H, int W, int oy,
                                          int ox, int r, float (*s)[kSpan * kSpan]) {
  const int span = kTile + 2 * r;
  for (int idx = threadIdx.x; idx < span * span; idx += kLossThreads) {
    const int row = idx / span, col = idx - row * span;
    const int gy = oy - r + row, gx = ox - r + col;
    const bool in = gy >= 0 && gy < H && gx >= 0 && gx < W;
    const int64_t off = static_cast<int64_t>(gy) * W + gx;
#pragma unroll
    for (int m = 0; m < kMaps; ++m) s[m][idx] = in ? src[m][off] : 0.0f;
  }
}

__global__ __launch_bounds__(kLossThreads) void ssim_fwd_kernel(
    const float *__restrict__ x, const float *__restrict__ y, const float *__restrict__ e,
    const float *__restrict__ m, int H, int W, Window win, float *__restrict__ A,
    float *__restrict__ B, float *__restrict__ C, float *__restrict__ partials) {
  __shared__ float s_in[2][kSpan * kSpan];
  __shared__ float s_h[5][kSpan * kTile];
  __shared__ float s_red[3][kLossThreads / 64];
  const int tiles_x = (W + kTile - 1) / kTile;
  const int ty = static_cast<int>(blockIdx.x) / tiles_x, tx = static_cast<int>(blockIdx.x) % tiles_x;
  const int oy = ty * kTile, ox = tx * kTile;
  const int r = win.r, span = kTile + 2 * r, taps = 2 * r + 1;
  const int64_t img = static_cast<int64_t>(blockIdx.y) * H * W;
  const float *const src[2] = {x + img, y + img};
  load_halo<2>(src, H, W, oy, ox, r, s_in);
  __syncthreads();
  // Horizontal pass: five moments at every halo row, for the tile's columns.
  for (int idx = threadIdx.x; idx < span * kTile; idx += kLossThreads) {
    const int row = idx / kTile, c = idx - row * kTile;
    const float *px = &s_in[0][row * span + c];
    const float *py = &s_in[1][row * span + c];
    float hx = 0, hy = 0, hxx = 0, hyy = 0, hxy = 0;
    for (int j = 0; j < taps; ++j) {
      const float g = win.g[j], a = px[j], b = py[j];
      hx = fmaf(g, a, hx);
      hy = fmaf(g, b, hy);
      hxx = fmaf(g, a * a, hxx);
      hyy = fmaf(g, b * b, hyy);
      hxy = fmaf(g, a * b, hxy);
    }
    s_h[0][idx] = hx;
    s_h[1][idx] = hy;
    s_h[2][idx] = hxx;
    s_h[3][idx] = hyy;
    s_h[4][idx] = hxy;
  }
  __syncthreads();
  // c1 = 0.01**2, c2 = 0.03**2 in double, then float32 (torch scalars).
  const float c1 = static_cast<float>(0.01 * 0.01), c2 = static_cast<float>(0.03 * 0.03);
  float sum_s = 0, sum_l1 = 0, sum_edge = 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int o = threadIdx.x + k * kLossThreads;
    const int py_ = o / kTile, px_ = o - py_ * kTile;
    float v[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < taps; ++i) {
      const float g = win.g[i];
      const int at = (py_ + i) * kTile + px_;
#pragma unroll
      for (int q = 0; q < 5; ++q) v[q] = fmaf(g, s_h[q][at], v[q]);
    }
    const int gy = oy + py_, gx = ox + px_;
    if (gy >= H || gx >= W) continue;
    const float mu1 = v[0], mu2 = v[1];
    const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2, mu12 = mu1 * mu2;
    const float s11 = v[2] - mu1_sq, s22 = v[3] - mu2_sq, s12 = v[4] - mu12;
    const float n1 = 2.0f * mu12 + c1, n2 = 2.0f * s12 + c2;
    const float d1 = mu1_sq + mu2_sq + c1, d2 = s11 + s22 + c2;
    const float den = d1 * d2;
    const float S = (n1 * n2) / den;
    // dS/dmu1 (E[x^2], E[xy] held), dS/dE[x^2], dS/dE[xy].
    const float a = 2.0f * mu2 * (n2 - n1) / den - 2.0f * mu1 * S * (1.0f / d1 - 1.0f / d2);
    const int64_t off = img + static_cast<int64_t>(gy) * W + gx;
    A[off] = a;
    B[off] = -S / d2;
    C[off] = 2.0f * n1 / den;
    const float xv = s_in[0][(py_ + r) * span + px_ + r], yv = s_in[1][(py_ + r) * span + px_ + r];
    sum_s += S;
    sum_l1 += fabsf(xv - yv);
    if (e != nullptr) sum_edge += m[off] * fabsf(xv - e[off]);
  }
  sum_s = wave_sum(sum_s);
  sum_l1 = wave_sum(sum_l1);
  sum_edge = wave_sum(sum_edge);
  const int w = static_cast<int>(threadIdx.x) / 64;
  if (lane_id() == 0) {
    s_red[0][w] = sum_s;
    s_red[1][w] = sum_l1;
    s_red[2][w] = sum_edge;
  }
  __syncthreads();
  if (threadIdx.x < 3) {
    float t = 0;
    for (int k = 0; k < kLossThreads / 64; ++k) t += s_red[threadIdx.x][k];
    const int64_t blk = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    partials[3 * blk + threadIdx.x] = t;
  }
}

// losses = {mean |x - y|, 1 - mean S, mean m |x - e|} from the block sums,
// summed in double in a fixed order.
__global__ __launch_bounds__(kLossThreads) void loss_reduce_kernel(const float *__restrict__ partials,
                                                                   int64_t n_blocks, double inv_n,
                                                                   float *__restrict__ losses) {
  __shared__ double s_red[3][kLossThreads / 64];
  double t[3] = {0, 0, 0};
  for (int64_t b = threadIdx.x; b < n_blocks; b += kLossThreads) {
#pragma unroll
    for (int k = 0; k < 3; ++k) t[k] += partials[3 * b + k];
  }
  const int w = static_cast<int>(threadIdx.x) / 64;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const double s = wave_sum(t[k]);
    if (lane_id() == 0) s_red[k][w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double s[3] = {0, 0, 0};
    for (int k = 0; k < 3; ++k)
      for (int j = 0; j < kLossThreads / 64; ++j) s[k] += s_red[k][j];
    losses[0] = static_cast<float>(s[1] * inv_n);
    losses[1] = static_cast<float>(1.0 - s[0] * inv_n);
    losses[2] = static_cast<float>(s[2] * inv_n);
  }
}

__global__ __launch_bounds__(kLossThreads) void ssim_bwd_kernel(
    const float *__restrict__ x, const float *__restrict__ y, const float *__restrict__ e,
    const float *__restrict__ m, const float *__restrict__ A, const float *__restrict__ B,
    const float *__restrict__ C, int H, int W, Window win, float inv_n,
    const float *__restrict__ scales, float *__restrict__ grad) {
  __shared__ float s_in[3][kSpan * kSpan];
  __shared__ float s_h[3][kSpan * kTile];
  const int tiles_x = (W + kTile - 1) / kTile;
  const int ty = static_cast<int>(blockIdx.x) / tiles_x, tx = static_cast<int>(blockIdx.x) % tiles_x;
  const int oy = ty * kTile, ox = tx * kTile;
  const int r = win.r, span = kTile + 2 * r, taps = 2 * r + 1;
  const int64_t img = static_cast<int64_t>(blockIdx.y) * H * W;
  const float *const src[3] = {A + img, B + img, C + img};
  load_halo<3>(src, H, W, oy, ox, r, s_in);
  __syncthreads();
  for (int idx = threadIdx.x; idx < span * kTile; idx += kLossThreads) {
    const int row = idx / kTile, c = idx - row * kTile;
    float h[3] = {0, 0, 0};
    for (int j = 0; j < taps; ++j) {
      const float g = win.g[j];
#pragma unroll
      for (int q = 0; q < 3; ++q) h[q] = fmaf(g, s_in[q][row * span + c + j], h[q]);
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) s_h[q][idx] = h[q];
  }
  __syncthreads();
  const float s_l1 = scales[0] * inv_n, s_ssim = scales[1] * inv_n, s_edge = scales[2] * inv_n;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int o = threadIdx.x + k * kLossThreads;
    const int py_ = o / kTile, px_ = o - py_ * kTile;
    const int gy = oy + py_, gx = ox + px_;
    if (gy >= H || gx >= W) continue;
    float v[3] = {0, 0, 0};
    for (int i = 0; i < taps; ++i) {
      const float g = win.g[i];
      const int at = (py_ + i) * kTile + px_;
#pragma unroll
      for (int q = 0; q < 3; ++q) v[q] = fmaf(g, s_h[q][at], v[q]);
    }
    const int64_t off = img + static_cast<int64_t>(gy) * W + gx;
    const float xv = x[off], yv = y[off];
    const float dssim = v[0] + 2.0f * xv * v[1] + yv * v[2];  // d (sum S) / dx
    float gv = s_l1 * sgn(xv - yv) - s_ssim * dssim;
    if (e != nullptr) gv += s_edge * m[off] * sgn(xv - e[off]);
    grad[off] = gv;
  }
}

// ------------------------------------------------------------------ TV --
// src/utils/loss.py:10-21 compute_tv_loss: sum over the three axes of
// |v[i+1] - v[i]|, divided by the number of differences for "mean".
constexpr int kTvBlocks = 1024;

__device__ __forceinline__ void tv_coords(int64_t i, int D1, int D2, int &a, int &b, int &c) {
  const int64_t plane = static_cast<int64_t>(D1) * D2;
  a = static_cast<int>(i / plane);
  const int64_t rem = i - a * plane;
  b = static_cast<int>(rem / D2);
  c = static_cast<int>(rem - static_cast<int64_t>(b) * D2);
}

// Grid-stride sum of |forward differences|; one partial per block (the grid
// is fixed, so the sum is deterministic).
__global__ __launch_bounds__(kLossThreads) void tv_fwd_kernel(const float *__restrict__ v, int D0,
                                                              int D1, int D2,
                                                              float *__restrict__ partials) {
  __shared__ float s_red[kLossThreads / 64];
  const int64_t n = static_cast<int64_t>(D0) * D1 * D2, plane = static_cast<int64_t>(D1) * D2;
  float acc = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kLossThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kLossThreads) {
    int a, b, c;
    tv_coords(i, D1, D2, a, b, c);
    const float x = v[i];
    if (a + 1 < D0) acc += fabsf(v[i + plane] - x);
    if (b + 1 < D1) acc += fabsf(v[i + D2] - x);
    if (c + 1 < D2) acc += fabsf(v[i + 1] - x);
  }
  acc = wave_sum(acc);
  if (lane_id() == 0) s_red[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0;
    for (int k = 0; k < kLossThreads / 64; ++k) t += s_red[k];
    partials[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(kLossThreads) void sum_reduce_kernel(const float *__restrict__ partials,
                                                                  int64_t n, double scale,
                                                                  float *__restrict__ out) {
  __shared__ double s_red[kLossThreads / 64];
  double t = 0;
  for (int64_t b = threadIdx.x; b < n; b += kLossThreads) t += partials[b];
  t = wave_sum(t);
  if (lane_id() == 0) s_red[threadIdx.x / 64] = t;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0;
    for (int k = 0; k < kLossThreads / 64; ++k) s += s_red[k];
    out[0] = static_cast<float>(s * scale);
  }
}

// d tv / d v = scale * sum over axes of sgn(v - v_prev) - sgn(v_next - v).
__global__ __launch_bounds__(kLossThreads) void tv_bwd_kernel(const float *__restrict__ v, int D0,
                                                              int D1, int D2,
                                                              const float *__restrict__ grad_out,
                                                              float scale,
                                                              float *__restrict__ grad) {
  const int64_t n = static_cast<int64_t>(D0) * D1 * D2, plane = static_cast<int64_t>(D1) * D2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLossThreads + threadIdx.x;
  if (i >= n) return;
  int a, b, c;
  tv_coords(i, D1, D2, a, b, c);
  const float x = v[i];
  float g = 0;
  if (a > 0) g += sgn(x - v[i - plane]);
  if (a + 1 < D0) g -= sgn(v[i + plane] - x);
  if (b > 0) g += sgn(x - v[i - D2]);
  if (b + 1 < D1) g -= sgn(v[i + D2] - x);
  if (c > 0) g += sgn(x - v[i - 1]);
  if (c + 1 < D2) g -= sgn(v[i + 1] - x);
  grad[i] = g * (grad_out[0] * scale);
}

int64_t tv_terms(int D0, int D1, int D2) {
  return static_cast<int64_t>(D0 - 1) * D1 * D2 + static_cast<int64_t>(D0) * (D1 - 1) * D2 +
         static_cast<int64_t>(D0) * D1 * (D2 - 1);
}

// ----------------------------------------------------------- hierarchy --
// src/utils/loss.py:27-71 compute_hierarchy_loss: children whose parent
// index is in the archive contribute relu(|diag(1/s) R^T (c - p)| - a)^2 / a^2
// (R from the parent's normalised quaternion, s its activated scales
// clamped at 1e-6, a = max(factor, 1e-6)); the loss is their mean.  The
// forward also stores each child's gradient for a unit upstream gradient
// and a count of 1, d/dc = 2 e / (a r) M^T M (c - p) with M = diag(1/s) R^T.
__global__ __launch_bounds__(kLossThreads) void hierarchy_fwd_kernel(
    const float *__restrict__ child_means, const int32_t *__restrict__ parent, int64_t n,
    const float *__restrict__ hist_means, const float *__restrict__ hist_scales,
    const float *__restrict__ hist_quats, int64_t hist_count, float allowed,
    float *__restrict__ grad_unit, float *__restrict__ partials) {
  __shared__ float s_red[2][kLossThreads / 64];
  float acc = 0, cnt = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kLossThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kLossThreads) {
    const int32_t pid = parent[i];
    float g0 = 0, g1 = 0, g2 = 0;
    if (pid >= 0 && pid < hist_count) {
      const float *q = hist_quats + 4 * static_cast<int64_t>(pid);
      const float nq = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
      const float den = fmaxf(nq, 1e-12f);
      const float w = q[0] / den, x = q[1] / den, y = q[2] / den, z = q[3] / den;
      // Rows of R^T are the columns of normalized_quat_to_rotmat (math.py:35-53).
      const float r00 = 1 - 2 * (y * y + z * z), r01 = 2 * (x * y - w * z), r02 = 2 * (x * z + w * y);
      const float r10 = 2 * (x * y + w * z), r11 = 1 - 2 * (x * x + z * z), r12 = 2 * (y * z - w * x);
      const float r20 = 2 * (x * z - w * y), r21 = 2 * (y * z + w * x), r22 = 1 - 2 * (x * x + y * y);
      const float *pm = hist_means + 3 * static_cast<int64_t>(pid);
      const float *ps = hist_scales + 3 * static_cast<int64_t>(pid);
      const float d0 = child_means[3 * i] - pm[0], d1 = child_means[3 * i + 1] - pm[1],
                  d2 = child_means[3 * i + 2] - pm[2];
      const float i0 = 1.0f / fmaxf(ps[0], 1e-6f), i1 = 1.0f / fmaxf(ps[1], 1e-6f),
                  i2 = 1.0f / fmaxf(ps[2], 1e-6f);
      // u = diag(1/s) R^T d
      const float u0 = (r00 * d0 + r10 * d1 + r20 * d2) * i0;
      const float u1 = (r01 * d0 + r11 * d1 + r21 * d2) * i1;
      const float u2 = (r02 * d0 + r12 * d1 + r22 * d2) * i2;
      const float rad = sqrtf(u0 * u0 + u1 * u1 + u2 * u2);
      const float e = fmaxf(rad - allowed, 0.0f) / allowed;
      acc += e * e;
      cnt += 1.0f;
      if (e > 0.0f) {
        const float k = 2.0f * e / (allowed * rad);
        const float v0 = k * u0 * i0, v1 = k * u1 * i1, v2 = k * u2 * i2;  // k diag(1/s) u
        g0 = r00 * v0 + r01 * v1 + r02 * v2;  // R v
        g1 = r10 * v0 + r11 * v1 + r12 * v2;
        g2 = r20 * v0 + r21 * v1 + r22 * v2;
      }
    }
    grad_unit[3 * i] = g0;
    grad_unit[3 * i + 1] = g1;
    grad_unit[3 * i + 2] = g2;
  }
  acc = wave_sum(acc);
  cnt = wave_sum(cnt);
  if (lane_id() == 0) {
    s_red[0][threadIdx.x / 64] = acc;
    s_red[1][threadIdx.x / 64] = cnt;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float t = 0;
    for (int k = 0; k < kLossThreads / 64; ++k) t += s_red[threadIdx.x][k];
    partials[2 * blockIdx.x + threadIdx.x] = t;
  }
}

// out[0] = sum / count (0 without valid children), out[1] = count.
__global__ __launch_bounds__(kLossThreads) void hierarchy_reduce_kernel(
    const float *__restrict__ partials, int64_t n_blocks, float *__restrict__ out) {
  __shared__ double s_red[2][kLossThreads / 64];
  double t[2] = {0, 0};
  for (int64_t b = threadIdx.x; b < n_blocks; b += kLossThreads) {
    t[0] += partials[2 * b];
    t[1] += partials[2 * b + 1];
  }
  for (int k = 0; k < 2; ++k) {
    const double v = wave_sum(t[k]);
    if (lane_id() == 0) s_red[k][threadIdx.x / 64] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0, c = 0;
    for (int k = 0; k < kLossThreads / 64; ++k) {
      s += s_red[0][k];
      c += s_red[1][k];
    }
    out[0] = c > 0 ? static_cast<float>(s / c) : 0.0f;
    out[1] = static_cast<float>(c);
  }
}

__global__ __launch_bounds__(kLossThreads) void hierarchy_bwd_kernel(
    const float *__restrict__ grad_unit, int64_t n3, const float *__restrict__ grad_out,
    const float *__restrict__ loss_count, float *__restrict__ v_means) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLossThreads + threadIdx.x;
  if (i >= n3) return;
  const float c = loss_count[1];
  v_means[i] = c > 0.0f ? grad_unit[i] * (grad_out[0] / c) : 0.0f;
}

struct LossSpace {
  float *A, *B, *C, *partials;
};

LossSpace carve_loss(Carver &cv, int64_t n_images, int H, int W) {
  const int64_t npix = n_images * H * W;
  const int64_t blocks = n_images * ceil_div(H, kTile) * ceil_div(W, kTile);
  LossSpace s;
  s.A = cv.take<float>(npix);
  s.B = cv.take<float>(npix);
  s.C = cv.take<float>(npix);
  s.partials = cv.take<float>(3 * blocks);
  return s;
}

int make_window(int window_size, Window &win, const char *what) {
  R2S_REQUIRE(window_size >= 1 && window_size % 2 == 1 && window_size <= 2 * kMaxRadius + 1,
              "%s: window_size must be odd and at most %d, got %d", what, 2 * kMaxRadius + 1,
              window_size);
  // metric.py:13-17: exp(-(x - ws // 2)^2 / (2 sigma^2)) with sigma 1.5, as
  // float32 values normalised by their float32 sum.
  const int r = window_size / 2;
  float e[2 * kMaxRadius + 1];
  float total = 0.0f;
  for (int i = 0; i < window_size; ++i) {
    const double d = static_cast<double>(i - r);
    e[i] = static_cast<float>(std::exp(-(d * d) / (2.0 * 1.5 * 1.5)));
    total += e[i];
  }
  for (int i = 0; i < window_size; ++i) win.g[i] = e[i] / total;
  win.r = r;
  return R2S_OK;
}

int check_loss_args(int64_t n_images, int H, int W, const char *what) {
  R2S_REQUIRE(n_images >= 0 && H >= 0 && W >= 0, "%s: negative size", what);
  R2S_REQUIRE(n_images <= 65535, "%s: at most 65535 images per call", what);
  R2S_REQUIRE(static_cast<int64_t>(H) * W <= kInt32Max, "%s: image too large", what);
  return R2S_OK;
}

int check_tv_args(int D0, int D1, int D2, const char *what) {
  R2S_REQUIRE(D0 >= 0 && D1 >= 0 && D2 >= 0, "%s: negative size", what);
  return R2S_OK;
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_hierarchy_workspace_bytes(int64_t n) {
  const int64_t blocks = std::max<int64_t>(
      1, std::min<int64_t>(r2s::kTvBlocks, r2s::ceil_div(n > 0 ? n : 0, r2s::kLossThreads)));
  r2s::Carver cv(nullptr);
  cv.take<float>(3 * (n > 0 ? n : 0));
  cv.take<float>(2 * blocks);
  return static_cast<int64_t>(cv.used);
}

int r2s_hierarchy_loss_fwd_f32(const float *child_means, const int32_t *parent, int64_t n,
                               const float *history_means, const float *parent_scales,
                               const float *history_quats, int64_t history_count,
                               float max_parent_distance_factor, float *out, void *workspace,
                               size_t workspace_bytes, r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "hierarchy_loss_fwd";
  R2S_REQUIRE(n >= 0 && history_count >= 0, "%s: negative size", what);
  R2S_REQUIRE(out != nullptr, "%s: null output", what);
  R2S_REQUIRE(n == 0 || (child_means && parent), "%s: null child arrays", what);
  R2S_REQUIRE(history_count == 0 || (history_means && parent_scales && history_quats),
              "%s: null history arrays", what);
  const int64_t need = r2s_hierarchy_workspace_bytes(n);
  if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
    r2s::set_error("%s: workspace of %zu bytes, %lld required", what, workspace_bytes,
                   (long long)need);
    return R2S_EWORKSPACE;
  }
  r2s::Carver cv(workspace);
  float *grad_unit = cv.take<float>(3 * n);
  const int64_t blocks =
      std::max<int64_t>(1, std::min<int64_t>(r2s::kTvBlocks, r2s::ceil_div(n, r2s::kLossThreads)));
  float *partials = cv.take<float>(2 * blocks);
  hipStream_t stream = r2s::as_stream(st);
  // loss.py:67: allowed = max(factor, 1e-6).
  const float allowed = std::max(max_parent_distance_factor, 1e-6f);
  r2s::hierarchy_fwd_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(r2s::kLossThreads), 0,
                              stream>>>(child_means, parent, n, history_means, parent_scales,
                                        history_quats, history_count, allowed, grad_unit,
                                        partials);
  R2S_RETURN_IF(r2s::check_launch(what));
  r2s::hierarchy_reduce_kernel<<<1, r2s::kLossThreads, 0, stream>>>(partials, blocks, out);
  return r2s::check_launch(what);
}

int r2s_hierarchy_loss_bwd_f32(int64_t n, const float *grad_out, const float *loss_out,
                               const void *workspace, size_t workspace_bytes, float *v_means,
                               r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "hierarchy_loss_bwd";
  R2S_REQUIRE(n >= 0, "%s: negative size", what);
  if (n == 0) return R2S_OK;
  R2S_REQUIRE(grad_out && loss_out && v_means, "%s: null pointer", what);
  if (workspace == nullptr ||
      static_cast<int64_t>(workspace_bytes) < r2s_hierarchy_workspace_bytes(n)) {
    r2s::set_error("%s: workspace smaller than the forward's", what);
    return R2S_EWORKSPACE;
  }
  const float *grad_unit = static_cast<const float *>(workspace);
  r2s::hierarchy_bwd_kernel<<<dim3(static_cast<uint32_t>(r2s::ceil_div(3 * n, r2s::kLossThreads))),
                              dim3(r2s::kLossThreads), 0, r2s::as_stream(st)>>>(
      grad_unit, 3 * n, grad_out, loss_out, v_means);
  return r2s::check_launch(what);
}

int64_t r2s_tv_workspace_bytes(void) {
  return static_cast<int64_t>(r2s::kTvBlocks * sizeof(float));
}

int r2s_tv_fwd_f32(const float *volume, int32_t D0, int32_t D1, int32_t D2, int32_t mean,
                   float *out, void *workspace, size_t workspace_bytes, r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "tv_fwd";
  R2S_RETURN_IF(r2s::check_tv_args(D0, D1, D2, what));
  R2S_REQUIRE(out != nullptr, "%s: null output", what);
  hipStream_t stream = r2s::as_stream(st);
  const int64_t n = static_cast<int64_t>(D0) * D1 * D2;
  if (n == 0) return r2s::device_fill<float>(out, 1, 0.0f, stream, what);
  R2S_REQUIRE(volume != nullptr, "%s: null volume", what);
  if (workspace == nullptr ||
      static_cast<int64_t>(workspace_bytes) < r2s_tv_workspace_bytes()) {
    r2s::set_error("%s: workspace of %zu bytes, %lld required", what, workspace_bytes,
                   (long long)r2s_tv_workspace_bytes());
    return R2S_EWORKSPACE;
  }
  float *partials = static_cast<float *>(workspace);
  const int64_t blocks = std::min<int64_t>(r2s::kTvBlocks, r2s::ceil_div(n, r2s::kLossThreads));
  r2s::tv_fwd_kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(r2s::kLossThreads), 0,
                       stream>>>(volume, D0, D1, D2, partials);
  R2S_RETURN_IF(r2s::check_launch(what));
  // loss.py:19-20: mean divides by max(1, number of differences).
  const int64_t terms = r2s::tv_terms(D0, D1, D2);
  const double scale = mean ? 1.0 / static_cast<double>(terms > 1 ? terms : 1) : 1.0;
  r2s::sum_reduce_kernel<<<1, r2s::kLossThreads, 0, stream>>>(partials, blocks, scale, out);
  return r2s::check_launch(what);
}

int r2s_tv_bwd_f32(const float *volume, int32_t D0, int32_t D1, int32_t D2, int32_t mean,
                   const float *grad_out, float *v_volume, r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "tv_bwd";
  R2S_RETURN_IF(r2s::check_tv_args(D0, D1, D2, what));
  const int64_t n = static_cast<int64_t>(D0) * D1 * D2;
  if (n == 0) return R2S_OK;
  R2S_REQUIRE(volume && grad_out && v_volume, "%s: null pointer", what);
  const int64_t terms = r2s::tv_terms(D0, D1, D2);
  const float scale =
      mean ? static_cast<float>(1.0 / static_cast<double>(terms > 1 ? terms : 1)) : 1.0f;
  r2s::tv_bwd_kernel<<<dim3(static_cast<uint32_t>(r2s::ceil_div(n, r2s::kLossThreads))),
                       dim3(r2s::kLossThreads), 0, r2s::as_stream(st)>>>(volume, D0, D1, D2,
                                                                         grad_out, scale,
                                                                         v_volume);
  return r2s::check_launch(what);
}

int64_t r2s_projection_loss_workspace_bytes(int64_t n_images, int32_t H, int32_t W) {
  r2s::Carver cv(nullptr);
  r2s::carve_loss(cv, n_images > 0 ? n_images : 0, H > 0 ? H : 0, W > 0 ? W : 0);
  return static_cast<int64_t>(cv.used);
}

int r2s_projection_loss_fwd_f32(const float *render, const float *target,
                                const float *edge_target, const float *edge_mask,
                                int64_t n_images, int32_t H, int32_t W, int32_t window_size,
                                float *losses, void *workspace, size_t workspace_bytes,
                                r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "projection_loss_fwd";
  R2S_RETURN_IF(r2s::check_loss_args(n_images, H, W, what));
  r2s::Window win;
  R2S_RETURN_IF(r2s::make_window(window_size, win, what));
  R2S_REQUIRE(losses != nullptr, "%s: null losses", what);
  R2S_REQUIRE((edge_target == nullptr) == (edge_mask == nullptr),
              "%s: edge_target and edge_mask go together", what);
  const int64_t npix = n_images * H * W;
  R2S_REQUIRE(npix > 0, "%s: empty images (the reference's mean is NaN)", what);
  R2S_REQUIRE(render && target, "%s: null image", what);
  const int64_t need = r2s_projection_loss_workspace_bytes(n_images, H, W);
  if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
    r2s::set_error("%s: workspace of %zu bytes, %lld required", what, workspace_bytes,
                   (long long)need);
    return R2S_EWORKSPACE;
  }
  r2s::Carver cv(workspace);
  const r2s::LossSpace s = r2s::carve_loss(cv, n_images, H, W);
  const int tiles = static_cast<int>(r2s::ceil_div(H, r2s::kTile) * r2s::ceil_div(W, r2s::kTile));
  hipStream_t stream = r2s::as_stream(st);
  r2s::ssim_fwd_kernel<<<dim3(tiles, static_cast<uint32_t>(n_images)), dim3(r2s::kLossThreads), 0,
                         stream>>>(render, target, edge_target, edge_mask, H, W, win, s.A, s.B,
                                   s.C, s.partials);
  R2S_RETURN_IF(r2s::check_launch(what));
  r2s::loss_reduce_kernel<<<1, r2s::kLossThreads, 0, stream>>>(
      s.partials, n_images * tiles, 1.0 / static_cast<double>(npix), losses);
  return r2s::check_launch(what);
}

int r2s_projection_loss_bwd_f32(const float *render, const float *target,
                                const float *edge_target, const float *edge_mask,
                                int64_t n_images, int32_t H, int32_t W, int32_t window_size,
                                const float *grad_scales, const void *workspace,
                                size_t workspace_bytes, float *v_render, r2s_stream_t st) {
  r2s::clear_error();
  const char *what = "projection_loss_bwd";
  R2S_RETURN_IF(r2s::check_loss_args(n_images, H, W, what));
  r2s::Window win;
  R2S_RETURN_IF(r2s::make_window(window_size, win, what));
  R2S_REQUIRE((edge_target == nullptr) == (edge_mask == nullptr),
              "%s: edge_target and edge_mask go together", what);
  const int64_t npix = n_images * H * W;
  if (npix == 0) return R2S_OK;
  R2S_REQUIRE(render && target && grad_scales && v_render, "%s: null pointer", what);
  const int64_t need = r2s_projection_loss_workspace_bytes(n_images, H, W);
  if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
    r2s::set_error("%s: workspace of %zu bytes, %lld required", what, workspace_bytes,
                   (long long)need);
    return R2S_EWORKSPACE;
  }
  r2s::Carver cv(const_cast<void *>(workspace));
  const r2s::LossSpace s = r2s::carve_loss(cv, n_images, H, W);
  const int tiles = static_cast<int>(r2s::ceil_div(H, r2s::kTile) * r2s::ceil_div(W, r2s::kTile));
  r2s::ssim_bwd_kernel<<<dim3(tiles, static_cast<uint32_t>(n_images)), dim3(r2s::kLossThreads), 0,
                         r2s::as_stream(st)>>>(render, target, edge_target, edge_mask, s.A, s.B,
                                               s.C, H, W, win,
                                               static_cast<float>(1.0 / static_cast<double>(npix)),
                                               grad_scales, v_render);
  return r2s::check_launch(what);
}

}  // extern "C"
