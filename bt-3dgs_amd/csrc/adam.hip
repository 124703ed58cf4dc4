// Adam step of the Gaussian parameter groups in one launch.
//
// The trainer steps one torch.optim.Adam per parameter group
// (src/models/gaussian_model.py:514-530, src/trainers/binary_tree.py:208-210);
// torch's multi-tensor Adam runs about ten element-wise kernels per
// optimizer.  Here one 2-D launch updates every (param, exp_avg, exp_avg_sq)
// triple: blockIdx.y picks the tensor, each thread four consecutive elements.
// The per-element arithmetic is torch's (torch/optim/adam.py
// _multi_tensor_adam, non-capturable): float32 with the step's scalars
// computed on the host in double and rounded to float, one rounding per
// torch kernel, and the same fused multiply-adds torch's element-wise
// kernels compile to:
//
//   g   = grad (+ weight_decay * param)
//   m   = lerp(m, g, 1 - beta1)
//   v   = v * beta2;  v = v + (1 - beta2) * (g * g)
//   d   = sqrt(v) / sqrt(1 - beta2^t) + eps
//   p   = p + step_size * (m / d),   step_size = -lr / (1 - beta1^t)
#include <algorithm>

#include "r2s_common.h"

namespace r2s {
namespace {

constexpr int kAdamThreads = 256;
constexpr int kAdamPerThread = 4;
constexpr int kAdamMaxTensors = 32;

struct AdamTable {
  r2s_adam_tensor_t t[kAdamMaxTensors];
};

// The roundings are spelled out (explicit FMAs, __fmul_rn / __fdiv_rn /
// __fadd_rn where torch's kernels round a product, quotient or sum on its
// own), so the compiler's contraction choices, which differ between the two
// load paths below, cannot change them.

// ATen's lerp: weight below one half from the start, else from the end.
__device__ __forceinline__ float lerp(float a, float b, float w) {
  const float d = b - a;
  return fabsf(w) < 0.5f ? fmaf(w, d, a) : fmaf(-d, 1.0f - w, b);
}

struct AdamScalars {
  float w1, b2, omb2, wd, bc2s, eps, ss;
};

__device__ __forceinline__ void adam_one(const AdamScalars &c, float &p, float g, float &m,
                                         float &v) {
  if (c.wd != 0.0f) g = fmaf(c.wd, p, g);  // grad.add(param, alpha=wd)
  m = lerp(m, g, c.w1);
  // mul_(beta2), then ATen's pointwise addcmul: self + value * (t1 * t2).
  v = fmaf(c.omb2, __fmul_rn(g, g), __fmul_rn(v, c.b2));
  const float den = __fadd_rn(__fdiv_rn(sqrtf(v), c.bc2s), c.eps);
  p = fmaf(c.ss, __fdiv_rn(m, den), p);  // addcdiv_: self + value * (t1 / t2)
}

// Each thread's four elements move as one 16-byte load or store per array
// when all four arrays are 16-byte aligned and the four are in range (the
// usual case); otherwise element by element.
__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamTable tab) {
  const r2s_adam_tensor_t &d = tab.t[blockIdx.y];
  const int64_t base =
      (static_cast<int64_t>(blockIdx.x) * kAdamThreads + threadIdx.x) * kAdamPerThread;
  if (base >= d.n) return;
  const AdamScalars c{d.lerp_weight, d.beta2, d.one_minus_beta2, d.weight_decay,
                      d.bias_correction2_sqrt, d.eps, d.step_size};
  const uintptr_t any = reinterpret_cast<uintptr_t>(d.param) |
                        reinterpret_cast<uintptr_t>(d.grad) |
                        reinterpret_cast<uintptr_t>(d.exp_avg) |
                        reinterpret_cast<uintptr_t>(d.exp_avg_sq);
  if (any % 16 == 0 && base + kAdamPerThread <= d.n) {
    static_assert(kAdamPerThread == 4, "one float4 per thread and array");
    float4 p = *reinterpret_cast<const float4 *>(d.param + base);
    const float4 g = *reinterpret_cast<const float4 *>(d.grad + base);
    float4 m = *reinterpret_cast<const float4 *>(d.exp_avg + base);
    float4 v = *reinterpret_cast<const float4 *>(d.exp_avg_sq + base);
    adam_one(c, p.x, g.x, m.x, v.x);
    adam_one(c, p.y, g.y, m.y, v.y);
    adam_one(c, p.z, g.z, m.z, v.z);
    adam_one(c, p.w, g.w, m.w, v.w);
    *reinterpret_cast<float4 *>(d.exp_avg + base) = m;
    *reinterpret_cast<float4 *>(d.exp_avg_sq + base) = v;
    *reinterpret_cast<float4 *>(d.param + base) = p;
    return;
  }
#pragma unroll
  for (int k = 0; k < kAdamPerThread; ++k) {
    const int64_t i = base + k;
    if (i >= d.n) break;
    float p = d.param[i], m = d.exp_avg[i], v = d.exp_avg_sq[i];
    adam_one(c, p, d.grad[i], m, v);
    d.exp_avg[i] = m;
    d.exp_avg_sq[i] = v;
    d.param[i] = p;
  }
}

}  // namespace
}  // namespace r2s

extern "C" {

int r2s_adam_step_f32(const r2s_adam_tensor_t *tensors, int32_t n_tensors, r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n_tensors >= 0 && (n_tensors == 0 || tensors != nullptr),
              "adam_step: bad tensor list");
  for (int32_t i = 0; i < n_tensors; ++i) {
    const r2s_adam_tensor_t &t = tensors[i];
    R2S_REQUIRE(t.n >= 0, "adam_step: tensor %d has a negative size", i);
    R2S_REQUIRE(t.n == 0 || (t.param && t.grad && t.exp_avg && t.exp_avg_sq),
                "adam_step: tensor %d has a null pointer", i);
  }
  hipStream_t stream = r2s::as_stream(st);
  constexpr int64_t per_block = r2s::kAdamThreads * r2s::kAdamPerThread;
  for (int32_t first = 0; first < n_tensors; first += r2s::kAdamMaxTensors) {
    const int32_t n = std::min<int32_t>(r2s::kAdamMaxTensors, n_tensors - first);
    r2s::AdamTable tab{};
    int64_t max_n = 0;
    for (int32_t i = 0; i < n; ++i) {
      tab.t[i] = tensors[first + i];
      max_n = std::max<int64_t>(max_n, tab.t[i].n);
    }
    if (max_n == 0) continue;
    const int64_t bx = r2s::ceil_div(max_n, per_block);
    R2S_REQUIRE(bx <= r2s::kInt32Max, "adam_step: tensor too large");
    r2s::adam_kernel<<<dim3(static_cast<uint32_t>(bx), static_cast<uint32_t>(n)),
                       dim3(r2s::kAdamThreads), 0, stream>>>(tab);
    R2S_RETURN_IF(r2s::check_launch("adam_step"));
  }
  return R2S_OK;
}

}  // extern "C"
