// Densify / prune index compaction: torch.where(mask)[0] followed by
// torch.where(~mask)[0] in one output array (the `sel` / `rest` / `keep`
// index lists of src/strategies/binary_tree.py:68,101-102,158).
//
// Three passes over 4096-entry tiles (4 waves x 16 rounds of 64 entries):
//   count    per round one ballot; popcounts give each tile's true count.
//   scan     exclusive scan of the tile counts (device scan).
//   scatter  per round the ballot again; a lane's rank among the trues of
//            its round is mbcnt(ballot), the round/wave/tile prefixes come
//            from scalar popcounts and the tile scan.  A false entry at
//            index i goes to n_true + (i - trues before i).
// Ascending order within each list is inherent; no atomics are used.
#include "r2s_common.h"
#include "r2s_scan.h"

namespace r2s {
namespace {

constexpr int kRounds = 16;
constexpr int kWaveSpan = 64 * kRounds;  // 1024
constexpr int kTile = 4 * kWaveSpan;     // 4096 entries per block

__global__ __launch_bounds__(256) void mask_count_kernel(const uint8_t *__restrict__ mask,
                                                         int64_t n,
                                                         uint32_t *__restrict__ tile_counts) {
  __shared__ uint32_t wsum[4];
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kTile + w * kWaveSpan;
  uint32_t c = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    const bool m = (i < n) && mask[i] != 0;
    c += static_cast<uint32_t>(__popcll(ballot(m)));
  }
  if (lane == 0) wsum[w] = c;
  __syncthreads();
  if (threadIdx.x == 0) tile_counts[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

__global__ __launch_bounds__(256) void mask_scatter_kernel(const uint8_t *__restrict__ mask,
                                                           int64_t n,
                                                           const int64_t *__restrict__ tile_base,
                                                           const int64_t *__restrict__ n_true_p,
                                                           int64_t *__restrict__ out) {
  __shared__ uint32_t wsum[4];
  const uint32_t w = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kTile + w * kWaveSpan;
  uint64_t bal[kRounds];
  uint32_t c = 0;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    const bool m = (i < n) && mask[i] != 0;
    bal[r] = ballot(m);
    c += static_cast<uint32_t>(__popcll(bal[r]));
  }
  if (lane == 0) wsum[w] = c;
  __syncthreads();
  uint32_t wave_off = 0;
  for (uint32_t k = 0; k < w; ++k) wave_off += wsum[k];
  const int64_t n_true = *n_true_p;
  int64_t trues_before = tile_base[blockIdx.x] + wave_off;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int64_t i = first + r * 64 + lane;
    if (i < n) {
      const int64_t t = trues_before + mbcnt(bal[r]);
      const bool m = (bal[r] >> lane) & 1ull;
      if (m)
        out[t] = i;
      else
        out[n_true + (i - t)] = i;
    }
    trues_before += __popcll(bal[r]);
  }
}

struct MaskSpace {
  uint32_t *counts;
  int64_t *base;
  int64_t *partials;
  int64_t ntiles;
};

MaskSpace carve_mask(Carver &cv, int64_t n) {
  MaskSpace s;
  s.ntiles = ceil_div(n, kTile);
  s.counts = cv.take<uint32_t>(s.ntiles);
  s.base = cv.take<int64_t>(s.ntiles);
  s.partials = cv.take<int64_t>(scan_partials_count(s.ntiles));
  return s;
}

}  // namespace
}  // namespace r2s

extern "C" {

int64_t r2s_mask_workspace_bytes(int64_t n) {
  r2s::Carver cv(nullptr);
  r2s::carve_mask(cv, n > 0 ? n : 0);
  return static_cast<int64_t>(cv.used);
}

int r2s_mask_split(const uint8_t *mask, int64_t n, int64_t *out, int64_t *n_true_dev, void *ws,
                   size_t ws_bytes, r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n >= 0, "mask_split: negative size");
  R2S_REQUIRE(n_true_dev != nullptr, "mask_split: null count");
  hipStream_t stream = r2s::as_stream(st);
  if (n == 0) return r2s::device_fill<int64_t>(n_true_dev, 1, 0, stream, "mask_split");
  R2S_REQUIRE(mask && out, "mask_split: null pointer");
  const int64_t need = r2s_mask_workspace_bytes(n);
  if (ws == nullptr || static_cast<int64_t>(ws_bytes) < need) {
    r2s::set_error("mask_split: workspace of %zu bytes, %lld required", ws_bytes, (long long)need);
    return R2S_EWORKSPACE;
  }
  r2s::Carver cv(ws);
  r2s::MaskSpace s = r2s::carve_mask(cv, n);
  const uint32_t nb = static_cast<uint32_t>(s.ntiles);
  r2s::mask_count_kernel<<<dim3(nb), dim3(256), 0, stream>>>(mask, n, s.counts);
  R2S_RETURN_IF(r2s::check_launch("mask_split count"));
  R2S_RETURN_IF((r2s::device_exclusive_scan<uint32_t, int64_t>(s.counts, s.ntiles, s.base,
                                                               n_true_dev, s.partials, stream,
                                                               "mask_split scan")));
  r2s::mask_scatter_kernel<<<dim3(nb), dim3(256), 0, stream>>>(mask, n, s.base, n_true_dev, out);
  return r2s::check_launch("mask_split scatter");
}

}  // extern "C"
