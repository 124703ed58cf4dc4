// Densify / prune of the binary-tree Gaussian table in one launch.
//
// The reference rebuilds every per-Gaussian array separately: an
// index_select / repeat / cat chain per parameter, per Adam moment, per tree
// buffer, per strategy statistic and per history archive
// (src/strategies/binary_tree.py:17-171, src/utils/ops.py:61-103), each a
// few small kernels.  Here every output row of every column is produced by
// one thread of a single 2-D launch: blockIdx.y picks the column, the thread
// index picks the destination row, and the row's source and class (kept,
// child +, child -, old, copy, archived) follow from the operation and the
// index lists of the compaction pass.  Each thread reads its source row
// once and writes its destination row once, so the launch streams the table
// at HBM rate; the index lists (8 B per row) stay in L2 / MALL across
// columns.
//
// Split children are computed in float32 in the reference's operation order
// (torch's elementwise kernels, one rounding per op): activated scales,
// first arg-max axis, normalised quaternion -> rotation column, the
// division by 1.6 done as a multiplication by the float reciprocal (torch's
// CUDA division by a host scalar), the clamp / logit inverse and the revised
// opacity.
#include "r2s_common.h"

namespace r2s {
namespace {

constexpr int kMaxCols = 32;
constexpr int kThreads = 256;

enum Op : int32_t { kSplit = 0, kDuplicate = 1, kRemove = 2 };
enum RowClass : int32_t { kKept = 0, kChildPlus = 1, kChildMinus = 2, kOld = 3, kNew = 4 };

struct Column {
  const uint32_t *src;
  uint32_t *dst;
  const uint32_t *extra;
  int64_t rows;
  int32_t width;
  int32_t role;
};

struct ColumnTable {
  Column c[kMaxCols];
};

struct Plan {
  int32_t op;
  int64_t n_in;          // rows of the live columns (duplicate)
  const int64_t *sel;
  int64_t n_sel;
  const int64_t *rest;   // rest (split) or keep (remove)
  int64_t n_rest;
  const uint8_t *mask;   // duplicate
  int64_t hist_rows;
};

struct Geometry {
  const float *quats;
  const float *raw_scales;
  float lo[3], hi[3], eps;
  int32_t sigmoid;
};

__device__ __forceinline__ void copy_row(uint32_t *__restrict__ d, const uint32_t *__restrict__ s,
                                         int w) {
  for (int k = 0; k < w; ++k) d[k] = s[k];
}

__device__ __forceinline__ void zero_row(uint32_t *__restrict__ d, int w) {
  for (int k = 0; k < w; ++k) d[k] = 0u;
}

// torch.clamp / clamp_min / clamp_max: NaN propagates.
__device__ __forceinline__ float t_clamp_min(float x, float lo) {
  return __builtin_isnan(x) ? x : (x < lo ? lo : x);
}
__device__ __forceinline__ float t_clamp_max(float x, float hi) {
  return __builtin_isnan(x) ? x : (x > hi ? hi : x);
}
__device__ __forceinline__ float t_clamp(float x, float lo, float hi) {
  return t_clamp_max(t_clamp_min(x, lo), hi);
}

// torch.argmax: first maximum; NaN counts as the largest value.
__device__ __forceinline__ bool arg_greater(float a, float b) {
  return a > b || (__builtin_isnan(a) && !__builtin_isnan(b));
}

#pragma clang fp contract(off)

__device__ __forceinline__ void activated_scales(const Geometry &g, int64_t s, float sc[3]) {
  // gaussian_model.py:258-264: lower + (upper - lower) * sigmoid(raw), or exp(raw).
  const float *r = g.raw_scales + 3 * s;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float x = r[k];
    if (g.sigmoid) {
      const float sig = 1.0f / (1.0f + expf(-x));
      const float span = g.hi[k] - g.lo[k];
      sc[k] = g.lo[k] + span * sig;
    } else {
      sc[k] = expf(x);
    }
  }
}

__device__ __forceinline__ int longest_axis(const float sc[3]) {
  int l = 0;
  if (arg_greater(sc[1], sc[l])) l = 1;
  if (arg_greater(sc[2], sc[l])) l = 2;
  return l;
}

// binary_tree.py:103-112: offset_world = R(normalize(q)) @ (s * e_longest).
// Only column `l` of R contributes; the other products are exact zeros.
__device__ __forceinline__ void child_offset(const Geometry &g, int64_t s, float off[3]) {
  float sc[3];
  activated_scales(g, s, sc);
  const int l = longest_axis(sc);
  const float *q = g.quats + 4 * s;
  // F.normalize: q / max(||q||, 1e-12)
  const float nrm = sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
  const float den = t_clamp_min(nrm, 1e-12f);
  const float w = q[0] / den, x = q[1] / den, y = q[2] / den, z = q[3] / den;
  float c0, c1, c2;  // column l of normalized_quat_to_rotmat (src/utils/math.py:35-53)
  if (l == 0) {
    c0 = 1.0f - 2.0f * (y * y + z * z);
    c1 = 2.0f * (x * y + w * z);
    c2 = 2.0f * (x * z - w * y);
  } else if (l == 1) {
    c0 = 2.0f * (x * y - w * z);
    c1 = 1.0f - 2.0f * (x * x + z * z);
    c2 = 2.0f * (y * z + w * x);
  } else {
    c0 = 2.0f * (x * z + w * y);
    c1 = 2.0f * (y * z - w * x);
    c2 = 1.0f - 2.0f * (x * x + y * y);
  }
  const float sl = sc[l];
  off[0] = c0 * sl;
  off[1] = c1 * sl;
  off[2] = c2 * sl;
}

// binary_tree.py:127-131 + gaussian_model.py:266-274.
__device__ __forceinline__ void child_raw_scales(const Geometry &g, int64_t s, float out[3]) {
  float sc[3];
  activated_scales(g, s, sc);
  const int l = longest_axis(sc);
  const float inv = 1.0f / 1.6f;
  sc[l] = t_clamp_min(sc[l] * inv, 1e-12f);
  const float lo_clip = 1e-6f, hi_clip = static_cast<float>(1.0 - 1e-6);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (g.sigmoid) {
      const float cmin = g.lo[k] + g.eps, cmax = g.hi[k] - g.eps;
      const float c = t_clamp(sc[k], cmin, cmax);
      float sig = (c - g.lo[k]) / (g.hi[k] - g.lo[k]);
      sig = t_clamp(sig, lo_clip, hi_clip);
      out[k] = logf(sig / (1.0f - sig));
    } else {
      out[k] = logf(t_clamp_min(sc[k], 1e-12f));
    }
  }
}

// binary_tree.py:132-135: log(expm1(1 - sqrt(1 - min(softplus(o), 0.9999)))).
__device__ __forceinline__ float child_raw_opacity(float o) {
  const float sp = (o > 20.0f) ? o : log1pf(expf(o));  // F.softplus, beta 1, threshold 20
  const float base = t_clamp_max(sp, 0.9999f);
  const float fresh = 1.0f - sqrtf(1.0f - base);
  return logf(expm1f(fresh));
}

#pragma clang fp contract(on)

__global__ __launch_bounds__(kThreads) void densify_kernel(Plan p, Geometry g, ColumnTable tab) {
  const Column c = tab.c[blockIdx.y];
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (o >= c.rows) return;
  const int w = c.width;
  uint32_t *dst = c.dst + o * w;

  if (c.role == R2S_COL_HISTORY) {
    if (o < p.hist_rows)
      copy_row(dst, c.src + o * w, w);
    else
      copy_row(dst, c.extra + p.sel[o - p.hist_rows] * w, w);
    return;
  }

  int64_t s, j = 0;
  int32_t cls;
  if (p.op == kRemove) {
    s = p.rest[o];
    cls = kKept;
  } else if (p.op == kSplit) {
    if (o < p.n_rest) {
      s = p.rest[o];
      cls = kKept;
    } else {
      j = o - p.n_rest;
      cls = kChildPlus;
      if (j >= p.n_sel) {
        j -= p.n_sel;
        cls = kChildMinus;
      }
      s = p.sel[j];
    }
  } else {
    if (o < p.n_in) {
      s = o;
      cls = kOld;
    } else {
      j = o - p.n_in;
      s = p.sel[j];
      cls = kNew;
    }
  }
  const bool child = (cls == kChildPlus || cls == kChildMinus);
  const uint32_t *src = c.src + s * w;

  switch (c.role) {
    case R2S_COL_ZERO_NEW:
      if (child || cls == kNew)
        zero_row(dst, w);
      else
        copy_row(dst, src, w);
      return;
    case R2S_COL_MEANS:
      if (child) {
        float off[3];
        child_offset(g, s, off);
        const float *m = reinterpret_cast<const float *>(src);
        float *d = reinterpret_cast<float *>(dst);
#pragma unroll
        for (int k = 0; k < 3; ++k) d[k] = (cls == kChildPlus) ? m[k] + off[k] : m[k] + (-off[k]);
      } else {
        copy_row(dst, src, w);
      }
      return;
    case R2S_COL_RAW_SCALES:
      if (child) {
        float r[3];
        child_raw_scales(g, s, r);
        float *d = reinterpret_cast<float *>(dst);
#pragma unroll
        for (int k = 0; k < 3; ++k) d[k] = r[k];
      } else {
        copy_row(dst, src, w);
      }
      return;
    case R2S_COL_RAW_OPACITIES:
      if (child)
        *reinterpret_cast<float *>(dst) = child_raw_opacity(*reinterpret_cast<const float *>(src));
      else
        copy_row(dst, src, w);
      return;
    case R2S_COL_PARENT:
    case R2S_COL_LEVEL: {
      const bool parent = c.role == R2S_COL_PARENT;
      if (child || cls == kNew) {
        const int32_t v = parent ? static_cast<int32_t>(p.hist_rows + j)
                                 : *reinterpret_cast<const int32_t *>(src) + 1;
        *reinterpret_cast<int32_t *>(dst) = v;
        // duplicate: the selected original row is updated the same way.
        if (cls == kNew) *reinterpret_cast<int32_t *>(c.dst + s) = v;
      } else if (!(cls == kOld && p.mask[o] != 0)) {
        *dst = *src;
      }
      return;
    }
    default:  // R2S_COL_COPY
      copy_row(dst, src, w);
      return;
  }
}

int check_columns(const Plan &p, const r2s_column_t *cols, int32_t n_cols, int64_t main_rows,
                  bool geometry, const char *what) {
  R2S_REQUIRE(n_cols >= 0 && (n_cols == 0 || cols != nullptr), "%s: bad column list", what);
  for (int32_t i = 0; i < n_cols; ++i) {
    const r2s_column_t &c = cols[i];
    R2S_REQUIRE(c.width >= 1 && c.width <= R2S_DENSIFY_MAX_WIDTH,
                "%s: column %d width %d outside [1, %d]", what, i, c.width,
                R2S_DENSIFY_MAX_WIDTH);
    R2S_REQUIRE(c.role >= R2S_COL_COPY && c.role <= R2S_COL_HISTORY, "%s: column %d role %d",
                what, i, c.role);
    const bool hist = c.role == R2S_COL_HISTORY;
    R2S_REQUIRE(!(hist && p.op == kRemove), "%s: column %d: remove takes no history column",
                what, i);
    const bool split_only = c.role == R2S_COL_MEANS || c.role == R2S_COL_RAW_SCALES ||
                            c.role == R2S_COL_RAW_OPACITIES;
    if (split_only && p.op == kSplit) {
      const int need = c.role == R2S_COL_RAW_OPACITIES ? 1 : 3;
      R2S_REQUIRE(c.width == need, "%s: column %d (role %d) needs width %d, got %d", what, i,
                  c.role, need, c.width);
      R2S_REQUIRE(c.role == R2S_COL_RAW_OPACITIES || geometry,
                  "%s: column %d needs the split geometry", what, i);
    }
    if (c.role == R2S_COL_PARENT || c.role == R2S_COL_LEVEL)
      R2S_REQUIRE(c.width == 1, "%s: column %d (parent/level) needs width 1", what, i);
    const int64_t want = hist ? p.hist_rows + p.n_sel : main_rows;
    R2S_REQUIRE(c.rows == want, "%s: column %d has %lld rows, the operation writes %lld", what, i,
                (long long)c.rows, (long long)want);
    R2S_REQUIRE(want == 0 || c.dst != nullptr, "%s: column %d: null destination", what, i);
    const bool reads_src = hist ? p.hist_rows > 0 : want > 0;
    R2S_REQUIRE(!reads_src || c.src != nullptr, "%s: column %d: null source", what, i);
    R2S_REQUIRE(!hist || p.n_sel == 0 || c.extra != nullptr,
                "%s: column %d: history column without its live column", what, i);
  }
  return R2S_OK;
}

int launch(const Plan &p, const Geometry &g, const r2s_column_t *cols, int32_t n_cols,
           hipStream_t stream, const char *what) {
  for (int32_t first = 0; first < n_cols; first += kMaxCols) {
    const int32_t n = (n_cols - first < kMaxCols) ? n_cols - first : kMaxCols;
    ColumnTable tab{};
    int64_t max_rows = 0;
    for (int32_t i = 0; i < n; ++i) {
      const r2s_column_t &c = cols[first + i];
      tab.c[i] = Column{static_cast<const uint32_t *>(c.src), static_cast<uint32_t *>(c.dst),
                        static_cast<const uint32_t *>(c.extra), c.rows, c.width, c.role};
      max_rows = c.rows > max_rows ? c.rows : max_rows;
    }
    if (max_rows == 0) continue;
    const int64_t bx = ceil_div(max_rows, kThreads);
    R2S_REQUIRE(bx <= kInt32Max, "%s: too many rows", what);
    densify_kernel<<<dim3(static_cast<uint32_t>(bx), static_cast<uint32_t>(n)), dim3(kThreads), 0,
                     stream>>>(p, g, tab);
    R2S_RETURN_IF(check_launch(what));
  }
  return R2S_OK;
}

}  // namespace
}  // namespace r2s

extern "C" {

int r2s_densify_split(const int64_t *sel, int64_t n_sel, const int64_t *rest, int64_t n_rest,
                      int64_t history_rows, const r2s_split_geometry_t *geometry,
                      const r2s_column_t *columns, int32_t n_columns, r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n_sel >= 0 && n_rest >= 0 && history_rows >= 0, "densify_split: negative size");
  R2S_REQUIRE(n_sel == 0 || sel, "densify_split: null sel");
  R2S_REQUIRE(n_rest == 0 || rest, "densify_split: null rest");
  if (history_rows + n_sel > r2s::kInt32Max) {
    r2s::set_error("densify_split: history index %lld exceeds int32",
                   (long long)(history_rows + n_sel));
    return R2S_ERANGE;
  }
  r2s::Plan p{r2s::kSplit, n_rest + n_sel, sel, n_sel, rest, n_rest, nullptr, history_rows};
  r2s::Geometry g{};
  if (geometry) {
    R2S_REQUIRE(n_sel == 0 || (geometry->quats && geometry->raw_scales),
                "densify_split: geometry without quats / raw_scales");
    g.quats = geometry->quats;
    g.raw_scales = geometry->raw_scales;
    for (int k = 0; k < 3; ++k) {
      g.lo[k] = geometry->scale_min[k];
      g.hi[k] = geometry->scale_max[k];
    }
    g.eps = geometry->scale_eps;
    g.sigmoid = geometry->sigmoid_scales;
  }
  R2S_RETURN_IF(r2s::check_columns(p, columns, n_columns, n_rest + 2 * n_sel, geometry != nullptr,
                                   "densify_split"));
  return r2s::launch(p, g, columns, n_columns, r2s::as_stream(st), "densify_split");
}

int r2s_densify_duplicate(const uint8_t *mask, int64_t n, const int64_t *sel, int64_t n_sel,
                          int64_t history_rows, const r2s_column_t *columns, int32_t n_columns,
                          r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n >= 0 && n_sel >= 0 && n_sel <= n && history_rows >= 0,
              "densify_duplicate: bad sizes");
  R2S_REQUIRE(n == 0 || mask, "densify_duplicate: null mask");
  R2S_REQUIRE(n_sel == 0 || sel, "densify_duplicate: null sel");
  if (history_rows + n_sel > r2s::kInt32Max) {
    r2s::set_error("densify_duplicate: history index %lld exceeds int32",
                   (long long)(history_rows + n_sel));
    return R2S_ERANGE;
  }
  r2s::Plan p{r2s::kDuplicate, n, sel, n_sel, nullptr, 0, mask, history_rows};
  R2S_RETURN_IF(r2s::check_columns(p, columns, n_columns, n + n_sel, false, "densify_duplicate"));
  return r2s::launch(p, r2s::Geometry{}, columns, n_columns, r2s::as_stream(st),
                     "densify_duplicate");
}

int r2s_densify_remove(const int64_t *keep, int64_t n_keep, const r2s_column_t *columns,
                       int32_t n_columns, r2s_stream_t st) {
  r2s::clear_error();
  R2S_REQUIRE(n_keep >= 0, "densify_remove: negative size");
  R2S_REQUIRE(n_keep == 0 || keep, "densify_remove: null keep");
  r2s::Plan p{r2s::kRemove, 0, nullptr, 0, keep, n_keep, nullptr, 0};
  R2S_RETURN_IF(r2s::check_columns(p, columns, n_columns, n_keep, false, "densify_remove"));
  return r2s::launch(p, r2s::Geometry{}, columns, n_columns, r2s::as_stream(st),
                     "densify_remove");
}

}  // extern "C"
