/*
 * r2s_oracle.c -- sequential CPU restatement of the r2splat rasterizer and
 * voxelizer (forward and backward).  TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg through
 * oracle/native.py; never linked into the product library.
 *
 * Built with -O2 -ffp-contract=off so every float operation rounds exactly
 * as written.  Expressions follow the reference kernels term by term; the
 * fast __expf of the reference is replaced by libm exp, so alpha values agree
 * to within a few ulp and the 1e-5 / 1e-6 alpha cut-offs can flip only for
 * values within that distance of the threshold.
 *
 * Sums run in list order per pixel / voxel (the reference's per-thread
 * accumulation order).  Backward partials are accumulated per intersection
 * record over the tile's pixels in row-major order and then added to the
 * outputs in record order.
 */
#include <math.h>
#include <stdint.h>

/* Range [start, end) of tile `key` in a sorted list with lower_bound offsets;
 * the last key's range ends at n_isects (RasterizeToPixelsFwd.cu:100-105). */
static void tile_range(const int32_t *offsets, int64_t key, int64_t n_keys,
                       int64_t n_isects, int64_t *start, int64_t *end) {
  *start = offsets[key];
  *end = (key == n_keys - 1) ? n_isects : offsets[key + 1];
}

#define DEFINE_ORACLE(T, SUF, EXP, ABS)                                           \
  /* RasterizeToPixelsFwd.cu:57-186 */                                            \
  void orc_raster_fwd_##SUF(const T *means2d, const T *conics, const T *opac,     \
                            const T *mus, const int32_t *tile_offsets,            \
                            const int32_t *flatten_ids, int64_t n_isects,         \
                            int64_t C, uint32_t W, uint32_t H, uint32_t ts,       \
                            uint32_t tw, uint32_t th, T *out) {                   \
    const int64_t n_tiles = (int64_t)tw * th, n_keys = C * n_tiles;               \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      const int64_t c = key / n_tiles, t = key % n_tiles;                         \
      const uint32_t ty = (uint32_t)(t / tw), tx = (uint32_t)(t % tw);            \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (uint32_t ly = 0; ly < ts; ++ly)                                        \
        for (uint32_t lx = 0; lx < ts; ++lx) {                                    \
          const uint32_t i = ty * ts + ly, j = tx * ts + lx;                      \
          if (i >= H || j >= W) continue;                                         \
          const T px = (T)j + (T)0.5, py = (T)i + (T)0.5;                         \
          T acc = (T)0;                                                           \
          for (int64_t r = s; r < e; ++r) {                                       \
            const int64_t g = flatten_ids[r];                                     \
            const T dx = px - means2d[2 * g], dy = py - means2d[2 * g + 1];       \
            const T a = conics[3 * g], b = conics[3 * g + 1],                     \
                    cc = conics[3 * g + 2];                                       \
            const T sigma = (T)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;  \
            const T alpha = opac[g] * mus[g] * EXP(-sigma);                       \
            if (sigma < (T)0 || ABS(alpha) < (T)1e-5) continue;                   \
            acc += alpha;                                                         \
          }                                                                       \
          out[c * (int64_t)H * W + (int64_t)i * W + j] = acc;                     \
        }                                                                         \
    }                                                                             \
  }                                                                               \
                                                                                  \
  /* RasterizeToPixelsBwd.cu:350-480 (both modes compute the same sums) */        \
  void orc_raster_bwd_##SUF(                                                      \
      const T *means2d, const T *conics, const T *opac, const T *mus,             \
      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,  \
      const T *v_img, int64_t C, uint32_t W, uint32_t H, uint32_t ts,             \
      uint32_t tw, uint32_t th, T *v_xy_abs, T *v_xy, T *v_conic, T *v_opac,      \
      T *v_mu) {                                                                  \
    const int64_t n_tiles = (int64_t)tw * th, n_keys = C * n_tiles;               \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      const int64_t c = key / n_tiles, t = key % n_tiles;                         \
      const uint32_t ty = (uint32_t)(t / tw), tx = (uint32_t)(t % tw);            \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      const T *vimg = v_img + c * (int64_t)H * W;                                 \
      for (int64_t r = s; r < e; ++r) {                                           \
        const int64_t g = flatten_ids[r];                                         \
        const T mx = means2d[2 * g], my = means2d[2 * g + 1];                     \
        const T a = conics[3 * g], b = conics[3 * g + 1], cc = conics[3 * g + 2]; \
        const T o = opac[g], mu = mus[g];                                         \
        T ax = 0, ay = 0, aax = 0, aay = 0, ca = 0, cb = 0, cc2 = 0, ao = 0,      \
          am = 0;                                                                 \
        for (uint32_t ly = 0; ly < ts; ++ly)                                      \
          for (uint32_t lx = 0; lx < ts; ++lx) {                                  \
            const uint32_t i = ty * ts + ly, j = tx * ts + lx;                    \
            if (i >= H || j >= W) continue;                                       \
            const T dx = ((T)j + (T)0.5) - mx, dy = ((T)i + (T)0.5) - my;         \
            const T sigma = (T)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;  \
            const T vis = EXP(-sigma);                                            \
            const T alpha = o * mu * vis;                                         \
            if (sigma < (T)0 || ABS(alpha) < (T)1e-5) continue;                   \
            const T v = vimg[(int64_t)i * W + j];                                 \
            const T v_sigma = -v * alpha;                                         \
            const T gx = -v_sigma * (a * dx + b * dy);                            \
            const T gy = -v_sigma * (cc * dy + b * dx);                           \
            ax += gx;                                                             \
            ay += gy;                                                             \
            aax += ABS(gx);                                                       \
            aay += ABS(gy);                                                       \
            ca += v_sigma * (T)0.5 * dx * dx;                                     \
            cb += v_sigma * dx * dy;                                              \
            cc2 += v_sigma * (T)0.5 * dy * dy;                                    \
            ao += v * mu * vis;                                                   \
            am += v * o * vis;                                                    \
          }                                                                       \
        v_xy[2 * g] += ax;                                                        \
        v_xy[2 * g + 1] += ay;                                                    \
        if (v_xy_abs) {                                                           \
          v_xy_abs[2 * g] += aax;                                                 \
          v_xy_abs[2 * g + 1] += aay;                                             \
        }                                                                         \
        v_conic[3 * g] += ca;                                                     \
        v_conic[3 * g + 1] += cb;                                                 \
        v_conic[3 * g + 2] += cc2;                                                \
        v_opac[g] += ao;                                                          \
        v_mu[g] += am;                                                            \
      }                                                                           \
    }                                                                             \
  }                                                                               \
                                                                                  \
  /* VoxelizeToVoxelsFwd.cu:69-221 */                                             \
  void orc_voxel_fwd_##SUF(const T *means3d, const T *conics, const T *opac,      \
                           const int32_t *tile_offsets, const int32_t *flatten_ids,\
                           int64_t n_isects, uint32_t D2, uint32_t D1,            \
                           uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,    \
                           uint32_t n0, T *out) {                                 \
    const int64_t n_keys = (int64_t)n2 * n1 * n0;                                 \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      const uint32_t b0 = (uint32_t)(key / ((int64_t)n1 * n2));                   \
      const uint32_t b1 = (uint32_t)((key / n2) % n1);                            \
      const uint32_t b2 = (uint32_t)(key % n2);                                   \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (uint32_t li = 0; li < ts; ++li)                                        \
        for (uint32_t lj = 0; lj < ts; ++lj)                                      \
          for (uint32_t lk = 0; lk < ts; ++lk) {                                  \
            const uint32_t i = b0 * ts + li, j = b1 * ts + lj, k = b2 * ts + lk;  \
            if (i >= D0 || j >= D1 || k >= D2) continue;                          \
            const T px = (T)k + (T)0.5, py = (T)j + (T)0.5, pz = (T)i + (T)0.5;   \
            T acc = (T)0;                                                         \
            for (int64_t r = s; r < e; ++r) {                                     \
              const int64_t g = flatten_ids[r];                                   \
              const T dx = px - means3d[3 * g], dy = py - means3d[3 * g + 1],     \
                      dz = pz - means3d[3 * g + 2];                               \
              const T *q = conics + 6 * g;                                        \
              const T sigma =                                                     \
                  (T)0.5 * (q[0] * dx * dx + q[3] * dy * dy + q[5] * dz * dz) +   \
                  q[1] * dx * dy + q[2] * dx * dz + q[4] * dy * dz;               \
              const T alpha = opac[g] * EXP(-sigma);                              \
              if (sigma < (T)0 || ABS(alpha) < (T)1e-6) continue;                 \
              acc += alpha;                                                       \
            }                                                                     \
            out[(int64_t)i * D1 * D2 + (int64_t)j * D2 + k] = acc;                \
          }                                                                       \
    }                                                                             \
  }                                                                               \
                                                                                  \
  /* VoxelizeToVoxelsBwd.cu:322-441 (both modes compute the same sums) */         \
  void orc_voxel_bwd_##SUF(const T *means3d, const T *conics, const T *opac,      \
                           const int32_t *tile_offsets, const int32_t *flatten_ids,\
                           int64_t n_isects, const T *v_vol, uint32_t D2,         \
                           uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2,    \
                           uint32_t n1, uint32_t n0, T *v_means, T *v_conics,     \
                           T *v_opac) {                                           \
    const int64_t n_keys = (int64_t)n2 * n1 * n0;                                 \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      const uint32_t b0 = (uint32_t)(key / ((int64_t)n1 * n2));                   \
      const uint32_t b1 = (uint32_t)((key / n2) % n1);                            \
      const uint32_t b2 = (uint32_t)(key % n2);                                   \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r) {                                           \
        const int64_t g = flatten_ids[r];                                         \
        const T mx = means3d[3 * g], my = means3d[3 * g + 1],                     \
                mz = means3d[3 * g + 2];                                          \
        const T *q = conics + 6 * g;                                              \
        const T a = q[0], p = q[1], qq = q[2], bb = q[3], rr = q[4], cz = q[5];   \
        const T o = opac[g];                                                      \
        T gx = 0, gy = 0, gz = 0, g0 = 0, g1 = 0, g2 = 0, g3 = 0, g4 = 0, g5 = 0, \
          go = 0;                                                                 \
        for (uint32_t li = 0; li < ts; ++li)                                      \
          for (uint32_t lj = 0; lj < ts; ++lj)                                    \
            for (uint32_t lk = 0; lk < ts; ++lk) {                                \
              const uint32_t i = b0 * ts + li, j = b1 * ts + lj,                  \
                             k = b2 * ts + lk;                                    \
              if (i >= D0 || j >= D1 || k >= D2) continue;                        \
              const T d1 = ((T)k + (T)0.5) - mx, d2 = ((T)j + (T)0.5) - my,       \
                      d3 = ((T)i + (T)0.5) - mz;                                  \
              const T sigma = (T)0.5 * (a * d1 * d1 + bb * d2 * d2 + cz * d3 * d3) \
                              + p * d1 * d2 + qq * d1 * d3 + rr * d2 * d3;        \
              const T vis = EXP(-sigma);                                          \
              const T alpha = o * vis;                                            \
              if (sigma < (T)0 || ABS(alpha) < (T)1e-6) continue;                 \
              const T v = v_vol[(int64_t)i * D1 * D2 + (int64_t)j * D2 + k];      \
              const T v_sigma = -v * o * vis;                                     \
              const T oI = o * vis;                                               \
              go += v * vis;                                                      \
              g0 += v_sigma * (T)0.5 * d1 * d1;                                   \
              g1 += v_sigma * d1 * d2;                                            \
              g2 += v_sigma * d1 * d3;                                            \
              g3 += v_sigma * (T)0.5 * d2 * d2;                                   \
              g4 += v_sigma * d2 * d3;                                            \
              g5 += v_sigma * (T)0.5 * d3 * d3;                                   \
              gx += v * oI * (a * d1 + p * d2 + qq * d3);                         \
              gy += v * oI * (bb * d2 + p * d1 + rr * d3);                        \
              gz += v * oI * (cz * d3 + qq * d1 + rr * d2);                       \
            }                                                                     \
        v_means[3 * g] += gx;                                                     \
        v_means[3 * g + 1] += gy;                                                 \
        v_means[3 * g + 2] += gz;                                                 \
        v_conics[6 * g] += g0;                                                    \
        v_conics[6 * g + 1] += g1;                                                \
        v_conics[6 * g + 2] += g2;                                                \
        v_conics[6 * g + 3] += g3;                                                \
        v_conics[6 * g + 4] += g4;                                                \
        v_conics[6 * g + 5] += g5;                                                \
        v_opac[g] += go;                                                          \
      }                                                                           \
    }                                                                             \
  }

DEFINE_ORACLE(float, f32, expf, fabsf)
DEFINE_ORACLE(double, f64, exp, fabs)
