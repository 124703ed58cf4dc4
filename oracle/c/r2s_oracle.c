/*
 * r2s_oracle.c -- sequential CPU restatement of the r2splat rasterizer and
 * voxelizer (forward and backward).  TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg through
 * oracle/native.py; never linked into the product library.
 *
 * Built with -O2 -ffp-contract=off so every operation rounds as written.
 * Expressions follow the reference kernels term by term; the reference's fast
 * __expf is replaced by libm exp in the build's precision.  Three precisions
 * are built: float (f32, the reference's arithmetic), double (f64) and the
 * x86 80-bit long double (f80), which anchors the double-precision kernels
 * the way f64 anchors the float ones.
 *
 * Sums run in list order per pixel / voxel (the reference's per-thread
 * accumulation order).  Backward partials are accumulated per intersection
 * record over the tile's pixels in row-major order and then added to the
 * outputs in record order (RasterizeToPixelsBwd.cu:412-452,
 * VoxelizeToVoxelsBwd.cu:382-422).  With OpenMP the tiles are shared out
 * over threads: forward pixels belong to one tile each, and the backward's
 * per-record partials are computed in parallel into a scratch array and then
 * added to the outputs sequentially in record order, so every result is
 * bit-identical to the sequential loops.
 *
 * The alpha test is "skip if sigma < 0 or |alpha| < thr" with thr a run-time
 * argument (1e-5 in 2D, 1e-6 in 3D in the reference).  With a non-NULL
 * `band` output, every term whose decision a lower-precision evaluation
 * could flip -- |sigma - sigma*| <= eta (S + |sigma*| + 1), where sigma* =
 * ln(|w| / thr) is the exponent at the cut-off and S the sum of the absolute
 * values of sigma's terms, or |sigma| <= eta S at the sign test -- adds the
 * absolute value of its contribution to each output it feeds, whether it
 * passed here or not.  An output with band 0 has no term near a cut-off; a
 * kernel may differ from this oracle by a flip only up to the band.  A
 * non-NULL `mag` output receives, per output, the sum over the terms that
 * passed of |term| (1 + S): a precision-u evaluation of sigma errs by about
 * u S, which is the relative error of exp(-sigma) and so of the term, and
 * summing in another order errs by about u |term| more; any evaluation order
 * differs from the exact sum by a small multiple of u mag.
 *
 * The forward entry points take an optional list of tile / brick keys
 * (`keys`, `n_sel`; NULL for all keys) and then write only those tiles'
 * pixels; the *_records entry points return the per-record partials of the
 * listed tiles' records (the rows the two-pass backward kernels store), so
 * a sample of a list too long for the whole oracle can still be checked.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* Range [start, end) of tile `key` in a sorted list with lower_bound offsets;
 * the last key's range ends at n_isects (RasterizeToPixelsFwd.cu:100-105). */
static void tile_range(const int32_t *offsets, int64_t key, int64_t n_keys,
                       int64_t n_isects, int64_t *start, int64_t *end) {
  *start = offsets[key];
  *end = (key == n_keys - 1) ? n_isects : offsets[key + 1];
}

/* Per-record values: partials, then their flip bands, then their |terms|. */
#define R2D 9  /* v_xy_abs 2, v_xy 2, v_conic 3, v_opac, v_mu */
#define R3D 10 /* v_means 3, v_conics 6, v_opac */

#define DEFINE_ORACLE(T, SUF, EXP, ABS, LOG)                                          \
  /* 1 when the alpha decision of a term with exponent sigma, magnitude sum S     \
   * and weight w lies within the flip bracket. */                                \
  static int in_band_##SUF(T sigma, T S, T w, T thr, T eta) {                     \
    if (eta <= (T)0 || sigma != sigma || w != w) return 0;                        \
    if (ABS(sigma) <= eta * S && S > (T)0) return 1;                              \
    const T aw = ABS(w);                                                          \
    if (!(aw > (T)0)) return 0;                                                   \
    const T star = LOG(aw / thr);                                                 \
    return ABS(sigma - star) <= eta * (S + ABS(star) + (T)1);                     \
  }                                                                               \
                                                                                  \
  /* The pixels of 2D tile `key` (RasterizeToPixelsFwd.cu:57-186). */             \
  static void raster_tile_fwd_##SUF(                                              \
      const T *means2d, const T *conics, const T *opac, const T *mus,             \
      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,  \
      int64_t n_keys, int64_t key, uint32_t W, uint32_t H, uint32_t ts,           \
      uint32_t tw, uint32_t th, T thr, T eta, T *out, T *band, T *mag) {          \
    const int64_t n_tiles = (int64_t)tw * th;                                     \
    const int64_t c = key / n_tiles, t = key % n_tiles;                           \
    const uint32_t ty = (uint32_t)(t / tw), tx = (uint32_t)(t % tw);              \
    int64_t s, e;                                                                 \
    tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                      \
    for (uint32_t ly = 0; ly < ts; ++ly)                                          \
      for (uint32_t lx = 0; lx < ts; ++lx) {                                      \
        const uint32_t i = ty * ts + ly, j = tx * ts + lx;                        \
        if (i >= H || j >= W) continue;                                           \
        const T px = (T)j + (T)0.5, py = (T)i + (T)0.5;                           \
        T acc = (T)0, bnd = (T)0, mg = (T)0;                                      \
        for (int64_t r = s; r < e; ++r) {                                         \
          const int64_t g = flatten_ids[r];                                       \
          const T dx = px - means2d[2 * g], dy = py - means2d[2 * g + 1];         \
          const T a = conics[3 * g], b = conics[3 * g + 1], cc = conics[3 * g + 2]; \
          const T sigma = (T)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;    \
          const T alpha = opac[g] * mus[g] * EXP(-sigma);                         \
          const T S = (T)0.5 * (ABS(a) * dx * dx + ABS(cc) * dy * dy) +           \
                      ABS(b * dx * dy);                                           \
          if (band && in_band_##SUF(sigma, S, opac[g] * mus[g], thr, eta))        \
            bnd += ABS(alpha);                                                    \
          if (sigma < (T)0 || ABS(alpha) < thr) continue;                         \
          acc += alpha;                                                           \
          mg += ABS(alpha) * ((T)1 + S);                                          \
        }                                                                         \
        const int64_t o = c * (int64_t)H * W + (int64_t)i * W + j;                \
        out[o] = acc;                                                             \
        if (band) band[o] = bnd;                                                  \
        if (mag) mag[o] = mg;                                                     \
      }                                                                           \
  }                                                                               \
                                                                                  \
  /* One 2D record's partials over its tile (RasterizeToPixelsBwd.cu:350-480):   \
   * p[0..9) partials, p[9..18) their bands, p[18..27) their |terms|. */         \
  static void raster_record_##SUF(const T *means2d, const T *conics,              \
                                  const T *opac, const T *mus, int64_t g,         \
                                  const T *vimg, uint32_t W, uint32_t H,          \
                                  uint32_t ts, uint32_t tx, uint32_t ty, T thr,   \
                                  T eta, int want_band, T *p) {                   \
    const T mx = means2d[2 * g], my = means2d[2 * g + 1];                         \
    const T a = conics[3 * g], b = conics[3 * g + 1], cc = conics[3 * g + 2];     \
    const T o = opac[g], mu = mus[g];                                             \
    for (int k = 0; k < 3 * R2D; ++k) p[k] = (T)0;                                \
    for (uint32_t ly = 0; ly < ts; ++ly)                                          \
      for (uint32_t lx = 0; lx < ts; ++lx) {                                      \
        const uint32_t i = ty * ts + ly, j = tx * ts + lx;                        \
        if (i >= H || j >= W) continue;                                           \
        const T dx = ((T)j + (T)0.5) - mx, dy = ((T)i + (T)0.5) - my;             \
        const T sigma = (T)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;      \
        const T vis = EXP(-sigma);                                                \
        const T alpha = o * mu * vis;                                             \
        const T S = (T)0.5 * (ABS(a) * dx * dx + ABS(cc) * dy * dy) +             \
                    ABS(b * dx * dy);                                             \
        const int edge = want_band && in_band_##SUF(sigma, S, o * mu, thr, eta);  \
        const int pass = !(sigma < (T)0 || ABS(alpha) < thr);                     \
        if (!pass && !edge) continue;                                             \
        const T v = vimg[(int64_t)i * W + j];                                     \
        const T v_sigma = -v * alpha;                                             \
        const T gx = -v_sigma * (a * dx + b * dy);                                \
        const T gy = -v_sigma * (cc * dy + b * dx);                               \
        const T t[R2D] = {ABS(gx), ABS(gy), gx, gy,                               \
                          v_sigma * (T)0.5 * dx * dx, v_sigma * dx * dy,          \
                          v_sigma * (T)0.5 * dy * dy, v * mu * vis, v * o * vis}; \
        if (edge)                                                                 \
          for (int k = 0; k < R2D; ++k) p[R2D + k] += ABS(t[k]);                  \
        if (!pass) continue;                                                      \
        for (int k = 0; k < R2D; ++k) {                                           \
          p[k] += t[k];                                                           \
          p[2 * R2D + k] += ABS(t[k]) * ((T)1 + S);                               \
        }                                                                         \
      }                                                                           \
  }                                                                               \
                                                                                  \
  /* keys NULL: every tile; else the n_sel listed tiles' pixels only. */          \
  void orc_raster_fwd_##SUF(const T *means2d, const T *conics, const T *opac,     \
                            const T *mus, const int32_t *tile_offsets,            \
                            const int32_t *flatten_ids, int64_t n_isects,         \
                            int64_t C, uint32_t W, uint32_t H, uint32_t ts,       \
                            uint32_t tw, uint32_t th, const int64_t *keys,        \
                            int64_t n_sel, T thr, T eta, T *out, T *band,         \
                            T *mag) {                                             \
    const int64_t n_keys = C * (int64_t)tw * th;                                  \
    const int64_t n_run = keys ? n_sel : n_keys;                                  \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t q = 0; q < n_run; ++q)                                           \
      raster_tile_fwd_##SUF(means2d, conics, opac, mus, tile_offsets,             \
                            flatten_ids, n_isects, n_keys, keys ? keys[q] : q, W, \
                            H, ts, tw, th, thr, eta, out, band, mag);             \
  }                                                                               \
                                                                                  \
  /* Per-record values (raster_record) of the listed tiles' records: those of    \
   * keys[q] start at row first[q] of part[][3 * R2D].  Returns 0. */            \
  int orc_raster_records_##SUF(                                                   \
      const T *means2d, const T *conics, const T *opac, const T *mus,             \
      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,  \
      const T *v_img, int64_t C, uint32_t W, uint32_t H, uint32_t ts,             \
      uint32_t tw, uint32_t th, const int64_t *keys, int64_t n_sel,               \
      const int64_t *first, T thr, T eta, T *part) {                              \
    const int64_t n_tiles = (int64_t)tw * th, n_keys = C * n_tiles;               \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t q = 0; q < n_sel; ++q) {                                         \
      const int64_t key = keys[q];                                                \
      const int64_t c = key / n_tiles, t = key % n_tiles;                         \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r)                                             \
        raster_record_##SUF(means2d, conics, opac, mus, flatten_ids[r],           \
                            v_img + c * (int64_t)H * W, W, H, ts,                 \
                            (uint32_t)(t % tw), (uint32_t)(t / tw), thr, eta,     \
                            eta > (T)0, part + (first[q] + (r - s)) * 3 * R2D);   \
    }                                                                             \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* Both reference modes compute the same sums.  band / mag [C*N][R2D] or      \
   * NULL.  Returns 0, or -1 if the partials' scratch cannot be allocated. */    \
  int orc_raster_bwd_##SUF(                                                       \
      const T *means2d, const T *conics, const T *opac, const T *mus,             \
      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,  \
      const T *v_img, int64_t C, uint32_t W, uint32_t H, uint32_t ts,             \
      uint32_t tw, uint32_t th, T thr, T eta, T *v_xy_abs, T *v_xy, T *v_conic,   \
      T *v_opac, T *v_mu, T *band, T *mag) {                                      \
    const int64_t n_tiles = (int64_t)tw * th, n_keys = C * n_tiles;               \
    const int K = 3 * R2D;                                                        \
    T *part = (T *)malloc(sizeof(T) * (size_t)K * (size_t)(n_isects > 0 ? n_isects : 1)); \
    if (!part) return -1;                                                         \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      const int64_t c = key / n_tiles, t = key % n_tiles;                         \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r)                                             \
        raster_record_##SUF(means2d, conics, opac, mus, flatten_ids[r],           \
                            v_img + c * (int64_t)H * W, W, H, ts,                 \
                            (uint32_t)(t % tw), (uint32_t)(t / tw), thr, eta,     \
                            band != NULL, part + (size_t)K * (size_t)r);          \
    }                                                                             \
    /* Record order, as the sequential loops add them. */                         \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r) {                                           \
        const int64_t g = flatten_ids[r];                                         \
        const T *pr = part + (size_t)K * (size_t)r;                               \
        if (v_xy_abs) {                                                           \
          v_xy_abs[2 * g] += pr[0];                                               \
          v_xy_abs[2 * g + 1] += pr[1];                                           \
        }                                                                         \
        v_xy[2 * g] += pr[2];                                                     \
        v_xy[2 * g + 1] += pr[3];                                                 \
        v_conic[3 * g] += pr[4];                                                  \
        v_conic[3 * g + 1] += pr[5];                                              \
        v_conic[3 * g + 2] += pr[6];                                              \
        v_opac[g] += pr[7];                                                       \
        v_mu[g] += pr[8];                                                         \
        if (band)                                                                 \
          for (int k = 0; k < R2D; ++k) band[R2D * g + k] += pr[R2D + k];         \
        if (mag)                                                                  \
          for (int k = 0; k < R2D; ++k) mag[R2D * g + k] += pr[2 * R2D + k];      \
      }                                                                           \
    }                                                                             \
    free(part);                                                                   \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  /* The voxels of brick `key` (VoxelizeToVoxelsFwd.cu:69-221). */               \
  static void voxel_brick_fwd_##SUF(                                              \
      const T *means3d, const T *conics, const T *opac,                           \
      const int32_t *tile_offsets, const int32_t *flatten_ids, int64_t n_isects,  \
      int64_t n_keys, int64_t key, int64_t koff, uint32_t D2, uint32_t D1,        \
      uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, T thr, T eta, T *out,   \
      T *band, T *mag) {                                                          \
    const int64_t ak = key + koff; /* the brick's index in the whole grid */     \
    const uint32_t b0 = (uint32_t)(ak / ((int64_t)n1 * n2));                      \
    const uint32_t b1 = (uint32_t)((ak / n2) % n1);                               \
    const uint32_t b2 = (uint32_t)(ak % n2);                                      \
    int64_t s, e;                                                                 \
    tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                      \
    for (uint32_t li = 0; li < ts; ++li)                                          \
      for (uint32_t lj = 0; lj < ts; ++lj)                                        \
        for (uint32_t lk = 0; lk < ts; ++lk) {                                    \
          const uint32_t i = b0 * ts + li, j = b1 * ts + lj, k = b2 * ts + lk;    \
          if (i >= D0 || j >= D1 || k >= D2) continue;                            \
          const T px = (T)k + (T)0.5, py = (T)j + (T)0.5, pz = (T)i + (T)0.5;     \
          T acc = (T)0, bnd = (T)0, mg = (T)0;                                    \
          for (int64_t r = s; r < e; ++r) {                                       \
            const int64_t g = flatten_ids[r];                                     \
            const T dx = px - means3d[3 * g], dy = py - means3d[3 * g + 1],       \
                    dz = pz - means3d[3 * g + 2];                                 \
            const T *q = conics + 6 * g;                                          \
            const T sigma =                                                       \
                (T)0.5 * (q[0] * dx * dx + q[3] * dy * dy + q[5] * dz * dz) +     \
                q[1] * dx * dy + q[2] * dx * dz + q[4] * dy * dz;                 \
            const T alpha = opac[g] * EXP(-sigma);                                \
            const T S = (T)0.5 * (ABS(q[0]) * dx * dx + ABS(q[3]) * dy * dy +     \
                                  ABS(q[5]) * dz * dz) +                          \
                        ABS(q[1] * dx * dy) + ABS(q[2] * dx * dz) +               \
                        ABS(q[4] * dy * dz);                                      \
            if (band && in_band_##SUF(sigma, S, opac[g], thr, eta))               \
              bnd += ABS(alpha);                                                  \
            if (sigma < (T)0 || ABS(alpha) < thr) continue;                       \
            acc += alpha;                                                         \
            mg += ABS(alpha) * ((T)1 + S);                                        \
          }                                                                       \
          const int64_t o = (int64_t)i * D1 * D2 + (int64_t)j * D2 + k;           \
          out[o] = acc;                                                           \
          if (band) band[o] = bnd;                                                \
          if (mag) mag[o] = mg;                                                   \
        }                                                                         \
  }                                                                               \
                                                                                  \
  /* One 3D record's partials over its brick (VoxelizeToVoxelsBwd.cu:322-441):   \
   * p[0..10) partials, p[10..20) their bands, p[20..30) their |terms|. */       \
  static void voxel_record_##SUF(const T *means3d, const T *conics,               \
                                 const T *opac, int64_t g, const T *v_vol,        \
                                 uint32_t D2, uint32_t D1, uint32_t D0,           \
                                 uint32_t ts, uint32_t b0, uint32_t b1,           \
                                 uint32_t b2, T thr, T eta, int want_band, T *p) {\
    const T mx = means3d[3 * g], my = means3d[3 * g + 1], mz = means3d[3 * g + 2];\
    const T *q = conics + 6 * g;                                                  \
    const T a = q[0], pp = q[1], qq = q[2], bb = q[3], rr = q[4], cz = q[5];      \
    const T o = opac[g];                                                          \
    for (int m = 0; m < 3 * R3D; ++m) p[m] = (T)0;                                \
    for (uint32_t li = 0; li < ts; ++li)                                          \
      for (uint32_t lj = 0; lj < ts; ++lj)                                        \
        for (uint32_t lk = 0; lk < ts; ++lk) {                                    \
          const uint32_t i = b0 * ts + li, j = b1 * ts + lj, k = b2 * ts + lk;    \
          if (i >= D0 || j >= D1 || k >= D2) continue;                            \
          const T d1 = ((T)k + (T)0.5) - mx, d2 = ((T)j + (T)0.5) - my,           \
                  d3 = ((T)i + (T)0.5) - mz;                                      \
          const T sigma = (T)0.5 * (a * d1 * d1 + bb * d2 * d2 + cz * d3 * d3) +  \
                          pp * d1 * d2 + qq * d1 * d3 + rr * d2 * d3;             \
          const T vis = EXP(-sigma);                                              \
          const T alpha = o * vis;                                                \
          const T S = (T)0.5 * (ABS(a) * d1 * d1 + ABS(bb) * d2 * d2 +            \
                                ABS(cz) * d3 * d3) +                              \
                      ABS(pp * d1 * d2) + ABS(qq * d1 * d3) + ABS(rr * d2 * d3);  \
          const int edge = want_band && in_band_##SUF(sigma, S, o, thr, eta);     \
          const int pass = !(sigma < (T)0 || ABS(alpha) < thr);                   \
          if (!pass && !edge) continue;                                           \
          const T v = v_vol[(int64_t)i * D1 * D2 + (int64_t)j * D2 + k];          \
          const T v_sigma = -v * o * vis;                                         \
          const T oI = o * vis;                                                   \
          const T t[R3D] = {v * oI * (a * d1 + pp * d2 + qq * d3),                \
                            v * oI * (bb * d2 + pp * d1 + rr * d3),               \
                            v * oI * (cz * d3 + qq * d1 + rr * d2),               \
                            v_sigma * (T)0.5 * d1 * d1,                           \
                            v_sigma * d1 * d2,                                    \
                            v_sigma * d1 * d3,                                    \
                            v_sigma * (T)0.5 * d2 * d2,                           \
                            v_sigma * d2 * d3,                                    \
                            v_sigma * (T)0.5 * d3 * d3,                           \
                            v * vis};                                             \
          if (edge)                                                               \
            for (int m = 0; m < R3D; ++m) p[R3D + m] += ABS(t[m]);                \
          if (!pass) continue;                                                    \
          for (int m = 0; m < R3D; ++m) {                                         \
            p[m] += t[m];                                                         \
            p[2 * R3D + m] += ABS(t[m]) * ((T)1 + S);                             \
          }                                                                       \
        }                                                                         \
  }                                                                               \
                                                                                  \
  /* n0 brick layers of lists (tile_offsets [n0, n1, n2]) starting at brick     \
   * key koff of the whole volume's grid (0 unless the lists are one z-slab's). */ \
  void orc_voxel_fwd_##SUF(const T *means3d, const T *conics, const T *opac,      \
                           const int32_t *tile_offsets, const int32_t *flatten_ids,\
                           int64_t n_isects, uint32_t D2, uint32_t D1,            \
                           uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1,    \
                           uint32_t n0, int64_t koff, const int64_t *keys,        \
                           int64_t n_sel, T thr, T eta, T *out, T *band, T *mag) {\
    const int64_t n_keys = (int64_t)n2 * n1 * n0;                                 \
    const int64_t n_run = keys ? n_sel : n_keys;                                  \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t q = 0; q < n_run; ++q)                                           \
      voxel_brick_fwd_##SUF(means3d, conics, opac, tile_offsets, flatten_ids,     \
                            n_isects, n_keys, keys ? keys[q] : q, koff, D2, D1,   \
                            D0, ts, n2, n1, thr, eta, out, band, mag);            \
  }                                                                               \
                                                                                  \
  int orc_voxel_records_##SUF(const T *means3d, const T *conics, const T *opac,   \
                              const int32_t *tile_offsets,                        \
                              const int32_t *flatten_ids, int64_t n_isects,       \
                              const T *v_vol, uint32_t D2, uint32_t D1,           \
                              uint32_t D0, uint32_t ts, uint32_t n2, uint32_t n1, \
                              uint32_t n0, int64_t koff, const int64_t *keys,     \
                              int64_t n_sel, const int64_t *first, T thr, T eta,  \
                              T *part) {                                          \
    const int64_t n_keys = (int64_t)n2 * n1 * n0;                                 \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t q = 0; q < n_sel; ++q) {                                         \
      const int64_t key = keys[q], ak = key + koff;                               \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r)                                             \
        voxel_record_##SUF(means3d, conics, opac, flatten_ids[r], v_vol, D2, D1,  \
                           D0, ts, (uint32_t)(ak / ((int64_t)n1 * n2)),           \
                           (uint32_t)((ak / n2) % n1), (uint32_t)(ak % n2),       \
                           thr, eta, eta > (T)0,                                  \
                           part + (first[q] + (r - s)) * 3 * R3D);                \
    }                                                                             \
    return 0;                                                                     \
  }                                                                               \
                                                                                  \
  int orc_voxel_bwd_##SUF(const T *means3d, const T *conics, const T *opac,       \
                          const int32_t *tile_offsets, const int32_t *flatten_ids,\
                          int64_t n_isects, const T *v_vol, uint32_t D2,          \
                          uint32_t D1, uint32_t D0, uint32_t ts, uint32_t n2,     \
                          uint32_t n1, uint32_t n0, T thr, T eta, T *v_means,     \
                          T *v_conics, T *v_opac, T *band, T *mag) {              \
    const int64_t n_keys = (int64_t)n2 * n1 * n0;                                 \
    const int K = 3 * R3D;                                                        \
    T *part = (T *)malloc(sizeof(T) * (size_t)K * (size_t)(n_isects > 0 ? n_isects : 1)); \
    if (!part) return -1;                                                         \
    _Pragma("omp parallel for schedule(dynamic, 4)")                              \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r)                                             \
        voxel_record_##SUF(means3d, conics, opac, flatten_ids[r], v_vol, D2, D1,  \
                           D0, ts, (uint32_t)(key / ((int64_t)n1 * n2)),          \
                           (uint32_t)((key / n2) % n1), (uint32_t)(key % n2),     \
                           thr, eta, band != NULL, part + (size_t)K * (size_t)r); \
    }                                                                             \
    for (int64_t key = 0; key < n_keys; ++key) {                                  \
      int64_t s, e;                                                               \
      tile_range(tile_offsets, key, n_keys, n_isects, &s, &e);                    \
      for (int64_t r = s; r < e; ++r) {                                           \
        const int64_t g = flatten_ids[r];                                         \
        const T *pr = part + (size_t)K * (size_t)r;                               \
        for (int m = 0; m < 3; ++m) v_means[3 * g + m] += pr[m];                  \
        for (int m = 0; m < 6; ++m) v_conics[6 * g + m] += pr[3 + m];             \
        v_opac[g] += pr[9];                                                       \
        if (band)                                                                 \
          for (int m = 0; m < R3D; ++m) band[R3D * g + m] += pr[R3D + m];         \
        if (mag)                                                                  \
          for (int m = 0; m < R3D; ++m) mag[R3D * g + m] += pr[2 * R3D + m];      \
      }                                                                           \
    }                                                                             \
    free(part);                                                                   \
    return 0;                                                                     \
  }

DEFINE_ORACLE(float, f32, expf, fabsf, logf)
DEFINE_ORACLE(double, f64, exp, fabs, log)
DEFINE_ORACLE(long double, f80, expl, fabsl, logl)
