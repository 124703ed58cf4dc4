/*
 * r2splat_hip.h -- C ABI of the MI355X (gfx950) Gaussian backend.
 *
 * Every entry point takes device pointers that the caller owns, plain sizes
 * and scalars, and a hipStream_t passed as `void*`.  Work is enqueued on that
 * stream; nothing here allocates or frees device memory: scratch space is a
 * caller-provided workspace whose size is returned by the *_workspace_bytes
 * queries (r2s_rasterize_fwd_noalloc_* instead uses a fixed device array that
 * the library holds on each GPU until the process ends).  Every function
 * returns R2S_OK (0) on success, otherwise a status code; r2s_last_error()
 * then holds a message for the calling thread.
 *
 * Layouts follow the reference operators (row-major, contiguous):
 *   covariances are packed upper-triangular (00, 01, 02, 11, 12, 22);
 *   quaternions are (w, x, y, z); images are [C, H, W]; volumes are
 *   [dim0, dim1, dim2] with x <-> dim2 fastest.
 *
 * The comment above each declaration names the reference interface it
 * replaces (paths relative to the BT-3DGS source tree).
 */
#ifndef R2SPLAT_HIP_H
#define R2SPLAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *r2s_stream_t; /* hipStream_t */

#define R2S_OK 0
#define R2S_EINVAL 1001    /* invalid argument (shape, size, pointer)      */
#define R2S_ERANGE 1002    /* size exceeds the int32 index limits          */
#define R2S_EHIP 1003      /* HIP runtime / launch error                    */
#define R2S_EWORKSPACE 1004 /* workspace smaller than the queried size      */

/* Message describing the last failure on the calling thread ("" if none). */
const char *r2s_last_error(void);
/* ABI revision of this header; bumped whenever a signature changes or an
 * entry is added. */
int r2s_abi_version(void);

/* ---------------------------------------------------------------------- */
/* Parameter transform                                                    */
/* ---------------------------------------------------------------------- */

/* r2splat/cuda/csrc/ParameterTransform.cpp:34-84 parameter_transform_fwd_tensor:
 * quats [n,4], raw_scales [n,3] -> covars [n,6], max_scales [n]. */
int r2s_parameter_transform_fwd_f32(const float *quats, const float *raw_scales,
                                    double scale_min, double scale_max,
                                    float *covars, float *max_scales,
                                    int64_t n, r2s_stream_t stream);
int r2s_parameter_transform_fwd_f64(const double *quats, const double *raw_scales,
                                    double scale_min, double scale_max,
                                    double *covars, double *max_scales,
                                    int64_t n, r2s_stream_t stream);

/* ParameterTransform.cpp:90-144 parameter_transform_bwd_tensor:
 * v_covars [n,6] -> v_quats [n,4], v_raw_scales [n,3]. */
int r2s_parameter_transform_bwd_f32(const float *quats, const float *raw_scales,
                                    double scale_min, double scale_max,
                                    const float *v_covars, float *v_quats,
                                    float *v_raw_scales, int64_t n,
                                    r2s_stream_t stream);
int r2s_parameter_transform_bwd_f64(const double *quats, const double *raw_scales,
                                    double scale_min, double scale_max,
                                    const double *v_covars, double *v_quats,
                                    double *v_raw_scales, int64_t n,
                                    r2s_stream_t stream);

/* r2splat/ops/direct.py:72-96 _prepare_forward_parameters, fused:
 * parameter_transform_fwd plus softplus(raw_opacities) -> opacities [n]. */
int r2s_prepare_gaussians_f32(const float *quats, const float *raw_scales,
                              const float *raw_opacities, double scale_min,
                              double scale_max, float *covars, float *max_scales,
                              float *opacities, int64_t n, r2s_stream_t stream);
int r2s_prepare_gaussians_f64(const double *quats, const double *raw_scales,
                              const double *raw_opacities, double scale_min,
                              double scale_max, double *covars, double *max_scales,
                              double *opacities, int64_t n, r2s_stream_t stream);

/* r2splat/ops/explicit.py:379 v_raw_opacities = v_opacity * sigmoid(raw),
 * with v_opacity = sum over cameras of v_opac_cn [C,n] plus optional
 * v_opac_3d [n] (explicit.py:319,370).  Either input may be NULL. */
int r2s_opacity_bwd_f32(const float *raw_opacities, const float *v_opac_cn,
                        const float *v_opac_3d, float *v_raw_opacities,
                        int64_t C, int64_t n, r2s_stream_t stream);
int r2s_opacity_bwd_f64(const double *raw_opacities, const double *v_opac_cn,
                        const double *v_opac_3d, double *v_raw_opacities,
                        int64_t C, int64_t n, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Cone-beam projection                                                   */
/* ---------------------------------------------------------------------- */

/* r2splat/cuda/csrc/WorldToImageProjection.cpp:38-119
 * world_to_image_projection_fwd_tensor: means [N,3], covars [N,6],
 * viewmats [C,4,4], Ks [C,3,3] -> means2d [C,N,2], cov2d [C,N,6],
 * radii [C,N,2] (int32).  `eps2d` and `radius_clip` are single precision in
 * the reference signature and are rounded to float before use. */
int r2s_world_to_image_projection_fwd_f32(
    const float *means, const float *covars, const float *viewmats,
    const float *Ks, uint32_t width, uint32_t height, float eps2d,
    float radius_clip, float *means2d, float *cov2d, int32_t *radii,
    int64_t C, int64_t N, r2s_stream_t stream);
int r2s_world_to_image_projection_fwd_f64(
    const double *means, const double *covars, const double *viewmats,
    const double *Ks, uint32_t width, uint32_t height, float eps2d,
    float radius_clip, double *means2d, double *cov2d, int32_t *radii,
    int64_t C, int64_t N, r2s_stream_t stream);

/* WorldToImageProjection.cpp:127-206 world_to_image_projection_bwd_tensor:
 * v_means2d [C,N,2], v_cov2d [C,N,6] -> v_means [N,3], v_covars [N,6]
 * (summed over cameras; fully written, no zero-init needed). */
int r2s_world_to_image_projection_bwd_f32(
    const float *means, const float *covars, const float *viewmats,
    const float *Ks, uint32_t width, uint32_t height, const float *v_means2d,
    const float *v_cov2d, float *v_means, float *v_covars, int64_t C,
    int64_t N, r2s_stream_t stream);
int r2s_world_to_image_projection_bwd_f64(
    const double *means, const double *covars, const double *viewmats,
    const double *Ks, uint32_t width, uint32_t height, const double *v_means2d,
    const double *v_cov2d, double *v_means, double *v_covars, int64_t C,
    int64_t N, r2s_stream_t stream);

/* r2splat/cuda/csrc/ConicsMu.cpp:35-80 conics_mu_fwd_tensor:
 * cov2d [total,6] -> conics [total,3], mus [total]. */
int r2s_conics_mu_fwd_f32(const float *cov2d, double eps, float *conics,
                          float *mus, int64_t total, r2s_stream_t stream);
int r2s_conics_mu_fwd_f64(const double *cov2d, double eps, double *conics,
                          double *mus, int64_t total, r2s_stream_t stream);

/* ConicsMu.cpp:87-159 conics_mu_bwd_tensor -> v_cov2d [total,6]. */
int r2s_conics_mu_bwd_f32(const float *cov2d, double eps, const float *conics,
                          const float *mus, const float *v_conics,
                          const float *v_mus, float *v_cov2d, int64_t total,
                          r2s_stream_t stream);
int r2s_conics_mu_bwd_f64(const double *cov2d, double eps, const double *conics,
                          const double *mus, const double *v_conics,
                          const double *v_mus, double *v_cov2d, int64_t total,
                          r2s_stream_t stream);

/* r2splat/ops/direct.py:149-161, fused: world_to_image_projection_fwd,
 * conics_mu_fwd and the opacity broadcast to [C,N], one pass.  As in the
 * reference, the radii use eps2d rounded to float and conics/mu use eps2d. */
int r2s_project_gaussians_fwd_f32(
    const float *means, const float *covars, const float *opacities,
    const float *viewmats, const float *Ks, uint32_t width, uint32_t height,
    double eps2d, float radius_clip, float *means2d, float *cov2d,
    int32_t *radii, float *conics, float *mus, float *opacity_cn, int64_t C,
    int64_t N, r2s_stream_t stream);
int r2s_project_gaussians_fwd_f64(
    const double *means, const double *covars, const double *opacities,
    const double *viewmats, const double *Ks, uint32_t width, uint32_t height,
    double eps2d, float radius_clip, double *means2d, double *cov2d,
    int32_t *radii, double *conics, double *mus, double *opacity_cn,
    int64_t C, int64_t N, r2s_stream_t stream);

/* r2splat/ops/explicit.py:299-316, fused: conics_mu_bwd followed by
 * world_to_image_projection_bwd (v_cov2d never touches HBM). */
int r2s_project_gaussians_bwd_f32(
    const float *means, const float *covars, const float *viewmats,
    const float *Ks, uint32_t width, uint32_t height, double eps2d,
    const float *cov2d, const float *conics, const float *mus,
    const float *v_means2d, const float *v_conics, const float *v_mus,
    float *v_means, float *v_covars, int64_t C, int64_t N,
    r2s_stream_t stream);
int r2s_project_gaussians_bwd_f64(
    const double *means, const double *covars, const double *viewmats,
    const double *Ks, uint32_t width, uint32_t height, double eps2d,
    const double *cov2d, const double *conics, const double *mus,
    const double *v_means2d, const double *v_conics, const double *v_mus,
    double *v_means, double *v_covars, int64_t C, int64_t N,
    r2s_stream_t stream);

/* The end of r2splat.ops' explicit backward in one pass per Gaussian, for
 * C >= 1 views: r2s_project_gaussians_bwd_* (explicit.py:299-316), plus
 * add_means [N,3] / add_covars [N,6] when given (the volume pass's
 * world-space gradients; both or neither), stored as v_means [N,3]; then
 * r2s_parameter_transform_bwd_* of that covariance gradient
 * (ParameterTransformBwd.cu:66-245) -> v_quats [N,4], v_raw_scales [N,3];
 * and r2s_opacity_bwd_* -> v_raw_opac [N] from v_opac_cn [C,N] and
 * v_opac_3d [N] (may be NULL).  Bit-identical to those three calls in turn
 * with v_covars = image + volume.  No reference counterpart (the reference
 * runs them as separate autograd nodes). */
int r2s_explicit_backward_tail_f32(
    const float *means, const float *covars, const float *viewmats, const float *Ks,
    uint32_t width, uint32_t height, double eps2d, const float *cov2d,
    const float *conics, const float *mus, const float *v_means2d,
    const float *v_conics, const float *v_mus, const float *add_means,
    const float *add_covars, const float *quats, const float *raw_scales, double smin,
    double smax, const float *raw_opac, const float *v_opac_cn, const float *v_opac_3d,
    float *v_means, float *v_quats, float *v_raw_scales, float *v_raw_opac, int64_t C,
    int64_t N, r2s_stream_t stream);
int r2s_explicit_backward_tail_f64(
    const double *means, const double *covars, const double *viewmats, const double *Ks,
    uint32_t width, uint32_t height, double eps2d, const double *cov2d,
    const double *conics, const double *mus, const double *v_means2d,
    const double *v_conics, const double *v_mus, const double *add_means,
    const double *add_covars, const double *quats, const double *raw_scales, double smin,
    double smax, const double *raw_opac, const double *v_opac_cn, const double *v_opac_3d,
    double *v_means, double *v_quats, double *v_raw_scales, double *v_raw_opac, int64_t C,
    int64_t N, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Tile binning                                                           */
/* ---------------------------------------------------------------------- */

/* Workspace for r2s_isect_count_* (n_items Gaussians) and
 * r2s_isect_emit_sort_* (n_isects records, keys on bits [0,end_bit)). */
int64_t r2s_isect_workspace_bytes(int64_t n_items, int64_t n_isects,
                                  uint32_t end_bit);

/* r2splat/cuda/csrc/IsectTiles.cpp:76-100 (count pass + int64 cumsum):
 * means2d [C,N,2], radii [C,N] or [C,N,2] -> tiles_per_gauss [C*N] (int32),
 * offsets [C*N+1] (int64, exclusive; offsets[C*N] = number of records). */
int r2s_isect_count_2d_f32(const float *means2d, const int32_t *radii,
                           int radii_is_rect, int64_t C, int64_t N,
                           uint32_t tile_size, uint32_t n_tiles_w,
                           uint32_t n_tiles_h, int32_t *tiles_per_gauss,
                           int64_t *offsets, void *workspace,
                           size_t workspace_bytes, r2s_stream_t stream);
int r2s_isect_count_2d_f64(const double *means2d, const int32_t *radii,
                           int radii_is_rect, int64_t C, int64_t N,
                           uint32_t tile_size, uint32_t n_tiles_w,
                           uint32_t n_tiles_h, int32_t *tiles_per_gauss,
                           int64_t *offsets, void *workspace,
                           size_t workspace_bytes, r2s_stream_t stream);

/* IsectTiles.cpp:113-169 (emit + stable radix sort on bits [0,end_bit)):
 * writes isect_ids [n_isects] (int64 key cid*T + ty*tw + tx) and
 * flatten_ids [n_isects] (int32 cid*N + g), ordered by (key, id).
 * emit_ids / isect_src (both or neither may be NULL; int32 [n_isects] each)
 * describe the records in emission order -- id-major, the records of one id
 * consecutive -- which the reference does not output: emit_ids[e] is the id
 * of emitted record e and isect_src[r] the emission index of sorted record
 * r.  The two-pass backward kernels (r2s_rasterize_bwd_emit_*,
 * r2s_voxelize_bwd_emit_*) take them.
 * tile_offsets (may be NULL; int32 [C*n_tiles_h*n_tiles_w]) receives what
 * r2s_isect_offset_encode computes from the sorted isect_ids, in the same
 * launch sequence: when one sort pass covers the key (at most 2048 keys) it
 * is read off that pass's digit offsets at no extra cost, else searched in
 * the sorted keys.  Not in the reference (whose isect_tiles returns no
 * offsets); r2splat.ops uses it in place of a separate encode call.
 * isect_ids may be NULL when tile_offsets is not: the keys are then not
 * written (the offsets and flatten_ids determine the list;
 * r2s_isect_keys_from_offsets recovers them), which r2splat.ops does, its
 * backward kernels finding each record's key from the offsets.
 * n_isects is the capacity of the outputs and the size the workspace is
 * queried for; the kernels read the record count from offsets[C*N] on the
 * device and write nothing when it exceeds n_isects.  A caller may thus
 * launch this before reading the count back, with a guessed capacity, and
 * call again with the exact count if the guess was short. */
int r2s_isect_emit_sort_2d_f32(const float *means2d, const int32_t *radii,
                               int radii_is_rect, int64_t C, int64_t N,
                               uint32_t tile_size, uint32_t n_tiles_w,
                               uint32_t n_tiles_h, const int64_t *offsets,
                               int64_t n_isects, uint32_t end_bit,
                               int64_t *isect_ids, int32_t *flatten_ids,
                               int32_t *emit_ids, int32_t *isect_src,
                               int32_t *tile_offsets, void *workspace,
                               size_t workspace_bytes,
                               r2s_stream_t stream);
int r2s_isect_emit_sort_2d_f64(const double *means2d, const int32_t *radii,
                               int radii_is_rect, int64_t C, int64_t N,
                               uint32_t tile_size, uint32_t n_tiles_w,
                               uint32_t n_tiles_h, const int64_t *offsets,
                               int64_t n_isects, uint32_t end_bit,
                               int64_t *isect_ids, int32_t *flatten_ids,
                               int32_t *emit_ids, int32_t *isect_src,
                               int32_t *tile_offsets, void *workspace,
                               size_t workspace_bytes,
                               r2s_stream_t stream);

/* r2splat/cuda/csrc/IsectTiles3D.cpp:72-96 (3D count + cumsum):
 * means3d [N,3], radii [N,3] -> tiles_per_gauss [N], offsets [N+1]. */
int r2s_isect_count_3d_f32(const float *means3d, const int32_t *radii,
                           int64_t N, uint32_t tile_size, uint32_t n_tiles_d2,
                           uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                           int32_t *tiles_per_gauss, int64_t *offsets,
                           void *workspace, size_t workspace_bytes,
                           r2s_stream_t stream);
int r2s_isect_count_3d_f64(const double *means3d, const int32_t *radii,
                           int64_t N, uint32_t tile_size, uint32_t n_tiles_d2,
                           uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                           int32_t *tiles_per_gauss, int64_t *offsets,
                           void *workspace, size_t workspace_bytes,
                           r2s_stream_t stream);

/* IsectTiles3D.cpp:109-161 (3D emit z->y->x + stable sort); emit_ids /
 * isect_src as for the 2D variant. */
int r2s_isect_emit_sort_3d_f32(const float *means3d, const int32_t *radii,
                               int64_t N, uint32_t tile_size,
                               uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                               uint32_t n_tiles_d0, const int64_t *offsets,
                               int64_t n_isects, uint32_t end_bit,
                               int64_t *isect_ids, int32_t *flatten_ids,
                               int32_t *emit_ids, int32_t *isect_src,
                               int32_t *tile_offsets, void *workspace,
                               size_t workspace_bytes,
                               r2s_stream_t stream);
int r2s_isect_emit_sort_3d_f64(const double *means3d, const int32_t *radii,
                               int64_t N, uint32_t tile_size,
                               uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                               uint32_t n_tiles_d0, const int64_t *offsets,
                               int64_t n_isects, uint32_t end_bit,
                               int64_t *isect_ids, int32_t *flatten_ids,
                               int32_t *emit_ids, int32_t *isect_src,
                               int32_t *tile_offsets, void *workspace,
                               size_t workspace_bytes,
                               r2s_stream_t stream);

/* Z-slab binning of large volumes.  IsectTiles3D.cpp:96-161 sizes one list
 * for the whole volume with int32 offsets (static_cast<int>(n_isects) at
 * IsectTiles3DKernel.cu:383-402), so a volume with 2^31 or more brick
 * records cannot be binned there.  These entries bin the brick layers
 * [z0, z1) of the dim0 axis alone: the records are those of the whole list
 * whose brick lies in the layers, in the same order, with keys relative to
 * layer z0 ((b0 - z0) n1 n2 + b1 n2 + b2).  No reference counterpart.
 *
 * r2s_isect_layer_counts_3d_*: counts [n_tiles_d0] int64, the records of
 * each brick layer (to plan slabs); workspace of (n_tiles_d0 + 1) * 8
 * bytes. */
int r2s_isect_layer_counts_3d_f32(const float *means3d, const int32_t *radii, int64_t N,
                                  uint32_t tile_size, uint32_t n_tiles_d2,
                                  uint32_t n_tiles_d1, uint32_t n_tiles_d0, int64_t *counts,
                                  void *workspace, size_t workspace_bytes,
                                  r2s_stream_t stream);
int r2s_isect_layer_counts_3d_f64(const double *means3d, const int32_t *radii, int64_t N,
                                  uint32_t tile_size, uint32_t n_tiles_d2,
                                  uint32_t n_tiles_d1, uint32_t n_tiles_d0, int64_t *counts,
                                  void *workspace, size_t workspace_bytes,
                                  r2s_stream_t stream);
/* As r2s_isect_count_3d_* / r2s_isect_emit_sort_3d_* for the layers
 * [z0, z1) (n_tiles_d0 is the whole grid's; keys below (z1 - z0) n1 n2). */
int r2s_isect_count_3d_slab_f32(const float *means3d, const int32_t *radii, int64_t N,
                                uint32_t tile_size, uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                                uint32_t n_tiles_d0, uint32_t z0, uint32_t z1,
                                int32_t *tiles_per_gauss, int64_t *offsets, void *workspace,
                                size_t workspace_bytes, r2s_stream_t stream);
int r2s_isect_count_3d_slab_f64(const double *means3d, const int32_t *radii, int64_t N,
                                uint32_t tile_size, uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                                uint32_t n_tiles_d0, uint32_t z0, uint32_t z1,
                                int32_t *tiles_per_gauss, int64_t *offsets, void *workspace,
                                size_t workspace_bytes, r2s_stream_t stream);
int r2s_isect_emit_sort_3d_slab_f32(const float *means3d, const int32_t *radii, int64_t N,
                                    uint32_t tile_size, uint32_t n_tiles_d2,
                                    uint32_t n_tiles_d1, uint32_t n_tiles_d0, uint32_t z0,
                                    uint32_t z1, const int64_t *offsets, int64_t n_isects,
                                    uint32_t end_bit, int64_t *isect_ids, int32_t *flatten_ids,
                                    int32_t *emit_ids, int32_t *isect_src,
                                    int32_t *tile_offsets, void *workspace,
                                    size_t workspace_bytes, r2s_stream_t stream);
int r2s_isect_emit_sort_3d_slab_f64(const double *means3d, const int32_t *radii, int64_t N,
                                    uint32_t tile_size, uint32_t n_tiles_d2,
                                    uint32_t n_tiles_d1, uint32_t n_tiles_d0, uint32_t z0,
                                    uint32_t z1, const int64_t *offsets, int64_t n_isects,
                                    uint32_t end_bit, int64_t *isect_ids, int32_t *flatten_ids,
                                    int32_t *emit_ids, int32_t *isect_src,
                                    int32_t *tile_offsets, void *workspace,
                                    size_t workspace_bytes, r2s_stream_t stream);

/* IsectTiles.cpp:176-215 isect_offset_encode_tensor and
 * IsectTiles3D.cpp:168-204 isect_offset_encode_3d_tensor:
 * tile_offsets[k] = lower_bound(isect_ids, k) for k in [0, n_keys). */
int r2s_isect_offset_encode(const int64_t *isect_ids, int64_t n_isects,
                            int64_t n_keys, int32_t *tile_offsets,
                            r2s_stream_t stream);

/* The isect_ids output of IsectTiles.cpp:113-169 / IsectTiles3D.cpp:109-161
 * recovered from a list's tile_offsets (the inverse of
 * r2s_isect_offset_encode; no entry of its own in the reference), for lists
 * sorted with isect_ids NULL: isect_ids[r] = the last key k with
 * tile_offsets[k] <= r, for the n_isects records; tile_offsets [n_keys],
 * tile_offsets[0] = 0. */
int r2s_isect_keys_from_offsets(const int32_t *tile_offsets, int64_t n_keys,
                                int64_t n_isects, int64_t *isect_ids,
                                r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Line-integral rasterizer                                               */
/* ---------------------------------------------------------------------- */

/* Workspace for r2s_rasterize_fwd_*: the partial tiles when heavy tiles are
 * split across several blocks (tile sizes 8, 16, 32 with 2048 or more
 * records per tile on average); 0 otherwise. */
int64_t r2s_rasterize_workspace_bytes(int64_t n_keys, int64_t n_isects,
                                      uint32_t tile_size, int dtype_bytes);

/* r2splat/cuda/csrc/RasterizeToPixels.cpp:25-114 rasterize_to_pixels_fwd_tensor:
 * image [C,H,W] = per pixel sum over the tile list of
 * opacity*mu*exp(-sigma), skipping sigma < 0 and |alpha| < 1e-5. */
int r2s_rasterize_fwd_f32(const float *means2d, const float *conics,
                          const float *opacities, const float *mus,
                          const int32_t *tile_offsets,
                          const int32_t *flatten_ids, int64_t n_isects,
                          int64_t C, int64_t N, uint32_t width, uint32_t height,
                          uint32_t tile_size, uint32_t n_tiles_w,
                          uint32_t n_tiles_h, float *image, void *workspace,
                          size_t workspace_bytes, r2s_stream_t stream);
int r2s_rasterize_fwd_f64(const double *means2d, const double *conics,
                          const double *opacities, const double *mus,
                          const int32_t *tile_offsets,
                          const int32_t *flatten_ids, int64_t n_isects,
                          int64_t C, int64_t N, uint32_t width, uint32_t height,
                          uint32_t tile_size, uint32_t n_tiles_w,
                          uint32_t n_tiles_h, double *image, void *workspace,
                          size_t workspace_bytes, r2s_stream_t stream);

/* No counterpart in the reference: r2s_rasterize_fwd_* for callers that
 * cannot allocate or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split partial tiles
 * live in a static device array of R2S_RASTER_SCRATCH_BYTES per GPU, held
 * until the process ends; a call whose partial tiles
 * (r2s_rasterize_workspace_bytes) exceed it fails with R2S_ERANGE.  The
 * array's address is looked up on the first call on each device, which must
 * be the current device and the stream's, and kept for the process: after a
 * hipDeviceReset() that address is stale, so a process that resets a device
 * must not call this entry point on it again.  All calls on one GPU share the
 * array: calls that overlap on one GPU (concurrent streams) race; calls on
 * one stream do not.  The image equals r2s_rasterize_fwd_*'s bit for bit. */
#define R2S_RASTER_SCRATCH_BYTES (32u << 20)
int r2s_rasterize_fwd_noalloc_f32(const float *means2d, const float *conics,
                                  const float *opacities, const float *mus,
                                  const int32_t *tile_offsets,
                                  const int32_t *flatten_ids, int64_t n_isects,
                                  int64_t C, int64_t N, uint32_t width,
                                  uint32_t height, uint32_t tile_size,
                                  uint32_t n_tiles_w, uint32_t n_tiles_h,
                                  float *image, r2s_stream_t stream);
int r2s_rasterize_fwd_noalloc_f64(const double *means2d, const double *conics,
                                  const double *opacities, const double *mus,
                                  const int32_t *tile_offsets,
                                  const int32_t *flatten_ids, int64_t n_isects,
                                  int64_t C, int64_t N, uint32_t width,
                                  uint32_t height, uint32_t tile_size,
                                  uint32_t n_tiles_w, uint32_t n_tiles_h,
                                  double *image, r2s_stream_t stream);

/* RasterizeToPixels.cpp:226-317 rasterize_to_pixels_bwd_per_gaussian_tensor
 * (isect_ids != NULL) and RasterizeToPixels.cpp:122-222
 * rasterize_to_pixels_bwd_tensor (isect_ids == NULL: the tile of each record
 * comes from tile_offsets).  Outputs are accumulated (+=): the caller zeroes
 * them.  v_means2d_abs may be NULL (absgrad off). */
int r2s_rasterize_bwd_f32(const float *means2d, const float *conics,
                          const float *opacities, const float *mus,
                          const int32_t *tile_offsets, const int64_t *isect_ids,
                          const int32_t *flatten_ids, int64_t n_isects,
                          const float *v_image, int64_t C, int64_t N,
                          uint32_t width, uint32_t height, uint32_t tile_size,
                          uint32_t n_tiles_w, uint32_t n_tiles_h,
                          float *v_means2d_abs, float *v_means2d,
                          float *v_conics, float *v_opacities, float *v_mus,
                          r2s_stream_t stream);
int r2s_rasterize_bwd_f64(const double *means2d, const double *conics,
                          const double *opacities, const double *mus,
                          const int32_t *tile_offsets, const int64_t *isect_ids,
                          const int32_t *flatten_ids, int64_t n_isects,
                          const double *v_image, int64_t C, int64_t N,
                          uint32_t width, uint32_t height, uint32_t tile_size,
                          uint32_t n_tiles_w, uint32_t n_tiles_h,
                          double *v_means2d_abs, double *v_means2d,
                          double *v_conics, double *v_opacities, double *v_mus,
                          r2s_stream_t stream);

/* Workspace of r2s_rasterize_bwd_emit_* / _rows_* over n_isects records of
 * n_items = C*N (view, Gaussian) pairs: one row of 8 values of dtype_bytes
 * per record (32 bytes in float), then a packed payload of 8 values per
 * pair. */
int64_t r2s_rasterize_bwd_workspace_bytes(int64_t n_isects, int64_t n_items,
                                          int dtype_bytes);

/* The same VJP as r2s_rasterize_bwd_* (RasterizeToPixelsBwd.cu:77-480) in
 * two passes, without one device-scope atomic per record and partial: the
 * records are walked in tile order and each record's partials are stored as
 * a row of the workspace at its emission index (isect_src); a second pass
 * walks the rows in emission order, where each Gaussian's records are
 * consecutive (emit_ids), sums them and stores each Gaussian's sums once.
 * Deterministic.  isect_ids may be NULL.  Outputs are stored, not
 * accumulated, for every Gaussian: zero where it has no record, so they
 * need no zeroing beforehand.  emit_ids must be as the emit-sort calls
 * write it (ids ascending). */
int r2s_rasterize_bwd_emit_f32(const float *means2d, const float *conics,
                               const float *opacities, const float *mus,
                               const int32_t *tile_offsets, const int64_t *isect_ids,
                               const int32_t *flatten_ids, const int32_t *emit_ids,
                               const int32_t *isect_src, int64_t n_isects,
                               const float *v_image, int64_t C, int64_t N,
                               uint32_t width, uint32_t height, uint32_t tile_size,
                               uint32_t n_tiles_w, uint32_t n_tiles_h,
                               float *v_means2d_abs, float *v_means2d, float *v_conics,
                               float *v_opacities, float *v_mus, void *workspace,
                               size_t workspace_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_emit_f64(const double *means2d, const double *conics,
                               const double *opacities, const double *mus,
                               const int32_t *tile_offsets, const int64_t *isect_ids,
                               const int32_t *flatten_ids, const int32_t *emit_ids,
                               const int32_t *isect_src, int64_t n_isects,
                               const double *v_image, int64_t C, int64_t N,
                               uint32_t width, uint32_t height, uint32_t tile_size,
                               uint32_t n_tiles_w, uint32_t n_tiles_h,
                               double *v_means2d_abs, double *v_means2d, double *v_conics,
                               double *v_opacities, double *v_mus, void *workspace,
                               size_t workspace_bytes, r2s_stream_t stream);

/* The two passes of r2s_rasterize_bwd_emit_* as separate calls (for callers
 * that schedule or time them apart).  _rows: the first pass; writes the
 * per-record rows at their emission index into `rows`
 * (r2s_rasterize_bwd_workspace_bytes, 16-byte aligned): 8 values
 * v_means2d (2), v_conics (3), T0 = sum of v exp(-sigma) over the record's
 * passing pixels, v_means2d_abs (2) -- the last two zero with absgrad == 0.
 * _reduce: the second pass; stores each Gaussian's sums, v_opacities =
 * mus sum(T0) and v_mus = opacities sum(T0) (the record partials mu T0 and
 * o T0, summed), zero for Gaussians without records (v_means2d_abs NULL
 * exactly when the rows were written with absgrad == 0).  No reference
 * counterpart. */
int r2s_rasterize_bwd_rows_f32(const float *means2d, const float *conics,
                               const float *opacities, const float *mus,
                               const int32_t *tile_offsets, const int64_t *isect_ids,
                               const int32_t *flatten_ids, const int32_t *isect_src,
                               int64_t n_isects, const float *v_image, int64_t C, int64_t N,
                               uint32_t width, uint32_t height, uint32_t tile_size,
                               uint32_t n_tiles_w, uint32_t n_tiles_h, int absgrad,
                               void *rows, size_t rows_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_rows_f64(const double *means2d, const double *conics,
                               const double *opacities, const double *mus,
                               const int32_t *tile_offsets, const int64_t *isect_ids,
                               const int32_t *flatten_ids, const int32_t *isect_src,
                               int64_t n_isects, const double *v_image, int64_t C, int64_t N,
                               uint32_t width, uint32_t height, uint32_t tile_size,
                               uint32_t n_tiles_w, uint32_t n_tiles_h, int absgrad,
                               void *rows, size_t rows_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_reduce_f32(const float *rows, const int32_t *emit_ids, int64_t n_isects,
                                 int64_t C, int64_t N, const float *opacities,
                                 const float *mus, float *v_means2d_abs, float *v_means2d,
                                 float *v_conics, float *v_opacities, float *v_mus,
                                 r2s_stream_t stream);
int r2s_rasterize_bwd_reduce_f64(const double *rows, const int32_t *emit_ids,
                                 int64_t n_isects, int64_t C, int64_t N,
                                 const double *opacities, const double *mus,
                                 double *v_means2d_abs, double *v_means2d, double *v_conics,
                                 double *v_opacities, double *v_mus, r2s_stream_t stream);

/* The rasterizer over a packed per-(view, Gaussian) payload: the same
 * operations as RasterizeToPixelsFwd.cu:57-186 / RasterizeToPixelsBwd.cu:
 * 350-480 (the reference reads the four arrays directly; it has no payload).
 * r2s_rasterize_pack_* writes the payload [C*N*8] of T
 * (r2s_rasterize_payload_bytes, 16-byte aligned): per pair the mean, the
 * conic, o mu = opacities * mus, the alpha test's limit and the culling
 * half-height; with v_means2d non-NULL it also stores zeros into the
 * two-pass backward's outputs (v_means2d_abs may be NULL).  Written once per
 * call, it serves both passes: r2s_rasterize_fwd_packed_* (tile sizes 8, 16
 * and 32; the same image as r2s_rasterize_fwd_* bit for bit; workspace as
 * r2s_rasterize_workspace_bytes) reads a record's data as one 32-byte load
 * instead of four arrays' lines, and r2s_rasterize_bwd_packed_* is
 * r2s_rasterize_bwd_emit_* without its own pack launch (workspace: the rows
 * only, r2s_rasterize_bwd_workspace_bytes(n_isects, 0, dtype_bytes); zeroed:
 * the outputs hold zeros already, from the pack call).  _bwd_rows_packed:
 * its first pass alone, as r2s_rasterize_bwd_rows_* over the given payload
 * (rows: r2s_rasterize_bwd_workspace_bytes(n_isects, 0, dtype_bytes)).
 * Used by r2splat.ops. */
int64_t r2s_rasterize_payload_bytes(int64_t n_items, int dtype_bytes);
int r2s_rasterize_pack_f32(const float *means2d, const float *conics,
                           const float *opacities, const float *mus, int64_t C, int64_t N,
                           float *payload, float *v_means2d_abs, float *v_means2d,
                           float *v_conics, float *v_opacities, float *v_mus,
                           r2s_stream_t stream);
int r2s_rasterize_pack_f64(const double *means2d, const double *conics,
                           const double *opacities, const double *mus, int64_t C, int64_t N,
                           double *payload, double *v_means2d_abs, double *v_means2d,
                           double *v_conics, double *v_opacities, double *v_mus,
                           r2s_stream_t stream);
/* r2s_project_gaussians_fwd_* and r2s_rasterize_pack_* on its outputs in one
 * launch (no counterpart in the reference, whose rasterizer has no payload):
 * the same outputs, payload and zeros bit for bit, without the pack's reads
 * of the projection's outputs.  payload (16-byte aligned) is required. */
int r2s_project_pack_fwd_f32(
    const float *means, const float *covars, const float *opacities,
    const float *viewmats, const float *Ks, uint32_t width, uint32_t height,
    double eps2d, float radius_clip, float *means2d, float *cov2d,
    int32_t *radii, float *conics, float *mus, float *opacity_cn, float *payload,
    float *v_means2d_abs, float *v_means2d, float *v_conics, float *v_opacities,
    float *v_mus, int64_t C, int64_t N, r2s_stream_t stream);
int r2s_project_pack_fwd_f64(
    const double *means, const double *covars, const double *opacities,
    const double *viewmats, const double *Ks, uint32_t width, uint32_t height,
    double eps2d, float radius_clip, double *means2d, double *cov2d,
    int32_t *radii, double *conics, double *mus, double *opacity_cn, double *payload,
    double *v_means2d_abs, double *v_means2d, double *v_conics, double *v_opacities,
    double *v_mus, int64_t C, int64_t N, r2s_stream_t stream);
int r2s_rasterize_fwd_packed_f32(const float *payload, const int32_t *tile_offsets,
                                 const int32_t *flatten_ids, int64_t n_isects, int64_t C,
                                 int64_t N, uint32_t width, uint32_t height,
                                 uint32_t tile_size, uint32_t n_tiles_w, uint32_t n_tiles_h,
                                 float *image, void *workspace, size_t workspace_bytes,
                                 r2s_stream_t stream);
int r2s_rasterize_fwd_packed_f64(const double *payload, const int32_t *tile_offsets,
                                 const int32_t *flatten_ids, int64_t n_isects, int64_t C,
                                 int64_t N, uint32_t width, uint32_t height,
                                 uint32_t tile_size, uint32_t n_tiles_w, uint32_t n_tiles_h,
                                 double *image, void *workspace, size_t workspace_bytes,
                                 r2s_stream_t stream);
int r2s_rasterize_bwd_packed_f32(const float *payload, const float *opacities,
                                 const float *mus, const int32_t *tile_offsets,
                                 const int64_t *isect_ids, const int32_t *flatten_ids,
                                 const int32_t *emit_ids, const int32_t *isect_src,
                                 int64_t n_isects, const float *v_image, int64_t C, int64_t N,
                                 uint32_t width, uint32_t height, uint32_t tile_size,
                                 uint32_t n_tiles_w, uint32_t n_tiles_h, float *v_means2d_abs,
                                 float *v_means2d, float *v_conics, float *v_opacities,
                                 float *v_mus, int zeroed, void *workspace,
                                 size_t workspace_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_packed_f64(const double *payload, const double *opacities,
                                 const double *mus, const int32_t *tile_offsets,
                                 const int64_t *isect_ids, const int32_t *flatten_ids,
                                 const int32_t *emit_ids, const int32_t *isect_src,
                                 int64_t n_isects, const double *v_image, int64_t C, int64_t N,
                                 uint32_t width, uint32_t height, uint32_t tile_size,
                                 uint32_t n_tiles_w, uint32_t n_tiles_h,
                                 double *v_means2d_abs, double *v_means2d, double *v_conics,
                                 double *v_opacities, double *v_mus, int zeroed,
                                 void *workspace, size_t workspace_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_rows_packed_f32(const float *payload, const int32_t *tile_offsets,
                                      const int64_t *isect_ids, const int32_t *flatten_ids,
                                      const int32_t *isect_src, int64_t n_isects,
                                      const float *v_image, int64_t C, int64_t N,
                                      uint32_t width, uint32_t height, uint32_t tile_size,
                                      uint32_t n_tiles_w, uint32_t n_tiles_h, int absgrad,
                                      void *rows, size_t rows_bytes, r2s_stream_t stream);
int r2s_rasterize_bwd_rows_packed_f64(const double *payload, const int32_t *tile_offsets,
                                      const int64_t *isect_ids, const int32_t *flatten_ids,
                                      const int32_t *isect_src, int64_t n_isects,
                                      const double *v_image, int64_t C, int64_t N,
                                      uint32_t width, uint32_t height, uint32_t tile_size,
                                      uint32_t n_tiles_w, uint32_t n_tiles_h, int absgrad,
                                      void *rows, size_t rows_bytes, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Volume mapping and voxelizer                                           */
/* ---------------------------------------------------------------------- */

/* r2splat/cuda/csrc/WorldToVolumeMapping.cpp:37-112
 * world_to_volume_mapping_fwd_tensor: means [N,3], covars [N,6],
 * ranges [3], centers [3] -> means3d [N,3], conics [N,6], radii [N,3].
 * (The reference's max_scales argument is unused and is not taken here.) */
int r2s_world_to_volume_mapping_fwd_f32(
    const float *means, const float *covars, const float *ranges,
    const float *centers, uint32_t dim2, uint32_t dim1, uint32_t dim0,
    double eps3d, double radius_clip, float *means3d, float *conics,
    int32_t *radii, int64_t N, r2s_stream_t stream);
int r2s_world_to_volume_mapping_fwd_f64(
    const double *means, const double *covars, const double *ranges,
    const double *centers, uint32_t dim2, uint32_t dim1, uint32_t dim0,
    double eps3d, double radius_clip, double *means3d, double *conics,
    int32_t *radii, int64_t N, r2s_stream_t stream);

/* WorldToVolumeMapping.cpp:119-192 world_to_volume_mapping_bwd_tensor. */
int r2s_world_to_volume_mapping_bwd_f32(
    const float *means, const float *covars, const float *ranges,
    const float *centers, uint32_t dim2, uint32_t dim1, uint32_t dim0,
    double eps3d, const float *v_means3d, const float *v_conics,
    float *v_means, float *v_covars, int64_t N, r2s_stream_t stream);
int r2s_world_to_volume_mapping_bwd_f64(
    const double *means, const double *covars, const double *ranges,
    const double *centers, uint32_t dim2, uint32_t dim1, uint32_t dim0,
    double eps3d, const double *v_means3d, const double *v_conics,
    double *v_means, double *v_covars, int64_t N, r2s_stream_t stream);

/* r2splat/cuda/csrc/VoxelizeToVoxels.cpp:31-108 voxelize_to_voxels_fwd_tensor:
 * volume [dim0,dim1,dim2] = per voxel sum of opacity*exp(-sigma) over the
 * brick list, skipping sigma < 0 and |alpha| < 1e-6.  Fully written. */
int r2s_voxelize_fwd_f32(const float *means3d, const float *conics,
                         const float *opacities, const int32_t *tile_offsets,
                         const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                         uint32_t dim2, uint32_t dim1, uint32_t dim0,
                         uint32_t tile_size, uint32_t n_tiles_d2,
                         uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                         float *volume, r2s_stream_t stream);
int r2s_voxelize_fwd_f64(const double *means3d, const double *conics,
                         const double *opacities, const int32_t *tile_offsets,
                         const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                         uint32_t dim2, uint32_t dim1, uint32_t dim0,
                         uint32_t tile_size, uint32_t n_tiles_d2,
                         uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                         double *volume, r2s_stream_t stream);

/* VoxelizeToVoxels.cpp:195-278 voxelize_to_voxels_bwd_per_gaussian_tensor
 * (isect_ids != NULL) and VoxelizeToVoxels.cpp:115-192
 * voxelize_to_voxels_bwd_tensor (isect_ids == NULL).  Accumulates (+=). */
int r2s_voxelize_bwd_f32(const float *means3d, const float *conics,
                         const float *opacities, const int32_t *tile_offsets,
                         const int64_t *isect_ids, const int32_t *flatten_ids,
                         int64_t n_isects, const float *v_volume, int64_t N,
                         uint32_t dim2, uint32_t dim1, uint32_t dim0,
                         uint32_t tile_size, uint32_t n_tiles_d2,
                         uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                         float *v_means3d, float *v_conics, float *v_opacities,
                         r2s_stream_t stream);
int r2s_voxelize_bwd_f64(const double *means3d, const double *conics,
                         const double *opacities, const int32_t *tile_offsets,
                         const int64_t *isect_ids, const int32_t *flatten_ids,
                         int64_t n_isects, const double *v_volume, int64_t N,
                         uint32_t dim2, uint32_t dim1, uint32_t dim0,
                         uint32_t tile_size, uint32_t n_tiles_d2,
                         uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                         double *v_means3d, double *v_conics,
                         double *v_opacities, r2s_stream_t stream);

/* Workspace of r2s_voxelize_bwd_emit_*: one row of 10 values of
 * dtype_bytes per record. */
int64_t r2s_voxelize_bwd_workspace_bytes(int64_t n_isects, int dtype_bytes);

/* The same VJP as r2s_voxelize_bwd_* (VoxelizeToVoxelsBwd.cu:71-441) in two
 * passes, as r2s_rasterize_bwd_emit_*: per-record rows stored at their
 * emission index, then summed per Gaussian and stored once.
 * Deterministic.  isect_ids may be NULL.  Outputs are stored for every
 * Gaussian, zero where it has no record, as for the rasterizer. */
int r2s_voxelize_bwd_emit_f32(const float *means3d, const float *conics,
                              const float *opacities, const int32_t *tile_offsets,
                              const int64_t *isect_ids, const int32_t *flatten_ids,
                              const int32_t *emit_ids, const int32_t *isect_src,
                              int64_t n_isects, const float *v_volume, int64_t N,
                              uint32_t dim2, uint32_t dim1, uint32_t dim0,
                              uint32_t tile_size, uint32_t n_tiles_d2,
                              uint32_t n_tiles_d1, uint32_t n_tiles_d0, float *v_means3d,
                              float *v_conics, float *v_opacities, void *workspace,
                              size_t workspace_bytes, r2s_stream_t stream);
int r2s_voxelize_bwd_emit_f64(const double *means3d, const double *conics,
                              const double *opacities, const int32_t *tile_offsets,
                              const int64_t *isect_ids, const int32_t *flatten_ids,
                              const int32_t *emit_ids, const int32_t *isect_src,
                              int64_t n_isects, const double *v_volume, int64_t N,
                              uint32_t dim2, uint32_t dim1, uint32_t dim0,
                              uint32_t tile_size, uint32_t n_tiles_d2,
                              uint32_t n_tiles_d1, uint32_t n_tiles_d0, double *v_means3d,
                              double *v_conics, double *v_opacities, void *workspace,
                              size_t workspace_bytes, r2s_stream_t stream);

/* One z-slab of a volume binned by r2s_isect_*_3d_slab_*: the lists of the
 * nz brick layers from layer z0 on (tile_offsets [nz, n1, n2], keys
 * relative to layer z0) against the whole volume [dim0, dim1, dim2] and its
 * upstream gradient.  The forward writes only the slab's voxel slices
 * [z0 ts, min((z0 + nz) ts, dim0)); the backward stores every Gaussian's
 * output (zero without records in the slab), so a caller sums the slabs'
 * outputs.  No reference counterpart (VoxelizeToVoxels.cpp:31-278 take one
 * list of the whole volume). */
int r2s_voxelize_fwd_slab_f32(const float *means3d, const float *conics,
                              const float *opacities, const int32_t *tile_offsets,
                              const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                              uint32_t dim2, uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                              uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t z0,
                              uint32_t nz, float *volume, r2s_stream_t stream);
int r2s_voxelize_fwd_slab_f64(const double *means3d, const double *conics,
                              const double *opacities, const int32_t *tile_offsets,
                              const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                              uint32_t dim2, uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                              uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t z0,
                              uint32_t nz, double *volume, r2s_stream_t stream);
int r2s_voxelize_bwd_emit_slab_f32(const float *means3d, const float *conics,
                                   const float *opacities, const int32_t *tile_offsets,
                                   const int64_t *isect_ids, const int32_t *flatten_ids,
                                   const int32_t *emit_ids, const int32_t *isect_src,
                                   int64_t n_isects, const float *v_volume, int64_t N,
                                   uint32_t dim2, uint32_t dim1, uint32_t dim0,
                                   uint32_t tile_size, uint32_t n_tiles_d2,
                                   uint32_t n_tiles_d1, uint32_t z0, uint32_t nz,
                                   float *v_means3d, float *v_conics, float *v_opacities,
                                   void *workspace, size_t workspace_bytes,
                                   r2s_stream_t stream);
int r2s_voxelize_bwd_emit_slab_f64(const double *means3d, const double *conics,
                                   const double *opacities, const int32_t *tile_offsets,
                                   const int64_t *isect_ids, const int32_t *flatten_ids,
                                   const int32_t *emit_ids, const int32_t *isect_src,
                                   int64_t n_isects, const double *v_volume, int64_t N,
                                   uint32_t dim2, uint32_t dim1, uint32_t dim0,
                                   uint32_t tile_size, uint32_t n_tiles_d2,
                                   uint32_t n_tiles_d1, uint32_t z0, uint32_t nz,
                                   double *v_means3d, double *v_conics, double *v_opacities,
                                   void *workspace, size_t workspace_bytes,
                                   r2s_stream_t stream);

/* The forward and the two-pass backward over the same brick lists (tile
 * size 8), for a caller that keeps the lists between them: the forward
 * also stores each record's reach mask (the brick rows its alpha-test
 * ellipsoid reaches, bit 8 * slice + row; reach [n_isects] at the record's
 * list position), and the backward takes them instead of recomputing them.
 * The masks are valid only for the means3d, conics, opacities and lists
 * the forward saw.  No reference counterpart (VoxelizeToVoxels.cpp:31-278
 * recompute everything per call). */
int r2s_voxelize_fwd_reach_f32(const float *means3d, const float *conics,
                               const float *opacities, const int32_t *tile_offsets,
                               const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                               uint32_t dim2, uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                               uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                               float *volume, uint64_t *reach, r2s_stream_t stream);
int r2s_voxelize_fwd_reach_f64(const double *means3d, const double *conics,
                               const double *opacities, const int32_t *tile_offsets,
                               const int32_t *flatten_ids, int64_t n_isects, int64_t N,
                               uint32_t dim2, uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                               uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                               double *volume, uint64_t *reach, r2s_stream_t stream);
int r2s_voxelize_bwd_emit_reach_f32(const float *means3d, const float *conics,
                                    const float *opacities, const int32_t *tile_offsets,
                                    const int64_t *isect_ids, const int32_t *flatten_ids,
                                    const int32_t *emit_ids, const int32_t *isect_src,
                                    int64_t n_isects, const float *v_volume, int64_t N,
                                    uint32_t dim2, uint32_t dim1, uint32_t dim0,
                                    uint32_t tile_size, uint32_t n_tiles_d2,
                                    uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                                    const uint64_t *reach, float *v_means3d, float *v_conics,
                                    float *v_opacities, void *workspace, size_t workspace_bytes,
                                    r2s_stream_t stream);
int r2s_voxelize_bwd_emit_reach_f64(const double *means3d, const double *conics,
                                    const double *opacities, const int32_t *tile_offsets,
                                    const int64_t *isect_ids, const int32_t *flatten_ids,
                                    const int32_t *emit_ids, const int32_t *isect_src,
                                    int64_t n_isects, const double *v_volume, int64_t N,
                                    uint32_t dim2, uint32_t dim1, uint32_t dim0,
                                    uint32_t tile_size, uint32_t n_tiles_d2,
                                    uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                                    const uint64_t *reach, double *v_means3d,
                                    double *v_conics, double *v_opacities, void *workspace,
                                    size_t workspace_bytes, r2s_stream_t stream);

/* The first pass of r2s_voxelize_bwd_emit_reach_* alone (as
 * r2s_voxelize_bwd_rows_*, with the forward's reach masks). */
int r2s_voxelize_bwd_rows_reach_f32(const float *means3d, const float *conics,
                                    const float *opacities, const int32_t *tile_offsets,
                                    const int64_t *isect_ids, const int32_t *flatten_ids,
                                    const int32_t *isect_src, int64_t n_isects,
                                    const float *v_volume, int64_t N, uint32_t dim2,
                                    uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                                    uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                                    uint32_t n_tiles_d0, const uint64_t *reach, void *rows,
                                    size_t rows_bytes, r2s_stream_t stream);
int r2s_voxelize_bwd_rows_reach_f64(const double *means3d, const double *conics,
                                    const double *opacities, const int32_t *tile_offsets,
                                    const int64_t *isect_ids, const int32_t *flatten_ids,
                                    const int32_t *isect_src, int64_t n_isects,
                                    const double *v_volume, int64_t N, uint32_t dim2,
                                    uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                                    uint32_t n_tiles_d2, uint32_t n_tiles_d1,
                                    uint32_t n_tiles_d0, const uint64_t *reach, void *rows,
                                    size_t rows_bytes, r2s_stream_t stream);

/* The first pass of r2s_voxelize_bwd_emit_slab_* alone (the rows of one
 * slab's records, as r2s_voxelize_bwd_rows_*). */
int r2s_voxelize_bwd_rows_slab_f32(const float *means3d, const float *conics,
                                   const float *opacities, const int32_t *tile_offsets,
                                   const int64_t *isect_ids, const int32_t *flatten_ids,
                                   const int32_t *isect_src, int64_t n_isects,
                                   const float *v_volume, int64_t N, uint32_t dim2,
                                   uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                                   uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t z0,
                                   uint32_t nz, void *rows, size_t rows_bytes,
                                   r2s_stream_t stream);
int r2s_voxelize_bwd_rows_slab_f64(const double *means3d, const double *conics,
                                   const double *opacities, const int32_t *tile_offsets,
                                   const int64_t *isect_ids, const int32_t *flatten_ids,
                                   const int32_t *isect_src, int64_t n_isects,
                                   const double *v_volume, int64_t N, uint32_t dim2,
                                   uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                                   uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t z0,
                                   uint32_t nz, void *rows, size_t rows_bytes,
                                   r2s_stream_t stream);

/* The two passes of r2s_voxelize_bwd_emit_* as separate calls, as for the
 * rasterizer (10 row values).  No reference counterpart. */
int r2s_voxelize_bwd_rows_f32(const float *means3d, const float *conics,
                              const float *opacities, const int32_t *tile_offsets,
                              const int64_t *isect_ids, const int32_t *flatten_ids,
                              const int32_t *isect_src, int64_t n_isects,
                              const float *v_volume, int64_t N, uint32_t dim2, uint32_t dim1,
                              uint32_t dim0, uint32_t tile_size, uint32_t n_tiles_d2,
                              uint32_t n_tiles_d1, uint32_t n_tiles_d0, void *rows,
                              size_t rows_bytes, r2s_stream_t stream);
int r2s_voxelize_bwd_rows_f64(const double *means3d, const double *conics,
                              const double *opacities, const int32_t *tile_offsets,
                              const int64_t *isect_ids, const int32_t *flatten_ids,
                              const int32_t *isect_src, int64_t n_isects,
                              const double *v_volume, int64_t N, uint32_t dim2,
                              uint32_t dim1, uint32_t dim0, uint32_t tile_size,
                              uint32_t n_tiles_d2, uint32_t n_tiles_d1, uint32_t n_tiles_d0,
                              void *rows, size_t rows_bytes, r2s_stream_t stream);
int r2s_voxelize_bwd_reduce_f32(const float *rows, const int32_t *emit_ids, int64_t n_isects,
                                int64_t N, float *v_means3d, float *v_conics,
                                float *v_opacities, r2s_stream_t stream);
int r2s_voxelize_bwd_reduce_f64(const double *rows, const int32_t *emit_ids,
                                int64_t n_isects, int64_t N, double *v_means3d,
                                double *v_conics, double *v_opacities, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Densify / prune index compaction                                        */
/* ---------------------------------------------------------------------- */

/* Workspace for r2s_mask_split. */
int64_t r2s_mask_workspace_bytes(int64_t n);

/* src/strategies/binary_tree.py:68,101-102,158 (torch.where(mask)[0] and
 * torch.where(~mask)[0]): mask [n] (bytes, nonzero = true) ->
 * out [n] int64 = ascending indices of true entries followed by ascending
 * indices of false entries; *n_true_dev (device int64) = number of trues. */
int r2s_mask_split(const uint8_t *mask, int64_t n, int64_t *out,
                   int64_t *n_true_dev, void *workspace,
                   size_t workspace_bytes, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Densify / prune: fused table rewrite                                    */
/* ---------------------------------------------------------------------- */

/* The Gaussian table of the binary-tree model is a set of columns with one
 * row per Gaussian: the trainable parameters, their Adam moments, the tree
 * buffers (parent, level), the strategy's per-Gaussian statistics and the
 * history archive.  split / duplicate / remove rebuild every column from the
 * selected (sel) and kept (rest) index lists in one launch.  Each column is
 * rows of `width` 4-byte words (float32 or int32); `dst` is a new array of
 * `rows` rows that the call fills completely. */
#define R2S_COL_COPY 0          /* new rows copy their source row              */
#define R2S_COL_ZERO_NEW 1      /* new rows are zero (Adam exp_avg/exp_avg_sq) */
#define R2S_COL_MEANS 2         /* split: mean +/- rotated longest axis        */
#define R2S_COL_RAW_SCALES 3    /* split: longest axis / 1.6, re-inverted      */
#define R2S_COL_RAW_OPACITIES 4 /* split: revised opacity 1 - sqrt(1 - o)      */
#define R2S_COL_PARENT 5        /* int32 parent links                          */
#define R2S_COL_LEVEL 6         /* int32 depths                                */
#define R2S_COL_HISTORY 7       /* dst = cat(src[0:history_rows], extra[sel])  */

#define R2S_DENSIFY_MAX_WIDTH 16

typedef struct r2s_column {
  const void *src;   /* [n_src, width]; for R2S_COL_HISTORY the archive     */
  void *dst;         /* [rows, width], written completely                  */
  const void *extra; /* R2S_COL_HISTORY: live column whose sel rows append */
  int64_t rows;      /* rows of dst (checked against the operation)        */
  int32_t width;     /* 4-byte words per row, 1..R2S_DENSIFY_MAX_WIDTH     */
  int32_t role;      /* R2S_COL_*                                          */
} r2s_column_t;

/* Scale activation of the model (src/models/gaussian_model.py:258-274):
 * bounded sigmoid min + (max - min) * sigmoid(raw) when sigmoid_scales != 0,
 * else exp(raw).  Per-axis bounds; repeat a scalar bound three times. */
typedef struct r2s_split_geometry {
  const float *quats;      /* [n, 4] (w, x, y, z), as stored (not normalised) */
  const float *raw_scales; /* [n, 3] */
  float scale_min[3];
  float scale_max[3];
  float scale_eps;
  int32_t sigmoid_scales;
} r2s_split_geometry_t;

/* src/strategies/binary_tree.py:93-148 split() together with
 * _append_history (:17-57) and src/utils/ops.py:61-103
 * _update_param_with_optimizer.  With rest = where(~mask) (n_rest rows) and
 * sel = where(mask) (n_sel rows), every non-history column gets
 * n_rest + 2 n_sel rows: the kept rows in `rest` order, then the children
 * [all +offset; all -offset] of the `sel` rows.  Parent rows of children are
 * history_rows + j (j = position in sel), levels level[sel] + 1.  History
 * columns get history_rows + n_sel rows.  `geometry` describes the live
 * (pre-split) quats and raw scales; it may be NULL when no column has role
 * MEANS or RAW_SCALES. */
int r2s_densify_split(const int64_t *sel, int64_t n_sel, const int64_t *rest,
                      int64_t n_rest, int64_t history_rows,
                      const r2s_split_geometry_t *geometry,
                      const r2s_column_t *columns, int32_t n_columns,
                      r2s_stream_t stream);

/* src/strategies/binary_tree.py:60-90 duplicate(): every non-history column
 * gets n + n_sel rows, the n old rows then copies of the sel rows.  Old rows
 * with mask[i] != 0 get parent history_rows + j and level + 1 (as do their
 * copies); Adam moments (R2S_COL_ZERO_NEW) of the copies are zero.  History
 * columns get history_rows + n_sel rows. */
int r2s_densify_duplicate(const uint8_t *mask, int64_t n, const int64_t *sel,
                          int64_t n_sel, int64_t history_rows,
                          const r2s_column_t *columns, int32_t n_columns,
                          r2s_stream_t stream);

/* src/strategies/binary_tree.py:151-171 remove(): every column gets the
 * n_keep rows keep = where(~mask), in order.  History columns are not
 * allowed (remove leaves the archive unchanged). */
int r2s_densify_remove(const int64_t *keep, int64_t n_keep,
                       const r2s_column_t *columns, int32_t n_columns,
                       r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Projection loss (L1 + SSIM + masked edge L1)                            */
/* ---------------------------------------------------------------------- */

/* Workspace of r2s_projection_loss_fwd/bwd: the SSIM partial-derivative
 * maps (3 floats per pixel) and per-tile sums; the forward fills it, the
 * backward reads it, so keep it between the two calls. */
int64_t r2s_projection_loss_workspace_bytes(int64_t n_images, int32_t H, int32_t W);

/* src/utils/loss.py:135-172 (BinaryTreeLossComputer.__call__, projection
 * terms) with ssim2d of src/utils/metric.py:36-54: render, target,
 * edge_target, edge_mask [n_images, H, W] float32 (one channel each; the
 * edge pair may both be NULL) ->
 * losses[3] (device) = { mean |render - target|,
 *                        1 - mean SSIM(render, target),
 *                        mean edge_mask |render - edge_target| }.
 * Gaussian window of window_size (odd, <= 15) and sigma 1.5, zero padding. */
int r2s_projection_loss_fwd_f32(const float *render, const float *target,
                                const float *edge_target, const float *edge_mask,
                                int64_t n_images, int32_t H, int32_t W,
                                int32_t window_size, float *losses, void *workspace,
                                size_t workspace_bytes, r2s_stream_t stream);

/* The VJP of the three losses above (autograd's backward of loss.py:143-172):
 * grad_scales[3] (device) = upstream gradients of the three losses ->
 * v_render [n_images, H, W].  Reads the workspace the forward filled. */
int r2s_projection_loss_bwd_f32(const float *render, const float *target,
                                const float *edge_target, const float *edge_mask,
                                int64_t n_images, int32_t H, int32_t W,
                                int32_t window_size, const float *grad_scales,
                                const void *workspace, size_t workspace_bytes,
                                float *v_render, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Volume TV regulariser                                                   */
/* ---------------------------------------------------------------------- */

/* Workspace of r2s_tv_fwd_f32 (per-block partial sums). */
int64_t r2s_tv_workspace_bytes(void);

/* src/utils/loss.py:10-21 compute_tv_loss: volume [D0, D1, D2] float32 ->
 * out[0] (device) = sum over the three axes of |v[i+1] - v[i]|, divided by
 * max(1, number of differences) when `mean` is nonzero (reduction "mean"). */
int r2s_tv_fwd_f32(const float *volume, int32_t D0, int32_t D1, int32_t D2,
                   int32_t mean, float *out, void *workspace, size_t workspace_bytes,
                   r2s_stream_t stream);

/* Its VJP (autograd's backward of loss.py:14-21): grad_out[0] (device) ->
 * v_volume [D0, D1, D2], sign(0) = 0 as torch.abs. */
int r2s_tv_bwd_f32(const float *volume, int32_t D0, int32_t D1, int32_t D2,
                   int32_t mean, const float *grad_out, float *v_volume,
                   r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Hierarchy loss                                                          */
/* ---------------------------------------------------------------------- */

/* Workspace of r2s_hierarchy_loss_fwd/bwd for n children. */
int64_t r2s_hierarchy_workspace_bytes(int64_t n);

/* src/utils/loss.py:27-71 compute_hierarchy_loss: child_means [n,3],
 * parent [n] int32 (archive indices; out-of-range = no parent),
 * history_means [h,3], parent_scales [h,3] (the archived scales already
 * activated), history_quats [h,4] with h >= history_count ->
 * out[0] (device) = mean over children with a parent of
 * relu(|diag(1/max(s,1e-6)) R^T (c - p)| - a)^2 / a^2, a = max(factor, 1e-6)
 * (0 when there is none), out[1] = that number of children.  Keep out and
 * the workspace for the backward. */
int r2s_hierarchy_loss_fwd_f32(const float *child_means, const int32_t *parent, int64_t n,
                               const float *history_means, const float *parent_scales,
                               const float *history_quats, int64_t history_count,
                               float max_parent_distance_factor, float *out,
                               void *workspace, size_t workspace_bytes,
                               r2s_stream_t stream);

/* Its VJP w.r.t. child_means: grad_out[0] (device) -> v_means [n,3]. */
int r2s_hierarchy_loss_bwd_f32(int64_t n, const float *grad_out, const float *loss_out,
                               const void *workspace, size_t workspace_bytes,
                               float *v_means, r2s_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Adam step                                                               */
/* ---------------------------------------------------------------------- */

/* One parameter tensor of an Adam step: float32 device arrays of n elements
 * and the step's scalars, computed by the caller in double as
 * torch/optim/adam.py does and rounded to float:
 *   lerp_weight = 1 - beta1, one_minus_beta2 = 1 - beta2,
 *   bias_correction2_sqrt = (1 - beta2^t)^0.5,
 *   step_size = -lr / (1 - beta1^t), t = the tensor's step count. */
typedef struct r2s_adam_tensor {
  float *param;
  const float *grad;
  float *exp_avg;
  float *exp_avg_sq;
  int64_t n;
  float lerp_weight;
  float beta2;
  float one_minus_beta2;
  float weight_decay;
  float bias_correction2_sqrt;
  float eps;
  float step_size;
} r2s_adam_tensor_t;

/* torch.optim.Adam.step (torch/optim/adam.py _multi_tensor_adam, the
 * non-capturable path) for every tensor of the list in one launch; the
 * trainer's per-group optimizers are built by
 * src/models/gaussian_model.py:514-530 and stepped by
 * src/trainers/binary_tree.py:208-210.  Updates param, exp_avg and
 * exp_avg_sq in place. */
int r2s_adam_step_f32(const r2s_adam_tensor_t *tensors, int32_t n_tensors,
                      r2s_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* R2SPLAT_HIP_H */
