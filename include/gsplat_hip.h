/*
 * gsplat_hip.h -- C ABI of libgsplat_hip.so, the MI355X (gfx950) kernels of the
 * differentiable 3D Gaussian splatting hot path.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are raw DEVICE pointers to contiguous, row-major
 *     buffers; float means IEEE fp32, masks are one byte per element (0/1).
 *   - Optional inputs/outputs are passed as NULL.
 *   - The caller owns every allocation (outputs included).  Entry points that
 *     need scratch memory take a `workspace` pointer whose size is returned by
 *     the matching *_workspace_size() query; the library clears what it needs
 *     inside the workspace itself, on `stream`.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *     null stream).  Nothing synchronises the host unless stated.
 *   - Every entry point returns GSPLAT_OK (0) or a negative error code; the
 *     message of the last failure on the calling thread is available from
 *     gsplat_last_error().  Argument errors are detected before anything is
 *     enqueued.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the mc8max/gsplat 1.5.3 source tree).
 */
#ifndef GSPLAT_HIP_H
#define GSPLAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *gsplat_stream_t;

enum {
    GSPLAT_OK = 0,
    GSPLAT_ERR_INVALID_ARGUMENT = -1,
    GSPLAT_ERR_UNSUPPORTED = -2,
    GSPLAT_ERR_LAUNCH = -3,
    GSPLAT_ERR_WORKSPACE = -4,
};

/* Camera models; values match gsplat::CameraModelType
 * (gsplat/cuda/include/Common.h:65-71, exposed as _C.CameraModelType,
 * gsplat/cuda/ext.cpp:38-44).  PINHOLE and ORTHO are implemented. */
enum {
    GSPLAT_CAMERA_PINHOLE = 0,
    GSPLAT_CAMERA_ORTHO = 1,
    GSPLAT_CAMERA_FISHEYE = 2,
};

/* Message of the last failed call on this thread ("" if none). */
const char *gsplat_last_error(void);

/* Library version string, e.g. "gsplat_hip 0.1.0 gfx950". */
const char *gsplat_version(void);

/* Identity of the interface the library was built from: 16 hex digits of
 * SHA-256 over this header's declarations (comments and whitespace removed;
 * gsplat_amd/abi.py:header_abi_hash).  A binding compares it with the digest
 * of the header it was written against and refuses a library that differs,
 * before binding any entry point.  No counterpart in the reference, whose op
 * schemas are compiled into the same module as its kernels
 * (gsplat/cuda/ext.cpp:711-808), so its callers cannot disagree with them. */
const char *gsplat_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Projection (EWA splatting of 3D Gaussians to 2D conics).                  */
/* ------------------------------------------------------------------------ */

/* Camera-space projection of B*C*N Gaussians given by mean and full 3x3
 * covariance (no culling, no eps2d): means2d = the pinhole (or orthographic)
 * projection of the mean, covars2d = J S J^T with the projection's Jacobian
 * J, the pinhole one evaluated with x/z and y/z clamped to 1.3x the field of
 * view.  camera_model: PINHOLE or ORTHO (others return
 * GSPLAT_ERR_UNSUPPORTED).
 * Replaces projection_ewa_simple_fwd
 *   (gsplat/cuda/csrc/Projection.cpp:41-80,
 *    gsplat/cuda/csrc/ProjectionEWASimple.cu:37-138; the probe of has_3dgs(),
 *    gsplat/cuda/_wrapper.py:181-184).
 * Inputs : means [B,C,N,3], covars [B,C,N,3,3], Ks [B,C,3,3].
 * Outputs: means2d [B,C,N,2], covars2d [B,C,N,2,2]. */
int gsplat_projection_simple_fwd(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *Ks, int32_t image_width, int32_t image_height, int32_t camera_model,
    float *means2d, float *covars2d, gsplat_stream_t stream);

/* Vector-Jacobian product of gsplat_projection_simple_fwd.
 * Replaces projection_ewa_simple_bwd
 *   (gsplat/cuda/csrc/Projection.cpp:82-127,
 *    gsplat/cuda/csrc/ProjectionEWASimple.cu:140-262).
 * Inputs : the forward's inputs, v_means2d [B,C,N,2], v_covars2d [B,C,N,2,2].
 * Outputs: v_means [B,C,N,3], v_covars [B,C,N,3,3] (every element written). */
int gsplat_projection_simple_bwd(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *Ks, int32_t image_width, int32_t image_height, int32_t camera_model,
    const float *v_means2d, const float *v_covars2d, float *v_means, float *v_covars,
    gsplat_stream_t stream);

/* Dense ("fused") projection of B*C*N rows.
 * Replaces projection_ewa_3dgs_fused_fwd
 *   (gsplat/cuda/csrc/Projection.cpp:129-200,
 *    gsplat/cuda/csrc/ProjectionEWA3DGSFused.cu:38-312).
 * Inputs : means [B,N,3]; either covars [B,N,6] (upper triangle) or
 *          quats [B,N,4] + scales [B,N,3]; opacities [B,N] (optional, enables
 *          the opacity-aware radius); viewmats [B,C,4,4]; Ks [B,C,3,3].
 * Outputs: radii [B,C,N,2] int32 (0,0 for culled rows), means2d [B,C,N,2],
 *          depths [B,C,N], conics [B,C,N,3], compensations [B,C,N] (optional;
 *          non-NULL also folds the compensation into the opacity cull).
 *          Culled rows get radii = 0 and zeros in every float output. */
int gsplat_projection_fused_fwd(
    int64_t B, int64_t C, int64_t N,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *opacities,
    const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height,
    float eps2d, float near_plane, float far_plane, float radius_clip,
    int32_t camera_model,
    int32_t *radii, float *means2d, float *depths, float *conics,
    float *compensations,
    gsplat_stream_t stream);

/* Backward of the dense projection.
 * Replaces projection_ewa_3dgs_fused_bwd
 *   (gsplat/cuda/csrc/Projection.cpp:202-306,
 *    gsplat/cuda/csrc/ProjectionEWA3DGSFused.cu:316-650).
 * Gradients are OVERWRITTEN (not accumulated): v_means [B,N,3]; v_covars
 * [B,N,6] or v_quats [B,N,4] + v_scales [B,N,3]; v_viewmats [B,C,4,4]
 * (optional).  Each Gaussian is owned by one thread that loops over the C
 * cameras, so no atomics are used and results are deterministic. */
int gsplat_projection_fused_bwd(
    int64_t B, int64_t C, int64_t N,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model,
    const int32_t *radii, const float *conics, const float *compensations,
    const float *v_means2d, const float *v_depths, const float *v_conics,
    const float *v_compensations,
    float *v_means, float *v_covars, float *v_quats, float *v_scales,
    float *v_viewmats,
    gsplat_stream_t stream);

/* Bytes of workspace gsplat_projection_packed_fwd needs for B*C*N rows. */
size_t gsplat_projection_packed_workspace_size(int64_t B, int64_t C, int64_t N);

/* Packed projection in ONE pass: rows that survive culling are compacted in
 * (b, c, g) row-major order with a decoupled look-back scan.
 * Replaces projection_ewa_3dgs_packed_fwd, whose two passes + host sync this
 * fuses (gsplat/cuda/csrc/Projection.cpp:308-437,
 *        gsplat/cuda/csrc/ProjectionEWA3DGSPacked.cu:39-398).
 * Every per-row output must have capacity for B*C*N rows; the number of rows
 * written (nnz) is stored to nnz_out (one int64 in device memory or in pinned
 * host memory from hipHostMalloc, which the device writes directly: the host
 * then reads it after the stream's next event, with no copy).  indptr [B*C+1]
 * int32;
 * batch_ids, camera_ids, gaussian_ids int64.  row_of [B*C*N] int32
 * (optional) receives, for every (b, c, g), its packed row or -1: the inverse
 * of (batch_ids, camera_ids, gaussian_ids), used by the gathers below.
 * row_opacities [B*C*N] (optional, needs opacities) receives each row's
 * opacities[b, g], the reference's opacities[batch_ids, gaussian_ids]
 * (gsplat/rendering.py:782). */
int gsplat_projection_packed_fwd(
    int64_t B, int64_t C, int64_t N,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *opacities,
    const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height,
    float eps2d, float near_plane, float far_plane, float radius_clip,
    int32_t camera_model,
    void *workspace, size_t workspace_bytes,
    int32_t *indptr, int64_t *batch_ids, int64_t *camera_ids,
    int64_t *gaussian_ids, int32_t *radii, float *means2d, float *depths,
    float *conics, float *compensations, int64_t *nnz_out, int32_t *row_of,
    float *row_opacities, gsplat_stream_t stream);

/* Allocation-free variant of gsplat_projection_packed_fwd, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, outputs and results as gsplat_projection_packed_fwd without
 * the workspace: the look-back scratch is a static device array of
 * 256 + 65536 * 8 bytes (512 KiB) per GPU, held until the process ends, so
 * B*C*N may be at most gsplat_projection_packed_fwd_noalloc_max_rows()
 * (65536 workgroups of 4096 rows = 268,435,456 rows); larger inputs return
 * GSPLAT_ERR_WORKSPACE.  Calls no hipMalloc/hipFree.  The scratch is shared
 * by every call on one GPU and cleared by each call before use: calls that
 * overlap on one GPU (concurrent streams or host threads) race. */
int gsplat_projection_packed_fwd_noalloc(
    int64_t B, int64_t C, int64_t N,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *opacities,
    const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height,
    float eps2d, float near_plane, float far_plane, float radius_clip,
    int32_t camera_model,
    int32_t *indptr, int64_t *batch_ids, int64_t *camera_ids,
    int64_t *gaussian_ids, int32_t *radii, float *means2d, float *depths,
    float *conics, float *compensations, int64_t *nnz_out, int32_t *row_of,
    float *row_opacities, gsplat_stream_t stream);

/* Largest B*C*N that gsplat_projection_packed_fwd_noalloc accepts. */
int64_t gsplat_projection_packed_fwd_noalloc_max_rows(void);

/* Backward of the packed projection over nnz rows.
 * Replaces projection_ewa_3dgs_packed_bwd
 *   (gsplat/cuda/csrc/Projection.cpp:439-576,
 *    gsplat/cuda/csrc/ProjectionEWA3DGSPacked.cu:400-783).
 * sparse_grad != 0: v_means [nnz,3], v_covars [nnz,6] / v_quats [nnz,4] +
 *   v_scales [nnz,3] are written row by row (no zero fill needed).
 * sparse_grad == 0: the per-Gaussian outputs [B,N,*] must be zero-filled by
 *   the caller; rows are accumulated with atomics unless B*C == 1, in which
 *   case each Gaussian has at most one row and plain stores are used.
 * v_viewmats [B,C,4,4] (optional) must be zero-filled by the caller. */
int gsplat_projection_packed_bwd(
    int64_t B, int64_t C, int64_t N, int64_t nnz,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model,
    const int64_t *batch_ids, const int64_t *camera_ids,
    const int64_t *gaussian_ids, const float *conics,
    const float *compensations,
    const float *v_means2d, const float *v_depths, const float *v_conics,
    const float *v_compensations, int32_t sparse_grad,
    float *v_means, float *v_covars, float *v_quats, float *v_scales,
    float *v_viewmats,
    gsplat_stream_t stream);

/* Backward of the packed projection driven by Gaussian: one thread per
 * (b, g) sums the gradients of its packed rows row_of[(b C + c) N + g]
 * (>= 0; the map written by gsplat_projection_packed_fwd) over the C
 * cameras and writes every dense gradient row once -- v_means [B,N,3],
 * v_covars [B,N,6] or v_quats [B,N,4] + v_scales [B,N,3], zeros for
 * Gaussians visible nowhere -- so the caller needs no zero fill and no
 * atomics are used.  v_depths and v_means may be NULL (zero gradient / not
 * wanted).  v_viewmats [B,C,4,4] (optional) must be zero-filled.
 * Same result as gsplat_projection_packed_bwd with sparse_grad == 0
 * (gsplat/cuda/csrc/Projection.cpp:439-576); used by rasterization() where
 * the row map is at hand.  Optional: v_row_opacities [nnz] with v_opacities
 * [B,N] receives each Gaussian's sum over its rows (the backward of the
 * row opacity gather), and v_means_add [B,N,3] is added to v_means (e.g.
 * the SH direction term); both are written densely. */
int gsplat_projection_packed_bwd_rows(
    int64_t B, int64_t C, int64_t N,
    const float *means, const float *covars, const float *quats,
    const float *scales, const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *row_of,
    const float *conics, const float *compensations,
    const float *v_means2d, const float *v_depths, const float *v_conics,
    const float *v_compensations,
    float *v_means, float *v_covars, float *v_quats, float *v_scales,
    float *v_viewmats, const float *v_row_opacities, float *v_opacities,
    const float *v_means_add,
    gsplat_stream_t stream);

/* gsplat_projection_packed_bwd_rows with the densification statistics of
 * DefaultStrategy._update_state (gsplat/strategy/default.py:235-268) in the
 * same pass, for one batch (B == 1): for every packed row r of Gaussian g,
 *   grad2d[g] += || (stat_grads[r,0] * stat_scale_x, stat_grads[r,1] * stat_scale_y) ||
 *   count[g]  += 1
 * stat_grads [nnz,2] are the rows' 2D mean gradients (absgrad or grad),
 * stat_scale_x/y = W/2 * C and H/2 * C; grad2d [N] and count [N] accumulate
 * in place.  Replaces the separate statistics pass (gsplat_grad2d_stats)
 * after the backward. */
int gsplat_projection_packed_bwd_rows_stats(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats, const float *Ks,
    int32_t image_width, int32_t image_height, float eps2d, int32_t camera_model,
    const int32_t *row_of, const float *conics, const float *compensations,
    const float *v_means2d, const float *v_depths, const float *v_conics,
    const float *v_compensations, float *v_means, float *v_covars, float *v_quats,
    float *v_scales, float *v_viewmats, const float *v_row_opacities,
    float *v_opacities, const float *v_means_add, const float *stat_grads,
    float stat_scale_x, float stat_scale_y, float *grad2d, float *count,
    gsplat_stream_t stream);

/* Covariance and/or precision matrices from quaternions and scales.
 * Replaces quat_scale_to_covar_preci_fwd
 *   (gsplat/cuda/csrc/QuatScaleToCovar.cpp:37-72,
 *    QuatScaleToCovarCUDA.cu:37-146).
 * quats [N,4] (w,x,y,z, any norm), scales [N,3]; covars = R S^2 R^T and
 * precis = R S^-2 R^T, each optional (NULL: not computed), [N,6] upper
 * triangle (xx, xy, xz, yy, yz, zz) when triu != 0, else [N,3,3]. */
int gsplat_quat_scale_to_covar_preci_fwd(
    int64_t N, const float *quats, const float *scales, int32_t triu,
    float *covars, float *precis, gsplat_stream_t stream);

/* Backward of the above.  Replaces quat_scale_to_covar_preci_bwd
 *   (QuatScaleToCovar.cpp:74-110, QuatScaleToCovarCUDA.cu:150-287).
 * v_covars / v_precis optional (NULL: zero gradient), same layout as the
 * forward's outputs; v_quats [N,4] and v_scales [N,3] are fully written. */
int gsplat_quat_scale_to_covar_preci_bwd(
    int64_t N, const float *quats, const float *scales, int32_t triu,
    const float *v_covars, const float *v_precis, float *v_quats,
    float *v_scales, gsplat_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Spherical harmonics (real SH, Sloan 2013 basis, degree 0..4).             */
/* ------------------------------------------------------------------------ */

/* Replaces spherical_harmonics_fwd
 *   (gsplat/cuda/csrc/SphericalHarmonics.cpp:33-55,
 *    gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:391-462).
 * dirs [M,3] (need not be unit length), coeffs [M,K,3], masks [M] (optional),
 * colors [M,3].  Masked-out rows are written as 0. */
int gsplat_sh_fwd(
    int64_t M, int32_t K, int32_t degree,
    const float *dirs, const float *coeffs, const uint8_t *masks,
    float *colors, gsplat_stream_t stream);

/* Replaces spherical_harmonics_bwd
 *   (gsplat/cuda/csrc/SphericalHarmonics.cpp:57-91,
 *    gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:465-552).
 * v_coeffs [M,K,3] is fully written (bands above `degree` and masked rows get
 * 0, so no zero fill is needed); v_dirs [M,3] optional, fully written. */
int gsplat_sh_bwd(
    int64_t M, int32_t K, int32_t degree,
    const float *dirs, const float *coeffs, const uint8_t *masks,
    const float *v_colors, float *v_coeffs, float *v_dirs,
    gsplat_stream_t stream);

/* SH colour of every packed row, driven by Gaussian (fuses the gathers the
 * packed path of rasterization() performs before SH).
 * Replaces, for packed rows, compute_directions + normalize_features_layout
 * + spherical_harmonics + clamp_min(colors + 0.5, 0)
 *   (gsplat/rendering.py:227-253, 170-213, 845-873;
 *    gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:391-462).
 * means [B,N,3], viewmats [B,C,4,4] (world->camera; the camera centre
 * -R^T t is taken from them), coeffs [B,N,K,3],
 * row_of [B,C,N] (packed row of (b,c,g) or -1, from
 * gsplat_projection_packed_fwd); writes colors [nnz,3] =
 * max(SH(normalize(mean - centre)) + 0.5, 0) for every packed row. */
int gsplat_sh_rows_fwd(
    int64_t B, int64_t C, int64_t N, int32_t K, int32_t degree,
    const float *means, const float *viewmats, const float *coeffs,
    const int32_t *row_of, float *colors, gsplat_stream_t stream);

/* Backward of gsplat_sh_rows_fwd.  Replaces spherical_harmonics_bwd plus
 * the index_put scatters of the coefficient and direction gradients
 *   (gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:465-552;
 *    autograd of gsplat/rendering.py:95-213).
 * v_colors [nnz,3]; v_coeffs [B,N,K,3] and v_means [B,N,3] are fully
 * written (zeros for Gaussians visible nowhere), summed over cameras in
 * camera order (deterministic). */
int gsplat_sh_rows_bwd(
    int64_t B, int64_t C, int64_t N, int32_t K, int32_t degree,
    const float *means, const float *viewmats, const float *coeffs,
    const int32_t *row_of, const float *v_colors, float *v_coeffs,
    float *v_means, gsplat_stream_t stream);

/* gsplat_sh_rows_bwd and gsplat_projection_packed_bwd_rows_stats in one
 * launch, for rasterization()'s packed front end: every workgroup runs the
 * SH backward of its 256 Gaussians (v_coeffs [B,N,K,3], fully written),
 * keeps each Gaussian's direction term of dL/dmean in registers, then runs
 * their geometry backward and adds that term to v_means (required).  The
 * results equal the two calls with the SH call's v_means passed as
 * v_means_add.  No view-matrix gradients; the statistics buffers
 * (stat_grads, grad2d, count) are all NULL or all given (one batch).
 * Replaces the backward of the packed rows' SH evaluation and of
 * projection_ewa_3dgs_packed (SphericalHarmonicsCUDA.cu:465-552,
 * Projection.cpp:439-576). */
int gsplat_projection_packed_bwd_rows_sh(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats,
    const float *Ks, int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *row_of, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, float *v_means,
    float *v_covars, float *v_quats, float *v_scales, const float *v_row_opacities,
    float *v_opacities, const float *stat_grads, float stat_scale_x,
    float stat_scale_y, float *grad2d, float *count, int32_t K, int32_t degree,
    const float *coeffs, const float *v_colors, float *v_coeffs,
    gsplat_stream_t stream);

/* out[row_of[b,c,g]] = src[b,g] for every packed row: the per-Gaussian
 * feature gather of the packed path (opacities / colours,
 * gsplat/rendering.py:782, 170-213).  src [B,N,F], out [nnz,F]. */
int gsplat_rows_gather(
    int64_t B, int64_t C, int64_t N, int32_t F, const float *src,
    const int32_t *row_of, float *out, gsplat_stream_t stream);

/* v_src[b,g] = sum over c of v_out[row_of[b,c,g]] (rows that exist): the
 * gradient of gsplat_rows_gather, replacing the autograd index_put of the
 * reference's gathers.  v_src [B,N,F] is fully written. */
int gsplat_rows_scatter_sum(
    int64_t B, int64_t C, int64_t N, int32_t F, const int32_t *row_of,
    const float *v_out, float *v_src, gsplat_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Tile intersection.                                                        */
/* ------------------------------------------------------------------------ */

/* Bytes of workspace gsplat_isect_count needs for n rows. */
size_t gsplat_isect_count_workspace_size(int64_t n);

/* Pass 1 of intersect_tile: tiles touched per row, plus the inclusive prefix
 * sum of those counts (one pass, decoupled look-back).
 * Replaces the first launch of intersect_tile_kernel and the at::cumsum in
 *   gsplat/cuda/csrc/Intersect.cpp:80-104, kernel IntersectTile.cu:133-288.
 * Rows: n = I*N (dense, image id = row / N) or nnz (packed, image_ids given).
 * conics [n,3] + opacities [n] both non-NULL select the ellipse ("AccuTile")
 * test, otherwise the axis-aligned box of `radii` is used.
 * Outputs tiles_per_gauss [n] int32 and cum_tiles [n] int64 (inclusive). */
int gsplat_isect_count(
    int64_t n, int64_t N, const int64_t *image_ids,
    const float *means2d, const int32_t *radii,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    void *workspace, size_t workspace_bytes,
    int32_t *tiles_per_gauss, int64_t *cum_tiles,
    gsplat_stream_t stream);

/* Pass 2 of intersect_tile: writes isect_ids [n_isects] (image|tile|depth
 * bits) and flatten_ids [n_isects] in row order, each row at
 * cum_tiles[row-1].  Same row/camera arguments as gsplat_isect_count.
 * Replaces the second launch of intersect_tile_kernel
 *   (gsplat/cuda/csrc/Intersect.cpp:118-143). */
int gsplat_isect_emit(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int64_t *cum_tiles,
    int64_t *isect_ids, int32_t *flatten_ids,
    gsplat_stream_t stream);

/* Sorted intersection, stage 1 of 2.  Counts the tiles of every row
 * (tiles_per_gauss [n]), orders the rows stably by their depth bits (ties by
 * row) -- depth_order [n] int32,
 * the rows in that order -- and gives every depth position its first slot:
 * depth_starts [n + 1] int64, the tile count of all rows before it in depth
 * order (depth_starts[n] = n_isects, also written to n_isects_out, device
 * int64) -- and packs every row's sweep inputs into row_records [n, 8] float
 * (16-byte aligned) for stage 2.  Same row/camera arguments as
 * gsplat_isect_count.
 * Together with stage 2 this replaces intersect_tile with sort=True
 *   (gsplat/cuda/csrc/Intersect.cpp:33-164: count, cumsum, emit, and the
 *    full-key radix sort of IntersectTile.cu:478-520). */
size_t gsplat_isect_prepare_workspace_size(int64_t n);
int gsplat_isect_prepare(
    int64_t n, int64_t N, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    void *workspace, size_t workspace_bytes, int32_t *tiles_per_gauss,
    int32_t *depth_order, int64_t *depth_starts, float *row_records,
    int64_t *n_isects_out, gsplat_stream_t stream);

/* Sorted intersection, stage 2 of 2.  Writes the intersections of the rows
 * in depth order (depth_order, depth_starts, row_records from stage 1) --
 * every row's
 * tiles at its depth-ordered slots -- then sorts them stably on the
 * image|tile key bits only.  The result equals the reference's full-key
 * stable sort of the row-order emission bit for bit: isect_ids [n_isects]
 * ascending, ties (same image, tile and depth bits) by row; flatten_ids
 * [n_isects] the rows. */
size_t gsplat_isect_emit_sorted_workspace_size(int64_t n_isects);
int gsplat_isect_emit_sorted(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *depth_order, const int64_t *depth_starts,
    const float *row_records, int64_t n_isects,
    void *workspace, size_t workspace_bytes,
    int64_t *isect_ids, int32_t *flatten_ids, gsplat_stream_t stream);

/* Stage 2 with the intersection count read on the device
 * (depth_starts[n], written by stage 1), so the caller can queue it right
 * behind stage 1 without waiting for the count on the host.  Same inputs
 * as gsplat_isect_emit_sorted, with `capacity` in place of n_isects:
 * isect_ids and flatten_ids hold capacity entries, the workspace is
 * gsplat_isect_emit_sorted_workspace_size(capacity), and the first
 * min(n_isects, capacity) entries are written.  When n_isects <= capacity
 * they equal gsplat_isect_emit_sorted's output; otherwise the caller must
 * run gsplat_isect_emit_sorted with room for n_isects.  No reference
 * counterpart: the reference reads the count on the host between the two
 * stages (gsplat/cuda/csrc/Intersect.cpp:104-122). */
int gsplat_isect_emit_sorted_dev(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *depth_order, const int64_t *depth_starts,
    const float *row_records, int64_t capacity,
    void *workspace, size_t workspace_bytes,
    int64_t *isect_ids, int32_t *flatten_ids, gsplat_stream_t stream);

/* Tile-first sorted intersection, stage 1 of 2 (the form rasterization()
 * uses).  Counts the tiles of every row (tiles_per_gauss [n]), gives every
 * row its first slot in row order -- row_starts [n + 1] int64, the tile
 * count of all rows before it (row_starts[n] = n_isects, also written to
 * n_isects_out: one int64 in device or pinned host memory, as nnz_out of
 * gsplat_projection_packed_fwd) -- and packs every row's sweep inputs into
 * row_records [n, 8] float (16-byte aligned) for stage 2.  Same row/camera
 * arguments as gsplat_isect_count; the workspace is
 * gsplat_isect_prepare_rows_workspace_size(n) bytes.
 * Together with stage 2 this replaces intersect_tile with sort=True and
 * intersect_offset (gsplat/cuda/csrc/Intersect.cpp:33-164: count, cumsum,
 * emit, the full-key radix sort of IntersectTile.cu:478-520, and the offset
 * encoding of IntersectTile.cu:391-439). */
size_t gsplat_isect_prepare_rows_workspace_size(int64_t n);
int gsplat_isect_prepare_rows(
    int64_t n, int64_t N, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    void *workspace, size_t workspace_bytes, int32_t *tiles_per_gauss,
    int64_t *row_starts, float *row_records, int64_t *n_isects_out,
    gsplat_stream_t stream);

/* Stage 1 split in two launches with the SH colours of the packed rows in
 * the first: gsplat_sh_rows_fwd's colours and the tile counts, in-workgroup
 * count prefixes and sweep records of gsplat_isect_prepare_rows, computed by
 * one launch whose workgroups alternate between the two kinds (the colour
 * rows wait on memory, the tile sweep on arithmetic, so the CUs run both at
 * once).  It replaces the SH evaluation of the packed rows
 * (gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:391-462, called from
 * rendering.py:845-873) and the count pass of Intersect.cpp:79-101.
 * Colour arguments as gsplat_sh_rows_fwd.  The intersection rows are the
 * first *n_dev of n_cap (n_dev: one int32 in device memory, such as the
 * packed projection's indptr[B*C]; n_cap <= B*C*N sizes every row buffer);
 * image_ids as gsplat_isect_prepare_rows (NULL for one image).  The
 * workspace (gsplat_isect_prepare_rows_workspace_size(n_cap) bytes) then goes
 * unchanged to gsplat_isect_row_starts, which finishes row_starts. */
int gsplat_sh_rows_fwd_isect_count(
    int64_t B, int64_t C, int64_t N, int32_t K, int32_t degree, const float *means,
    const float *viewmats, const float *coeffs, const int32_t *row_of, float *colors,
    int64_t n_cap, const int32_t *n_dev, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, void *workspace, size_t workspace_bytes,
    int32_t *tiles_per_gauss, int64_t *row_starts, float *row_records,
    gsplat_stream_t stream);

/* The second launch of that split: row_starts [n + 1] and *n_isects_out for
 * the n rows (= *n_dev) gsplat_sh_rows_fwd_isect_count counted, as
 * gsplat_isect_prepare_rows writes them (the cumsum of Intersect.cpp:104-105). */
int gsplat_isect_row_starts(
    int64_t n, const void *workspace, size_t workspace_bytes, int64_t *row_starts,
    int64_t *n_isects_out, gsplat_stream_t stream);

/* Tile-first sorted intersection, stage 2 of 2.  Writes every row's tiles at
 * its row-order slots (row_starts, row_records from stage 1), sorts the
 * intersections stably on the image|tile bits, then sorts every tile's rows
 * stably on their depth bits (one workgroup per tile; in LDS up to 4,096
 * rows, through the output buffers above that).  isect_ids [n_isects] and
 * flatten_ids [n_isects] equal the reference's full-key stable sort of the
 * row-order emission bit for bit; offsets [I, tile_height, tile_width] int32
 * (fully written) is the first intersection of every tile, as
 * gsplat_isect_offsets would compute it from isect_ids. */
size_t gsplat_isect_emit_tiles_workspace_size(int64_t n_isects);
int gsplat_isect_emit_tiles(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int64_t *row_starts, const float *row_records, int64_t n_isects,
    void *workspace, size_t workspace_bytes,
    int64_t *isect_ids, int32_t *flatten_ids, int32_t *offsets,
    gsplat_stream_t stream);

/* Stage 2 with the intersection count read on the device (row_starts[n]),
 * so it can be queued behind stage 1 before the host knows the count:
 * `capacity` in place of n_isects sizes isect_ids, flatten_ids and the
 * workspace, and the first min(n_isects, capacity) entries are written (with
 * the offsets of those).  When n_isects <= capacity they equal
 * gsplat_isect_emit_tiles' output; otherwise the caller must run
 * gsplat_isect_emit_tiles with room for n_isects.  No reference
 * counterpart: the reference reads the count on the host between the two
 * stages (gsplat/cuda/csrc/Intersect.cpp:104-122). */
int gsplat_isect_emit_tiles_dev(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int64_t *row_starts, const float *row_records, int64_t capacity,
    void *workspace, size_t workspace_bytes,
    int64_t *isect_ids, int32_t *flatten_ids, int32_t *offsets,
    gsplat_stream_t stream);

/* Bytes of workspace gsplat_sort_pairs_u64_u32 needs for n pairs. */
size_t gsplat_sort_pairs_workspace_size(int64_t n);

/* Stable LSD radix sort of (key, value) pairs on key bits [0, num_bits).
 * Results land in keys_out/vals_out; the inputs are used as ping-pong
 * buffers and are clobbered.  Replaces radix_sort_double_buffer
 *   (gsplat/cuda/csrc/IntersectTile.cu:478-520, cub::DeviceRadixSort). */
int gsplat_sort_pairs_u64_u32(
    int64_t n, int32_t num_bits,
    uint64_t *keys_in, uint32_t *vals_in,
    uint64_t *keys_out, uint32_t *vals_out,
    void *workspace, size_t workspace_bytes,
    gsplat_stream_t stream);

/* Tile start offsets: offsets[i*n_tiles + t] = #{k : isect_ids[k] >> 32 <
 * (i << tile_n_bits | t)}; all zeros when n_isects == 0.
 * Replaces intersect_offset (gsplat/cuda/csrc/Intersect.cpp:320-337,
 *   kernel IntersectTile.cu:391-474). */
int gsplat_isect_offsets(
    int64_t n_isects, const int64_t *isect_ids, int64_t I,
    int32_t tile_width, int32_t tile_height, int32_t *offsets,
    gsplat_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Tile rasterizer.                                                          */
/* ------------------------------------------------------------------------ */

/* Front-to-back alpha compositing, one workgroup per tile.
 * Replaces rasterize_to_pixels_3dgs_fwd
 *   (gsplat/cuda/csrc/Rasterization.cpp:42-120,
 *    gsplat/cuda/csrc/RasterizeToPixels3DGSFwd.cu:41-302).
 * Rows: n_rows = I*N (dense) or nnz (packed); means2d [n,2], conics [n,3],
 * colors [n,CDIM], opacities [n]; backgrounds [I,CDIM] and masks
 * [I,tile_height,tile_width] optional; tile_offsets [I,th,tw];
 * flatten_ids [n_isects].
 * Outputs: render_colors [I,H,W,CDIM], render_alphas [I,H,W],
 *          last_ids [I,H,W] int32, render_transmittance [I,H,W] (optional:
 *          the final transmittance T = 1 - alpha of each pixel, kept at full
 *          precision for the backward).
 * CDIM in {1,2,3,4,5,8,9,16,17,32,33}; tile_size in {4,8,16}. */
int gsplat_rasterize_fwd(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    float *render_colors, float *render_alphas, int32_t *last_ids,
    float *render_transmittance, gsplat_stream_t stream);

/* Back-to-front replay of the compositing.
 * Replaces rasterize_to_pixels_3dgs_bwd
 *   (gsplat/cuda/csrc/Rasterization.cpp:122-214,
 *    gsplat/cuda/csrc/RasterizeToPixels3DGSBwd.cu:39-412).
 * render_transmittance (optional) is the forward's final T per pixel; when
 * NULL, T is taken as 1 - render_alphas as the reference does, which loses
 * relative precision for pixels that end near the 1e-4 cutoff.
 * v_render_alphas may be NULL (a zero alpha gradient).
 * Gradient outputs are ACCUMULATED and must be zero-filled by the caller:
 * v_means2d [n,2], v_conics [n,3], v_colors [n,CDIM], v_opacities [n],
 * v_means2d_abs [n,2] (optional; sum over pixels of |dL/dmean2d|).
 * tile_counter (optional, one uint32, zero on entry): when given, a grid of
 * the workgroups that fit on the device takes the tiles one after another
 * from it (no partial last round); NULL launches one workgroup per tile. */
int gsplat_rasterize_bwd(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    const float *render_alphas, const float *render_transmittance,
    const int32_t *last_ids,
    const float *v_render_colors, const float *v_render_alphas,
    float *v_means2d_abs, float *v_means2d, float *v_conics,
    float *v_colors, float *v_opacities, uint32_t *tile_counter,
    gsplat_stream_t stream);

/* Replay state for a backward that runs one unit per forward batch instead
 * of one per tile.  Pair of gsplat_rasterize_fwd / gsplat_rasterize_bwd: the
 * reference runs rasterize_to_pixels_3dgs_fwd then _bwd
 * (gsplat/cuda/_wrapper.py:1709-1836) with the backward replaying each tile
 * back to front from its end; these two keep that arithmetic but split each
 * tile's replay at the forward's batch boundaries (tile_size^2 consecutive
 * intersections of the tile), so the parts of one tile run in parallel.
 *
 * gsplat_rasterize_replay_size: bytes of the replay workspace (256-byte
 *   aligned) for these sizes; 0 for invalid sizes.  It holds, per batch
 *   boundary of every tile, each pixel's transmittance there and the colour
 *   the next batch composited (4 * (1 + CDIM) bytes per pixel per
 *   boundary), and the list of (tile, batch) units up to each tile's last
 *   contributor.
 * gsplat_rasterize_fwd_replay: gsplat_rasterize_fwd (render_transmittance
 *   required) that also fills the replay workspace.
 * gsplat_rasterize_bwd_replay: gsplat_rasterize_bwd with
 *   render_transmittance, tile_counter and the replay workspace of the
 *   forward call on the same inputs all required (render_alphas is not
 *   needed).  The gradients agree with gsplat_rasterize_bwd's to float32
 *   summation order.
 * expected_depth_channel (-1 for none; no counterpart in the reference op,
 *   whose caller does this in torch, gsplat/rendering.py:1259-1267): the
 *   forward writes that colour channel divided by max(alpha, 1e-10), the
 *   expected depth of render modes ED and RGB+ED, into render_colors and
 *   (when expected_depth is not NULL) into expected_depth [I,H,W]; the
 *   backward, given that expected_depth and the same channel, takes
 *   v_render_colors as the gradient of the divided output, adding the
 *   division's alpha term to the alpha gradient.  The caller keeps only the
 *   one channel for the backward, not the returned render.
 * zero_fill, zero_fill_count (NULL, 0 for none; no counterpart in the
 *   reference): a float buffer the forward launch also sets to zero, for
 *   the gradient accumulators gsplat_rasterize_bwd_replay adds into, so
 *   that no fill runs between the forward and the backward.
 * color_last (NULL for none; no counterpart in the reference, whose caller
 *   concatenates a depth channel to the colours with torch,
 *   gsplat/rendering.py:1025-1045): the last of the cdim channels kept
 *   apart, colors then holding cdim - 1 channels per row (NULL when cdim is
 *   1) and color_last [n_rows] the last one; the backward then writes that
 *   channel's gradient to v_color_last [n_rows] and the others to v_colors
 *   [n_rows, cdim - 1].  The outputs equal those of the concatenated rows
 *   bit for bit. */
size_t gsplat_rasterize_replay_size(
    int64_t I, int32_t tile_width, int32_t tile_height, int32_t tile_size,
    int64_t n_isects, int32_t cdim);

int gsplat_rasterize_fwd_replay(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *color_last,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    float *render_colors, float *render_alphas, int32_t *last_ids,
    float *render_transmittance, void *replay, size_t replay_bytes,
    int32_t expected_depth_channel, float *expected_depth, float *zero_fill,
    int64_t zero_fill_count, gsplat_stream_t stream);

int gsplat_rasterize_bwd_replay(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *color_last,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    const float *render_transmittance, const int32_t *last_ids,
    const float *v_render_colors, const float *v_render_alphas,
    float *v_means2d_abs, float *v_means2d, float *v_conics,
    float *v_colors, float *v_color_last, float *v_opacities,
    uint32_t *tile_counter,
    const void *replay, size_t replay_bytes, const float *expected_depth,
    int32_t expected_depth_channel, gsplat_stream_t stream);

/* Rasterize to indices: the (Gaussian, pixel) pairs each pixel composites
 * over the isect batches [range_start, range_end) of its tile (batches of
 * tile_size^2, front to back), starting from the pixel's transmittance
 * transmittances [I,H,W].  Replaces rasterize_to_indices_3dgs
 *   (gsplat/cuda/csrc/Rasterization.cpp:216-308,
 *    RasterizeToIndices3DGS.cu:36-271) in two steps around the one host
 * read of the pair count, as the reference:
 *  1. ..._count writes chunk_cnts [I*H*W] (pairs per pixel), chunk_starts
 *     [I*H*W] (exclusive prefix) and n_elems (device int64, the total);
 *     workspace of gsplat_rasterize_to_indices_workspace_size(I*H*W) bytes.
 *  2. ..._write writes gaussian_ids [n_elems] (row % N) and pixel_ids
 *     [n_elems] (image * H * W + i * W + j), pixel-major, front to back.
 * Rows: means2d [I*N,2], conics [I*N,3], opacities [I*N] (or packed rows with
 * I = 1, N = nnz).  Decisions are those of gsplat_rasterize_fwd. */
size_t gsplat_rasterize_to_indices_workspace_size(int64_t n_pixels);
int gsplat_rasterize_to_indices_count(
    int64_t range_start, int64_t range_end, int64_t I, int64_t N,
    int64_t n_isects, const float *transmittances, const float *means2d,
    const float *conics, const float *opacities, int32_t image_width,
    int32_t image_height, int32_t tile_size, int32_t tile_width,
    int32_t tile_height, const int32_t *tile_offsets, const int32_t *flatten_ids,
    int32_t *chunk_cnts, int32_t *chunk_starts, int64_t *n_elems,
    void *workspace, size_t workspace_bytes, gsplat_stream_t stream);
int gsplat_rasterize_to_indices_write(
    int64_t range_start, int64_t range_end, int64_t I, int64_t N,
    int64_t n_isects, const float *transmittances, const float *means2d,
    const float *conics, const float *opacities, int32_t image_width,
    int32_t image_height, int32_t tile_size, int32_t tile_width,
    int32_t tile_height, const int32_t *tile_offsets, const int32_t *flatten_ids,
    const int32_t *chunk_starts, int64_t *gaussian_ids, int64_t *pixel_ids,
    gsplat_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Densification statistics.                                                 */
/* ------------------------------------------------------------------------ */

/* Running-state update of DefaultStrategy._update_state
 *   (gsplat/strategy/default.py:218-268): for every visible row,
 *   grad2d[g] += ||(grads[r,0] * scale_x, grads[r,1] * scale_y)|| and
 *   count[g] += 1 (scale_x = W/2 * n_cameras, scale_y = H/2 * n_cameras).
 * grads [n_rows,2] (the 2D mean gradient or absgrad); packed rows give
 * gaussian_ids [n_rows] (int64, ids outside [0, N) are skipped); dense rows
 * [C,N] give radii [n_rows,2] instead and count where both radii are > 0.
 * grad2d [N] and count [N] are ACCUMULATED (float atomics, as the
 * reference's index_add_). */
int gsplat_grad2d_stats(
    int64_t n_rows, int64_t N, const float *grads, const int64_t *gaussian_ids,
    const int32_t *radii, float scale_x, float scale_y, float *grad2d,
    float *count, gsplat_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Fused Adam (no bias correction, optional per-row mask).                   */
/* ------------------------------------------------------------------------ */

typedef struct gsplat_adam_tensor {
    float *param;           /* [n_rows, row_size], updated in place */
    const float *grad;      /* [n_rows, row_size] */
    float *exp_avg;         /* [n_rows, row_size], updated in place */
    float *exp_avg_sq;      /* [n_rows, row_size], updated in place */
    const uint8_t *valid;   /* [n_rows] or NULL; rows with 0 are untouched */
    int64_t n_rows;
    int64_t row_size;
    float lr;
} gsplat_adam_tensor;

/* One launch updating every tensor of the list (a single HBM pass).
 * Replaces the per-tensor launches of adam_kernel issued by
 *   gsplat/optimizers/selective_adam.py:63-101
 *   (gsplat/cuda/csrc/Adam.cpp:37-66, AdamCUDA.cu:35-110).
 * `tensors` is a HOST array; at most 64 entries. */
int gsplat_adam_multi(
    const gsplat_adam_tensor *tensors, int32_t n_tensors,
    float b1, float b2, float eps, gsplat_stream_t stream);

/* Single-tensor form with the reference op's argument list.
 * Replaces the `adam` op (gsplat/cuda/ext.cpp:753, Adam.cpp:37-66). */
int gsplat_adam(
    float *param, const float *param_grad, float *exp_avg, float *exp_avg_sq,
    const uint8_t *valid, int64_t n_rows, int64_t row_size,
    float lr, float b1, float b2, float eps, gsplat_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GSPLAT_HIP_H */
