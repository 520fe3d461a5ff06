/*
 * exact_ref.c -- TEST INFRASTRUCTURE ONLY (the parity oracle).
 *
 * Plain-C restatement, on the host, of the parts of the splatting path whose
 * outputs are integers or must be reproduced bit for bit:
 *   - EWA projection forward (validity, radii, means2d, depths, conics,
 *     compensation) -- gsplat/cuda/csrc/ProjectionEWA3DGSFused.cu:38-234 with
 *     the math of gsplat/cuda/include/Utils.cuh:174-257, 424-432, 542-581;
 *   - tile-set enumeration per row, ellipse ("AccuTile") and axis-aligned box
 *     variants -- gsplat/cuda/csrc/IntersectTile.cu:38-121, 133-288;
 *   - the natural log used by the opacity-aware extents and the exponential
 *     that turns a Gaussian's Mahalanobis term into its alpha.
 * Every floating-point operation is written out in the order the product
 * kernels use -- each a * b + c that the kernels fuse as an explicit fmaf
 * (correctly rounded in the C library as on the GPU) -- and this file is
 * compiled with -ffp-contract=off, so IEEE single precision gives identical
 * bits on the CPU and the GPU.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may load
 * this code, and only as a checker.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ALPHA_THRESHOLD (1.f / 255.f)
#define GAUSSIAN_EXTEND 3.33f
#define MIN_COMPENSATION 0.005f

static int32_t sat_f2i(float x) {
    if (!(x == x)) return 0;
    if (x >= 2147483648.f) return 2147483647;
    if (x <= -2147483648.f) return (-2147483647 - 1);
    return (int32_t)x;
}

static int imin(int a, int b) { return a < b ? a : b; }
static int imax(int a, int b) { return a > b ? a : b; }

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ln(x) by the series of 2*atanh(s), s = (m-1)/(m+1) (same constants and
 * order as the device function). */
float oracle_portable_logf(float x) {
    if (!(x > 0.f)) return NAN;
    if (x == INFINITY) return x;
    uint32_t bits = f2u(x);
    int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127;
    float m = u2f((bits & 0x007fffffu) | 0x3f800000u);
    if (e == -127) {
        float xs = x * 8388608.f;
        bits = f2u(xs);
        e = (int32_t)((bits >> 23) & 0xffu) - 127 - 23;
        m = u2f((bits & 0x007fffffu) | 0x3f800000u);
    }
    if (m > 1.41421356f) {
        m = m * 0.5f;
        e = e + 1;
    }
    const float f = m - 1.f;
    const float s = f / (2.f + f);
    const float z = s * s;
    const float r = z * (0.666666667f + z * (0.4f + z * (0.285714286f + z * 0.222222222f)));
    const float lnm = (s + s) + s * r;
    const float ef = (float)e;
    return ef * 0x1.62e3p-1f + (lnm + ef * 0x1.2fefa2p-17f);
}

void oracle_portable_logf_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_portable_logf(x[i]);
}

/* e^x by Cody-Waite reduction (x = k ln2 + r, two-part ln2) and the
 * degree-6 minimax polynomial of e^r with 1 + r + r^2/2 fixed (coefficients
 * from oracle/exp_poly_fit.py) in fused multiply-adds: the device
 * portable_expf, operation for operation (fmaf and rintf are correctly
 * rounded, so the bits agree). */
float oracle_portable_expf(float x) {
    if (!(x == x)) return x;
    if (x < -87.f) return 0.f;
    if (x > 88.f) return INFINITY;
    const float kf = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-kf, 0x1.63p-1f, x);
    r = fmaf(-kf, -0x1.bd0106p-13f, r);
    float p = 0x1.6e2dp-10f;
    p = fmaf(p, r, 0x1.1264c4p-7f);
    p = fmaf(p, r, 0x1.555414p-5f);
    p = fmaf(p, r, 0x1.55544ap-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.f);
    p = fmaf(p, r, 1.f);
    const float scale = u2f((uint32_t)((int32_t)kf + 127) << 23);
    return p * scale;
}

void oracle_portable_expf_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_portable_expf(x[i]);
}

/* ----------------------------------------------------------------------- */
/* Projection forward                                                       */
/* ----------------------------------------------------------------------- */
static void quat_to_rot(float w, float x, float y, float z, float M[9]) {
    const float n2 = fmaf(w, w, fmaf(z, z, fmaf(y, y, x * x)));
    const float inv = 1.0f / sqrtf(n2);
    x = x * inv; y = y * inv; z = z * inv; w = w * inv;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float wx = w * x, wy = w * y, wz = w * z;
    M[0] = fmaf(-2.f, y2 + z2, 1.f);
    M[1] = 2.f * (xy - wz);
    M[2] = 2.f * (xz + wy);
    M[3] = 2.f * (xy + wz);
    M[4] = fmaf(-2.f, x2 + z2, 1.f);
    M[5] = 2.f * (yz - wx);
    M[6] = 2.f * (xz - wy);
    M[7] = 2.f * (yz + wx);
    M[8] = fmaf(-2.f, x2 + y2, 1.f);
}

/* a0 b0 + a1 b1 + a2 b2 as a product and two fused multiply-adds */
static float dot3(float a0, float b0, float a1, float b1, float a2, float b2) {
    return fmaf(a2, b2, fmaf(a1, b1, a0 * b0));
}

/* returns 1 if the row survives culling */
static int project_one(const float *vm, const float *K, const float *mean,
                       const float *covar6, const float *quat, const float *scale,
                       int has_opacity, float opacity, int calc_comp,
                       int camera_model, float W, float H, float eps2d,
                       float near_plane, float far_plane, float radius_clip,
                       float out[7], int32_t rad[2]) {
    float R[9], t[3];
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) R[i * 3 + j] = vm[i * 4 + j];
        t[i] = vm[i * 4 + 3];
    }
    const float fx = K[0], fy = K[4], cx = K[2], cy = K[5];
    const float p0 = mean[0], p1 = mean[1], p2 = mean[2];
    const float mcx = fmaf(R[2], p2, fmaf(R[1], p1, fmaf(R[0], p0, t[0])));
    const float mcy = fmaf(R[5], p2, fmaf(R[4], p1, fmaf(R[3], p0, t[1])));
    const float mcz = fmaf(R[8], p2, fmaf(R[7], p1, fmaf(R[6], p0, t[2])));
    if (mcz < near_plane || mcz > far_plane) return 0;

    float S00, S01, S02, S11, S12, S22;
    if (covar6) {
        S00 = covar6[0]; S01 = covar6[1]; S02 = covar6[2];
        S11 = covar6[3]; S12 = covar6[4]; S22 = covar6[5];
    } else {
        float M[9], A[9];
        quat_to_rot(quat[0], quat[1], quat[2], quat[3], M);
        for (int i = 0; i < 3; ++i) {
            A[i * 3 + 0] = M[i * 3 + 0] * scale[0];
            A[i * 3 + 1] = M[i * 3 + 1] * scale[1];
            A[i * 3 + 2] = M[i * 3 + 2] * scale[2];
        }
#define DOTR(i, j) dot3(A[(i)*3+0], A[(j)*3+0], A[(i)*3+1], A[(j)*3+1], A[(i)*3+2], A[(j)*3+2])
        S00 = DOTR(0, 0); S01 = DOTR(0, 1); S02 = DOTR(0, 2);
        S11 = DOTR(1, 1); S12 = DOTR(1, 2); S22 = DOTR(2, 2);
#undef DOTR
    }
    const float Sf[9] = {S00, S01, S02, S01, S11, S12, S02, S12, S22};
    float Bm[9];
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            Bm[i * 3 + j] = dot3(R[i * 3 + 0], Sf[0 * 3 + j], R[i * 3 + 1], Sf[1 * 3 + j],
                                 R[i * 3 + 2], Sf[2 * 3 + j]);
#define SC(i, j) dot3(Bm[(i)*3+0], R[(j)*3+0], Bm[(i)*3+1], R[(j)*3+1], Bm[(i)*3+2], R[(j)*3+2])
    const float s00 = SC(0, 0), s01 = SC(0, 1), s02 = SC(0, 2);
    const float s11 = SC(1, 1), s12 = SC(1, 2), s22 = SC(2, 2);
#undef SC
    float J00, J02, J11, J12, mx, my;
    if (camera_model == 1) {
        J00 = fx; J11 = fy; J02 = 0.f; J12 = 0.f;
        mx = fmaf(fx, mcx, cx);
        my = fmaf(fy, mcy, cy);
    } else {
        const float tan_fovx = (0.5f * W) / fx;
        const float tan_fovy = (0.5f * H) / fy;
        const float lim_x_pos = (W - cx) / fx + 0.3f * tan_fovx;
        const float lim_x_neg = cx / fx + 0.3f * tan_fovx;
        const float lim_y_pos = (H - cy) / fy + 0.3f * tan_fovy;
        const float lim_y_neg = cy / fy + 0.3f * tan_fovy;
        const float rz = 1.f / mcz;
        const float rz2 = rz * rz;
        const float tx = mcz * fminf(lim_x_pos, fmaxf(-lim_x_neg, mcx * rz));
        const float ty = mcz * fminf(lim_y_pos, fmaxf(-lim_y_neg, mcy * rz));
        J00 = fx * rz;
        J11 = fy * rz;
        J02 = ((-fx) * tx) * rz2;
        J12 = ((-fy) * ty) * rz2;
        mx = fmaf(fx * mcx, rz, cx);
        my = fmaf(fy * mcy, rz, cy);
    }
    const float u0 = fmaf(s02, J02, s00 * J00);
    const float u1 = fmaf(s12, J02, s01 * J00);
    const float u2 = fmaf(s22, J02, s02 * J00);
    const float w1 = fmaf(s12, J12, s11 * J11);
    const float w2 = fmaf(s22, J12, s12 * J11);
    const float c00 = fmaf(J02, u2, J00 * u0);
    const float c01 = fmaf(J12, u2, J11 * u1);
    const float c11 = fmaf(J12, w2, J11 * w1);
    const float c01sq = c01 * c01;
    const float det_orig = fmaf(c00, c11, -c01sq);
    const float c00b = c00 + eps2d;
    const float c11b = c11 + eps2d;
    const float det = fmaf(c00b, c11b, -c01sq);
    if (!(det > 0.f)) return 0;
    const float comp = sqrtf(fmaxf(MIN_COMPENSATION * MIN_COMPENSATION, det_orig / det));
    const float inv_det = 1.f / det;
    float extend = GAUSSIAN_EXTEND;
    if (has_opacity) {
        float op = opacity;
        if (calc_comp) op = op * comp;
        if (op < ALPHA_THRESHOLD) return 0;
        extend = fminf(GAUSSIAN_EXTEND, sqrtf(2.f * oracle_portable_logf(op / ALPHA_THRESHOLD)));
    }
    const float rx = ceilf(extend * sqrtf(c00b));
    const float ry = ceilf(extend * sqrtf(c11b));
    if (rx <= radius_clip && ry <= radius_clip) return 0;
    if (mx + rx <= 0.f || mx - rx >= W || my + ry <= 0.f || my - ry >= H) return 0;
    out[0] = mx; out[1] = my; out[2] = mcz;
    out[3] = c11b * inv_det; out[4] = (-c01) * inv_det; out[5] = c00b * inv_det;
    out[6] = comp;
    rad[0] = sat_f2i(rx);
    rad[1] = sat_f2i(ry);
    return 1;
}

/* Dense projection of B*C*N rows; culled rows get zeros. */
void oracle_projection_fwd(int64_t B, int64_t C, int64_t N, const float *means,
                           const float *covars, const float *quats, const float *scales,
                           const float *opacities, const float *viewmats, const float *Ks,
                           int32_t W, int32_t H, float eps2d, float near_plane,
                           float far_plane, float radius_clip, int32_t calc_comp,
                           int32_t camera_model, int32_t *radii, float *means2d,
                           float *depths, float *conics, float *comps, uint8_t *valid) {
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < C; ++c)
            for (int64_t g = 0; g < N; ++g) {
                const int64_t row = (b * C + c) * N + g;
                const int64_t bg = b * N + g;
                float out[7] = {0, 0, 0, 0, 0, 0, 0};
                int32_t rad[2] = {0, 0};
                const int ok = project_one(
                    viewmats + (b * C + c) * 16, Ks + (b * C + c) * 9, means + bg * 3,
                    covars ? covars + bg * 6 : 0, quats ? quats + bg * 4 : 0,
                    scales ? scales + bg * 3 : 0, opacities != 0,
                    opacities ? opacities[bg] : 0.f, calc_comp, camera_model,
                    (float)W, (float)H, eps2d, near_plane, far_plane, radius_clip, out, rad);
                if (!ok) {
                    memset(out, 0, sizeof(out));
                    rad[0] = rad[1] = 0;
                }
                valid[row] = (uint8_t)ok;
                radii[row * 2] = rad[0];
                radii[row * 2 + 1] = rad[1];
                means2d[row * 2] = out[0];
                means2d[row * 2 + 1] = out[1];
                depths[row] = out[2];
                conics[row * 3] = out[3];
                conics[row * 3 + 1] = out[4];
                conics[row * 3 + 2] = out[5];
                if (comps) comps[row] = out[6];
            }
}

/* ----------------------------------------------------------------------- */
/* Tile sets                                                                */
/* ----------------------------------------------------------------------- */
static void ellipse_line(float A, float B, float C, float disc, float t, float px,
                         float py, int isY, float coord, float *lo, float *hi) {
    const float p_u = isY ? py : px;
    const float p_v = isY ? px : py;
    const float coeff = isY ? A : C;
    const float h = coord - p_u;
    const float sq = sqrtf((disc * h) * h + t * coeff);
    const float mbh = (-B) * h;
    *lo = (mbh - sq) / coeff + p_v;
    *hi = (mbh + sq) / coeff + p_v;
}

/* Enumerates the tiles of one row; writes tile ids to `tiles` (if non-null)
 * and returns their number. */
static int32_t row_tiles(const float *mean, const int32_t *rad, const float *conic,
                         const float *opacity, int tile_size, int tw, int th,
                         int64_t *tiles) {
    const float radius_x = (float)rad[0];
    const float radius_y = (float)rad[1];
    if (radius_x <= 0.f || radius_y <= 0.f) return 0;
    const float mxv = mean[0], myv = mean[1];
    const float ts = (float)tile_size;
    int32_t count = 0;
    if (conic && opacity) {
        const float A = conic[0], B = conic[1], C = conic[2];
        const float disc = B * B - A * C;
        const float t = fminf(GAUSSIAN_EXTEND * GAUSSIAN_EXTEND,
                              2.0f * oracle_portable_logf(*opacity / ALPHA_THRESHOLD));
        if (!(t >= 0.f) || !(disc < 0.f)) return 0;
        const float nt = (-t) / disc;
        const float x_ext = sqrtf(nt * C);
        const float y_ext = sqrtf(nt * A);
        float bmin_x = mxv - x_ext, bmin_y = myv - y_ext;
        float bmax_x = mxv + x_ext, bmax_y = myv + y_ext;
        const float bx_over_c = (B * x_ext) / C;
        const float by_over_a = (B * y_ext) / A;
        float amin_x = myv + bx_over_c, amin_y = mxv + by_over_a;
        float amax_x = myv - bx_over_c, amax_y = mxv - by_over_a;
        int rmin_x = imax(0, imin(tw, sat_f2i(bmin_x / ts)));
        int rmin_y = imax(0, imin(th, sat_f2i(bmin_y / ts)));
        int rmax_x = imax(0, imin(tw, sat_f2i(bmax_x / ts + 1.f)));
        int rmax_y = imax(0, imin(th, sat_f2i(bmax_y / ts + 1.f)));
        const int y_span = rmax_y - rmin_y;
        const int x_span = rmax_x - rmin_x;
        if (y_span == 0 || x_span == 0) return 0;
        const int isY = y_span < x_span;
        if (isY) {
            int ti; float tf;
            ti = rmin_x; rmin_x = rmin_y; rmin_y = ti;
            ti = rmax_x; rmax_x = rmax_y; rmax_y = ti;
            tf = bmin_x; bmin_x = bmin_y; bmin_y = tf;
            tf = bmax_x; bmax_x = bmax_y; bmax_y = tf;
            tf = amin_x; amin_x = amin_y; amin_y = tf;
            tf = amax_x; amax_x = amax_y; amax_y = tf;
        }
        float max_lo = bmax_y, max_hi = bmin_y, min_lo, min_hi;
        float min_line = (float)rmin_x * ts;
        if (bmin_x <= min_line) {
            ellipse_line(A, B, C, disc, t, mxv, myv, isY, min_line, &min_lo, &min_hi);
        } else {
            min_lo = max_lo;
            min_hi = max_hi;
        }
        for (int u = rmin_x; u < rmax_x; ++u) {
            const float max_line = min_line + ts;
            if (max_line <= bmax_x)
                ellipse_line(A, B, C, disc, t, mxv, myv, isY, max_line, &max_lo, &max_hi);
            float e_min, e_max;
            if (min_line <= amin_y && amin_y < max_line) e_min = bmin_y;
            else e_min = fminf(min_lo, max_lo);
            if (min_line <= amax_y && amax_y < max_line) e_max = bmax_y;
            else e_max = fmaxf(min_hi, max_hi);
            const int v0 = imax(rmin_y, imin(rmax_y, sat_f2i(e_min / ts)));
            const int v1 = imin(rmax_y, imax(rmin_y, sat_f2i(e_max / ts + 1.f)));
            if (v1 > v0) {
                for (int v = v0; v < v1; ++v) {
                    if (tiles) tiles[count] = isY ? (int64_t)u * tw + v : (int64_t)v * tw + u;
                    ++count;
                }
            }
            min_lo = max_lo;
            min_hi = max_hi;
            min_line = max_line;
        }
        return count;
    }
    const float trx = radius_x / ts, try_ = radius_y / ts;
    const float tx = mxv / ts, ty = myv / ts;
    const int x0 = imin(imax(0, sat_f2i(floorf(tx - trx))), tw);
    const int y0 = imin(imax(0, sat_f2i(floorf(ty - try_))), th);
    const int x1 = imin(imax(0, sat_f2i(ceilf(tx + trx))), tw);
    const int y1 = imin(imax(0, sat_f2i(ceilf(ty + try_))), th);
    for (int y = y0; y < y1; ++y)
        for (int x = x0; x < x1; ++x) {
            if (tiles) tiles[count] = (int64_t)y * tw + x;
            ++count;
        }
    return count;
}

/* Tile counts of n rows (conics/opacities may be NULL for the box test). */
void oracle_isect_count(int64_t n, const float *means2d, const int32_t *radii,
                        const float *conics, const float *opacities, int32_t tile_size,
                        int32_t tile_width, int32_t tile_height, int32_t *counts) {
    for (int64_t i = 0; i < n; ++i)
        counts[i] = row_tiles(means2d + 2 * i, radii + 2 * i,
                              conics ? conics + 3 * i : 0, opacities ? opacities + i : 0,
                              tile_size, tile_width, tile_height, 0);
}

/* Emits (key, flatten_id) in row order; offsets[i] = first slot of row i. */
void oracle_isect_emit(int64_t n, int64_t N, const int64_t *image_ids,
                       const float *means2d, const int32_t *radii, const float *depths,
                       const float *conics, const float *opacities, int32_t tile_size,
                       int32_t tile_width, int32_t tile_height, int32_t tile_n_bits,
                       const int64_t *row_offsets, int64_t *tile_scratch,
                       int64_t *isect_ids, int32_t *flatten_ids) {
    for (int64_t i = 0; i < n; ++i) {
        const int32_t cnt = row_tiles(means2d + 2 * i, radii + 2 * i,
                                      conics ? conics + 3 * i : 0,
                                      opacities ? opacities + i : 0, tile_size,
                                      tile_width, tile_height, tile_scratch);
        const int64_t iid = image_ids ? image_ids[i] : i / N;
        const int64_t depth_lo = (int64_t)f2u(depths[i]);
        int64_t cur = row_offsets[i];
        for (int32_t k = 0; k < cnt; ++k) {
            isect_ids[cur] = (iid << (32 + tile_n_bits)) | (tile_scratch[k] << 32) | depth_lo;
            flatten_ids[cur] = (int32_t)i;
            ++cur;
        }
    }
}
