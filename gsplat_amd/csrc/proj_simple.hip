// projection_ewa_simple_{fwd,bwd}: the camera-space projection of a 3D
// Gaussian (mean and full 3x3 covariance) to its image-plane mean and 2x2
// covariance, for pinhole and orthographic cameras
// (gsplat/cuda/csrc/ProjectionEWASimple.cu:37-260, math of
// gsplat/cuda/include/Utils.cuh:473-660; the op behind gsplat.cuda.proj()).
//
// One thread per (batch, camera, Gaussian) row.  Rows are 12 + 36 B in and
// 8 + 16 B out, so the kernels are HBM streams; loads are scalar per row
// (stride 3 / 9 floats) and coalesce across the wave into contiguous spans.
//
// Forward:  mean2d = (fx x/z + cx, fy y/z + cy),  cov2d = J S J^T, with the
// pinhole Jacobian J = [[fx/z, 0, -fx tx/z^2], [0, fy/z, -fy ty/z^2]] where
// (tx, ty) are (x, y) with x/z, y/z clamped to 1.3x the field of view.
// Orthographic: J = [[fx, 0, 0], [0, fy, 0]], mean2d = (fx x + cx, fy y + cy).
// Backward: the vector-Jacobian product of the forward; the clamp zeroes the
// gradient through x/z (y/z) outside the field of view, where tx = z * limit.
#include "common.h"

namespace gs {
namespace {

constexpr int kSimpleThreads = 256;

struct PinholeLimits {
    float lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg;
};

__device__ __forceinline__ PinholeLimits pinhole_limits(float fx, float fy, float cx,
                                                        float cy, float W, float H) {
    const float tan_fovx = 0.5f * W / fx;
    const float tan_fovy = 0.5f * H / fy;
    return {(W - cx) / fx + 0.3f * tan_fovx, cx / fx + 0.3f * tan_fovx,
            (H - cy) / fy + 0.3f * tan_fovy, cy / fy + 0.3f * tan_fovy};
}

__global__ void __launch_bounds__(kSimpleThreads)
    proj_simple_fwd_kernel(int64_t rows, int64_t CN, int64_t N,
                           const float *__restrict__ means,
                           const float *__restrict__ covars,
                           const float *__restrict__ Ks, float W, float H,
                           int ortho, float *__restrict__ means2d,
                           float *__restrict__ covars2d) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows)
        return;
    const float *K = Ks + (r / N) * 9;  // (b, c) = r / N over B*C cameras
    (void)CN;
    const float fx = K[0], cx = K[2], fy = K[4], cy = K[5];
    const float x = means[r * 3 + 0], y = means[r * 3 + 1], z = means[r * 3 + 2];
    float S[9];
#pragma unroll
    for (int k = 0; k < 9; ++k)
        S[k] = covars[r * 9 + k];
    float j00, j11, j02, j12, mx, my;
    if (ortho) {
        j00 = fx;
        j11 = fy;
        j02 = 0.f;
        j12 = 0.f;
        mx = fx * x + cx;
        my = fy * y + cy;
    } else {
        const PinholeLimits L = pinhole_limits(fx, fy, cx, cy, W, H);
        const float rz = 1.f / z;
        const float rz2 = rz * rz;
        const float tx = z * fminf(L.lim_x_pos, fmaxf(-L.lim_x_neg, x * rz));
        const float ty = z * fminf(L.lim_y_pos, fmaxf(-L.lim_y_neg, y * rz));
        j00 = fx * rz;
        j11 = fy * rz;
        j02 = -fx * tx * rz2;
        j12 = -fy * ty * rz2;
        mx = fx * x * rz + cx;
        my = fy * y * rz + cy;
    }
    // A = J S (2x3), cov2d = A J^T; J has zeros at (0,1) and (1,0)
    const float a00 = j00 * S[0] + j02 * S[6], a01 = j00 * S[1] + j02 * S[7],
                a02 = j00 * S[2] + j02 * S[8];
    const float a10 = j11 * S[3] + j12 * S[6], a11 = j11 * S[4] + j12 * S[7],
                a12 = j11 * S[5] + j12 * S[8];
    means2d[r * 2 + 0] = mx;
    means2d[r * 2 + 1] = my;
    covars2d[r * 4 + 0] = a00 * j00 + a02 * j02;
    covars2d[r * 4 + 1] = a01 * j11 + a02 * j12;
    covars2d[r * 4 + 2] = a10 * j00 + a12 * j02;
    covars2d[r * 4 + 3] = a11 * j11 + a12 * j12;
}

// The backward runs in double from the float32 inputs: dL/dS = J^T G J and
// the Jacobian VJP sum terms that cancel (float32 put single elements of
// v_covars past rtol 1e-4 where the float32 restatement of the same math
// stays within it).  The clamp decisions are the forward's float32 ones.
__global__ void __launch_bounds__(kSimpleThreads)
    proj_simple_bwd_kernel(int64_t rows, int64_t N, const float *__restrict__ means,
                           const float *__restrict__ covars,
                           const float *__restrict__ Ks, float W, float H,
                           int ortho, const float *__restrict__ v_means2d,
                           const float *__restrict__ v_covars2d,
                           float *__restrict__ v_means,
                           float *__restrict__ v_covars) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows)
        return;
    const float *K = Ks + (r / N) * 9;
    const float fxf = K[0], cxf = K[2], fyf = K[4], cyf = K[5];
    const double fx = fxf, fy = fyf;
    const float xf = means[r * 3 + 0], yf = means[r * 3 + 1], zf = means[r * 3 + 2];
    const double x = xf, y = yf, z = zf;
    double S[9];
#pragma unroll
    for (int k = 0; k < 9; ++k)
        S[k] = covars[r * 9 + k];
    const double gm0 = v_means2d[r * 2 + 0], gm1 = v_means2d[r * 2 + 1];
    const double G[4] = {v_covars2d[r * 4 + 0], v_covars2d[r * 4 + 1],
                         v_covars2d[r * 4 + 2], v_covars2d[r * 4 + 3]};
    double j00, j11, j02, j12;
    double rz = 0.0, rz2 = 0.0, tx = 0.0, ty = 0.0;
    bool in_x = true, in_y = true;
    if (ortho) {
        j00 = fx;
        j11 = fy;
        j02 = 0.0;
        j12 = 0.0;
    } else {
        // the forward's float32 clamp (limits and x/z, y/z)
        const PinholeLimits L = pinhole_limits(fxf, fyf, cxf, cyf, W, H);
        const float rzf = 1.f / zf;
        const float ux = xf * rzf, uy = yf * rzf;
        in_x = ux <= L.lim_x_pos && ux >= -L.lim_x_neg;
        in_y = uy <= L.lim_y_pos && uy >= -L.lim_y_neg;
        rz = 1.0 / z;
        rz2 = rz * rz;
        tx = z * (double)fminf(L.lim_x_pos, fmaxf(-L.lim_x_neg, ux));
        ty = z * (double)fminf(L.lim_y_pos, fmaxf(-L.lim_y_neg, uy));
        j00 = fx * rz;
        j11 = fy * rz;
        j02 = -fx * tx * rz2;
        j12 = -fy * ty * rz2;
    }
    // dL/dS = J^T G J   (J: rows (j00, 0, j02), (0, j11, j12))
    const double Jm[6] = {j00, 0.0, j02, 0.0, j11, j12};
    double GJ[6];  // G J (2x3)
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        GJ[c] = G[0] * Jm[c] + G[1] * Jm[3 + c];
        GJ[3 + c] = G[2] * Jm[c] + G[3] * Jm[3 + c];
    }
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int c = 0; c < 3; ++c)
            v_covars[r * 9 + i * 3 + c] = (float)(Jm[i] * GJ[c] + Jm[3 + i] * GJ[3 + c]);

    if (ortho) {
        v_means[r * 3 + 0] = (float)(fx * gm0);
        v_means[r * 3 + 1] = (float)(fy * gm1);
        v_means[r * 3 + 2] = 0.f;
        return;
    }
    // dL/dJ = G J S^T + G^T J S; only J00, J11, J02, J12 depend on the mean
    double GtJ[6];  // G^T J
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        GtJ[c] = G[0] * Jm[c] + G[2] * Jm[3 + c];
        GtJ[3 + c] = G[1] * Jm[c] + G[3] * Jm[3 + c];
    }
    double vJ[6];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 3; ++c)
            vJ[i * 3 + c] = (GJ[i * 3 + 0] * S[c * 3 + 0] + GJ[i * 3 + 1] * S[c * 3 + 1] +
                             GJ[i * 3 + 2] * S[c * 3 + 2]) +
                            (GtJ[i * 3 + 0] * S[0 * 3 + c] + GtJ[i * 3 + 1] * S[1 * 3 + c] +
                             GtJ[i * 3 + 2] * S[2 * 3 + c]);
    const double rz3 = rz2 * rz;
    double vx = fx * rz * gm0;
    double vy = fy * rz * gm1;
    double vz = -(fx * x * gm0 + fy * y * gm1) * rz2;
    // J00 = fx/z, J11 = fy/z
    vz += -fx * rz2 * vJ[0] - fy * rz2 * vJ[4];
    // J02 = -fx tx/z^2 with tx = x inside the clamp, z*limit outside it
    if (in_x) {
        vx += -fx * rz2 * vJ[2];
        vz += 2.0 * fx * tx * rz3 * vJ[2];
    } else {
        vz += fx * tx * rz3 * vJ[2];
    }
    if (in_y) {
        vy += -fy * rz2 * vJ[5];
        vz += 2.0 * fy * ty * rz3 * vJ[5];
    } else {
        vz += fy * ty * rz3 * vJ[5];
    }
    v_means[r * 3 + 0] = (float)vx;
    v_means[r * 3 + 1] = (float)vy;
    v_means[r * 3 + 2] = (float)vz;
}

int check_camera_model(int32_t camera_model, const char *what) {
    if (camera_model == 0 || camera_model == 1)
        return GSPLAT_OK;
    return fail(GSPLAT_ERR_UNSUPPORTED,
                std::string(what) + ": only pinhole (0) and ortho (1) cameras are built");
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gsplat_projection_simple_fwd(int64_t B, int64_t C, int64_t N,
                                            const float *means, const float *covars,
                                            const float *Ks, int32_t image_width,
                                            int32_t image_height, int32_t camera_model,
                                            float *means2d, float *covars2d,
                                            gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0, "projection_simple_fwd: negative size");
    GS_TRY(check_camera_model(camera_model, "projection_simple_fwd"));
    const int64_t rows = B * C * N;
    if (rows == 0)
        return GSPLAT_OK;
    GS_REQUIRE(means && covars && Ks && means2d && covars2d,
               "projection_simple_fwd: NULL buffer");
    proj_simple_fwd_kernel<<<(unsigned)ceil_div(rows, kSimpleThreads), kSimpleThreads, 0,
                             as_stream(stream)>>>(rows, C * N, N, means, covars, Ks,
                                                  (float)image_width, (float)image_height,
                                                  camera_model == 1, means2d, covars2d);
    return check_launch("proj_simple_fwd_kernel");
}

extern "C" int gsplat_projection_simple_bwd(int64_t B, int64_t C, int64_t N,
                                            const float *means, const float *covars,
                                            const float *Ks, int32_t image_width,
                                            int32_t image_height, int32_t camera_model,
                                            const float *v_means2d, const float *v_covars2d,
                                            float *v_means, float *v_covars,
                                            gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0, "projection_simple_bwd: negative size");
    GS_TRY(check_camera_model(camera_model, "projection_simple_bwd"));
    const int64_t rows = B * C * N;
    if (rows == 0)
        return GSPLAT_OK;
    GS_REQUIRE(means && covars && Ks && v_means2d && v_covars2d && v_means && v_covars,
               "projection_simple_bwd: NULL buffer");
    proj_simple_bwd_kernel<<<(unsigned)ceil_div(rows, kSimpleThreads), kSimpleThreads, 0,
                             as_stream(stream)>>>(
        rows, N, means, covars, Ks, (float)image_width, (float)image_height,
        camera_model == 1, v_means2d, v_covars2d, v_means, v_covars);
    return check_launch("proj_simple_bwd_kernel");
}
