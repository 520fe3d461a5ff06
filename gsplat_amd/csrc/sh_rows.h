// Spherical-harmonics basis and the packed-row colour forward, shared by
// sh.hip and the intersection's fused colour-and-count launch (isect.hip).
//
// Basis: the Sloan 2013 real SH up to degree 4 as
// gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:37-388 evaluates it.
#pragma once

#include "common.h"

namespace gs {
namespace {

constexpr int kShThreads = 256;

constexpr float kY0 = 0.2820947917738781f;
constexpr float kY1 = 0.48860251190292f;
constexpr float kY2a = 1.092548430592079f;
constexpr float kY2b = 0.9461746957575601f;
constexpr float kY2c = 0.3153915652525201f;
constexpr float kY2d = 0.5462742152960395f;
constexpr float kY3a = 2.285228997322329f;
constexpr float kY3b = 0.4570457994644658f;
constexpr float kY3c = 1.445305721320277f;
constexpr float kY3d = 1.865881662950577f;
constexpr float kY3e = 1.119528997770346f;
constexpr float kY3f = 0.5900435899266435f;
constexpr float kY4a = 4.683325804901025f;
constexpr float kY4b = 2.007139630671868f;
constexpr float kY4c = 3.31161143515146f;
constexpr float kY4d = 0.47308734787878f;
constexpr float kY4e = 1.770130769779931f;
constexpr float kY4f = 1.984313483298443f;
constexpr float kY4g = 1.006230589874905f;
constexpr float kY4h = 0.6258357354491763f;

template <int DEG> struct ShShape {
    static constexpr int NB = (DEG + 1) * (DEG + 1);
    static constexpr int ROW = NB * 3;
    static constexpr int PITCH = (ROW % 2 == 0) ? ROW + 1 : ROW;
};

// Basis values Y[0..NB) at the unit direction (x, y, z).
template <int DEG>
__device__ __forceinline__ void sh_basis(float x, float y, float z, float *Y) {
    Y[0] = kY0;
    if (DEG < 1)
        return;
    Y[1] = -kY1 * y;
    Y[2] = kY1 * z;
    Y[3] = -kY1 * x;
    if (DEG < 2)
        return;
    const float z2 = z * z;
    const float fTmp0B = -kY2a * z;
    const float fC1 = x * x - y * y;
    const float fS1 = 2.f * x * y;
    Y[4] = kY2d * fS1;
    Y[5] = fTmp0B * y;
    Y[6] = kY2b * z2 - kY2c;
    Y[7] = fTmp0B * x;
    Y[8] = kY2d * fC1;
    if (DEG < 3)
        return;
    const float fTmp0C = -kY3a * z2 + kY3b;
    const float fTmp1B = kY3c * z;
    const float fC2 = x * fC1 - y * fS1;
    const float fS2 = x * fS1 + y * fC1;
    Y[9] = -kY3f * fS2;
    Y[10] = fTmp1B * fS1;
    Y[11] = fTmp0C * y;
    Y[12] = z * (kY3d * z2 - kY3e);
    Y[13] = fTmp0C * x;
    Y[14] = fTmp1B * fC1;
    Y[15] = -kY3f * fC2;
    if (DEG < 4)
        return;
    const float fTmp0D = z * (-kY4a * z2 + kY4b);
    const float fTmp1C = kY4c * z2 - kY4d;
    const float fTmp2B = -kY4e * z;
    const float fC3 = x * fC2 - y * fS2;
    const float fS3 = x * fS2 + y * fC2;
    Y[16] = kY4h * fS3;
    Y[17] = fTmp2B * fS2;
    Y[18] = fTmp1C * fS1;
    Y[19] = fTmp0D * y;
    Y[20] = kY4f * z * Y[12] - kY4g * Y[6];
    Y[21] = fTmp0D * x;
    Y[22] = fTmp1C * fC1;
    Y[23] = fTmp2B * fC2;
    Y[24] = kY4h * fC3;
}

// Camera centre -R^T t of a row-major world->camera matrix (the camera
// position of rendering.py:216-224).
__device__ __forceinline__ void camera_centre(const float *vm, float *cp) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
        cp[j] = -(vm[0 * 4 + j] * vm[3] + vm[1 * 4 + j] * vm[7] + vm[2 * 4 + j] * vm[11]);
}

struct ShRowsArgs {
    int64_t B, C, N;
    int K;
    const float *means;   // [B, N, 3]
    const float *viewmats;  // [B, C, 4, 4] world->camera
    const float *coeffs;  // [B, N, K, 3]
    const int32_t *row_of;  // [B, C, N]
    bool vec_ok;
};

// One Gaussian's inputs to the packed-row forward: its packed row in camera
// 0, its mean and its coefficients.
template <int DEG> struct ShRowIn {
    int32_t row0;
    float m[3];
    float cf[ShShape<DEG>::ROW];
};

// The loads of Gaussian bg (a thread's coefficients go straight to
// registers, with 16-byte loads when a row is a whole number of float4,
// which leaves occupancy to the registers instead of the ~12.5 KB per wave
// an LDS staging takes).  Returns whether any camera sees it; nothing else
// is loaded for one no camera sees.
template <int DEG>
__device__ __forceinline__ bool sh_rows_fwd_load(const ShRowsArgs &a, int64_t bg,
                                                 ShRowIn<DEG> &in) {
    using S = ShShape<DEG>;
    if (bg >= a.B * a.N)
        return false;
    const int64_t b = bg / a.N, g = bg - b * a.N;
    in.row0 = a.row_of[b * a.C * a.N + g];
    bool vis = in.row0 >= 0;
    for (int64_t c = 1; c < a.C; ++c)
        vis |= a.row_of[(b * a.C + c) * a.N + g] >= 0;
    if (!vis)
        return false;
    in.m[0] = a.means[bg * 3 + 0];
    in.m[1] = a.means[bg * 3 + 1];
    in.m[2] = a.means[bg * 3 + 2];
    if (S::ROW % 4 == 0 && a.vec_ok) {
        const float4 *src = reinterpret_cast<const float4 *>(a.coeffs + bg * S::ROW);
#pragma unroll
        for (int i = 0; i < S::ROW / 4; ++i) {
            const float4 v = src[i];
            in.cf[4 * i + 0] = v.x;
            in.cf[4 * i + 1] = v.y;
            in.cf[4 * i + 2] = v.z;
            in.cf[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < S::ROW; ++i)
            in.cf[i] = a.coeffs[bg * (int64_t)a.K * 3 + i];
    }
    return true;
}

// colors[row] = max(SH(normalised mean - camera centre) + 0.5, 0) for every
// camera's packed row of the visible Gaussian bg.
template <int DEG>
__device__ __forceinline__ void sh_rows_fwd_eval(const ShRowsArgs &a,
                                                 float *__restrict__ colors, int64_t bg,
                                                 const ShRowIn<DEG> &in) {
    using S = ShShape<DEG>;
    const int64_t b = bg / a.N, g = bg - b * a.N;
    for (int64_t c = 0; c < a.C; ++c) {
        const int32_t r = c == 0 ? in.row0 : a.row_of[(b * a.C + c) * a.N + g];
        if (r < 0)
            continue;
        float Y[S::NB];
        if (DEG > 0) {
            float cp[3];
            camera_centre(a.viewmats + (b * a.C + c) * 16, cp);
            const float dx = in.m[0] - cp[0], dy = in.m[1] - cp[1], dz = in.m[2] - cp[2];
            const float inorm = 1.f / sqrtf(dx * dx + dy * dy + dz * dz);
            sh_basis<DEG>(dx * inorm, dy * inorm, dz * inorm, Y);
        } else {
            Y[0] = kY0;
        }
        float o0 = 0.f, o1 = 0.f, o2 = 0.f;
#pragma unroll
        for (int k = 0; k < S::NB; ++k) {
            o0 += Y[k] * in.cf[k * 3 + 0];
            o1 += Y[k] * in.cf[k * 3 + 1];
            o2 += Y[k] * in.cf[k * 3 + 2];
        }
        colors[(int64_t)r * 3 + 0] = fmaxf(o0 + 0.5f, 0.f);
        colors[(int64_t)r * 3 + 1] = fmaxf(o1 + 0.5f, 0.f);
        colors[(int64_t)r * 3 + 2] = fmaxf(o2 + 0.5f, 0.f);
    }
}

// One thread per Gaussian.
template <int DEG>
__device__ __forceinline__ void sh_rows_fwd_row(const ShRowsArgs &a,
                                                float *__restrict__ colors,
                                                int64_t bg) {
    ShRowIn<DEG> in;
    if (sh_rows_fwd_load<DEG>(a, bg, in))
        sh_rows_fwd_eval<DEG>(a, colors, bg, in);
}

}  // namespace
}  // namespace gs
