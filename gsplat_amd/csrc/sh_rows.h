// Spherical-harmonics basis and the packed-row colour forward and backward,
// shared by sh.hip, the intersection's fused colour-and-count launch
// (isect.hip) and the projection's fused colour-and-geometry backward
// (projection.hip).
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
    // LDS pitch of a staged row.  Rows of a multiple of four floats get a
    // pitch of an odd number of 16-byte chunks: the staging's 16-byte stores,
    // the threads' 16-byte row reads and the write-out's 16-byte reads then
    // take distinct banks across a wave.  Other rows get an odd pitch (4-byte
    // row reads on distinct banks).
    static constexpr int PITCH = (ROW % 4 == 0) ? ((ROW / 4) % 2 == 1 ? ROW : ROW + 4)
                                 : (ROW % 2 == 0) ? ROW + 1 : ROW;
    static constexpr bool VEC = ROW % 4 == 0;
};

// The four floats at offset e (a multiple of 4) of a span of staged rows.
template <int DEG>
__device__ __forceinline__ float4 staged_chunk(const float *s, int e) {
    using S = ShShape<DEG>;
    if constexpr (S::VEC) {
        const int r = e / S::ROW;
        return *reinterpret_cast<const float4 *>(s + r * S::PITCH + (e - r * S::ROW));
    } else {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int ek = e + k;
            const int r = ek / S::ROW;
            v[k] = s[r * S::PITCH + (ek - r * S::ROW)];
        }
        return make_float4(v[0], v[1], v[2], v[3]);
    }
}

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

// Gradient of sum_k G[k] * Y_k w.r.t. the unit direction components
// (treated as independent; the normalisation VJP is applied by the caller).
template <int DEG>
__device__ __forceinline__ void sh_basis_grad(float x, float y, float z,
                                              const float *G, float &gx,
                                              float &gy, float &gz) {
    gx = gy = gz = 0.f;
    if (DEG < 1)
        return;
    gx += -kY1 * G[3];
    gy += -kY1 * G[1];
    gz += kY1 * G[2];
    if (DEG < 2)
        return;
    const float z2 = z * z;
    const float fC1 = x * x - y * y;
    const float fS1 = 2.f * x * y;
    // Y4 = b*fS1, Y5 = -a z y, Y6 = d z^2 - e, Y7 = -a z x, Y8 = b*fC1
    gx += kY2d * 2.f * y * G[4] - kY2a * z * G[7] + kY2d * 2.f * x * G[8];
    gy += kY2d * 2.f * x * G[4] - kY2a * z * G[5] - kY2d * 2.f * y * G[8];
    gz += -kY2a * y * G[5] + 2.f * kY2b * z * G[6] - kY2a * x * G[7];
    if (DEG < 3)
        return;
    const float fTmp0C = -kY3a * z2 + kY3b;
    const float fC2 = x * fC1 - y * fS1;
    const float fS2 = x * fS1 + y * fC1;
    // d fC2 = (3 fC1, -3 fS1), d fS2 = (3 fS1, 3 fC1)
    gx += -kY3f * 3.f * fS1 * G[9] + kY3c * z * 2.f * y * G[10] +
          fTmp0C * G[13] + kY3c * z * 2.f * x * G[14] -
          kY3f * 3.f * fC1 * G[15];
    gy += -kY3f * 3.f * fC1 * G[9] + kY3c * z * 2.f * x * G[10] +
          fTmp0C * G[11] - kY3c * z * 2.f * y * G[14] +
          kY3f * 3.f * fS1 * G[15];
    gz += kY3c * fS1 * G[10] - 2.f * kY3a * z * y * G[11] +
          (3.f * kY3d * z2 - kY3e) * G[12] - 2.f * kY3a * z * x * G[13] +
          kY3c * fC1 * G[14];
    if (DEG < 4)
        return;
    const float fTmp0D = z * (-kY4a * z2 + kY4b);
    const float dTmp0D = -3.f * kY4a * z2 + kY4b;
    const float fTmp1C = kY4c * z2 - kY4d;
    // d fC3 = (4 fC2, -4 fS2), d fS3 = (4 fS2, 4 fC2)
    gx += kY4h * 4.f * fS2 * G[16] - kY4e * z * 3.f * fS1 * G[17] +
          fTmp1C * 2.f * y * G[18] + fTmp0D * G[21] +
          fTmp1C * 2.f * x * G[22] - kY4e * z * 3.f * fC1 * G[23] +
          kY4h * 4.f * fC2 * G[24];
    gy += kY4h * 4.f * fC2 * G[16] - kY4e * z * 3.f * fC1 * G[17] +
          fTmp1C * 2.f * x * G[18] + fTmp0D * G[19] -
          fTmp1C * 2.f * y * G[22] + kY4e * z * 3.f * fS1 * G[23] -
          kY4h * 4.f * fS2 * G[24];
    gz += -kY4e * fS2 * G[17] + 2.f * kY4c * z * fS1 * G[18] +
          y * dTmp0D * G[19] +
          (kY4f * (4.f * kY3d * z2 * z - 2.f * kY3e * z) -
           kY4g * 2.f * kY2b * z) * G[20] +
          x * dTmp0D * G[21] + 2.f * kY4c * z * fC1 * G[22] -
          kY4e * fC2 * G[23];
}

// Copy the coefficient prefix (NB bands) of rows [r0, r0 + nrows) into LDS
// with pitch PITCH floats per row.  With `vis` (an LDS flag per row), rows
// whose flag is 0 are not read (their LDS rows hold zeros).  Every load
// of a thread is issued before the first LDS write, so a wave waits for
// memory once per tile instead of once per 16-byte chunk.  STREAM makes the
// 16-byte loads non-temporal (the backward reads each row once: 104 -> 99 us
// for the fused SH/geometry backward at config 1).
template <int DEG, bool STREAM = false>
__device__ __forceinline__ void stage_coeffs(const float *__restrict__ coeffs,
                                             int64_t r0, int nrows, int K,
                                             bool vec_ok, float *s,
                                             const uint8_t *vis = nullptr) {
    using S = ShShape<DEG>;
    const int total = nrows * S::ROW;
    if (vec_ok) {
        // K == NB and the span is 16-byte aligned: 16-byte loads.
        const float4 *src =
            reinterpret_cast<const float4 *>(coeffs + r0 * S::ROW);
        const int nvec = total >> 2;
        constexpr int NI = (kShThreads * S::ROW / 4 + kShThreads - 1) / kShThreads;
        // chunks of rows that are not read leave zeros in LDS (never used)
        float4 q[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int v = (int)threadIdx.x + i * kShThreads;
            const int e = v << 2;
            const bool take = v < nvec && (vis == nullptr || vis[e / S::ROW] ||
                                           vis[(e + 3) / S::ROW]);
            if (!take) {
                q[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            } else if constexpr (STREAM) {
                q[i] = ld_stream4(src + v);
            } else {
                q[i] = src[v];
            }
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((int)threadIdx.x + i * kShThreads >= nvec)
                break;
            const int e = ((int)threadIdx.x + i * kShThreads) << 2;
            if constexpr (S::VEC) {
                const int row = e / S::ROW;
                *reinterpret_cast<float4 *>(s + row * S::PITCH + (e - row * S::ROW)) = q[i];
            } else {
                const float vals[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int ek = e + k;
                    const int row = ek / S::ROW;
                    s[row * S::PITCH + (ek - row * S::ROW)] = vals[k];
                }
            }
        }
        for (int e = (nvec << 2) + threadIdx.x; e < total; e += kShThreads) {
            const int row = e / S::ROW;
            if (vis != nullptr && !vis[row])
                continue;
            s[row * S::PITCH + (e - row * S::ROW)] = coeffs[r0 * S::ROW + e];
        }
    } else {
        constexpr int NI = S::ROW;  // ceil(kShThreads * ROW / kShThreads)
        float q[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int e = (int)threadIdx.x + i * kShThreads;
            const int row = e / S::ROW;
            const bool take = e < total && (vis == nullptr || vis[row]);
            q[i] = take ? coeffs[(r0 + row) * (int64_t)K * 3 + (e - row * S::ROW)]
                        : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((int)threadIdx.x + i * kShThreads >= total)
                break;
            const int e = (int)threadIdx.x + i * kShThreads;
            const int row = e / S::ROW;
            s[row * S::PITCH + (e - row * S::ROW)] = q[i];
        }
    }
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

// Visibility of the thread's Gaussian (its packed row in camera 0 is
// returned in *row0), its mean (loaded before the barrier so the load
// overlaps the visibility round trip), and the workgroup's coefficient tile
// staged in LDS.
template <int DEG>
__device__ __forceinline__ bool sh_rows_prologue(const ShRowsArgs &a,
                                                 int64_t r0, int nrows,
                                                 float *s_coef, uint8_t *s_vis,
                                                 int32_t *row0, float *mean) {
    const int t = threadIdx.x;
    bool vis = false;
    *row0 = -1;
    mean[0] = mean[1] = mean[2] = 0.f;
    if (t < nrows) {
        const int64_t bg = r0 + t;
        const int64_t b = bg / a.N, g = bg - b * a.N;
        mean[0] = a.means[bg * 3 + 0];
        mean[1] = a.means[bg * 3 + 1];
        mean[2] = a.means[bg * 3 + 2];
        *row0 = a.row_of[b * a.C * a.N + g];
        vis = *row0 >= 0;
        for (int64_t c = 1; c < a.C; ++c)
            vis |= a.row_of[(b * a.C + c) * a.N + g] >= 0;
    }
    s_vis[t] = vis ? 1 : 0;
    __syncthreads();
    stage_coeffs<DEG, true>(a.coeffs, r0, nrows, a.K, a.vec_ok, s_coef, s_vis);
    __syncthreads();
    return vis;
}

// The packed-row backward of the 256 Gaussians from r0 (a whole workgroup,
// which it synchronises): writes their dense coefficient-gradient rows and
// returns each thread's direction term of dL/dmean in vm.  The workgroup's
// coefficient span is staged in LDS with 16-byte loads, and the gradient
// rows leave through the same tile with 16-byte stores.
template <int DEG>
__device__ __forceinline__ void sh_rows_bwd_block(const ShRowsArgs &a,
                                                  const float *__restrict__ v_colors,
                                                  float *__restrict__ v_coeffs,
                                                  int64_t r0, float vm[3]) {
    using S = ShShape<DEG>;
    __shared__ alignas(16) float s_buf[kShThreads * S::PITCH];
    __shared__ uint8_t s_vis[kShThreads];
    const int64_t BN = a.B * a.N;
    const int nrows = (int)((BN - r0) < kShThreads ? (BN - r0) : kShThreads);
    int32_t row0;
    float mean[3];
    const bool vis =
        sh_rows_prologue<DEG>(a, r0, nrows, s_buf, s_vis, &row0, mean);
    const int t = threadIdx.x;
    const int64_t bg = r0 + t;
    float acc[S::ROW];
#pragma unroll
    for (int k = 0; k < S::ROW; ++k)
        acc[k] = 0.f;
    float vm0 = 0.f, vm1 = 0.f, vm2 = 0.f;
    if (vis) {
        const int64_t b = bg / a.N, g = bg - b * a.N;
        const float mx = mean[0], my = mean[1], mz = mean[2];
        const float *cf = s_buf + t * S::PITCH;
        for (int64_t c = 0; c < a.C; ++c) {
            const int32_t r = c == 0 ? row0 : a.row_of[(b * a.C + c) * a.N + g];
            if (r < 0)
                continue;
            float Y[S::NB];
            float x = 0.f, y = 0.f, z = 0.f, inorm = 0.f;
            if (DEG > 0) {
                float cp[3];
                camera_centre(a.viewmats + (b * a.C + c) * 16, cp);
                const float dx = mx - cp[0], dy = my - cp[1], dz = mz - cp[2];
                inorm = 1.f / sqrtf(dx * dx + dy * dy + dz * dz);
                x = dx * inorm;
                y = dy * inorm;
                z = dz * inorm;
                sh_basis<DEG>(x, y, z, Y);
            } else {
                Y[0] = kY0;
            }
            // colour value again for the clamp's gradient mask
            float o0 = 0.f, o1 = 0.f, o2 = 0.f;
#pragma unroll
            for (int k = 0; k < S::NB; ++k) {
                o0 += Y[k] * cf[k * 3 + 0];
                o1 += Y[k] * cf[k * 3 + 1];
                o2 += Y[k] * cf[k * 3 + 2];
            }
            const float w0 = v_colors[(int64_t)r * 3 + 0];
            const float w1 = v_colors[(int64_t)r * 3 + 1];
            const float w2 = v_colors[(int64_t)r * 3 + 2];
            const float v0 = o0 + 0.5f >= 0.f ? w0 : 0.f;
            const float v1 = o1 + 0.5f >= 0.f ? w1 : 0.f;
            const float v2 = o2 + 0.5f >= 0.f ? w2 : 0.f;
#pragma unroll
            for (int k = 0; k < S::NB; ++k) {
                acc[k * 3 + 0] += Y[k] * v0;
                acc[k * 3 + 1] += Y[k] * v1;
                acc[k * 3 + 2] += Y[k] * v2;
            }
            if (DEG > 0) {
                float G[S::NB];
#pragma unroll
                for (int k = 0; k < S::NB; ++k)
                    G[k] = cf[k * 3 + 0] * v0 + cf[k * 3 + 1] * v1 +
                           cf[k * 3 + 2] * v2;
                float gx, gy, gz;
                sh_basis_grad<DEG>(x, y, z, G, gx, gy, gz);
                const float dot = gx * x + gy * y + gz * z;
                vm0 += (gx - dot * x) * inorm;
                vm1 += (gy - dot * y) * inorm;
                vm2 += (gz - dot * z) * inorm;
            }
        }
    }
    vm[0] = vm0;
    vm[1] = vm1;
    vm[2] = vm2;
    __syncthreads();  // every thread is done reading its staged coefficients
    if (t < nrows) {
        float *o = s_buf + t * S::PITCH;
        if constexpr (S::VEC) {
#pragma unroll
            for (int k = 0; k < S::ROW; k += 4)
                *reinterpret_cast<float4 *>(o + k) =
                    make_float4(acc[k], acc[k + 1], acc[k + 2], acc[k + 3]);
        } else {
#pragma unroll
            for (int k = 0; k < S::ROW; ++k)
                o[k] = acc[k];
        }
    }
    __syncthreads();
    const int rowlen = a.K * 3;
    const int total = nrows * rowlen;
    float *dst = v_coeffs + r0 * rowlen;
    if (a.vec_ok) {
        float4 *dst4 = reinterpret_cast<float4 *>(dst);
        const int nvec = total >> 2;
        for (int v = threadIdx.x; v < nvec; v += kShThreads)
            dst4[v] = staged_chunk<DEG>(s_buf, v << 2);
        for (int e = (nvec << 2) + threadIdx.x; e < total; e += kShThreads) {
            const int rr = e / S::ROW;
            dst[e] = s_buf[rr * S::PITCH + (e - rr * S::ROW)];
        }
    } else {
        for (int e = threadIdx.x; e < total; e += kShThreads) {
            const int rr = e / rowlen;
            const int col = e - rr * rowlen;
            dst[e] = col < S::ROW ? s_buf[rr * S::PITCH + col] : 0.f;
        }
    }
}

}  // namespace
}  // namespace gs
