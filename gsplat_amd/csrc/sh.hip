// Real spherical-harmonics colour evaluation, forward and backward.
//
// Semantics: gsplat/cuda/csrc/SphericalHarmonicsCUDA.cu:37-388 (the Sloan 2013
// basis up to degree 4, evaluated at the normalised direction) and the launch
// wrappers :391-552.  colors[c] = sum_k Y_k(dir/|dir|) * coeffs[k][c].
//
// MI355X design: the coefficient rows ([M, K, 3], 192 B per row at K = 16)
// are the HBM stream.  A 256-row workgroup copies its contiguous coefficient
// span into LDS with 16-byte loads (1 KiB per wave instruction), then every
// thread evaluates one row -- all three channels -- from LDS.  Rows are padded
// to an odd LDS pitch so the per-row reads are bank-conflict free.  The
// backward writes the full [M, K, 3] gradient (zeros above the used degree and
// for masked rows) through the same LDS tile with 16-byte stores, so the
// caller needs no zero fill.  One thread per row also makes the direction
// gradient a plain store instead of the reference's per-channel atomics.
#include "sh_rows.h"

namespace gs {
namespace {

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
// memory once per tile instead of once per 16-byte chunk.
template <int DEG>
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
            q[i] = take ? src[v] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((int)threadIdx.x + i * kShThreads >= nvec)
                break;
            const int e = ((int)threadIdx.x + i * kShThreads) << 2;
            const float vals[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int ek = e + k;
                const int row = ek / S::ROW;
                s[row * S::PITCH + (ek - row * S::ROW)] = vals[k];
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

template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_fwd_kernel(int64_t M, int K, const float *__restrict__ dirs,
                  const float *__restrict__ coeffs,
                  const uint8_t *__restrict__ masks, float *__restrict__ colors,
                  bool vec_ok) {
    using S = ShShape<DEG>;
    __shared__ float s_coef[kShThreads * S::PITCH];
    const int64_t r0 = (int64_t)blockIdx.x * kShThreads;
    const int nrows = (int)((M - r0) < kShThreads ? (M - r0) : kShThreads);
    stage_coeffs<DEG>(coeffs, r0, nrows, K, vec_ok, s_coef);
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= nrows)
        return;
    const int64_t row = r0 + t;
    float out0 = 0.f, out1 = 0.f, out2 = 0.f;
    if (masks == nullptr || masks[row]) {
        float Y[S::NB];
        if (DEG > 0) {
            const float dx = dirs[row * 3 + 0], dy = dirs[row * 3 + 1],
                        dz = dirs[row * 3 + 2];
            const float inorm = 1.f / sqrtf(dx * dx + dy * dy + dz * dz);
            sh_basis<DEG>(dx * inorm, dy * inorm, dz * inorm, Y);
        } else {
            Y[0] = kY0;
        }
        const float *c = s_coef + t * S::PITCH;
#pragma unroll
        for (int k = 0; k < S::NB; ++k) {
            out0 += Y[k] * c[k * 3 + 0];
            out1 += Y[k] * c[k * 3 + 1];
            out2 += Y[k] * c[k * 3 + 2];
        }
    }
    colors[row * 3 + 0] = out0;
    colors[row * 3 + 1] = out1;
    colors[row * 3 + 2] = out2;
}

template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_bwd_kernel(int64_t M, int K, const float *__restrict__ dirs,
                  const float *__restrict__ coeffs,
                  const uint8_t *__restrict__ masks,
                  const float *__restrict__ v_colors,
                  float *__restrict__ v_coeffs, float *__restrict__ v_dirs,
                  bool vec_ok) {
    using S = ShShape<DEG>;
    __shared__ float s_buf[kShThreads * S::PITCH];
    const int64_t r0 = (int64_t)blockIdx.x * kShThreads;
    const int nrows = (int)((M - r0) < kShThreads ? (M - r0) : kShThreads);
    const int t = threadIdx.x;
    const int64_t row = r0 + t;
    const bool in_range = t < nrows;
    const bool active = in_range && (masks == nullptr || masks[row]);

    float vc0 = 0.f, vc1 = 0.f, vc2 = 0.f, x = 0.f, y = 0.f, z = 0.f,
          inorm = 0.f;
    if (active) {
        vc0 = v_colors[row * 3 + 0];
        vc1 = v_colors[row * 3 + 1];
        vc2 = v_colors[row * 3 + 2];
        if (DEG > 0) {
            const float dx = dirs[row * 3 + 0], dy = dirs[row * 3 + 1],
                        dz = dirs[row * 3 + 2];
            inorm = 1.f / sqrtf(dx * dx + dy * dy + dz * dz);
            x = dx * inorm;
            y = dy * inorm;
            z = dz * inorm;
        }
    }
    // direction gradient needs the coefficients
    if (DEG > 0 && v_dirs != nullptr) {
        stage_coeffs<DEG>(coeffs, r0, nrows, K, vec_ok, s_buf);
        __syncthreads();
        if (in_range) {
            float vdx = 0.f, vdy = 0.f, vdz = 0.f;
            if (active) {
                float G[S::NB];
                const float *c = s_buf + t * S::PITCH;
#pragma unroll
                for (int k = 0; k < S::NB; ++k)
                    G[k] = c[k * 3 + 0] * vc0 + c[k * 3 + 1] * vc1 +
                           c[k * 3 + 2] * vc2;
                float gx, gy, gz;
                sh_basis_grad<DEG>(x, y, z, G, gx, gy, gz);
                const float dot = gx * x + gy * y + gz * z;
                vdx = (gx - dot * x) * inorm;
                vdy = (gy - dot * y) * inorm;
                vdz = (gz - dot * z) * inorm;
            }
            v_dirs[row * 3 + 0] = vdx;
            v_dirs[row * 3 + 1] = vdy;
            v_dirs[row * 3 + 2] = vdz;
        }
        __syncthreads();
    } else if (v_dirs != nullptr && in_range) {
        v_dirs[row * 3 + 0] = 0.f;
        v_dirs[row * 3 + 1] = 0.f;
        v_dirs[row * 3 + 2] = 0.f;
    }

    // v_coeffs[k][c] = Y_k * v_c, staged in LDS then streamed out
    if (in_range) {
        float Y[S::NB];
        if (DEG > 0)
            sh_basis<DEG>(x, y, z, Y);
        else
            Y[0] = kY0;
        float *o = s_buf + t * S::PITCH;
#pragma unroll
        for (int k = 0; k < S::NB; ++k) {
            o[k * 3 + 0] = active ? Y[k] * vc0 : 0.f;
            o[k * 3 + 1] = active ? Y[k] * vc1 : 0.f;
            o[k * 3 + 2] = active ? Y[k] * vc2 : 0.f;
        }
    }
    __syncthreads();
    const int rowlen = K * 3;
    const int total = nrows * rowlen;
    float *dst = v_coeffs + r0 * rowlen;
    if (vec_ok && K == S::NB) {
        float4 *dst4 = reinterpret_cast<float4 *>(dst);
        const int nvec = total >> 2;
        for (int v = threadIdx.x; v < nvec; v += kShThreads) {
            const int e = v << 2;
            float vals[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int ek = e + k;
                const int r = ek / S::ROW;
                vals[k] = s_buf[r * S::PITCH + (ek - r * S::ROW)];
            }
            dst4[v] = make_float4(vals[0], vals[1], vals[2], vals[3]);
        }
        for (int e = (nvec << 2) + threadIdx.x; e < total; e += kShThreads) {
            const int r = e / S::ROW;
            dst[e] = s_buf[r * S::PITCH + (e - r * S::ROW)];
        }
    } else {
        for (int e = threadIdx.x; e < total; e += kShThreads) {
            const int r = e / rowlen;
            const int col = e - r * rowlen;
            dst[e] = col < S::ROW ? s_buf[r * S::PITCH + col] : 0.f;
        }
    }
}

// ---------------------------------------------------------------------------
// SH over packed rows, driven by Gaussian.
//
// The packed layout keeps one row per visible (camera, Gaussian) pair; the
// reference gathers [nnz, K, 3] coefficients and view directions for them
// and scatters the gradients back with index_put (rendering.py:227-253,
// 845-873).  Here each thread owns one Gaussian (b, g): its coefficients are
// staged once (coalesced, skipped when it is visible in no camera) and it
// loops over the C cameras through row_of[(b C + c) N + g] (the packed row,
// or -1).  The forward writes colors[row] = max(SH(dir) + 0.5, 0) with
// dir = mean - campos, campos = -R^T t of the camera (rendering.py:872,
// taken from the view matrix in the kernel); the backward accumulates the
// coefficient and mean gradients over the cameras in registers and writes
// every Gaussian's gradient row once -- deterministic, no atomics, no
// zero fill.
// ---------------------------------------------------------------------------
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
    stage_coeffs<DEG>(a.coeffs, r0, nrows, a.K, a.vec_ok, s_coef, s_vis);
    __syncthreads();
    return vis;
}

// One thread per Gaussian (sh_rows_fwd_row, sh_rows.h).
template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_rows_fwd_kernel(const ShRowsArgs a, float *__restrict__ colors) {
    sh_rows_fwd_row<DEG>(a, colors, (int64_t)blockIdx.x * kShThreads + threadIdx.x);
}

template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_rows_bwd_kernel(const ShRowsArgs a, const float *__restrict__ v_colors,
                       float *__restrict__ v_coeffs,
                       float *__restrict__ v_means) {
    using S = ShShape<DEG>;
    __shared__ float s_buf[kShThreads * S::PITCH];
    __shared__ uint8_t s_vis[kShThreads];
    const int64_t r0 = (int64_t)blockIdx.x * kShThreads;
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
    if (t < nrows) {
        v_means[bg * 3 + 0] = vm0;
        v_means[bg * 3 + 1] = vm1;
        v_means[bg * 3 + 2] = vm2;
    }
    __syncthreads();  // every thread is done reading its staged coefficients
    if (t < nrows) {
        float *o = s_buf + t * S::PITCH;
#pragma unroll
        for (int k = 0; k < S::ROW; ++k)
            o[k] = acc[k];
    }
    __syncthreads();
    const int rowlen = a.K * 3;
    const int total = nrows * rowlen;
    float *dst = v_coeffs + r0 * rowlen;
    if (a.vec_ok) {
        float4 *dst4 = reinterpret_cast<float4 *>(dst);
        const int nvec = total >> 2;
        for (int v = threadIdx.x; v < nvec; v += kShThreads) {
            const int e = v << 2;
            float vals[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int ek = e + k;
                const int rr = ek / S::ROW;
                vals[k] = s_buf[rr * S::PITCH + (ek - rr * S::ROW)];
            }
            dst4[v] = make_float4(vals[0], vals[1], vals[2], vals[3]);
        }
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

using namespace gs;

#define GS_SH_LAUNCH(KERNEL, DEG, ...)                                         \
    KERNEL<DEG><<<grid, kShThreads, 0, st>>>(__VA_ARGS__)

extern "C" int gsplat_sh_fwd(int64_t M, int32_t K, int32_t degree,
                             const float *dirs, const float *coeffs,
                             const uint8_t *masks, float *colors,
                             gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(M >= 0, "sh_fwd: negative M");
    GS_REQUIRE(degree >= 0 && degree <= 4, "sh_fwd: degree must be in [0, 4]");
    GS_REQUIRE((degree + 1) * (degree + 1) <= K,
               "sh_fwd: K must be >= (degree + 1)^2");
    if (M == 0)
        return GSPLAT_OK;
    GS_REQUIRE(coeffs && colors && (degree == 0 || dirs), "sh_fwd: NULL buffer");
    const int nb = (degree + 1) * (degree + 1);
    const bool vec_ok = (K == nb) && aligned16(coeffs);
    const dim3 grid((unsigned)ceil_div(M, kShThreads));
    hipStream_t st = as_stream(stream);
    switch (degree) {
    case 0: GS_SH_LAUNCH(sh_fwd_kernel, 0, M, K, dirs, coeffs, masks, colors, vec_ok); break;
    case 1: GS_SH_LAUNCH(sh_fwd_kernel, 1, M, K, dirs, coeffs, masks, colors, vec_ok); break;
    case 2: GS_SH_LAUNCH(sh_fwd_kernel, 2, M, K, dirs, coeffs, masks, colors, vec_ok); break;
    case 3: GS_SH_LAUNCH(sh_fwd_kernel, 3, M, K, dirs, coeffs, masks, colors, vec_ok); break;
    default: GS_SH_LAUNCH(sh_fwd_kernel, 4, M, K, dirs, coeffs, masks, colors, vec_ok); break;
    }
    return check_launch("sh_fwd_kernel");
}

extern "C" int gsplat_sh_bwd(int64_t M, int32_t K, int32_t degree,
                             const float *dirs, const float *coeffs,
                             const uint8_t *masks, const float *v_colors,
                             float *v_coeffs, float *v_dirs,
                             gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(M >= 0, "sh_bwd: negative M");
    GS_REQUIRE(degree >= 0 && degree <= 4, "sh_bwd: degree must be in [0, 4]");
    GS_REQUIRE((degree + 1) * (degree + 1) <= K,
               "sh_bwd: K must be >= (degree + 1)^2");
    if (M == 0)
        return GSPLAT_OK;
    GS_REQUIRE(coeffs && v_colors && v_coeffs && (degree == 0 || dirs),
               "sh_bwd: NULL buffer");
    const int nb = (degree + 1) * (degree + 1);
    const bool vec_ok = (K == nb) && aligned16(coeffs) && aligned16(v_coeffs);
    const dim3 grid((unsigned)ceil_div(M, kShThreads));
    hipStream_t st = as_stream(stream);
    switch (degree) {
    case 0: GS_SH_LAUNCH(sh_bwd_kernel, 0, M, K, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs, vec_ok); break;
    case 1: GS_SH_LAUNCH(sh_bwd_kernel, 1, M, K, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs, vec_ok); break;
    case 2: GS_SH_LAUNCH(sh_bwd_kernel, 2, M, K, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs, vec_ok); break;
    case 3: GS_SH_LAUNCH(sh_bwd_kernel, 3, M, K, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs, vec_ok); break;
    default: GS_SH_LAUNCH(sh_bwd_kernel, 4, M, K, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs, vec_ok); break;
    }
    return check_launch("sh_bwd_kernel");
}

#define GS_SH_ROWS_LAUNCH(KERNEL, DEG, ...)                                    \
    KERNEL<DEG><<<grid, kShThreads, 0, st>>>(__VA_ARGS__)

static int sh_rows_check(int64_t B, int64_t C, int64_t N, int32_t K,
                         int32_t degree, const float *means, const float *viewmats,
                         const float *coeffs, const int32_t *row_of) {
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0, "sh_rows: negative size");
    GS_REQUIRE(degree >= 0 && degree <= 4, "sh_rows: degree must be in [0, 4]");
    GS_REQUIRE((degree + 1) * (degree + 1) <= K,
               "sh_rows: K must be >= (degree + 1)^2");
    if (B * N > 0)
        GS_REQUIRE(means && viewmats && coeffs && row_of, "sh_rows: NULL input");
    return GSPLAT_OK;
}

extern "C" int gsplat_sh_rows_fwd(int64_t B, int64_t C, int64_t N, int32_t K,
                                  int32_t degree, const float *means,
                                  const float *viewmats, const float *coeffs,
                                  const int32_t *row_of, float *colors,
                                  gsplat_stream_t stream) {
    clear_error();
    GS_TRY(sh_rows_check(B, C, N, K, degree, means, viewmats, coeffs, row_of));
    if (B * N == 0 || C == 0)
        return GSPLAT_OK;
    GS_REQUIRE(colors != nullptr, "sh_rows_fwd: NULL colors");
    const int nb = (degree + 1) * (degree + 1);
    ShRowsArgs a{B, C, N, K, means, viewmats, coeffs, row_of,
                 (K == nb) && aligned16(coeffs)};
    const dim3 grid((unsigned)ceil_div(B * N, kShThreads));
    hipStream_t st = as_stream(stream);
    switch (degree) {
    case 0: GS_SH_ROWS_LAUNCH(sh_rows_fwd_kernel, 0, a, colors); break;
    case 1: GS_SH_ROWS_LAUNCH(sh_rows_fwd_kernel, 1, a, colors); break;
    case 2: GS_SH_ROWS_LAUNCH(sh_rows_fwd_kernel, 2, a, colors); break;
    case 3: GS_SH_ROWS_LAUNCH(sh_rows_fwd_kernel, 3, a, colors); break;
    default: GS_SH_ROWS_LAUNCH(sh_rows_fwd_kernel, 4, a, colors); break;
    }
    return check_launch("sh_rows_fwd_kernel");
}

extern "C" int gsplat_sh_rows_bwd(int64_t B, int64_t C, int64_t N, int32_t K,
                                  int32_t degree, const float *means,
                                  const float *viewmats, const float *coeffs,
                                  const int32_t *row_of, const float *v_colors,
                                  float *v_coeffs, float *v_means,
                                  gsplat_stream_t stream) {
    clear_error();
    GS_TRY(sh_rows_check(B, C, N, K, degree, means, viewmats, coeffs, row_of));
    if (B * N == 0)
        return GSPLAT_OK;
    GS_REQUIRE(v_coeffs && v_means, "sh_rows_bwd: NULL output");
    GS_REQUIRE(C == 0 || v_colors != nullptr, "sh_rows_bwd: NULL v_colors");
    const int nb = (degree + 1) * (degree + 1);
    ShRowsArgs a{B, C, N, K, means, viewmats, coeffs, row_of,
                 (K == nb) && aligned16(coeffs) && aligned16(v_coeffs)};
    const dim3 grid((unsigned)ceil_div(B * N, kShThreads));
    hipStream_t st = as_stream(stream);
    switch (degree) {
    case 0: GS_SH_ROWS_LAUNCH(sh_rows_bwd_kernel, 0, a, v_colors, v_coeffs, v_means); break;
    case 1: GS_SH_ROWS_LAUNCH(sh_rows_bwd_kernel, 1, a, v_colors, v_coeffs, v_means); break;
    case 2: GS_SH_ROWS_LAUNCH(sh_rows_bwd_kernel, 2, a, v_colors, v_coeffs, v_means); break;
    case 3: GS_SH_ROWS_LAUNCH(sh_rows_bwd_kernel, 3, a, v_colors, v_coeffs, v_means); break;
    default: GS_SH_ROWS_LAUNCH(sh_rows_bwd_kernel, 4, a, v_colors, v_coeffs, v_means); break;
    }
    return check_launch("sh_rows_bwd_kernel");
}
