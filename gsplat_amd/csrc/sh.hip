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

template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_fwd_kernel(int64_t M, int K, const float *__restrict__ dirs,
                  const float *__restrict__ coeffs,
                  const uint8_t *__restrict__ masks, float *__restrict__ colors,
                  bool vec_ok) {
    using S = ShShape<DEG>;
    __shared__ alignas(16) float s_coef[kShThreads * S::PITCH];
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
    __shared__ alignas(16) float s_buf[kShThreads * S::PITCH];
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
        stage_coeffs<DEG, true>(coeffs, r0, nrows, K, vec_ok, s_buf);
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
        float g[S::ROW];
#pragma unroll
        for (int k = 0; k < S::NB; ++k) {
            g[k * 3 + 0] = active ? Y[k] * vc0 : 0.f;
            g[k * 3 + 1] = active ? Y[k] * vc1 : 0.f;
            g[k * 3 + 2] = active ? Y[k] * vc2 : 0.f;
        }
        float *o = s_buf + t * S::PITCH;
        if constexpr (S::VEC) {
#pragma unroll
            for (int k = 0; k < S::ROW; k += 4)
                *reinterpret_cast<float4 *>(o + k) =
                    make_float4(g[k], g[k + 1], g[k + 2], g[k + 3]);
        } else {
#pragma unroll
            for (int k = 0; k < S::ROW; ++k)
                o[k] = g[k];
        }
    }
    __syncthreads();
    const int rowlen = K * 3;
    const int total = nrows * rowlen;
    float *dst = v_coeffs + r0 * rowlen;
    if (vec_ok && K == S::NB) {
        float4 *dst4 = reinterpret_cast<float4 *>(dst);
        const int nvec = total >> 2;
        for (int v = threadIdx.x; v < nvec; v += kShThreads)
            dst4[v] = staged_chunk<DEG>(s_buf, v << 2);
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
// One thread per Gaussian (sh_rows_fwd_row, sh_rows.h).
template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_rows_fwd_kernel(const ShRowsArgs a, float *__restrict__ colors) {
    sh_rows_fwd_row<DEG>(a, colors, (int64_t)blockIdx.x * kShThreads + threadIdx.x);
}

// One thread per Gaussian (sh_rows_bwd_block, sh_rows.h).
template <int DEG>
__global__ void __launch_bounds__(kShThreads)
    sh_rows_bwd_kernel(const ShRowsArgs a, const float *__restrict__ v_colors,
                       float *__restrict__ v_coeffs,
                       float *__restrict__ v_means) {
    const int64_t r0 = (int64_t)blockIdx.x * kShThreads;
    float vm[3];
    sh_rows_bwd_block<DEG>(a, v_colors, v_coeffs, r0, vm);
    const int64_t bg = r0 + threadIdx.x;
    if (bg < a.B * a.N) {
        v_means[bg * 3 + 0] = vm[0];
        v_means[bg * 3 + 1] = vm[1];
        v_means[bg * 3 + 2] = vm[2];
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
