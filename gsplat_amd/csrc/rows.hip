// Per-Gaussian features to packed rows and back.
//
// The packed layout (one row per visible (b, c, g), gsplat/cuda/csrc/
// ProjectionEWA3DGSPacked.cu:234-284) makes rasterization() gather
// per-Gaussian features into rows -- opacities[batch_ids, gaussian_ids],
// colors[batch_ids, gaussian_ids] (gsplat/rendering.py:782, 170-213) -- and
// autograd scatter the row gradients back with index_put(accumulate=True),
// which PyTorch runs as a sort plus a segmented sum.
//
// Both directions here are driven by Gaussian through the inverse map
// row_of[(b C + c) N + g] (packed row or -1) that the packed projection
// writes: the gather reads each Gaussian's feature row once and stores it to
// its rows; the scatter sums a Gaussian's row gradients over the C cameras in
// camera order and writes its gradient row once (zeros when it is visible
// nowhere).  Deterministic, no atomics, no zero fill; consecutive threads
// take consecutive Gaussians, so the per-Gaussian streams are coalesced.
#include "common.h"

namespace gs {
namespace {

constexpr int kRowsThreads = 256;

__global__ void __launch_bounds__(kRowsThreads)
    rows_gather_kernel(int64_t B, int64_t C, int64_t N, int F,
                       const float *__restrict__ src,
                       const int32_t *__restrict__ row_of,
                       float *__restrict__ out) {
    const int64_t bg = (int64_t)blockIdx.x * kRowsThreads + threadIdx.x;
    if (bg >= B * N)
        return;
    const int64_t b = bg / N, g = bg - b * N;
    const float *s = src + bg * F;
    for (int64_t c = 0; c < C; ++c) {
        const int32_t r = row_of[(b * C + c) * N + g];
        if (r < 0)
            continue;
        float *o = out + (int64_t)r * F;
        for (int f = 0; f < F; ++f)
            o[f] = s[f];
    }
}

template <int F>
__global__ void __launch_bounds__(kRowsThreads)
    rows_scatter_kernel_fixed(int64_t B, int64_t C, int64_t N,
                              const int32_t *__restrict__ row_of,
                              const float *__restrict__ v_out,
                              float *__restrict__ v_src) {
    const int64_t bg = (int64_t)blockIdx.x * kRowsThreads + threadIdx.x;
    if (bg >= B * N)
        return;
    const int64_t b = bg / N, g = bg - b * N;
    float acc[F];
#pragma unroll
    for (int f = 0; f < F; ++f)
        acc[f] = 0.f;
    for (int64_t c = 0; c < C; ++c) {
        const int32_t r = row_of[(b * C + c) * N + g];
        if (r < 0)
            continue;
#pragma unroll
        for (int f = 0; f < F; ++f)
            acc[f] += v_out[(int64_t)r * F + f];
    }
#pragma unroll
    for (int f = 0; f < F; ++f)
        v_src[bg * F + f] = acc[f];
}

__global__ void __launch_bounds__(kRowsThreads)
    rows_scatter_kernel(int64_t B, int64_t C, int64_t N, int F,
                        const int32_t *__restrict__ row_of,
                        const float *__restrict__ v_out,
                        float *__restrict__ v_src) {
    const int64_t bg = (int64_t)blockIdx.x * kRowsThreads + threadIdx.x;
    if (bg >= B * N)
        return;
    const int64_t b = bg / N, g = bg - b * N;
    float *d = v_src + bg * F;
    for (int f = 0; f < F; ++f)
        d[f] = 0.f;
    for (int64_t c = 0; c < C; ++c) {
        const int32_t r = row_of[(b * C + c) * N + g];
        if (r < 0)
            continue;
        for (int f = 0; f < F; ++f)
            d[f] += v_out[(int64_t)r * F + f];
    }
}

int rows_check(int64_t B, int64_t C, int64_t N, int32_t F, const int32_t *row_of) {
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0 && F >= 0, "rows: negative size");
    if (B * C * N > 0)
        GS_REQUIRE(row_of != nullptr, "rows: NULL row_of");
    return GSPLAT_OK;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gsplat_rows_gather(int64_t B, int64_t C, int64_t N, int32_t F,
                                  const float *src, const int32_t *row_of,
                                  float *out, gsplat_stream_t stream) {
    clear_error();
    GS_TRY(rows_check(B, C, N, F, row_of));
    if (B * N == 0 || C == 0 || F == 0)
        return GSPLAT_OK;
    GS_REQUIRE(src && out, "rows_gather: NULL buffer");
    rows_gather_kernel<<<(unsigned)ceil_div(B * N, kRowsThreads), kRowsThreads,
                         0, as_stream(stream)>>>(B, C, N, F, src, row_of, out);
    return check_launch("rows_gather_kernel");
}

extern "C" int gsplat_rows_scatter_sum(int64_t B, int64_t C, int64_t N,
                                       int32_t F, const int32_t *row_of,
                                       const float *v_out, float *v_src,
                                       gsplat_stream_t stream) {
    clear_error();
    GS_TRY(rows_check(B, C, N, F, row_of));
    if (B * N == 0 || F == 0)
        return GSPLAT_OK;
    GS_REQUIRE(v_src != nullptr && (C == 0 || v_out != nullptr),
               "rows_scatter_sum: NULL buffer");
    const unsigned grid = (unsigned)ceil_div(B * N, kRowsThreads);
    hipStream_t st = as_stream(stream);
    switch (F) {
    case 1:
        rows_scatter_kernel_fixed<1><<<grid, kRowsThreads, 0, st>>>(B, C, N, row_of, v_out, v_src);
        break;
    case 3:
        rows_scatter_kernel_fixed<3><<<grid, kRowsThreads, 0, st>>>(B, C, N, row_of, v_out, v_src);
        break;
    default:
        rows_scatter_kernel<<<grid, kRowsThreads, 0, st>>>(B, C, N, F, row_of, v_out, v_src);
        break;
    }
    return check_launch("rows_scatter_kernel");
}
