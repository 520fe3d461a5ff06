// Densification statistics: the running-state update of
// gsplat/strategy/default.py:218-268 (DefaultStrategy._update_state) in one
// pass over the rows.  Per visible (camera, Gaussian) row:
//   grad2d[g] += || (gx * W/2 * C, gy * H/2 * C) ||,   count[g] += 1
// where (gx, gy) is the row's 2D mean gradient (absgrad or grad).  The
// reference runs it as clone, two column scales, a norm and two index_add_
// launches over the [nnz, 2] gradient; here the gradient is read once.
#include "common.h"

namespace gs {
namespace {

constexpr int kStatsThreads = 256;

// N Gaussians; rows: packed (gaussian_ids given: row r belongs to Gaussian
// ids[r]) or dense [C, N] (row r = c * N + g, counted only where both radii
// are > 0).
__global__ void __launch_bounds__(kStatsThreads)
    grad2d_stats_kernel(int64_t n_rows, int64_t N, const float *__restrict__ grads,
                        const int64_t *__restrict__ gaussian_ids,
                        const int32_t *__restrict__ radii, float scale_x,
                        float scale_y, float *__restrict__ grad2d,
                        float *__restrict__ count) {
    const int64_t r = (int64_t)blockIdx.x * kStatsThreads + threadIdx.x;
    if (r >= n_rows)
        return;
    int64_t g;
    if (gaussian_ids != nullptr) {
        g = gaussian_ids[r];
        if (g < 0 || g >= N)  // not a Gaussian of this batch
            return;
    } else {
        if (!(radii[2 * r] > 0 && radii[2 * r + 1] > 0))
            return;
        g = r % N;
    }
    // two scalar loads: the gradient may be a 4-byte-aligned view
    const float x = grads[2 * r] * scale_x, y = grads[2 * r + 1] * scale_y;
    atomic_add_f32(grad2d + g, sqrtf(x * x + y * y));
    atomic_add_f32(count + g, 1.f);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gsplat_grad2d_stats(int64_t n_rows, int64_t N, const float *grads,
                                   const int64_t *gaussian_ids, const int32_t *radii,
                                   float scale_x, float scale_y, float *grad2d,
                                   float *count, gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(n_rows >= 0 && N >= 0, "grad2d_stats: negative size");
    if (n_rows == 0)
        return GSPLAT_OK;
    GS_REQUIRE(grads && grad2d && count, "grad2d_stats: NULL buffer");
    GS_REQUIRE(N > 0, "grad2d_stats: N must be positive");
    GS_REQUIRE(gaussian_ids != nullptr || radii != nullptr,
               "grad2d_stats: dense rows need radii");
    hipStream_t st = as_stream(stream);
    grad2d_stats_kernel<<<(unsigned)ceil_div(n_rows, kStatsThreads), kStatsThreads,
                          0, st>>>(n_rows, N, grads, gaussian_ids, radii, scale_x,
                                   scale_y, grad2d, count);
    return check_launch("grad2d_stats_kernel");
}
