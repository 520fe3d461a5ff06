// Tile rasterizer: front-to-back alpha compositing (forward) and its
// back-to-front replay (backward).
//
// Semantics: gsplat/cuda/csrc/RasterizeToPixels3DGSFwd.cu:41-213 and
// RasterizeToPixels3DGSBwd.cu:39-301.  Per pixel (px, py) = (j + .5, i + .5),
// for the depth-sorted Gaussians of its tile:
//   sigma = 0.5 (a dx^2 + c dy^2) + b dx dy,  dx = mean.x - px, dy = mean.y - py
//   alpha = min(0.99, o exp(-sigma)); skipped if sigma < 0 or alpha < 1/255
//   stop (exclusive) once T (1 - alpha) <= 1e-4;  C += c alpha T;  T *= 1 - alpha
//   colors = C + T bg, alphas = 1 - T, last_ids = isect index of the last
//   Gaussian composited (0 if none).
//
// The two discontinuous decisions that depend on exp() are taken on sigma
// against per-Gaussian thresholds computed once per tile load:
//   alpha < 1/255     <=>  sigma > ln(o / (1/255))          ("sig_max")
//   o exp(-sigma) > .99 <=> sigma < ln(o / 0.99)            ("sig_clamp")
// sigma is evaluated in a fixed IEEE order without contraction, the logs are
// portable_logf and exp(-sigma) is portable_expf (below 1 ulp, built from
// correctly rounded operations only), so alpha, the running transmittance
// and every compositing decision -- the set of composited Gaussians, the
// termination point, last_ids -- are reproducible bit for bit by the host
// oracle.
//
// MI355X design: one workgroup per tile (tile_size^2 threads = 4 waves at
// 16x16, each wave a 16x4 pixel strip), Gaussians staged in LDS in batches of
// one per thread (float4 geometry, float4 thresholds+conic, CDIM colours).
// The forward ends a batch early when every pixel of the wave is done (the
// per-lane loop exits when the wave's exec mask empties) and skips remaining
// batches once the whole tile is done (__syncthreads_count).
// The backward recovers T back to front in double (one Newton-refined
// reciprocal per Gaussian), reduces each Gaussian's gradient over the wave
// with a branch-free DPP reduction (row butterflies + row broadcasts, total
// in the last lane), accumulates the waves in LDS (ds_add_f32) and issues
// one global atomic per value per Gaussian per TILE, 8x fewer than one per
// 32-lane warp.  Both kernels are compiled per (CDIM, tile size) so every
// loop bound and reduction count is a constant.
#include "common.h"

namespace gs {
namespace {

struct RasterArgs {
    int64_t I, n_rows, n_isects;
    const float *means2d, *conics, *colors, *opacities, *backgrounds;
    const uint8_t *masks;
    int32_t W, H, tile_size, tile_width, tile_height;
    const int32_t *tile_offsets, *flatten_ids;
};

// exact (uncontracted) Mahalanobis term; the host oracle uses this order
__device__ __forceinline__ float gauss_sigma(float a, float b, float c,
                                             float dx, float dy) {
#pragma clang fp contract(off)
    return 0.5f * ((a * dx) * dx + (c * dy) * dy) + (b * dx) * dy;
}

// per-Gaussian decision thresholds (see file comment)
__device__ __forceinline__ void alpha_thresholds(float o, float &sig_max,
                                                 float &sig_clamp) {
    if (o > 0.f) {
        sig_max = portable_logf(o / kAlphaThreshold);
        sig_clamp = portable_logf(o / kMaxAlpha);
    } else {
        sig_max = -__builtin_inff();  // zero or NaN opacity never composites
        sig_clamp = -__builtin_inff();
    }
}

__device__ __forceinline__ void tile_coords(const RasterArgs &a, int64_t &image,
                                            int32_t &tile, int32_t &ty,
                                            int32_t &tx) {
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;
    const int64_t gid = blockIdx.x;
    image = gid / n_tiles;
    tile = (int32_t)(gid - image * n_tiles);
    ty = tile / a.tile_width;
    tx = tile - ty * a.tile_width;
}

// 16-lane rows of a wave that hold pixels: 1 for 4x4 tiles (16 threads),
// 4 for 8x8 (one full wave) and 16x16 (four full waves).
template <int TILE> struct TileShape {
    static constexpr int BS = TILE * TILE;
    static constexpr int ROWS = BS >= 64 ? 4 : BS / 16;
    static constexpr int LAST = 16 * ROWS - 1;  // lane holding a wave sum
    static_assert(BS % 16 == 0, "tile must hold whole 16-lane rows");
};

template <int CDIM, int TILE>
__global__ void __launch_bounds__(TILE * TILE) rasterize_fwd_kernel(
    const RasterArgs a, float *__restrict__ render_colors,
    float *__restrict__ render_alphas, int32_t *__restrict__ last_ids,
    float *__restrict__ render_T) {
    constexpr int BS = TileShape<TILE>::BS;
    __shared__ float4 s_geo[BS];          // (x, y, opacity, sig_max)
    __shared__ float4 s_con[BS];          // (a, b, c, sig_clamp)
    __shared__ float s_col[BS * CDIM];

    int64_t image;
    int32_t tile, ty, tx;
    tile_coords(a, image, tile, ty, tx);
    const int tr = threadIdx.x;
    const int i = ty * TILE + tr / TILE;
    const int j = tx * TILE + tr % TILE;
    const bool inside = i < a.H && j < a.W;
    const int64_t pix = ((int64_t)image * a.H + i) * a.W + j;
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;

    if (a.masks != nullptr && !a.masks[image * n_tiles + tile]) {
        if (inside) {
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                render_colors[pix * CDIM + k] =
                    a.backgrounds ? a.backgrounds[image * CDIM + k] : 0.f;
            render_alphas[pix] = 0.f;
            last_ids[pix] = 0;
            if (render_T != nullptr)
                render_T[pix] = 1.f;
        }
        return;
    }

    const int32_t *offs = a.tile_offsets + image * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (image == a.I - 1 && tile == n_tiles - 1)
                                  ? (int32_t)a.n_isects
                                  : offs[tile + 1];
    const int num_batches = (range_end - range_start + BS - 1) / BS;

    float T = 1.f;
    int32_t cur_idx = 0;
    bool done = !inside;
    float acc[CDIM];
#pragma unroll
    for (int k = 0; k < CDIM; ++k)
        acc[k] = 0.f;

    for (int b = 0; b < num_batches; ++b) {
        if (__syncthreads_count(done) >= BS)
            break;
        const int32_t batch_start = range_start + b * BS;
        const int32_t idx = batch_start + tr;
        if (idx < range_end) {
            const int32_t g = a.flatten_ids[idx];
            const float2 xy = reinterpret_cast<const float2 *>(a.means2d)[g];
            const float o = a.opacities[g];
            float sig_max, sig_clamp;
            alpha_thresholds(o, sig_max, sig_clamp);
            s_geo[tr] = make_float4(xy.x, xy.y, o, sig_max);
            s_con[tr] = make_float4(a.conics[g * 3 + 0], a.conics[g * 3 + 1],
                                    a.conics[g * 3 + 2], sig_clamp);
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                s_col[tr * CDIM + k] = a.colors[(int64_t)g * CDIM + k];
        }
        __syncthreads();
        const int batch_size = min(BS, range_end - batch_start);
        for (int t = 0; t < batch_size && !done; ++t) {
            const float4 geo = s_geo[t];
            const float4 con = s_con[t];
            const float dx = geo.x - px, dy = geo.y - py;
            const float sigma = gauss_sigma(con.x, con.y, con.z, dx, dy);
            if (sigma < 0.f || sigma > geo.w)
                continue;
            const float vis = portable_expf(-sigma);
            const float alpha = sigma < con.w ? kMaxAlpha : geo.z * vis;
            const float next_T = T * (1.f - alpha);
            if (next_T <= kTransmittanceThreshold) {
                done = true;
                break;
            }
            const float w = alpha * T;
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                acc[k] += s_col[t * CDIM + k] * w;
            cur_idx = batch_start + t;
            T = next_T;
        }
    }
    if (inside) {
        render_alphas[pix] = 1.f - T;
#pragma unroll
        for (int k = 0; k < CDIM; ++k)
            render_colors[pix * CDIM + k] =
                a.backgrounds ? acc[k] + T * a.backgrounds[image * CDIM + k]
                              : acc[k];
        last_ids[pix] = cur_idx;
        if (render_T != nullptr)
            render_T[pix] = T;
    }
}

template <int CDIM, int TILE, bool ABS>
__global__ void __launch_bounds__(TILE * TILE) rasterize_bwd_kernel(
    const RasterArgs a, const float *__restrict__ render_alphas,
    const float *__restrict__ render_T, const int32_t *__restrict__ last_ids,
    const float *__restrict__ v_render_colors,
    const float *__restrict__ v_render_alphas,
    float *__restrict__ v_means2d_abs, float *__restrict__ v_means2d,
    float *__restrict__ v_conics, float *__restrict__ v_colors,
    float *__restrict__ v_opacities) {
    using TS = TileShape<TILE>;
    constexpr int BS = TS::BS;
    // per-Gaussian sums: xy(2), conic(3), colour(CDIM), opacity(1) [, |xy|(2)]
    constexpr int NACC = 2 + 3 + CDIM + 1 + (ABS ? 2 : 0);
    __shared__ float4 s_geo[BS];
    __shared__ float4 s_con[BS];
    __shared__ float s_col[BS * CDIM];
    __shared__ float s_acc[NACC * BS];
    __shared__ int32_t s_gid[BS];
    __shared__ int32_t s_hit[BS];

    int64_t image;
    int32_t tile, ty, tx;
    tile_coords(a, image, tile, ty, tx);
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;
    if (a.masks != nullptr && !a.masks[image * n_tiles + tile])
        return;
    const int tr = threadIdx.x;
    const int i = ty * TILE + tr / TILE;
    const int j = tx * TILE + tr % TILE;
    const bool inside = i < a.H && j < a.W;
    const int64_t pix = ((int64_t)image * a.H + (inside ? i : 0)) * a.W +
                        (inside ? j : 0);
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const bool last_lane = lane_id() == (uint32_t)TS::LAST;

    const int32_t *offs = a.tile_offsets + image * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (image == a.I - 1 && tile == n_tiles - 1)
                                  ? (int32_t)a.n_isects
                                  : offs[tile + 1];
    const int num_batches = (range_end - range_start + BS - 1) / BS;

    // The transmittance itself when the forward stored it: 1 - (1 - T)
    // loses most of T's significant bits once T nears the 1e-4 cutoff.
    const float T_final =
        inside ? (render_T != nullptr ? render_T[pix] : 1.f - render_alphas[pix])
               : 1.f;
    // T before each Gaussian is recovered back to front by undoing the
    // forward's products.  It is carried in double and each step multiplies
    // by 1 / (1 - alpha) refined to ~2^-46 by one Newton step from the fp32
    // reciprocal, so T keeps only the forward's own rounding instead of one
    // extra float32 rounding per Gaussian behind it.
    double T64 = (double)T_final;
    float T = T_final;
    const int32_t bin_final = inside ? last_ids[pix] : -1;
    float v_c[CDIM], buffer[CDIM];
    float bg_dot = 0.f;
#pragma unroll
    for (int k = 0; k < CDIM; ++k) {
        v_c[k] = inside ? v_render_colors[pix * CDIM + k] : 0.f;
        buffer[k] = 0.f;
        if (a.backgrounds)
            bg_dot += a.backgrounds[image * CDIM + k] * v_c[k];
    }
    const float v_a = inside ? v_render_alphas[pix] : 0.f;
    const int32_t wave_bin_final = wave_max_i32(bin_final);

    for (int b = 0; b < num_batches; ++b) {
        __syncthreads();
        const int32_t batch_end = range_end - 1 - b * BS;
        const int batch_size = min(BS, batch_end + 1 - range_start);
        const int32_t idx = batch_end - tr;
        if (idx >= range_start) {
            const int32_t g = a.flatten_ids[idx];
            s_gid[tr] = g;
            const float2 xy = reinterpret_cast<const float2 *>(a.means2d)[g];
            const float o = a.opacities[g];
            float sig_max, sig_clamp;
            alpha_thresholds(o, sig_max, sig_clamp);
            s_geo[tr] = make_float4(xy.x, xy.y, o, sig_max);
            s_con[tr] = make_float4(a.conics[g * 3 + 0], a.conics[g * 3 + 1],
                                    a.conics[g * 3 + 2], sig_clamp);
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                s_col[tr * CDIM + k] = a.colors[(int64_t)g * CDIM + k];
        }
        s_hit[tr] = 0;
#pragma unroll
        for (int k = 0; k < NACC; ++k)
            s_acc[k * BS + tr] = 0.f;
        __syncthreads();

        // slots t with isect index batch_end - t > wave_bin_final are behind
        // every pixel of this wave
        const int t0 = max(0, batch_end - wave_bin_final);
        for (int t = t0; t < batch_size; ++t) {
            const int32_t isect = batch_end - t;
            const float4 geo = s_geo[t];
            const float4 con = s_con[t];
            const float dx = geo.x - px, dy = geo.y - py;
            const float sigma = gauss_sigma(con.x, con.y, con.z, dx, dy);
            const bool valid = inside && isect <= bin_final && sigma >= 0.f &&
                               sigma <= geo.w;
            if (!__ballot(valid))
                continue;
            float g[NACC];
#pragma unroll
            for (int k = 0; k < NACC; ++k)
                g[k] = 0.f;
            if (valid) {
                const float vis = portable_expf(-sigma);
                const bool clamped = sigma < con.w;
                const float alpha = clamped ? kMaxAlpha : geo.z * vis;
                // alpha <= 0.99, so 1 - alpha >= 0.01 (the reference's
                // 1e-6 floor never binds)
                const float one_minus = fmaxf(kMinOneMinusAlpha, 1.f - alpha);
                const float ra = __builtin_amdgcn_rcpf(one_minus);
                const double d = (double)one_minus;
                double r = (double)ra;
                r = __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
                T64 = T64 * r;
                T = (float)T64;
                const float fac = alpha * T;
                float v_alpha = 0.f;
#pragma unroll
                for (int k = 0; k < CDIM; ++k) {
                    const float ck = s_col[t * CDIM + k];
                    g[5 + k] = fac * v_c[k];
                    v_alpha += (ck * T - buffer[k] * ra) * v_c[k];
                    buffer[k] += ck * fac;
                }
                v_alpha += T_final * ra * v_a;
                if (a.backgrounds)
                    v_alpha += -T_final * ra * bg_dot;
                if (!clamped) {
                    const float v_sigma = -geo.z * vis * v_alpha;
                    g[2] = 0.5f * v_sigma * dx * dx;
                    g[3] = v_sigma * dx * dy;
                    g[4] = 0.5f * v_sigma * dy * dy;
                    g[0] = v_sigma * (con.x * dx + con.y * dy);
                    g[1] = v_sigma * (con.y * dx + con.z * dy);
                    g[5 + CDIM] = vis * v_alpha;
                    if (ABS) {
                        g[6 + CDIM] = fabsf(g[0]);
                        g[7 + CDIM] = fabsf(g[1]);
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < NACC; ++k)
                g[k] = wave_sum_to_last<TS::ROWS>(g[k]);
            if (last_lane) {
#pragma unroll
                for (int k = 0; k < NACC; ++k)
                    atomicAdd(&s_acc[k * BS + t], g[k]);
                s_hit[t] = 1;
            }
        }
        __syncthreads();
        if (tr < batch_size && s_hit[tr]) {
            const int32_t g = s_gid[tr];
            atomic_add_f32(v_means2d + (int64_t)g * 2 + 0, s_acc[0 * BS + tr]);
            atomic_add_f32(v_means2d + (int64_t)g * 2 + 1, s_acc[1 * BS + tr]);
            atomic_add_f32(v_conics + (int64_t)g * 3 + 0, s_acc[2 * BS + tr]);
            atomic_add_f32(v_conics + (int64_t)g * 3 + 1, s_acc[3 * BS + tr]);
            atomic_add_f32(v_conics + (int64_t)g * 3 + 2, s_acc[4 * BS + tr]);
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                atomic_add_f32(v_colors + (int64_t)g * CDIM + k,
                               s_acc[(5 + k) * BS + tr]);
            atomic_add_f32(v_opacities + g, s_acc[(5 + CDIM) * BS + tr]);
            if (ABS) {
                atomic_add_f32(v_means2d_abs + (int64_t)g * 2 + 0,
                               s_acc[(6 + CDIM) * BS + tr]);
                atomic_add_f32(v_means2d_abs + (int64_t)g * 2 + 1,
                               s_acc[(7 + CDIM) * BS + tr]);
            }
        }
    }
}

int check_raster(const RasterArgs &a, int cdim) {
    GS_REQUIRE(a.I >= 0 && a.n_rows >= 0 && a.n_isects >= 0,
               "rasterize: negative size");
    GS_REQUIRE(a.tile_size == 4 || a.tile_size == 8 || a.tile_size == 16,
               "rasterize: tile_size must be 4, 8 or 16");
    GS_REQUIRE(a.W > 0 && a.H > 0, "rasterize: image size must be positive");
    GS_REQUIRE((int64_t)a.tile_width * a.tile_size >= a.W &&
                   (int64_t)a.tile_height * a.tile_size >= a.H,
               "rasterize: tile grid does not cover the image");
    GS_REQUIRE(a.n_isects < (1ll << 31), "rasterize: more than 2^31 isects");
    GS_REQUIRE(a.tile_offsets != nullptr, "rasterize: NULL tile_offsets");
    if (a.n_isects > 0)
        GS_REQUIRE(a.flatten_ids && a.means2d && a.conics && a.colors &&
                       a.opacities,
                   "rasterize: NULL Gaussian buffer");
    switch (cdim) {
    case 1: case 2: case 3: case 4: case 5: case 8: case 9: case 16: case 17:
    case 32: case 33:
        return GSPLAT_OK;
    default:
        return fail(GSPLAT_ERR_UNSUPPORTED,
                    "rasterize: unsupported channel count " +
                        std::to_string(cdim) +
                        " (supported: 1,2,3,4,5,8,9,16,17,32,33)");
    }
}

#define GS_CDIM_SWITCH(CDIM_VAR, MACRO, ...)                                   \
    switch (CDIM_VAR) {                                                        \
    case 1: MACRO(1, __VA_ARGS__); break;                                      \
    case 2: MACRO(2, __VA_ARGS__); break;                                      \
    case 3: MACRO(3, __VA_ARGS__); break;                                      \
    case 4: MACRO(4, __VA_ARGS__); break;                                      \
    case 5: MACRO(5, __VA_ARGS__); break;                                      \
    case 8: MACRO(8, __VA_ARGS__); break;                                      \
    case 9: MACRO(9, __VA_ARGS__); break;                                      \
    case 16: MACRO(16, __VA_ARGS__); break;                                    \
    case 17: MACRO(17, __VA_ARGS__); break;                                    \
    case 32: MACRO(32, __VA_ARGS__); break;                                    \
    default: MACRO(33, __VA_ARGS__); break;                                    \
    }

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gsplat_rasterize_fwd(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *tile_offsets,
    const int32_t *flatten_ids, float *render_colors, float *render_alphas,
    int32_t *last_ids, float *render_transmittance, gsplat_stream_t stream) {
    clear_error();
    RasterArgs a{I, n_rows, n_isects, means2d, conics, colors, opacities,
                 backgrounds, masks, image_width, image_height, tile_size,
                 tile_width, tile_height, tile_offsets, flatten_ids};
    GS_TRY(check_raster(a, cdim));
    if (I == 0)
        return GSPLAT_OK;
    GS_REQUIRE(render_colors && render_alphas && last_ids,
               "rasterize_fwd: NULL output");
    const int64_t blocks = I * (int64_t)tile_width * tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_fwd: too many tiles");
    hipStream_t st = as_stream(stream);
#define GS_FWD(C, TILE)                                                        \
    rasterize_fwd_kernel<C, TILE><<<(unsigned)blocks, TILE * TILE, 0, st>>>(   \
        a, render_colors, render_alphas, last_ids, render_transmittance)
    if (tile_size == 16) {
        GS_CDIM_SWITCH(cdim, GS_FWD, 16)
    } else if (tile_size == 8) {
        GS_CDIM_SWITCH(cdim, GS_FWD, 8)
    } else {
        GS_CDIM_SWITCH(cdim, GS_FWD, 4)
    }
#undef GS_FWD
    return check_launch("rasterize_fwd_kernel");
}

extern "C" int gsplat_rasterize_bwd(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *opacities, const float *backgrounds, const uint8_t *masks,
    int32_t image_width, int32_t image_height, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *tile_offsets,
    const int32_t *flatten_ids, const float *render_alphas,
    const float *render_transmittance, const int32_t *last_ids,
    const float *v_render_colors,
    const float *v_render_alphas, float *v_means2d_abs, float *v_means2d,
    float *v_conics, float *v_colors, float *v_opacities,
    gsplat_stream_t stream) {
    clear_error();
    RasterArgs a{I, n_rows, n_isects, means2d, conics, colors, opacities,
                 backgrounds, masks, image_width, image_height, tile_size,
                 tile_width, tile_height, tile_offsets, flatten_ids};
    GS_TRY(check_raster(a, cdim));
    if (I == 0 || n_isects == 0)
        return GSPLAT_OK;
    GS_REQUIRE((render_alphas || render_transmittance) && last_ids &&
                   v_render_colors && v_render_alphas,
               "rasterize_bwd: NULL input");
    GS_REQUIRE(v_means2d && v_conics && v_colors && v_opacities,
               "rasterize_bwd: NULL gradient output");
    const int64_t blocks = I * (int64_t)tile_width * tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_bwd: too many tiles");
    hipStream_t st = as_stream(stream);
#define GS_BWD(C, TILE, ABS)                                                   \
    rasterize_bwd_kernel<C, TILE, ABS><<<(unsigned)blocks, TILE * TILE, 0,     \
                                         st>>>(                                \
        a, render_alphas, render_transmittance, last_ids, v_render_colors,     \
        v_render_alphas, v_means2d_abs, v_means2d, v_conics, v_colors,         \
        v_opacities)
    const bool abs = v_means2d_abs != nullptr;
    if (tile_size == 16) {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 16, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 16, false) }
    } else if (tile_size == 8) {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 8, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 8, false) }
    } else {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 4, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 4, false) }
    }
#undef GS_BWD
    return check_launch("rasterize_bwd_kernel");
}
