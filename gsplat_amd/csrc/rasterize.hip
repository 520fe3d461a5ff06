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
// The backward runs 16x16 tiles with 128 threads of two pixels each,
// recovers T back to front in double (one Newton-refined reciprocal per
// Gaussian), sums a lane's two pixels branch-free, reduces each Gaussian's
// gradient over every 16-lane row with four DPP butterflies, adds the eight
// row sums of the tile in LDS (one lane per row) and issues one global atomic
// per value per Gaussian per TILE, 8x fewer than one per 32-lane warp.  Both kernels are compiled per (CDIM, tile size) so every
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
    // Expected depth (render modes ED, RGB+ED): the forward writes colour
    // channel ed_channel divided by max(alpha, 1e-10), the division
    // rendering.py:1259-1267 applies to the render, and (when ed_depth is
    // set) the same value per pixel into ed_depth [I,H,W]; the backward reads
    // that output from ed_depth to take the gradient back through the
    // division.  -1: no channel is divided.
    int32_t ed_channel = -1;
    float *ed_depth = nullptr;
    // Last channel kept apart (a depth channel appended to the colours):
    // with color_last set the rows of colors hold CDIM - 1 channels and
    // channel CDIM - 1 of row g is color_last[g], so no concatenated copy of
    // the two is formed; the backward then writes that channel's gradient
    // to v_color_last [n_rows] and the others to v_colors [n_rows, CDIM - 1].
    const float *color_last = nullptr;
    float *v_color_last = nullptr;
};

// Channel k of row g's colour (see RasterArgs::color_last).
template <int CDIM>
__device__ __forceinline__ float raster_colour(const RasterArgs &a, int64_t g, int k) {
    if (a.color_last != nullptr)
        return k == CDIM - 1 ? a.color_last[g] : a.colors[g * (CDIM - 1) + k];
    return a.colors[g * CDIM + k];
}

// Replay state written by the forward for a backward split into units of
// one part: Q = tile_size^2 / 4 consecutive intersections of a tile.
//   records  per part boundary m >= 1 of a tile, per pixel of the tile: the
//            transmittance before part m and the colour part m composited
//            (float32, summed from zero within the part); record slot
//            (range_start + m * Q - 1) / Q, so slots of different tiles
//            never meet and ceil(n_isects / Q) slots cover every tile;
//   units    (tile, part) pairs of every part up to the tile's last
//            contributor, appended per tile by the forward;
//   count    the number of units (zeroed before the forward);
//   tile_last per tile with units: the isect index of its last contributor.
// A unit's backward starts from its end boundary's record instead of
// replaying every part behind it, so the units of one tile run side by side
// and no workgroup holds a long tile at the end of the launch.
struct ReplayState {
    uint32_t *count;
    int2 *units;
    float *records;
    int32_t *tile_last;  // per tile: its last contributor's isect index, or -1
    // optional: a buffer the forward also zero-fills, each workgroup a
    // slice (the backward's atomic accumulators, so that no fill launch
    // runs between the loss and the backward)
    float *zero;
    int64_t zero_n;
};

// Replay parts per forward batch: a part is BS / kReplayParts consecutive
// intersections of a tile.
constexpr int kReplayParts = 4;

// record slot of a tile's part boundary m >= 1 (parts of q intersections)
__device__ __forceinline__ int64_t replay_record_slot(int32_t range_start, int m,
                                                      int q) {
    return ((int64_t)range_start + (int64_t)m * q - 1) / q;
}

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

// Conservative pixel-centre box of {sigma <= sig_max}: for a positive
// definite conic Q = [[a, b], [b, c]], sigma = 1/2 d^T Q d <= s holds only
// for |dx| <= sqrt(2 s c / det) and |dy| <= sqrt(2 s a / det).  The float
// sigma of gauss_sigma can undershoot the exact one by a few ulp of
// 1/2 (a dx^2 + c dy^2) + |b dx dy|, which is at most 4 ac/det times sigma,
// and det = ac - b^2 itself carries a relative error of order eps ac/det; the
// extents are therefore widened by (1 + 1e-3 + 1e-6 ac/det), more than 4x
// the worst of both, plus 1 px, so rounding can never put a composited pixel
// outside.  Degenerate conics get an unbounded box and Gaussians that never
// composite (sig_max < 0 or NaN) an empty one.  Used only to skip work: a
// pixel outside the box fails the exact test anyway.
__device__ __forceinline__ float4 alpha_support_box(float mx, float my, float a,
                                                    float b, float c,
                                                    float sig_max) {
    if (!(sig_max >= 0.f))
        return make_float4(__builtin_inff(), __builtin_inff(),
                           -__builtin_inff(), -__builtin_inff());
    const float det = a * c - b * b;
    // hardware reciprocal and square root: a few ulp, far inside the widening
    const float idet = __builtin_amdgcn_rcpf(det);
    const float widen = 1.001f + 1e-6f * (a * c * idet);
    const float s2 = 2.f * sig_max * idet;
    const float ex = __builtin_amdgcn_sqrtf(s2 * c) * widen + 1.f;
    const float ey = __builtin_amdgcn_sqrtf(s2 * a) * widen + 1.f;
    if (!(det > 0.f) || !(a > 0.f) || !(c > 0.f) || !(ex < 1e30f) ||
        !(ey < 1e30f))
        return make_float4(-__builtin_inff(), -__builtin_inff(),
                           __builtin_inff(), __builtin_inff());
    return make_float4(mx - ex, my - ey, mx + ex, my + ey);  // x0, y0, x1, y1
}

// Bit w set when the box reaches a pixel centre of wave w's strip of tile
// (tx, ty): the strips are WROWS whole tile rows each, NW of them.
template <int TILE, int NW, int WROWS>
__device__ __forceinline__ uint32_t strip_mask(float4 box, int32_t tx,
                                               int32_t ty) {
    static_assert(NW <= 8, "strip masks are kept in 8 bits");
    const float cx0 = (float)(tx * TILE) + 0.5f;
    const float cx1 = cx0 + (float)(TILE - 1);
    uint32_t m = 0;
    if (box.x <= cx1 && box.z >= cx0) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float cy0 = (float)(ty * TILE + w * WROWS) + 0.5f;
            const float cy1 = cy0 + (float)(WROWS - 1);
            if (box.y <= cy1 && box.w >= cy0)
                m |= 1u << w;
        }
    }
    return m;
}

// strip_mask refined by the ellipse itself.  For d = mean - pixel centre,
// sigma(d) = 1/2 (a u^2 + c v^2) + b u v is convex, so over a strip's
// rectangle of pixel centres it is 0 when the mean lies inside and otherwise
// smallest on an edge, where it is a parabola with its vertex at
// u = -b v / a (rows) or v = -b u / c (columns), clamped to the edge.  A
// strip is dropped when that minimum exceeds sig_max by more than 10^-3
// sig_max + 10^-4 S, with S = 1/2 a U^2 + |b| U V + 1/2 c V^2 (U, V the
// largest |u|, |v| over the strip) bounding every term gauss_sigma adds:
// its float rounding, and this evaluation's, are below 10^-6 S, and an
// inexact vertex only raises the parabola by a second-order amount.  So a
// dropped strip holds no pixel centre with gauss_sigma <= sig_max.  Only
// positive definite conics are refined (the others keep the box's mask).
template <int TILE, int NW, int WROWS>
__device__ __forceinline__ uint32_t strip_mask_exact(uint32_t m, float mx, float my,
                                                     float a, float b, float c,
                                                     float sig_max, int32_t tx,
                                                     int32_t ty) {
    if (m == 0u || !(a > 0.f) || !(c > 0.f) || !(a * c - b * b > 0.f))
        return m;
    const float cx0 = (float)(tx * TILE) + 0.5f;
    const float u0 = mx - (cx0 + (float)(TILE - 1)), u1 = mx - cx0;
    const float ia = __builtin_amdgcn_rcpf(a), ic = __builtin_amdgcn_rcpf(c);
    const float U = fmaxf(fabsf(u0), fabsf(u1));
    const bool u_in = u0 <= 0.f && u1 >= 0.f;
    const float ab = fabsf(b);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        if (!((m >> w) & 1u))
            continue;
        const float cy0 = (float)(ty * TILE + w * WROWS) + 0.5f;
        const float v0 = my - (cy0 + (float)(WROWS - 1)), v1 = my - cy0;
        if (u_in && v0 <= 0.f && v1 >= 0.f)
            continue;
        // rows v = v0 and v = v1
        const float ua = fminf(u1, fmaxf(u0, -b * v0 * ia));
        const float ub = fminf(u1, fmaxf(u0, -b * v1 * ia));
        const float qa = 0.5f * (a * ua * ua + c * v0 * v0) + b * ua * v0;
        const float qb = 0.5f * (a * ub * ub + c * v1 * v1) + b * ub * v1;
        // columns u = u0 and u = u1
        const float va = fminf(v1, fmaxf(v0, -b * u0 * ic));
        const float vb = fminf(v1, fmaxf(v0, -b * u1 * ic));
        const float qc = 0.5f * (a * u0 * u0 + c * va * va) + b * u0 * va;
        const float qd = 0.5f * (a * u1 * u1 + c * vb * vb) + b * u1 * vb;
        const float qmin = fminf(fminf(qa, qb), fminf(qc, qd));
        const float V = fmaxf(fabsf(v0), fabsf(v1));
        const float S = 0.5f * (a * U * U + c * V * V) + ab * U * V;
        if (qmin > sig_max + 1e-3f * sig_max + 1e-4f * S)
            m &= ~(1u << w);
    }
    return m;
}

// Appends, in slot order, the slots s < n whose strip mask holds this wave's
// bit to list; returns the count (uniform over the wave).
template <typename SlotT>
__device__ __forceinline__ int wave_work_list(const uint8_t *wmask, int t0,
                                              int n, int wave, SlotT *list) {
    int n_work = 0;
    for (int c0 = 0; c0 < n; c0 += kWave) {
        const int slot = c0 + (int)lane_id();
        const bool take = slot < n && slot >= t0 && ((wmask[slot] >> wave) & 1u);
        const uint64_t bal = wave_ballot(take);
        if (take)
            list[n_work + __popcll(bal & lanemask_lt())] = (SlotT)slot;
        n_work += __popcll(bal);
    }
    __builtin_amdgcn_wave_barrier();
    return n_work;
}

// wave_work_list that also gives, for every replay part q (slots
// [q Q, (q + 1) Q)), the list position where the part's items end.
template <int Q, int NQ, typename SlotT>
__device__ __forceinline__ int wave_work_list_parts(const uint8_t *wmask, int n,
                                                    int wave, SlotT *list,
                                                    int (&part_end)[NQ]) {
    int n_work = 0;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
        part_end[q] = -1;
    for (int c0 = 0; c0 < n; c0 += kWave) {
        const int slot = c0 + (int)lane_id();
        const bool take = slot < n && ((wmask[slot] >> wave) & 1u);
        const uint64_t bal = wave_ballot(take);
        if (take)
            list[n_work + __popcll(bal & lanemask_lt())] = (SlotT)slot;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int e = (q + 1) * Q - c0;  // part end relative to the chunk
            if (e > 0 && e <= kWave)
                part_end[q] = n_work + __popcll(e == kWave ? bal : bal & ((1ull << e) - 1));
        }
        n_work += __popcll(bal);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < NQ; ++q)
        if (part_end[q] < 0)
            part_end[q] = n_work;
    return n_work;
}

__device__ __forceinline__ void tile_coords(const RasterArgs &a, int64_t gid,
                                            int64_t &image, int32_t &tile,
                                            int32_t &ty, int32_t &tx) {
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;
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
    static_assert(BS % 16 == 0, "tile must hold whole 16-lane rows");
};

// One staged Gaussian of the forward: every field at a constant offset from
// one slot address, and the intersection index in the word after the
// colours (the last_ids candidate, read with the colours).
template <int CDIM> struct FwdSlot {
    float4 geo;                           // (x, y, opacity, sig_max)
    float4 con;                           // (a, b, c, sig_clamp)
    float col[(CDIM + 1 + 3) / 4 * 4];    // CDIM colours, isect index bits, pad
};

// Eight waves per SIMD for the 16x16 kernel of up to five channels: its
// registers fit 64 VGPRs without spills, and the two prefetch register sets
// of the work loop would otherwise cost one wave of occupancy.
template <int CDIM, int TILE> constexpr int fwd_min_waves() {
    return (TILE == 16 && CDIM <= 5) ? 8 : 1;
}

template <int CDIM, int TILE>
__global__ void __launch_bounds__(TILE * TILE, (fwd_min_waves<CDIM, TILE>())) rasterize_fwd_kernel(
    const RasterArgs a, float *__restrict__ render_colors,
    float *__restrict__ render_alphas, int32_t *__restrict__ last_ids,
    float *__restrict__ render_T, const ReplayState rs) {
    constexpr int BS = TileShape<TILE>::BS;
    constexpr int NW = (BS + kWave - 1) / kWave;       // waves per tile
    constexpr int WROWS = (kWave < BS ? kWave : BS) / TILE;  // rows per wave
    __shared__ FwdSlot<CDIM> s_slot[BS];
    __shared__ uint8_t s_wmask[BS];       // waves a Gaussian can reach
    __shared__ uint8_t s_list[NW][BS];    // per-wave work list
    __shared__ int32_t s_last;            // the tile's last contributor

    int64_t image;
    int32_t tile, ty, tx;
    tile_coords(a, blockIdx.x, image, tile, ty, tx);
    const int tr = threadIdx.x;
    const int i = ty * TILE + tr / TILE;
    const int j = tx * TILE + tr % TILE;
    const bool inside = i < a.H && j < a.W;
    const int64_t pix = ((int64_t)image * a.H + i) * a.W + j;
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;

    if (rs.zero != nullptr) {
        // this workgroup's slice of the buffer to clear; the stores drain
        // while the tile composites
        const int64_t per = (rs.zero_n + gridDim.x - 1) / gridDim.x;
        const int64_t z0 = (int64_t)blockIdx.x * per;
        const int64_t z1 = min(z0 + per, rs.zero_n);
        for (int64_t z = z0 + tr; z < z1; z += TILE * TILE)
            rs.zero[z] = 0.f;
    }

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
    // per-lane state as wave masks: votes come straight from the compares and
    // combine in scalar registers, and the selects read the mask directly
    const uint64_t lanes_m = wave_ballot(true);
    uint64_t done_m = wave_ballot(!inside);
    // the colour is summed per batch (seg, from zero) and the batch sums into
    // acc; a batch sum is also what the replay records keep
    float acc[CDIM], seg[CDIM];
#pragma unroll
    for (int k = 0; k < CDIM; ++k) {
        acc[k] = 0.f;
        seg[k] = 0.f;
    }
    if (tr == 0)
        s_last = -1;

    constexpr int Q = BS / kReplayParts;   // intersections per replay part
    for (int b = 0; b < num_batches; ++b) {
        if (__syncthreads_count(__builtin_amdgcn_inverse_ballot_w64(done_m)) >= BS)
            break;
        const int32_t batch_start = range_start + b * BS;
        const int32_t idx = batch_start + tr;
        if (idx < range_end) {
            const int32_t g = a.flatten_ids[idx];
            const float2 xy = reinterpret_cast<const float2 *>(a.means2d)[g];
            const float o = a.opacities[g];
            float sig_max, sig_clamp;
            alpha_thresholds(o, sig_max, sig_clamp);
            const float ca = a.conics[g * 3 + 0], cb = a.conics[g * 3 + 1],
                        cc = a.conics[g * 3 + 2];
            FwdSlot<CDIM> &sl = s_slot[tr];
            sl.geo = make_float4(xy.x, xy.y, o, sig_max);
            sl.con = make_float4(ca, cb, cc, sig_clamp);
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                sl.col[k] = raster_colour<CDIM>(a, g, k);
            sl.col[CDIM] = __int_as_float(idx);
            s_wmask[tr] = (uint8_t)strip_mask_exact<TILE, NW, WROWS>(
                strip_mask<TILE, NW, WROWS>(
                    alpha_support_box(xy.x, xy.y, ca, cb, cc, sig_max), tx, ty),
                xy.x, xy.y, ca, cb, cc, sig_max, tx, ty);
        }
        __syncthreads();
        const int batch_size = min(BS, range_end - batch_start);
        // the staged Gaussians whose alpha support reaches this wave's strip
        // (no other can composite on its pixels), in depth order
        const int wave = tr / kWave;
        // Replay part q of the batch covers slots [q Q, (q + 1) Q): the
        // work list is walked part by part, and at the end of each part its
        // record gets, for the pixels not yet done when it started, T at its
        // start and the colour it composited; the part's colour joins the
        // total.
        int part_end[kReplayParts];
        const int n_work = wave_work_list_parts<Q>(s_wmask, batch_size, wave,
                                                   s_list[wave], part_end);
        const int n_parts = (batch_size + Q - 1) / Q;
        // One work item: staged Gaussian t on this wave's strip.
        auto work_item = [&](const FwdSlot<CDIM> &sl, const float4 geo,
                             const float4 con) __attribute__((always_inline)) {
            const float dx = geo.x - px, dy = geo.y - py;
            const float sigma = gauss_sigma(con.x, con.y, con.z, dx, dy);
            const uint64_t take_m =
                wave_ballot(sigma >= 0.f) & wave_ballot(sigma <= geo.w) & ~done_m;
            if (take_m == 0)
                return;
            // the slot's colours and isect index in 16-byte reads, issued
            // before the exp so that their LDS round trip passes behind it
            constexpr int NQ = (CDIM + 1 + 3) / 4;
            float cq[4 * NQ];
#pragma unroll
            for (int c = 0; c < NQ; ++c) {
                const float4 v = reinterpret_cast<const float4 *>(sl.col)[c];
                cq[4 * c + 0] = v.x;
                cq[4 * c + 1] = v.y;
                cq[4 * c + 2] = v.z;
                cq[4 * c + 3] = v.w;
            }
            // keep the reads here: the scheduler would sink them to their use
            __builtin_amdgcn_sched_barrier(0);
            // every lane runs the arithmetic (the exp clamps any sigma into
            // range); lanes that do not take the Gaussian keep their state
            // through selects
            const float vis = portable_expf_nonpos(-sigma);
            const float alpha = sigma < con.w ? kMaxAlpha : geo.z * vis;
            const float next_T = T * (1.f - alpha);
            const uint64_t stop_m = wave_ballot(next_T <= kTransmittanceThreshold);
            const bool upd = __builtin_amdgcn_inverse_ballot_w64(take_m & ~stop_m);
            // a lane that keeps its state adds c * 0 (= +0, exact): the colour
            // loads stay unconditional instead of each turning into its own
            // exec-masked branch and LDS round trip
            const float w = upd ? alpha * T : 0.f;
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                seg[k] = fmaf(cq[k], w, seg[k]);
            const int32_t slot_idx = __float_as_int(cq[CDIM]);
            cur_idx = upd ? slot_idx : cur_idx;
            T = upd ? next_T : T;
            done_m |= take_m & stop_m;
        };
        int n = 0;
        for (int q = 0; q < n_parts; ++q) {
        const float T_part = T;
        const uint64_t done_part = done_m;
        // wave-uniform loop over the part's items in pairs: the next item's
        // slot and geometry are read one item ahead, into the other of two
        // register sets, so the list and geometry round trips overlap the
        // current item's arithmetic and no register copies carry them over
        const int n_end = part_end[q];
        if (n < n_end) {
            // a slot's address, formed once where its entry is read (24-bit
            // multiply: the list holds u8 slots)
            auto slot = [&](int i) __attribute__((always_inline)) -> const FwdSlot<CDIM> * {
                return reinterpret_cast<const FwdSlot<CDIM> *>(
                    reinterpret_cast<const char *>(s_slot) +
                    __umul24((uint32_t)s_list[wave][i], (uint32_t)sizeof(FwdSlot<CDIM>)));
            };
            const FwdSlot<CDIM> *sl_a = slot(n);
            float4 geo_a = sl_a->geo, con_a = sl_a->con;
            for (; n < n_end; n += 2) {
                if (done_m == lanes_m) {
                    n = n_work;
                    break;
                }
                const FwdSlot<CDIM> *sl_b = slot(min(n + 1, n_end - 1));
                const float4 geo_b = sl_b->geo, con_b = sl_b->con;
                work_item(*sl_a, geo_a, con_a);
                if (n + 1 >= n_end) {
                    n = n_end;
                    break;
                }
                if (done_m == lanes_m) {
                    n = n_work;
                    break;
                }
                sl_a = slot(min(n + 2, n_end - 1));
                geo_a = sl_a->geo;
                con_a = sl_a->con;
                work_item(*sl_b, geo_b, con_b);
            }
        }
        const int m = b * kReplayParts + q;
        if (rs.records != nullptr && m >= 1 &&
            !__builtin_amdgcn_inverse_ballot_w64(done_part)) {
            float *rec = rs.records + replay_record_slot(range_start, m, Q) *
                                          (int64_t)((1 + CDIM) * BS);
            rec[tr] = T_part;
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                rec[(1 + k) * BS + tr] = seg[k];
        }
#pragma unroll
        for (int k = 0; k < CDIM; ++k) {
            acc[k] += seg[k];
            seg[k] = 0.f;
        }
        }
    }
    if (rs.units != nullptr) {
        // one replay unit per part up to the tile's last contributor (a pixel
        // composited something iff its T dropped below 1)
        __syncthreads();
        if (inside && T < 1.f)
            atomicMax(&s_last, cur_idx);
        __syncthreads();
        if (tr == 0 && s_last >= range_start) {
            rs.tile_last[blockIdx.x] = s_last;
            const int nu = (s_last - range_start) / Q + 1;
            const uint32_t base = atomicAdd(rs.count, (uint32_t)nu);
            for (int u = 0; u < nu; ++u)
                rs.units[base + u] = make_int2((int32_t)blockIdx.x, u);
        }
    }
    if (inside) {
        const float alpha_out = 1.f - T;
        render_alphas[pix] = alpha_out;
        // the expected-depth channel over the clamped alpha, in the render's
        // float32 as the reference's division (rendering.py:1259-1267)
        float v_ed = 0.f;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) {
            const float v = a.backgrounds ? acc[k] + T * a.backgrounds[image * CDIM + k]
                                          : acc[k];
            if (k == a.ed_channel)
                v_ed = v;
            else
                render_colors[pix * CDIM + k] = v;
        }
        if (a.ed_channel >= 0) {
            const float ed = v_ed / fmaxf(alpha_out, kMinExpectedDepthAlpha);
            render_colors[pix * CDIM + a.ed_channel] = ed;
            if (a.ed_depth != nullptr)
                a.ed_depth[pix] = ed;
        }
        last_ids[pix] = cur_idx;
        if (render_T != nullptr)
            render_T[pix] = T;
    }
}

// Transposed row reduction of N values.  Four DPP steps, each pairing every
// lane with the lane whose in-row index differs in one bit (row_mirror: bit
// 3, row_half_mirror: bit 2, quad_perm [2,3,0,1]: bit 1, quad_perm [1,0,3,2]:
// bit 0; in that order every partner agrees with the lane on the bits of the
// earlier steps): two registers A, B become one, lanes with the bit clear
// keeping A's sum and lanes with it set B's, so each step halves the
// registers in flight (3 instructions per pair instead of 2 per value).  A
// register left unpaired is summed on both sides.  Afterwards register f of
// lane l (in-row index) holds the 16-lane row sum of value
// RowReduce<N>::value(f, l).
template <int N> struct RowReduce {
    static constexpr int N1 = (N + 1) / 2, N2 = (N1 + 1) / 2;
    static constexpr int N3 = (N2 + 1) / 2, N4 = (N3 + 1) / 2;
    // input register of a step's output register r for a lane whose step bit
    // is `hi`, the step having n inputs
    static constexpr int src(int r, int n, bool hi) {
        return (2 * r + 1 < n && hi) ? 2 * r + 1 : 2 * r;
    }
    static constexpr int value(int f, int l) {
        const int r3 = src(f, N3, (l & 1) != 0);
        const int r2 = src(r3, N2, (l & 2) != 0);
        const int r1 = src(r2, N1, (l & 4) != 0);
        return src(r1, N, (l & 8) != 0);
    }
    // the first (register, lane) holding a value adds it; later copies skip
    static constexpr bool owner(int f, int l) {
        for (int g = 0; g <= f; ++g)
            for (int m = 0; m < 16; ++m) {
                if (g == f && m == l)
                    return true;
                if (value(g, m) == value(f, l))
                    return false;
            }
        return true;
    }
    // value index this lane adds from register f, or -1
    __device__ static int lane_value(int f, int l) {
        int v = -1;
#pragma unroll
        for (int m = 0; m < 16; ++m)
            if (m == l)
                v = owner(f, m) ? value(f, m) : -1;
        return v;
    }
};

template <int CTRL, int N>
__device__ __forceinline__ void row_reduce_step(const float (&in)[N],
                                                float (&out)[(N + 1) / 2],
                                                bool hi) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
        const float send = hi ? in[2 * j] : in[2 * j + 1];
        const float keep = hi ? in[2 * j + 1] : in[2 * j];
        out[j] = keep + dpp_f32<CTRL>(send);
    }
    if constexpr (N % 2 == 1)
        out[N / 2] = in[N - 1] + dpp_f32<CTRL>(in[N - 1]);
}

template <int N>
__device__ __forceinline__ void row_reduce(const float (&v)[N],
                                           float (&out)[RowReduce<N>::N4]) {
    using R = RowReduce<N>;
    const uint32_t l = lane_id() & 15u;
    float a[R::N1], b[R::N2], c[R::N3];
    row_reduce_step<kDppRowMirror>(v, a, (l & 8u) != 0);
    row_reduce_step<kDppRowHalfMirror>(a, b, (l & 4u) != 0);
    row_reduce_step<kDppQuadXor2>(b, c, (l & 2u) != 0);
    row_reduce_step<kDppQuadXor1>(c, out, (l & 1u) != 0);
}

// Backward launch shape: at 16x16 every thread takes PX = 2 pixels (two
// vertically adjacent rows), so each broadcast LDS read of a staged Gaussian
// serves twice the pixels and a lane sums its two pixels before the wave
// reduction (half the reductions and LDS atomics per tile).
template <int TILE> struct BwdShape {
    static constexpr int BS = TILE * TILE;       // pixels of a tile
    static constexpr int PX = TILE == 16 ? 2 : 1;
    static constexpr int THREADS = BS / PX;
    // Gaussians staged per batch: one replay part of the forward (a quarter
    // of its batch), so a replay unit is one batch
    static constexpr int BATCH = BS / kReplayParts;
    static constexpr int ROWS = THREADS >= 64 ? 4 : THREADS / 16;
    static constexpr int LAST = 16 * ROWS - 1;   // lane holding a wave sum
    static_assert(THREADS % 16 == 0, "whole 16-lane rows");
};

// LDS of one backward workgroup (reused tile after tile).
template <int CDIM, int TILE, bool ABS> struct BwdSmem {
    using SH = BwdShape<TILE>;
    static constexpr int NB = SH::BATCH;
    static constexpr int NACC = 2 + 3 + CDIM + 1 + (ABS ? 2 : 0);
    static constexpr int NW = (SH::THREADS + kWave - 1) / kWave;
    float4 geo[NB];
    float4 con[NB];
    float col[NB * CDIM];
    float acc[NW][NACC * NB];  // per-wave sums (each wave writes its own)
    int32_t gid[NB];
    uint8_t wmask[NB];        // waves a Gaussian can reach
    uint8_t list[NW][NB];     // per-wave work list (slots < 256)
    int32_t tile_bin;
    int64_t next_tile;
};

template <int CDIM, int TILE, bool ABS>
__device__ __forceinline__ void rasterize_bwd_tile(
    const RasterArgs &a, int64_t tile_gid, const float *__restrict__ render_alphas,
    const float *__restrict__ render_T, const int32_t *__restrict__ last_ids,
    const float *__restrict__ v_render_colors,
    const float *__restrict__ v_render_alphas,
    float *__restrict__ v_means2d_abs, float *__restrict__ v_means2d,
    float *__restrict__ v_conics, float *__restrict__ v_colors,
    float *__restrict__ v_opacities, BwdSmem<CDIM, TILE, ABS> &sm,
    int32_t unit, const float *__restrict__ records,
    const int32_t *__restrict__ tile_last,
    uint32_t *__restrict__ queue_counter, uint32_t &queue_next) {
    using SH = BwdShape<TILE>;
    constexpr int NB = SH::BATCH;
    constexpr int PX = SH::PX;
    constexpr int NT = SH::THREADS;
    constexpr int SLOTS = NB > NT ? NB / NT : 1;  // staged Gaussians per thread
    // per-Gaussian sums: xy(2), conic(3), colour(CDIM), opacity(1) [, |xy|(2)]
    constexpr int NACC = 2 + 3 + CDIM + 1 + (ABS ? 2 : 0);
    constexpr int NW = (NT + kWave - 1) / kWave;  // waves per tile
    float4 *s_geo = sm.geo;
    float4 *s_con = sm.con;
    float *s_col = sm.col;
    auto &s_acc = sm.acc;
    int32_t *s_gid = sm.gid;
    uint8_t *s_wmask = sm.wmask;
    auto &s_list = sm.list;
    int32_t &s_tile_bin = sm.tile_bin;

    int64_t image;
    int32_t tile, ty, tx;
    tile_coords(a, tile_gid, image, tile, ty, tx);
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;
    if (a.masks != nullptr && !a.masks[image * n_tiles + tile])
        return;
    const int tr = threadIdx.x;
    const int wave = tr / kWave;

    const int32_t *offs = a.tile_offsets + image * n_tiles;
    const int32_t range_start = offs[tile];
    const int32_t range_end = (image == a.I - 1 && tile == n_tiles - 1)
                                  ? (int32_t)a.n_isects
                                  : offs[tile + 1];
    // One unit: its replay range is known from the forward's tile_last, so
    // its rows are loaded now, beside the pixel state below.
    int32_t unit_end = 0;
    constexpr int SLOTS_U = NB > NT ? NB / NT : 1;
    int32_t g_pref[SLOTS_U];
    if (unit >= 0) {
        unit_end = min(range_end, tile_last[tile_gid] + 1);
        const int32_t lo_u = range_start + unit * NB;
        const int32_t end_u = min(lo_u + NB, unit_end) - 1;
#pragma unroll
        for (int q = 0; q < SLOTS_U; ++q) {
            const int slot = tr + q * NT;
            const int32_t idx = end_u - slot;
            g_pref[q] = (slot < NB && idx >= lo_u) ? a.flatten_ids[idx] : 0;
        }
    } else if (tr == 0) {
        s_tile_bin = -1;
    }

    // per-pixel state; pixel p of thread tr is (row PX * (tr / TILE) + p,
    // column tr % TILE) of the tile, so a thread's pixels share one column
    // (one dx per Gaussian)
    const float px = (float)(tx * TILE + tr % TILE) + 0.5f;
    float py[PX], Kv[PX];
    double Bv[PX];
    double T64[PX];
    int32_t bin_final[PX];
    float v_c[PX][CDIM];
    int32_t wave_bin = -1;
#pragma unroll
    for (int p = 0; p < PX; ++p) {
        const int i = ty * TILE + PX * (tr / TILE) + p;
        const int j = tx * TILE + tr % TILE;
        const bool inside = i < a.H && j < a.W;
        const int64_t pix = ((int64_t)image * a.H + (inside ? i : 0)) * a.W +
                            (inside ? j : 0);
        py[p] = (float)i + 0.5f;
        // The transmittance itself when the forward stored it: 1 - (1 - T)
        // loses most of T's significant bits once T nears the 1e-4 cutoff.
        const float T_final = inside ? (render_T != nullptr ? render_T[pix]
                                                            : 1.f - render_alphas[pix])
                                     : 1.f;
        // T before each Gaussian is recovered back to front by undoing the
        // forward's products.  It is carried in double and each step
        // multiplies by 1 / (1 - alpha) refined to ~2^-46 by one Newton step
        // from the fp32 reciprocal, so T keeps only the forward's own rounding
        // instead of one extra float32 rounding per Gaussian behind it.
        T64[p] = (double)T_final;
        bin_final[p] = inside ? last_ids[pix] : -1;
        wave_bin = max(wave_bin, bin_final[p]);
#pragma unroll
        for (int k = 0; k < CDIM; ++k)
            v_c[p][k] = inside ? v_render_colors[pix * CDIM + k] : 0.f;
        float v_a = (inside && v_render_alphas != nullptr) ? v_render_alphas[pix]
                                                           : 0.f;
        if (a.ed_channel >= 0 && inside) {
            // out = v / max(alpha, 1e-10): dL/dv = g / den, and the alpha
            // output gets -g v / den^2 = -(g / den) out where the clamp
            // passes.  This runs for every unit of a tile, so g / den is the
            // hardware reciprocal (1 ulp) times g, not a division sequence.
            const float alpha_out = 1.f - T_final;
            const float den = fmaxf(alpha_out, kMinExpectedDepthAlpha);
            float g = 0.f;
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                g = k == a.ed_channel ? v_c[p][k] : g;
            const float gd = g * __builtin_amdgcn_rcpf(den);
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                v_c[p][k] = k == a.ed_channel ? gd : v_c[p][k];
            if (alpha_out >= kMinExpectedDepthAlpha)
                v_a -= gd * a.ed_depth[pix];
        }
        float bg_dot = 0.f;
        if (a.backgrounds) {
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                bg_dot += a.backgrounds[image * CDIM + k] * v_c[p][k];
        }
        // d loss / d alpha_g = T_g (c_g . v_c) - (B_g - K) / (1 - alpha_g)
        // with B_g = sum over the Gaussians behind g (already replayed) of
        // (c . v_c) alpha T, and K = T_final (v_alpha - bg . v_c): the
        // reference's per-channel colour buffer folded into one running sum.
        Bv[p] = 0.0;
        Kv[p] = T_final * (v_a - bg_dot);
    }
    const int32_t wave_bin_final = wave_max_i32(wave_bin);
    // The forward saturates most pixels long before the end of the tile's
    // range (on dense scenes after a small fraction of it); every Gaussian
    // behind the tile's last contributor has a zero gradient, so the replay
    // starts there instead of at the end of the range.  A unit has it from
    // the forward; a whole tile takes the maximum of its pixels' last_ids.
    int32_t replay_end = unit_end;
    if (unit < 0) {
        __syncthreads();
        atomicMax(&s_tile_bin, wave_bin);
        __syncthreads();
        replay_end = min(range_end, s_tile_bin + 1);
    }
    // Whole tile (unit < 0): batches of NB back from replay_end.  One unit:
    // the forward's replay part `unit` of the tile, [lo, min(lo + Q,
    // replay_end)), starting from the forward's record at its end boundary:
    // T there, and the colour composited behind it as the sum of the later
    // parts' records (in double).
    int num_batches;
    int32_t first_end, lo;
    if (unit < 0) {
        num_batches = max(0, replay_end - range_start + NB - 1) / NB;
        first_end = replay_end - 1;
        lo = range_start;
    } else {
        constexpr int Q = NB;  // a replay part is one batch
        static_assert(NB * kReplayParts == SH::BS, "part size");
        const int nu = max(0, replay_end - range_start + Q - 1) / Q;
        if (unit >= nu)
            return;
        num_batches = 1;
        lo = range_start + unit * Q;
        first_end = min(lo + Q, replay_end) - 1;
        if (unit < nu - 1) {
            // A pixel whose last contributor lies before part m was done
            // before m: the forward kept no record for it there, its T at m is
            // the final one and m composited nothing on it.
            constexpr int RS = (1 + CDIM) * SH::BS;  // floats per record
#pragma unroll
            for (int p = 0; p < PX; ++p) {
                const int lp = (PX * (tr / TILE) + p) * TILE + tr % TILE;
                double bv = 0.0;
                for (int m = unit + 1; m < nu && bin_final[p] >= range_start + m * Q;
                     ++m) {
                    const float *r = records + replay_record_slot(range_start, m, Q) * RS;
                    if (m == unit + 1) {
                        T64[p] = (double)r[lp];
                    }
#pragma unroll
                    for (int k = 0; k < CDIM; ++k)
                        bv += (double)r[(1 + k) * SH::BS + lp] * (double)v_c[p][k];
                }
                Bv[p] = bv;
            }
        }
    }

    // B - K, the running sum the loop carries (B grows, K is fixed)
    double BK[PX];
#pragma unroll
    for (int p = 0; p < PX; ++p)
        BK[p] = Bv[p] - (double)Kv[p];

    // the tile-sum slot this lane adds from every reduced register
    using RR = RowReduce<NACC>;
    int red_slot[RR::N4];
#pragma unroll
    for (int f = 0; f < RR::N4; ++f)
        red_slot[f] = RR::lane_value(f, (int)(lane_id() & 15u));

    // No barrier before restaging: each thread stages exactly the slots it
    // flushed at the end of the previous batch (slot = tr + q * NT in both),
    // and every other read of the staged data ended at the barrier before
    // that flush.
    for (int b = 0; b < num_batches; ++b) {
        __syncthreads();
        const int32_t batch_end = first_end - b * NB;
        const int batch_size = min(NB, batch_end + 1 - lo);
#pragma unroll
        for (int q = 0; q < SLOTS; ++q) {
            const int slot = tr + q * NT;
            if (slot >= NB)
                break;
            const int32_t idx = batch_end - slot;
            if (idx >= lo) {
                const int32_t g = unit >= 0 ? g_pref[q] : a.flatten_ids[idx];
                s_gid[slot] = g;
                const float2 xy = reinterpret_cast<const float2 *>(a.means2d)[g];
                const float o = a.opacities[g];
                float sig_max, sig_clamp;
                alpha_thresholds(o, sig_max, sig_clamp);
                const float ca = a.conics[g * 3 + 0], cb = a.conics[g * 3 + 1],
                            cc = a.conics[g * 3 + 2];
                s_geo[slot] = make_float4(xy.x, xy.y, o, sig_max);
                s_con[slot] = make_float4(ca, cb, cc, sig_clamp);
#pragma unroll
                for (int k = 0; k < CDIM; ++k)
                    s_col[slot * CDIM + k] = raster_colour<CDIM>(a, g, k);
                // which waves' pixel strips the Gaussian's alpha support can
                // reach (wave w holds rows w * WROWS .. of the tile)
                constexpr int WROWS = (kWave < NT ? kWave : NT) * PX / TILE;
                s_wmask[slot] = (uint8_t)strip_mask_exact<TILE, NW, WROWS>(
                    strip_mask<TILE, NW, WROWS>(
                        alpha_support_box(xy.x, xy.y, ca, cb, cc, sig_max), tx, ty),
                    xy.x, xy.y, ca, cb, cc, sig_max, tx, ty);
            } else {
                s_wmask[slot] = 0;
            }
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int k = 0; k < NACC; ++k)
                    s_acc[w][slot * NACC + k] = 0.f;
        }
        __syncthreads();
        // The next queue entry is taken here, by one thread, and read only
        // after this unit: the atomic's latency (long while many workgroups
        // take entries at once) passes behind the work below.
        if (b == 0 && queue_counter != nullptr && tr == 0)
            queue_next = atomicAdd(queue_counter, 1u);

        // this wave's work list, in slot order: Gaussians in front of the
        // wave's last contributor (slots t with isect index batch_end - t >
        // wave_bin_final are behind every pixel of the wave) whose alpha
        // support reaches the wave's pixels
        const int t0 = max(0, batch_end - wave_bin_final);
        const int n_work = wave_work_list(s_wmask, t0, batch_size, wave, s_list[wave]);
        // One work item: Gaussian t of the batch on this wave's pixels.
        auto work_item = [&](const int t, const int col_o, const int acc_o,
                             const float4 geo,
                             const float4 con) __attribute__((always_inline)) {
            const int32_t isect = batch_end - t;
            const float dx = geo.x - px;
            float dy[PX], sigma[PX];
            bool valid[PX];
            uint64_t any_m = 0;
#pragma unroll
            for (int p = 0; p < PX; ++p) {
                dy[p] = geo.y - py[p];
                sigma[p] = gauss_sigma(con.x, con.y, con.z, dx, dy[p]);
                // votes straight from the compares, combined in scalar
                // registers; the selects below read the mask
                const uint64_t valid_m = wave_ballot(isect <= bin_final[p]) &
                                         wave_ballot(sigma[p] >= 0.f) &
                                         wave_ballot(sigma[p] <= geo.w);
                valid[p] = __builtin_amdgcn_inverse_ballot_w64(valid_m);
                any_m |= valid_m;
            }
            if (any_m == 0)
                return;
            // Branch-free over the lane's pixels: an invalid pixel runs the
            // same arithmetic and its contributions are zeroed through
            // selects (fac, w, T64), so nothing is carried through divergent
            // control flow.  Per lane it accumulates the sums over its
            // pixels that the gradient needs:
            //   V = sum vs, Vy = sum vs dy, Vyy = sum vs dy^2 (vs = dL/dsigma),
            //   Vo = sum e^-sigma dL/dalpha, colour sums of alpha T v_c.
            float V = 0.f, Vy = 0.f, Vyy = 0.f, Vo = 0.f, ax = 0.f, ay = 0.f;
            float cg[CDIM];
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                cg[k] = 0.f;
#pragma unroll
            for (int p = 0; p < PX; ++p) {
                // invalid pixels run on their own sigma (the exp clamps it);
                // every contribution of theirs is selected away below
                const float vis = portable_expf_nonpos(-sigma[p]);
                const bool clamped = sigma[p] < con.w;
                const float alpha = clamped ? kMaxAlpha : geo.z * vis;
                // alpha <= 0.99, so 1 - alpha >= 0.01 (the reference's 1e-6
                // floor never binds)
                const float one_minus = fmaxf(kMinOneMinusAlpha, 1.f - alpha);
                const float ra = __builtin_amdgcn_rcpf(one_minus);
                const double d = (double)one_minus;
                double r = (double)ra;
                r = __builtin_fma(r, __builtin_fma(-d, r, 1.0), r);
                T64[p] = valid[p] ? T64[p] * r : T64[p];
                const float fac = valid[p] ? alpha * (float)T64[p] : 0.f;
                // c . v_c: a float32 sum over many channels loses digits the
                // cancelling difference below needs (the 32-channel conic
                // gradient's worst element went from 2.1x to 0.5x the float32
                // restatement's error with this sum in double)
                float scv;
                if constexpr (CDIM > 4) {
                    double sd = 0.0;
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) {
                        sd = __builtin_fma((double)s_col[col_o + k], (double)v_c[p][k], sd);
                        cg[k] += fac * v_c[p][k];
                    }
                    scv = (float)sd;
                } else {
                    scv = 0.f;
#pragma unroll
                    for (int k = 0; k < CDIM; ++k) {
                        scv += s_col[col_o + k] * v_c[p][k];
                        cg[k] += fac * v_c[p][k];
                    }
                }
                // The two terms cancel for a Gaussian in front of much of
                // the pixel's colour (BK holds the colour behind it less K),
                // so the difference and the running sum are taken in double:
                // in float32 they put the conic gradient of such Gaussians
                // up to 2.8x further from the exact value than a float32
                // autograd evaluation of the same formula.
                const float v_alpha = (float)(T64[p] * (double)scv - BK[p] * r);
                BK[p] += (double)fac * (double)scv;
                // a clamped alpha does not depend on the Gaussian's geometry
                // or opacity
                const float w = (valid[p] && !clamped) ? vis * v_alpha : 0.f;
                const float vs = -geo.z * w;
                const float vy = vs * dy[p];
                Vo += w;
                V += vs;
                Vy += vy;
                Vyy += vy * dy[p];
                if constexpr (ABS) {
                    ax += fabsf(vs * (con.x * dx + con.y * dy[p]));
                    ay += fabsf(vs * (con.y * dx + con.z * dy[p]));
                }
            }
            // the lane's gradient terms: d/dmean = sum vs (Q d), d/dconic =
            // sum vs (dx^2 / 2, dx dy, dy^2 / 2), with dx shared by the
            // lane's pixels
            float gv[NACC];
            gv[0] = con.x * (dx * V) + con.y * Vy;
            gv[1] = con.y * (dx * V) + con.z * Vy;
            gv[2] = 0.5f * (dx * dx) * V;
            gv[3] = dx * Vy;
            gv[4] = 0.5f * Vyy;
#pragma unroll
            for (int k = 0; k < CDIM; ++k)
                gv[5 + k] = cg[k];
            gv[5 + CDIM] = Vo;
            if constexpr (ABS) {
                gv[6 + CDIM] = ax;
                gv[7 + CDIM] = ay;
            }
            // sums over each 16-lane row, one value per lane; then the four
            // rows summed by two cross-row swaps (lanes l and l ^ 32, then
            // rows 2r and 2r + 1), and the wave's sums stored by the first
            // row into the wave's own slots: no LDS atomics
            float red[RR::N4];
            row_reduce<NACC>(gv, red);
#pragma unroll
            for (int f = 0; f < RR::N4; ++f) {
                if constexpr (SH::ROWS == 4) {
                    const uint32_t u = __float_as_uint(red[f]);
                    const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                    const float s2 = __uint_as_float(h[0]) + __uint_as_float(h[1]);
                    const uint32_t u2 = __float_as_uint(s2);
                    const auto r = __builtin_amdgcn_permlane16_swap(u2, u2, false, false);
                    red[f] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                }
                if (lane_id() < 16u && red_slot[f] >= 0)
                    s_acc[wave][acc_o + red_slot[f]] = red[f];
            }
        };
        // Software pipeline over pairs of items: the next item's slot and
        // geometry are read one item ahead, into the other of two register
        // sets, so the two dependent LDS round trips overlap the current
        // item's arithmetic and no register copies carry them over.
        // a slot's colour and sum offsets are formed where its entry is read
        // (24-bit multiplies: the list holds u8 slots)
        int t_a = n_work > 0 ? (int)s_list[wave][0] : 0;
        int col_a = (int)__umul24((uint32_t)t_a, CDIM), acc_a = (int)__umul24((uint32_t)t_a, NACC);
        float4 geo_a = s_geo[t_a], con_a = s_con[t_a];
        for (int n = 0; n < n_work; n += 2) {
            const int t_b = s_list[wave][min(n + 1, n_work - 1)];
            const int col_b = (int)__umul24((uint32_t)t_b, CDIM);
            const int acc_b = (int)__umul24((uint32_t)t_b, NACC);
            const float4 geo_b = s_geo[t_b], con_b = s_con[t_b];
            work_item(t_a, col_a, acc_a, geo_a, con_a);
            if (n + 1 >= n_work)
                break;
            t_a = s_list[wave][min(n + 2, n_work - 1)];
            col_a = (int)__umul24((uint32_t)t_a, CDIM);
            acc_a = (int)__umul24((uint32_t)t_a, NACC);
            geo_a = s_geo[t_a];
            con_a = s_con[t_a];
            work_item(t_b, col_b, acc_b, geo_b, con_b);
        }
        __syncthreads();
        // Flush: the batch's (slot, sum) pairs spread over all threads, one
        // global atomic each, the two waves' sums added first.  A sum that
        // is zero (a Gaussian no pixel took, or a term that vanished) adds
        // nothing and is skipped.
        for (int e = tr; e < batch_size * NACC; e += NT) {
            const int slot = e / NACC;
            const int k = e - slot * NACC;
            float v = s_acc[0][e];
#pragma unroll
            for (int w = 1; w < NW; ++w)
                v += s_acc[w][e];
            if (v == 0.f)
                continue;
            const int64_t g = s_gid[slot];
            float *dst;
            if (k < 2)
                dst = v_means2d + g * 2 + k;
            else if (k < 5)
                dst = v_conics + g * 3 + (k - 2);
            else if (k < 5 + CDIM)
                dst = a.v_color_last == nullptr ? v_colors + g * CDIM + (k - 5)
                      : k == 4 + CDIM           ? a.v_color_last + g
                                                : v_colors + g * (CDIM - 1) + (k - 5);
            else if (k == 5 + CDIM)
                dst = v_opacities + g;
            else
                dst = v_means2d_abs + g * 2 + (k - 6 - CDIM);
            atomic_add_f32(dst, v);
        }
    }
}


// One tile per workgroup, or (tile_counter != NULL, a zeroed counter) a
// grid sized to the resident workgroups in which every workgroup takes tile
// after tile from the counter until none is left: no partial last round of
// workgroups, and a heavy tile never waits behind a full round.
template <int CDIM, int TILE, bool ABS>
__global__ void __launch_bounds__(BwdShape<TILE>::THREADS) rasterize_bwd_kernel(
    const RasterArgs a, const float *__restrict__ render_alphas,
    const float *__restrict__ render_T, const int32_t *__restrict__ last_ids,
    const float *__restrict__ v_render_colors,
    const float *__restrict__ v_render_alphas,
    float *__restrict__ v_means2d_abs, float *__restrict__ v_means2d,
    float *__restrict__ v_conics, float *__restrict__ v_colors,
    float *__restrict__ v_opacities, uint32_t *__restrict__ tile_counter,
    int64_t n_tiles_total, const ReplayState rs) {
    __shared__ BwdSmem<CDIM, TILE, ABS> sm;
    const bool queue = tile_counter != nullptr;
    // with replay state the queue hands out the forward's units, otherwise
    // whole tiles
    const int64_t n_work = rs.units != nullptr ? (int64_t)*rs.count : n_tiles_total;
    // entry k = blockIdx.x first, then gridDim.x + the counter's values
    int64_t k = blockIdx.x;
    while (k < n_work) {
        int64_t gid = k;
        int32_t unit = -1;
        if (rs.units != nullptr) {
            const int2 e = rs.units[k];
            gid = e.x;
            unit = e.y;
        }
        uint32_t next = 0xffffffffu;  // thread 0's next entry, once taken
        rasterize_bwd_tile<CDIM, TILE, ABS>(
            a, gid, render_alphas, render_T, last_ids, v_render_colors,
            v_render_alphas, v_means2d_abs, v_means2d, v_conics, v_colors,
            v_opacities, sm, unit, rs.records, rs.tile_last,
            queue ? tile_counter : nullptr, next);
        if (!queue)
            break;
        __syncthreads();  // the unit is finished with the LDS
        if (threadIdx.x == 0) {
            if (next == 0xffffffffu)  // the unit ended before taking one
                next = atomicAdd(tile_counter, 1u);
            sm.next_tile = (int64_t)gridDim.x + next;
        }
        __syncthreads();
        k = sm.next_tile;
    }
}

// Rasterize to indices (rasterize_to_indices_3dgs, RasterizeToIndices3DGS.cu
// :36-196): the (Gaussian, pixel) pairs each pixel composites over the isect
// batches [range_start, range_end) of its tile (batches of tile_size^2),
// starting from the pixel's given transmittance.  The compositing decisions
// are the forward kernel's (exact sigma order, thresholds on sigma,
// portable_expf), so the pairs agree with rasterize_fwd bit for bit.  COUNT
// writes the per-pixel counts; otherwise the pairs go to the per-pixel
// starts from the scan of those counts.  One workgroup per tile.  The write
// pass takes each staged Gaussian's id modulo N once, at staging, and stores
// only the Gaussian ids while compositing; each pixel's constant pixel id
// fills its range afterwards, one pixel at a time per wave, in 64-lane
// coalesced stores.
template <int TILE, bool COUNT>
__global__ void __launch_bounds__(TILE * TILE) rasterize_indices_kernel(
    const RasterArgs a, int64_t N, int64_t range_start, int64_t range_end,
    const float *__restrict__ trans_in, const uint32_t *__restrict__ starts,
    uint32_t *__restrict__ counts, int64_t *__restrict__ gaussian_ids,
    int64_t *__restrict__ pixel_ids) {
    constexpr int BS = TileShape<TILE>::BS;
    __shared__ float4 s_geo[BS];   // (x, y, opacity, sig_max)
    __shared__ float4 s_con[BS];   // (a, b, c, sig_clamp)
    __shared__ int32_t s_id[BS];

    int64_t image;
    int32_t tile, ty, tx;
    tile_coords(a, blockIdx.x, image, tile, ty, tx);
    const int tr = threadIdx.x;
    const int i = ty * TILE + tr / TILE;
    const int j = tx * TILE + tr % TILE;
    const bool inside = i < a.H && j < a.W;
    const int64_t pix = ((int64_t)image * a.H + i) * a.W + j;
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const int64_t n_tiles = (int64_t)a.tile_width * a.tile_height;

    const int32_t *offs = a.tile_offsets + image * n_tiles;
    const int32_t range_lo = offs[tile];
    const int32_t range_hi = (image == a.I - 1 && tile == n_tiles - 1)
                                 ? (int32_t)a.n_isects
                                 : offs[tile + 1];
    const int64_t num_batches = (range_hi - range_lo + BS - 1) / BS;
    const int64_t b_end = range_end < num_batches ? range_end : num_batches;

    float T = inside ? trans_in[pix] : 1.f;
    bool done = !inside;
    uint32_t cnt = 0;
    const uint32_t base = (!COUNT && inside) ? starts[pix] : 0u;
    for (int64_t b = range_start; b < b_end; ++b) {
        if (__syncthreads_count(done) >= BS)
            break;
        const int32_t batch_start = range_lo + (int32_t)b * BS;
        const int32_t idx = batch_start + tr;
        if (idx < range_hi) {
            const int32_t g = a.flatten_ids[idx];
            if constexpr (!COUNT)
                s_id[tr] = N >= (1ll << 31) ? g : (int32_t)((uint32_t)g % (uint32_t)N);
            const float2 xy = reinterpret_cast<const float2 *>(a.means2d)[g];
            const float o = a.opacities[g];
            float sig_max, sig_clamp;
            alpha_thresholds(o, sig_max, sig_clamp);
            s_geo[tr] = make_float4(xy.x, xy.y, o, sig_max);
            s_con[tr] = make_float4(a.conics[g * 3 + 0], a.conics[g * 3 + 1],
                                    a.conics[g * 3 + 2], sig_clamp);
        }
        __syncthreads();
        const int batch_size = min(BS, range_hi - batch_start);
        for (int t = 0; t < batch_size; ++t) {
            if (!wave_ballot(!done))
                break;
            const float4 geo = s_geo[t];
            const float4 con = s_con[t];
            const float sigma = gauss_sigma(con.x, con.y, con.z, geo.x - px, geo.y - py);
            const bool take = !done && sigma >= 0.f && sigma <= geo.w;
            if (!wave_ballot(take))
                continue;
            const float vis = portable_expf_nonpos(-sigma);
            const float alpha = sigma < con.w ? kMaxAlpha : geo.z * vis;
            const float next_T = T * (1.f - alpha);
            const bool stop = next_T <= kTransmittanceThreshold;
            const bool emit = take && !stop;
            if (!COUNT && emit)
                gaussian_ids[base + cnt] = s_id[t];
            cnt += emit ? 1u : 0u;
            T = emit ? next_T : T;
            done = done || (take && stop);
        }
    }
    if constexpr (COUNT) {
        if (inside)
            counts[pix] = cnt;
    } else {
        // every thread leaves the batch loop together (its exits are
        // workgroup-uniform), so the barrier below is reached by all
        __shared__ uint32_t s_pbase[BS];
        __shared__ uint32_t s_pcnt[BS];
        s_pbase[tr] = base;
        s_pcnt[tr] = cnt;  // 0 outside the image
        __syncthreads();
        // a wave's lanes: 64, or all BS threads of a smaller tile (4x4 tiles
        // run 16 lanes, and the stride is theirs)
        constexpr uint32_t NL = BS < kWave ? BS : kWave;
        const int w0 = tr - (int)lane_id();  // the wave's first thread
        for (int q = 0; q < (int)NL; ++q) {
            const int tq = w0 + q;
            const uint32_t sq = s_pbase[tq], cq = s_pcnt[tq];
            const int64_t pq =
                ((int64_t)image * a.H + ty * TILE + tq / TILE) * a.W + tx * TILE + tq % TILE;
            for (uint32_t k = lane_id(); k < cq; k += NL)
                pixel_ids[sq + k] = pq;
        }
    }
}

__global__ void indices_total_kernel(const uint32_t *__restrict__ starts,
                                     const uint32_t *__restrict__ counts, int64_t n,
                                     int64_t *__restrict__ total) {
    total[0] = (int64_t)starts[n - 1] + (int64_t)counts[n - 1];
}

// Workgroups of `kernel` (block threads, static LDS) that fit on the device
// at once, capped at `work`.
int resident_grid(const void *kernel, int block, int64_t work, int64_t *grid) {
    int dev = 0, per_cu = 0, cus = 0;
    GS_REQUIRE(hipGetDevice(&dev) == hipSuccess, "hipGetDevice failed");
    GS_REQUIRE(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel,
                                                           block, 0) == hipSuccess,
               "hipOccupancyMaxActiveBlocksPerMultiprocessor failed");
    GS_REQUIRE(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                     dev) == hipSuccess,
               "hipDeviceGetAttribute failed");
    const int64_t g = (int64_t)(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    *grid = g < work ? g : work;
    return GSPLAT_OK;
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
        GS_REQUIRE(a.flatten_ids && a.means2d && a.conics &&
                       (a.colors || (a.color_last && cdim == 1)) && a.opacities,
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

namespace {

__global__ void replay_clear_kernel(uint32_t *count) { *count = 0u; }

__global__ void zero_f32_kernel(float *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = 0.f;
}

// Replay workspace: [count, padded to 256 B][units][records], each part
// 256-byte aligned.
struct ReplayLayout {
    int64_t n_records, max_units, n_tiles;
    size_t units_off, tile_last_off, records_off, bytes;
};

ReplayLayout replay_layout(int64_t I, int32_t tile_width, int32_t tile_height,
                           int32_t tile_size, int64_t n_isects, int32_t cdim) {
    const int64_t bs = (int64_t)tile_size * tile_size;
    const int64_t q = bs / kReplayParts;
    ReplayLayout l;
    l.n_records = q > 0 ? (n_isects + q - 1) / q : 0;
    l.n_tiles = I * (int64_t)tile_width * tile_height;
    l.max_units = l.n_records + l.n_tiles;
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    l.units_off = 256;
    l.tile_last_off = l.units_off + up((size_t)l.max_units * sizeof(int2));
    l.records_off = l.tile_last_off + up((size_t)l.n_tiles * sizeof(int32_t));
    l.bytes = l.records_off +
              (size_t)l.n_records * (size_t)bs * (size_t)(1 + cdim) * sizeof(float);
    return l;
}

int replay_state(void *ws, size_t ws_bytes, const RasterArgs &a, int cdim,
                 ReplayState *rs) {
    const ReplayLayout l = replay_layout(a.I, a.tile_width, a.tile_height,
                                         a.tile_size, a.n_isects, cdim);
    GS_REQUIRE(ws != nullptr, "rasterize replay: NULL replay workspace");
    GS_REQUIRE(ws_bytes >= l.bytes,
               "rasterize replay: workspace of " + std::to_string(ws_bytes) +
                   " bytes, " + std::to_string(l.bytes) + " needed");
    GS_REQUIRE(((uintptr_t)ws & 255u) == 0,
               "rasterize replay: workspace must be 256-byte aligned");
    char *base = static_cast<char *>(ws);
    rs->count = reinterpret_cast<uint32_t *>(base);
    rs->units = reinterpret_cast<int2 *>(base + l.units_off);
    rs->records = reinterpret_cast<float *>(base + l.records_off);
    rs->tile_last = reinterpret_cast<int32_t *>(base + l.tile_last_off);
    return GSPLAT_OK;
}

int rasterize_fwd_impl(const RasterArgs &a, int32_t cdim, float *render_colors,
                       float *render_alphas, int32_t *last_ids,
                       float *render_transmittance, const ReplayState &rs,
                       gsplat_stream_t stream) {
    if (a.I == 0 || a.tile_width == 0 || a.tile_height == 0) {
        // no tile workgroups: the buffer to clear gets a launch of its own
        if (rs.zero != nullptr && rs.zero_n > 0) {
            zero_f32_kernel<<<(unsigned)ceil_div(rs.zero_n, 256), 256, 0,
                              as_stream(stream)>>>(rs.zero, rs.zero_n);
            return check_launch("zero_f32_kernel");
        }
        return GSPLAT_OK;
    }
    GS_REQUIRE(render_colors && render_alphas && last_ids,
               "rasterize_fwd: NULL output");
    const int64_t blocks = a.I * (int64_t)a.tile_width * a.tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_fwd: too many tiles");
    hipStream_t st = as_stream(stream);
    if (rs.count != nullptr) {
        replay_clear_kernel<<<1, 1, 0, st>>>(rs.count);
        GS_TRY(check_launch("replay_clear_kernel"));
    }
#define GS_FWD(C, TILE)                                                        \
    rasterize_fwd_kernel<C, TILE><<<(unsigned)blocks, TILE * TILE, 0, st>>>(   \
        a, render_colors, render_alphas, last_ids, render_transmittance, rs)
    if (a.tile_size == 16) {
        GS_CDIM_SWITCH(cdim, GS_FWD, 16)
    } else if (a.tile_size == 8) {
        GS_CDIM_SWITCH(cdim, GS_FWD, 8)
    } else {
        GS_CDIM_SWITCH(cdim, GS_FWD, 4)
    }
#undef GS_FWD
    return check_launch("rasterize_fwd_kernel");
}

int rasterize_bwd_impl(const RasterArgs &a, int32_t cdim,
                       const float *render_alphas,
                       const float *render_transmittance, const int32_t *last_ids,
                       const float *v_render_colors, const float *v_render_alphas,
                       float *v_means2d_abs, float *v_means2d, float *v_conics,
                       float *v_colors, float *v_opacities, uint32_t *tile_counter,
                       const ReplayState &rs, gsplat_stream_t stream) {
    if (a.I == 0 || a.n_isects == 0)
        return GSPLAT_OK;
    GS_REQUIRE((render_alphas || render_transmittance) && last_ids &&
                   v_render_colors,
               "rasterize_bwd: NULL input");
    GS_REQUIRE(v_means2d && v_conics && v_opacities &&
                   (v_colors || (a.v_color_last && cdim == 1)),
               "rasterize_bwd: NULL gradient output");
    const int64_t blocks = a.I * (int64_t)a.tile_width * a.tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_bwd: too many tiles");
    hipStream_t st = as_stream(stream);
    // the replayed units are known on the device only: a resident grid takes
    // them from the counter, sized for the most units there can be
    const int64_t work = rs.units != nullptr
                             ? replay_layout(a.I, a.tile_width, a.tile_height,
                                             a.tile_size, a.n_isects, cdim).max_units
                             : blocks;
#define GS_BWD(C, TILE, ABS)                                                   \
    {                                                                          \
        auto kern = rasterize_bwd_kernel<C, TILE, ABS>;                        \
        int64_t grid = work;                                                   \
        if (tile_counter != nullptr)                                           \
            GS_TRY(resident_grid((const void *)kern, BwdShape<TILE>::THREADS,  \
                                 work, &grid));                                \
        kern<<<(unsigned)grid, BwdShape<TILE>::THREADS, 0, st>>>(              \
            a, render_alphas, render_transmittance, last_ids, v_render_colors, \
            v_render_alphas, v_means2d_abs, v_means2d, v_conics, v_colors,     \
            v_opacities, tile_counter, blocks, rs);                            \
    }
    const bool abs = v_means2d_abs != nullptr;
    if (a.tile_size == 16) {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 16, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 16, false) }
    } else if (a.tile_size == 8) {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 8, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 8, false) }
    } else {
        if (abs) { GS_CDIM_SWITCH(cdim, GS_BWD, 4, true) }
        else { GS_CDIM_SWITCH(cdim, GS_BWD, 4, false) }
    }
#undef GS_BWD
    return check_launch("rasterize_bwd_kernel");
}

}  // namespace

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
    return rasterize_fwd_impl(a, cdim, render_colors, render_alphas, last_ids,
                              render_transmittance, ReplayState{}, stream);
}

extern "C" size_t gsplat_rasterize_replay_size(int64_t I, int32_t tile_width,
                                               int32_t tile_height,
                                               int32_t tile_size,
                                               int64_t n_isects, int32_t cdim) {
    if (I < 0 || tile_width < 0 || tile_height < 0 || tile_size <= 0 ||
        n_isects < 0 || cdim <= 0)
        return 0;
    return replay_layout(I, tile_width, tile_height, tile_size, n_isects, cdim).bytes;
}

extern "C" int gsplat_rasterize_fwd_replay(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *color_last, const float *opacities, const float *backgrounds,
    const uint8_t *masks, int32_t image_width, int32_t image_height,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    float *render_colors, float *render_alphas, int32_t *last_ids,
    float *render_transmittance, void *replay, size_t replay_bytes,
    int32_t expected_depth_channel, float *expected_depth, float *zero_fill,
    int64_t zero_fill_count, gsplat_stream_t stream) {
    clear_error();
    RasterArgs a{I, n_rows, n_isects, means2d, conics, colors, opacities,
                 backgrounds, masks, image_width, image_height, tile_size,
                 tile_width, tile_height, tile_offsets, flatten_ids};
    a.color_last = color_last;
    GS_TRY(check_raster(a, cdim));
    GS_REQUIRE(render_transmittance != nullptr,
               "rasterize_fwd_replay: NULL render_transmittance");
    GS_REQUIRE(expected_depth_channel >= -1 && expected_depth_channel < cdim,
               "rasterize_fwd_replay: expected_depth_channel out of range");
    a.ed_channel = expected_depth_channel;
    a.ed_depth = expected_depth_channel >= 0 ? expected_depth : nullptr;
    GS_REQUIRE(zero_fill_count >= 0 && (zero_fill_count == 0 || zero_fill != nullptr),
               "rasterize_fwd_replay: NULL zero_fill with a nonzero count");
    ReplayState rs{};
    GS_TRY(replay_state(replay, replay_bytes, a, cdim, &rs));
    rs.zero = zero_fill_count > 0 ? zero_fill : nullptr;
    rs.zero_n = zero_fill_count;
    return rasterize_fwd_impl(a, cdim, render_colors, render_alphas, last_ids,
                              render_transmittance, rs, stream);
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
    uint32_t *tile_counter, gsplat_stream_t stream) {
    clear_error();
    RasterArgs a{I, n_rows, n_isects, means2d, conics, colors, opacities,
                 backgrounds, masks, image_width, image_height, tile_size,
                 tile_width, tile_height, tile_offsets, flatten_ids};
    GS_TRY(check_raster(a, cdim));
    return rasterize_bwd_impl(a, cdim, render_alphas, render_transmittance,
                              last_ids, v_render_colors, v_render_alphas,
                              v_means2d_abs, v_means2d, v_conics, v_colors,
                              v_opacities, tile_counter, ReplayState{}, stream);
}

extern "C" int gsplat_rasterize_bwd_replay(
    int64_t I, int64_t n_rows, int64_t n_isects, int32_t cdim,
    const float *means2d, const float *conics, const float *colors,
    const float *color_last, const float *opacities, const float *backgrounds,
    const uint8_t *masks, int32_t image_width, int32_t image_height,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    const float *render_transmittance, const int32_t *last_ids,
    const float *v_render_colors, const float *v_render_alphas,
    float *v_means2d_abs, float *v_means2d, float *v_conics, float *v_colors,
    float *v_color_last, float *v_opacities, uint32_t *tile_counter,
    const void *replay, size_t replay_bytes, const float *expected_depth,
    int32_t expected_depth_channel, gsplat_stream_t stream) {
    clear_error();
    RasterArgs a{I, n_rows, n_isects, means2d, conics, colors, opacities,
                 backgrounds, masks, image_width, image_height, tile_size,
                 tile_width, tile_height, tile_offsets, flatten_ids};
    a.color_last = color_last;
    a.v_color_last = v_color_last;
    GS_REQUIRE((color_last == nullptr) == (v_color_last == nullptr),
               "rasterize_bwd_replay: color_last and v_color_last go together");
    GS_TRY(check_raster(a, cdim));
    GS_REQUIRE(render_transmittance != nullptr,
               "rasterize_bwd_replay: NULL render_transmittance");
    GS_REQUIRE(expected_depth_channel >= -1 && expected_depth_channel < cdim,
               "rasterize_bwd_replay: expected_depth_channel out of range");
    GS_REQUIRE(expected_depth_channel < 0 || expected_depth != nullptr,
               "rasterize_bwd_replay: the expected-depth channel needs the "
               "forward's expected_depth");
    a.ed_channel = expected_depth_channel;
    a.ed_depth = const_cast<float *>(expected_depth);
    GS_REQUIRE(tile_counter != nullptr,
               "rasterize_bwd_replay: NULL tile_counter (the units are taken "
               "from it)");
    ReplayState rs{};
    GS_TRY(replay_state(const_cast<void *>(replay), replay_bytes, a, cdim, &rs));
    return rasterize_bwd_impl(a, cdim, nullptr, render_transmittance, last_ids,
                              v_render_colors, v_render_alphas, v_means2d_abs,
                              v_means2d, v_conics, v_colors, v_opacities,
                              tile_counter, rs, stream);
}

// Shared argument handling of the two indices entry points.  The op has no
// colours; the shared raster checks get means2d as a stand-in pointer (never
// read).
static int indices_args(int64_t I, int64_t N, int64_t n_isects,
                        const float *means2d, const float *conics,
                        const float *opacities, int32_t image_width,
                        int32_t image_height, int32_t tile_size, int32_t tile_width,
                        int32_t tile_height, const int32_t *tile_offsets,
                        const int32_t *flatten_ids, const float *transmittances,
                        int64_t range_start, RasterArgs *a) {
    *a = RasterArgs{I, I * N, n_isects, means2d, conics, means2d, opacities,
                    nullptr, nullptr, image_width, image_height, tile_size,
                    tile_width, tile_height, tile_offsets, flatten_ids};
    GS_TRY(check_raster(*a, 1));
    GS_REQUIRE(N > 0, "rasterize_to_indices: N must be positive");
    GS_REQUIRE(range_start >= 0, "rasterize_to_indices: negative range_start");
    GS_REQUIRE(transmittances != nullptr, "rasterize_to_indices: NULL transmittances");
    GS_REQUIRE(I * (int64_t)image_width * image_height < (1ll << 32),
               "rasterize_to_indices: too many pixels");
    return GSPLAT_OK;
}

extern "C" size_t gsplat_rasterize_to_indices_workspace_size(int64_t n_pixels) {
    return lookback_bytes(ceil_div(n_pixels > 0 ? n_pixels : 1, 2048));
}

extern "C" int gsplat_rasterize_to_indices_count(
    int64_t range_start, int64_t range_end, int64_t I, int64_t N, int64_t n_isects,
    const float *transmittances, const float *means2d, const float *conics,
    const float *opacities, int32_t image_width, int32_t image_height,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids, int32_t *chunk_cnts,
    int32_t *chunk_starts, int64_t *n_elems, void *workspace,
    size_t workspace_bytes, gsplat_stream_t stream) {
    clear_error();
    RasterArgs a;
    GS_TRY(indices_args(I, N, n_isects, means2d, conics, opacities, image_width,
                        image_height, tile_size, tile_width, tile_height,
                        tile_offsets, flatten_ids, transmittances, range_start, &a));
    if (I == 0)
        return GSPLAT_OK;
    GS_REQUIRE(chunk_cnts && chunk_starts && n_elems,
               "rasterize_to_indices_count: NULL output");
    const int64_t n_pix = I * (int64_t)image_width * image_height;
    GS_REQUIRE(workspace != nullptr &&
                   workspace_bytes >= gsplat_rasterize_to_indices_workspace_size(n_pix),
               "rasterize_to_indices_count: workspace too small");
    const int64_t blocks = I * (int64_t)tile_width * tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_to_indices: too many tiles");
    hipStream_t st = as_stream(stream);
    uint32_t *cnt = reinterpret_cast<uint32_t *>(chunk_cnts);
    uint32_t *start = reinterpret_cast<uint32_t *>(chunk_starts);
#define GS_IDX(TILE)                                                           \
    rasterize_indices_kernel<TILE, true><<<(unsigned)blocks, TILE * TILE, 0, st>>>( \
        a, N, range_start, range_end, transmittances, nullptr, cnt, nullptr,   \
        nullptr)
    if (tile_size == 16) GS_IDX(16);
    else if (tile_size == 8) GS_IDX(8);
    else GS_IDX(4);
#undef GS_IDX
    GS_TRY(check_launch("rasterize_indices_kernel"));
    GS_TRY(scan_u32_exclusive(cnt, start, n_pix, workspace, st));
    indices_total_kernel<<<1, 1, 0, st>>>(start, cnt, n_pix, n_elems);
    return check_launch("indices_total_kernel");
}

extern "C" int gsplat_rasterize_to_indices_write(
    int64_t range_start, int64_t range_end, int64_t I, int64_t N, int64_t n_isects,
    const float *transmittances, const float *means2d, const float *conics,
    const float *opacities, int32_t image_width, int32_t image_height,
    int32_t tile_size, int32_t tile_width, int32_t tile_height,
    const int32_t *tile_offsets, const int32_t *flatten_ids,
    const int32_t *chunk_starts, int64_t *gaussian_ids, int64_t *pixel_ids,
    gsplat_stream_t stream) {
    clear_error();
    RasterArgs a;
    GS_TRY(indices_args(I, N, n_isects, means2d, conics, opacities, image_width,
                        image_height, tile_size, tile_width, tile_height,
                        tile_offsets, flatten_ids, transmittances, range_start, &a));
    if (I == 0)
        return GSPLAT_OK;
    GS_REQUIRE(chunk_starts && gaussian_ids && pixel_ids,
               "rasterize_to_indices_write: NULL buffer");
    const int64_t blocks = I * (int64_t)tile_width * tile_height;
    GS_REQUIRE(blocks < (1ll << 31), "rasterize_to_indices: too many tiles");
    hipStream_t st = as_stream(stream);
    const uint32_t *start = reinterpret_cast<const uint32_t *>(chunk_starts);
#define GS_IDX(TILE)                                                           \
    rasterize_indices_kernel<TILE, false><<<(unsigned)blocks, TILE * TILE, 0, st>>>( \
        a, N, range_start, range_end, transmittances, start, nullptr,          \
        gaussian_ids, pixel_ids)
    if (tile_size == 16) GS_IDX(16);
    else if (tile_size == 8) GS_IDX(8);
    else GS_IDX(4);
#undef GS_IDX
    return check_launch("rasterize_indices_kernel");
}
