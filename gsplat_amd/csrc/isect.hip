// Tile intersection: per-row tile sets, key emission and tile offsets.
//
// Semantics: gsplat/cuda/csrc/IntersectTile.cu
//   :38-121  ellipse ("AccuTile") column sweep,
//   :133-288 count / emit kernel (ellipse test when conics+opacities are
//            given, otherwise the axis-aligned box of the integer radii),
//   :391-439 tile offsets by key-boundary detection,
// and the host logic of gsplat/cuda/csrc/Intersect.cpp:33-164 (key layout
// image | tile | depth-bits, image_n_bits = bit_length(I), tile_n_bits =
// bit_length(tiles)).
//
// MI355X design: the count pass also produces the inclusive int64 prefix of
// the counts with a decoupled look-back, so the reference's separate cumsum
// kernel disappears.  Every floating-point step that decides which tiles are
// emitted runs in a fixed IEEE order with contraction disabled, with a
// defined float->int conversion (saturating, NaN -> 0) and a portable log, so
// the C host oracle reproduces the integer outputs bit for bit.  Count and
// emit call the same device function, so the two passes agree exactly.
#include "common.h"

namespace gs {
namespace {

constexpr int kIsectThreads = 256;

struct IsectArgs {
    int64_t n;      // rows
    int64_t N;      // Gaussians per image (dense layout)
    int64_t I;      // images
    const int64_t *image_ids;  // packed layout: image of each row
    const float *means2d;
    const int32_t *radii;
    const float *depths;
    const float *conics;
    const float *opacities;
    int32_t tile_size, tile_width, tile_height;
    int32_t tile_n_bits;
};

struct Emitter {
    int64_t *isect_ids;
    int32_t *flatten_ids;
    int64_t cursor;
    int64_t end;      // first slot of the next row (writes stay below it)
    int64_t key_hi;   // (image << (32 + tile_n_bits))
    int64_t depth_lo; // zero-extended depth bits
    int32_t flat;
    __device__ __forceinline__ void put(int64_t tile_id) {
        if (cursor < end) {
            isect_ids[cursor] = key_hi | (tile_id << 32) | depth_lo;
            flatten_ids[cursor] = flat;
        }
        ++cursor;
    }
};

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }

// Lower / upper root of the conic level set along the line u = coord.
__device__ __forceinline__ void ellipse_line(float A, float B, float C,
                                             float disc, float t, float px,
                                             float py, bool isY, float coord,
                                             float &lo, float &hi) {
#pragma clang fp contract(off)
    const float p_u = isY ? py : px;
    const float p_v = isY ? px : py;
    const float coeff = isY ? A : C;
    const float h = coord - p_u;
    const float sq = sqrtf((disc * h) * h + t * coeff);
    const float mbh = (-B) * h;
    lo = (mbh - sq) / coeff + p_v;
    hi = (mbh + sq) / coeff + p_v;
}

// Number of tiles touched by one row; emits them when `em` is non-null.
template <bool EMIT>
__device__ __forceinline__ int32_t row_tiles(const IsectArgs &a, int64_t idx,
                                             Emitter *em) {
#pragma clang fp contract(off)
    const int2 r = reinterpret_cast<const int2 *>(a.radii)[idx];
    const float radius_x = (float)r.x;
    const float radius_y = (float)r.y;
    if (radius_x <= 0.f || radius_y <= 0.f)
        return 0;
    const float2 mean = reinterpret_cast<const float2 *>(a.means2d)[idx];
    const int tw = a.tile_width, th = a.tile_height;
    const float ts = (float)a.tile_size;

    if (a.conics != nullptr && a.opacities != nullptr) {
        const float A = a.conics[idx * 3 + 0];
        const float B = a.conics[idx * 3 + 1];
        const float C = a.conics[idx * 3 + 2];
        const float disc = B * B - A * C;
        const float opacity = a.opacities[idx];
        const float t = fminf(kGaussianExtend * kGaussianExtend,
                              2.0f * portable_logf(opacity / kAlphaThreshold));
        // Guard: the level set is empty unless t >= 0 and the conic is
        // positive definite (disc < 0); the reference reaches 0 tiles in these
        // cases through NaN extents, here they are made explicit.
        if (!(t >= 0.f) || !(disc < 0.f))
            return 0;
        const float nt = (-t) / disc;
        const float x_ext = sqrtf(nt * C);
        const float y_ext = sqrtf(nt * A);
        float bmin_x = mean.x - x_ext, bmin_y = mean.y - y_ext;
        float bmax_x = mean.x + x_ext, bmax_y = mean.y + y_ext;
        const float bx_over_c = (B * x_ext) / C;
        const float by_over_a = (B * y_ext) / A;
        // argmin/argmax: (.x = y where x is extreme, .y = x where y is extreme)
        float amin_x = mean.y + bx_over_c, amin_y = mean.x + by_over_a;
        float amax_x = mean.y - bx_over_c, amax_y = mean.x - by_over_a;
        int rmin_x = imax(0, imin(tw, sat_f2i(bmin_x / ts)));
        int rmin_y = imax(0, imin(th, sat_f2i(bmin_y / ts)));
        int rmax_x = imax(0, imin(tw, sat_f2i(bmax_x / ts + 1.f)));
        int rmax_y = imax(0, imin(th, sat_f2i(bmax_y / ts + 1.f)));
        const int y_span = rmax_y - rmin_y;
        const int x_span = rmax_x - rmin_x;
        if (y_span == 0 || x_span == 0)
            return 0;
        const bool isY = y_span < x_span;
        if (isY) {
            // sweep along y: swap the roles of the axes
            int ti;
            float tf;
            ti = rmin_x; rmin_x = rmin_y; rmin_y = ti;
            ti = rmax_x; rmax_x = rmax_y; rmax_y = ti;
            tf = bmin_x; bmin_x = bmin_y; bmin_y = tf;
            tf = bmax_x; bmax_x = bmax_y; bmax_y = tf;
            tf = amin_x; amin_x = amin_y; amin_y = tf;
            tf = amax_x; amax_x = amax_y; amax_y = tf;
        }
        int32_t count = 0;
        // (lo, hi) roots at the previous and current line
        float max_lo = bmax_y, max_hi = bmin_y;
        float min_lo, min_hi;
        float min_line = (float)rmin_x * ts;
        if (bmin_x <= min_line) {
            ellipse_line(A, B, C, disc, t, mean.x, mean.y, isY, min_line,
                         min_lo, min_hi);
        } else {
            min_lo = max_lo;
            min_hi = max_hi;
        }
        for (int u = rmin_x; u < rmax_x; ++u) {
            const float max_line = min_line + ts;
            if (max_line <= bmax_x)
                ellipse_line(A, B, C, disc, t, mean.x, mean.y, isY, max_line,
                             max_lo, max_hi);
            float e_min, e_max;
            if (min_line <= amin_y && amin_y < max_line)
                e_min = bmin_y;
            else
                e_min = fminf(min_lo, max_lo);
            if (min_line <= amax_y && amax_y < max_line)
                e_max = bmax_y;
            else
                e_max = fmaxf(min_hi, max_hi);
            const int v0 = imax(rmin_y, imin(rmax_y, sat_f2i(e_min / ts)));
            const int v1 = imin(rmax_y, imax(rmin_y, sat_f2i(e_max / ts + 1.f)));
            if (v1 > v0) {
                count += v1 - v0;
                if (EMIT) {
                    for (int v = v0; v < v1; ++v) {
                        const int64_t tile =
                            isY ? (int64_t)u * tw + v : (int64_t)v * tw + u;
                        em->put(tile);
                    }
                }
            }
            min_lo = max_lo;
            min_hi = max_hi;
            min_line = max_line;
        }
        return count;
    }

    // axis-aligned box of the integer radii
    const float trx = radius_x / ts, try_ = radius_y / ts;
    const float tx = mean.x / ts, ty = mean.y / ts;
    const int x0 = imin(imax(0, sat_f2i(floorf(tx - trx))), tw);
    const int y0 = imin(imax(0, sat_f2i(floorf(ty - try_))), th);
    const int x1 = imin(imax(0, sat_f2i(ceilf(tx + trx))), tw);
    const int y1 = imin(imax(0, sat_f2i(ceilf(ty + try_))), th);
    if (EMIT) {
        for (int y = y0; y < y1; ++y)
            for (int x = x0; x < x1; ++x)
                em->put((int64_t)y * tw + x);
    }
    return (y1 - y0) * (x1 - x0);
}

__global__ void __launch_bounds__(kIsectThreads)
    isect_count_kernel(const IsectArgs a, Lookback lb,
                       int32_t *__restrict__ tiles_per_gauss,
                       int64_t *__restrict__ cum_tiles) {
    __shared__ uint32_t s_ticket;
    __shared__ uint64_t s_wave_tot[kIsectThreads / kWave];
    __shared__ uint64_t s_prefix;
    const uint32_t bid = lb_ticket(lb, &s_ticket);
    const int64_t idx = (int64_t)bid * kIsectThreads + threadIdx.x;
    int32_t cnt = 0;
    if (idx < a.n)
        cnt = row_tiles<false>(a, idx, nullptr);
    // block scan of the counts
    const uint64_t incl = wave_inclusive_scan_u64((uint64_t)cnt);
    const uint32_t wave = threadIdx.x / kWave;
    if (lane_id() == kWave - 1)
        s_wave_tot[wave] = incl;
    __syncthreads();
    uint64_t wave_off = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kIsectThreads / kWave; ++w) {
        const uint64_t v = s_wave_tot[w];
        wave_off += (w < (int)wave) ? v : 0ull;
        total += v;
    }
    if (wave == 0) {
        const uint64_t excl = lb_exclusive_prefix(lb, bid, total);
        if (lane_id() == 0)
            s_prefix = excl;
    }
    __syncthreads();
    if (idx < a.n) {
        tiles_per_gauss[idx] = cnt;
        cum_tiles[idx] = (int64_t)(s_prefix + wave_off + incl);
    }
}

__global__ void __launch_bounds__(kIsectThreads)
    isect_emit_kernel(const IsectArgs a, const int64_t *__restrict__ cum_tiles,
                      int64_t *__restrict__ isect_ids,
                      int32_t *__restrict__ flatten_ids) {
    const int64_t idx = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    if (idx >= a.n)
        return;
    const int32_t r0 = a.radii[idx * 2], r1 = a.radii[idx * 2 + 1];
    if (r0 <= 0 || r1 <= 0)
        return;
    Emitter em;
    em.isect_ids = isect_ids;
    em.flatten_ids = flatten_ids;
    em.cursor = idx == 0 ? 0 : cum_tiles[idx - 1];
    em.end = cum_tiles[idx];
    const int64_t iid = a.image_ids != nullptr ? a.image_ids[idx] : idx / a.N;
    em.key_hi = iid << (32 + a.tile_n_bits);
    em.depth_lo = (int64_t)(uint64_t)__float_as_uint(a.depths[idx]);
    em.flat = (int32_t)idx;
    row_tiles<true>(a, idx, &em);
}

// ---------------------------------------------------------------------------
// Sorted intersection in two stages.
//
// The reference sorts the emitted (key, row) pairs on all 32 + tile_bits +
// image_bits key bits (IntersectTile.cu:478-520).  Its result is the order by
// (image|tile, depth bits, row): the sort is stable and rows are emitted in
// ascending order.  The same order is produced here with far fewer bits
// moved:
//   1. rows are sorted stably by their depth bits (32-bit keys, one per
//      row instead of one per intersection);
//   2. every row's intersections are written to the slots the row occupies
//      in the depth-ordered layout (the prefix of the depth-ordered counts);
//   3. one stable radix sort on the image|tile bits only (usually one or two
//      passes) groups them by tile, keeping depth order (ties by row) inside.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kIsectThreads)
    isect_count_keys_kernel(const IsectArgs a, int32_t *__restrict__ tiles_per_gauss,
                            uint64_t *__restrict__ depth_keys,
                            uint32_t *__restrict__ rows) {
    const int64_t idx = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    if (idx >= a.n)
        return;
    tiles_per_gauss[idx] = row_tiles<false>(a, idx, nullptr);
    depth_keys[idx] = (uint64_t)__float_as_uint(a.depths[idx]);
    rows[idx] = (uint32_t)idx;
}

constexpr int kScanItemsPerThread = 16;
constexpr int kScanBlockRows = kIsectThreads * kScanItemsPerThread;

// For the depth order `order` (rows, depth ascending): each row's first slot
// in the depth-ordered emission, row_start[order[i]] = sum_{i' < i}
// tiles_per_gauss[order[i']], and the total (n_isects).  Blocks of 4096
// entries (16 consecutive per thread) chained by decoupled look-back.
__global__ void __launch_bounds__(kIsectThreads)
    depth_order_starts_kernel(int64_t n, const uint32_t *__restrict__ order,
                              const int32_t *__restrict__ tiles_per_gauss,
                              Lookback lb, int64_t *__restrict__ row_start,
                              int64_t *__restrict__ n_isects_out) {
    __shared__ uint32_t s_ticket;
    __shared__ uint64_t s_wave_tot[kIsectThreads / kWave];
    __shared__ uint64_t s_prefix;
    const uint32_t bid = lb_ticket(lb, &s_ticket);
    const int64_t i0 = (int64_t)bid * kScanBlockRows +
                       (int64_t)threadIdx.x * kScanItemsPerThread;
    uint32_t rows[kScanItemsPerThread];
    uint32_t cnt[kScanItemsPerThread];
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItemsPerThread; ++k) {
        const int64_t i = i0 + k;
        rows[k] = i < n ? order[i] : 0u;
        cnt[k] = i < n ? (uint32_t)tiles_per_gauss[rows[k]] : 0u;
        sum += cnt[k];
    }
    const uint64_t incl = wave_inclusive_scan_u64(sum);
    const uint32_t wave = threadIdx.x / kWave;
    if (lane_id() == kWave - 1)
        s_wave_tot[wave] = incl;
    __syncthreads();
    uint64_t wave_off = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kIsectThreads / kWave; ++w) {
        const uint64_t v = s_wave_tot[w];
        wave_off += (w < (int)wave) ? v : 0ull;
        total += v;
    }
    if (wave == 0) {
        const uint64_t excl = lb_exclusive_prefix(lb, bid, total);
        if (lane_id() == 0)
            s_prefix = excl;
    }
    __syncthreads();
    uint64_t run = s_prefix + wave_off + (incl - sum);
#pragma unroll
    for (int k = 0; k < kScanItemsPerThread; ++k) {
        if (i0 + k < n)
            row_start[rows[k]] = (int64_t)run;
        run += cnt[k];
    }
    if (i0 < n && i0 + kScanItemsPerThread >= n)
        *n_isects_out = (int64_t)run;  // the thread holding the last entry
}

// Row-order emission (the rows' own order spreads the rows with many tiles
// over the launch), each row written at its slots of the depth-ordered
// layout.
__global__ void __launch_bounds__(kIsectThreads)
    isect_emit_at_kernel(const IsectArgs a, const int32_t *__restrict__ tiles_per_gauss,
                         const int64_t *__restrict__ row_start,
                         uint64_t *__restrict__ isect_ids,
                         uint32_t *__restrict__ flatten_ids) {
    const int64_t idx = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    if (idx >= a.n)
        return;
    const int32_t count = tiles_per_gauss[idx];
    if (count == 0)
        return;
    Emitter em;
    em.isect_ids = reinterpret_cast<int64_t *>(isect_ids);
    em.flatten_ids = reinterpret_cast<int32_t *>(flatten_ids);
    em.cursor = row_start[idx];
    em.end = em.cursor + count;
    const int64_t iid = a.image_ids != nullptr ? a.image_ids[idx] : idx / a.N;
    em.key_hi = iid << (32 + a.tile_n_bits);
    em.depth_lo = (int64_t)(uint64_t)__float_as_uint(a.depths[idx]);
    em.flat = (int32_t)idx;
    row_tiles<true>(a, idx, &em);
}

struct PrepLayout {
    size_t keys_a, keys_b, vals_a, vals_b, lookback, sort_ws, total;
};

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

PrepLayout prep_layout(int64_t n) {
    PrepLayout L;
    const size_t k = align256((size_t)n * 8), v = align256((size_t)n * 4);
    L.keys_a = 0;
    L.keys_b = k;
    L.vals_a = 2 * k;
    L.vals_b = 2 * k + v;
    L.lookback = 2 * k + 2 * v;
    L.sort_ws = L.lookback + align256(lookback_bytes(ceil_div(n, kScanBlockRows)));
    L.total = L.sort_ws + radix_sort_workspace_bytes(n);
    return L;
}

struct EmitLayout {
    size_t keys, vals, sort_ws, total;
};

EmitLayout emit_layout(int64_t n_isects) {
    EmitLayout L;
    L.keys = 0;
    L.vals = align256((size_t)n_isects * 8);
    L.sort_ws = L.vals + align256((size_t)n_isects * 4);
    L.total = L.sort_ws + radix_sort_workspace_bytes(n_isects);
    return L;
}

__global__ void isect_offsets_kernel(int64_t n_isects,
                                     const int64_t *__restrict__ isect_ids,
                                     int64_t n_slots, int32_t tile_n_bits,
                                     int32_t n_tiles,
                                     int32_t *__restrict__ offsets) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_isects)
        return;
    const int64_t mask = (1ll << tile_n_bits) - 1;
    const int64_t key = isect_ids[idx] >> 32;
    const int64_t cur = (key >> tile_n_bits) * n_tiles + (key & mask);
    if (idx == 0) {
        for (int64_t i = 0; i <= cur && i < n_slots; ++i)
            offsets[i] = 0;
    } else {
        const int64_t pkey = isect_ids[idx - 1] >> 32;
        if (pkey != key) {
            const int64_t prev = (pkey >> tile_n_bits) * n_tiles + (pkey & mask);
            for (int64_t i = prev + 1; i <= cur && i < n_slots; ++i)
                offsets[i] = (int32_t)idx;
        }
    }
    if (idx == n_isects - 1) {
        for (int64_t i = cur + 1; i < n_slots; ++i)
            offsets[i] = (int32_t)n_isects;
    }
}

__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = v;
}

int bit_length(int64_t v) {
    int b = 0;
    while (v > 0) {
        ++b;
        v >>= 1;
    }
    return b;
}

int make_args(int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
              const float *means2d, const int32_t *radii, const float *depths,
              const float *conics, const float *opacities, int32_t tile_size,
              int32_t tile_width, int32_t tile_height, IsectArgs &a) {
    GS_REQUIRE(n >= 0, "isect: negative row count");
    GS_REQUIRE(tile_size > 0 && tile_width > 0 && tile_height > 0,
               "isect: tile sizes must be positive");
    GS_REQUIRE(image_ids != nullptr || N > 0 || n == 0,
               "isect: dense layout needs N > 0");
    if (n > 0)
        GS_REQUIRE(means2d && radii, "isect: NULL means2d/radii");
    const int tb = bit_length((int64_t)tile_width * tile_height);
    a.n = n;
    a.N = N;
    a.I = I;
    a.image_ids = image_ids;
    a.means2d = means2d;
    a.radii = radii;
    a.depths = depths;
    a.conics = conics;
    a.opacities = opacities;
    a.tile_size = tile_size;
    a.tile_width = tile_width;
    a.tile_height = tile_height;
    a.tile_n_bits = tb;
    return GSPLAT_OK;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gsplat_isect_count_workspace_size(int64_t n) {
    return lookback_bytes(ceil_div(n, kIsectThreads));
}

extern "C" int gsplat_isect_count(int64_t n, int64_t N,
                                  const int64_t *image_ids,
                                  const float *means2d, const int32_t *radii,
                                  const float *conics, const float *opacities,
                                  int32_t tile_size, int32_t tile_width,
                                  int32_t tile_height, void *workspace,
                                  size_t workspace_bytes,
                                  int32_t *tiles_per_gauss, int64_t *cum_tiles,
                                  gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, 0, image_ids, means2d, radii, nullptr, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(tiles_per_gauss && cum_tiles, "isect_count: NULL output");
    GS_REQUIRE(n < (1ll << 31), "isect_count: more than 2^31 rows");
    const int64_t blocks = ceil_div(n, kIsectThreads);
    GS_REQUIRE(workspace && workspace_bytes >= lookback_bytes(blocks),
               "isect_count: workspace too small");
    hipStream_t st = as_stream(stream);
    GS_TRY(clear_lookback(workspace, blocks, st));
    isect_count_kernel<<<(unsigned)blocks, kIsectThreads, 0, st>>>(
        a, lookback_from(workspace), tiles_per_gauss, cum_tiles);
    return check_launch("isect_count_kernel");
}

extern "C" int gsplat_isect_emit(int64_t n, int64_t N, int64_t I,
                                 const int64_t *image_ids,
                                 const float *means2d, const int32_t *radii,
                                 const float *depths, const float *conics,
                                 const float *opacities, int32_t tile_size,
                                 int32_t tile_width, int32_t tile_height,
                                 const int64_t *cum_tiles, int64_t *isect_ids,
                                 int32_t *flatten_ids, gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, I, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && cum_tiles && isect_ids && flatten_ids,
               "isect_emit: NULL buffer");
    GS_REQUIRE(I > 0, "isect_emit: I must be positive");
    const int ib = bit_length(I);
    GS_REQUIRE(ib + a.tile_n_bits <= 32,
               "isect_emit: image and tile ids need more than 32 bits");
    isect_emit_kernel<<<(unsigned)ceil_div(n, kIsectThreads), kIsectThreads, 0,
                        as_stream(stream)>>>(a, cum_tiles, isect_ids,
                                             flatten_ids);
    return check_launch("isect_emit_kernel");
}

extern "C" int gsplat_isect_offsets(int64_t n_isects, const int64_t *isect_ids,
                                    int64_t I, int32_t tile_width,
                                    int32_t tile_height, int32_t *offsets,
                                    gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(n_isects >= 0 && I >= 0, "isect_offsets: negative size");
    GS_REQUIRE(tile_width > 0 && tile_height > 0,
               "isect_offsets: tile sizes must be positive");
    const int64_t n_tiles = (int64_t)tile_width * tile_height;
    const int64_t n_slots = I * n_tiles;
    if (n_slots == 0)
        return GSPLAT_OK;
    GS_REQUIRE(offsets != nullptr, "isect_offsets: NULL offsets");
    hipStream_t st = as_stream(stream);
    if (n_isects == 0) {
        fill_i32_kernel<<<(unsigned)ceil_div(n_slots, 256), 256, 0, st>>>(
            offsets, n_slots, 0);
        return check_launch("fill_i32_kernel");
    }
    GS_REQUIRE(isect_ids != nullptr, "isect_offsets: NULL isect_ids");
    const int tb = bit_length(n_tiles);
    isect_offsets_kernel<<<(unsigned)ceil_div(n_isects, 256), 256, 0, st>>>(
        n_isects, isect_ids, n_slots, tb, (int32_t)n_tiles, offsets);
    return check_launch("isect_offsets_kernel");
}

extern "C" size_t gsplat_isect_prepare_workspace_size(int64_t n) {
    return prep_layout(n > 0 ? n : 0).total;
}

extern "C" int gsplat_isect_prepare(int64_t n, int64_t N, const int64_t *image_ids,
                                    const float *means2d, const int32_t *radii,
                                    const float *depths, const float *conics,
                                    const float *opacities, int32_t tile_size,
                                    int32_t tile_width, int32_t tile_height,
                                    void *workspace, size_t workspace_bytes,
                                    int32_t *tiles_per_gauss, int64_t *row_start,
                                    int64_t *n_isects_out, gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, 0, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && tiles_per_gauss && row_start && n_isects_out,
               "isect_prepare: NULL buffer");
    GS_REQUIRE(n < (1ll << 31), "isect_prepare: more than 2^31 rows");
    const PrepLayout L = prep_layout(n);
    GS_REQUIRE(workspace && workspace_bytes >= L.total,
               "isect_prepare: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    uint64_t *keys_a = reinterpret_cast<uint64_t *>(ws + L.keys_a);
    uint64_t *keys_b = reinterpret_cast<uint64_t *>(ws + L.keys_b);
    uint32_t *vals_a = reinterpret_cast<uint32_t *>(ws + L.vals_a);
    uint32_t *vals_b = reinterpret_cast<uint32_t *>(ws + L.vals_b);
    hipStream_t st = as_stream(stream);
    const unsigned grid = (unsigned)ceil_div(n, kIsectThreads);
    isect_count_keys_kernel<<<grid, kIsectThreads, 0, st>>>(a, tiles_per_gauss,
                                                             keys_a, vals_a);
    GS_TRY(check_launch("isect_count_keys_kernel"));
    bool in_b = false;
    GS_TRY(radix_sort_ping_pong(n, 0, 32, keys_a, vals_a, keys_b, vals_b,
                                ws + L.sort_ws, workspace_bytes - L.sort_ws, st,
                                &in_b));
    const uint32_t *order = in_b ? vals_b : vals_a;
    const int64_t scan_blocks = ceil_div(n, kScanBlockRows);
    GS_TRY(clear_lookback(ws + L.lookback, scan_blocks, st));
    depth_order_starts_kernel<<<(unsigned)scan_blocks, kIsectThreads, 0, st>>>(
        n, order, tiles_per_gauss, lookback_from(ws + L.lookback), row_start,
        n_isects_out);
    return check_launch("depth_order_starts_kernel");
}

extern "C" size_t gsplat_isect_emit_sorted_workspace_size(int64_t n_isects) {
    return emit_layout(n_isects > 0 ? n_isects : 0).total;
}

extern "C" int gsplat_isect_emit_sorted(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *tiles_per_gauss,
    const int64_t *row_start, int64_t n_isects, void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, I, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    GS_REQUIRE(n_isects >= 0, "isect_emit_sorted: negative n_isects");
    if (n == 0 || n_isects == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && tiles_per_gauss && row_start && isect_ids && flatten_ids,
               "isect_emit_sorted: NULL buffer");
    GS_REQUIRE(I > 0, "isect_emit_sorted: I must be positive");
    const int ib = bit_length(I);
    GS_REQUIRE(ib + a.tile_n_bits <= 32,
               "isect_emit_sorted: image and tile ids need more than 32 bits");
    GS_REQUIRE(n_isects < (1ll << 31), "isect_emit_sorted: more than 2^31 isects");
    const EmitLayout L = emit_layout(n_isects);
    GS_REQUIRE(workspace && workspace_bytes >= L.total,
               "isect_emit_sorted: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    uint64_t *tmp_keys = reinterpret_cast<uint64_t *>(ws + L.keys);
    uint32_t *tmp_vals = reinterpret_cast<uint32_t *>(ws + L.vals);
    uint64_t *out_keys = reinterpret_cast<uint64_t *>(isect_ids);
    uint32_t *out_vals = reinterpret_cast<uint32_t *>(flatten_ids);
    // emit where the tile passes will start so that they end in the outputs
    const int end_bit = 32 + a.tile_n_bits + ib;
    const bool odd = radix_sort_passes(end_bit - 32) % 2 == 1;
    uint64_t *ka = odd ? tmp_keys : out_keys, *kb = odd ? out_keys : tmp_keys;
    uint32_t *va = odd ? tmp_vals : out_vals, *vb = odd ? out_vals : tmp_vals;
    hipStream_t st = as_stream(stream);
    isect_emit_at_kernel<<<(unsigned)ceil_div(n, kIsectThreads), kIsectThreads,
                           0, st>>>(a, tiles_per_gauss, row_start, ka, va);
    GS_TRY(check_launch("isect_emit_at_kernel"));
    bool in_b = false;
    GS_TRY(radix_sort_ping_pong(n_isects, 32, end_bit, ka, va, kb, vb,
                                ws + L.sort_ws, workspace_bytes - L.sort_ws, st,
                                &in_b));
    if ((in_b ? kb : ka) != out_keys)
        return copy_pairs(n_isects, in_b ? kb : ka, in_b ? vb : va, out_keys,
                          out_vals, st);
    return GSPLAT_OK;
}
