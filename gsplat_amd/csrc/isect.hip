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
#include <algorithm>

#include "radix.h"
#include "sh_rows.h"

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

// Per-row state of the ellipse ("AccuTile") column sweep, or of the
// axis-aligned box when no conics/opacities are given.  After the axis swap
// (isY), columns u in [rmin_x, rmax_x) are swept along x and each column
// covers rows v in [v0, v1) of tiles.
struct Sweep {
    bool accu, isY;
    bool pow2;     // tile size is a power of two: x / ts == x * inv_ts exactly
    float A, B, C, disc, t, mx, my, ts, inv_ts;
    float bmin_x, bmax_x, bmin_y, bmax_y, amin_y, amax_y;
    int rmin_x, rmax_x, rmin_y, rmax_y;
};

// x / ts, as a multiplication when ts is a power of two (both give the
// correctly rounded x / ts).
__device__ __forceinline__ float div_ts(const Sweep &sw, float x) {
    return sw.pow2 ? x * sw.inv_ts : x / sw.ts;
}

// Opacity-derived squared extent of the ellipse level set (the sweep's t).
__device__ __forceinline__ float sweep_extent(float opacity) {
#pragma clang fp contract(off)
    return fminf(kGaussianExtend * kGaussianExtend,
                 2.0f * portable_logf(opacity / kAlphaThreshold));
}

// Fills *sw from one row's values (mean, conic A B C and extent t for the
// ellipse sweep, integer radii for both); returns false when the row
// touches no tile.
__device__ __forceinline__ bool sweep_setup_vals(const IsectArgs &a, float mx,
                                                 float my, float A, float B,
                                                 float C, float t,
                                                 float radius_x, float radius_y,
                                                 Sweep *sw) {
#pragma clang fp contract(off)
    if (radius_x <= 0.f || radius_y <= 0.f)
        return false;
    const float2 mean = make_float2(mx, my);
    const int tw = a.tile_width, th = a.tile_height;
    const float ts = (float)a.tile_size;
    sw->ts = ts;
    sw->pow2 = (a.tile_size & (a.tile_size - 1)) == 0;
    sw->inv_ts = 1.f / ts;
    sw->mx = mean.x;
    sw->my = mean.y;

    if (a.conics != nullptr && a.opacities != nullptr) {
        sw->accu = true;
        const float disc = B * B - A * C;
        // Guard: the level set is empty unless t >= 0 and the conic is
        // positive definite (disc < 0); the reference reaches 0 tiles in these
        // cases through NaN extents, here they are made explicit.
        if (!(t >= 0.f) || !(disc < 0.f))
            return false;
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
        int rmin_x = imax(0, imin(tw, sat_f2i(div_ts(*sw, bmin_x))));
        int rmin_y = imax(0, imin(th, sat_f2i(div_ts(*sw, bmin_y))));
        int rmax_x = imax(0, imin(tw, sat_f2i(div_ts(*sw, bmax_x) + 1.f)));
        int rmax_y = imax(0, imin(th, sat_f2i(div_ts(*sw, bmax_y) + 1.f)));
        const int y_span = rmax_y - rmin_y;
        const int x_span = rmax_x - rmin_x;
        if (y_span == 0 || x_span == 0)
            return false;
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
        sw->isY = isY;
        sw->A = A;
        sw->B = B;
        sw->C = C;
        sw->disc = disc;
        sw->t = t;
        sw->bmin_x = bmin_x;
        sw->bmax_x = bmax_x;
        sw->bmin_y = bmin_y;
        sw->bmax_y = bmax_y;
        sw->amin_y = amin_y;
        sw->amax_y = amax_y;
        sw->rmin_x = rmin_x;
        sw->rmax_x = rmax_x;
        sw->rmin_y = rmin_y;
        sw->rmax_y = rmax_y;
        return true;
    }

    // axis-aligned box of the integer radii; "columns" are tile rows y, each
    // covering tiles x in [x0, x1)
    sw->accu = false;
    sw->isY = true;
    const float trx = div_ts(*sw, radius_x), try_ = div_ts(*sw, radius_y);
    const float tx = div_ts(*sw, mean.x), ty = div_ts(*sw, mean.y);
    sw->rmin_y = imin(imax(0, sat_f2i(floorf(tx - trx))), tw);
    sw->rmin_x = imin(imax(0, sat_f2i(floorf(ty - try_))), th);
    sw->rmax_y = imin(imax(0, sat_f2i(ceilf(tx + trx))), tw);
    sw->rmax_x = imin(imax(0, sat_f2i(ceilf(ty + try_))), th);
    return sw->rmax_y > sw->rmin_y && sw->rmax_x > sw->rmin_x;
}

// The row's values from the row arrays.
__device__ __forceinline__ bool sweep_setup(const IsectArgs &a, int64_t idx,
                                            Sweep *sw) {
    const int2 r = reinterpret_cast<const int2 *>(a.radii)[idx];
    const float2 mean = reinterpret_cast<const float2 *>(a.means2d)[idx];
    float A = 0.f, B = 0.f, C = 0.f, t = 0.f;
    if (a.conics != nullptr && a.opacities != nullptr) {
        A = a.conics[idx * 3 + 0];
        B = a.conics[idx * 3 + 1];
        C = a.conics[idx * 3 + 2];
        t = sweep_extent(a.opacities[idx]);
    }
    return sweep_setup_vals(a, mean.x, mean.y, A, B, C, t, (float)r.x,
                            (float)r.y, sw);
}

// One row packed in 32 bytes for the depth-ordered emission: (mean, A, B),
// (C, t, depth bits, image id) -- t < 0 when a radius is not positive, so the
// sweep sees no tile -- or, for the box, (mean, radii), (0, 0, depth bits,
// image id).
struct alignas(16) RowRec {
    float4 p, q;
};

__device__ __forceinline__ RowRec row_record(const IsectArgs &a, int64_t idx) {
    const int2 r = reinterpret_cast<const int2 *>(a.radii)[idx];
    const float2 mean = reinterpret_cast<const float2 *>(a.means2d)[idx];
    const int64_t iid = a.image_ids != nullptr ? a.image_ids[idx] : idx / a.N;
    const float dbits = a.depths[idx];
    RowRec rec;
    if (a.conics != nullptr && a.opacities != nullptr) {
        const float t = (r.x > 0 && r.y > 0) ? sweep_extent(a.opacities[idx]) : -1.f;
        rec.p = make_float4(mean.x, mean.y, a.conics[idx * 3 + 0], a.conics[idx * 3 + 1]);
        rec.q = make_float4(a.conics[idx * 3 + 2], t, dbits, __int_as_float((int)iid));
    } else {
        rec.p = make_float4(mean.x, mean.y, (float)r.x, (float)r.y);
        rec.q = make_float4(0.f, 0.f, dbits, __int_as_float((int)iid));
    }
    return rec;
}

__device__ __forceinline__ bool sweep_setup_rec(const IsectArgs &a,
                                                const RowRec &rec, Sweep *sw) {
    if (a.conics != nullptr && a.opacities != nullptr)
        return sweep_setup_vals(a, rec.p.x, rec.p.y, rec.p.z, rec.p.w, rec.q.x,
                                rec.q.y, 1.f, 1.f, sw);
    return sweep_setup_vals(a, rec.p.x, rec.p.y, 0.f, 0.f, 0.f, 0.f, rec.p.z,
                            rec.p.w, sw);
}

// Tile rows [v0, v1) of column u from the roots at its two lines.
__device__ __forceinline__ void sweep_span(const Sweep &sw, float min_line,
                                           float max_line, float min_lo,
                                           float min_hi, float max_lo,
                                           float max_hi, int &v0, int &v1) {
#pragma clang fp contract(off)
    float e_min, e_max;
    if (min_line <= sw.amin_y && sw.amin_y < max_line)
        e_min = sw.bmin_y;
    else
        e_min = fminf(min_lo, max_lo);
    if (min_line <= sw.amax_y && sw.amax_y < max_line)
        e_max = sw.bmax_y;
    else
        e_max = fmaxf(min_hi, max_hi);
    v0 = imax(sw.rmin_y, imin(sw.rmax_y, sat_f2i(div_ts(sw, e_min))));
    v1 = imin(sw.rmax_y, imax(sw.rmin_y, sat_f2i(div_ts(sw, e_max) + 1.f)));
}

__device__ __forceinline__ void sweep_roots(const Sweep &sw, float line,
                                            float &lo, float &hi) {
    ellipse_line(sw.A, sw.B, sw.C, sw.disc, sw.t, sw.mx, sw.my, sw.isY, line,
                 lo, hi);
}

// Tile id of (column u, row v) of the sweep.
__device__ __forceinline__ int64_t sweep_tile(const Sweep &sw, int tw, int u,
                                              int v) {
    return sw.isY ? (int64_t)u * tw + v : (int64_t)v * tw + u;
}

// Number of tiles touched by one row; emits them (column by column, rows v
// ascending) when EMIT.  The sweep carries the roots of the previous line
// from column to column (IntersectTile.cu:38-121).
template <bool EMIT>
__device__ __forceinline__ int32_t sweep_tiles(const IsectArgs &a,
                                               const Sweep &sw, Emitter *em) {
#pragma clang fp contract(off)
    const int tw = a.tile_width;
    if (!sw.accu) {
        if (EMIT) {
            for (int y = sw.rmin_x; y < sw.rmax_x; ++y)
                for (int x = sw.rmin_y; x < sw.rmax_y; ++x)
                    em->put((int64_t)y * tw + x);
        }
        return (sw.rmax_x - sw.rmin_x) * (sw.rmax_y - sw.rmin_y);
    }
    const float ts = sw.ts;
    int32_t count = 0;
    // (lo, hi) roots at the previous and current line
    float max_lo = sw.bmax_y, max_hi = sw.bmin_y;
    float min_lo, min_hi;
    float min_line = (float)sw.rmin_x * ts;
    if (sw.bmin_x <= min_line) {
        sweep_roots(sw, min_line, min_lo, min_hi);
    } else {
        min_lo = max_lo;
        min_hi = max_hi;
    }
    for (int u = sw.rmin_x; u < sw.rmax_x; ++u) {
        const float max_line = min_line + ts;
        if (max_line <= sw.bmax_x)
            sweep_roots(sw, max_line, max_lo, max_hi);
        int v0, v1;
        sweep_span(sw, min_line, max_line, min_lo, min_hi, max_lo, max_hi, v0, v1);
        if (v1 > v0) {
            count += v1 - v0;
            if (EMIT) {
                for (int v = v0; v < v1; ++v)
                    em->put(sweep_tile(sw, tw, u, v));
            }
        }
        min_lo = max_lo;
        min_hi = max_hi;
        min_line = max_line;
    }
    return count;
}

template <bool EMIT>
__device__ __forceinline__ int32_t row_tiles(const IsectArgs &a, int64_t idx,
                                             Emitter *em) {
    Sweep sw;
    if (!sweep_setup(a, idx, &sw))
        return 0;
    return sweep_tiles<EMIT>(a, sw, em);
}

// The last column j in [rmin_x - 1, rmax_x - 1] whose right line
// (j + 1) * ts lies at or left of bmax_x (rmin_x - 1: none).  Lines are
// exact integers in float, so they equal the sweep's running sums.
__device__ __forceinline__ int sweep_last_line(const Sweep &sw) {
#pragma clang fp contract(off)
    int lo = sw.rmin_x - 1, hi = sw.rmax_x - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((float)(mid + 1) * sw.ts <= sw.bmax_x)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Column u of the sweep evaluated on its own, with the sweep's carried state
// in closed form: the roots a column ends with are those of the last line
// j + 1 <= min(u, J) + 1 evaluated so far (J = sweep_last_line), or the
// initial (bmax_y, bmin_y) when none was; a column starts with the previous
// column's, and the first column with its own left line when bmin_x lies at
// or left of it.  Gives exactly the [v0, v1) of row_tiles.
__device__ __forceinline__ void sweep_column(const Sweep &sw, int J, int u,
                                             int &v0, int &v1) {
#pragma clang fp contract(off)
    const float ts = sw.ts;
    if (!sw.accu) {
        v0 = sw.rmin_y;
        v1 = sw.rmax_y;
        return;
    }
    const float min_line = (float)u * ts;
    const float max_line = (float)(u + 1) * ts;
    float min_lo, min_hi, max_lo, max_hi;
    // roots the column ends with
    const int je = u < J ? u : J;
    if (je >= sw.rmin_x) {
        sweep_roots(sw, (float)(je + 1) * ts, max_lo, max_hi);
    } else {
        max_lo = sw.bmax_y;
        max_hi = sw.bmin_y;
    }
    // roots the column starts with
    if (u == sw.rmin_x) {
        if (sw.bmin_x <= min_line) {
            sweep_roots(sw, min_line, min_lo, min_hi);
        } else {
            min_lo = sw.bmax_y;
            min_hi = sw.bmin_y;
        }
    } else {
        const int js = (u - 1) < J ? (u - 1) : J;
        if (js == je) {
            min_lo = max_lo;
            min_hi = max_hi;
        } else if (js >= sw.rmin_x) {
            sweep_roots(sw, (float)(js + 1) * ts, min_lo, min_hi);
        } else {
            min_lo = sw.bmax_y;
            min_hi = sw.bmin_y;
        }
    }
    sweep_span(sw, min_line, max_line, min_lo, min_hi, max_lo, max_hi, v0, v1);
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
                            uint32_t *__restrict__ depth_keys,
                            uint32_t *__restrict__ rows,
                            RowRec *__restrict__ recs) {
    const int64_t idx = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    if (idx >= a.n)
        return;
    const RowRec rec = row_record(a, idx);
    recs[idx] = rec;
    Sweep sw;
    tiles_per_gauss[idx] =
        sweep_setup_rec(a, rec, &sw) ? sweep_tiles<false>(a, sw, nullptr) : 0;
    depth_keys[idx] = __float_as_uint(rec.q.z);
    rows[idx] = (uint32_t)idx;
}

constexpr int kScanItemsPerThread = 16;
constexpr int kScanBlockRows = kIsectThreads * kScanItemsPerThread;

// For the depth order `order` (rows, depth ascending): the first slot of
// every depth position in the depth-ordered emission, dstart[i] =
// sum_{i' < i} tiles_per_gauss[order[i']], dstart[n] = n_isects (also
// written to *n_isects_out).  Blocks of 4096 entries (16 consecutive per
// thread) chained by decoupled look-back.
__global__ void __launch_bounds__(kIsectThreads)
    depth_order_starts_kernel(int64_t n, const uint32_t *__restrict__ order,
                              const int32_t *__restrict__ tiles_per_gauss,
                              Lookback lb, int64_t *__restrict__ dstart,
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
            dstart[i0 + k] = (int64_t)run;
        run += cnt[k];
    }
    if (i0 < n && i0 + kScanItemsPerThread >= n) {
        // the thread holding the last entry
        dstart[n] = (int64_t)run;
        *n_isects_out = (int64_t)run;
    }
}

// Ordered emission.  The rows in the given order (`order`: the depth order,
// or NULL: row order) own consecutive slot ranges (the prefix dstart of their
// counts in that order); the slots are cut into chunks of kEmitSlots and
// each wave writes one chunk, front to back, with consecutive lanes on
// consecutive slots:
//   1. the rows that overlap the chunk (from chunk_first, 64 per batch) set
//      up their sweeps (kept in LDS);
//   2. their columns, in (row, column) order, are evaluated one per lane
//      (sweep_column), giving one segment -- an arithmetic run of tile ids --
//      per column, kEmitCols columns at a time; a column finds its row the
//      same way (rows mark their first column, running maximum);
//   3. the chunk's slots are expanded tile by tile: every segment reaching
//      into the chunk marks its first slot there and a running maximum over
//      the slots (DPP scan) gives each slot its segment.
// Every wave writes the same number of slots whatever the rows' tile counts
// (1 to thousands: a large row is shared by the waves of its chunks), and
// every store is coalesced.  The layout equals that of row_tiles<true>
// (column by column, rows v ascending) at each row's slots.
constexpr int kEmitWaves = kIsectThreads / kWave;
constexpr int kEmitCols = 4 * kWave;   // segments per batch (4 per lane)
constexpr int kEmitSlots = 4 * kWave;  // slots per wave
enum { kRowA, kRowB, kRowC, kRowDisc, kRowT, kRowMx, kRowMy, kRowBminX,
       kRowBmaxX, kRowBminY, kRowBmaxY, kRowAminY, kRowAmaxY, kRowFloats };
enum { kRowRminX, kRowRmaxX, kRowRminY, kRowRmaxY, kRowJ, kRowFlags,
       kRowFlat, kRowInts };

// chunk_first[c] = the depth position whose slot range holds slot
// c * kEmitSlots (rows without tiles own no slot).  Also clears the
// `zero_words` words at `zero` (the tile sort's first counts) for the launch
// that follows.
__global__ void __launch_bounds__(kIsectThreads)
    emit_chunk_first_kernel(int64_t n, const int64_t *__restrict__ dstart,
                            int64_t cap, int32_t *__restrict__ chunk_first,
                            uint32_t *__restrict__ zero, int64_t zero_words) {
    const int64_t i = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    for (int64_t z = i; z < zero_words; z += (int64_t)gridDim.x * kIsectThreads)
        zero[z] = 0u;
    if (i >= n)
        return;
    // slots at or past the capacity are not emitted (cap >= dstart[n] on
    // the exact path)
    const int64_t lo = dstart[i], hi = min(dstart[i + 1], cap);
    for (int64_t c = (lo + kEmitSlots - 1) / kEmitSlots; c * kEmitSlots < hi; ++c)
        chunk_first[c] = (int32_t)i;
}

__global__ void __launch_bounds__(kIsectThreads)
    isect_emit_depth_kernel(const IsectArgs a,
                            const uint32_t *__restrict__ order,
                            const int64_t *__restrict__ dstart,
                            const RowRec *__restrict__ recs,
                            const int32_t *__restrict__ chunk_first,
                            int64_t n_isects, const int64_t *__restrict__ n_dev,
                            uint32_t *__restrict__ isect_keys,
                            uint32_t *__restrict__ flatten_ids) {
    __shared__ float s_f[kEmitWaves][kRowFloats][kWave];
    __shared__ int32_t s_i[kEmitWaves][kRowInts][kWave];
    __shared__ uint32_t s_key[kEmitWaves][kWave];
    __shared__ int32_t s_colpre[kEmitWaves][kWave + 1];
    __shared__ int32_t s_first[kEmitWaves][kEmitCols];
    __shared__ int32_t s_meta[kEmitWaves][kEmitCols];
    __shared__ int32_t s_start[kEmitWaves][kEmitCols];
    __shared__ int32_t s_own[kEmitWaves][kEmitCols > kEmitSlots ? kEmitCols : kEmitSlots];

    const int wave = threadIdx.x / kWave;
    const int lane = (int)lane_id();
    const int64_t chunk = (int64_t)blockIdx.x * kEmitWaves + wave;
    const int64_t S = chunk * kEmitSlots;
    if (n_dev != nullptr)  // count on the device, n_isects the capacity
        n_isects = min(n_isects, *n_dev);
    if (S >= n_isects)
        return;
    const int64_t E = n_isects < S + kEmitSlots ? n_isects : S + kEmitSlots;
    const int tw = a.tile_width;
    const float ts = (float)a.tile_size;
    const float inv_ts = 1.f / ts;
    const bool pow2 = (a.tile_size & (a.tile_size - 1)) == 0;

    for (int64_t pb = chunk_first[chunk]; pb < a.n; pb += kWave) {
        const int64_t base = dstart[pb];  // first slot of the batch
        if (base >= E)
            break;
        // 1. rows of the batch that start before the chunk's end
        const int64_t p = pb + lane;
        Sweep sw;
        bool has = false;
        if (p < a.n && dstart[p] < E) {
            const int64_t row = order != nullptr ? (int64_t)order[p] : p;
            const RowRec rec = recs[row];
            has = sweep_setup_rec(a, rec, &sw);
            if (has) {
                float *f = &s_f[wave][0][lane];
                f[kRowA * kWave] = sw.A;
                f[kRowB * kWave] = sw.B;
                f[kRowC * kWave] = sw.C;
                f[kRowDisc * kWave] = sw.disc;
                f[kRowT * kWave] = sw.t;
                f[kRowMx * kWave] = sw.mx;
                f[kRowMy * kWave] = sw.my;
                f[kRowBminX * kWave] = sw.bmin_x;
                f[kRowBmaxX * kWave] = sw.bmax_x;
                f[kRowBminY * kWave] = sw.bmin_y;
                f[kRowBmaxY * kWave] = sw.bmax_y;
                f[kRowAminY * kWave] = sw.amin_y;
                f[kRowAmaxY * kWave] = sw.amax_y;
                int32_t *q = &s_i[wave][0][lane];
                q[kRowRminX * kWave] = sw.rmin_x;
                q[kRowRmaxX * kWave] = sw.rmax_x;
                q[kRowRminY * kWave] = sw.rmin_y;
                q[kRowRmaxY * kWave] = sw.rmax_y;
                q[kRowJ * kWave] = sw.accu ? sweep_last_line(sw) : 0;
                q[kRowFlags * kWave] = (sw.accu ? 1 : 0) | (sw.isY ? 2 : 0);
                q[kRowFlat * kWave] = (int32_t)row;
                s_key[wave][lane] = (uint32_t)__float_as_int(rec.q.w) << a.tile_n_bits;
            }
        }
        const int ncols = has ? sw.rmax_x - sw.rmin_x : 0;
        const int col_incl = (int)wave_inclusive_scan_u32((uint32_t)ncols);
        s_colpre[wave][lane + 1] = col_incl;
        if (lane == 0)
            s_colpre[wave][0] = 0;
        const int total_cols = __shfl(col_incl, kWave - 1);
        __builtin_amdgcn_wave_barrier();

        int64_t seg_base = base;  // first slot of the current column batch
        for (int cb = 0; cb < total_cols && seg_base < E; cb += kEmitCols) {
            const int nseg =
                total_cols - cb < kEmitCols ? total_cols - cb : kEmitCols;
            // owner row of every column of the batch: each row marks its
            // first column in the batch, a running maximum fills the rest
#pragma unroll
            for (int q = 0; q < kEmitCols / kWave; ++q)
                s_own[wave][q * kWave + lane] = -1;
            __builtin_amdgcn_wave_barrier();
            if (ncols > 0) {
                const int lo = col_incl - ncols, hi = col_incl;
                if (lo < cb + nseg && hi > cb)
                    s_own[wave][(lo > cb ? lo : cb) - cb] = lane;
            }
            __builtin_amdgcn_wave_barrier();
            // 2. segments: column cb + 64 q + lane, slice by slice
            int batch_total = 0;
            int row_carry = -1;
            int starts[kEmitCols / kWave], lens[kEmitCols / kWave];
#pragma unroll
            for (int q = 0; q < kEmitCols / kWave; ++q) {
                const int k = q * kWave + lane;  // segment index in the batch
                starts[q] = 0;
                lens[q] = 0;
                if (q * kWave >= nseg)
                    continue;
                const int r = max(wave_inclusive_max_i32(s_own[wave][k]), row_carry);
                row_carry = __shfl(r, kWave - 1);
                int len = 0;
                if (k < nseg) {
                    const int c = cb + k;
                    Sweep cs;
                    const float *f = &s_f[wave][0][r];
                    cs.A = f[kRowA * kWave];
                    cs.B = f[kRowB * kWave];
                    cs.C = f[kRowC * kWave];
                    cs.disc = f[kRowDisc * kWave];
                    cs.t = f[kRowT * kWave];
                    cs.mx = f[kRowMx * kWave];
                    cs.my = f[kRowMy * kWave];
                    cs.bmin_x = f[kRowBminX * kWave];
                    cs.bmax_x = f[kRowBmaxX * kWave];
                    cs.bmin_y = f[kRowBminY * kWave];
                    cs.bmax_y = f[kRowBmaxY * kWave];
                    cs.amin_y = f[kRowAminY * kWave];
                    cs.amax_y = f[kRowAmaxY * kWave];
                    cs.ts = ts;
                    cs.inv_ts = inv_ts;
                    cs.pow2 = pow2;
                    const int32_t *qi = &s_i[wave][0][r];
                    cs.rmin_x = qi[kRowRminX * kWave];
                    cs.rmax_x = qi[kRowRmaxX * kWave];
                    cs.rmin_y = qi[kRowRminY * kWave];
                    cs.rmax_y = qi[kRowRmaxY * kWave];
                    const int flags = qi[kRowFlags * kWave];
                    cs.accu = flags & 1;
                    cs.isY = (flags >> 1) & 1;
                    const int u = cs.rmin_x + (c - s_colpre[wave][r]);
                    int v0, v1;
                    sweep_column(cs, qi[kRowJ * kWave], u, v0, v1);
                    len = v1 > v0 ? v1 - v0 : 0;
                    s_first[wave][k] = (int32_t)sweep_tile(cs, tw, u, v0);
                    s_meta[wave][k] = r | (cs.isY ? 0x100 : 0);
                }
                const int incl = (int)wave_inclusive_scan_u32((uint32_t)len);
                starts[q] = batch_total + incl - len;
                lens[q] = len;
                if (k < nseg)
                    s_start[wave][k] = starts[q];
                batch_total += __shfl(incl, kWave - 1);
            }
            // 3. the chunk's slots: owner segment of every slot of [S, E)
            // (each segment that reaches into the chunk marks its first slot
            // there, a running maximum fills the rest)
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < kEmitSlots / kWave; ++q)
                s_own[wave][q * kWave + lane] = -1;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < kEmitCols / kWave; ++q) {
                if (lens[q] > 0) {
                    const int64_t lo = seg_base + starts[q];
                    const int64_t hi = lo + lens[q];
                    if (lo < E && hi > S)
                        s_own[wave][(int)((lo > S ? lo : S) - S)] = q * kWave + lane;
                }
            }
            __builtin_amdgcn_wave_barrier();
            const int64_t seg_end = seg_base + batch_total;
            int seg_carry = -1;
#pragma unroll
            for (int q = 0; q < kEmitSlots / kWave; ++q) {
                const int i = q * kWave + lane;
                const int sk = max(wave_inclusive_max_i32(s_own[wave][i]), seg_carry);
                seg_carry = __shfl(sk, kWave - 1);
                const int64_t slot = S + i;
                if (sk >= 0 && slot < E && slot < seg_end) {
                    const int meta = s_meta[wave][sk];
                    const int r = meta & 0xFF;
                    const int off = (int)(slot - seg_base) - s_start[wave][sk];
                    const uint32_t tile =
                        (uint32_t)s_first[wave][sk] +
                        (uint32_t)off * ((meta & 0x100) ? 1u : (uint32_t)tw);
                    isect_keys[slot] = s_key[wave][r] | tile;
                    flatten_ids[slot] = (uint32_t)s_i[wave][kRowFlat][r];
                }
            }
            seg_base += batch_total;
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// ---------------------------------------------------------------------------
// Sorted intersection, tile first (the form rasterization() uses).
//
//   1. isect_count_rows_kernel: every row's tile count and sweep record,
//      and the row-order exclusive prefix of the counts (prefix inside each
//      workgroup; isect_starts_scan_kernel adds the totals of the
//      workgroups before); starts[n] = n_isects.  A decoupled look-back over the ~2,600
//      workgroups of this VALU-heavy kernel took 71 us at config 1, against
//      24 us for the counts alone: every waiting workgroup polls its
//      predecessors' status words through the device-coherent level.
//   2. emission in row order (isect_emit_depth_kernel with no order): a
//      32-bit image|tile key and the row per slot.
//   3. a stable radix sort on the image|tile bits: the slots grouped by
//      tile, in row order inside each tile.
//   4. tile_bounds_kernel: the first slot of every tile from the sorted keys
//      (the reference's isect_offset_encode).
//   5. tile_depth_sort_kernel: one workgroup per tile sorts the tile's rows
//      stably on their 32 depth bits -- in LDS up to 2,560 or 4,096 rows,
//      by the mean tile depth (radix passes over the top 16 bits of the
//      tile's depth range, then the rows that tie on those bits by odd-even
//      transposition), through global scratch above -- and writes the
//      64-bit ids and the rows.
// The reference sorts stably on image|tile|depth over row-order emission,
// which orders by (image|tile, depth bits, row); steps 3 and 5 produce that
// order.  The depth order is taken per tile (~1,000 rows at config 1) in LDS
// instead of over all rows through device memory.
// ---------------------------------------------------------------------------
// The rows [blk * kIsectThreads, ...) of isect_count_rows_kernel from their
// records (`rec` holds row_record of the thread's row where it is below
// a.n): a whole workgroup, which it synchronises.
__device__ __forceinline__ void isect_count_rows_from(
    const IsectArgs &a, int64_t blk, const RowRec &rec,
    int32_t *__restrict__ tiles_per_gauss, RowRec *__restrict__ recs,
    int64_t *__restrict__ starts, uint64_t *__restrict__ block_tot) {
    __shared__ uint64_t s_wave_tot[kIsectThreads / kWave];
    const int64_t idx = blk * kIsectThreads + threadIdx.x;
    int32_t cnt = 0;
    if (idx < a.n) {
        recs[idx] = rec;
        Sweep sw;
        cnt = sweep_setup_rec(a, rec, &sw) ? sweep_tiles<false>(a, sw, nullptr) : 0;
    }
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
    if (idx < a.n) {
        tiles_per_gauss[idx] = cnt;
        // the prefix inside the workgroup; isect_starts_scan_kernel adds
        // the workgroup's own prefix
        starts[idx] = (int64_t)(wave_off + incl - (uint64_t)cnt);
    }
    if (threadIdx.x == 0)
        block_tot[blk] = total;
}

__global__ void __launch_bounds__(kIsectThreads)
    isect_count_rows_kernel(const IsectArgs a, int32_t *__restrict__ tiles_per_gauss,
                            RowRec *__restrict__ recs,
                            int64_t *__restrict__ starts,
                            uint64_t *__restrict__ block_tot) {
    const int64_t idx = (int64_t)blockIdx.x * kIsectThreads + threadIdx.x;
    RowRec rec{};
    if (idx < a.n)
        rec = row_record(a, idx);
    isect_count_rows_from(a, blockIdx.x, rec, tiles_per_gauss, recs, starts, block_tot);
}

// The packed rows' SH colours and their tile counts in one launch.  Thread i
// takes Gaussian i's colours and packed row i's tile count.  Its count row
// is loaded first and its coefficient row after; loads complete in issue
// order, so the tile sweep (arithmetic) runs while the coefficient row (the
// SH forward's wait) is still in flight, where the two kernels one after
// the other each waited alone.  The row count comes from the device
// (*n_dev, written by the projection); rows at or past it count nothing.
static_assert(kShThreads == kIsectThreads, "one workgroup shape for both parts");

template <int DEG>
__global__ void __launch_bounds__(kIsectThreads)
    sh_rows_count_kernel(const ShRowsArgs sa, float *__restrict__ colors, IsectArgs ia,
                         const int32_t *__restrict__ n_dev,
                         int32_t *__restrict__ tiles_per_gauss,
                         RowRec *__restrict__ recs, int64_t *__restrict__ starts,
                         uint64_t *__restrict__ block_tot) {
    const int64_t blk = blockIdx.x;
    const int64_t i = blk * kIsectThreads + threadIdx.x;
    const int64_t n = *n_dev;
    const bool counting = blk * kIsectThreads < n;  // the whole workgroup
    ia.n = n;
    RowRec rec{};
    if (i < n)
        rec = row_record(ia, i);
    ShRowIn<DEG> in;
    const bool vis = sh_rows_fwd_load<DEG>(sa, i, in);
    if (counting)
        isect_count_rows_from(ia, blk, rec, tiles_per_gauss, recs, starts, block_tot);
    if (vis)
        sh_rows_fwd_eval<DEG>(sa, colors, i, in);
}

// Row starts from the per-workgroup prefixes of isect_count_rows_kernel, in
// one launch: each workgroup takes kStartsGroup consecutive count
// workgroups, sums the totals of all count workgroups before them (a
// block-wide reduction, the totals being few: ~2,600 at config 1) and adds
// the running prefix to their rows.  The last workgroup writes starts[n]
// and *n_isects_out.  (One workgroup scanning the totals and a second pass
// adding them took 4.7 + 4.3 us at config 1.)
constexpr int kStartsGroup = 8;

__global__ void __launch_bounds__(kIsectThreads)
    isect_starts_scan_kernel(int64_t n, int64_t n_blocks,
                             const uint64_t *__restrict__ block_tot,
                             int64_t *__restrict__ starts,
                             int64_t *__restrict__ n_isects_out) {
    __shared__ uint64_t s_wave[kIsectThreads / kWave];
    __shared__ uint64_t s_grp[kStartsGroup];
    const int64_t b0 = (int64_t)blockIdx.x * kStartsGroup;
    // every load is issued before the reduction: the rows' own prefixes,
    // the group's totals and the totals before the group
    int64_t own[kStartsGroup];
#pragma unroll
    for (int k = 0; k < kStartsGroup; ++k) {
        const int64_t i = (b0 + k) * kIsectThreads + threadIdx.x;
        own[k] = i < n ? starts[i] : 0;
    }
    if (threadIdx.x < kStartsGroup)
        s_grp[threadIdx.x] =
            b0 + threadIdx.x < n_blocks ? block_tot[b0 + threadIdx.x] : 0ull;
    uint64_t sum = 0;
    for (int64_t b = threadIdx.x; b < b0; b += kIsectThreads)
        sum += block_tot[b];
    sum = wave_inclusive_scan_u64(sum);
    if (lane_id() == kWave - 1)
        s_wave[threadIdx.x / kWave] = sum;
    __syncthreads();
    uint64_t run = 0;
#pragma unroll
    for (int w = 0; w < kIsectThreads / kWave; ++w)
        run += s_wave[w];
#pragma unroll
    for (int k = 0; k < kStartsGroup; ++k) {
        const int64_t i = (b0 + k) * kIsectThreads + threadIdx.x;
        if (i < n)
            starts[i] = own[k] + (int64_t)run;
        run += s_grp[k];
    }
    if (threadIdx.x == 0 && b0 + kStartsGroup >= n_blocks) {
        starts[n] = (int64_t)run;
        *n_isects_out = (int64_t)run;
    }
}


// offsets[s] = the first slot whose image|tile key is that of tile slot s
// (image * n_tiles + tile), or n when none is.  Every slot boundary i in
// [0, n] fills the tile slots between the keys of slots i - 1 and i; a
// thread takes four consecutive boundaries with one 16-byte load of their
// keys (keys is 16-byte aligned and padded to a multiple of 4 entries).
// With n_dev the slot count is min(n, *n_dev).
constexpr int kBoundsPer = 4;

__global__ void tile_bounds_kernel(int64_t n, const int64_t *__restrict__ n_dev,
                                   const uint32_t *__restrict__ keys,
                                   int64_t n_slots, int32_t tile_n_bits,
                                   int32_t n_tiles, int32_t *__restrict__ offsets) {
    if (n_dev != nullptr)
        n = min(n, *n_dev);
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kBoundsPer;
    if (i0 > n)
        return;
    const uint32_t mask = (1u << tile_n_bits) - 1u;
    auto slot = [&](uint32_t k) {
        return (int64_t)(k >> tile_n_bits) * n_tiles + (int64_t)(k & mask);
    };
    uint32_t k[kBoundsPer + 1];  // keys of slots i0 - 1 .. i0 + 3
    k[0] = i0 > 0 ? keys[i0 - 1] : 0u;
    if (i0 < n) {
        const uint4 q = *reinterpret_cast<const uint4 *>(keys + i0);
        k[1] = q.x;
        k[2] = q.y;
        k[3] = q.z;
        k[4] = q.w;
    }
#pragma unroll
    for (int j = 0; j < kBoundsPer; ++j) {
        const int64_t i = i0 + j;
        if (i > n)
            break;
        const int64_t cur = i < n ? slot(k[j + 1]) : n_slots;
        const int64_t prev = i > 0 ? slot(k[j]) : -1;
        for (int64_t s = prev + 1; s <= cur && s < n_slots; ++s)
            offsets[s] = (int32_t)i;
    }
}

constexpr int kSegThreads = 256;  // a multiple of the 256 digits
constexpr int kSegWaves = kSegThreads / kWave;
constexpr int kSegDigitBits = 8;
constexpr int kSegRadix = 1 << kSegDigitBits;
constexpr int kSegPasses = 32 / kSegDigitBits;
// Tiles of up to CAP rows are sorted in LDS, larger ones through global
// scratch; the kernel comes in two LDS capacities (tile_depth_sort_kernel).
constexpr int kSegCapSmall = 2560;
constexpr int kSegCapLarge = 4096;

template <int MAXK>
struct SegSmem {
    uint32_t keys[MAXK];
    uint32_t vals[MAXK];
    uint32_t cnt[kSegWaves][kSegRadix];
    uint32_t off[kSegRadix];
    uint32_t wave[kSegWaves];
    uint32_t bits_or[kSegWaves];
    uint32_t bits_and[kSegWaves];
};

__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v |= (uint32_t)__shfl_xor((int)v, o);
    return v;
}
__device__ __forceinline__ uint32_t wave_and_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v &= (uint32_t)__shfl_xor((int)v, o);
    return v;
}

// The key bits that differ between the workgroup's keys (OR ^ AND of the
// per-thread partials); digits with none of them are constant and their
// passes leave the order unchanged.
template <class SM>
__device__ __forceinline__ uint32_t block_varying_bits(uint32_t o, uint32_t an,
                                                       SM &sm) {
    o = wave_or_u32(o);
    an = wave_and_u32(an);
    const int w = threadIdx.x / kWave;
    if (lane_id() == 0) {
        sm.bits_or[w] = o;
        sm.bits_and[w] = an;
    }
    __syncthreads();
    uint32_t bo = 0u, ba = ~0u;
#pragma unroll
    for (int ww = 0; ww < kSegWaves; ++ww) {
        bo |= sm.bits_or[ww];
        ba &= sm.bits_and[ww];
    }
    return bo ^ ba;
}

// Stable rank of a span of at most ITEMS * 64 keys per wave (k[j] of a lane
// at base + 64 j + lane, valid below S, the end of the wave's span) on the
// digit at `shift`: rank[j] is the number of earlier keys of the wave's
// span with the same digit, and sm.cnt[w][d] the span's count of digit d.
// Items past S are skipped as a whole.  (Comparing only the digit bits that
// vary over the tile takes fewer ballots, but its branches cost registers
// and occupancy: slower at config 1.)
template <int ITEMS, class SM>
__device__ __forceinline__ void seg_rank(const uint32_t (&k)[ITEMS], int base,
                                         int S, int shift, SM &sm,
                                         uint32_t (&rank)[ITEMS]) {
    const int w = threadIdx.x / kWave;
    const int lane = (int)lane_id();
    for (int i = threadIdx.x; i < kSegWaves * kSegRadix; i += kSegThreads)
        (&sm.cnt[0][0])[i] = 0u;
    __syncthreads();
    // items of this wave with at least one key below S (wave-uniform)
    const int live = S > base ? min(ITEMS, (S - base + kWave - 1) / kWave) : 0;
    uint32_t *cnt = sm.cnt[w];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        if (j < live) {
            const bool valid = base + j * kWave + lane < S;
            const uint32_t d = (k[j] >> shift) & (kSegRadix - 1);
            const uint64_t peers = match_digit(d, kSegDigitBits, wave_ballot(valid));
            const uint64_t before = peers & lanemask_lt();
            uint32_t r = 0;
            if (valid)
                r = cnt[d] + (uint32_t)__popcll(before);
            rank[j] = r;
            __builtin_amdgcn_wave_barrier();
            if (valid && before == 0)
                cnt[d] += (uint32_t)__popcll(peers);
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
}

// Keys per wave when S keys are split evenly over the workgroup's waves in
// whole 64-key items (the input order is wave, item, lane).
__device__ __forceinline__ int seg_span(int S) {
    return (S + kSegWaves * kWave - 1) / (kSegWaves * kWave) * kWave;
}

// LSD passes over the 8-bit digits of bits [lo_bit, hi_bit) of the keys k
// (wave w's items at base + 64 j + lane, valid below lim): each pass ranks
// stably, reorders the tile through LDS and reloads every thread's items, so
// after the last pass both the registers and sm.keys/sm.vals hold the order.
template <int ITEMS, int MAXK>
__device__ __forceinline__ void seg_lsd_passes(uint32_t (&k)[ITEMS],
                                               uint32_t (&v)[ITEMS], int base,
                                               int lim, int lo_bit, int hi_bit,
                                               SegSmem<MAXK> &sm) {
    const int tid = threadIdx.x;
    const int w = tid / kWave;
    const int lane = (int)lane_id();
    uint32_t rank[ITEMS];
    for (int shift = lo_bit; shift < hi_bit; shift += kSegDigitBits) {
        seg_rank<ITEMS>(k, base, lim, shift, sm, rank);
        {
            // digit starts, and each wave's start inside its digit (thread d
            // for digit d)
            const int d = tid;
            uint32_t c[kSegWaves], tot = 0u;
#pragma unroll
            for (int ww = 0; ww < kSegWaves; ++ww) {
                c[ww] = d < kSegRadix ? sm.cnt[ww][d] : 0u;
                tot += c[ww];
            }
            uint32_t total;
            uint32_t run = block_exclusive_u32<kSegThreads>(tot, sm.wave, &total);
            if (d < kSegRadix) {
#pragma unroll
                for (int ww = 0; ww < kSegWaves; ++ww) {
                    sm.cnt[ww][d] = run;
                    run += c[ww];
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const int i = base + j * kWave + lane;
            if (i < lim) {
                const uint32_t d = (k[j] >> shift) & (kSegRadix - 1);
                const uint32_t pos = sm.cnt[w][d] + rank[j];
                sm.keys[pos] = k[j];
                sm.vals[pos] = v[j];
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const int i = base + j * kWave + lane;
            if (i < lim) {
                k[j] = sm.keys[i];
                v[j] = sm.vals[i];
            }
        }
        __syncthreads();
    }
}

// Block-wide minimum and maximum of the threads' partials.
template <class SM>
__device__ __forceinline__ void block_min_max(uint32_t lo, uint32_t hi, SM &sm,
                                              uint32_t &kmin, uint32_t &kmax) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        lo = min(lo, (uint32_t)__shfl_xor((int)lo, o));
        hi = max(hi, (uint32_t)__shfl_xor((int)hi, o));
    }
    const int w = threadIdx.x / kWave;
    if (lane_id() == 0) {
        sm.bits_or[w] = lo;
        sm.bits_and[w] = hi;
    }
    __syncthreads();
    kmin = ~0u;
    kmax = 0u;
#pragma unroll
    for (int ww = 0; ww < kSegWaves; ++ww) {
        kmin = min(kmin, sm.bits_or[ww]);
        kmax = max(kmax, sm.bits_and[ww]);
    }
}

// Key bits the LDS sort ranks by radix passes: the top kSegCoarseBits bits
// of the tile's key range (two passes); runs of keys equal in those bits are
// then put in order by transposition, stably, within 2 kSegRunMax phases
// (else passes over every bit of the range follow).
constexpr int kSegCoarseBits = 16;
constexpr int kSegRunMax = 32;

// Tile of S <= 64 * ITEMS * kSegWaves rows, sorted in LDS.  The keys are
// ranked relative to the tile's smallest key, on the top bits of the range
// first: a stable sort on k >> c (the passes) followed by a stable sort of
// every run of equal k >> c (transposition) is the stable sort on k, since
// k >> c is monotone in k.  A tile whose runs are not sorted within the
// phase limit is sorted again by passes over all bits of k, starting from
// the order reached; that order keeps equal keys in input order (their
// coarse keys are equal too, and transposition never swaps them), so the
// result is the same stable sort.
template <int ITEMS, int MAXK>
__device__ void seg_sort_lds(int S, const uint32_t *__restrict__ rows_in,
                             const uint32_t *__restrict__ depth_bits,
                             uint64_t key_hi, int64_t *__restrict__ out_ids,
                             int32_t *__restrict__ out_rows, SegSmem<MAXK> &sm) {
    static_assert(ITEMS * kWave * kSegWaves <= MAXK, "tile exceeds LDS");
    const int tid = threadIdx.x;
    const int w = tid / kWave;
    const int lane = (int)lane_id();
    // the tile split evenly over the waves, in whole items: wave w holds
    // [base, lim) = [w * span, (w + 1) * span) cut at S
    const int span = seg_span(S);
    const int base = w * span;
    const int lim = min(S, base + span);
    uint32_t k[ITEMS], v[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int i = base + j * kWave + lane;
        v[j] = i < lim ? rows_in[i] : 0u;
    }
    uint32_t lo = ~0u, hi = 0u;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int i = base + j * kWave + lane;
        k[j] = i < lim ? depth_bits[v[j]] : 0u;
        if (i < lim) {
            lo = min(lo, k[j]);
            hi = max(hi, k[j]);
        }
    }
    uint32_t kmin, kmax;
    block_min_max(lo, hi, sm, kmin, kmax);
    const uint32_t range = kmax - kmin;
    const int bits = range != 0u ? 32 - __clz((int)range) : 0;
    const int coarse = bits > kSegCoarseBits ? bits - kSegCoarseBits : 0;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j)
        k[j] -= kmin;
    // one round of passes over the coarse bits, and a second over all bits
    // only if a run is too long (a single call site keeps one copy of the
    // unrolled passes)
    for (int lo_bit = coarse;;) {
        seg_lsd_passes<ITEMS>(k, v, base, lim, lo_bit, bits, sm);
        if (lo_bit == 0)
            break;
        // runs of equal coarse key (the passes left the order in LDS), put
        // in order by odd-even transposition: each phase compares the
        // disjoint pairs (i, i + 1) of one parity and swaps those with equal
        // coarse keys out of order (equal keys never move, so the result is
        // stable).  A full round (both parities) without a swap leaves every
        // run sorted; a run of L keys needs at most L phases, and a tile
        // still swapping after 2 kSegRunMax phases takes the full passes.
        bool long_run = false;
        constexpr int PAIRS = (ITEMS + 1) / 2;  // pairs per thread and phase
        for (int ph = 0, quiet = 0;; ++ph) {
            const int par = ph & 1;
            bool swapped = false;
#pragma unroll
            for (int r = 0; r < PAIRS; ++r) {
                const int i = 2 * (tid + r * kSegThreads) + par;
                if (i + 1 < S) {
                    const uint32_t ka = sm.keys[i], kb = sm.keys[i + 1];
                    if ((ka >> lo_bit) == (kb >> lo_bit) && ka > kb) {
                        const uint32_t va = sm.vals[i], vb = sm.vals[i + 1];
                        sm.keys[i] = kb;
                        sm.keys[i + 1] = ka;
                        sm.vals[i] = vb;
                        sm.vals[i + 1] = va;
                        swapped = true;
                    }
                }
            }
            quiet = __syncthreads_or(swapped) ? 0 : quiet + 1;
            if (quiet == 2)
                break;
            if (ph >= 2 * kSegRunMax) {
                long_run = true;
                break;
            }
        }
        // long_run is the same in every thread (set from a block-wide vote)
        const bool any_long = long_run;
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const int i = base + j * kWave + lane;
            if (i < lim) {
                k[j] = sm.keys[i];
                v[j] = sm.vals[i];
            }
        }
        if (!any_long)
            break;
        __syncthreads();
        lo_bit = 0;
    }
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int i = base + j * kWave + lane;
        if (i < lim) {
            out_ids[i] = (int64_t)(key_hi | (k[j] + kmin));
            out_rows[i] = (int32_t)v[j];
        }
    }
}

// Tile of more than CAP rows: LSD passes through global scratch, one
// chunk of CAP keys after another, each chunk ranked in LDS and
// written at the running digit offsets (stable: chunks in order, ranks
// stable inside each).  Scratch pairs: p1 (own keys and values) and p2
// (keys then values in the tile's 8-byte id range, free until the final
// write); the prologue writes the pair that leaves the result in p1 after
// the passes.
template <int CAP>
__device__ void seg_sort_global(int64_t S, const uint32_t *__restrict__ rows_in,
                                const uint32_t *__restrict__ depth_bits,
                                uint64_t key_hi, uint32_t *__restrict__ p1k,
                                uint32_t *__restrict__ p1v,
                                int64_t *__restrict__ out_ids,
                                int32_t *__restrict__ out_rows,
                                SegSmem<CAP> &sm) {
    constexpr int ITEMS = CAP / kSegThreads;
    const int tid = threadIdx.x;
    const int w = tid / kWave;
    const int lane = (int)lane_id();
    uint32_t *p2k = reinterpret_cast<uint32_t *>(out_ids);
    uint32_t *p2v = p2k + S;
    uint32_t o = 0u, an = ~0u;
    for (int64_t i = tid; i < S; i += kSegThreads) {
        const uint32_t key = depth_bits[rows_in[i]];
        o |= key;
        an &= key;
    }
    const uint32_t varying = block_varying_bits(o, an, sm);
    int npass = 0;
    for (int p = 0; p < kSegPasses; ++p)
        npass += ((varying >> (p * kSegDigitBits)) & (kSegRadix - 1)) != 0u;
    uint32_t *sk = (npass & 1) ? p2k : p1k;
    uint32_t *sv = (npass & 1) ? p2v : p1v;
    uint32_t *dk = (npass & 1) ? p1k : p2k;
    uint32_t *dv = (npass & 1) ? p1v : p2v;
    for (int64_t i = tid; i < S; i += kSegThreads) {
        const uint32_t r = rows_in[i];
        sk[i] = depth_bits[r];
        sv[i] = r;
    }
    __threadfence_block();
    __syncthreads();
    for (int p = 0; p < kSegPasses; ++p) {
        const int shift = p * kSegDigitBits;
        if (((varying >> shift) & (kSegRadix - 1)) == 0u)
            continue;
        // digit totals over the tile -> running start of every digit
        for (int i = tid; i < kSegRadix; i += kSegThreads)
            sm.cnt[0][i] = 0u;
        __syncthreads();
        for (int64_t i = tid; i < S; i += kSegThreads)
            atomicAdd(&sm.cnt[0][(sk[i] >> shift) & (kSegRadix - 1)], 1u);
        __syncthreads();
        {
            uint32_t total;
            const uint32_t o = block_exclusive_u32<kSegThreads>(
                tid < kSegRadix ? sm.cnt[0][tid] : 0u, sm.wave, &total);
            if (tid < kSegRadix)
                sm.off[tid] = o;
        }
        __syncthreads();
        for (int64_t c0 = 0; c0 < S; c0 += CAP) {
            const int cs = (int)(S - c0 < CAP ? S - c0 : CAP);
            const int span = seg_span(cs);
            const int base = w * span;
            const int lim = min(cs, base + span);
            uint32_t k[ITEMS], v[ITEMS], rank[ITEMS];
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                const int i = base + j * kWave + lane;
                k[j] = i < lim ? sk[c0 + i] : 0u;
                v[j] = i < lim ? sv[c0 + i] : 0u;
            }
            seg_rank<ITEMS>(k, base, lim, shift, sm, rank);
            if (tid < kSegRadix) {
                const int d = tid;
                uint32_t run = sm.off[d];
#pragma unroll
                for (int ww = 0; ww < kSegWaves; ++ww) {
                    const uint32_t c = sm.cnt[ww][d];
                    sm.cnt[ww][d] = run;
                    run += c;
                }
                sm.off[d] = run;
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                const int i = base + j * kWave + lane;
                if (i < lim) {
                    const uint32_t d = (k[j] >> shift) & (kSegRadix - 1);
                    const uint32_t pos = sm.cnt[w][d] + rank[j];
                    dk[pos] = k[j];
                    dv[pos] = v[j];
                }
            }
            __syncthreads();
        }
        __threadfence_block();
        __syncthreads();
        uint32_t *t = sk; sk = dk; dk = t;
        t = sv; sv = dv; dv = t;
    }
    // the result is in p1 (sk == p1k), apart from the ids it is written over
    for (int64_t i = tid; i < S; i += kSegThreads) {
        const uint32_t key = sk[i];
        const uint32_t r = sv[i];
        out_ids[i] = (int64_t)(key_hi | key);
        out_rows[i] = (int32_t)r;
    }
}

// The tile slot's range [start, start + S) and its 64-bit key prefix.
struct SegTile {
    int64_t start, S;
    uint64_t key_hi;
};

__device__ __forceinline__ SegTile seg_tile(int64_t s, int64_t n,
                                            const int32_t *__restrict__ offsets,
                                            int64_t n_slots, int32_t tile_n_bits,
                                            int32_t n_tiles) {
    SegTile t;
    t.start = offsets[s];
    const int64_t end = s + 1 < n_slots ? (int64_t)offsets[s + 1] : n;
    t.S = end - t.start;
    const uint32_t key = (uint32_t)((s / n_tiles) << tile_n_bits) |
                         (uint32_t)(s % n_tiles);
    t.key_hi = (uint64_t)key << 32;
    return t;
}

// One workgroup per tile slot (image * n_tiles + tile): the tile's rows,
// grouped by the tile sort in row order, sorted stably on their depth bits.
// rows_in may be out_rows itself (each workgroup reads its range before it
// writes it); p1k/p1v is scratch of at least n entries each.  Tiles of all
// sizes share one launch: a separate launch for the few large tiles (after
// the small ones) put their whole sort on the critical path (25 us at
// config 1 for ~50 tiles of 2,049-2,406 rows).  The LDS holds CAP rows:
// 2,560 (25 KB, six workgroups per CU) where tiles average up to
// kSegDeepMean rows, else 4,096 (38 KB, four per CU).  At config 1 (1,158
// rows a tile on average, 2,406 at most) 2,560 takes 51.7 us against
// 54.5 us for 3,072 (five per CU), 4,096 took 62.5 us and 2,048 (seven per
// CU, the ~50 larger tiles through global scratch) 92 us; at config 4
// (1,874 on average, 729 tiles of 3,073-3,802 rows) 3,072 sent a fifth of
// the rows through global scratch.
template <int CAP>
__global__ void __launch_bounds__(kSegThreads)
    tile_depth_sort_kernel(int64_t n, const int64_t *__restrict__ n_dev,
                           const int32_t *__restrict__ offsets, int64_t n_slots,
                           int32_t tile_n_bits, int32_t n_tiles,
                           const uint32_t *__restrict__ depth_bits,
                           const uint32_t *rows_in, uint32_t *__restrict__ p1k,
                           uint32_t *__restrict__ p1v,
                           int64_t *__restrict__ isect_ids, int32_t *out_rows) {
    __shared__ SegSmem<CAP> sm;
    if (n_dev != nullptr)
        n = min(n, *n_dev);
    const int64_t s = blockIdx.x;
    const SegTile t = seg_tile(s, n, offsets, n_slots, tile_n_bits, n_tiles);
    if (t.S <= 0)
        return;
    const uint32_t *rin = rows_in + t.start;
    int64_t *oid = isect_ids + t.start;
    int32_t *orow = out_rows + t.start;
    // keys per thread: a tile of S rows needs S <= ITEMS * kSegThreads
    constexpr int I = CAP / kSegThreads;  // items per thread at CAP
    static_assert(I * kSegThreads == CAP && I >= 8, "LDS tile size");
    if (t.S <= (I / 8) * kSegThreads)
        seg_sort_lds<I / 8>((int)t.S, rin, depth_bits, t.key_hi, oid, orow, sm);
    else if (t.S <= (I / 4) * kSegThreads)
        seg_sort_lds<I / 4>((int)t.S, rin, depth_bits, t.key_hi, oid, orow, sm);
    else if (t.S <= (I / 2) * kSegThreads)
        seg_sort_lds<I / 2>((int)t.S, rin, depth_bits, t.key_hi, oid, orow, sm);
    else if (t.S <= CAP)
        seg_sort_lds<I>((int)t.S, rin, depth_bits, t.key_hi, oid, orow, sm);
    else
        seg_sort_global<CAP>(t.S, rin, depth_bits, t.key_hi, p1k + t.start,
                             p1v + t.start, oid, orow, sm);
}

// Mean rows per tile above which the depth sort takes the 4,096-row LDS.
constexpr int64_t kSegDeepMean = 1500;

struct PrepLayout {
    size_t keys_a, keys_b, vals_b, lookback, sort_ws, total;
};

// Depth keys are all 32 float bits of the depth, as unsigned integers: the
// reference zero-extends them into the low word of the 64-bit id
// (IntersectTile.cu:190-192), so a negative depth orders after every
// positive one.
constexpr int kDepthKeyBits = 32;

inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }

PrepLayout prep_layout(int64_t n) {
    PrepLayout L;
    const size_t v = align256((size_t)n * 4);
    L.keys_a = 0;
    L.keys_b = v;
    L.vals_b = 2 * v;
    L.lookback = 3 * v;
    L.sort_ws = L.lookback + align256(lookback_bytes(ceil_div(n, kScanBlockRows)));
    L.total = L.sort_ws + radix_sort_workspace_bytes(n);
    return L;
}

struct EmitLayout {
    size_t keys_a, keys_b, vals, chunks, sort_ws, total;
};

EmitLayout emit_layout(int64_t n_isects) {
    EmitLayout L;
    const size_t v = align256((size_t)n_isects * 4);
    L.keys_a = 0;
    L.keys_b = v;
    L.vals = 2 * v;
    L.chunks = 3 * v;
    L.sort_ws = L.chunks + align256((size_t)ceil_div(n_isects, kEmitSlots) * 4);
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
                                    int32_t *tiles_per_gauss, int32_t *depth_order,
                                    int64_t *depth_starts, float *row_records,
                                    int64_t *n_isects_out, gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, 0, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && tiles_per_gauss && depth_order && depth_starts &&
                   row_records && n_isects_out,
               "isect_prepare: NULL buffer");
    GS_REQUIRE(reinterpret_cast<uintptr_t>(row_records) % 16 == 0,
               "isect_prepare: row_records must be 16-byte aligned");
    GS_REQUIRE(n < (1ll << 31), "isect_prepare: more than 2^31 rows");
    const PrepLayout L = prep_layout(n);
    GS_REQUIRE(workspace && workspace_bytes >= L.total,
               "isect_prepare: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    uint32_t *keys_a = reinterpret_cast<uint32_t *>(ws + L.keys_a);
    uint32_t *keys_b = reinterpret_cast<uint32_t *>(ws + L.keys_b);
    uint32_t *vals_a = reinterpret_cast<uint32_t *>(depth_order);
    uint32_t *vals_b = reinterpret_cast<uint32_t *>(ws + L.vals_b);
    hipStream_t st = as_stream(stream);
    const unsigned grid = (unsigned)ceil_div(n, kIsectThreads);
    isect_count_keys_kernel<<<grid, kIsectThreads, 0, st>>>(
        a, tiles_per_gauss, keys_a, vals_a, reinterpret_cast<RowRec *>(row_records));
    GS_TRY(check_launch("isect_count_keys_kernel"));
    bool in_b = false;
    GS_TRY(radix_sort_u32(n, kDepthKeyBits, keys_a, vals_a, keys_b, vals_b,
                          ws + L.sort_ws, workspace_bytes - L.sort_ws, st, &in_b,
                          nullptr, nullptr));
    if (in_b)
        GS_TRY(copy_u32(n, vals_b, vals_a, st));
    const int64_t scan_blocks = ceil_div(n, kScanBlockRows);
    GS_TRY(clear_lookback(ws + L.lookback, scan_blocks, st));
    depth_order_starts_kernel<<<(unsigned)scan_blocks, kIsectThreads, 0, st>>>(
        n, vals_a, tiles_per_gauss, lookback_from(ws + L.lookback), depth_starts,
        n_isects_out);
    return check_launch("depth_order_starts_kernel");
}

extern "C" size_t gsplat_isect_emit_sorted_workspace_size(int64_t n_isects) {
    return emit_layout(n_isects > 0 ? n_isects : 0).total;
}

static int emit_sorted_impl(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *depth_order,
    const int64_t *depth_starts, const float *row_records, int64_t n_isects,
    const int64_t *n_dev, void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    gsplat_stream_t stream) {
    IsectArgs a;
    GS_TRY(make_args(n, N, I, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    GS_REQUIRE(n_isects >= 0, "isect_emit_sorted: negative n_isects");
    if (n == 0 || n_isects == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && depth_order && depth_starts && row_records && isect_ids &&
                   flatten_ids,
               "isect_emit_sorted: NULL buffer");
    GS_REQUIRE(reinterpret_cast<uintptr_t>(row_records) % 16 == 0,
               "isect_emit_sorted: row_records must be 16-byte aligned");
    GS_REQUIRE(I > 0, "isect_emit_sorted: I must be positive");
    const int ib = bit_length(I);
    GS_REQUIRE(ib + a.tile_n_bits <= 32,
               "isect_emit_sorted: image and tile ids need more than 32 bits");
    GS_REQUIRE(n_isects < (1ll << 31), "isect_emit_sorted: more than 2^31 isects");
    const EmitLayout L = emit_layout(n_isects);
    GS_REQUIRE(workspace && workspace_bytes >= L.total,
               "isect_emit_sorted: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    // The emission writes 32-bit (image | tile) keys in depth order; a
    // stable sort on those bits alone then gives the reference's order, and
    // its last pass writes the 64-bit isect ids (key << 32 | depth bits of
    // the row) and the rows straight into the outputs.
    const int key_bits = a.tile_n_bits + ib;
    const int passes = radix_sort_passes(key_bits);
    uint32_t *ka = reinterpret_cast<uint32_t *>(ws + L.keys_a);
    uint32_t *kb = reinterpret_cast<uint32_t *>(ws + L.keys_b);
    uint32_t *tmp_vals = reinterpret_cast<uint32_t *>(ws + L.vals);
    uint32_t *out_vals = reinterpret_cast<uint32_t *>(flatten_ids);
    // the passes alternate a -> b -> a ...: emit into the pair whose
    // partner (odd pass count) or itself (even) receives the last pass
    uint32_t *va = passes % 2 == 1 ? tmp_vals : out_vals;
    uint32_t *vb = passes % 2 == 1 ? out_vals : tmp_vals;
    hipStream_t st = as_stream(stream);
    int32_t *chunk_first = reinterpret_cast<int32_t *>(ws + L.chunks);
    size_t z_off;
    int64_t z_words;
    radix_sort_first_counts(n_isects, &z_off, &z_words);
    emit_chunk_first_kernel<<<(unsigned)ceil_div(n, kIsectThreads), kIsectThreads,
                              0, st>>>(n, depth_starts, n_isects, chunk_first,
                                       reinterpret_cast<uint32_t *>(ws + L.sort_ws + z_off),
                                       z_words);
    GS_TRY(check_launch("emit_chunk_first_kernel"));
    const int64_t chunks = ceil_div(n_isects, kEmitSlots);
    isect_emit_depth_kernel<<<(unsigned)ceil_div(chunks, kEmitWaves),
                              kIsectThreads, 0, st>>>(
        a, reinterpret_cast<const uint32_t *>(depth_order), depth_starts,
        reinterpret_cast<const RowRec *>(row_records), chunk_first, n_isects,
        n_dev, ka, va);
    GS_TRY(check_launch("isect_emit_depth_kernel"));
    bool in_b = false;
    GS_TRY(radix_sort_u32(n_isects, key_bits, ka, va, kb, vb, ws + L.sort_ws,
                          workspace_bytes - L.sort_ws, st, &in_b,
                          reinterpret_cast<const uint32_t *>(depths),
                          reinterpret_cast<uint64_t *>(isect_ids), n_dev, true));
    GS_REQUIRE((in_b ? vb : va) == out_vals, "isect_emit_sorted: pass parity");
    return GSPLAT_OK;
}

extern "C" int gsplat_isect_emit_sorted(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *depth_order,
    const int64_t *depth_starts, const float *row_records, int64_t n_isects,
    void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    gsplat_stream_t stream) {
    clear_error();
    return emit_sorted_impl(n, N, I, image_ids, means2d, radii, depths, conics,
                            opacities, tile_size, tile_width, tile_height,
                            depth_order, depth_starts, row_records, n_isects,
                            nullptr, workspace, workspace_bytes, isect_ids,
                            flatten_ids, stream);
}

extern "C" int gsplat_isect_emit_sorted_dev(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int32_t *depth_order,
    const int64_t *depth_starts, const float *row_records, int64_t capacity,
    void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(depth_starts != nullptr, "isect_emit_sorted_dev: NULL depth_starts");
    // the intersection count is depth_starts[n], read by the kernels
    return emit_sorted_impl(n, N, I, image_ids, means2d, radii, depths, conics,
                            opacities, tile_size, tile_width, tile_height,
                            depth_order, depth_starts, row_records, capacity,
                            depth_starts + n, workspace, workspace_bytes,
                            isect_ids, flatten_ids, stream);
}

// ---------------------------------------------------------------------------
// Tile-first sorted intersection (the kernels above, from
// isect_count_rows_kernel to tile_depth_sort_kernel).
// ---------------------------------------------------------------------------
extern "C" size_t gsplat_isect_prepare_rows_workspace_size(int64_t n) {
    // per-workgroup totals
    return align256((size_t)ceil_div(n > 0 ? n : 0, kIsectThreads) * 8);
}

extern "C" int gsplat_isect_prepare_rows(int64_t n, int64_t N, const int64_t *image_ids,
                                         const float *means2d, const int32_t *radii,
                                         const float *depths, const float *conics,
                                         const float *opacities, int32_t tile_size,
                                         int32_t tile_width, int32_t tile_height,
                                         void *workspace, size_t workspace_bytes,
                                         int32_t *tiles_per_gauss, int64_t *row_starts,
                                         float *row_records, int64_t *n_isects_out,
                                         gsplat_stream_t stream) {
    clear_error();
    IsectArgs a;
    GS_TRY(make_args(n, N, 0, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(depths && tiles_per_gauss && row_starts && row_records && n_isects_out,
               "isect_prepare_rows: NULL buffer");
    GS_REQUIRE(reinterpret_cast<uintptr_t>(row_records) % 16 == 0,
               "isect_prepare_rows: row_records must be 16-byte aligned");
    GS_REQUIRE(n < (1ll << 31), "isect_prepare_rows: more than 2^31 rows");
    const int64_t blocks = ceil_div(n, kIsectThreads);
    GS_REQUIRE(workspace && workspace_bytes >= gsplat_isect_prepare_rows_workspace_size(n),
               "isect_prepare_rows: workspace too small");
    uint64_t *block_tot = reinterpret_cast<uint64_t *>(workspace);
    hipStream_t st = as_stream(stream);
    isect_count_rows_kernel<<<(unsigned)blocks, kIsectThreads, 0, st>>>(
        a, tiles_per_gauss, reinterpret_cast<RowRec *>(row_records), row_starts,
        block_tot);
    GS_TRY(check_launch("isect_count_rows_kernel"));
    isect_starts_scan_kernel<<<(unsigned)ceil_div(blocks, kStartsGroup), kIsectThreads,
                               0, st>>>(n, blocks, block_tot, row_starts, n_isects_out);
    return check_launch("isect_starts_scan_kernel");
}

extern "C" int gsplat_sh_rows_fwd_isect_count(
    int64_t B, int64_t C, int64_t N, int32_t K, int32_t degree, const float *means,
    const float *viewmats, const float *coeffs, const int32_t *row_of, float *colors,
    int64_t n_cap, const int32_t *n_dev, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, void *workspace, size_t workspace_bytes,
    int32_t *tiles_per_gauss, int64_t *row_starts, float *row_records,
    gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0 && K > 0, "sh_rows_fwd_isect_count: bad sizes");
    GS_REQUIRE(degree >= 0 && degree <= 4, "sh_rows_fwd_isect_count: degree must be in [0, 4]");
    GS_REQUIRE((degree + 1) * (degree + 1) <= K,
               "sh_rows_fwd_isect_count: K too small for the degree");
    GS_REQUIRE(n_cap >= 0 && n_cap <= B * C * N,
               "sh_rows_fwd_isect_count: n_cap must be at most B*C*N");
    IsectArgs ia;
    // image of a row: image_ids[row] with several images, else row / n_cap (0)
    GS_TRY(make_args(n_cap, image_ids ? 0 : (n_cap > 0 ? n_cap : 1), 0, image_ids,
                     means2d, radii, depths, conics, opacities, tile_size, tile_width,
                     tile_height, ia));
    if (B * N == 0 || C == 0)
        return GSPLAT_OK;
    GS_REQUIRE(means && viewmats && coeffs && row_of && colors && n_dev,
               "sh_rows_fwd_isect_count: NULL buffer");
    GS_REQUIRE(depths && conics && opacities && tiles_per_gauss && row_starts && row_records,
               "sh_rows_fwd_isect_count: NULL buffer");
    GS_REQUIRE(reinterpret_cast<uintptr_t>(row_records) % 16 == 0,
               "sh_rows_fwd_isect_count: row_records must be 16-byte aligned");
    GS_REQUIRE(n_cap < (1ll << 31), "sh_rows_fwd_isect_count: more than 2^31 rows");
    GS_REQUIRE(workspace &&
                   workspace_bytes >= gsplat_isect_prepare_rows_workspace_size(n_cap),
               "sh_rows_fwd_isect_count: workspace too small");
    const int nb = (degree + 1) * (degree + 1);
    ShRowsArgs sa{B, C, N, K, means, viewmats, coeffs, row_of,
                  (K == nb) && aligned16(coeffs)};
    const int64_t grid = std::max(ceil_div(B * N, (int64_t)kShThreads),
                                  ceil_div(n_cap, (int64_t)kIsectThreads));
    uint64_t *block_tot = reinterpret_cast<uint64_t *>(workspace);
    RowRec *recs = reinterpret_cast<RowRec *>(row_records);
    hipStream_t st = as_stream(stream);
#define GS_SHC(DEG)                                                            \
    sh_rows_count_kernel<DEG><<<(unsigned)grid, kIsectThreads, 0, st>>>(       \
        sa, colors, ia, n_dev, tiles_per_gauss, recs, row_starts, block_tot)
    switch (degree) {
    case 0: GS_SHC(0); break;
    case 1: GS_SHC(1); break;
    case 2: GS_SHC(2); break;
    case 3: GS_SHC(3); break;
    default: GS_SHC(4); break;
    }
#undef GS_SHC
    return check_launch("sh_rows_count_kernel");
}

extern "C" int gsplat_isect_row_starts(int64_t n, const void *workspace,
                                       size_t workspace_bytes, int64_t *row_starts,
                                       int64_t *n_isects_out, gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(n > 0 && n < (1ll << 31), "isect_row_starts: n must be in [1, 2^31)");
    GS_REQUIRE(row_starts && n_isects_out, "isect_row_starts: NULL buffer");
    GS_REQUIRE(workspace && workspace_bytes >= gsplat_isect_prepare_rows_workspace_size(n),
               "isect_row_starts: workspace too small");
    const int64_t blocks = ceil_div(n, (int64_t)kIsectThreads);
    isect_starts_scan_kernel<<<(unsigned)ceil_div(blocks, kStartsGroup), kIsectThreads,
                               0, as_stream(stream)>>>(
        n, blocks, reinterpret_cast<const uint64_t *>(workspace), row_starts, n_isects_out);
    return check_launch("isect_starts_scan_kernel");
}

extern "C" size_t gsplat_isect_emit_tiles_workspace_size(int64_t n_isects) {
    return emit_layout(n_isects > 0 ? n_isects : 0).total;
}

static int emit_tiles_impl(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int64_t *row_starts,
    const float *row_records, int64_t n_isects, const int64_t *n_dev,
    void *workspace, size_t workspace_bytes, int64_t *isect_ids,
    int32_t *flatten_ids, int32_t *offsets, gsplat_stream_t stream) {
    IsectArgs a;
    GS_TRY(make_args(n, N, I, image_ids, means2d, radii, depths, conics,
                     opacities, tile_size, tile_width, tile_height, a));
    GS_REQUIRE(n_isects >= 0, "isect_emit_tiles: negative n_isects");
    GS_REQUIRE(I > 0, "isect_emit_tiles: I must be positive");
    GS_REQUIRE(offsets != nullptr, "isect_emit_tiles: NULL offsets");
    const int64_t n_tiles = (int64_t)tile_width * tile_height;
    const int64_t n_slots = I * n_tiles;
    GS_REQUIRE(n_slots < (1ll << 31), "isect_emit_tiles: more than 2^31 tiles");
    const int ib = bit_length(I);
    GS_REQUIRE(ib + a.tile_n_bits <= 32,
               "isect_emit_tiles: image and tile ids need more than 32 bits");
    hipStream_t st = as_stream(stream);
    if (n == 0 || n_isects == 0) {
        fill_i32_kernel<<<(unsigned)ceil_div(n_slots, 256), 256, 0, st>>>(
            offsets, n_slots, 0);
        return check_launch("fill_i32_kernel");
    }
    GS_REQUIRE(depths && row_starts && row_records && isect_ids && flatten_ids,
               "isect_emit_tiles: NULL buffer");
    GS_REQUIRE(reinterpret_cast<uintptr_t>(row_records) % 16 == 0,
               "isect_emit_tiles: row_records must be 16-byte aligned");
    GS_REQUIRE(n_isects < (1ll << 31), "isect_emit_tiles: more than 2^31 isects");
    const EmitLayout L = emit_layout(n_isects);
    GS_REQUIRE(workspace && workspace_bytes >= L.total,
               "isect_emit_tiles: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    const int key_bits = a.tile_n_bits + ib;
    const int passes = radix_sort_passes(key_bits);
    uint32_t *ka = reinterpret_cast<uint32_t *>(ws + L.keys_a);
    uint32_t *kb = reinterpret_cast<uint32_t *>(ws + L.keys_b);
    uint32_t *tmp_vals = reinterpret_cast<uint32_t *>(ws + L.vals);
    uint32_t *out_vals = reinterpret_cast<uint32_t *>(flatten_ids);
    // the tile sort leaves the rows in flatten_ids (emit into the pair that
    // the last pass writes out of), where the depth sort reorders them
    uint32_t *va = passes % 2 == 1 ? tmp_vals : out_vals;
    uint32_t *vb = passes % 2 == 1 ? out_vals : tmp_vals;
    int32_t *chunk_first = reinterpret_cast<int32_t *>(ws + L.chunks);
    size_t z_off;
    int64_t z_words;
    radix_sort_first_counts(n_isects, &z_off, &z_words);
    emit_chunk_first_kernel<<<(unsigned)ceil_div(n, kIsectThreads), kIsectThreads,
                              0, st>>>(n, row_starts, n_isects, chunk_first,
                                       reinterpret_cast<uint32_t *>(ws + L.sort_ws + z_off),
                                       z_words);
    GS_TRY(check_launch("emit_chunk_first_kernel"));
    const int64_t chunks = ceil_div(n_isects, kEmitSlots);
    isect_emit_depth_kernel<<<(unsigned)ceil_div(chunks, kEmitWaves),
                              kIsectThreads, 0, st>>>(
        a, nullptr, row_starts, reinterpret_cast<const RowRec *>(row_records),
        chunk_first, n_isects, n_dev, ka, va);
    GS_TRY(check_launch("isect_emit_depth_kernel"));
    bool in_b = false;
    GS_TRY(radix_sort_u32(n_isects, key_bits, ka, va, kb, vb, ws + L.sort_ws,
                          workspace_bytes - L.sort_ws, st, &in_b, nullptr, nullptr,
                          n_dev, true));
    GS_REQUIRE((in_b ? vb : va) == out_vals, "isect_emit_tiles: pass parity");
    const uint32_t *sorted_keys = in_b ? kb : ka;
    uint32_t *free_keys = in_b ? ka : kb;
    tile_bounds_kernel<<<(unsigned)ceil_div(n_isects + 1, 256 * kBoundsPer), 256, 0, st>>>(
        n_isects, n_dev, sorted_keys, n_slots, a.tile_n_bits, (int32_t)n_tiles,
        offsets);
    GS_TRY(check_launch("tile_bounds_kernel"));
    // n_isects is the count or, with n_dev, the capacity sized from the
    // previous call's count: either way the mean tile depth of this scene
    if (n_isects > kSegDeepMean * n_slots)
        tile_depth_sort_kernel<kSegCapLarge><<<(unsigned)n_slots, kSegThreads, 0, st>>>(
            n_isects, n_dev, offsets, n_slots, a.tile_n_bits, (int32_t)n_tiles,
            reinterpret_cast<const uint32_t *>(depths), out_vals, free_keys, tmp_vals,
            isect_ids, flatten_ids);
    else
        tile_depth_sort_kernel<kSegCapSmall><<<(unsigned)n_slots, kSegThreads, 0, st>>>(
            n_isects, n_dev, offsets, n_slots, a.tile_n_bits, (int32_t)n_tiles,
            reinterpret_cast<const uint32_t *>(depths), out_vals, free_keys, tmp_vals,
            isect_ids, flatten_ids);
    return check_launch("tile_depth_sort_kernel");
}

extern "C" int gsplat_isect_emit_tiles(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int64_t *row_starts,
    const float *row_records, int64_t n_isects, void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    int32_t *offsets, gsplat_stream_t stream) {
    clear_error();
    return emit_tiles_impl(n, N, I, image_ids, means2d, radii, depths, conics,
                           opacities, tile_size, tile_width, tile_height, row_starts,
                           row_records, n_isects, nullptr, workspace, workspace_bytes,
                           isect_ids, flatten_ids, offsets, stream);
}

extern "C" int gsplat_isect_emit_tiles_dev(
    int64_t n, int64_t N, int64_t I, const int64_t *image_ids,
    const float *means2d, const int32_t *radii, const float *depths,
    const float *conics, const float *opacities, int32_t tile_size,
    int32_t tile_width, int32_t tile_height, const int64_t *row_starts,
    const float *row_records, int64_t capacity, void *workspace,
    size_t workspace_bytes, int64_t *isect_ids, int32_t *flatten_ids,
    int32_t *offsets, gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(row_starts != nullptr, "isect_emit_tiles_dev: NULL row_starts");
    // the intersection count is row_starts[n], read by the kernels
    return emit_tiles_impl(n, N, I, image_ids, means2d, radii, depths, conics,
                           opacities, tile_size, tile_width, tile_height, row_starts,
                           row_records, capacity, row_starts + n, workspace,
                           workspace_bytes, isect_ids, flatten_ids, offsets, stream);
}
