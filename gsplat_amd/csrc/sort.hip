// Stable LSD radix sort of (uint64 or uint32 key, uint32 value) pairs and a
// device-wide exclusive scan, both hand-written for wave64.
//
// Replaces cub::DeviceRadixSort::SortPairs as used by radix_sort_double_buffer
// (gsplat/cuda/csrc/IntersectTile.cu:478-520): keys are sorted on a bit range,
// ties keep their input order.
//
// Per pass (digit of up to 8 bits, 1024-key tiles up to 2M keys, 4096-key
// tiles above, so that a large sort's scatter fits one round of resident
// workgroups), two launches:
//   1. radix_hist_kernel    digit counts per tile with LDS atomics, written
//                           tile-major (coalesced), and added to the counts
//                           of the tile's group (about sqrt(tiles) tiles,
//                           one global atomic per digit and tile);
//   2. radix_scatter_kernel forms its tile's prefix of every digit from the
//                           counts of the groups before it and of the tiles
//                           before it in its own group (about 2 sqrt(tiles)
//                           loads per digit), ranks every key stably inside
//                           its tile (wave64 match ballots, order wave, item,
//                           lane), reorders the tile by digit in LDS, and
//                           writes each digit run with consecutive threads on
//                           consecutive addresses.  It also clears the group
//                           counts of the next pass.
// A column-scan launch between the two (one workgroup per 4 digits) cost
// ~7 us per pass of pure latency at config 1.  No single-pass (decoupled
// look-back) sort: on this GPU a look-back step is a cross-XCD round trip
// and a workgroup ticket a serialized device atomic, which cost more at
// these sizes than the extra launch boundary.
// radix_sort_ping_pong alternates between two buffer pairs and reports which
// one holds the result, so callers that fill the first pair themselves can
// choose it to make the result land where they want it.
#include "radix.h"

namespace gs {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
// Keys per thread of a tile: short tiles (more workgroups, shorter serial
// ranking chains) for small sorts, longer ones for large sorts.
constexpr int kSortItemsSmall = 4;   // 1024-key tiles
constexpr int kSortItemsLarge = 16;  // 4096-key tiles
constexpr int64_t kSortSmallMax = 1ll << 21;
inline int sort_items(int64_t n) {
    return n <= kSortSmallMax ? kSortItemsSmall : kSortItemsLarge;
}
constexpr int kDigitBits = 8;
constexpr int kRadix = 1 << kDigitBits;

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

// Digit counts of one tile, block-major: hist[tile * 256 + d], also added to
// group_hist[(tile / group_tiles) * 256 + d] (zero on entry).
template <int ITEMS, typename K>
__global__ void __launch_bounds__(kSortThreads)
    radix_hist_kernel(const K *__restrict__ keys, int64_t n, int shift,
                      int bits, uint32_t *__restrict__ hist,
                      uint32_t *__restrict__ group_hist, int group_tiles,
                      const int64_t *__restrict__ n_dev) {
    constexpr int kSortItems = ITEMS;
    constexpr int kSortTile = kSortThreads * ITEMS;
    __shared__ uint32_t s_cnt[kSortWaves][kRadix];
    if (n_dev != nullptr)  // key count on the device, n the capacity
        n = min(n, *n_dev);
    const uint32_t mask = (1u << bits) - 1u;
    for (int i = threadIdx.x; i < kSortWaves * kRadix; i += kSortThreads)
        (&s_cnt[0][0])[i] = 0u;
    __syncthreads();
    const int w = threadIdx.x / kWave;
    const int64_t base = (int64_t)blockIdx.x * kSortTile + (int64_t)w * kWave * kSortItems;
    K kk[kSortItems];
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane_id();
        kk[j] = i < n ? keys[i] : (K)0;
    }
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane_id();
        if (i < n)
            atomicAdd(&s_cnt[w][(uint32_t)(kk[j] >> shift) & mask], 1u);
    }
    __syncthreads();
    const int d = threadIdx.x;  // kSortThreads == kRadix
    uint32_t tot = 0;
#pragma unroll
    for (int ww = 0; ww < kSortWaves; ++ww)
        tot += s_cnt[ww][d];
    hist[(int64_t)blockIdx.x * kRadix + d] = tot;
    if (tot != 0u)
        atomicAdd(&group_hist[(int64_t)(blockIdx.x / group_tiles) * kRadix + d], tot);
}

// Stable scatter of one tile: ranks come from wave64 match ballots
// (order: wave, item, lane = input order), the tile is reordered by digit in
// LDS, then every digit run is written out with consecutive threads on
// consecutive addresses.  With keys64_out (32-bit keys only) the keys are
// written there as (key << 32 | low_bits[value]) instead of to keys_out.
template <int ITEMS, typename K>
__global__ void __launch_bounds__(kSortThreads)
    radix_scatter_kernel(const K *__restrict__ keys_in,
                         const uint32_t *__restrict__ vals_in,
                         K *__restrict__ keys_out,
                         uint32_t *__restrict__ vals_out, int64_t n, int shift,
                         int bits, const uint32_t *__restrict__ hist,
                         const uint32_t *__restrict__ group_hist, int group_tiles,
                         int n_groups, uint32_t *__restrict__ next_group_hist,
                         const uint32_t *__restrict__ low_bits,
                         uint64_t *__restrict__ keys64_out,
                         const int64_t *__restrict__ n_dev) {
    constexpr int kSortItems = ITEMS;
    // the next pass's group counts start from zero (this pass reads only
    // its own); n_tiles >= n_groups, so the workgroups cover them
    if (next_group_hist != nullptr &&
        (int64_t)blockIdx.x * kRadix + threadIdx.x < (int64_t)n_groups * kRadix)
        next_group_hist[(int64_t)blockIdx.x * kRadix + threadIdx.x] = 0u;
    if (n_dev != nullptr)  // key count on the device, n the capacity
        n = min(n, *n_dev);
    // workgroups past the device count have no key to move (the whole
    // workgroup sees the same count, so the return is uniform)
    if ((int64_t)blockIdx.x * (kSortThreads * ITEMS) >= n)
        return;
    constexpr int kSortTile = kSortThreads * ITEMS;
    __shared__ K s_keys[kSortTile];
    __shared__ uint32_t s_vals[kSortTile];
    __shared__ uint32_t s_cnt[kSortWaves][kRadix];
    __shared__ uint32_t s_lstart[kRadix];  // digit start inside the tile
    __shared__ uint32_t s_gstart[kRadix];  // digit start of this tile, global
    __shared__ uint32_t s_wave[kSortWaves];
    const uint32_t mask = (1u << bits) - 1u;
    const int tid = threadIdx.x;
    const int64_t tile_base = (int64_t)blockIdx.x * kSortTile;

    // the tile's keys first, so their round trip overlaps the one of the
    // digit totals and prefixes below
    const int w = tid / kWave;
    const uint32_t lane = lane_id();
    const int64_t base = tile_base + (int64_t)w * kWave * kSortItems;
    K k[kSortItems];
    uint32_t v[kSortItems];
    uint32_t rank[kSortItems];
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        const bool valid = i < n;
        k[j] = valid ? keys_in[i] : ~(K)0;
        v[j] = valid ? vals_in[i] : 0u;
    }
    // global start of every digit for this tile: digit base (over the digit
    // totals) + the digit's count in the tiles before this one (the groups
    // before this tile's group, then the tiles before it in the group)
    {
        const int d = tid;
        const int g = (int)(blockIdx.x / group_tiles);
        uint32_t tot = 0u, pre = 0u;
        if (d <= (int)mask) {  // digits above the pass's bits have no keys
#pragma unroll 8
            for (int gg = 0; gg < n_groups; ++gg) {
                const uint32_t c = group_hist[(int64_t)gg * kRadix + d];
                tot += c;
                pre += gg < g ? c : 0u;
            }
#pragma unroll 8
            for (int64_t tt = (int64_t)g * group_tiles; tt < (int64_t)blockIdx.x; ++tt)
                pre += hist[tt * kRadix + d];
        }
        uint32_t total;
        const uint32_t dbase = block_exclusive_u32<kSortThreads>(tot, s_wave, &total);
        s_gstart[tid] = dbase + pre;
    }
    for (int i = tid; i < kSortWaves * kRadix; i += kSortThreads)
        (&s_cnt[0][0])[i] = 0u;
    __syncthreads();

    rank_wave_span<ITEMS>(k, base, n, shift, bits, s_cnt[w], rank);
    __syncthreads();
    // digit starts inside the tile, and each wave's start within its digit
    {
        const int d = tid;
        uint32_t c[kSortWaves], tot = 0;
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww) {
            c[ww] = s_cnt[ww][d];
            tot += c[ww];
        }
        uint32_t count;
        const uint32_t start = block_exclusive_u32<kSortThreads>(tot, s_wave, &count);
        s_lstart[d] = start;
        uint32_t run = start;
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww) {
            s_cnt[ww][d] = run;
            run += c[ww];
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        if (i < n) {
            const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
            const uint32_t pos = s_cnt[w][d] + rank[j];
            s_keys[pos] = k[j];
            s_vals[pos] = v[j];
        }
    }
    __syncthreads();
    const int64_t rem = n - tile_base;
    const int count = rem < kSortTile ? (int)rem : kSortTile;
    // unrolled so that a thread's gathers of low bits are in flight together
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int i = tid + j * kSortThreads;
        if (i < count) {
            const K key = s_keys[i];
            const uint32_t val = s_vals[i];
            const uint32_t d = (uint32_t)(key >> shift) & mask;
            const uint64_t g = (uint64_t)s_gstart[d] + (uint32_t)(i - s_lstart[d]);
            if constexpr (sizeof(K) == 4) {
                if (keys64_out != nullptr)
                    keys64_out[g] = ((uint64_t)key << 32) | low_bits[val];
                else
                    keys_out[g] = key;
            } else {
                keys_out[g] = key;
            }
            vals_out[g] = val;
        }
    }
}

// Exclusive scan of n uint32 values (single pass, decoupled look-back).
__global__ void __launch_bounds__(kScanThreads)
    scan_u32_kernel(const uint32_t *__restrict__ in, uint32_t *__restrict__ out,
                    int64_t n, Lookback lb) {
    __shared__ uint32_t s_ticket;
    __shared__ uint64_t s_wave_tot[kScanThreads / kWave];
    __shared__ uint64_t s_prefix;
    const uint32_t bid = lb_ticket(lb, &s_ticket);
    const int64_t base = (int64_t)bid * kScanTile + (int64_t)threadIdx.x * kScanItems;
    uint32_t vals[kScanItems];
    uint64_t sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        vals[j] = i < n ? in[i] : 0u;
        sum += vals[j];
    }
    const uint64_t incl = wave_inclusive_scan_u64(sum);
    const int w = threadIdx.x / kWave;
    if (lane_id() == kWave - 1)
        s_wave_tot[w] = incl;
    __syncthreads();
    uint64_t wave_off = 0, total = 0;
#pragma unroll
    for (int ww = 0; ww < kScanThreads / kWave; ++ww) {
        const uint64_t t = s_wave_tot[ww];
        wave_off += ww < w ? t : 0ull;
        total += t;
    }
    if (w == 0) {
        const uint64_t excl = lb_exclusive_prefix(lb, bid, total);
        if (lane_id() == 0)
            s_prefix = excl;
    }
    __syncthreads();
    uint64_t run = s_prefix + wave_off + (incl - sum);
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        if (i < n)
            out[i] = (uint32_t)run;
        run += vals[j];
    }
}

__global__ void copy_pairs_kernel(const uint64_t *__restrict__ ks,
                                  const uint32_t *__restrict__ vs,
                                  uint64_t *__restrict__ kd,
                                  uint32_t *__restrict__ vd, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        kd[i] = ks[i];
        vd[i] = vs[i];
    }
}

__global__ void copy_u32_kernel(const uint32_t *__restrict__ src,
                                uint32_t *__restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = src[i];
}


struct SortLayout {
    int64_t n_tiles;
    int group_tiles, n_groups;
    size_t hist_off, group_off[2], total;
};

SortLayout sort_layout(int64_t n) {
    SortLayout L;
    L.n_tiles = ceil_div(n > 0 ? n : 1, (int64_t)kSortThreads * sort_items(n));
    // groups of about sqrt(tiles) tiles
    int gt = 1;
    while ((int64_t)gt * gt < L.n_tiles)
        ++gt;
    L.group_tiles = gt;
    L.n_groups = (int)ceil_div(L.n_tiles, (int64_t)gt);
    const size_t tbytes = ((size_t)L.n_tiles * kRadix * 4 + 255) / 256 * 256;
    const size_t gbytes = ((size_t)L.n_groups * kRadix * 4 + 255) / 256 * 256;
    L.hist_off = 0;
    L.group_off[0] = tbytes;
    L.group_off[1] = tbytes + gbytes;
    L.total = tbytes + 2 * gbytes;
    return L;
}

__global__ void zero_u32_kernel(uint32_t *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        p[i] = 0u;
}

}  // namespace

int radix_sort_passes(int num_bits) {
    if (num_bits <= 0)
        return 0;
    // as few passes as digits of at most kDigitBits allow
    return (num_bits + kDigitBits - 1) / kDigitBits;
}

size_t radix_sort_workspace_bytes(int64_t n) { return sort_layout(n).total; }

template <typename K>
int radix_sort_impl(int64_t n, int begin_bit, int end_bit, K *keys_a,
                    uint32_t *vals_a, K *keys_b, uint32_t *vals_b, void *workspace,
                    size_t workspace_bytes, hipStream_t st, bool *result_in_b,
                    const uint32_t *low_bits, uint64_t *keys64_out,
                    const int64_t *n_dev, bool counts_zeroed) {
    *result_in_b = false;
    const int num_bits = end_bit - begin_bit;
    if (n == 0 || num_bits <= 0)
        return GSPLAT_OK;
    GS_REQUIRE(n < (1ll << 32), "radix sort: n must be below 2^32");
    const SortLayout L = sort_layout(n);
    GS_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
               "radix sort: workspace too small");
    char *ws = reinterpret_cast<char *>(workspace);
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws + L.hist_off);
    uint32_t *group[2] = {reinterpret_cast<uint32_t *>(ws + L.group_off[0]),
                          reinterpret_cast<uint32_t *>(ws + L.group_off[1])};
    const int passes = radix_sort_passes(num_bits);
    int shift = begin_bit;
    K *ksrc = keys_a, *kdst = keys_b;
    uint32_t *vsrc = vals_a, *vdst = vals_b;
    const bool small = sort_items(n) == kSortItemsSmall;
    const int64_t gwords = (int64_t)L.n_groups * kRadix;
    if (!counts_zeroed) {
        zero_u32_kernel<<<(unsigned)ceil_div(gwords, 256), 256, 0, st>>>(group[0],
                                                                          gwords);
        GS_TRY(check_launch("zero_u32_kernel"));
    }
    for (int p = 0; p < passes; ++p) {
        const int remaining = end_bit - shift;
        const int bits = (remaining + (passes - p) - 1) / (passes - p);
        uint64_t *k64 = p == passes - 1 ? keys64_out : nullptr;
        uint32_t *gcur = group[p & 1];
        uint32_t *gnext = p + 1 < passes ? group[(p + 1) & 1] : nullptr;
        if (small)
            radix_hist_kernel<kSortItemsSmall, K><<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
                ksrc, n, shift, bits, hist, gcur, L.group_tiles, n_dev);
        else
            radix_hist_kernel<kSortItemsLarge, K><<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
                ksrc, n, shift, bits, hist, gcur, L.group_tiles, n_dev);
        GS_TRY(check_launch("radix_hist_kernel"));
        if (small)
            radix_scatter_kernel<kSortItemsSmall, K><<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
                ksrc, vsrc, kdst, vdst, n, shift, bits, hist, gcur, L.group_tiles,
                L.n_groups, gnext, low_bits, k64, n_dev);
        else
            radix_scatter_kernel<kSortItemsLarge, K><<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
                ksrc, vsrc, kdst, vdst, n, shift, bits, hist, gcur, L.group_tiles,
                L.n_groups, gnext, low_bits, k64, n_dev);
        GS_TRY(check_launch("radix_scatter_kernel"));
        shift += bits;
        K *tk = ksrc; ksrc = kdst; kdst = tk;
        uint32_t *tv = vsrc; vsrc = vdst; vdst = tv;
    }
    *result_in_b = (vsrc == vals_b);
    return GSPLAT_OK;
}

int radix_sort_ping_pong(int64_t n, int begin_bit, int end_bit, uint64_t *keys_a,
                         uint32_t *vals_a, uint64_t *keys_b, uint32_t *vals_b,
                         void *workspace, size_t workspace_bytes,
                         hipStream_t st, bool *result_in_b) {
    return radix_sort_impl<uint64_t>(n, begin_bit, end_bit, keys_a, vals_a, keys_b,
                                     vals_b, workspace, workspace_bytes, st,
                                     result_in_b, nullptr, nullptr, nullptr, false);
}

int radix_sort_u32(int64_t n, int num_bits, uint32_t *keys_a, uint32_t *vals_a,
                   uint32_t *keys_b, uint32_t *vals_b, void *workspace,
                   size_t workspace_bytes, hipStream_t st, bool *result_in_b,
                   const uint32_t *low_bits, uint64_t *keys64_out,
                   const int64_t *n_dev, bool counts_zeroed) {
    GS_REQUIRE(num_bits >= 0 && num_bits <= 32, "radix sort: num_bits in [0, 32]");
    GS_REQUIRE(keys64_out == nullptr || (low_bits != nullptr && num_bits > 0),
               "radix sort: 64-bit output needs low bits and at least one pass");
    return radix_sort_impl<uint32_t>(n, 0, num_bits, keys_a, vals_a, keys_b, vals_b,
                                     workspace, workspace_bytes, st, result_in_b,
                                     low_bits, keys64_out, n_dev, counts_zeroed);
}

void radix_sort_first_counts(int64_t n, size_t *offset, int64_t *words) {
    const SortLayout L = sort_layout(n);
    *offset = L.group_off[0];
    *words = (int64_t)L.n_groups * kRadix;
}

int copy_pairs(int64_t n, const uint64_t *ks, const uint32_t *vs, uint64_t *kd,
               uint32_t *vd, hipStream_t st) {
    if (n == 0)
        return GSPLAT_OK;
    copy_pairs_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(ks, vs, kd, vd, n);
    return check_launch("copy_pairs_kernel");
}

int copy_u32(int64_t n, const uint32_t *src, uint32_t *dst, hipStream_t st) {
    if (n == 0)
        return GSPLAT_OK;
    copy_u32_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(src, dst, n);
    return check_launch("copy_u32_kernel");
}

// Exclusive scan used by other translation units of the library.
int scan_u32_exclusive(const uint32_t *in, uint32_t *out, int64_t n, void *ws,
                       hipStream_t st) {
    if (n == 0)
        return GSPLAT_OK;
    const int64_t blocks = ceil_div(n, kScanTile);
    GS_TRY(clear_lookback(ws, blocks, st));
    scan_u32_kernel<<<(unsigned)blocks, kScanThreads, 0, st>>>(
        in, out, n, lookback_from(ws));
    return check_launch("scan_u32_kernel");
}

}  // namespace gs

using namespace gs;

extern "C" size_t gsplat_sort_pairs_workspace_size(int64_t n) {
    return radix_sort_workspace_bytes(n);
}

extern "C" int gsplat_sort_pairs_u64_u32(int64_t n, int32_t num_bits,
                                         uint64_t *keys_in, uint32_t *vals_in,
                                         uint64_t *keys_out, uint32_t *vals_out,
                                         void *workspace,
                                         size_t workspace_bytes,
                                         gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(n >= 0, "sort_pairs: negative n");
    GS_REQUIRE(num_bits >= 0 && num_bits <= 64, "sort_pairs: num_bits in [0, 64]");
    if (n == 0)
        return GSPLAT_OK;
    GS_REQUIRE(keys_in && vals_in && keys_out && vals_out,
               "sort_pairs: NULL buffer");
    GS_REQUIRE(n < (1ll << 32), "sort_pairs: n must be below 2^32");
    GS_REQUIRE(workspace != nullptr &&
                   workspace_bytes >= radix_sort_workspace_bytes(n),
               "sort_pairs: workspace too small");
    hipStream_t st = as_stream(stream);
    bool in_b = false;
    GS_TRY(radix_sort_ping_pong(n, 0, num_bits, keys_in, vals_in, keys_out,
                                vals_out, workspace, workspace_bytes, st, &in_b));
    if (!in_b)
        return copy_pairs(n, keys_in, vals_in, keys_out, vals_out, st);
    return GSPLAT_OK;
}
