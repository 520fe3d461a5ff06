// Stable LSD radix sort of (uint64 key, uint32 value) pairs and a device-wide
// exclusive scan, both hand-written for wave64.
//
// Replaces cub::DeviceRadixSort::SortPairs as used by radix_sort_double_buffer
// (gsplat/cuda/csrc/IntersectTile.cu:478-520): keys are sorted on bits
// [0, num_bits), ties keep their input order.
//
// Per pass (digit of up to 10 bits):
//   1. radix_hist_kernel   each 4096-key tile counts its digits; ranks come
//                          from wave64 "match" ballots, so no LDS atomics;
//   2. scan_u32_kernel     one exclusive scan over the digit-major
//                          [radix][tiles] count table (single pass, decoupled
//                          look-back);
//   3. radix_scatter_kernel recomputes the stable rank of every key inside its
//                          tile (wave-major, item, lane order) and writes it
//                          to its global slot.
// The pass count is kept odd where possible (digit width up to 10 bits), so
// the result lands in the output buffers without a final copy.
#include "common.h"

namespace gs {
namespace {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // keys per workgroup
constexpr int kMaxDigitBits = 10;
constexpr int kMaxRadix = 1 << kMaxDigitBits;

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

// Lanes of the wave holding the same digit as this lane (among `valid`).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, int bits,
                                                uint64_t valid) {
    uint64_t peers = valid;
    for (int b = 0; b < bits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

__global__ void __launch_bounds__(kSortThreads)
    radix_hist_kernel(const uint64_t *__restrict__ keys, int64_t n, int shift,
                      int bits, uint32_t *__restrict__ hist, int64_t n_tiles) {
    __shared__ uint32_t s_cnt[kSortWaves][kMaxRadix];
    const int radix = 1 << bits;
    const uint32_t mask = (uint32_t)radix - 1u;
    for (int i = threadIdx.x; i < kSortWaves * kMaxRadix; i += kSortThreads)
        (&s_cnt[0][0])[i] = 0u;
    __syncthreads();
    const int w = threadIdx.x / kWave;
    const uint32_t lane = lane_id();
    const int64_t base = (int64_t)blockIdx.x * kSortTile + (int64_t)w * kWave * kSortItems;
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        const bool valid = i < n;
        const uint32_t d = valid ? (uint32_t)(keys[i] >> shift) & mask : 0u;
        const uint64_t vmask = __ballot(valid);
        if (vmask == 0)
            break;
        const uint64_t peers = match_digit(d, bits, vmask);
        if (valid && (peers & lanemask_lt()) == 0)
            s_cnt[w][d] += (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int d = threadIdx.x; d < radix; d += kSortThreads) {
        uint32_t tot = 0;
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww)
            tot += s_cnt[ww][d];
        hist[(int64_t)d * n_tiles + blockIdx.x] = tot;
    }
}

__global__ void __launch_bounds__(kSortThreads)
    radix_scatter_kernel(const uint64_t *__restrict__ keys_in,
                         const uint32_t *__restrict__ vals_in,
                         uint64_t *__restrict__ keys_out,
                         uint32_t *__restrict__ vals_out, int64_t n, int shift,
                         int bits, const uint32_t *__restrict__ offsets,
                         int64_t n_tiles) {
    __shared__ uint32_t s_cnt[kSortWaves][kMaxRadix];
    __shared__ uint32_t s_goff[kMaxRadix];
    const int radix = 1 << bits;
    const uint32_t mask = (uint32_t)radix - 1u;
    for (int i = threadIdx.x; i < kSortWaves * kMaxRadix; i += kSortThreads)
        (&s_cnt[0][0])[i] = 0u;
    for (int d = threadIdx.x; d < radix; d += kSortThreads)
        s_goff[d] = offsets[(int64_t)d * n_tiles + blockIdx.x];
    __syncthreads();

    const int w = threadIdx.x / kWave;
    const uint32_t lane = lane_id();
    const int64_t base = (int64_t)blockIdx.x * kSortTile + (int64_t)w * kWave * kSortItems;
    uint64_t k[kSortItems];
    uint32_t v[kSortItems];
    uint32_t rank[kSortItems];
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        const bool valid = i < n;
        k[j] = valid ? keys_in[i] : 0ull;
        v[j] = valid ? vals_in[i] : 0u;
    }
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        const bool valid = i < n;
        const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
        const uint64_t vmask = __ballot(valid);
        const uint64_t peers = match_digit(d, bits, vmask);
        uint32_t r = 0;
        if (valid)
            r = s_cnt[w][d] + (uint32_t)__popcll(peers & lanemask_lt());
        rank[j] = r;
        __builtin_amdgcn_wave_barrier();
        if (valid && (peers & lanemask_lt()) == 0)
            s_cnt[w][d] += (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    // exclusive prefix over the waves for every digit
    for (int d = threadIdx.x; d < radix; d += kSortThreads) {
        uint32_t run = 0;
#pragma unroll
        for (int ww = 0; ww < kSortWaves; ++ww) {
            const uint32_t t = s_cnt[ww][d];
            s_cnt[ww][d] = run;
            run += t;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        if (i < n) {
            const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
            const uint64_t pos = (uint64_t)s_goff[d] + s_cnt[w][d] + rank[j];
            keys_out[pos] = k[j];
            vals_out[pos] = v[j];
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

struct SortLayout {
    int64_t n_tiles;
    int64_t table;          // entries of the [radix][tiles] count table
    int64_t scan_blocks;
    size_t hist_off, scanned_off, lb_off, total;
};

SortLayout sort_layout(int64_t n) {
    SortLayout L;
    L.n_tiles = ceil_div(n > 0 ? n : 1, kSortTile);
    L.table = (int64_t)kMaxRadix * L.n_tiles;
    L.scan_blocks = ceil_div(L.table, kScanTile);
    const size_t tbytes = ((size_t)L.table * 4 + 255) / 256 * 256;
    L.hist_off = 0;
    L.scanned_off = tbytes;
    L.lb_off = 2 * tbytes;
    L.total = L.lb_off + lookback_bytes(L.scan_blocks);
    return L;
}

}  // namespace

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
    return sort_layout(n).total;
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
    const SortLayout L = sort_layout(n);
    GS_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
               "sort_pairs: workspace too small");
    hipStream_t st = as_stream(stream);
    char *ws = reinterpret_cast<char *>(workspace);
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws + L.hist_off);
    uint32_t *scanned = reinterpret_cast<uint32_t *>(ws + L.scanned_off);
    void *lbws = ws + L.lb_off;

    if (num_bits == 0) {
        copy_pairs_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(
            keys_in, vals_in, keys_out, vals_out, n);
        return check_launch("copy_pairs_kernel");
    }
    // choose an odd number of passes with digits of at most 10 bits
    int passes = (num_bits + 7) / 8;
    if (passes % 2 == 0) {
        if ((num_bits + passes - 2) / (passes - 1) <= kMaxDigitBits && passes > 1)
            passes -= 1;
        else
            passes += 1;
    }
    int shift = 0;
    uint64_t *ksrc = keys_in, *kdst = keys_out;
    uint32_t *vsrc = vals_in, *vdst = vals_out;
    for (int p = 0; p < passes; ++p) {
        const int remaining = num_bits - shift;
        const int bits = (remaining + (passes - p) - 1) / (passes - p);
        if (bits <= 0)
            break;
        const int64_t table = ((int64_t)1 << bits) * L.n_tiles;
        radix_hist_kernel<<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
            ksrc, n, shift, bits, hist, L.n_tiles);
        GS_TRY(check_launch("radix_hist_kernel"));
        GS_TRY(scan_u32_exclusive(hist, scanned, table, lbws, st));
        radix_scatter_kernel<<<(unsigned)L.n_tiles, kSortThreads, 0, st>>>(
            ksrc, vsrc, kdst, vdst, n, shift, bits, scanned, L.n_tiles);
        GS_TRY(check_launch("radix_scatter_kernel"));
        shift += bits;
        uint64_t *tk = ksrc; ksrc = kdst; kdst = tk;
        uint32_t *tv = vsrc; vsrc = vdst; vdst = tv;
    }
    if (ksrc != keys_out) {
        copy_pairs_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(
            ksrc, vsrc, keys_out, vals_out, n);
        return check_launch("copy_pairs_kernel");
    }
    return GSPLAT_OK;
}
