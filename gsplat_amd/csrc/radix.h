// Stable radix ranking for wave64, shared by the device-wide sort (sort.hip)
// and the per-tile depth sort (isect.hip).
#pragma once

#include "common.h"

namespace gs {

// Lanes of the wave holding the same digit as this lane (among `valid`).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, int bits,
                                                uint64_t valid) {
    uint64_t peers = valid;
    for (int b = 0; b < bits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = wave_ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

// Stable ranks of a wave's span of ITEMS * 64 keys (key j of a lane at
// base + 64 j + lane; order item, lane = input order): rank[j] is the number
// of earlier keys of the span with the same digit plus cnt[digit] on entry,
// and cnt[d] is advanced by the span's count of digit d.  Keys at or past n
// are ignored.
template <int ITEMS, typename K>
__device__ __forceinline__ void rank_wave_span(const K (&k)[ITEMS], int64_t base,
                                               int64_t n, int shift, int bits,
                                               uint32_t *cnt,
                                               uint32_t (&rank)[ITEMS]) {
    const uint32_t mask = (1u << bits) - 1u;
    const uint32_t lane = lane_id();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int64_t i = base + (int64_t)j * kWave + lane;
        const bool valid = i < n;
        const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
        const uint64_t vmask = wave_ballot(valid);
        const uint64_t peers = match_digit(d, bits, vmask);
        uint32_t r = 0;
        if (valid)
            r = cnt[d] + (uint32_t)__popcll(peers & lanemask_lt());
        rank[j] = r;
        __builtin_amdgcn_wave_barrier();
        if (valid && (peers & lanemask_lt()) == 0)
            cnt[d] += (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
    }
}

// Exclusive prefix over the THREADS values v of the workgroup (one per
// thread); returns the thread's exclusive prefix, *total gets the sum.
// s_wave holds THREADS / 64 words; the caller separates two calls that share
// it by a barrier.
template <int THREADS>
__device__ __forceinline__ uint32_t block_exclusive_u32(uint32_t v,
                                                        uint32_t *s_wave,
                                                        uint32_t *total) {
    constexpr int kWaves = THREADS / kWave;
    const uint32_t incl = wave_inclusive_scan_u32(v);
    const int w = threadIdx.x / kWave;
    if (lane_id() == kWave - 1)
        s_wave[w] = incl;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
        const uint32_t t = s_wave[ww];
        off += ww < w ? t : 0u;
        tot += t;
    }
    *total = tot;
    return off + incl - v;
}

}  // namespace gs
