// Shared device and host helpers for the gfx950 kernels of libgsplat_hip.so.
//
// Device side: the splatting constants, wave64 reductions built on DPP row
// operations, saturating float->int conversion, a portable natural log whose
// result is reproducible bit for bit on the host, and the decoupled look-back
// prefix used by the single-pass compaction kernels.
// Host side: per-thread error text and argument / launch checks shared by the
// extern "C" entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/gsplat_hip.h"

namespace gs {

// Constants of the splatting model (gsplat/cuda/include/Common.h:73-93,
// gsplat/cuda/_constants.py:16-29).
constexpr float kAlphaThreshold = 1.f / 255.f;
constexpr float kGaussianExtend = 3.33f;
constexpr float kMaxAlpha = 0.99f;
constexpr float kTransmittanceThreshold = 1e-4f;
constexpr float kMinCompensation = 0.005f;
constexpr float kMinOneMinusAlpha = 1e-6f;
// clamp of the alpha that divides the expected depth (render_alphas.clamp(
// min=1e-10), gsplat/rendering.py:1259-1267)
constexpr float kMinExpectedDepthAlpha = 1e-10f;

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Host-side error plumbing.
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
void clear_error();
int fail(int code, const std::string &msg);
// Returns GSPLAT_OK or GSPLAT_ERR_LAUNCH after a kernel launch.
int check_launch(const char *what);

#define GS_REQUIRE(cond, msg)                                                  \
    do {                                                                       \
        if (!(cond))                                                           \
            return ::gs::fail(GSPLAT_ERR_INVALID_ARGUMENT, (msg));             \
    } while (0)

#define GS_TRY(expr)                                                           \
    do {                                                                       \
        int _gs_rc = (expr);                                                   \
        if (_gs_rc != GSPLAT_OK)                                               \
            return _gs_rc;                                                     \
    } while (0)

inline hipStream_t as_stream(gsplat_stream_t s) {
    return reinterpret_cast<hipStream_t>(s);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void *p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------

// Float -> int32 with defined results for every input: NaN -> 0, values
// beyond the int32 range saturate, everything else truncates toward zero.
// The same rule is spelled out in the host oracle.
__device__ __forceinline__ int32_t sat_f2i(float x) {
    if (!(x == x))
        return 0;
    if (x >= 2147483648.f)
        return 2147483647;
    if (x <= -2147483648.f)
        return (-2147483647 - 1);
    return (int32_t)x;
}

// Natural logarithm from its series: x = 2^e * m with m in [sqrt(1/2),
// sqrt(2)), s = (m-1)/(m+1), ln m = 2s + 2s^3/3 + 2s^5/5 + 2s^7/7 + 2s^9/9.
// Only IEEE +, -, *, / are used and contraction is disabled, so the host
// oracle reproduces every bit.  Valid for positive normal x; returns NaN for
// x <= 0 or NaN, +inf for +inf.  Accuracy is a few ulp, which matches the
// fast log the reference uses for the opacity-aware extent.
__device__ __forceinline__ float portable_logf(float x) {
#pragma clang fp contract(off)
    if (!(x > 0.f))
        return __builtin_nanf("");
    if (x == __builtin_inff())
        return x;
    uint32_t bits = __float_as_uint(x);
    int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127;
    float m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
    if (e == -127) {
        // subnormal input: renormalise by 2^23
        float xs = x * 8388608.f;
        bits = __float_as_uint(xs);
        e = (int32_t)((bits >> 23) & 0xffu) - 127 - 23;
        m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
    }
    if (m > 1.41421356f) {
        m = m * 0.5f;
        e = e + 1;
    }
    const float f = m - 1.f;
    const float s = f / (2.f + f);
    const float z = s * s;
    const float r =
        z * (0.666666667f + z * (0.4f + z * (0.285714286f + z * 0.222222222f)));
    const float lnm = (s + s) + s * r;
    const float ef = (float)e;
    // ln 2 split as hi + lo with hi carrying 7 trailing zero bits, so ef*hi
    // is exact for |e| <= 128.
    return ef * 0x1.62e3p-1f + (lnm + ef * 0x1.2fefa2p-17f);
}

// Natural exponential by Cody-Waite range reduction and a minimax polynomial:
// x = k ln2 + r with k = rint(x log2e), |r| <= ln2/2, r computed with a
// two-part ln2 (the high part has 9 significant bits, so k*hi is exact);
// e^r ~ 1 + r + r^2/2 + c3 r^3 + ... + c6 r^6, the degree-6 polynomial of
// least maximum relative error on [-ln2/2, ln2/2] with its first three
// coefficients fixed to those of e^r (exact in float32), fitted by linear
// programming (oracle/exp_poly_fit.py): 6.2e-9 relative, and float32
// coefficients.  Horner form with fused multiply-adds; e^x = e^r * 2^k.
// Error below 0.9 ulp over every float in [-87, 88] (checked exhaustively
// against the double exp); 0 below that range, +inf above, NaN passes
// through.  Only correctly rounded IEEE operations (fma, rint, mul) are
// used, so the host oracle reproduces every bit with fmaf and rintf.
__device__ __forceinline__ float portable_expf(float x) {
#pragma clang fp contract(off)
    if (!(x == x))
        return x;
    if (x < -87.f)
        return 0.f;
    if (x > 88.f)
        return __builtin_inff();
    const float kf = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-kf, 0x1.63p-1f, x);
    r = __builtin_fmaf(-kf, -0x1.bd0106p-13f, r);
    float p = 0x1.6e2dp-10f;
    p = __builtin_fmaf(p, r, 0x1.1264c4p-7f);
    p = __builtin_fmaf(p, r, 0x1.555414p-5f);
    p = __builtin_fmaf(p, r, 0x1.55544ap-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.f);
    p = __builtin_fmaf(p, r, 1.f);
    const float scale = __int_as_float(((int32_t)kf + 127) << 23);
    return p * scale;
}

// portable_expf without its range checks, for the rasterizer's -sigma: for
// every x in [-87, 0] the result is bit-identical to portable_expf(x) (the
// scaling by 2^k, k in [-126, 0], is one ldexp, exactly the product p * 2^k
// that portable_expf forms).  The rasterizer uses the value only where
// 0 <= sigma <= ln(255 o), so x >= -87 unless the opacity exceeds
// e^87 / 255 (about 2.4e35); below -87 this returns the ldexp of the
// polynomial (e^x to ~1 ulp, or 0) where portable_expf returns 0.  Other x
// (NaN, positive, -inf) give values the callers select away.
__device__ __forceinline__ float portable_expf_nonpos(float x) {
#pragma clang fp contract(off)
    const float kf = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-kf, 0x1.63p-1f, x);
    r = __builtin_fmaf(-kf, -0x1.bd0106p-13f, r);
    float p = 0x1.6e2dp-10f;
    p = __builtin_fmaf(p, r, 0x1.1264c4p-7f);
    p = __builtin_fmaf(p, r, 0x1.555414p-5f);
    p = __builtin_fmaf(p, r, 0x1.55544ap-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.f);
    p = __builtin_fmaf(p, r, 1.f);
    return __builtin_ldexpf(p, (int32_t)kf);
}

// Non-temporal 16-byte load of data read once, in whole lines per wave (its
// lines are not worth keeping in the caches).  Per-lane pieces of a line
// must not use it: each piece would fetch the line again.
__device__ __forceinline__ float4 ld_stream4(const float4 *p) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    const v4f_t x = __builtin_nontemporal_load(reinterpret_cast<const v4f_t *>(p));
    return make_float4(x.x, x.y, x.z, x.w);
}

// Non-temporal 16-byte store of data written once, in whole lines per wave.
__device__ __forceinline__ void st_stream4(float4 *p, float4 x) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    const v4f_t v = {x.x, x.y, x.z, x.w};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f_t *>(p));
}

// DPP row operations (gfx9 encodings).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// DPP move restricted to the rows set in ROW_MASK; rows outside the mask
// (and out-of-range sources) read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32_rows(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over each 16-lane row of the wave, branch free: every lane ends with
// its row's sum.  Every lane of the row must be active.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32_rows<0xB1, 0xF>(v);   // quad_perm:[1,0,3,2]
    v += dpp_f32_rows<0x4E, 0xF>(v);   // quad_perm:[2,3,0,1]
    v += dpp_f32_rows<0x141, 0xF>(v);  // row_half_mirror
    v += dpp_f32_rows<0x140, 0xF>(v);  // row_mirror
    return v;
}

// Sum over the first ROWS (1 or 4) 16-lane rows of a wave, branch free: row
// sums, then the row broadcasts 15 (rows 1, 3 += rows 0, 2) and 31 (rows 2,
// 3 += row 1) fold everything into row 3.  The total is in lane
// 16 * ROWS - 1.  Every lane of those rows must be active.
template <int ROWS>
__device__ __forceinline__ float wave_sum_to_last(float v) {
    static_assert(ROWS == 1 || ROWS == 4, "ROWS must be 1 or 4");
    v = row_sum16(v);
    if (ROWS == 4) {
        v += dpp_f32_rows<0x142, 0xA>(v);  // row_bcast:15
        v += dpp_f32_rows<0x143, 0xC>(v);  // row_bcast:31
    }
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active):
// Kogge-Stone within each 16-lane row (row_shr 1, 2, 4, 8; sources outside
// the row read 0), then row broadcasts 15 and 31 carry the row totals.
__device__ __forceinline__ uint32_t wave_inclusive_scan_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);
    return v;
}

// Inclusive running maximum over the 64 lanes of a wave (all lanes active)
// for values >= -1 (-1 is the identity), same pattern as the sum scan.
__device__ __forceinline__ int wave_inclusive_max_i32(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x111, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x112, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x114, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x118, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x142, 0xA, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x143, 0xC, 0xF, false));
    return v;
}

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the lanes of a wave; every lane receives the total (in a scalar
// register).  Must be called in wave-uniform control flow where every 16-lane
// row is either fully active or fully inactive (true for workgroups whose size
// is a multiple of 16); inactive rows are excluded through EXEC.  The
// association order is fixed, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    const int iv = __float_as_int(v);
    const uint64_t ex = __builtin_amdgcn_read_exec();
    const float r0 = (ex & 0xffffull)
                         ? __int_as_float(__builtin_amdgcn_readlane(iv, 0))
                         : 0.f;
    const float r1 = ((ex >> 16) & 0xffffull)
                         ? __int_as_float(__builtin_amdgcn_readlane(iv, 16))
                         : 0.f;
    const float r2 = ((ex >> 32) & 0xffffull)
                         ? __int_as_float(__builtin_amdgcn_readlane(iv, 32))
                         : 0.f;
    const float r3 = ((ex >> 48) & 0xffffull)
                         ? __int_as_float(__builtin_amdgcn_readlane(iv, 48))
                         : 0.f;
    return (r0 + r1) + (r2 + r3);
}

// Maximum over the wave.  In a partially populated wave the shuffles may read
// lanes that never ran; their stale values can only raise the result, so use
// it only where an over-estimate is harmless (a conservative bound).
__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v = max(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Mask of the active lanes where p holds.  The builtin takes the predicate
// as a lane mask, where __ballot(int) first materialises it in a VGPR and
// compares it again (two VALU instructions per vote).
__device__ __forceinline__ uint64_t wave_ballot(bool p) {
    return __builtin_amdgcn_ballot_w64(p);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    return (1ull << lane_id()) - 1ull;
}

// Inclusive scan of a 64-bit value over the wave (Hillis-Steele).
__device__ __forceinline__ uint64_t wave_inclusive_scan_u64(uint64_t v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint64_t o = __shfl_up(v, off);
        if (lane >= (uint32_t)off)
            v += o;
    }
    return v;
}

__device__ __forceinline__ void atomic_add_f32(float *p, float v) {
    unsafeAtomicAdd(p, v);
}

// ---------------------------------------------------------------------------
// Decoupled look-back prefix (single-pass scan across workgroups).
//
// Workgroups take a ticket in launch order so every predecessor of a ticket
// holder is already resident or finished; each publishes its aggregate, then
// its inclusive prefix, in a 64-bit status word: flag in bits 62-63, value in
// bits 0-61.  The status array and the ticket counter must be zero before the
// launch (see clear_lookback).
// ---------------------------------------------------------------------------
constexpr uint64_t kLbFlagAgg = 1ull << 62;
constexpr uint64_t kLbFlagInc = 2ull << 62;
constexpr uint64_t kLbValMask = (1ull << 62) - 1ull;

struct Lookback {
    uint32_t *ticket;  // one counter
    uint64_t *status;  // one word per workgroup
};

// Bytes of workspace for n_blocks workgroups (ticket padded to 256 B).
inline size_t lookback_bytes(int64_t n_blocks) {
    return 256 + (size_t)n_blocks * sizeof(uint64_t);
}

inline Lookback lookback_from(void *ws) {
    Lookback lb;
    lb.ticket = reinterpret_cast<uint32_t *>(ws);
    lb.status = reinterpret_cast<uint64_t *>(reinterpret_cast<char *>(ws) + 256);
    return lb;
}

// Zero the ticket and status words (a kernel, not a memset, so the sequence
// stays valid under stream capture).
int clear_lookback(void *ws, int64_t n_blocks, hipStream_t stream);

// Stable LSD radix sort of (uint64 key, uint32 value) pairs on key bits
// [begin_bit, end_bit) (sort.hip).  Passes alternate a -> b -> a ...;
// *result_in_b tells which pair holds the sorted result (the other pair is
// clobbered).  radix_sort_passes(bits) is the number of passes it makes.
int radix_sort_passes(int num_bits);
size_t radix_sort_workspace_bytes(int64_t n);
int radix_sort_ping_pong(int64_t n, int begin_bit, int end_bit, uint64_t *keys_a,
                         uint32_t *vals_a, uint64_t *keys_b, uint32_t *vals_b,
                         void *workspace, size_t workspace_bytes,
                         hipStream_t st, bool *result_in_b);
// The same sort on (uint32 key, uint32 value) pairs, key bits [0, num_bits),
// num_bits <= 32.  With keys64_out (and low_bits) the last pass writes the
// keys as (key << 32 | low_bits[value]) into keys64_out instead of the key
// buffer.  With n_dev the number of keys is min(n, *n_dev), read on the
// device: n is then a capacity that sizes the launches and the workspace.
// With counts_zeroed the caller has already cleared the words
// radix_sort_first_counts() names (saving the sort's own clearing launch).
int radix_sort_u32(int64_t n, int num_bits, uint32_t *keys_a, uint32_t *vals_a,
                   uint32_t *keys_b, uint32_t *vals_b, void *workspace,
                   size_t workspace_bytes, hipStream_t st, bool *result_in_b,
                   const uint32_t *low_bits, uint64_t *keys64_out,
                   const int64_t *n_dev = nullptr, bool counts_zeroed = false);
// The uint32 words of a sort workspace (for n keys) that must be zero when
// the sort starts: *offset bytes into the workspace, *words long.
void radix_sort_first_counts(int64_t n, size_t *offset, int64_t *words);
int copy_u32(int64_t n, const uint32_t *src, uint32_t *dst, hipStream_t st);
int copy_pairs(int64_t n, const uint64_t *ks, const uint32_t *vs, uint64_t *kd,
               uint32_t *vd, hipStream_t st);
// Exclusive prefix sum of n uint32 values; `ws` holds a look-back workspace
// of lookback_bytes(ceil(n / 2048)) bytes.
int scan_u32_exclusive(const uint32_t *in, uint32_t *out, int64_t n, void *ws,
                       hipStream_t st);

__device__ __forceinline__ uint64_t lb_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lb_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup-uniform ticket (call from every thread; contains a barrier).
__device__ __forceinline__ uint32_t lb_ticket(const Lookback &lb,
                                              uint32_t *smem_slot) {
    if (threadIdx.x == 0)
        *smem_slot = atomicAdd(lb.ticket, 1u);
    __syncthreads();
    return *smem_slot;
}

// Predecessor status words each lane examines per look-back step: one step
// covers 64 * kLbWords workgroups, so the inclusive prefix crosses that many
// workgroups per round trip through the device-coherent level of the
// memory hierarchy.
constexpr int kLbWords = 4;

// Called by all 64 lanes of ONE wave after `aggregate` of workgroup `bid` is
// known; returns (in every lane) the exclusive prefix of workgroup bid and
// publishes its inclusive prefix.
__device__ __forceinline__ uint64_t lb_exclusive_prefix(const Lookback &lb,
                                                        uint32_t bid,
                                                        uint64_t aggregate) {
    const uint32_t lane = lane_id();
    if (bid == 0) {
        if (lane == 0)
            lb_store(lb.status, kLbFlagInc | aggregate);
        return 0;
    }
    if (lane == 0)
        lb_store(lb.status + bid, kLbFlagAgg | aggregate);
    uint64_t excl = 0;
    int64_t base = (int64_t)bid - 1;
    while (true) {
        // lane l holds predecessors base - l * kLbWords - k, nearest first;
        // indices below 0 read as an inclusive prefix of 0
        uint64_t s[kLbWords];
#pragma unroll
        for (int k = 0; k < kLbWords; ++k) {
            const int64_t idx = base - (int64_t)lane * kLbWords - k;
            s[k] = idx >= 0 ? lb_load(lb.status + idx) : kLbFlagInc;
        }
        // wait until every predecessor in the window has published something
        while (true) {
            bool pending = false;
#pragma unroll
            for (int k = 0; k < kLbWords; ++k)
                pending |= (s[k] >> 62) == 0;
            if (!wave_ballot(pending))
                break;
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int k = 0; k < kLbWords; ++k)
                if ((s[k] >> 62) == 0)
                    s[k] = lb_load(lb.status + (base - (int64_t)lane * kLbWords - k));
        }
        int kf = kLbWords;  // this lane's nearest inclusive word
#pragma unroll
        for (int k = kLbWords - 1; k >= 0; --k)
            if ((s[k] >> 62) == 2)
                kf = k;
        uint64_t v = 0;
#pragma unroll
        for (int k = 0; k < kLbWords; ++k)
            if (k <= kf)
                v += s[k] & kLbValMask;
        const uint64_t inc = wave_ballot(kf < kLbWords);
        if (inc) {
            const uint32_t first = __builtin_ctzll(inc);  // closest inclusive
            if (lane > first)
                v = 0;
        }
        for (int off = 32; off >= 1; off >>= 1)
            v += __shfl_xor(v, off);
        excl += v;
        if (inc)
            break;
        base -= 64 * kLbWords;
    }
    if (lane == 0)
        lb_store(lb.status + bid, kLbFlagInc | (excl + aggregate));
    return excl;
}

}  // namespace gs
