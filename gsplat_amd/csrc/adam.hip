// Fused Adam without bias correction, one launch over a list of parameter
// tensors.  Semantics of gsplat/cuda/csrc/AdamCUDA.cu:35-69:
//   m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g*g;  p += -lr*m / (sqrt(v)+eps)
// rows whose `valid` byte is 0 are left untouched.
//
// Design: the pass is a pure HBM stream (28 B per element: read p, g, m, v;
// write p, m, v).  Every workgroup owns a 4096-element chunk of exactly one
// tensor, so one launch covers all tensors without per-element tensor lookup;
// each thread moves 16-byte vectors (4 per chunk pass) so a wave issues
// 1 KiB-wide coalesced loads; all of a thread's loads are issued before its
// first update, and the accesses are non-temporal (streamed once).  Ordinary
// stores made this kernel 4% faster at 3.3 GB but left its lines dirty in
// the caches: the next training step's reads of the same parameters (the
// trainer's torch.cat of the SH coefficients) then ran 23% slower, and the
// step 2% slower.  The arithmetic is done in the order written
// above with contraction disabled, which makes the result bit-for-bit
// reproducible by a float32 host restatement.
#include "common.h"

namespace gs {
namespace {

constexpr int kAdamThreads = 256;
constexpr int kAdamVecPerThread = 4;
constexpr int64_t kAdamChunk = (int64_t)kAdamThreads * kAdamVecPerThread * 4;
constexpr int kAdamMaxTensors = 24;


struct AdamDesc {
    float *p;
    const float *g;
    float *m;
    float *v;
    const uint8_t *valid;
    int64_t numel;
    int64_t row_size;
    int64_t block_begin;  // first workgroup of this tensor
    float lr;
    int32_t vec_ok;       // all four buffers 16-byte aligned
};

struct AdamTable {
    AdamDesc t[kAdamMaxTensors];
    int32_t n;
};

__device__ __forceinline__ void adam_update(float &p, float g, float &m,
                                            float &v, float lr, float b1,
                                            float b2, float eps) {
#pragma clang fp contract(off)
    m = b1 * m + (1.0f - b1) * g;
    v = b2 * v + (1.0f - b2) * g * g;
    const float step = -lr * m / (sqrtf(v) + eps);
    p += step;
}

__device__ __forceinline__ bool row_valid(const AdamDesc &d, int64_t e) {
    if (d.valid == nullptr)
        return true;
    return d.valid[e / d.row_size] != 0;
}

__global__ void __launch_bounds__(kAdamThreads)
    adam_multi_kernel(const AdamTable tab, float b1, float b2, float eps) {
    // Select the tensor owning this workgroup (uniform across the block).
    const int64_t bid = blockIdx.x;
    int ti = 0;
    for (int i = 1; i < tab.n; ++i)
        if (bid >= tab.t[i].block_begin)
            ti = i;
    AdamDesc d;
#pragma unroll
    for (int i = 0; i < kAdamMaxTensors; ++i)
        if (i == ti)
            d = tab.t[i];

    const int64_t chunk_begin = (bid - d.block_begin) * kAdamChunk;
    const int64_t chunk_end =
        chunk_begin + kAdamChunk < d.numel ? chunk_begin + kAdamChunk : d.numel;

    if (d.vec_ok) {
        const int64_t nvec_total = d.numel >> 2;
        float4 *p4 = reinterpret_cast<float4 *>(d.p);
        const float4 *g4 = reinterpret_cast<const float4 *>(d.g);
        float4 *m4 = reinterpret_cast<float4 *>(d.m);
        float4 *v4 = reinterpret_cast<float4 *>(d.v);
        const int64_t vbase = chunk_begin >> 2;
        // every load of the thread is issued before the first update, so a
        // wave waits for memory once per chunk
        float4 P[kAdamVecPerThread], G[kAdamVecPerThread], M[kAdamVecPerThread],
            V[kAdamVecPerThread];
        bool ok[kAdamVecPerThread];
#pragma unroll
        for (int it = 0; it < kAdamVecPerThread; ++it) {
            const int64_t q = vbase + (int64_t)it * kAdamThreads + threadIdx.x;
            ok[it] = q < nvec_total && (q << 2) < chunk_end;
            if (ok[it]) {
                P[it] = ld_stream4(&p4[q]);
                G[it] = ld_stream4(&g4[q]);
                M[it] = ld_stream4(&m4[q]);
                V[it] = ld_stream4(&v4[q]);
            }
        }
#pragma unroll
        for (int it = 0; it < kAdamVecPerThread; ++it) {
            if (!ok[it])
                continue;
            const int64_t q = vbase + (int64_t)it * kAdamThreads + threadIdx.x;
            const int64_t e0 = q << 2;
            float4 &p = P[it], &m = M[it], &v = V[it];
            const float4 g = G[it];
            if (d.valid == nullptr) {
                adam_update(p.x, g.x, m.x, v.x, d.lr, b1, b2, eps);
                adam_update(p.y, g.y, m.y, v.y, d.lr, b1, b2, eps);
                adam_update(p.z, g.z, m.z, v.z, d.lr, b1, b2, eps);
                adam_update(p.w, g.w, m.w, v.w, d.lr, b1, b2, eps);
            } else {
                if (row_valid(d, e0 + 0))
                    adam_update(p.x, g.x, m.x, v.x, d.lr, b1, b2, eps);
                if (row_valid(d, e0 + 1))
                    adam_update(p.y, g.y, m.y, v.y, d.lr, b1, b2, eps);
                if (row_valid(d, e0 + 2))
                    adam_update(p.z, g.z, m.z, v.z, d.lr, b1, b2, eps);
                if (row_valid(d, e0 + 3))
                    adam_update(p.w, g.w, m.w, v.w, d.lr, b1, b2, eps);
            }
            st_stream4(&p4[q], p);
            st_stream4(&m4[q], m);
            st_stream4(&v4[q], v);
        }
        // scalar tail (numel not a multiple of 4) handled by the last chunk
        const int64_t tail_begin = nvec_total << 2;
        if (chunk_end == d.numel && tail_begin < d.numel) {
            const int64_t e = tail_begin + threadIdx.x;
            if (e < d.numel && row_valid(d, e)) {
                float p = d.p[e], m = d.m[e], v = d.v[e];
                adam_update(p, d.g[e], m, v, d.lr, b1, b2, eps);
                d.p[e] = p;
                d.m[e] = m;
                d.v[e] = v;
            }
        }
    } else {
        for (int64_t e = chunk_begin + threadIdx.x; e < chunk_end;
             e += kAdamThreads) {
            if (!row_valid(d, e))
                continue;
            float p = d.p[e], m = d.m[e], v = d.v[e];
            adam_update(p, d.g[e], m, v, d.lr, b1, b2, eps);
            d.p[e] = p;
            d.m[e] = m;
            d.v[e] = v;
        }
    }
}

int launch_adam_table(const gsplat_adam_tensor *tensors, int n, float b1,
                      float b2, float eps, hipStream_t stream) {
    AdamTable tab;
    int64_t blocks = 0;
    int k = 0;
    for (int i = 0; i < n; ++i) {
        const gsplat_adam_tensor &t = tensors[i];
        const int64_t numel = t.n_rows * t.row_size;
        if (numel == 0)
            continue;
        AdamDesc &d = tab.t[k++];
        d.p = t.param;
        d.g = t.grad;
        d.m = t.exp_avg;
        d.v = t.exp_avg_sq;
        d.valid = t.valid;
        d.numel = numel;
        d.row_size = t.row_size;
        d.block_begin = blocks;
        d.lr = t.lr;
        d.vec_ok = aligned16(t.param) && aligned16(t.grad) &&
                   aligned16(t.exp_avg) && aligned16(t.exp_avg_sq);
        blocks += ceil_div(numel, kAdamChunk);
    }
    tab.n = k;
    if (k == 0)
        return GSPLAT_OK;
    GS_REQUIRE(blocks < (1ll << 31), "adam: too many elements for one launch");
    adam_multi_kernel<<<(unsigned)blocks, kAdamThreads, 0, stream>>>(tab, b1,
                                                                      b2, eps);
    return check_launch("adam_multi_kernel");
}

}  // namespace
}  // namespace gs

extern "C" int gsplat_adam_multi(const gsplat_adam_tensor *tensors,
                                 int32_t n_tensors, float b1, float b2,
                                 float eps, gsplat_stream_t stream) {
    using namespace gs;
    clear_error();
    GS_REQUIRE(n_tensors >= 0 && n_tensors <= 64,
               "adam_multi: n_tensors must be in [0, 64]");
    GS_REQUIRE(n_tensors == 0 || tensors != nullptr, "adam_multi: tensors is NULL");
    for (int i = 0; i < n_tensors; ++i) {
        const gsplat_adam_tensor &t = tensors[i];
        GS_REQUIRE(t.n_rows >= 0 && t.row_size >= 0,
                   "adam_multi: negative tensor size");
        if (t.n_rows * t.row_size > 0)
            GS_REQUIRE(t.param && t.grad && t.exp_avg && t.exp_avg_sq,
                       "adam_multi: NULL buffer");
    }
    for (int i = 0; i < n_tensors; i += kAdamMaxTensors) {
        const int n = n_tensors - i < kAdamMaxTensors ? n_tensors - i
                                                      : kAdamMaxTensors;
        GS_TRY(launch_adam_table(tensors + i, n, b1, b2, eps, as_stream(stream)));
    }
    return GSPLAT_OK;
}

extern "C" int gsplat_adam(float *param, const float *param_grad,
                           float *exp_avg, float *exp_avg_sq,
                           const uint8_t *valid, int64_t n_rows,
                           int64_t row_size, float lr, float b1, float b2,
                           float eps, gsplat_stream_t stream) {
    gsplat_adam_tensor t;
    t.param = param;
    t.grad = param_grad;
    t.exp_avg = exp_avg;
    t.exp_avg_sq = exp_avg_sq;
    t.valid = valid;
    t.n_rows = n_rows;
    t.row_size = row_size;
    t.lr = lr;
    return gsplat_adam_multi(&t, 1, b1, b2, eps, stream);
}
