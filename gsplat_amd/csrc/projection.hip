// EWA projection of 3D Gaussians to screen-space conics, forward and
// backward, dense ("fused") and packed layouts.
//
// Semantics follow gsplat/cuda/csrc/ProjectionEWA3DGSFused.cu:38-234 and
// ProjectionEWA3DGSPacked.cu:39-286 (math in gsplat/cuda/include/Utils.cuh:
// posW2C :50, covarW2C :83, quat_to_rotmat :174, quat_scale_to_covar :223,
// add_blur :424, persp_proj :542, persp_proj_vjp :583).
//
// MI355X design:
//   * one thread per (camera, Gaussian) row, consecutive lanes on consecutive
//     Gaussians so the AoS input rows ([N,3], [N,4]) of a wave form one
//     contiguous span (768 B / 1 KiB) and every output row stream is written
//     contiguously;
//   * the forward is written in a fixed IEEE operation order with contraction
//     disabled, so the integer outputs (radii, validity, packed order) are
//     reproducible bit for bit by the C host oracle;
//   * the packed forward is ONE launch: each workgroup projects 4096 rows
//     into registers, counts the survivors with wave ballots, gets its
//     output offset from a decoupled look-back prefix and writes the
//     survivors (replacing the reference's count pass, host cumsum/sync and
//     second launch, which projects every row twice);
//   * the dense backward gives each Gaussian to one thread that loops over
//     the C cameras, so gradients need no atomics and are deterministic.
#include <mutex>

#include "sh_rows.h"

namespace gs {
namespace {

constexpr int kProjThreads = 256;

struct Cam {
    float R[9];  // row-major world->camera rotation
    float t[3];
    float fx, fy, cx, cy;
    // forward perspective clamp limits (set_fwd_limits)
    float lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg;
};

__device__ __forceinline__ void load_cam(const float *viewmat, const float *K,
                                         Cam &cam) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
            cam.R[i * 3 + j] = viewmat[i * 4 + j];
        cam.t[i] = viewmat[i * 4 + 3];
    }
    cam.fx = K[0];
    cam.fy = K[4];
    cam.cx = K[2];
    cam.cy = K[5];
}

// Camera constants of the forward's perspective Jacobian clamp (persp_proj,
// Utils.cuh:542): computed once per camera load instead of per row; the
// values are the same IEEE results the per-row formula gives.
__device__ __forceinline__ void set_fwd_limits(Cam &cam, float W, float H) {
#pragma clang fp contract(off)
    const float tan_fovx = (0.5f * W) / cam.fx;
    const float tan_fovy = (0.5f * H) / cam.fy;
    cam.lim_x_pos = (W - cam.cx) / cam.fx + 0.3f * tan_fovx;
    cam.lim_x_neg = cam.cx / cam.fx + 0.3f * tan_fovx;
    cam.lim_y_pos = (H - cam.cy) / cam.fy + 0.3f * tan_fovy;
    cam.lim_y_neg = cam.cy / cam.fy + 0.3f * tan_fovy;
}

// Symmetric 3x3 stored as (00, 01, 02, 11, 12, 22).
struct Sym3 {
    float a00, a01, a02, a11, a12, a22;
};

struct ProjOut {
    float mx, my, depth;
    float ca, cb, cc;  // conic (upper triangle of the inverse 2D covariance)
    float comp;
    int32_t rx, ry;
};

// ---------------------------------------------------------------------------
// Exact forward: a fixed sequence of IEEE operations in which every a * b + c
// is one explicit fused multiply-add (fmaf, correctly rounded on the GPU and
// in the host's C library) and nothing else is contracted.  Returns false
// for culled rows.  The host oracle (oracle/exact_ref.c) restates this
// sequence operation for operation.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void quat_to_rot_exact(float w, float x, float y,
                                                  float z, float M[9]) {
#pragma clang fp contract(off)
    const float n2 = fmaf(w, w, fmaf(z, z, fmaf(y, y, x * x)));
    const float inv = 1.0f / sqrtf(n2);
    x = x * inv;
    y = y * inv;
    z = z * inv;
    w = w * inv;
    const float x2 = x * x, y2 = y * y, z2 = z * z;
    const float xy = x * y, xz = x * z, yz = y * z;
    const float wx = w * x, wy = w * y, wz = w * z;
    M[0] = fmaf(-2.f, y2 + z2, 1.f);
    M[1] = 2.f * (xy - wz);
    M[2] = 2.f * (xz + wy);
    M[3] = 2.f * (xy + wz);
    M[4] = fmaf(-2.f, x2 + z2, 1.f);
    M[5] = 2.f * (yz - wx);
    M[6] = 2.f * (xz - wy);
    M[7] = 2.f * (yz + wx);
    M[8] = fmaf(-2.f, x2 + y2, 1.f);
}

// a0 b0 + a1 b1 + a2 b2 as a product and two fused multiply-adds
__device__ __forceinline__ float dot3_exact(float a0, float b0, float a1, float b1,
                                            float a2, float b2) {
#pragma clang fp contract(off)
    return fmaf(a2, b2, fmaf(a1, b1, a0 * b0));
}

__device__ __forceinline__ Sym3 covar_from_quat_scale_exact(const float *q,
                                                            const float *s) {
#pragma clang fp contract(off)
    float M[9];
    quat_to_rot_exact(q[0], q[1], q[2], q[3], M);
    float A[9];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        A[i * 3 + 0] = M[i * 3 + 0] * s[0];
        A[i * 3 + 1] = M[i * 3 + 1] * s[1];
        A[i * 3 + 2] = M[i * 3 + 2] * s[2];
    }
#define GS_DOT_ROWS(i, j)                                                      \
    dot3_exact(A[(i) * 3 + 0], A[(j) * 3 + 0], A[(i) * 3 + 1], A[(j) * 3 + 1],   \
               A[(i) * 3 + 2], A[(j) * 3 + 2])
    Sym3 S;
    S.a00 = GS_DOT_ROWS(0, 0);
    S.a01 = GS_DOT_ROWS(0, 1);
    S.a02 = GS_DOT_ROWS(0, 2);
    S.a11 = GS_DOT_ROWS(1, 1);
    S.a12 = GS_DOT_ROWS(1, 2);
    S.a22 = GS_DOT_ROWS(2, 2);
#undef GS_DOT_ROWS
    return S;
}

__device__ __forceinline__ bool project_exact(
    const Cam &cam, const float *mean, const float *covar6, const float *quat,
    const float *scale, bool has_opacity, float opacity, bool calc_comp,
    int camera_model, float W, float H, float eps2d, float near_plane,
    float far_plane, float radius_clip, ProjOut &o) {
#pragma clang fp contract(off)
    const float *R = cam.R;
    const float p0 = mean[0], p1 = mean[1], p2 = mean[2];
    const float mcx = fmaf(R[2], p2, fmaf(R[1], p1, fmaf(R[0], p0, cam.t[0])));
    const float mcy = fmaf(R[5], p2, fmaf(R[4], p1, fmaf(R[3], p0, cam.t[1])));
    const float mcz = fmaf(R[8], p2, fmaf(R[7], p1, fmaf(R[6], p0, cam.t[2])));
    if (mcz < near_plane || mcz > far_plane)
        return false;

    Sym3 S;
    if (covar6 != nullptr) {
        S.a00 = covar6[0];
        S.a01 = covar6[1];
        S.a02 = covar6[2];
        S.a11 = covar6[3];
        S.a12 = covar6[4];
        S.a22 = covar6[5];
    } else {
        S = covar_from_quat_scale_exact(quat, scale);
    }
    // B = R * S
    const float Sf[9] = {S.a00, S.a01, S.a02, S.a01, S.a11,
                         S.a12, S.a02, S.a12, S.a22};
    float Bm[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            Bm[i * 3 + j] = dot3_exact(R[i * 3 + 0], Sf[0 * 3 + j], R[i * 3 + 1],
                                       Sf[1 * 3 + j], R[i * 3 + 2], Sf[2 * 3 + j]);
    // Sc = B * R^T (upper triangle)
#define GS_SC(i, j)                                                            \
    dot3_exact(Bm[(i) * 3 + 0], R[(j) * 3 + 0], Bm[(i) * 3 + 1], R[(j) * 3 + 1], \
               Bm[(i) * 3 + 2], R[(j) * 3 + 2])
    const float s00 = GS_SC(0, 0), s01 = GS_SC(0, 1), s02 = GS_SC(0, 2);
    const float s11 = GS_SC(1, 1), s12 = GS_SC(1, 2), s22 = GS_SC(2, 2);
#undef GS_SC

    float J00, J02, J11, J12, mx, my;
    if (camera_model == GSPLAT_CAMERA_ORTHO) {
        J00 = cam.fx;
        J11 = cam.fy;
        J02 = 0.f;
        J12 = 0.f;
        mx = fmaf(cam.fx, mcx, cam.cx);
        my = fmaf(cam.fy, mcy, cam.cy);
    } else {
        const float rz = 1.f / mcz;
        const float rz2 = rz * rz;
        const float tx =
            mcz * fminf(cam.lim_x_pos, fmaxf(-cam.lim_x_neg, mcx * rz));
        const float ty =
            mcz * fminf(cam.lim_y_pos, fmaxf(-cam.lim_y_neg, mcy * rz));
        J00 = cam.fx * rz;
        J11 = cam.fy * rz;
        J02 = ((-cam.fx) * tx) * rz2;
        J12 = ((-cam.fy) * ty) * rz2;
        mx = fmaf(cam.fx * mcx, rz, cam.cx);
        my = fmaf(cam.fy * mcy, rz, cam.cy);
    }
    // cov2d = J Sc J^T with J = [[J00, 0, J02], [0, J11, J12]]
    const float u0 = fmaf(s02, J02, s00 * J00);
    const float u1 = fmaf(s12, J02, s01 * J00);
    const float u2 = fmaf(s22, J02, s02 * J00);
    const float w1 = fmaf(s12, J12, s11 * J11);
    const float w2 = fmaf(s22, J12, s12 * J11);
    const float c00 = fmaf(J02, u2, J00 * u0);
    const float c01 = fmaf(J12, u2, J11 * u1);
    const float c11 = fmaf(J12, w2, J11 * w1);

    // low-pass blur + compensation (add_blur)
    const float c01sq = c01 * c01;
    const float det_orig = fmaf(c00, c11, -c01sq);
    const float c00b = c00 + eps2d;
    const float c11b = c11 + eps2d;
    const float det = fmaf(c00b, c11b, -c01sq);
    if (!(det > 0.f))
        return false;
    const float comp =
        sqrtf(fmaxf(kMinCompensation * kMinCompensation, det_orig / det));
    const float inv_det = 1.f / det;

    float extend = kGaussianExtend;
    if (has_opacity) {
        float op = opacity;
        if (calc_comp)
            op = op * comp;
        if (op < kAlphaThreshold)
            return false;
        extend = fminf(kGaussianExtend,
                       sqrtf(2.f * portable_logf(op / kAlphaThreshold)));
    }
    const float rx = ceilf(extend * sqrtf(c00b));
    const float ry = ceilf(extend * sqrtf(c11b));
    if (rx <= radius_clip && ry <= radius_clip)
        return false;
    if (mx + rx <= 0.f || mx - rx >= W || my + ry <= 0.f || my - ry >= H)
        return false;

    o.mx = mx;
    o.my = my;
    o.depth = mcz;
    o.ca = c11b * inv_det;
    o.cb = (-c01) * inv_det;
    o.cc = c00b * inv_det;
    o.comp = comp;
    o.rx = sat_f2i(rx);
    o.ry = sat_f2i(ry);
    return true;
}

// ---------------------------------------------------------------------------
// Forward kernels.
// ---------------------------------------------------------------------------
struct FwdArgs {
    int64_t B, C, N;
    const float *means, *covars, *quats, *scales, *opacities;
    const float *viewmats, *Ks;
    float W, H, eps2d, near_plane, far_plane, radius_clip;
    int camera_model;
    bool calc_comp;
    bool idx32;  // B * C * N < 2^31: row index arithmetic in 32 bits
};

// row = (b * C + c) * N + g  ->  bc = b * C + c, g, the Gaussian's input
// row b * N + g, and (optionally) b and c themselves
__device__ __forceinline__ void split_row(const FwdArgs &a, int64_t row,
                                          int64_t &bc, int64_t &g, int64_t &bg,
                                          int64_t *b_out = nullptr,
                                          int64_t *c_out = nullptr) {
    int64_t b;
    if (a.B * a.C == 1) {
        // one image: no division
        bc = 0;
        g = row;
        bg = row;
        b = 0;
    } else if (a.idx32) {
        const uint32_t r = (uint32_t)row, n = (uint32_t)a.N;
        const uint32_t q = r / n;
        bc = q;
        g = r - q * n;
        b = q / (uint32_t)a.C;
        bg = b * a.N + g;
    } else {
        bc = row / a.N;
        g = row - bc * a.N;
        b = bc / a.C;
        bg = b * a.N + g;
    }
    if (b_out != nullptr) {
        *b_out = b;
        *c_out = bc - b * a.C;
    }
}

// Camera of (batch, camera) row bc: loaded once per wave (scalar loads) when
// all the wave's rows belong to one camera row, per lane otherwise.
__device__ __forceinline__ void load_row_cam(const FwdArgs &a, int64_t bc,
                                             Cam &cam) {
    const int64_t bc0 = ((int64_t)__builtin_amdgcn_readfirstlane((int)(bc >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)bc);
    if (!wave_ballot(bc != bc0))
        load_cam(a.viewmats + bc0 * 16, a.Ks + bc0 * 9, cam);
    else
        load_cam(a.viewmats + bc * 16, a.Ks + bc * 9, cam);
    set_fwd_limits(cam, a.W, a.H);
}

__device__ __forceinline__ bool project_flat_row(const FwdArgs &a, int64_t row,
                                                 ProjOut &o) {
    int64_t bc, g, bg;
    split_row(a, row, bc, g, bg);
    Cam cam;
    load_row_cam(a, bc, cam);
    return project_exact(
        cam, a.means + bg * 3, a.covars ? a.covars + bg * 6 : nullptr,
        a.quats ? a.quats + bg * 4 : nullptr,
        a.scales ? a.scales + bg * 3 : nullptr, a.opacities != nullptr,
        a.opacities ? a.opacities[bg] : 0.f, a.calc_comp, a.camera_model, a.W,
        a.H, a.eps2d, a.near_plane, a.far_plane, a.radius_clip, o);
}

__global__ void __launch_bounds__(kProjThreads)
    projection_fused_fwd_kernel(const FwdArgs a, int32_t *__restrict__ radii,
                                float *__restrict__ means2d,
                                float *__restrict__ depths,
                                float *__restrict__ conics,
                                float *__restrict__ compensations) {
    const int64_t row = (int64_t)blockIdx.x * kProjThreads + threadIdx.x;
    if (row >= a.B * a.C * a.N)
        return;
    ProjOut o;
    const bool valid = project_flat_row(a, row, o);
    if (!valid) {
        o.mx = o.my = o.depth = o.ca = o.cb = o.cc = o.comp = 0.f;
        o.rx = o.ry = 0;
    }
    reinterpret_cast<int2 *>(radii)[row] = make_int2(o.rx, o.ry);
    reinterpret_cast<float2 *>(means2d)[row] = make_float2(o.mx, o.my);
    depths[row] = o.depth;
    conics[row * 3 + 0] = o.ca;
    conics[row * 3 + 1] = o.cb;
    conics[row * 3 + 2] = o.cc;
    if (compensations != nullptr)
        compensations[row] = o.comp;
}

// Packed forward workgroup: 1024 threads x kPackItems rows = 4096 rows in
// kPackItems slices of 1024 consecutive rows (one wave reads 64 consecutive
// Gaussians per slice).  Every input of a thread's rows is loaded before any
// of them is projected, so a wave waits for memory once; the projected rows
// stay in registers between the survivor count and the write (inputs are
// read once).  Few, large workgroups keep the look-back chain that orders
// them short (245 links per million rows).
constexpr int kPackThreads = 1024;
constexpr int kPackItems = 4;
constexpr int kPackRows = kPackThreads * kPackItems;

template <bool COVARS>
__global__ void __launch_bounds__(kPackThreads) projection_packed_fwd_kernel(
    const FwdArgs a, Lookback lb, int32_t *__restrict__ indptr,
    int64_t *__restrict__ batch_ids, int64_t *__restrict__ camera_ids,
    int64_t *__restrict__ gaussian_ids, int32_t *__restrict__ radii,
    float *__restrict__ means2d, float *__restrict__ depths,
    float *__restrict__ conics, float *__restrict__ compensations,
    int64_t *__restrict__ nnz_out, int32_t *__restrict__ row_of,
    float *__restrict__ row_opacities) {
    constexpr int NW = kPackThreads / kWave;
    static_assert(kPackItems * NW <= kWave, "one wave scans the wave counts");
    __shared__ uint32_t s_ticket;
    __shared__ uint32_t s_cnt[kPackItems * NW];  // survivors per (slice, wave)
    __shared__ uint32_t s_off[kPackItems * NW];  // their exclusive prefix
    __shared__ uint64_t s_prefix;
    __shared__ uint32_t s_total;

    const int64_t n_rows = a.B * a.C * a.N;
    const uint32_t bid = lb_ticket(lb, &s_ticket);
    const int64_t base = (int64_t)bid * kPackRows;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = lane_id();

    // phase 0: row indices, the camera of the wave's first row, then every
    // input of the thread's rows (rows past the end read the last row and
    // are dropped).  The camera is loaded before the rows: loads complete in
    // issue order, so waiting for the camera does not wait for the rows, and
    // projecting slice j waits only for the loads of slices 0..j.
    int64_t bc[kPackItems], g[kPackItems], bgs[kPackItems], bi[kPackItems],
        ci[kPackItems];
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
        const int64_t row = base + (int64_t)j * kPackThreads + threadIdx.x;
        split_row(a, row < n_rows ? row : n_rows - 1, bc[j], g[j], bgs[j], &bi[j],
                  &ci[j]);
    }
    const int64_t bc0 =
        ((int64_t)__builtin_amdgcn_readfirstlane((int)(bc[0] >> 32)) << 32) |
        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)bc[0]);
    Cam cam0;
    load_cam(a.viewmats + bc0 * 16, a.Ks + bc0 * 9, cam0);
    float mean[kPackItems][3], quat[kPackItems][4], scale[kPackItems][3];
    float cov[kPackItems][6], opac[kPackItems];
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
        const int64_t bg = bgs[j];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            mean[j][k] = a.means[bg * 3 + k];
        if constexpr (COVARS) {
#pragma unroll
            for (int k = 0; k < 6; ++k)
                cov[j][k] = a.covars[bg * 6 + k];
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                quat[j][k] = a.quats[bg * 4 + k];
#pragma unroll
            for (int k = 0; k < 3; ++k)
                scale[j][k] = a.scales[bg * 3 + k];
        }
        opac[j] = a.opacities ? a.opacities[bg] : 0.f;
    }

    // phase 1: project; the camera loaded above serves every row when all
    // rows of the wave belong to its camera row
    bool mixed = false;
#pragma unroll
    for (int j = 0; j < kPackItems; ++j)
        mixed |= bc[j] != bc0;
    const bool one_cam = !wave_ballot(mixed);
    set_fwd_limits(cam0, a.W, a.H);
    ProjOut o[kPackItems];
    uint64_t bal[kPackItems];
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
        const int64_t row = base + (int64_t)j * kPackThreads + threadIdx.x;
        Cam cam;
        if (one_cam) {
            cam = cam0;
        } else {
            load_cam(a.viewmats + bc[j] * 16, a.Ks + bc[j] * 9, cam);
            set_fwd_limits(cam, a.W, a.H);
        }
        const bool valid =
            project_exact(cam, mean[j], COVARS ? cov[j] : nullptr,
                          COVARS ? nullptr : quat[j],
                          COVARS ? nullptr : scale[j], a.opacities != nullptr,
                          opac[j], a.calc_comp, a.camera_model, a.W, a.H,
                          a.eps2d, a.near_plane, a.far_plane, a.radius_clip,
                          o[j]) &&
            row < n_rows;
        bal[j] = wave_ballot(valid);
        if (lane == 0)
            s_cnt[j * NW + wave] = (uint32_t)__popcll(bal[j]);
    }
    __syncthreads();
    // survivors before each (slice, wave) in row order, and the block's
    // output offset
    if (wave == 0) {
        const uint32_t c = lane < (uint32_t)(kPackItems * NW) ? s_cnt[lane] : 0u;
        const uint32_t inc = (uint32_t)wave_inclusive_scan_u64(c);
        if (lane < (uint32_t)(kPackItems * NW))
            s_off[lane] = inc - c;
        const uint32_t total = __shfl(inc, kWave - 1);
        const uint64_t excl = lb_exclusive_prefix(lb, bid, total);
        if (lane == 0) {
            s_prefix = excl;
            s_total = total;
        }
    }
    __syncthreads();
    const int64_t block_out = (int64_t)s_prefix;

    // phase 2: write the survivors at their packed positions
#pragma unroll
    for (int j = 0; j < kPackItems; ++j) {
        const int64_t row = base + (int64_t)j * kPackThreads + threadIdx.x;
        if (row >= n_rows)
            break;
        const bool valid = (bal[j] >> lane) & 1ull;
        const int64_t pos = block_out + s_off[j * NW + wave] +
                            (uint32_t)__popcll(bal[j] & lanemask_lt());
        if (g[j] == 0) {
            // first Gaussian of camera row bc: its exclusive position is indptr
            indptr[bc[j]] = (int32_t)pos;
        }
        if (row_of != nullptr)
            row_of[row] = valid ? (int32_t)pos : -1;
        if (!valid)
            continue;
        batch_ids[pos] = bi[j];
        camera_ids[pos] = ci[j];
        gaussian_ids[pos] = g[j];
        reinterpret_cast<int2 *>(radii)[pos] = make_int2(o[j].rx, o[j].ry);
        reinterpret_cast<float2 *>(means2d)[pos] = make_float2(o[j].mx, o[j].my);
        depths[pos] = o[j].depth;
        conics[pos * 3 + 0] = o[j].ca;
        conics[pos * 3 + 1] = o[j].cb;
        conics[pos * 3 + 2] = o[j].cc;
        if (compensations != nullptr)
            compensations[pos] = o[j].comp;
        // the row's opacity, opacities[b, g] (read above for the culling)
        if (row_opacities != nullptr)
            row_opacities[pos] = opac[j];
    }
    const int64_t last_bid = (n_rows - 1) / kPackRows;
    if ((int64_t)bid == last_bid && threadIdx.x == 0) {
        const int64_t nnz = block_out + s_total;
        indptr[a.B * a.C] = (int32_t)nnz;
        *nnz_out = nnz;
    }
}

// ---------------------------------------------------------------------------
// Backward math (contraction allowed; validated against autograd).
//
// The vector-Jacobian products run in double precision from the float32
// inputs.  The covariance chain (2D inverse -> camera covariance -> world
// covariance -> scaled rotation -> quaternion and scales) multiplies the
// upstream gradient by J^T ... J, whose entries are ~f/z, and then contracts
// the result with the Gaussian's axes; for an axis close to the viewing ray
// the terms cancel by orders of magnitude, and float32 loses that many
// digits of the scale and quaternion gradients.  On gfx950 a double FMA
// issues at the rate of an unpacked float32 FMA, and these kernels are bound
// by memory latency, so the double chain costs no time.
// ---------------------------------------------------------------------------
template <typename T>
struct Mat3 {
    T m[9];  // row-major
};
using M3 = Mat3<float>;
using M3d = Mat3<double>;

template <typename T>
__device__ __forceinline__ Mat3<T> mm(const Mat3<T> &a, const Mat3<T> &b) {
    Mat3<T> r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            r.m[i * 3 + j] = a.m[i * 3 + 0] * b.m[0 * 3 + j] +
                             a.m[i * 3 + 1] * b.m[1 * 3 + j] +
                             a.m[i * 3 + 2] * b.m[2 * 3 + j];
    return r;
}
template <typename T>
__device__ __forceinline__ Mat3<T> mtm(const Mat3<T> &a, const Mat3<T> &b) {  // a^T b
    Mat3<T> r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            r.m[i * 3 + j] = a.m[0 * 3 + i] * b.m[0 * 3 + j] +
                             a.m[1 * 3 + i] * b.m[1 * 3 + j] +
                             a.m[2 * 3 + i] * b.m[2 * 3 + j];
    return r;
}
template <typename T>
__device__ __forceinline__ Mat3<T> mmt(const Mat3<T> &a, const Mat3<T> &b) {  // a b^T
    Mat3<T> r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            r.m[i * 3 + j] = a.m[i * 3 + 0] * b.m[j * 3 + 0] +
                             a.m[i * 3 + 1] * b.m[j * 3 + 1] +
                             a.m[i * 3 + 2] * b.m[j * 3 + 2];
    return r;
}

// Rotation of the normalised (w, x, y, z) quaternion, in double.
__device__ __forceinline__ void quat_to_rot_d(const float qf[4], double R[9]) {
    const double q0 = qf[0], q1 = qf[1], q2 = qf[2], q3 = qf[3];
    const double inv = 1.0 / sqrt(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    const double w = q0 * inv, x = q1 * inv, y = q2 * inv, z = q3 * inv;
    R[0] = 1.0 - 2.0 * (y * y + z * z);
    R[1] = 2.0 * (x * y - w * z);
    R[2] = 2.0 * (x * z + w * y);
    R[3] = 2.0 * (x * y + w * z);
    R[4] = 1.0 - 2.0 * (x * x + z * z);
    R[5] = 2.0 * (y * z - w * x);
    R[6] = 2.0 * (x * z - w * y);
    R[7] = 2.0 * (y * z + w * x);
    R[8] = 1.0 - 2.0 * (x * x + y * y);
}

// Symmetric 3x3 matrix: (xx, xy, xz, yy, yz, zz).
struct Sym3d {
    double v[6];
    __device__ __forceinline__ double at(int i, int j) const {
        // index of (i, j) in the upper triangle
        const int a = i < j ? i : j, b = i < j ? j : i;
        return v[a == 0 ? b : (a == 1 ? 2 + b : 5)];
    }
};

// A S A^T for a general A (given by a functor of (i, j)) and symmetric S.
template <typename AT>
__device__ __forceinline__ Sym3d congruence(const AT &A, const Sym3d &S) {
    double T[9];  // A S
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            T[i * 3 + j] = A(i, 0) * S.at(0, j) + A(i, 1) * S.at(1, j) + A(i, 2) * S.at(2, j);
    Sym3d r;
    int k = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = i; j < 3; ++j)
            r.v[k++] = T[i * 3 + 0] * A(j, 0) + T[i * 3 + 1] * A(j, 1) + T[i * 3 + 2] * A(j, 2);
    return r;
}

// Gaussian geometry for the backward: the raw inputs (float) and the world
// covariance in double, recomputed from them.
struct GaussGeom {
    Sym3d S;    // world covariance
    float q[4]; // raw quaternion (quats path only)
    float s[3]; // scales
};

__device__ __forceinline__ void load_geom(const float *covar6, const float *quat,
                                          const float *scale, GaussGeom &G) {
    if (covar6 != nullptr) {
#pragma unroll
        for (int k = 0; k < 6; ++k)
            G.S.v[k] = covar6[k];
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        G.q[i] = quat[i];
#pragma unroll
    for (int i = 0; i < 3; ++i)
        G.s[i] = scale[i];
    double Rq[9];
    quat_to_rot_d(G.q, Rq);
    const double s2[3] = {(double)G.s[0] * G.s[0], (double)G.s[1] * G.s[1],
                          (double)G.s[2] * G.s[2]};
    int k = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = i; j < 3; ++j)
            G.S.v[k++] = Rq[i * 3 + 0] * Rq[j * 3 + 0] * s2[0] +
                         Rq[i * 3 + 1] * Rq[j * 3 + 1] * s2[1] +
                         Rq[i * 3 + 2] * Rq[j * 3 + 2] * s2[2];
}

// Gradient of one (camera, Gaussian) row: accumulates dL/dmean (world),
// dL/dS (world covariance, symmetric) and, if wanted, dL/dR, dL/dt.
__device__ __forceinline__ void project_row_vjp(
    const Cam &cam, const float *mean, const GaussGeom &G, int camera_model,
    float W, float H, float eps2d, const float *conic, bool has_comp,
    float comp_f, float v_comp_f, float v_mx_f, float v_my_f, float v_depth_f,
    const float *v_conic, double v_mean[3], Sym3d &v_S, bool want_cam, M3d &v_R,
    double v_t[3]) {
    const float *Rf = cam.R;
    auto R = [&](int i, int j) -> double { return (double)Rf[i * 3 + j]; };
    auto Rt = [&](int i, int j) -> double { return (double)Rf[j * 3 + i]; };
    const double p[3] = {mean[0], mean[1], mean[2]};
    double mc[3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
        mc[i] = R(i, 0) * p[0] + R(i, 1) * p[1] + R(i, 2) * p[2] + (double)cam.t[i];
    const Sym3d Sc = congruence(R, G.S);
    const double v_mx = v_mx_f, v_my = v_my_f;

    // d/d(cov2d): inverse VJP  dL/dC = -Ci * dL/dCi * Ci (symmetric)
    const double ia = conic[0], ib = conic[1], ic = conic[2];
    const double ga = v_conic[0], gb = 0.5 * (double)v_conic[1], gc = v_conic[2];
    const double t00 = ia * ga + ib * gb, t01 = ia * gb + ib * gc;
    const double t11 = ib * gb + ic * gc;
    double vc00 = -(t00 * ia + t01 * ib);
    double vc01 = -(t00 * ib + t01 * ic);
    double vc11 = -((ib * ga + ic * gb) * ib + t11 * ic);
    if (has_comp) {
        // comp = sqrt(det(C) / det(C + eps I)); conic is the blurred inverse
        const double comp = comp_f, eps = eps2d;
        const double det_conic = ia * ic - ib * ib;
        const double v_sqr_comp = (double)v_comp_f * 0.5 / (comp + 1e-6);
        const double one_minus = 1.0 - comp * comp;
        vc00 += v_sqr_comp * (one_minus * ia - eps * det_conic);
        vc01 += v_sqr_comp * (one_minus * ib);
        vc11 += v_sqr_comp * (one_minus * ic - eps * det_conic);
    }

    const double fx = cam.fx, fy = cam.fy;
    const double x = mc[0], y = mc[1], z = mc[2];
    double J[6];  // row-major 2x3
    double vmc[3];
    if (camera_model == GSPLAT_CAMERA_ORTHO) {
        J[0] = fx; J[1] = 0.0; J[2] = 0.0;
        J[3] = 0.0; J[4] = fy; J[5] = 0.0;
        vmc[0] = fx * v_mx;
        vmc[1] = fy * v_my;
        vmc[2] = 0.0;
    } else {
        // the clamp limits are the forward's float32 values
        const float tan_fovx = 0.5f * W / cam.fx, tan_fovy = 0.5f * H / cam.fy;
        const double lim_x_pos = (W - cam.cx) / cam.fx + 0.3f * tan_fovx;
        const double lim_x_neg = cam.cx / cam.fx + 0.3f * tan_fovx;
        const double lim_y_pos = (H - cam.cy) / cam.fy + 0.3f * tan_fovy;
        const double lim_y_neg = cam.cy / cam.fy + 0.3f * tan_fovy;
        const double rz = 1.0 / z, rz2 = rz * rz, rz3 = rz2 * rz;
        const double xr = x * rz, yr = y * rz;
        const double tx = z * fmin(lim_x_pos, fmax(-lim_x_neg, xr));
        const double ty = z * fmin(lim_y_pos, fmax(-lim_y_neg, yr));
        J[0] = fx * rz; J[1] = 0.0; J[2] = -fx * tx * rz2;
        J[3] = 0.0; J[4] = fy * rz; J[5] = -fy * ty * rz2;
        vmc[0] = fx * rz * v_mx;
        vmc[1] = fy * rz * v_my;
        vmc[2] = -(fx * x * v_mx + fy * y * v_my) * rz2;
        // dL/dJ = (G + G^T) J Sc with G = dL/dcov2d; only the columns 0 and 2
        // of row 0 and columns 1 and 2 of row 1 depend on the mean
        const double g00 = vc00 + vc00, g01 = vc01 + vc01, g11 = vc11 + vc11;
        double JS[6];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int c = 0; c < 3; ++c)
                JS[r * 3 + c] = J[r * 3 + 0] * Sc.at(0, c) + J[r * 3 + 1] * Sc.at(1, c) +
                                J[r * 3 + 2] * Sc.at(2, c);
        const double vJ00 = g00 * JS[0] + g01 * JS[3];
        const double vJ02 = g00 * JS[2] + g01 * JS[5];
        const double vJ11 = g01 * JS[1] + g11 * JS[4];
        const double vJ12 = g01 * JS[2] + g11 * JS[5];
        if (xr <= lim_x_pos && xr >= -lim_x_neg)
            vmc[0] += -fx * rz2 * vJ02;
        else
            vmc[2] += -fx * rz3 * vJ02 * tx;
        if (yr <= lim_y_pos && yr >= -lim_y_neg)
            vmc[1] += -fy * rz2 * vJ12;
        else
            vmc[2] += -fy * rz3 * vJ12 * ty;
        vmc[2] += -fx * rz2 * vJ00 - fy * rz2 * vJ11 +
                  2.0 * fx * tx * rz3 * vJ02 + 2.0 * fy * ty * rz3 * vJ12;
    }
    // v_Sc = J^T G J (symmetric)
    Sym3d vSc;
    {
        double GJ[6];  // G (2x2) * J (2x3)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            GJ[0 * 3 + c] = vc00 * J[c] + vc01 * J[3 + c];
            GJ[1 * 3 + c] = vc01 * J[c] + vc11 * J[3 + c];
        }
        int k = 0;
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = i; j < 3; ++j)
                vSc.v[k++] = J[0 * 3 + i] * GJ[0 * 3 + j] + J[1 * 3 + i] * GJ[1 * 3 + j];
    }
    vmc[2] += (double)v_depth_f;

    // mean: mc = R p + t
#pragma unroll
    for (int j = 0; j < 3; ++j)
        v_mean[j] += R(0, j) * vmc[0] + R(1, j) * vmc[1] + R(2, j) * vmc[2];
    // covariance: Sc = R S R^T  ->  dS = R^T dSc R
    const Sym3d dS = congruence(Rt, vSc);
#pragma unroll
    for (int k = 0; k < 6; ++k)
        v_S.v[k] += dS.v[k];
    if (want_cam) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
#pragma unroll
            for (int j = 0; j < 3; ++j)
                v_R.m[i * 3 + j] += vmc[i] * p[j];
            v_t[i] += vmc[i];
        }
        // dR = dSc R S^T + dSc^T R S = 2 dSc R S (both symmetric)
        double RS[9];
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                RS[i * 3 + j] = R(i, 0) * G.S.at(0, j) + R(i, 1) * G.S.at(1, j) +
                                R(i, 2) * G.S.at(2, j);
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                v_R.m[i * 3 + j] += 2.0 * (vSc.at(i, 0) * RS[0 * 3 + j] +
                                           vSc.at(i, 1) * RS[1 * 3 + j] +
                                           vSc.at(i, 2) * RS[2 * 3 + j]);
    }
}

// dL/dS (symmetric) -> dL/dquat, dL/dscale  (quat_scale_to_covar_vjp +
// quat_to_rotmat_vjp, Utils.cuh:197-296), for the Gaussian (q, s).
__device__ __forceinline__ void covar_vjp_to_quat_scale(const float qf[4],
                                                        const double s[3],
                                                        const Sym3d &v_S,
                                                        double v_q[4],
                                                        double v_s[3]) {
    double Rq[9];
    quat_to_rot_d(qf, Rq);
    // S = M M^T with M = Rq diag(s):  dM = (dS + dS^T) M = 2 dS M
    double vM[9];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k)
            vM[i * 3 + k] = 2.0 * s[k] * (v_S.at(i, 0) * Rq[0 * 3 + k] +
                                          v_S.at(i, 1) * Rq[1 * 3 + k] +
                                          v_S.at(i, 2) * Rq[2 * 3 + k]);
    // ds_k = sum_i Rq[i][k] dM[i][k];  dRq = dM diag(s)
#pragma unroll
    for (int k = 0; k < 3; ++k)
        v_s[k] = Rq[0 * 3 + k] * vM[0 * 3 + k] + Rq[1 * 3 + k] * vM[1 * 3 + k] +
                 Rq[2 * 3 + k] * vM[2 * 3 + k];
    double m[9];  // m[r*3+c] = dL/dRq[r][c]
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int k = 0; k < 3; ++k)
            m[i * 3 + k] = vM[i * 3 + k] * s[k];
    // rotation-matrix VJP w.r.t. the normalised quaternion (w, x, y, z)
    const double q0 = qf[0], q1 = qf[1], q2 = qf[2], q3 = qf[3];
    const double inv = 1.0 / sqrt(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    const double w = q0 * inv, x = q1 * inv, y = q2 * inv, z = q3 * inv;
    const double dw = 2.0 * (x * (m[7] - m[5]) + y * (m[2] - m[6]) +
                             z * (m[3] - m[1]));
    const double dx = 2.0 * (-2.0 * x * (m[4] + m[8]) + y * (m[1] + m[3]) +
                             z * (m[2] + m[6]) + w * (m[7] - m[5]));
    const double dy = 2.0 * (x * (m[1] + m[3]) - 2.0 * y * (m[0] + m[8]) +
                             z * (m[5] + m[7]) + w * (m[2] - m[6]));
    const double dz = 2.0 * (x * (m[2] + m[6]) + y * (m[5] + m[7]) -
                             2.0 * z * (m[0] + m[4]) + w * (m[3] - m[1]));
    const double dot = dw * w + dx * x + dy * y + dz * z;
    v_q[0] = (dw - dot * w) * inv;
    v_q[1] = (dx - dot * x) * inv;
    v_q[2] = (dy - dot * y) * inv;
    v_q[3] = (dz - dot * z) * inv;
}

// dL/dS (symmetric) as the gradient of the triu covars input: each
// off-diagonal entry stands for both of its places.
__device__ __forceinline__ void covar6_grad(const Sym3d &v_S, float out[6]) {
    out[0] = (float)v_S.v[0];
    out[1] = (float)(2.0 * v_S.v[1]);
    out[2] = (float)(2.0 * v_S.v[2]);
    out[3] = (float)v_S.v[3];
    out[4] = (float)(2.0 * v_S.v[4]);
    out[5] = (float)v_S.v[5];
}

struct BwdArgs {
    int64_t B, C, N;
    const float *means, *covars, *quats, *scales, *viewmats, *Ks;
    float W, H, eps2d;
    int camera_model;
    const float *conics, *compensations;
    const float *v_means2d, *v_depths, *v_conics, *v_compensations;
    float *v_means, *v_covars, *v_quats, *v_scales, *v_viewmats;
    // packed rows only (all nullable): per-row opacity gradients summed into
    // v_opacities[b, g], and a dense [B, N, 3] term added to v_means
    const float *v_row_opacities;
    float *v_opacities;
    const float *v_means_add;
    // densification statistics (B == 1): per packed row,
    // grad2d[g] += ||(stat_grads[row] * (stat_sx, stat_sy))||, count[g] += 1
    const float *stat_grads;
    float stat_sx, stat_sy;
    float *grad2d, *count;
};

// Reduce v_R (9) and v_t (3) of the workgroup and add them to the camera's
// viewmat gradient.  Must be reached by every thread of the block.
__device__ __forceinline__ void flush_viewmat_grad(float *v_viewmat,
                                                   const M3d &v_R,
                                                   const double v_t[3],
                                                   float *s_red) {
    const uint32_t wave = threadIdx.x / kWave;
    float vals[12];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
            vals[i * 4 + j] = (float)v_R.m[i * 3 + j];
        vals[i * 4 + 3] = (float)v_t[i];
    }
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        const float s = wave_sum(vals[k]);
        if (lane_id() == 0)
            s_red[wave * 12 + k] = s;
    }
    __syncthreads();
    if (threadIdx.x < 12) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < kProjThreads / kWave; ++w)
            acc += s_red[w * 12 + threadIdx.x];
        atomic_add_f32(v_viewmat + threadIdx.x, acc);
    }
    __syncthreads();
}

// One thread per (b, g) of workgroup `blk`; loops over the C cameras.  The
// rows are the dense (b, c, g) rows (visible when both radii are positive)
// or, with row_of, the packed rows row_of[(b C + c) N + g] (visible when
// >= 0).  vm_add (three floats per thread, or NULL) is added to v_means
// like a.v_means_add.
template <bool kWantCam>
__device__ __forceinline__ void projection_bwd_gaussian(
    const BwdArgs &a, const int32_t *__restrict__ radii,
    const int32_t *__restrict__ row_of, int64_t blk, const float *vm_add,
    float *s_red) {
    const int64_t bg = blk * kProjThreads + threadIdx.x;
    const bool in_range = bg < a.B * a.N;
    const int64_t b = in_range ? bg / a.N : 0;
    const int64_t g = in_range ? bg % a.N : 0;

    // the geometry is only read for Gaussians visible in some camera
    bool seen = false;
    if (in_range) {
        for (int64_t c = 0; c < a.C && !seen; ++c) {
            const int64_t row = (b * a.C + c) * a.N + g;
            if (row_of != nullptr) {
                seen = row_of[row] >= 0;
            } else {
                const int2 r = reinterpret_cast<const int2 *>(radii)[row];
                seen = r.x > 0 && r.y > 0;
            }
        }
    }
    GaussGeom G;
    if (seen)
        load_geom(a.covars ? a.covars + bg * 6 : nullptr,
                  a.quats ? a.quats + bg * 4 : nullptr,
                  a.scales ? a.scales + bg * 3 : nullptr, G);
    double v_mean[3] = {0.0, 0.0, 0.0};
    float v_op = 0.f;
    float stat_norm = 0.f, stat_rows = 0.f;
    Sym3d v_S;
#pragma unroll
    for (int i = 0; i < 6; ++i)
        v_S.v[i] = 0.0;
    constexpr bool want_cam = kWantCam;

    // b is not uniform across the block when N is small; the camera loop is
    // over C for every thread, and the viewmat flush is done per (b, c) by
    // the threads that share that b (per-lane atomics when mixed).
    for (int64_t c = 0; c < a.C; ++c) {
        M3d v_R;
        double v_t[3] = {0.0, 0.0, 0.0};
#pragma unroll
        for (int i = 0; i < 9; ++i)
            v_R.m[i] = 0.0;
        bool active = false;
        int64_t bc = b * a.C + c;
        if (seen) {
            int64_t row = bc * a.N + g;
            if (row_of != nullptr) {
                row = row_of[row];
                active = row >= 0;
            } else {
                const int2 r = reinterpret_cast<const int2 *>(radii)[row];
                active = r.x > 0 && r.y > 0;
            }
            if (active) {
                if (a.v_row_opacities != nullptr)
                    v_op += a.v_row_opacities[row];
                if (a.stat_grads != nullptr) {
                    const float sx = a.stat_grads[row * 2] * a.stat_sx;
                    const float sy = a.stat_grads[row * 2 + 1] * a.stat_sy;
                    stat_norm += sqrtf(sx * sx + sy * sy);
                    stat_rows += 1.f;
                }
                Cam cam;
                load_cam(a.viewmats + bc * 16, a.Ks + bc * 9, cam);
                const bool has_comp = a.v_compensations != nullptr;
                project_row_vjp(
                    cam, a.means + bg * 3, G, a.camera_model, a.W, a.H, a.eps2d,
                    a.conics + row * 3, has_comp,
                    has_comp ? a.compensations[row] : 0.f,
                    has_comp ? a.v_compensations[row] : 0.f,
                    a.v_means2d[row * 2], a.v_means2d[row * 2 + 1],
                    a.v_depths != nullptr ? a.v_depths[row] : 0.f,
                    a.v_conics + row * 3, v_mean, v_S, want_cam, v_R, v_t);
            }
        }
        if (want_cam) {
            // b is uniform over the block unless the block straddles two
            // batches (only when N is not a multiple of the block size).
            const int64_t first = blk * kProjThreads;
            const int64_t last_row = first + kProjThreads - 1 < a.B * a.N - 1
                                         ? first + kProjThreads - 1
                                         : a.B * a.N - 1;
            const int64_t b0 = first / a.N;
            if (b0 == last_row / a.N) {
                flush_viewmat_grad(a.v_viewmats + (b0 * a.C + c) * 16, v_R,
                                   v_t, s_red);
            } else if (active) {
                float *dst = a.v_viewmats + bc * 16;
#pragma unroll
                for (int i = 0; i < 3; ++i) {
#pragma unroll
                    for (int j = 0; j < 3; ++j)
                        atomic_add_f32(dst + i * 4 + j, (float)v_R.m[i * 3 + j]);
                    atomic_add_f32(dst + i * 4 + 3, (float)v_t[i]);
                }
            }
        }
    }
    if (!in_range)
        return;
    if (a.v_means != nullptr) {
        // rounded to float32 before the added term: the sum autograd forms
        // when the two gradients of the means come from separate nodes
        float vm[3] = {(float)v_mean[0], (float)v_mean[1], (float)v_mean[2]};
        if (vm_add != nullptr) {
#pragma unroll
            for (int k = 0; k < 3; ++k)
                vm[k] += vm_add[k];
        } else if (a.v_means_add != nullptr) {
#pragma unroll
            for (int k = 0; k < 3; ++k)
                vm[k] += a.v_means_add[bg * 3 + k];
        }
        a.v_means[bg * 3 + 0] = vm[0];
        a.v_means[bg * 3 + 1] = vm[1];
        a.v_means[bg * 3 + 2] = vm[2];
    }
    if (a.v_opacities != nullptr)
        a.v_opacities[bg] = v_op;
    if (a.grad2d != nullptr && stat_rows > 0.f) {
        a.grad2d[bg] += stat_norm;
        a.count[bg] += stat_rows;
    }
    if (!seen) {
        // visible in no camera: zero gradient rows
        if (a.covars != nullptr) {
            if (a.v_covars != nullptr)
                for (int k = 0; k < 6; ++k)
                    a.v_covars[bg * 6 + k] = 0.f;
        } else {
            if (a.v_quats != nullptr)
                reinterpret_cast<float4 *>(a.v_quats)[bg] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (a.v_scales != nullptr)
                for (int k = 0; k < 3; ++k)
                    a.v_scales[bg * 3 + k] = 0.f;
        }
        return;
    }
    if (a.covars != nullptr) {
        if (a.v_covars != nullptr) {
            covar6_grad(v_S, a.v_covars + bg * 6);
        }
    } else {
        double v_q[4], v_s[3];
        const double sd[3] = {G.s[0], G.s[1], G.s[2]};
        covar_vjp_to_quat_scale(G.q, sd, v_S, v_q, v_s);
        if (a.v_quats != nullptr)
            reinterpret_cast<float4 *>(a.v_quats)[bg] =
                make_float4((float)v_q[0], (float)v_q[1], (float)v_q[2], (float)v_q[3]);
        if (a.v_scales != nullptr) {
            a.v_scales[bg * 3 + 0] = (float)v_s[0];
            a.v_scales[bg * 3 + 1] = (float)v_s[1];
            a.v_scales[bg * 3 + 2] = (float)v_s[2];
        }
    }
}

template <bool kWantCam>
__global__ void __launch_bounds__(kProjThreads)
    projection_fused_bwd_kernel(const BwdArgs a, const int32_t *__restrict__ radii,
                                const int32_t *__restrict__ row_of) {
    __shared__ float s_red[(kProjThreads / kWave) * 12];
    projection_bwd_gaussian<kWantCam>(a, radii, row_of, blockIdx.x, nullptr, s_red);
}

// The packed path's backward through the row map with the SH colours' in the
// same launch: each workgroup first runs the SH backward of its 256
// Gaussians (coalesced coefficient tiles through LDS, dense v_coeffs rows),
// which keeps each thread's direction term of dL/dmean in registers, then
// their geometry backward, which adds that term.  Workgroups in the
// memory-bound SH part and in the latency-bound double-precision part share
// the CUs, and the direction term makes no round trip through memory.
static_assert(kProjThreads == kShThreads, "one workgroup shape for both parts");

template <int DEG>
__global__ void __launch_bounds__(kProjThreads)
    sh_projection_bwd_kernel(const BwdArgs a, const ShRowsArgs sa,
                             const float *__restrict__ v_colors,
                             float *__restrict__ v_coeffs,
                             const int32_t *__restrict__ row_of) {
    float vm[3];
    sh_rows_bwd_block<DEG>(sa, v_colors, v_coeffs, (int64_t)blockIdx.x * kShThreads, vm);
    projection_bwd_gaussian<false>(a, nullptr, row_of, blockIdx.x, vm, nullptr);
}

__global__ void __launch_bounds__(kProjThreads) projection_packed_bwd_kernel(
    const BwdArgs a, int64_t nnz, const int64_t *__restrict__ batch_ids,
    const int64_t *__restrict__ camera_ids,
    const int64_t *__restrict__ gaussian_ids, int sparse_grad,
    int single_image) {
    __shared__ float s_red[(kProjThreads / kWave) * 12];
    const int64_t i = (int64_t)blockIdx.x * kProjThreads + threadIdx.x;
    const bool active = i < nnz;
    const bool want_cam = a.v_viewmats != nullptr;
    double v_mean[3] = {0.0, 0.0, 0.0};
    Sym3d v_S;
    M3d v_R;
    double v_t[3] = {0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < 9; ++k)
        v_R.m[k] = 0.0;
#pragma unroll
    for (int k = 0; k < 6; ++k)
        v_S.v[k] = 0.0;
    int64_t b = 0, c = 0, g = 0;
    GaussGeom G;
    if (active) {
        b = batch_ids[i];
        c = camera_ids[i];
        g = gaussian_ids[i];
        const int64_t bg = b * a.N + g;
        const int64_t bc = b * a.C + c;
        load_geom(a.covars ? a.covars + bg * 6 : nullptr,
                  a.quats ? a.quats + bg * 4 : nullptr,
                  a.scales ? a.scales + bg * 3 : nullptr, G);
        Cam cam;
        load_cam(a.viewmats + bc * 16, a.Ks + bc * 9, cam);
        const bool has_comp = a.v_compensations != nullptr;
        project_row_vjp(cam, a.means + bg * 3, G, a.camera_model, a.W, a.H,
                        a.eps2d, a.conics + i * 3, has_comp,
                        has_comp ? a.compensations[i] : 0.f,
                        has_comp ? a.v_compensations[i] : 0.f,
                        a.v_means2d[i * 2], a.v_means2d[i * 2 + 1],
                        a.v_depths[i], a.v_conics + i * 3, v_mean, v_S,
                        want_cam, v_R, v_t);
    }
    if (want_cam) {
        // rows are sorted by (b, c): the block usually sees one camera
        const int64_t bc = b * a.C + c;
        const int64_t first = (int64_t)blockIdx.x * kProjThreads;
        const int64_t bc0 = batch_ids[first] * a.C + camera_ids[first];
        const bool uniform = __syncthreads_and(!active || bc == bc0);
        if (uniform) {
            flush_viewmat_grad(a.v_viewmats + bc0 * 16, v_R, v_t, s_red);
        } else if (active) {
            float *dst = a.v_viewmats + bc * 16;
#pragma unroll
            for (int r = 0; r < 3; ++r) {
#pragma unroll
                for (int k = 0; k < 3; ++k)
                    atomic_add_f32(dst + r * 4 + k, (float)v_R.m[r * 3 + k]);
                atomic_add_f32(dst + r * 4 + 3, (float)v_t[r]);
            }
        }
    }
    if (!active)
        return;
    float v_q[4] = {0.f, 0.f, 0.f, 0.f}, v_s[3] = {0.f, 0.f, 0.f};
    float v_c6[6];
    if (a.covars != nullptr) {
        covar6_grad(v_S, v_c6);
    } else {
        double q4[4], s3[3];
        const double sd[3] = {G.s[0], G.s[1], G.s[2]};
        covar_vjp_to_quat_scale(G.q, sd, v_S, q4, s3);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v_q[k] = (float)q4[k];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            v_s[k] = (float)s3[k];
    }
    float v_meanf[3] = {(float)v_mean[0], (float)v_mean[1], (float)v_mean[2]};
    const bool direct = sparse_grad || single_image;
    const int64_t dst = sparse_grad ? i : b * a.N + g;
    if (direct) {
        if (a.v_means) {
            a.v_means[dst * 3 + 0] = v_meanf[0];
            a.v_means[dst * 3 + 1] = v_meanf[1];
            a.v_means[dst * 3 + 2] = v_meanf[2];
        }
        if (a.covars != nullptr) {
            if (a.v_covars)
                for (int k = 0; k < 6; ++k)
                    a.v_covars[dst * 6 + k] = v_c6[k];
        } else {
            if (a.v_quats)
                reinterpret_cast<float4 *>(a.v_quats)[dst] =
                    make_float4(v_q[0], v_q[1], v_q[2], v_q[3]);
            if (a.v_scales)
                for (int k = 0; k < 3; ++k)
                    a.v_scales[dst * 3 + k] = v_s[k];
        }
    } else {
        if (a.v_means)
            for (int k = 0; k < 3; ++k)
                atomic_add_f32(a.v_means + dst * 3 + k, v_meanf[k]);
        if (a.covars != nullptr) {
            if (a.v_covars)
                for (int k = 0; k < 6; ++k)
                    atomic_add_f32(a.v_covars + dst * 6 + k, v_c6[k]);
        } else {
            if (a.v_quats)
                for (int k = 0; k < 4; ++k)
                    atomic_add_f32(a.v_quats + dst * 4 + k, v_q[k]);
            if (a.v_scales)
                for (int k = 0; k < 3; ++k)
                    atomic_add_f32(a.v_scales + dst * 3 + k, v_s[k]);
        }
    }
}

int check_common(int64_t B, int64_t C, int64_t N, const float *means,
                 const float *covars, const float *quats, const float *scales,
                 const float *viewmats, const float *Ks, int32_t W, int32_t H,
                 int32_t camera_model) {
    GS_REQUIRE(B >= 0 && C >= 0 && N >= 0, "projection: negative size");
    GS_REQUIRE(camera_model == GSPLAT_CAMERA_PINHOLE ||
                   camera_model == GSPLAT_CAMERA_ORTHO,
               "projection: only the pinhole and ortho camera models are "
               "implemented");
    GS_REQUIRE(W > 0 && H > 0, "projection: image size must be positive");
    if (B * C * N > 0) {
        GS_REQUIRE(means && viewmats && Ks, "projection: NULL input");
        GS_REQUIRE(covars != nullptr || (quats != nullptr && scales != nullptr),
                   "projection: covars or (quats, scales) required");
    }
    return GSPLAT_OK;
}


// ---------------------------------------------------------------------------
// Covariance / precision from quaternion and scale
//   (quat_scale_to_covar_preci_fwd/bwd, QuatScaleToCovarCUDA.cu:37-236,
//    Utils.cuh:223-340).  Covariance R diag(s)^2 R^T, precision
//   R diag(1/s)^2 R^T; triu layout (xx, xy, xz, yy, yz, zz), else row-major
//   3x3.  One thread per Gaussian.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void write_sym(const M3 &S, bool triu, float *out) {
    if (triu) {
        out[0] = S.m[0]; out[1] = S.m[1]; out[2] = S.m[2];
        out[3] = S.m[4]; out[4] = S.m[5]; out[5] = S.m[8];
    } else {
#pragma unroll
        for (int i = 0; i < 9; ++i)
            out[i] = S.m[i];
    }
}

// dL/dS as a full matrix: triu entries cover both off-diagonal places, so
// each place gets half of the entry's gradient.
// (A full 3x3 gradient enters through its symmetric part: the covariance
// is symmetric.)
__device__ __forceinline__ Sym3d read_sym_grad(const float *g, bool triu) {
    Sym3d v;
    if (triu) {
        v.v[0] = g[0];       v.v[1] = 0.5 * g[1]; v.v[2] = 0.5 * g[2];
        v.v[3] = g[3];       v.v[4] = 0.5 * g[4]; v.v[5] = g[5];
    } else {
        v.v[0] = g[0];
        v.v[1] = 0.5 * ((double)g[1] + g[3]);
        v.v[2] = 0.5 * ((double)g[2] + g[6]);
        v.v[3] = g[4];
        v.v[4] = 0.5 * ((double)g[5] + g[7]);
        v.v[5] = g[8];
    }
    return v;
}

__global__ void __launch_bounds__(kProjThreads)
    covar_preci_fwd_kernel(int64_t N, const float *__restrict__ quats,
                           const float *__restrict__ scales, bool triu,
                           float *__restrict__ covars, float *__restrict__ precis) {
    const int64_t i = (int64_t)blockIdx.x * kProjThreads + threadIdx.x;
    if (i >= N)
        return;
    const int osz = triu ? 6 : 9;
    M3 R;
    quat_to_rot_exact(quats[i * 4 + 0], quats[i * 4 + 1], quats[i * 4 + 2],
                      quats[i * 4 + 3], R.m);
    const float s[3] = {scales[i * 3 + 0], scales[i * 3 + 1], scales[i * 3 + 2]};
    if (covars != nullptr) {
        M3 A;
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k)
                A.m[r * 3 + k] = R.m[r * 3 + k] * s[k];
        write_sym(mmt(A, A), triu, covars + i * osz);
    }
    if (precis != nullptr) {
        M3 A;
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k)
                A.m[r * 3 + k] = R.m[r * 3 + k] * (1.f / s[k]);
        write_sym(mmt(A, A), triu, precis + i * osz);
    }
}

__global__ void __launch_bounds__(kProjThreads)
    covar_preci_bwd_kernel(int64_t N, const float *__restrict__ quats,
                           const float *__restrict__ scales, bool triu,
                           const float *__restrict__ v_covars,
                           const float *__restrict__ v_precis,
                           float *__restrict__ v_quats, float *__restrict__ v_scales) {
    const int64_t i = (int64_t)blockIdx.x * kProjThreads + threadIdx.x;
    if (i >= N)
        return;
    const int osz = triu ? 6 : 9;
    float q[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        q[k] = quats[i * 4 + k];
    double sd[3];
#pragma unroll
    for (int k = 0; k < 3; ++k)
        sd[k] = scales[i * 3 + k];
    double vq[4] = {0.0, 0.0, 0.0, 0.0}, vs[3] = {0.0, 0.0, 0.0};
    if (v_covars != nullptr) {
        double gq[4], gs3[3];
        covar_vjp_to_quat_scale(q, sd, read_sym_grad(v_covars + i * osz, triu), gq, gs3);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            vq[k] += gq[k];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            vs[k] += gs3[k];
    }
    if (v_precis != nullptr) {
        // the precision is the covariance of scales 1/s: chain through
        // d(1/s)/ds = -1/s^2
        double inv_s[3];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            inv_s[k] = 1.0 / sd[k];
        double gq[4], gs3[3];
        covar_vjp_to_quat_scale(q, inv_s, read_sym_grad(v_precis + i * osz, triu), gq, gs3);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            vq[k] += gq[k];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            vs[k] += -(inv_s[k] * inv_s[k]) * gs3[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v_quats[i * 4 + k] = (float)vq[k];
#pragma unroll
    for (int k = 0; k < 3; ++k)
        v_scales[i * 3 + k] = (float)vs[k];
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gsplat_projection_fused_fwd(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *opacities,
    const float *viewmats, const float *Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane,
    float radius_clip, int32_t camera_model, int32_t *radii, float *means2d,
    float *depths, float *conics, float *compensations,
    gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    const int64_t rows = B * C * N;
    if (rows == 0)
        return GSPLAT_OK;
    GS_REQUIRE(radii && means2d && depths && conics, "projection: NULL output");
    FwdArgs a{B, C, N, means, covars, quats, scales, opacities, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, near_plane,
              far_plane, radius_clip, camera_model, compensations != nullptr,
              rows < (int64_t(1) << 31)};
    projection_fused_fwd_kernel<<<(unsigned)ceil_div(rows, kProjThreads),
                                  kProjThreads, 0, as_stream(stream)>>>(
        a, radii, means2d, depths, conics, compensations);
    return check_launch("projection_fused_fwd_kernel");
}

extern "C" size_t gsplat_projection_packed_workspace_size(int64_t B, int64_t C,
                                                          int64_t N) {
    return lookback_bytes(ceil_div(B * C * N, kPackRows));
}

namespace gs {
namespace {

// The packed forward over a caller-checked look-back workspace of at least
// lookback_bytes(ceil(B*C*N / kPackRows)) bytes.
int packed_fwd_launch(int64_t B, int64_t C, int64_t N, const float *means,
                      const float *covars, const float *quats, const float *scales,
                      const float *opacities, const float *viewmats, const float *Ks,
                      int32_t image_width, int32_t image_height, float eps2d,
                      float near_plane, float far_plane, float radius_clip,
                      int32_t camera_model, void *workspace, int32_t *indptr,
                      int64_t *batch_ids, int64_t *camera_ids, int64_t *gaussian_ids,
                      int32_t *radii, float *means2d, float *depths, float *conics,
                      float *compensations, int64_t *nnz_out, int32_t *row_of,
                      float *row_opacities, hipStream_t st) {
    const int64_t rows = B * C * N;
    const int64_t blocks = ceil_div(rows, kPackRows);
    GS_TRY(clear_lookback(workspace, blocks, st));
    FwdArgs a{B, C, N, means, covars, quats, scales, opacities, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, near_plane,
              far_plane, radius_clip, camera_model, compensations != nullptr,
              rows < (int64_t(1) << 31)};
    if (covars != nullptr)
        projection_packed_fwd_kernel<true><<<(unsigned)blocks, kPackThreads, 0, st>>>(
            a, lookback_from(workspace), indptr, batch_ids, camera_ids,
            gaussian_ids, radii, means2d, depths, conics, compensations,
            nnz_out, row_of, row_opacities);
    else
        projection_packed_fwd_kernel<false><<<(unsigned)blocks, kPackThreads, 0, st>>>(
            a, lookback_from(workspace), indptr, batch_ids, camera_ids,
            gaussian_ids, radii, means2d, depths, conics, compensations,
            nnz_out, row_of, row_opacities);
    return check_launch("projection_packed_fwd_kernel");
}

int check_packed_fwd(int64_t B, int64_t C, int64_t N, const float *means,
                     const float *covars, const float *quats, const float *scales,
                     const float *opacities, const float *viewmats, const float *Ks,
                     int32_t image_width, int32_t image_height, int32_t camera_model,
                     int32_t *indptr, int64_t *batch_ids, int64_t *camera_ids,
                     int64_t *gaussian_ids, int32_t *radii, float *means2d,
                     float *depths, float *conics, int64_t *nnz_out,
                     float *row_opacities) {
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    const int64_t rows = B * C * N;
    GS_REQUIRE(indptr && nnz_out, "projection_packed: NULL indptr/nnz_out");
    if (rows == 0)
        return fail(GSPLAT_ERR_INVALID_ARGUMENT,
                    "projection_packed: zero rows must be handled by the caller");
    GS_REQUIRE(batch_ids && camera_ids && gaussian_ids && radii && means2d &&
                   depths && conics,
               "projection_packed: NULL output");
    GS_REQUIRE(rows < (1ll << 31), "projection_packed: more than 2^31 rows");
    GS_REQUIRE(row_opacities == nullptr || opacities != nullptr,
               "projection_packed: row opacities need opacities");
    return GSPLAT_OK;
}

// Scratch of the allocation-free packed forward: the look-back ticket and
// status words of up to kNoAllocMaxBlocks workgroups (kPackRows rows each).
// Each device holds its own copy for the life of the process; host code
// reaches it only through the address hipGetSymbolAddress returns on that
// device (the symbol's name is a host-side stand-in).
constexpr int64_t kNoAllocMaxBlocks = int64_t(1) << 16;
constexpr size_t kNoAllocScratchBytes = 256 + size_t(kNoAllocMaxBlocks) * sizeof(uint64_t);

}  // namespace

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the current device, looked up once per device.
int device_scratch(void **out) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess)
        return fail(GSPLAT_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(err));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(GSPLAT_ERR_UNSUPPORTED, "projection_packed_fwd_noalloc: device index " +
                                                std::to_string(dev) + " out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || p == nullptr)
            return fail(GSPLAT_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") +
                                               hipGetErrorString(err));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GSPLAT_OK;
}

}  // namespace
}  // namespace gs

extern "C" int gsplat_projection_packed_fwd(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *opacities,
    const float *viewmats, const float *Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane,
    float radius_clip, int32_t camera_model, void *workspace,
    size_t workspace_bytes, int32_t *indptr, int64_t *batch_ids,
    int64_t *camera_ids, int64_t *gaussian_ids, int32_t *radii,
    float *means2d, float *depths, float *conics, float *compensations,
    int64_t *nnz_out, int32_t *row_of, float *row_opacities,
    gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_packed_fwd(B, C, N, means, covars, quats, scales, opacities, viewmats,
                            Ks, image_width, image_height, camera_model, indptr,
                            batch_ids, camera_ids, gaussian_ids, radii, means2d, depths,
                            conics, nnz_out, row_opacities));
    const int64_t blocks = ceil_div(B * C * N, kPackRows);
    GS_REQUIRE(workspace != nullptr && workspace_bytes >= lookback_bytes(blocks),
               "projection_packed: workspace too small");
    return packed_fwd_launch(B, C, N, means, covars, quats, scales, opacities, viewmats,
                             Ks, image_width, image_height, eps2d, near_plane, far_plane,
                             radius_clip, camera_model, workspace, indptr, batch_ids,
                             camera_ids, gaussian_ids, radii, means2d, depths, conics,
                             compensations, nnz_out, row_of, row_opacities,
                             as_stream(stream));
}

extern "C" int64_t gsplat_projection_packed_fwd_noalloc_max_rows(void) {
    return kNoAllocMaxBlocks * kPackRows;
}

extern "C" int gsplat_projection_packed_fwd_noalloc(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *opacities,
    const float *viewmats, const float *Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane,
    float radius_clip, int32_t camera_model, int32_t *indptr, int64_t *batch_ids,
    int64_t *camera_ids, int64_t *gaussian_ids, int32_t *radii, float *means2d,
    float *depths, float *conics, float *compensations, int64_t *nnz_out,
    int32_t *row_of, float *row_opacities, gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_packed_fwd(B, C, N, means, covars, quats, scales, opacities, viewmats,
                            Ks, image_width, image_height, camera_model, indptr,
                            batch_ids, camera_ids, gaussian_ids, radii, means2d, depths,
                            conics, nnz_out, row_opacities));
    const int64_t blocks = ceil_div(B * C * N, kPackRows);
    if (blocks > kNoAllocMaxBlocks)
        return fail(GSPLAT_ERR_WORKSPACE,
                    "projection_packed_fwd_noalloc: " + std::to_string(B * C * N) +
                        " rows exceed the static scratch's limit of " +
                        std::to_string(kNoAllocMaxBlocks * kPackRows) + " rows");
    void *ws = nullptr;
    GS_TRY(device_scratch(&ws));
    return packed_fwd_launch(B, C, N, means, covars, quats, scales, opacities, viewmats,
                             Ks, image_width, image_height, eps2d, near_plane, far_plane,
                             radius_clip, camera_model, ws, indptr, batch_ids, camera_ids,
                             gaussian_ids, radii, means2d, depths, conics, compensations,
                             nnz_out, row_of, row_opacities, as_stream(stream));
}

extern "C" int gsplat_projection_fused_bwd(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats,
    const float *Ks, int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *radii, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, float *v_means,
    float *v_covars, float *v_quats, float *v_scales, float *v_viewmats,
    gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    if (B * N == 0)
        return GSPLAT_OK;
    GS_REQUIRE(radii && conics && v_means2d && v_depths && v_conics && v_means,
               "projection_fused_bwd: NULL buffer");
    GS_REQUIRE(v_compensations == nullptr || compensations != nullptr,
               "projection_fused_bwd: v_compensations needs compensations");
    if (covars == nullptr)
        GS_REQUIRE(v_quats && v_scales,
                   "projection_fused_bwd: v_quats/v_scales required");
    BwdArgs a{B, C, N, means, covars, quats, scales, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, camera_model,
              conics, compensations, v_means2d, v_depths, v_conics,
              v_compensations, v_means, v_covars, v_quats, v_scales,
              v_viewmats};
    auto kernel = v_viewmats != nullptr ? projection_fused_bwd_kernel<true>
                                        : projection_fused_bwd_kernel<false>;
    kernel<<<(unsigned)ceil_div(B * N, kProjThreads), kProjThreads, 0,
             as_stream(stream)>>>(a, radii, nullptr);
    return check_launch("projection_fused_bwd_kernel");
}

namespace gs {
namespace {

int packed_bwd_rows_launch(const BwdArgs &a, const int32_t *row_of, hipStream_t st) {
    GS_REQUIRE((a.v_row_opacities == nullptr) == (a.v_opacities == nullptr),
               "projection_packed_bwd_rows: v_row_opacities and v_opacities go together");
    GS_REQUIRE(a.v_means_add == nullptr || a.v_means != nullptr,
               "projection_packed_bwd_rows: v_means_add needs v_means");
    GS_REQUIRE(row_of && a.conics && a.v_means2d && a.v_conics,
               "projection_packed_bwd_rows: NULL buffer");
    GS_REQUIRE(a.v_compensations == nullptr || a.compensations != nullptr,
               "projection_packed_bwd_rows: v_compensations needs compensations");
    auto kernel = a.v_viewmats != nullptr ? projection_fused_bwd_kernel<true>
                                          : projection_fused_bwd_kernel<false>;
    kernel<<<(unsigned)ceil_div(a.B * a.N, kProjThreads), kProjThreads, 0, st>>>(
        a, nullptr, row_of);
    return check_launch("projection_fused_bwd_kernel");
}

}  // namespace
}  // namespace gs

extern "C" int gsplat_projection_packed_bwd_rows(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats,
    const float *Ks, int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *row_of, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, float *v_means,
    float *v_covars, float *v_quats, float *v_scales, float *v_viewmats,
    const float *v_row_opacities, float *v_opacities, const float *v_means_add,
    gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    if (B * N == 0)
        return GSPLAT_OK;
    BwdArgs a{B, C, N, means, covars, quats, scales, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, camera_model,
              conics, compensations, v_means2d, v_depths, v_conics,
              v_compensations, v_means, v_covars, v_quats, v_scales,
              v_viewmats, v_row_opacities, v_opacities, v_means_add,
              nullptr, 0.f, 0.f, nullptr, nullptr};
    return packed_bwd_rows_launch(a, row_of, as_stream(stream));
}

extern "C" int gsplat_projection_packed_bwd_rows_stats(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats,
    const float *Ks, int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *row_of, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, float *v_means,
    float *v_covars, float *v_quats, float *v_scales, float *v_viewmats,
    const float *v_row_opacities, float *v_opacities, const float *v_means_add,
    const float *stat_grads, float stat_scale_x, float stat_scale_y, float *grad2d,
    float *count, gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    GS_REQUIRE(B == 1, "projection_packed_bwd_rows_stats: one batch only");
    GS_REQUIRE(stat_grads && grad2d && count,
               "projection_packed_bwd_rows_stats: NULL statistics buffer");
    if (B * N == 0)
        return GSPLAT_OK;
    BwdArgs a{B, C, N, means, covars, quats, scales, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, camera_model,
              conics, compensations, v_means2d, v_depths, v_conics,
              v_compensations, v_means, v_covars, v_quats, v_scales,
              v_viewmats, v_row_opacities, v_opacities, v_means_add,
              stat_grads, stat_scale_x, stat_scale_y, grad2d, count};
    return packed_bwd_rows_launch(a, row_of, as_stream(stream));
}

extern "C" int gsplat_projection_packed_bwd_rows_sh(
    int64_t B, int64_t C, int64_t N, const float *means, const float *covars,
    const float *quats, const float *scales, const float *viewmats,
    const float *Ks, int32_t image_width, int32_t image_height, float eps2d,
    int32_t camera_model, const int32_t *row_of, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, float *v_means,
    float *v_covars, float *v_quats, float *v_scales, const float *v_row_opacities,
    float *v_opacities, const float *stat_grads, float stat_scale_x,
    float stat_scale_y, float *grad2d, float *count, int32_t K, int32_t degree,
    const float *coeffs, const float *v_colors, float *v_coeffs,
    gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    const bool stats = stat_grads != nullptr || grad2d != nullptr || count != nullptr;
    if (stats) {
        GS_REQUIRE(stat_grads && grad2d && count,
                   "projection_packed_bwd_rows_sh: NULL statistics buffer");
        GS_REQUIRE(B == 1, "projection_packed_bwd_rows_sh: statistics for one batch only");
    }
    GS_REQUIRE(degree >= 0 && degree <= 4,
               "projection_packed_bwd_rows_sh: degree must be in [0, 4]");
    const int nb = (degree + 1) * (degree + 1);
    GS_REQUIRE(K >= nb, "projection_packed_bwd_rows_sh: K too small for the degree");
    if (B * N == 0)
        return GSPLAT_OK;
    GS_REQUIRE(v_means && coeffs && v_colors && v_coeffs,
               "projection_packed_bwd_rows_sh: NULL buffer");
    GS_REQUIRE((v_row_opacities == nullptr) == (v_opacities == nullptr),
               "projection_packed_bwd_rows_sh: v_row_opacities and v_opacities go together");
    GS_REQUIRE(row_of && conics && v_means2d && v_conics,
               "projection_packed_bwd_rows_sh: NULL buffer");
    GS_REQUIRE(v_compensations == nullptr || compensations != nullptr,
               "projection_packed_bwd_rows_sh: v_compensations needs compensations");
    BwdArgs a{B, C, N, means, covars, quats, scales, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, camera_model,
              conics, compensations, v_means2d, v_depths, v_conics,
              v_compensations, v_means, v_covars, v_quats, v_scales,
              nullptr, v_row_opacities, v_opacities, nullptr,
              stat_grads, stat_scale_x, stat_scale_y, grad2d, count};
    ShRowsArgs sa{B, C, N, K, means, viewmats, coeffs, row_of,
                  (K == nb) && aligned16(coeffs) && aligned16(v_coeffs)};
    const unsigned grid = (unsigned)ceil_div(B * N, kProjThreads);
    hipStream_t st = as_stream(stream);
#define GS_SHP(DEG)                                                            \
    sh_projection_bwd_kernel<DEG><<<grid, kProjThreads, 0, st>>>(a, sa, v_colors, \
                                                                v_coeffs, row_of)
    switch (degree) {
    case 0: GS_SHP(0); break;
    case 1: GS_SHP(1); break;
    case 2: GS_SHP(2); break;
    case 3: GS_SHP(3); break;
    default: GS_SHP(4); break;
    }
#undef GS_SHP
    return check_launch("sh_projection_bwd_kernel");
}

extern "C" int gsplat_projection_packed_bwd(
    int64_t B, int64_t C, int64_t N, int64_t nnz, const float *means,
    const float *covars, const float *quats, const float *scales,
    const float *viewmats, const float *Ks, int32_t image_width,
    int32_t image_height, float eps2d, int32_t camera_model,
    const int64_t *batch_ids, const int64_t *camera_ids,
    const int64_t *gaussian_ids, const float *conics,
    const float *compensations, const float *v_means2d, const float *v_depths,
    const float *v_conics, const float *v_compensations, int32_t sparse_grad,
    float *v_means, float *v_covars, float *v_quats, float *v_scales,
    float *v_viewmats, gsplat_stream_t stream) {
    clear_error();
    GS_TRY(check_common(B, C, N, means, covars, quats, scales, viewmats, Ks,
                        image_width, image_height, camera_model));
    GS_REQUIRE(nnz >= 0, "projection_packed_bwd: negative nnz");
    if (nnz == 0)
        return GSPLAT_OK;
    GS_REQUIRE(batch_ids && camera_ids && gaussian_ids && conics && v_means2d &&
                   v_depths && v_conics,
               "projection_packed_bwd: NULL buffer");
    GS_REQUIRE(v_compensations == nullptr || compensations != nullptr,
               "projection_packed_bwd: v_compensations needs compensations");
    BwdArgs a{B, C, N, means, covars, quats, scales, viewmats, Ks,
              (float)image_width, (float)image_height, eps2d, camera_model,
              conics, compensations, v_means2d, v_depths, v_conics,
              v_compensations, v_means, v_covars, v_quats, v_scales,
              v_viewmats};
    projection_packed_bwd_kernel<<<(unsigned)ceil_div(nnz, kProjThreads),
                                   kProjThreads, 0, as_stream(stream)>>>(
        a, nnz, batch_ids, camera_ids, gaussian_ids, sparse_grad,
        (B * C == 1) ? 1 : 0);
    return check_launch("projection_packed_bwd_kernel");
}

extern "C" int gsplat_quat_scale_to_covar_preci_fwd(int64_t N, const float *quats,
                                                    const float *scales,
                                                    int32_t triu, float *covars,
                                                    float *precis,
                                                    gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(N >= 0, "quat_scale_to_covar_preci_fwd: negative N");
    if (N == 0 || (covars == nullptr && precis == nullptr))
        return GSPLAT_OK;
    GS_REQUIRE(quats && scales, "quat_scale_to_covar_preci_fwd: NULL input");
    covar_preci_fwd_kernel<<<(unsigned)ceil_div(N, kProjThreads), kProjThreads, 0,
                             as_stream(stream)>>>(N, quats, scales, triu != 0,
                                                  covars, precis);
    return check_launch("covar_preci_fwd_kernel");
}

extern "C" int gsplat_quat_scale_to_covar_preci_bwd(
    int64_t N, const float *quats, const float *scales, int32_t triu,
    const float *v_covars, const float *v_precis, float *v_quats, float *v_scales,
    gsplat_stream_t stream) {
    clear_error();
    GS_REQUIRE(N >= 0, "quat_scale_to_covar_preci_bwd: negative N");
    if (N == 0)
        return GSPLAT_OK;
    GS_REQUIRE(quats && scales && v_quats && v_scales,
               "quat_scale_to_covar_preci_bwd: NULL buffer");
    covar_preci_bwd_kernel<<<(unsigned)ceil_div(N, kProjThreads), kProjThreads, 0,
                             as_stream(stream)>>>(N, quats, scales, triu != 0,
                                                  v_covars, v_precis, v_quats,
                                                  v_scales);
    return check_launch("covar_preci_bwd_kernel");
}
