// Error plumbing, version string and small utility kernels shared by the
// extern "C" entry points of libgsplat_hip.so.
#include "common.h"

namespace gs {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string &msg) {
    set_error(msg);
    return code;
}

int check_launch(const char *what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(GSPLAT_ERR_LAUNCH,
                    std::string(what) + ": " + hipGetErrorString(err));
    return GSPLAT_OK;
}

__global__ void clear_lookback_kernel(uint32_t *ticket, uint64_t *status,
                                      int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0)
        *ticket = 0u;
    if (i < n)
        status[i] = 0ull;
}

int clear_lookback(void *ws, int64_t n_blocks, hipStream_t stream) {
    Lookback lb = lookback_from(ws);
    const int64_t n = n_blocks > 0 ? n_blocks : 1;
    clear_lookback_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, stream>>>(
        lb.ticket, lb.status, n_blocks);
    return check_launch("clear_lookback");
}

}  // namespace gs

extern "C" const char *gsplat_last_error(void) {
    return gs::g_last_error.c_str();
}

extern "C" const char *gsplat_version(void) {
    return "gsplat_hip 0.1.0 gfx950";
}

// The build passes the digest of include/gsplat_hip.h's declarations.
#ifndef GSPLAT_ABI_HASH
#error "GSPLAT_ABI_HASH must be defined by the build (digest of include/gsplat_hip.h)"
#endif

extern "C" const char *gsplat_abi_version(void) {
    return GSPLAT_ABI_HASH;
}
