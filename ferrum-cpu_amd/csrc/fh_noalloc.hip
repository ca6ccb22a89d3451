// fh_noalloc.hip — fh_q8_0_linear_noalloc_async: the decode and batched-decode
// Q8_0 linear (FH_W8A32, m <= 64) for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).
//
// The kernels are the ones fh_q8_0_linear_async runs: the GEMV for m <= 2 (no
// scratch) and the skinny matrix-core GEMM for 3 <= m <= 64, whose split-K
// partial sums and per-tile arrival counters live in `scratch` below instead of
// the context's grow-on-demand workspace.  The arrival counters are cleared
// by a small kernel before every split launch.
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy (kFhNoallocScratchBytes) until the process ends, at its own
// address.  Host code never passes the array's name to a kernel (on the host
// it is only a stand-in symbol): on the first call on each device, with that
// device current, hipGetSymbolAddress gives that device's address, which is
// kept per device and is what the launches use.  Every call on one GPU shares
// that GPU's array, so calls that overlap on one GPU (two streams, two
// threads) race; calls in one stream order are safe.
#include <mutex>
#include <string>

#include "fh_internal.hpp"

namespace {

// 12 MiB: the largest split-K layout the skinny GEMM picks for m <= 64 on a
// 256-CU part is 127 tiles x 8 splits x 2048 outputs x 4 bytes (8.3 MB) plus
// the counters; a shape that would need more is refused (FH_ERR_LIMIT).
constexpr size_t kFhNoallocScratchBytes = size_t(12) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kFhNoallocScratchBytes];

std::mutex g_lock;
void* g_ptr[kMaxDevices] = {};  // scratch's device address, per device (nullptr until looked up)

// This device's address of `scratch` (device current); looked up once.
int scratch_on(fh_ctx* ctx, void** out) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_noalloc: device index above 63");
    std::lock_guard<std::mutex> hold(g_lock);
    if (!g_ptr[ctx->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return fh_hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
        if (!p) return fh_fail(ctx, FH_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
        g_ptr[ctx->device] = p;
    }
    *out = g_ptr[ctx->device];
    return FH_OK;
}

}  // namespace

extern "C" int fh_q8_0_linear_noalloc_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                            const float* d_bias, size_t bias_len, float* d_y, int numerics) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!w) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: weight is NULL");
    if (numerics != FH_W8A32 && numerics != FH_W8A8 && numerics != FH_W8A32_EXACT && numerics != FH_W8A8_FAST)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: unknown numerics " + std::to_string(numerics));
    if (w->device != ctx->device)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: weight lives on another device");
    if (k != w->k)
        return fh_fail(ctx, FH_ERR_DIM, "linear_forward: input width " + std::to_string(k) +
                                            " \xe2\x89\xa0 weight rows " + std::to_string(w->k));
    if ((d_bias == nullptr) != (bias_len == 0) || (bias_len != 0 && bias_len != w->n))
        return fh_fail(ctx, FH_ERR_DIM, "linear_forward: bias length " + std::to_string(bias_len) +
                                            " \xe2\x89\xa0 out_features " + std::to_string(w->n));
    if (numerics != FH_W8A32 || w->kind != FH_WEIGHT_Q8_0)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear_noalloc: only FH_W8A32 on a Q8_0 weight runs without allocation");
    if (m > 64)
        return fh_fail(ctx, FH_ERR_LIMIT,
                       "fh_q8_0_linear_noalloc: m = " + std::to_string(m) + " is above 64 (the decode shapes)");
    if (m == 0) return FH_OK;
    if (!d_x || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x or y is NULL");
    if (reinterpret_cast<uintptr_t>(d_x) & 15)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x must be 16-byte aligned");
    if (w->n > 0x7FFFFFFFu || w->k > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: a dimension is above 2^31 - 1");
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) FH_HIP(ctx, hipSetDevice(ctx->device));
    void* base = nullptr;
    int rc = scratch_on(ctx, &base);
    if (rc) return rc;
    if (m <= 2) {
        rc = fh_launch_gemv_w8a32(ctx, w, d_x, m, d_bias, d_y);
        if (rc >= 0) return rc;
    }
    return fh_launch_skinny_scratch(ctx, w, d_x, m, d_bias, d_y, fh_scratch{base, kFhNoallocScratchBytes});
}
