// fh_qlinear.hip — ferrum_core's packed per-row int8 / int4 linear on gfx950.
//
//   y[i, j] = b[j] + sum_{p ascending} (x[i, p] * scale[p]) * level(p, j)
//
// is ops::qlinear (ops.rs:316-377) with qaccum_cols (ops.rs:268-305) over a
// QWeight (quant.rs:130-217): rows p = input features, one symmetric f32
// scale per row, int8 levels or int4 levels in the split-half nibble layout
// (column c < half in the low nibble of byte c, else the high nibble of byte
// c - half, half = ceil(n / 2)).  The reference starts every output at its
// bias and adds the products in ascending p without FMA; so does this kernel,
// so its outputs are the reference's bit for bit.  That fixes one sequential
// sum per output column: K is never split, and the parallelism is the columns
// (and rows of x).
//
// Device layout: the reference's row-major bytes, each row padded to a
// multiple of 64 bytes (16-byte-aligned dword loads, whole cache lines).
// Lane l of the grid owns dword l of every row: 4 int8 columns, or the 4 low
// and 4 high nibble columns of 4 bytes.  A wave reads 256 contiguous bytes per
// row; each lane keeps two batches of 16 rows' dwords in flight (double
// buffered) while it accumulates the previous batch in order.
#include "fh_internal.hpp"

#pragma clang fp contract(off)

struct fh_qweight {
    int device = 0;
    size_t k = 0, n = 0, row_bytes = 0, pitch = 0;
    int kind = 0;
    float* scales = nullptr;
    uint8_t* q = nullptr;
    void* base = nullptr;
};

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 512;  // rows p of scaled activations staged in LDS at a time
constexpr int kBatch = 16;   // weight dwords per lane per batch

__device__ __forceinline__ float level8(uint32_t w, int t) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * t)) & 0xFFu));
}
// quant.rs:222-225 nibble_to_i8: sign-extend a 4-bit level
__device__ __forceinline__ float level4(uint32_t w, int t, bool hi) {
    const uint32_t nib = (w >> (8 * t + (hi ? 4 : 0))) & 0xFu;
    return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(nib << 4)) >> 4);
}

// KIND 0: int8, 1: int4.  M rows of x per workgroup (grid.y over row groups).
template <int KIND, int M>
__global__ void __launch_bounds__(kThreads)
    k_qlinear(const uint8_t* __restrict__ q, const float* __restrict__ scales, const float* __restrict__ x,
              const float* __restrict__ bias, float* __restrict__ y, int m, int k, int n, int pitch) {
    constexpr int C = KIND == 0 ? 4 : 8;  // outputs per lane
    __shared__ float a[M][kChunk];
    const int lane_dw = blockIdx.x * kThreads + threadIdx.x;  // dword of the row this lane owns
    const int row0 = blockIdx.y * M;
    const int half = (n + 1) / 2;
    int col[C];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        col[t] = 4 * lane_dw + t;
        if (KIND == 1) col[4 + t] = half + 4 * lane_dw + t;
    }
    bool live[C];
#pragma unroll
    for (int c = 0; c < C; c++) live[c] = KIND == 0 ? col[c] < n : (c < 4 ? col[c] < half : col[c] < n);
    // every output starts at its bias (ops.rs: the bias is fused first)
    float acc[M][C];
#pragma unroll
    for (int i = 0; i < M; i++)
#pragma unroll
        for (int c = 0; c < C; c++) acc[i][c] = bias && live[c] ? bias[col[c]] : 0.0f;
    const bool active = 4 * lane_dw < pitch;
    const uint8_t* qp = q + 4 * static_cast<size_t>(active ? lane_dw : 0);
    for (int p0 = 0; p0 < k; p0 += kChunk) {
        const int pn = min(kChunk, k - p0);
        __syncthreads();  // the previous chunk's activations are consumed
        // a'[i, p] = x[i, p] * scale[p] (ops.rs:331-339)
        for (int e = threadIdx.x; e < M * kChunk; e += kThreads) {
            const int i = e / kChunk, pp = e % kChunk;
            a[i][pp] = (pp < pn && row0 + i < m) ? x[static_cast<size_t>(row0 + i) * k + p0 + pp] * scales[p0 + pp]
                                                 : 0.0f;
        }
        __syncthreads();
        if (!active) continue;
        uint32_t buf[2][kBatch];
        auto load = [&](int b, int pb) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < kBatch; u++) {
                const int pp = min(pb + u, pn - 1);  // clamped: rows past the chunk are loaded, never used
                buf[b][u] = *reinterpret_cast<const uint32_t*>(qp + static_cast<size_t>(p0 + pp) * pitch);
            }
        };
        load(0, 0);
        for (int pb = 0, b = 0; pb < pn; pb += kBatch, b ^= 1) {
            if (pb + kBatch < pn) load(b ^ 1, pb + kBatch);
#pragma unroll
            for (int u = 0; u < kBatch; u++) {
                if (pb + u >= pn) break;
                const uint32_t w = buf[b][u];
#pragma unroll
                for (int i = 0; i < M; i++) {
                    const float ap = a[i][pb + u];
#pragma unroll
                    for (int c = 0; c < C; c++) {
                        const float lv = KIND == 0 ? level8(w, c) : level4(w, c & 3, c >= 4);
                        acc[i][c] = acc[i][c] + ap * lv;
                    }
                }
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int i = 0; i < M; i++) {
        if (row0 + i >= m) break;
#pragma unroll
        for (int c = 0; c < C; c++)
            if (live[c]) y[static_cast<size_t>(row0 + i) * n + col[c]] = acc[i][c];
    }
}

template <int KIND>
int launch(fh_ctx* ctx, const fh_qweight* w, const float* x, size_t m, const float* bias, float* y) {
    const size_t dwords = w->pitch / 4;
    const unsigned gx = static_cast<unsigned>((dwords + kThreads - 1) / kThreads);
    const int mi = static_cast<int>(m), ki = static_cast<int>(w->k), ni = static_cast<int>(w->n);
    const int pi = static_cast<int>(w->pitch);
    if (m == 1) {
        hipLaunchKernelGGL((k_qlinear<KIND, 1>), dim3(gx, 1), dim3(kThreads), 0, ctx->stream, w->q, w->scales, x, bias,
                           y, mi, ki, ni, pi);
    } else {
        hipLaunchKernelGGL((k_qlinear<KIND, 4>), dim3(gx, static_cast<unsigned>((m + 3) / 4)), dim3(kThreads), 0,
                           ctx->stream, w->q, w->scales, x, bias, y, mi, ki, ni, pi);
    }
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

}  // namespace

int fh_qweight_upload(fh_ctx* ctx, const float* scales, const uint8_t* q, size_t k, size_t n, int kind,
                      fh_qweight** out) {
    if (!ctx || !out) return FH_ERR_INVALID;
    ctx->err.clear();
    *out = nullptr;
    if (kind != FH_QINT8 && kind != FH_QINT4)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_qweight_upload: unknown kind " + std::to_string(kind));
    if (!scales || !q || k == 0 || n == 0)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_qweight_upload: empty weight or NULL pointer");
    if (k > 0x7FFFFFFFu || n > 0x7FFFFFF0u)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_qweight_upload: a dimension is above 2^31 - 1");
    auto* w = new fh_qweight();
    w->device = ctx->device;
    w->k = k;
    w->n = n;
    w->kind = kind;
    w->row_bytes = kind == FH_QINT8 ? n : (n + 1) / 2;
    w->pitch = (w->row_bytes + 63) / 64 * 64;
    const size_t sbytes = fh_align256(k * sizeof(float));
    hipError_t e = hipMalloc(&w->base, sbytes + k * w->pitch);
    if (e != hipSuccess) {
        delete w;
        return fh_hip_fail(ctx, e, "hipMalloc (qweight)");
    }
    w->scales = static_cast<float*>(w->base);
    w->q = static_cast<uint8_t*>(w->base) + sbytes;
    e = hipMemcpyAsync(w->scales, scales, k * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(w->q, 0, k * w->pitch, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(w->q, w->pitch, q, w->row_bytes, w->row_bytes, k, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(w->base);
        delete w;
        return fh_hip_fail(ctx, e, "qweight upload");
    }
    *out = w;
    return FH_OK;
}

void fh_qweight_free(fh_qweight* w) {
    if (!w) return;
    if (w->base) (void)hipFree(w->base);
    delete w;
}

int fh_qlinear_async(fh_ctx* ctx, const fh_qweight* w, const float* d_x, size_t m, size_t k, const float* d_bias,
                     size_t bias_len, float* d_y) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!w) return fh_fail(ctx, FH_ERR_INVALID, "fh_qlinear: weight is NULL");
    if (k != w->k)
        return fh_fail(ctx, FH_ERR_DIM, "qlinear: input width " + std::to_string(k) + " ≠ weight rows " +
                                            std::to_string(w->k));
    if (!((bias_len == 0 && !d_bias) || (bias_len == w->n && d_bias)))
        return fh_fail(ctx, FH_ERR_DIM, "qlinear: bias length " + std::to_string(bias_len) + " ≠ out_features " +
                                            std::to_string(w->n));
    if (m == 0) return FH_OK;
    if (!d_x || !d_y) return fh_fail(ctx, FH_ERR_INVALID, "fh_qlinear: x or y is NULL");
    if (m > 0x7FFFFFFFu / 4 || m * w->n > (size_t(1) << 40))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_qlinear: m is too large");
    if (ctx->device != w->device)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_qlinear: the weight lives on another device");
    FH_HIP(ctx, hipSetDevice(ctx->device));
    return w->kind == FH_QINT8 ? launch<0>(ctx, w, d_x, m, d_bias, d_y) : launch<1>(ctx, w, d_x, m, d_bias, d_y);
}
