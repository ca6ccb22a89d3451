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
// multiple of 64 bytes.  A workgroup owns one 64-byte column tile of every row
// (64 int8 columns, or 64 low- and 64 high-nibble int4 columns).  With several
// rows of x (k_qlinear) it walks K in chunks of 512 rows: all 256 threads
// stream a chunk (32 KB, row segments of 16 bytes) and its scaled activations
// into one LDS buffer while wave i sums the previous chunk for x row i, one
// lane per column, in ascending p.  With one row (k_qlinear_row, the decode
// case) one wave sums and three form the products.  The sums are dependency
// chains of K adds, so the columns (and rows of x) are the parallelism and the
// chunk pipeline keeps the loads in flight meanwhile.
#include <type_traits>

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

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTile = 64;    // column bytes per workgroup
constexpr int kChunk = 512;  // rows p per LDS chunk
constexpr int kSegs = kChunk * kTile / 16 / kThreads;  // 16-byte row segments per thread and chunk

// quant.rs:222-225 nibble_to_i8: sign-extend a 4-bit level
__device__ __forceinline__ float level4(uint32_t b, bool hi) {
    const uint32_t nib = (hi ? b >> 4 : b) & 0xFu;
    return static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(nib << 4)) >> 4);
}

// KIND 0: int8, 1: int4.  M rows of x per workgroup (grid.y over row groups),
// one summing wave per row.
template <int KIND, int M>
__global__ void __launch_bounds__(kThreads)
    k_qlinear(const uint8_t* __restrict__ q, const float* __restrict__ scales, const float* __restrict__ x,
              const float* __restrict__ bias, float* __restrict__ y, int m, int k, int n, int pitch) {
    static_assert(M <= kThreads / 64, "one summing wave per row");
    __shared__ __align__(16) uint8_t wt[2][kChunk][kTile];
    __shared__ float a[2][M][kChunk];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c0 = blockIdx.x * kTile, row0 = blockIdx.y * M;
    const int half = (n + 1) / 2;
    // the column(s) lane `lane` of a summing wave owns
    const int col_lo = c0 + lane, col_hi = half + c0 + lane;
    const bool live_lo = KIND == 0 ? col_lo < n : col_lo < half;
    const bool live_hi = KIND == 1 && col_hi < n;
    const bool summing = wave < M && row0 + wave < m;
    // every output starts at its bias (the reference fuses the bias first)
    float acc_lo = bias && live_lo ? bias[col_lo] : 0.0f;
    float acc_hi = bias && live_hi ? bias[col_hi] : 0.0f;
    const int chunks = (k + kChunk - 1) / kChunk;
    constexpr int kAPer = kChunk / kThreads;  // activation rows per thread and chunk
    u4 seg[kSegs];
    float xv[M][kAPer], sv[kAPer];
    // Chunk c: thread t loads segment t % 4 of rows t / 4 + 64 j, and x and the
    // scale of rows t + 256 j (all clamped to valid rows: rows past K are
    // loaded, never summed).
    auto fetch = [&](int c) __attribute__((always_inline)) {
        const int p0 = c * kChunk;
#pragma unroll
        for (int j = 0; j < kSegs; j++) {
            const int p = min(p0 + (tid >> 2) + j * (kThreads / 4), k - 1);
            seg[j] = *reinterpret_cast<const u4*>(q + static_cast<size_t>(p) * pitch + c0 + (tid & 3) * 16);
        }
#pragma unroll
        for (int j = 0; j < kAPer; j++) {
            const int p = min(p0 + tid + j * kThreads, k - 1);
            sv[j] = scales[p];
#pragma unroll
            for (int i = 0; i < M; i++) xv[i][j] = x[static_cast<size_t>(min(row0 + i, m - 1)) * k + p];
        }
    };
    // a'[i, p] = x[i, p] * scale[p] (ops.rs:331-339) and the levels, into buffer b
    auto store = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kSegs; j++)
            *reinterpret_cast<u4*>(&wt[b][(tid >> 2) + j * (kThreads / 4)][(tid & 3) * 16]) = seg[j];
#pragma unroll
        for (int j = 0; j < kAPer; j++)
#pragma unroll
            for (int i = 0; i < M; i++) a[b][i][tid + j * kThreads] = xv[i][j] * sv[j];
    };
    fetch(0);
    store(0);
    __syncthreads();
    for (int c = 0; c < chunks; c++) {
        const int b = c & 1;
        if (c + 1 < chunks) fetch(c + 1);  // next chunk in flight during the sums
        if (summing) {
            const int pn = min(kChunk, k - c * kChunk);
            const float* ar = a[b][wave];
            for (int u = 0; u < pn; u++) {
                const uint32_t wb = wt[b][u][lane];
                const float ap = ar[u];
                if (KIND == 0) {
                    acc_lo = acc_lo + ap * static_cast<float>(static_cast<int8_t>(wb));
                } else {
                    acc_lo = acc_lo + ap * level4(wb, false);
                    acc_hi = acc_hi + ap * level4(wb, true);
                }
            }
        }
        if (c + 1 < chunks) store(b ^ 1);  // the other buffer: last read two chunks ago
        __syncthreads();
    }
    if (summing) {
        float* yr = y + static_cast<size_t>(row0 + wave) * n;
        if (live_lo) yr[col_lo] = acc_lo;
        if (live_hi) yr[col_hi] = acc_hi;
    }
}

// One row of x (the decode case).  A sum is a chain of K dependent adds, so
// the time of the kernel is K times the cost of one step of that chain.  Here
// the summing wave (wave 0) does nothing but the adds: waves 1-3 form the
// products a'[p] * level(p, j) of the next chunk into LDS meanwhile (the same
// f32 multiplications the reference makes), so each step of the chain is one
// add and a quarter of a 16-byte LDS read.
//
// LDS holds a chunk's products as float4 [group g of 4 rows][column], so the
// summing lane reads 4 consecutive rows of its column at once.  Columns are
// permuted within a group row (low 3 bits XOR ((col >> 3) + g)) so that the
// producers' 16-byte writes spread over the banks; the summing wave reads one
// contiguous group row, conflict-free under any permutation.
//
// TW is the column tile in bytes (16, 32 or 64).  At 16 and 32 a chunk is
// 48 KB of products, so a narrow tile means a long chunk: for a narrow output
// the chain then runs ~4x longer per chunk against the same LDS traffic, and
// the producers' writes no longer hold up the summing wave's reads (a
// dependent f32 add takes ~5.75 cycles; with 64-byte tiles and 48 KB chunks
// the products' write and read took ~70 % of the CU's LDS bandwidth during the
// chain).  TW = 64 serves wide outputs (more tiles than CUs): its chunks are
// 32 KB, so two workgroups share a CU, and two producer waves fill a chunk
// (the third repeats their work, writing the same values).
template <int KIND, int TW>
__global__ void __launch_bounds__(kThreads)
    k_qlinear_row(const uint8_t* __restrict__ q, const float* __restrict__ scales, const float* __restrict__ x,
                  const float* __restrict__ bias, float* __restrict__ y, int k, int n, int pitch) {
    static_assert(TW == 16 || TW == 32 || TW == 64, "column tile of 16, 32 or 64 bytes");
    constexpr int kSegs = TW / 16;                             // 16-byte segments per row tile
    constexpr int kRows = TW == 64 ? (KIND == 0 ? 128 : 64)     // rows p per chunk: 128 producer jobs
                                   : (KIND == 0 ? 768 : 384) / kSegs;  // 192 producer jobs
    constexpr int kGroups = kRows / 4;
    constexpr int kCols = KIND == 0 ? TW : 2 * TW;             // output columns per workgroup
    __shared__ float4 prod[2][kGroups * kCols];
    const int tid = threadIdx.x, lane = tid & 63;
    // Summing lanes: one column each (int8; int4 at TW <= 32, lanes < TW on the
    // low-nibble columns, the next TW on the high ones), or, for int4 at
    // TW = 64, the low and the high column of byte lane (two chains).
    constexpr bool kTwo = KIND == 1 && TW == 64;
    constexpr int kLane = KIND == 0 || kTwo ? TW : 2 * TW;  // lanes that own columns
    const int lr = lane % kLane;  // lanes past them mirror lane % kLane and store nothing
    const int c0 = blockIdx.x * TW;
    const int half = (n + 1) / 2;
    const int chunks = (k + kRows - 1) / kRows;
    auto slot = [](int col, int g) __attribute__((always_inline)) { return col ^ (((col >> 3) + g) & 7); };

    // wave-uniform role (a scalar branch: every wave meets the same barriers)
    if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0) {
        // the summing wave: column col_lo (and col_hi for int4 at TW = 64)
        const bool hi_lane = KIND == 1 && !kTwo && lr >= TW;
        const int col_lo = hi_lane ? half + c0 + lr - TW : c0 + lr, col_hi = half + c0 + lr;
        const bool live_lo = lane < kLane && col_lo < (KIND == 0 || hi_lane ? n : half);
        const bool live_hi = kTwo && col_hi < n;
        float acc_lo = bias && live_lo ? bias[col_lo] : 0.0f;
        float acc_hi = bias && live_hi ? bias[col_hi] : 0.0f;
        __syncthreads();  // chunk 0 is in LDS
        for (int c = 0; c < chunks; c++) {
            const float4* pb = prod[c & 1];
            const int pn = min(kRows, k - c * kRows);
            const int gn = pn >> 2;
            auto add4 = [](float acc, float4 v) __attribute__((always_inline)) {
                return (((acc + v.x) + v.y) + v.z) + v.w;
            };
            // two chains (int4 at TW = 64) are independent; their adds
            // alternate so each waits on its own chain only (written one chain
            // after the other, in-order issue serialises them)
            auto step = [&](int g) __attribute__((always_inline)) {
                const float4 v = pb[g * kCols + slot(lr, g)];
                if constexpr (!kTwo) {
                    acc_lo = add4(acc_lo, v);
                } else {
                    const float4 h = pb[g * kCols + slot(TW + lr, g)];
                    acc_lo = acc_lo + v.x;
                    acc_hi = acc_hi + h.x;
                    acc_lo = acc_lo + v.y;
                    acc_hi = acc_hi + h.y;
                    acc_lo = acc_lo + v.z;
                    acc_hi = acc_hi + h.z;
                    acc_lo = acc_lo + v.w;
                    acc_hi = acc_hi + h.w;
                }
            };
            if (gn == kGroups) {
#pragma unroll 32
                for (int g = 0; g < kGroups; g++) step(g);
            } else {
                for (int g = 0; g < gn; g++) step(g);
                const int rest = pn & 3;  // rows of a last, partial group
                if (rest) {
                    const float4 v = pb[gn * kCols + slot(lr, gn)];
                    acc_lo = acc_lo + v.x;
                    if (rest > 1) acc_lo = acc_lo + v.y;
                    if (rest > 2) acc_lo = acc_lo + v.z;
                    if (kTwo) {
                        const float4 h = pb[gn * kCols + slot(TW + lr, gn)];
                        acc_hi = acc_hi + h.x;
                        if (rest > 1) acc_hi = acc_hi + h.y;
                        if (rest > 2) acc_hi = acc_hi + h.z;
                    }
                }
            }
            __syncthreads();  // chunk c + 1 is in LDS; buffer c & 1 is free
        }
        if (live_lo) y[col_lo] = acc_lo;
        if (live_hi) y[col_hi] = acc_hi;
        return;
    }

    // The producers: thread t owns rows 4g..4g+3 of a chunk and 16-byte column
    // segment s (for int4, the low or the high nibbles of it: hs = 0 or 4).
    constexpr int kHalfJobs = kGroups * kSegs;  // jobs per nibble half (int4) or per chunk (int8)
    const int t = tid - 64;
    const int tj = t % kHalfJobs, h = KIND == 0 ? 0 : (t / kHalfJobs) % 2;
    const int g = tj / kSegs, s = tj % kSegs;
    const int hs = h * 4;
    const int colb = h * TW + s * 16;
    u4 wv[2][4];
    float xv[2][4], sv[2][4];
    // Chunk c's rows into register set S (rows past K clamp to K - 1: loaded,
    // never summed).
    auto fetch = [&](auto S, int c) __attribute__((always_inline)) {
        const int p0 = c * kRows + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int p = min(p0 + r, k - 1);
            wv[S][r] = *reinterpret_cast<const u4*>(q + static_cast<size_t>(p) * pitch + c0 + s * 16);
            xv[S][r] = x[p];
            sv[S][r] = scales[p];
        }
    };
    auto produce = [&](auto S, int b) __attribute__((always_inline)) {
        float a[4];
#pragma unroll
        for (int r = 0; r < 4; r++) a[r] = xv[S][r] * sv[S][r];  // ops.rs:331-339
        float4* pb = prod[b] + g * kCols;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float lv[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t byte = (wv[S][r][i >> 2] >> (8 * (i & 3))) & 0xFFu;
                lv[r] = KIND == 0 ? static_cast<float>(static_cast<int8_t>(static_cast<uint8_t>(byte)))
                                  : level4(byte >> hs, false);
            }
            pb[slot(colb + i, g)] = make_float4(a[0] * lv[0], a[1] * lv[1], a[2] * lv[2], a[3] * lv[3]);
        }
    };
    std::integral_constant<int, 0> s0;
    std::integral_constant<int, 1> s1;
    fetch(s0, 0);
    if (chunks > 1) fetch(s1, 1);
    produce(s0, 0);
    __syncthreads();
    // Step c: set c & 1 held chunk c (its products are in LDS), so it takes
    // chunk c + 2; chunk c + 1's products go to buffer (c + 1) & 1.
    auto step = [&](auto S, int c) __attribute__((always_inline)) {
        if (c + 2 < chunks) fetch(S, c + 2);
        if (c + 1 < chunks) produce(std::integral_constant<int, 1 - S>{}, (c + 1) & 1);
        __syncthreads();
    };
    for (int c = 0; c < chunks; c += 2) {
        step(s0, c);
        if (c + 1 < chunks) step(s1, c + 1);
    }
}

template <int KIND>
int launch(fh_ctx* ctx, const fh_qweight* w, const float* x, size_t m, const float* bias, float* y) {
    const unsigned gx = static_cast<unsigned>(w->pitch / kTile);
    const int mi = static_cast<int>(m), ki = static_cast<int>(w->k), ni = static_cast<int>(w->n);
    const int pi = static_cast<int>(w->pitch);
    if (m == 1) {
        // the narrowest tile that still keeps the grid within one workgroup per CU
        if (gx <= 64)
            hipLaunchKernelGGL((k_qlinear_row<KIND, 16>), dim3(gx * 4), dim3(kThreads), 0, ctx->stream, w->q,
                               w->scales, x, bias, y, ki, ni, pi);
        else if (gx <= 128)
            hipLaunchKernelGGL((k_qlinear_row<KIND, 32>), dim3(gx * 2), dim3(kThreads), 0, ctx->stream, w->q,
                               w->scales, x, bias, y, ki, ni, pi);
        else
            hipLaunchKernelGGL((k_qlinear_row<KIND, 64>), dim3(gx), dim3(kThreads), 0, ctx->stream, w->q, w->scales,
                               x, bias, y, ki, ni, pi);
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
