// fh_exact.hip — FH_W8A32_EXACT: the Q8_0 linear bit for bit as ferrum_core
// computes it over the expanded weights.
//
// ferrum_core expands a Q8_0 matrix to f32 at load (w = f32(f16 d) * q, exact:
// loader/decode.rs:97-100, gguf/tensors.rs:58-87) and runs linear_forward
// (ops.rs:233-256): matmul_block accumulates every output from zero, adding
// the products x[p] * w[p][j] in ascending p with a rounding after each
// product and each add (ops.rs:29-126, no fused multiply-add), and
// matmul_bias_block adds the bias after the contraction (ops.rs:132-148).  The
// row split over threads (parallel.rs:90-92) never splits an output's sum, so
// the result does not depend on the thread count.  The reference's roadmap
// names this contract for a packed Q8_0 forward
// (q8_0_packed_forward_equals_expanded).
//
// One sequential sum per output is therefore fixed: K is never split, and the
// parallelism is the output rows (and rows of x).  A workgroup owns 64
// consecutive output rows j and one row of x: three producer waves stream the
// rows' quants chunk by chunk (96 or 192 positions p, 16-byte row segments), form
// the products in f32 and store them in LDS (double-buffered), while the first
// wave (one lane per output row) adds the previous chunk's products in
// ascending p; the producers' loads run two chunks ahead.  The opt-in exact
// mode; FH_W8A32 is the fast one.
#include "fh_internal.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;
constexpr int kRows = 64;                         // output rows per workgroup: one per summing lane
constexpr int kProducers = kThreads - 64;         // waves 1..3

// Chunk geometry for P positions per chunk (P a multiple of 96: whole Q8_0
// blocks, and the chunk's 16-byte segments split evenly over the producers
// with every producer's segments at the same positions).  P = 192 for narrow
// weights (fewer, longer chunks); P = 96 for wide ones (51 KB of LDS, three
// workgroups per CU).
template <int P>
struct Geo {
    static constexpr int kSegRow = P / 16;               // 16-byte quant segments per row and chunk
    static constexpr int kSegs = kRows * kSegRow;
    static constexpr int kPer = kSegs / kProducers;      // segments per producer thread and chunk
    static constexpr int kStride = P + 4;                // LDS row pitch in floats (spreads the summing lanes' banks)
    static_assert(P % 96 == 0, "whole blocks, even producer split");
    static_assert(kSegs % kProducers == 0 && kProducers % kSegRow == 0, "producer geometry");
};

// A producer thread's share of one chunk: kPer 16-value row segments of rows
// r = s / kSegRow (s = pt + i * kProducers), all at the same positions
// p = c * P + (pt % kSegRow) * 16, so one 16-float slice of x serves every
// segment.  Q8_0 weights: 16 quants and their block's f16 scale per segment;
// F32 weights: the 16 values.
template <int P, bool F32>
struct Share {
    uint4 q[Geo<P>::kPer][F32 ? 4 : 1];
    uint32_t d[Geo<P>::kPer];
    float4 x[4];
};

struct WeightPtrs {
    const int8_t* qs;      // Q8_0 quant plane [n][k]
    const uint16_t* dsc;   // its f16 scales [n][k / 32]
    const float* f32;      // or F32 rows [n][pitch] (pitch = k rounded up to 16, zero-padded)
    int pitch;
};

// Issue the loads of chunk c (rows past n clamped: computed, never stored;
// positions past k skipped).
template <int P, bool F32>
__device__ __forceinline__ void load(const WeightPtrs& wp, const float* __restrict__ xr, int j0, int n, int k, int c,
                                     int pt, Share<P, F32>& sh) {
    using G = Geo<P>;
    const int p = c * P + (pt % G::kSegRow) * 16;
    if (p >= k) return;
    const size_t kb = static_cast<size_t>(k) / 32;
#pragma unroll
    for (int i = 0; i < G::kPer; i++) {
        const int r = (pt + i * kProducers) / G::kSegRow;
        const size_t row = static_cast<size_t>(min(j0 + r, n - 1));
        if constexpr (F32) {
            const uint4* src = reinterpret_cast<const uint4*>(wp.f32 + row * static_cast<size_t>(wp.pitch) + p);
#pragma unroll
            for (int v = 0; v < 4; v++) sh.q[i][v] = src[v];
        } else {
            sh.q[i][0] = *reinterpret_cast<const uint4*>(wp.qs + row * static_cast<size_t>(k) + p);
            sh.d[i] = wp.dsc[row * kb + static_cast<size_t>(p >> 5)];
        }
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
        // (positions past k: clamped loads whose products are never summed)
        const int e = p + 4 * v;
        sh.x[v] = make_float4(xr[min(e, k - 1)], xr[min(e + 1, k - 1)], xr[min(e + 2, k - 1)], xr[min(e + 3, k - 1)]);
    }
}

// The products of chunk c into buf[r * kStride + p - c * P].
template <int P, bool F32>
__device__ __forceinline__ void produce(int k, int c, int pt, const Share<P, F32>& sh, float* buf) {
    using G = Geo<P>;
    const int q = pt % G::kSegRow;
    if (c * P + q * 16 >= k) return;
#pragma unroll
    for (int i = 0; i < G::kPer; i++) {
        const int r = (pt + i * kProducers) / G::kSegRow;
        float* o = buf + r * G::kStride + q * 16;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float xs[4] = {sh.x[v].x, sh.x[v].y, sh.x[v].z, sh.x[v].w};
            float4 pr;
            float* e = &pr.x;
            if constexpr (F32) {
                const uint32_t ws[4] = {sh.q[i][v].x, sh.q[i][v].y, sh.q[i][v].z, sh.q[i][v].w};
#pragma unroll
                for (int b = 0; b < 4; b++) e[b] = xs[b] * __builtin_bit_cast(float, ws[b]);
            } else {
                const float d = fh_h2f(static_cast<uint16_t>(sh.d[i]));
                const uint32_t word = v == 0 ? sh.q[i][0].x : v == 1 ? sh.q[i][0].y : v == 2 ? sh.q[i][0].z : sh.q[i][0].w;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const float level = static_cast<float>(static_cast<int8_t>((word >> (8 * b)) & 0xFFu));
                    const float wv = d * level;  // exact: an f16 value times an 8-bit integer
                    e[b] = xs[b] * wv;
                }
            }
            *reinterpret_cast<float4*>(o + v * 4) = pr;
        }
    }
}

template <int P, bool F32>
__global__ void __launch_bounds__(kThreads)
    k_linear_exact(WeightPtrs wp, const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y,
                   int m, int n, int k) {
    constexpr int kStride = Geo<P>::kStride;
    __shared__ __align__(16) float prod[2][kRows * kStride];
    const int tid = threadIdx.x;
    const int j0 = blockIdx.x * kRows;
    const int chunks = (k + P - 1) / P;
    // wave-uniform roles (a scalar branch: both sides meet the same barriers,
    // 1 + chunks per row of x)
    const bool summing = __builtin_amdgcn_readfirstlane(tid >> 6) == 0;
    for (int i = blockIdx.y; i < m; i += gridDim.y) {
        const float* xr = x + static_cast<size_t>(i) * k;
        if (summing) {
            const int j = j0 + tid;
            const float* own = nullptr;
            float acc = 0.0f;
            __syncthreads();  // chunk 0 is in LDS
            for (int c = 0; c < chunks; c++) {
                own = prod[c & 1] + tid * kStride;
                const int pn = min(P, k - c * P);  // a multiple of 32 for Q8_0 weights
                int g = 0;
                for (; g + 32 <= pn; g += 32) {
                    // all eight reads in flight before the chain of 32 adds
                    float4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const float4*>(own + g + 4 * u);
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        acc = acc + v[u].x;
                        acc = acc + v[u].y;
                        acc = acc + v[u].z;
                        acc = acc + v[u].w;
                    }
                }
                for (; g < pn; g++) acc = acc + own[g];  // (F32 rows whose k is not a multiple of 32)
                __syncthreads();  // chunk c + 1 is in LDS; buffer c & 1 is free again
            }
            if (j < n) y[static_cast<size_t>(i) * n + j] = bias ? acc + bias[j] : acc;
        } else {
            // Loads run two chunks ahead of the products: `a` holds the even
            // chunks, `b` the odd ones.
            const int pt = tid - 64;
            Share<P, F32> a, b;
            load(wp, xr, j0, n, k, 0, pt, a);
            if (chunks > 1) load(wp, xr, j0, n, k, 1, pt, b);
            produce(k, 0, pt, a, prod[0]);
            __syncthreads();
            for (int c = 0; c < chunks; c += 2) {
                if (c + 2 < chunks) load(wp, xr, j0, n, k, c + 2, pt, a);
                if (c + 1 < chunks) produce(k, c + 1, pt, b, prod[1]);
                __syncthreads();
                if (c + 1 < chunks) {
                    if (c + 3 < chunks) load(wp, xr, j0, n, k, c + 3, pt, b);
                    if (c + 2 < chunks) produce(k, c + 2, pt, a, prod[0]);
                    __syncthreads();
                }
            }
        }
        // The next row's chunk 0 goes to buffer 0, whose last reader finished
        // before the final barrier above.
    }
}

}  // namespace

int fh_launch_linear_exact(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y) {
    if (w->n > 0x7FFFFFFFu || w->k > 0x7FFFFFFFu || m > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: a dimension is above 2^31 - 1");
    if (w->n == 0 || m == 0) return FH_OK;
    const unsigned gx = static_cast<unsigned>((w->n + kRows - 1) / kRows);
    const unsigned gy = static_cast<unsigned>(m < 65535 ? m : 65535);
    const WeightPtrs wp{w->qs, w->d, w->f32, static_cast<int>(w->pitch)};
    const int mi = static_cast<int>(m), ni = static_cast<int>(w->n), ki = static_cast<int>(w->k);
    if (w->kind == FH_WEIGHT_F32)
        hipLaunchKernelGGL((k_linear_exact<96, true>), dim3(gx, gy), dim3(kThreads), 0, ctx->stream, wp, x, bias, y, mi,
                           ni, ki);
    else if (w->n >= 16384)
        hipLaunchKernelGGL((k_linear_exact<96, false>), dim3(gx, gy), dim3(kThreads), 0, ctx->stream, wp, x, bias, y, mi,
                           ni, ki);
    else
        hipLaunchKernelGGL((k_linear_exact<192, false>), dim3(gx, gy), dim3(kThreads), 0, ctx->stream, wp, x, bias, y,
                           mi, ni, ki);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
