// fh_llama.hip — the Llama / Qwen block pieces on gfx950 (ferrum_core's
// llm.rs), batched over rows: each row is one sequence of a batched decode.
//
//  k_rmsnorm     RmsNorm::forward_row (llm.rs:58-65): x * (1 / sqrt(mean(x^2)
//                + eps)) * w, one workgroup per row; optionally the residual
//                add in front of it (h = x + r, written to s).
//  k_rope        apply_rope (llm.rs:146-175) with RopeScaling::angle
//                (llm.rs:118-121), NORM (adjacent pairs) or NEOX (split
//                halves), each row at its own position (read on the device).
//  k_swiglu      FeedForward's gate (llm.rs:415-421): (g / (1 + exp(-g))) * u.
//  k_embed_rows  LlamaModel::embed (llm.rs:588-596) for a row of token ids
//                held on the device.
// Grouped-query attention is the attention kernel of fh_block.hip with
// query head h reading kv head h / (n_heads / n_kv).
// Arithmetic is written without contraction, as the reference has no FMA.
#include "fh_internal.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;

template <bool kAdd, int kPer>
__global__ void __launch_bounds__(kThreads) k_rmsnorm(const float* x, const float* __restrict__ r, float* s_out, int d,
                                                     const float* __restrict__ w, float eps, float* __restrict__ out) {
    __shared__ float red[kThreads / 64];
    const size_t base = static_cast<size_t>(blockIdx.x) * d;
    float v[kPer], wv[kPer];
    // every load is issued before the reduction
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        v[i] = c < d ? (kAdd ? x[base + c] + r[base + c] : x[base + c]) : 0.0f;
        wv[i] = c < d ? w[c] : 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        if (c < d) {
            if (s_out) s_out[base + c] = v[i];
            ss += v[i] * v[i];
        }
    }
    const float ms = fh::block_sum(ss, red) / static_cast<float>(d);
    const float inv = 1.0f / sqrtf(ms + eps);
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        if (c < d) out[base + c] = v[i] * inv * wv[i];
    }
}

// One thread per (row, head, pair).
__global__ void __launch_bounds__(kThreads) k_rope(float* __restrict__ x, int rows, int ld, int n_heads, int hd,
                                                  int rope_dim, const uint32_t* __restrict__ dpos, float base, int neox,
                                                  const float* __restrict__ ff, float linear_factor) {
    const int half = rope_dim / 2;
    const size_t id = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (id >= static_cast<size_t>(rows) * n_heads * half) return;
    const int i = static_cast<int>(id % half);
    const int h = static_cast<int>((id / half) % n_heads);
    const int r = static_cast<int>(id / (static_cast<size_t>(half) * n_heads));
    float* xh = x + static_cast<size_t>(r) * ld + static_cast<size_t>(h) * hd;
    const int ia = neox ? i : 2 * i, ib = neox ? i + half : 2 * i + 1;
    float a = xh[ia], b = xh[ib];
    fh::rope_rotate(a, b, static_cast<int>(dpos[r]), i, rope_dim, base, ff, linear_factor);
    xh[ia] = a;
    xh[ib] = b;
}

__global__ void __launch_bounds__(kThreads) k_swiglu(const float* __restrict__ g, const float* __restrict__ u, int rows,
                                                    int n, int ld, float* __restrict__ out) {
    const size_t id = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (id >= static_cast<size_t>(rows) * n) return;
    const size_t r = id / n, j = id % n;
    const float gv = g[r * ld + j];
    out[id] = (gv / (1.0f + expf(-gv))) * u[r * ld + j];
}

__global__ void __launch_bounds__(kThreads) k_embed_rows(const float* __restrict__ tok_w, int vocab, int d,
                                                        const uint32_t* __restrict__ tokens, int rows,
                                                        float* __restrict__ out) {
    const size_t id = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (id >= static_cast<size_t>(rows) * d) return;
    const size_t r = id / d, c = id % d;
    const uint32_t t = tokens[r];
    // An id past the vocabulary (never one the sampler returns) poisons the row.
    out[id] = t < static_cast<uint32_t>(vocab) ? tok_w[static_cast<size_t>(t) * d + c] : __builtin_nanf("");
}

unsigned blocks_for(size_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

}  // namespace

int fh_launch_rmsnorm(fh_ctx* ctx, const float* x, const float* r, float* s, size_t rows, size_t d, const float* w,
                      float eps, float* out) {
    if (d > 32 * static_cast<size_t>(kThreads)) return fh_fail(ctx, FH_ERR_LIMIT, "fh_rmsnorm: rows wider than 8192");
    const dim3 grid(static_cast<unsigned>(rows)), block(kThreads);
    const int di = static_cast<int>(d);
    if (d <= 8 * static_cast<size_t>(kThreads)) {
        if (r) hipLaunchKernelGGL((k_rmsnorm<true, 8>), grid, block, 0, ctx->stream, x, r, s, di, w, eps, out);
        else hipLaunchKernelGGL((k_rmsnorm<false, 8>), grid, block, 0, ctx->stream, x, r, s, di, w, eps, out);
    } else {
        if (r) hipLaunchKernelGGL((k_rmsnorm<true, 32>), grid, block, 0, ctx->stream, x, r, s, di, w, eps, out);
        else hipLaunchKernelGGL((k_rmsnorm<false, 32>), grid, block, 0, ctx->stream, x, r, s, di, w, eps, out);
    }
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_rope(fh_ctx* ctx, float* x, size_t rows, size_t ld, size_t n_heads, size_t hd, size_t rope_dim,
                   const uint32_t* dpos, float base, int rope_type, const float* freq_factors, float linear_factor) {
    const size_t n = rows * n_heads * (rope_dim / 2);
    if (n == 0) return FH_OK;
    hipLaunchKernelGGL(k_rope, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, x, static_cast<int>(rows),
                       static_cast<int>(ld), static_cast<int>(n_heads), static_cast<int>(hd),
                       static_cast<int>(rope_dim), dpos, base, rope_type, freq_factors, linear_factor);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_swiglu(fh_ctx* ctx, const float* g, const float* u, size_t rows, size_t n, size_t ld, float* out) {
    hipLaunchKernelGGL(k_swiglu, dim3(blocks_for(rows * n)), dim3(kThreads), 0, ctx->stream, g, u,
                       static_cast<int>(rows), static_cast<int>(n), static_cast<int>(ld), out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_embed_rows(fh_ctx* ctx, const float* tok_w, size_t vocab, size_t d, const uint32_t* tokens, size_t rows,
                         float* out) {
    hipLaunchKernelGGL(k_embed_rows, dim3(blocks_for(rows * d)), dim3(kThreads), 0, ctx->stream, tok_w,
                       static_cast<int>(vocab), static_cast<int>(d), tokens, static_cast<int>(rows), out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
