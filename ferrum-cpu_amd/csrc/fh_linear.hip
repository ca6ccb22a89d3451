// fh_linear.hip — Q8_0 linear layers on gfx950.
//
//   y[i, j] = sum_p x[i, p] * W[j, p] (+ b[j])      W = f16(d) * q, exact in f32
//
// is ferrum_core's ops::linear_forward on its f32 expansion of the GGUF tensor
// (ops.rs:233-256, loader/decode.rs:97-100).  The reference sums the products
// in ascending p without FMA and adds the bias last; these kernels keep the
// bias last but reduce in a parallel order with FMA, which moves the last bits
// (judged at 1e-5 relative, see tests/test_gpu_linear.py).
//
// Kernels
//  k_gemv_w8a32  m <= 2 (decode).  HBM-bound: every weight byte is read once,
//                16 quants per lane per 16-byte load, dequantised in registers;
//                the activation chunks a lane needs stay in its registers for
//                every row it visits.  G lanes share a row and finish it with a
//                butterfly shuffle reduction; 64/G rows per wave per step.
//                With a LayerNorm prologue (fh_q8_0_linear_ln) every wave
//                first forms LayerNorm(x + r) of the rows it holds.
//  m >= 3 (and rows too long for the GEMV) go to the matrix-core GEMM in
//                fh_gemm.hip.
//  k_linear_w8a8 llama.cpp numerics: x is Q8_0-encoded per 32 (bit-exact
//                q8_0_block), exact int32 block dots with sdot4, then
//                sum_b f32(dot_b) * (d_w * d_x) + b (blocks summed in parallel).
//                Larger problems go to the int8-MFMA kernel in fh_gemm.hip,
//                which sums the blocks in order and is bit-exact.
#include "fh_internal.hpp"

#include <type_traits>

// The epilogues round every product and sum as the reference does (its GELU
// and bias adds have no FMA); the dot products use explicit fmaf.
#pragma clang fp contract(off)

__global__ void fh_k_encode_split(const float* __restrict__ x, size_t nblocks, uint32_t* __restrict__ qx,
                                  uint16_t* __restrict__ dx);

namespace {

constexpr int kWaves = 4;  // waves per block of the GEMV with the LayerNorm prologue (the plain GEMV: one)
constexpr int kLnMaxK = 2048;  // widest row the GEMV's LayerNorm prologue takes
// W8A8 runs on the int8 matrix cores (one wave per 32- or 64-row x 64-column
// output tile, every Q8_0 block in order) once there are this many tiles;
// fewer waves, each walking all of K, lose to the block-parallel kernel below.
constexpr size_t kW8a8MfmaTiles = 96;

__device__ __forceinline__ float sbyte(uint32_t w, int i) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * i)) & 0xFFu));
}

using fh::group_sum;
using fh::group_total;
using fh::rdlane;

// Q8_0 GEMV, m = M <= 2.  A wave owns `per_wave` consecutive row-sets (a
// row-set = 64 / G rows, G lanes per row); it issues the loads of up to U
// row-sets at once — CPL 16-byte quant chunks and their f16 scales per lane —
// next to its activation chunks, so a whole batch costs one memory latency.
// Lane gl of a row holds chunks gl, gl + G, ... (coalesced: the G lanes of a
// row read G consecutive 16-byte chunks).
// kLn: the activations are LayerNorm(x + ln.r) (the residual add and the
// LayerNorm in front of this linear).  The G lanes of a row group hold the
// whole row, so every wave forms the row's mean and variance with group
// shuffles; wave 0 of block 0 writes x + r to ln.s (when given).
template <int G, int CPL, int M, int U, bool kBias, bool kLn>
__global__ void __launch_bounds__(kLn ? 64 * kWaves : 64)
    k_gemv_w8a32(const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc, const float* __restrict__ x,
                 const float* __restrict__ bias, float* __restrict__ y, int n, int k, int per_wave, int act,
                 fh_ln_args ln) {
    constexpr int RW = 64 / G;  // rows per row-set
    // The LayerNorm prologue shares its row statistics across a workgroup of
    // kWaves waves; the plain GEMV runs one wave per workgroup, which spreads
    // a small layer's waves over more CUs (2304 x 768: 3.20 -> 3.04 us).
    constexpr int kW = kLn ? kWaves : 1;
    const int lane = threadIdx.x & 63;
    const int grp = lane / G, gl = lane % G;
    const int k16 = k >> 4, kb = k >> 5;
    const int nsets = (n + RW - 1) / RW;
    const int wave = blockIdx.x * kW + (threadIdx.x >> 6);
    const int set0 = wave * per_wave;
    if (!kLn && set0 >= nsets) return;  // (with kLn every wave joins the LayerNorm's barriers first)
    const int set1 = min(nsets, set0 + per_wave);
    [[maybe_unused]] __shared__ __align__(16) float ln_x[kLn ? M : 1][kLn ? kLnMaxK : 4];
    [[maybe_unused]] __shared__ float ln_red[kLn ? 2 * M : 1][kW];

    // Every load below is unconditional, from a clamped (always valid)
    // address, so the compiler issues them back to back without waits; the
    // lanes and rows past the end are zeroed when the data is used.
    // A chunk past the row end (k16 not a multiple of G) re-reads the last one
    // and gets its activations masked to +0.0 bit-wise, so it adds nothing.
    float xr[M][CPL][16];
    if constexpr (!kLn) {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ci = min(gl + c * G, k16 - 1);
            const uint32_t keep = gl + c * G < k16 ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float4* src = reinterpret_cast<const float4*>(x + static_cast<size_t>(m) * k + ci * 16);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float4 f = src[v];
                    const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        xr[m][c][4 * v + e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, fv[e]) & keep);
                }
            }
        }
    }
    // kLn: LayerNorm::forward (layer/norm.rs:46-82) of each row of x + r,
    // once per workgroup: thread t holds elements t, t + 256, ... (loaded
    // here, before any weight load), the workgroup sums them in a fixed
    // order, writes (v - mean) * (1 / sqrt(var + 1e-5)) * gamma + beta to LDS,
    // and every wave reads its chunks back from there.  Workgroup 0 writes
    // x + r to ln.s.  It runs after the first batch's weight loads are in
    // flight, so their latency covers it.
    constexpr int kLnPer = kLnMaxK / (64 * kW);
    [[maybe_unused]] float lv[kLn ? M : 1][kLn ? kLnPer : 1], lg[kLn ? kLnPer : 1], lb[kLn ? kLnPer : 1];
    if constexpr (kLn) {
#pragma unroll
        for (int i = 0; i < kLnPer; i++) {
            const int c = threadIdx.x + i * 64 * kW;
            const int cc = min(c, k - 1);
            lg[i] = ln.gamma[cc];
            lb[i] = ln.beta[cc];
#pragma unroll
            for (int m = 0; m < M; m++)
                lv[m][i] = ln.r ? x[static_cast<size_t>(m) * k + cc] + ln.r[static_cast<size_t>(m) * k + cc]
                                : x[static_cast<size_t>(m) * k + cc];
        }
    }
    auto layer_norm = [&]() __attribute__((always_inline)) {
        if constexpr (kLn) {
            const int w = threadIdx.x >> 6;
            float mean[M], rsd[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < kLnPer; i++)
                    if (threadIdx.x + i * 64 * kW < k) s += lv[m][i];
                s = group_total<64>(s);
                if ((threadIdx.x & 63) == 0) ln_red[m][w] = s;
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < M; m++) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < kW; i++) s += ln_red[m][i];
                mean[m] = s / static_cast<float>(k);
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < kLnPer; i++)
                    if (threadIdx.x + i * 64 * kW < k) {
                        const float dv = lv[m][i] - mean[m];
                        ss += dv * dv;
                    }
                ss = group_total<64>(ss);
                if ((threadIdx.x & 63) == 0) ln_red[M + m][w] = ss;
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < M; m++) {
                float ss = 0.0f;
#pragma unroll
                for (int i = 0; i < kW; i++) ss += ln_red[M + m][i];
                rsd[m] = 1.0f / sqrtf(ss / static_cast<float>(k) + 1e-5f);
#pragma unroll
                for (int i = 0; i < kLnPer; i++) {
                    const int c = threadIdx.x + i * 64 * kW;
                    if (c < k) {
                        ln_x[m][c] = ((lv[m][i] - mean[m]) * rsd[m]) * lg[i] + lb[i];
                        if (ln.s && blockIdx.x == 0) ln.s[static_cast<size_t>(m) * k + c] = lv[m][i];
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const bool valid = gl + c * G < k16;
                const int ci = min(gl + c * G, k16 - 1);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const float4* src = reinterpret_cast<const float4*>(&ln_x[m][ci * 16]);
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const float4 f = src[v];
                        xr[m][c][4 * v] = valid ? f.x : 0.0f;
                        xr[m][c][4 * v + 1] = valid ? f.y : 0.0f;
                        xr[m][c][4 * v + 2] = valid ? f.z : 0.0f;
                        xr[m][c][4 * v + 3] = valid ? f.w : 0.0f;
                    }
                }
            }
        }
    };
    if (set0 >= nsets) {
        if constexpr (kLn) layer_norm();  // the workgroup's barriers need every wave
        return;
    }
    [[maybe_unused]] bool normed = false;

    // One batch of row-sets [sb, sb + U).  Full batches have no branches, so
    // every load is consumed before the next batch reuses its registers.  The
    // short last batch (kTail) loads its own row-sets only (slots past the end
    // re-read its last row-set: cache hits, never computed) and skips the
    // empty slots; nothing follows it.
    // Bias, then the optional GELU the caller's next op would apply
    // (activation::gelu, activation.rs:9-12), rounded as the reference does.
    auto finish = [](float v, float b, int a) __attribute__((always_inline)) {
        if (kBias) v = v + b;
        if (a == FH_ACT_GELU) v = 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * v * v * v)));
        return v;
    };
    auto batch = [&](int sb, auto tail) __attribute__((always_inline)) {
        constexpr bool kTail = decltype(tail)::value;
        uint4 qv[U][CPL];
        uint32_t dh[U][CPL];
        float bv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = min((kTail ? min(sb + u, set1 - 1) : sb + u) * RW + grp, n - 1);
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const int ci = min(gl + c * G, k16 - 1);
                qv[u][c] = *reinterpret_cast<const uint4*>(qs + static_cast<size_t>(row) * k + ci * 16);
                dh[u][c] = dsc[static_cast<size_t>(row) * kb + (ci >> 1)];
            }
            bv[u] = kBias ? bias[row] : 0.0f;
        }
        // Keep the scheduler from interleaving the batch's loads with its math:
        // all of them go out before the first wait.
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kLn) {
            if (!normed) {  // wave-uniform
                layer_norm();
                normed = true;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (kTail && sb + u >= set1) break;  // wave-uniform
            float acc[M];
#pragma unroll
            for (int m = 0; m < M; m++) acc[m] = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const float dvc = fh_h2f(static_cast<uint16_t>(dh[u][c]));
                const uint32_t wq[4] = {qv[u][c].x, qv[u][c].y, qv[u][c].z, qv[u][c].w};
                float wf[16];
#pragma unroll
                for (int t = 0; t < 16; t++) wf[t] = sbyte(wq[t >> 2], t & 3);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    float sacc = 0.0f;
#pragma unroll
                    for (int t = 0; t < 16; t++) sacc = fmaf(xr[m][c][t], wf[t], sacc);
                    acc[m] = fmaf(dvc, sacc, acc[m]);
                }
            }
            const int row = (sb + u) * RW + grp;
            if (G <= 16) {
#pragma unroll
                for (int m = 0; m < M; m++) acc[m] = group_sum<G>(acc[m]);
                if (gl == 0 && row < n) {
#pragma unroll
                    for (int m = 0; m < M; m++) y[static_cast<size_t>(m) * n + row] = finish(acc[m], bv[u], act);
                }
            } else {
                // G = 32 or 64: 16-lane row totals, then across rows with readlane
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const float r16 = group_sum<16>(acc[m]);
                    const float lo = rdlane(r16, 0) + rdlane(r16, 16);
                    const float hi = rdlane(r16, 32) + rdlane(r16, 48);
                    const float tot = G == 64 ? lo + hi : (grp == 0 ? lo : hi);
                    if (gl == 0 && row < n) y[static_cast<size_t>(m) * n + row] = finish(tot, bv[u], act);
                }
            }
        }
    };
    int sb = set0;
    for (; sb + U <= set1; sb += U) batch(sb, std::false_type{});
    if (sb < set1) batch(sb, std::true_type{});
}

// ---- W8A8 ------------------------------------------------------------------------
// One lane per Q8_0 block of a (activation row, weight row) pair; G lanes per
// pair reduce with a butterfly.  Block dots are exact (sdot4 on int8).
template <int G>
__global__ void __launch_bounds__(256)
    k_linear_w8a8(const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc, const int8_t* __restrict__ qx,
                  const uint16_t* __restrict__ dx, const float* __restrict__ bias, float* __restrict__ y, int m, int n,
                  int k) {
    constexpr int RW = 64 / G;
    const int lane = threadIdx.x & 63;
    const int grp = lane / G, gl = lane % G;
    const int kb = k >> 5;
    const size_t pairs = static_cast<size_t>(m) * n;
    const size_t set = (blockIdx.x * static_cast<size_t>(4) + (threadIdx.x >> 6));
    const size_t pair = set * RW + grp;
    const bool live = pair < pairs;
    const int i = live ? static_cast<int>(pair / n) : 0, j = live ? static_cast<int>(pair % n) : 0;
    float acc = 0.0f;
    if (live) {
        for (int b = gl; b < kb; b += G) {
            const int4* a = reinterpret_cast<const int4*>(qx + static_cast<size_t>(i) * k + b * 32);
            const int4* w = reinterpret_cast<const int4*>(qs + static_cast<size_t>(j) * k + b * 32);
            int s = 0;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int4 av = a[h], wv = w[h];
                s = __builtin_amdgcn_sdot4(av.x, wv.x, s, false);
                s = __builtin_amdgcn_sdot4(av.y, wv.y, s, false);
                s = __builtin_amdgcn_sdot4(av.z, wv.z, s, false);
                s = __builtin_amdgcn_sdot4(av.w, wv.w, s, false);
            }
            const float dd = fh_h2f(dsc[static_cast<size_t>(j) * kb + b]) * fh_h2f(dx[static_cast<size_t>(i) * kb + b]);
            acc = fmaf(static_cast<float>(s), dd, acc);
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (live && gl == 0) y[pair] = bias ? acc + bias[j] : acc;
}

// Row-sets per wave: enough waves to cover the chip (12 per CU on 256 CUs)
// before a wave takes more than one row-set; beyond U, whole batches of U.
template <int G, int CPL, int M, int U>
int launch_gemv(fh_ctx* ctx, const fh_q8_0* w, const float* x, const float* bias, float* y, int act,
                const fh_ln_args* ln) {
    constexpr int RW = 64 / G;
    const size_t nsets = (w->n + RW - 1) / RW;
    size_t per_wave = (nsets + 3071) / 3072;
    if (per_wave < 1) per_wave = 1;
    if (per_wave > static_cast<size_t>(U)) per_wave = ((per_wave + U - 1) / U) * U;
    const size_t waves = (nsets + per_wave - 1) / per_wave;
    const size_t wpb = ln ? kWaves : 1;  // waves per workgroup, as the kernel's kW
    const size_t blocks = (waves + wpb - 1) / wpb;
    // The bias-free form (ops::matmul, the tied lm_head) is its own instance.
    auto kernel = bias ? k_gemv_w8a32<G, CPL, M, U, true, false> : k_gemv_w8a32<G, CPL, M, U, false, false>;
    // The LayerNorm prologue serves rows of at most 2048 (at most 2 chunks
    // per lane at G = 64); longer rows take the two-kernel path.
    if (ln) {
        if constexpr (G == 64 && CPL > 2) {
            return -1;
        } else {
            kernel = bias ? k_gemv_w8a32<G, CPL, M, U, true, true> : k_gemv_w8a32<G, CPL, M, U, false, true>;
        }
    }
    const fh_ln_args none{nullptr, nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(static_cast<unsigned>(64 * wpb)), 0, ctx->stream, w->qs, w->d,
                       x, bias, y, static_cast<int>(w->n), static_cast<int>(w->k), static_cast<int>(per_wave), act,
                       ln ? *ln : none);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

// Lanes per row (G) and 16-quant chunks per lane (CPL) for a row of k quants:
// G = 64 with CPL = ceil(k/16/64) for long rows; shorter rows take the
// smallest power-of-two G with at most 4 chunks per lane.  U keeps about 12
// quant loads in flight per lane.
template <int M>
int dispatch_gemv(fh_ctx* ctx, const fh_q8_0* w, const float* x, const float* bias, float* y, int act,
                  const fh_ln_args* ln = nullptr) {
    const size_t k16 = w->k / 16;
#define FH_GEMV(G, C) return launch_gemv<G, C, M, (12 / C > 0 ? 12 / C : 1)>(ctx, w, x, bias, y, act, ln)
    if (k16 >= 64) {
        switch ((k16 + 63) / 64) {
            case 1: FH_GEMV(64, 1);
            case 2: FH_GEMV(64, 2);
            case 3: FH_GEMV(64, 3);
            case 4: FH_GEMV(64, 4);
            case 5: FH_GEMV(64, 5);
            case 6: FH_GEMV(64, 6);
            case 7:
            case 8: FH_GEMV(64, 8);
            default: return -1;  // caller falls back to the tiled kernel
        }
    }
    const size_t g = (k16 + 3) / 4;  // lanes needed at 4 chunks per lane
    const size_t cpl16 = (k16 + 15) / 16;
    // Narrow outputs with rows of 48-63 chunks: a row per wave (up to 16 lanes
    // idle) gives four times the waves of 16 lanes per row, which pays for a
    // 768 x 768 layer (2.88 -> 2.44 us) but not for 2304 or more rows.
    if (k16 >= 48 && w->n <= 1024) FH_GEMV(64, 1);
    if (g > 8) {  // G = 16
        if (cpl16 == 3) FH_GEMV(16, 3);
        FH_GEMV(16, 4);
    }
    if (g > 4) FH_GEMV(8, 4);
    if (g > 2) FH_GEMV(4, 4);
    if (g > 1) FH_GEMV(2, 4);
    FH_GEMV(1, 4);
#undef FH_GEMV
}

template <int G>
int launch_w8a8(fh_ctx* ctx, const fh_q8_0* w, const int8_t* qx, const uint16_t* dx, size_t m, const float* bias,
                float* y) {
    constexpr int RW = 64 / G;
    const size_t pairs = m * w->n;
    const size_t sets = (pairs + RW - 1) / RW;
    const size_t blocks = (sets + 3) / 4;
    hipLaunchKernelGGL((k_linear_w8a8<G>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream, w->qs, w->d,
                       qx, dx, bias, y, static_cast<int>(m), static_cast<int>(w->n), static_cast<int>(w->k));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

}  // namespace

int fh_launch_linear_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                           int act) {
    if (reinterpret_cast<uintptr_t>(x) & 15)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x must be 16-byte aligned");
    if (w->n > 0x7FFFFFFFu || w->k > 0x7FFFFFFFu || m > 0x7FFFFFFFu)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: a dimension is above 2^31 - 1");
    if (m <= 2) {
        int rc = m == 1 ? dispatch_gemv<1>(ctx, w, x, bias, y, act) : dispatch_gemv<2>(ctx, w, x, bias, y, act);
        if (rc >= 0) return rc;
    }
    return fh_launch_gemm_w8a32(ctx, w, x, m, bias, y, act);
}

int fh_launch_gemv_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y) {
    if (m == 1) return dispatch_gemv<1>(ctx, w, x, bias, y, FH_ACT_NONE);
    if (m == 2) return dispatch_gemv<2>(ctx, w, x, bias, y, FH_ACT_NONE);
    return -1;
}

int fh_launch_linear_ln_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_ln_args& ln,
                              const float* bias, float* y, int act) {
    const bool aligned = !((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(ln.r) |
                            reinterpret_cast<uintptr_t>(ln.gamma) | reinterpret_cast<uintptr_t>(ln.beta) |
                            reinterpret_cast<uintptr_t>(ln.s)) & 15);
    if (m <= 2 && aligned && w->n <= 0x7FFFFFFFu) {
        int rc = m == 1 ? dispatch_gemv<1>(ctx, w, x, bias, y, act, &ln) : dispatch_gemv<2>(ctx, w, x, bias, y, act, &ln);
        if (rc >= 0) return rc;
    }
    // Other shapes: the add + LayerNorm kernel into the context's activation
    // area, then the plain linear.
    void* h = nullptr;
    int rc = fh_act_area(ctx, m * w->k * sizeof(float), &h);
    if (rc) return rc;
    rc = fh_launch_add_layernorm(ctx, x, ln.r, ln.s, m, w->k, ln.gamma, ln.beta, static_cast<float*>(h));
    if (rc) return rc;
    return fh_launch_linear_w8a32(ctx, w, static_cast<float*>(h), m, bias, y, act);
}

// (fast: the matrix-core kernels fuse each block term into the sum; the
// block-parallel kernel below sums blocks in parallel in either mode)
int fh_launch_linear_w8a8(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                          bool fast) {
    if (reinterpret_cast<uintptr_t>(x) & 3)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_linear: x must be 4-byte aligned");
    if (w->n > 0x7FFFFFFFu || w->k > 0x7FFFFFFFu || m * w->n > 0x7FFFFFFFu * size_t(64))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: problem too large for the W8A8 kernel");
    const size_t tile_rows = m >= 64 ? 64 : 32;
    if (m >= 32 && (m + tile_rows - 1) / tile_rows * ((w->n + 63) / 64) >= kW8a8MfmaTiles)
        return fh_launch_gemm_w8a8(ctx, w, x, m, bias, y, fast);
    const size_t kb = w->k / 32;
    const size_t qbytes = fh_align256(m * w->k), dbytes = fh_align256(m * kb * 2);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, qbytes + dbytes, &ws);
    if (rc) return rc;
    int8_t* qx = static_cast<int8_t*>(ws);
    uint16_t* dx = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + qbytes);
    const size_t nb = m * kb;
    hipLaunchKernelGGL(fh_k_encode_split, dim3(static_cast<unsigned>((nb + 255) / 256)), dim3(256), 0, ctx->stream, x,
                       nb, reinterpret_cast<uint32_t*>(qx), dx);
    FH_HIP(ctx, hipGetLastError());
    if (kb >= 64) return launch_w8a8<64>(ctx, w, qx, dx, m, bias, y);
    if (kb >= 16) return launch_w8a8<16>(ctx, w, qx, dx, m, bias, y);
    if (kb >= 4) return launch_w8a8<4>(ctx, w, qx, dx, m, bias, y);
    return launch_w8a8<1>(ctx, w, qx, dx, m, bias, y);
}
