// fh_internal.hpp — shared host/device definitions of libferrum_hip (gfx950).
//
// Device weight layout ("split planes", built once at upload):
//   qs : int8  [n][k]      the Q8_0 quants, row-major; every row starts 32-B
//                          aligned (k % 32 == 0), so a lane loads 16 quants
//                          with one 16-byte global load.
//   d  : uint16 [n][k/32]  the f16 block scales, as stored in GGUF.
// Together 34 B per 32 weights, exactly the GGUF footprint: the repack only
// separates GGUF's interleaved 34-byte blocks (which are 2-byte aligned) into
// two naturally aligned planes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/ferrum_hip.h"

struct fh_ctx {
    int device = 0;
    int num_cus = 1;             // compute units of the device
    hipStream_t own = nullptr;   // created by fh_ctx_create
    hipStream_t stream = nullptr;  // where work is enqueued (own, borrowed, or NULL = legacy default)
    std::string err;
    // Grow-on-demand device workspace for intermediate buffers (activation
    // quants, sampler rows).  Reused across calls on this context.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Zero-initialised device state that kernels leave zeroed again when they
    // finish (the split sampler's per-row barriers).  Never shares ws.
    void* sync = nullptr;
    size_t sync_bytes = 0;
    // Zero-initialised counters that kernels leave at zero (the split-K
    // GEMM's per-tile arrival counts).  Separate from sync: the sampler's
    // generation tags there must never be reset behind its back.
    void* counters = nullptr;
    size_t counters_bytes = 0;
    // Grow-on-demand activation staging (a LayerNorm output feeding a
    // linear), separate from ws, which the linear itself may use.
    void* act = nullptr;
    size_t act_bytes = 0;
    // Grow-on-demand device copies of the blocking calls' host arguments and
    // results (each blocking call synchronises before it returns, so one
    // area serves them all).
    void* io = nullptr;
    size_t io_bytes = 0;
    // Pinned host staging for the blocking calls' small arguments (one DMA
    // copy each way instead of one pageable copy per argument).
    void* pin = nullptr;
    size_t pin_bytes = 0;
    // Device status word: kernels OR in FH_STATUS_* bits (a bounded wait that
    // gave up, decreasing recent offsets); fh_sync and the blocking calls read
    // and clear it.
    unsigned* status = nullptr;
    // Workgroups of the split sampler one CU holds at once (occupancy API;
    // -1 until asked).
    int split_per_cu = -1;
    // Testing hooks (fh_debug_sampler_faults): a split-sampler segment that
    // publishes nothing, and a lower poll limit for the bounded waits.
    int test_skip_segment = -1;
    unsigned test_spin_limit = 0;
};

// Read and clear ctx->status after the stream has drained; FH_OK or the error
// its bits stand for.
int fh_take_status(fh_ctx* ctx);

constexpr int8_t kFhBadRowExp = -128;

// Weight storage kinds behind an fh_q8_0 handle.
enum { FH_WEIGHT_Q8_0 = 0, FH_WEIGHT_F32 = 1 };

struct fh_q8_0 {
    int device = 0;
    int kind = FH_WEIGHT_Q8_0;
    size_t n = 0, k = 0, kb = 0;
    // FH_WEIGHT_F32: rows [n][pitch] f32, pitch = k rounded up to 16 floats,
    // the padding zero (a tensor the reference stores as F32: ne0 % 32 != 0,
    // or an unquantized file).  qs / d / rexp unused.
    float* f32 = nullptr;
    size_t pitch = 0;
    int8_t* qs = nullptr;
    uint16_t* d = nullptr;
    // Per row j, e_j with 127 * max_b |d_jb| * 2^e_j in [2^14, 2^15) (0 for a
    // row without non-zero scales, kFhBadRowExp for a row with a non-finite
    // scale): every GEMM recomputes the flagged rows' outputs exactly (the
    // kernels read only the flag; e_j is the exponent an exact two-term f16
    // split of 2^e_j * d * q would take).  Derived from d at upload.
    int8_t* rexp = nullptr;
    void* base = nullptr;  // the one allocation holding all planes
};

// ---- error plumbing ---------------------------------------------------------
int fh_fail(fh_ctx* ctx, int code, const std::string& msg);
int fh_hip_fail(fh_ctx* ctx, hipError_t e, const char* what);
#define FH_HIP(ctx, call)                                          \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return fh_hip_fail((ctx), e_, #call); \
    } while (0)

// Make sure ctx->ws holds at least `bytes` (device, 256-B aligned).
int fh_workspace(fh_ctx* ctx, size_t bytes, void** out);
// The same for ctx->act.
int fh_act_area(fh_ctx* ctx, size_t bytes, void** out);
// Make sure ctx->sync holds at least `bytes`, zeroed when (re)allocated.
// Growing is refused while the stream is being captured into a graph.
int fh_sync_area(fh_ctx* ctx, size_t bytes, void** out);
// The same for ctx->counters.
int fh_counter_area(fh_ctx* ctx, size_t bytes, void** out);
// Round up to a multiple of 256 bytes.
static inline size_t fh_align256(size_t b) { return (b + 255) & ~(size_t)255; }

// ---- launchers implemented in the kernel translation units -------------------
int fh_launch_repack(fh_ctx* ctx, const uint8_t* d_raw, size_t n, size_t k, int8_t* qs,
                     uint16_t* d);
int fh_launch_row_exponents(fh_ctx* ctx, const uint16_t* d, size_t n, size_t kb, int8_t* rexp);
int fh_launch_unpack(fh_ctx* ctx, const int8_t* qs, const uint16_t* d, size_t n, size_t k,
                     uint8_t* d_raw);
int fh_launch_linear_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m,
                           const float* bias, float* y, int act = FH_ACT_NONE);
// LayerNorm of (x + r) feeding the linear; s (nullable) receives x + r.
struct fh_ln_args {
    const float* r;
    const float* gamma;
    const float* beta;
    float* s;
};
int fh_launch_linear_ln_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_ln_args& ln,
                              const float* bias, float* y, int act);
// The fused edges of the skinny GEMM (3 <= m <= 64).  Row statistics
// ("stats"): per row and 32-column group, the group's mean and sum of squared
// deviations (M2), [rows][groups][2] floats (k, n % 32 == 0).
struct fh_edge {
    float* stats;         // norm in: the input rows' statistics (read); residual out: y's (written)
    const float* gamma;   // norm in: LayerNorm gamma / RmsNorm weight
    const float* beta;    // norm in: LayerNorm beta (null: RmsNorm)
    float eps;            // norm in
    int rms;              // norm in: 1 = RmsNorm
    const float* r;       // residual out: y = r + (x W^T + b); may be y itself
};
// y = act(norm(x) W^T + b), the norm formed from e.stats as the activations
// are staged; -1 for a shape the skinny GEMM does not take.
int fh_launch_skinny_norm_in(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_edge& e,
                             const float* bias, float* y, int act);
// y = r + (x W^T + b) and y's row statistics into e.stats; -1 for a shape the
// skinny GEMM does not take (n % 32 != 0 included).
int fh_launch_skinny_res_out(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_edge& e,
                             const float* bias, float* y);
// The same two edges as separate kernels (any shape): y += ... is done by
// the caller's plain linear; these add the residual and form the statistics
// (k_residual_stats), or normalise rows from statistics (k_norm_from_stats).
int fh_launch_residual_stats(fh_ctx* ctx, const float* t, const float* r, float* y, size_t rows, size_t n,
                             float* stats);
int fh_launch_norm_from_stats(fh_ctx* ctx, const float* x, size_t rows, size_t k, const fh_edge& e, float* out);
// act (FH_ACT_*) is applied to the outputs: in the skinny GEMM's epilogue at
// m <= 64, else by the separate GELU kernel.
int fh_launch_gemm_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m,
                         const float* bias, float* y, int act = FH_ACT_NONE);
// The decode GEMV alone (m <= 2, W8A32, no workspace); -1 when the row is too
// long for it (the caller then takes the GEMM).
int fh_launch_gemv_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y);
// A device scratch area a caller owns (no allocation by the launcher).
struct fh_scratch {
    void* ptr;
    size_t bytes;
};
// The skinny GEMM (3 <= m <= 64) with its split-K partials and arrival
// counters in `scratch` (counters cleared by a kernel first); FH_ERR_LIMIT when
// the shape needs more than scratch.bytes.
int fh_launch_skinny_scratch(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                             const fh_scratch& scratch);
// W8A8 (fast: FH_W8A8_FAST, each block term fused into the sum by one FMA).
int fh_launch_gemm_w8a8(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m,
                        const float* bias, float* y, bool fast);
int fh_launch_linear_w8a8(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m,
                          const float* bias, float* y, bool fast);
// FH_W8A32_EXACT: ferrum_core's sequential sums, bit for bit (no K split).
int fh_launch_linear_exact(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y);
int fh_launch_encode(fh_ctx* ctx, const float* x, size_t n, uint8_t* out);
int fh_launch_embed_rows_pos(fh_ctx* ctx, const float* tok_w, const float* pos_w, size_t vocab, size_t max_seq,
                             size_t d, const uint32_t* tokens, const uint32_t* pos, size_t rows, uint32_t* hist,
                             size_t hist_stride, float* out);
int fh_launch_embed_one(fh_ctx* ctx, const float* tok_w, const float* pos_w, size_t vocab, size_t d,
                        const uint32_t* token, size_t pos, float* out);
int fh_launch_layernorm(fh_ctx* ctx, const float* x, size_t rows, size_t d, const float* gamma,
                        const float* beta, float* y);
int fh_launch_gelu(fh_ctx* ctx, float* x, size_t n);
int fh_launch_add(fh_ctx* ctx, float* x, const float* y, size_t n);
// ln = LayerNorm(x + y) (y nullable: LayerNorm(x)); s (nullable, may be x)
// receives x + y.  d <= 2048.
int fh_launch_add_layernorm(fh_ctx* ctx, const float* x, const float* y, float* s, size_t rows, size_t d,
                            const float* gamma, const float* beta, float* ln);
// A prompt block of `rows` consecutive positions pos0 .. pos0 + rows - 1 of
// one sequence: their k / v rows into the cache, then each row's attention.
int fh_launch_attention_prefill(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t d, size_t heads,
                                size_t pos0, size_t rows, float* out);
// The same for `seqs` sequences at once (sequence s: rows s * rows .. of qkv
// and out, caches at kc / vc + s * seq_stride): head width 64 on the fp32
// matrix cores (fh_attn_prefill.hip), others one sequence at a time.
int fh_launch_attention_prefill_seqs(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t seq_stride,
                                     size_t d, size_t heads, size_t pos0, size_t rows, size_t seqs, float* out);
int fh_launch_attention_decode(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t d, size_t heads,
                               size_t pos, float* out);
int fh_launch_gqa_attention_decode(fh_ctx* ctx, const float* qkv, size_t ld, size_t rows, size_t n_heads, size_t n_kv,
                                   size_t hd, float* kc, float* vc, size_t cap, const uint32_t* dpos, size_t max_pos,
                                   float* out);
// The same with apply_rope on each row's q and k first (fh_launch_rope's
// rotation, inside the attention kernel for batched launches, else
// fh_launch_rope in place on qkv's q and k heads before the attention).
int fh_launch_gqa_attention_rope_decode(fh_ctx* ctx, float* qkv, size_t ld, size_t rows, size_t n_heads, size_t n_kv,
                                        size_t hd, float* kc, float* vc, size_t cap, const uint32_t* dpos,
                                        size_t max_pos, size_t rope_dim, float base, int rope_type,
                                        const float* freq_factors, float linear_factor, float* out);
int fh_launch_rmsnorm(fh_ctx* ctx, const float* x, const float* r, float* s, size_t rows, size_t d, const float* w,
                      float eps, float* out);
int fh_launch_rope(fh_ctx* ctx, float* x, size_t rows, size_t ld, size_t n_heads, size_t hd, size_t rope_dim,
                   const uint32_t* dpos, float base, int rope_type, const float* freq_factors, float linear_factor);
int fh_launch_swiglu(fh_ctx* ctx, const float* g, const float* u, size_t rows, size_t n, size_t ld, float* out);
int fh_launch_embed_rows(fh_ctx* ctx, const float* tok_w, size_t vocab, size_t d, const uint32_t* tokens, size_t rows,
                         float* out);
int fh_launch_dequant(fh_ctx* ctx, const uint8_t* raw, size_t n, float* out);
int fh_launch_block_dots(fh_ctx* ctx, const fh_q8_0* w, const int8_t* qx, size_t m,
                         int32_t* dots);
int fh_launch_sample(fh_ctx* ctx, const float* logits, size_t rows, size_t vocab, int kind,
                     const fh_sampling_params* p, const uint32_t* recent,
                     const uint32_t* offsets, const uint64_t* draws, uint32_t* out);

// ---- device helpers ---------------------------------------------------------
#ifdef __HIPCC__
// IEEE half -> float, exact for every code (gguf/dequant.rs:7-35 semantics; the
// hardware conversion is exact, subnormals included).
__device__ __forceinline__ float fh_h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

namespace fh {
// apply_rope's rotation of one pair (llm.rs:146-175, the angle of
// RopeScaling::angle, llm.rs:118-121): pair i of rope_dim / 2 at position
// pos, the frequency in float64 then rounded, as the reference computes it;
// one definition for every kernel that rotates, so they give the same bits.
__device__ __forceinline__ void rope_rotate(float& a, float& b, int pos, int i, int rope_dim, float base,
                                            const float* ff, float linear_factor) {
#pragma clang fp contract(off)
    const float freq = static_cast<float>(pow(static_cast<double>(base), -2.0 * i / static_cast<double>(rope_dim)));
    const float f = ff ? ff[i] : 1.0f;
    const float theta = static_cast<float>(pos) * freq / f * (1.0f / linear_factor);
    const float sn = sinf(theta), cs = cosf(theta);
    const float x = a, y = b;
    a = x * cs - y * sn;
    b = x * sn + y * cs;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rdlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over each group of G consecutive lanes (G a power of two <= 16), every
// lane of the group ending with the same total: quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if (G >= 2) v += dpp<0xB1>(v);
    if (G >= 4) v += dpp<0x4E>(v);
    if (G >= 8) v += dpp<0x141>(v);
    if (G >= 16) v += dpp<0x140>(v);
    return v;
}

// Sum over each group of G lanes for any power of two G <= 64 (every lane of
// the group gets the total): 16-lane rows by DPP, then across rows with
// readlane.
template <int G>
__device__ __forceinline__ float group_total(float v) {
    if constexpr (G <= 16) {
        return group_sum<G>(v);
    } else {
        const float r16 = group_sum<16>(v);
        const float lo = rdlane(r16, 0) + rdlane(r16, 16);
        const float hi = rdlane(r16, 32) + rdlane(r16, 48);
        return G == 64 ? lo + hi : ((threadIdx.x & 63) < 32 ? lo : hi);
    }
}

// Sum over the workgroup in a fixed order (wave sums, then waves in order);
// red holds one float per wave.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < static_cast<int>(blockDim.x >> 6); i++) s += red[i];
    return s;
}
}  // namespace fh
#endif
