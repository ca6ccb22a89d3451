// fh_q8_0.hip — Q8_0 block codec on gfx950: weight repack/unpack at upload,
// the bit-exact Q8_0 encoder (weights and W8A8 activations), dequant, and the
// int32 block-dot checking kernel.
//
// Encode semantics (quant::q8_0_block, ferrum_core/src/quant.rs:271-280):
//   amax = fold(0, max(|x_i|))      f32::max ignores NaN; fmaxf does too
//   d    = amax / 127               IEEE division (hipcc's default '/' is
//                                   correctly rounded, div_scale/div_fixup)
//   id   = d != 0 ? 1 / d : 0
//   q_i  = saturate_i8(round_half_away(x_i * id)), NaN -> 0   (Rust `as i8`)
//   scale stored as f32_to_f16(d)   (gguf_write/blocks.rs:12-61)
// Quantization uses the f32 d; only the stored scale is rounded to f16.
#include "fh_internal.hpp"

namespace {

constexpr int kThreads = 256;

// IEEE binary16 encode with round-to-nearest-even, overflow to Inf, Inf kept,
// NaN -> sign | 0x7E00 (the reference's canonical quiet NaN).  Finite values
// and infinities use the hardware conversion (v_cvt_f16_f32 rounds to nearest
// even and keeps f16 subnormals under the default FP16 denormal mode); NaN is
// canonicalised by hand because the hardware keeps payload bits.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0)
        return static_cast<uint16_t>(((u >> 16) & 0x8000u) | 0x7E00u);
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Rust `f32::round(v) as i8`: half away from zero, saturating, NaN -> 0.
__device__ __forceinline__ int round_sat_i8(float v) {
    float r = roundf(v);
    if (r != r) return 0;
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return static_cast<int>(r);
}

// One Q8_0 block: 32 consecutive floats -> 32 int8 (packed into 8 dwords) and
// the f16 scale.
__device__ __forceinline__ uint16_t encode_block(const float* __restrict__ x, uint32_t q[8]) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = x[i];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float p = v[w * 4 + b] * id;
            word |= (static_cast<uint32_t>(round_sat_i8(p)) & 0xFFu) << (8 * b);
        }
        q[w] = word;
    }
    return f32_to_f16_bits(d);
}

// GGUF layout (34-byte blocks, 2-byte aligned) -> split planes.
__global__ void __launch_bounds__(kThreads) k_repack(const uint16_t* __restrict__ raw, size_t nblocks,
                                                     uint32_t* __restrict__ qs, uint16_t* __restrict__ d) {
    size_t b = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (b >= nblocks) return;
    const uint16_t* src = raw + b * 17;
    d[b] = src[0];
    uint32_t* dst = qs + b * 8;
#pragma unroll
    for (int w = 0; w < 8; w++) dst[w] = static_cast<uint32_t>(src[1 + 2 * w]) | (static_cast<uint32_t>(src[2 + 2 * w]) << 16);
}

// One thread per weight row: e = 15 - E for 127 * max_b |d_b| = f * 2^E,
// f in [0.5, 1); 0 for a row of zero scales, kFhBadRowExp if any scale is
// inf or NaN.
__global__ void __launch_bounds__(kThreads) k_row_exponents(const uint16_t* __restrict__ d, size_t n, size_t kb,
                                                            int8_t* __restrict__ rexp) {
    size_t j = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (j >= n) return;
    float mx = 0.0f;
    bool bad = false;
    for (size_t b = 0; b < kb; b++) {
        const float v = fabsf(fh_h2f(d[j * kb + b]));
        if (v <= 65504.0f) mx = fmaxf(mx, v);
        else bad = true;  // inf or NaN
    }
    int e = 0;
    if (mx > 0.0f) {
        const float top = mx * 127.0f;  // exact: 11 x 7 significant bits
        e = 15 - (static_cast<int>((__builtin_bit_cast(uint32_t, top) >> 23) & 0xFF) - 126);
    }
    rexp[j] = bad ? kFhBadRowExp : static_cast<int8_t>(e);
}

__global__ void __launch_bounds__(kThreads) k_unpack(const uint32_t* __restrict__ qs, const uint16_t* __restrict__ d,
                                                     size_t nblocks, uint16_t* __restrict__ raw) {
    size_t b = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (b >= nblocks) return;
    uint16_t* dst = raw + b * 17;
    dst[0] = d[b];
    const uint32_t* src = qs + b * 8;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        dst[1 + 2 * w] = static_cast<uint16_t>(src[w] & 0xFFFFu);
        dst[2 + 2 * w] = static_cast<uint16_t>(src[w] >> 16);
    }
}

// f32 -> GGUF Q8_0 bytes, one block per thread.
__global__ void __launch_bounds__(kThreads) k_encode_gguf(const float* __restrict__ x, size_t nblocks,
                                                          uint16_t* __restrict__ out) {
    size_t b = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (b >= nblocks) return;
    uint32_t q[8];
    uint16_t d16 = encode_block(x + b * 32, q);
    uint16_t* dst = out + b * 17;
    dst[0] = d16;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        dst[1 + 2 * w] = static_cast<uint16_t>(q[w] & 0xFFFFu);
        dst[2 + 2 * w] = static_cast<uint16_t>(q[w] >> 16);
    }
}

__global__ void __launch_bounds__(kThreads) k_dequant(const uint16_t* __restrict__ raw, size_t nblocks,
                                                      float* __restrict__ out) {
    size_t b = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (b >= nblocks) return;
    const uint16_t* src = raw + b * 17;
    float d = fh_h2f(src[0]);
#pragma unroll
    for (int w = 0; w < 16; w++) {
        uint16_t pair = src[1 + w];
        out[b * 32 + 2 * w] = d * static_cast<float>(static_cast<int8_t>(pair & 0xFF));
        out[b * 32 + 2 * w + 1] = d * static_cast<float>(static_cast<int8_t>(pair >> 8));
    }
}

// dots[i, j, b] for int8 activations [m, k] against the weight quants.  One
// thread per (i, j, b); sdot4 is exact integer arithmetic.
__global__ void __launch_bounds__(kThreads) k_block_dots(const int8_t* __restrict__ qx, const int8_t* __restrict__ qs,
                                                         size_t m, size_t n, size_t kb, int32_t* __restrict__ dots) {
    size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (t >= m * n * kb) return;
    size_t b = t % kb, j = (t / kb) % n, i = t / (kb * n);
    const int* a = reinterpret_cast<const int*>(qx + i * kb * 32 + b * 32);
    const int* w = reinterpret_cast<const int*>(qs + j * kb * 32 + b * 32);
    int s = 0;
#pragma unroll
    for (int u = 0; u < 8; u++) s = __builtin_amdgcn_sdot4(a[u], w[u], s, false);
    dots[t] = s;
}

inline unsigned grid_for(size_t items) { return static_cast<unsigned>((items + kThreads - 1) / kThreads); }

}  // namespace

// f32 [m, k] -> split-plane Q8_0 activations (qx int8 [m, k], dx f16 [m, k/32]).
// Used by the W8A8 linear; same per-block arithmetic as the GGUF encoder.
__global__ void __launch_bounds__(256) fh_k_encode_split(const float* __restrict__ x, size_t nblocks,
                                                         uint32_t* __restrict__ qx, uint16_t* __restrict__ dx) {
    size_t b = blockIdx.x * static_cast<size_t>(256) + threadIdx.x;
    if (b >= nblocks) return;
    uint32_t q[8];
    dx[b] = encode_block(x + b * 32, q);
    uint4* dst = reinterpret_cast<uint4*>(qx + b * 8);
    dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
    dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
}

// f32 [m, k] -> Q8_0 activations in the W8A8 matrix-core panel: per 32-row
// tile and block b (a fragment), 1 KiB of quants in MFMA lane order (lane
// g * 32 + r holds row r's quants 16 g .. 16 g + 15) and the 32 row scales
// as f32.  Rows m .. m_pad - 1 are zero.  Same per-block arithmetic as the
// GGUF encoder.  One wave per fragment: lane g * 32 + r reads row r's
// elements 16 g .. 16 g + 15 and writes exactly their 16 panel bytes (the
// wave's stores are one contiguous KiB); the block's maximum is the larger
// of the two halves' (fmaxf drops NaN in any order, so it is the same value).
// V4: x is 16-byte aligned (float4 loads); otherwise 4-byte loads.
template <bool V4>
__global__ void __launch_bounds__(256) fh_k_encode_panel(const float* __restrict__ x, int m, int m_pad, int kb,
                                                         uint4* __restrict__ qp, float* __restrict__ dp) {
    const int lane = threadIdx.x & 63;
    const size_t frag = blockIdx.x * static_cast<size_t>(4) + (threadIdx.x >> 6);  // tile * kb + b
    if (frag >= static_cast<size_t>(m_pad / 32) * kb) return;  // (the whole wave)
    const int tile = static_cast<int>(frag / kb), b = static_cast<int>(frag % kb);
    const int r = lane & 31, g = lane >> 5, row = tile * 32 + r;
    float v[16];
    if (row < m) {
        const float* src = x + (static_cast<size_t>(row) * kb + b) * 32 + g * 16;
        if (V4) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 f = reinterpret_cast<const float4*>(src)[i];
                v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = src[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t q[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) word |= (static_cast<uint32_t>(round_sat_i8(v[w * 4 + e] * id)) & 0xFFu) << (8 * e);
        q[w] = word;
    }
    qp[frag * 64 + lane] = make_uint4(q[0], q[1], q[2], q[3]);
    if (g == 0) dp[frag * 32 + r] = fh_h2f(f32_to_f16_bits(d));
}

template __global__ void fh_k_encode_panel<true>(const float*, int, int, int, uint4*, float*);
template __global__ void fh_k_encode_panel<false>(const float*, int, int, int, uint4*, float*);

int fh_launch_repack(fh_ctx* ctx, const uint8_t* d_raw, size_t n, size_t k, int8_t* qs, uint16_t* d) {
    if (reinterpret_cast<uintptr_t>(d_raw) & 1)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_upload: device bytes must be 2-byte aligned");
    size_t nb = n * (k / 32);
    hipLaunchKernelGGL(k_repack, dim3(grid_for(nb)), dim3(kThreads), 0, ctx->stream,
                       reinterpret_cast<const uint16_t*>(d_raw), nb, reinterpret_cast<uint32_t*>(qs), d);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_row_exponents(fh_ctx* ctx, const uint16_t* d, size_t n, size_t kb, int8_t* rexp) {
    hipLaunchKernelGGL(k_row_exponents, dim3(grid_for(n)), dim3(kThreads), 0, ctx->stream, d, n, kb, rexp);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_unpack(fh_ctx* ctx, const int8_t* qs, const uint16_t* d, size_t n, size_t k, uint8_t* d_raw) {
    size_t nb = n * (k / 32);
    hipLaunchKernelGGL(k_unpack, dim3(grid_for(nb)), dim3(kThreads), 0, ctx->stream,
                       reinterpret_cast<const uint32_t*>(qs), d, nb, reinterpret_cast<uint16_t*>(d_raw));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_encode(fh_ctx* ctx, const float* x, size_t n, uint8_t* out) {
    if ((reinterpret_cast<uintptr_t>(x) & 3) || (reinterpret_cast<uintptr_t>(out) & 1))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_encode: x must be 4-byte and out 2-byte aligned");
    size_t nb = n / 32;
    hipLaunchKernelGGL(k_encode_gguf, dim3(grid_for(nb)), dim3(kThreads), 0, ctx->stream, x, nb,
                       reinterpret_cast<uint16_t*>(out));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_dequant(fh_ctx* ctx, const uint8_t* raw, size_t n, float* out) {
    if ((reinterpret_cast<uintptr_t>(raw) & 1) || (reinterpret_cast<uintptr_t>(out) & 3))
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_dequant: bytes must be 2-byte and out 4-byte aligned");
    size_t nb = n / 32;
    hipLaunchKernelGGL(k_dequant, dim3(grid_for(nb)), dim3(kThreads), 0, ctx->stream,
                       reinterpret_cast<const uint16_t*>(raw), nb, out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_block_dots(fh_ctx* ctx, const fh_q8_0* w, const int8_t* qx, size_t m, int32_t* dots) {
    if (reinterpret_cast<uintptr_t>(qx) & 3)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_q8_0_block_dots: qx must be 4-byte aligned");
    size_t total = m * w->n * w->kb;
    hipLaunchKernelGGL(k_block_dots, dim3(grid_for(total)), dim3(kThreads), 0, ctx->stream, qx, w->qs, m,
                       w->n, w->kb, dots);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
