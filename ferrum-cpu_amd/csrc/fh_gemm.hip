// fh_gemm.hip — Q8_0 W8A32 linear for m >= 3 on the gfx950 matrix cores.
//
//   y[i, j] = sum_b d_jb * sum_{p in block b} x[i, p] * q[j, p]  (+ bias[j])
//
// is ferrum_core's ops::linear_forward on the f32 expansion W = f16(d) * q of a
// GGUF Q8_0 tensor (ops.rs:233-256, gguf/dequant.rs:37-49).  The quants are
// integers in [-127, 127], exact in f16, so the inner block sums run on
// v_mfma_f32_32x32x16_f16 once the activations are in f16 too.  An f32
// activation keeps its 24-bit significand as two f16 terms:
//
//   x[i, p] * 2^e_i = h + l,   h = f16(x * 2^e_i),   l = f16(x * 2^e_i - h)
//
// with one power-of-two scale per row (the row's largest finite |x| lands in
// [2^14, 2^15), so neither term overflows and l stays normal for every value
// that matters).  h + l carries 22 significant bits; the products h*q and l*q
// are exact and the matrix core sums them in f32.  Each Q8_0 block's partial
// sum (four MFMAs: h and l, two K halves) is scaled by the block's weight
// scale with one FMA per output into the running f32 sum; the row scale 2^-e_i
// is applied exactly at the end, and the bias is added last, as the reference
// does.  Non-finite activations keep l = 0, so inf and NaN propagate as they
// do in the reference's products (inf * 0 = NaN, inf * q = inf).
//
// Work split: for the mid-size tiles k_split_rows writes the h/l terms once
// per call into a panel laid out for the GEMM's staging ([row tile][block]
// [row][h 32 | l 32], 128 B per row and block, so a stage is one contiguous
// read); the large-m block-scaled kernel (k_gemm_bscale) instead takes only
// the row scales (k_row_scales, one read of x) and splits the activations
// while staging them, which saves the panel's write and re-read.  k_gemm_mfma stages
// KW Q8_0 blocks of the activation panel and of the weight rows per step into
// LDS (double buffered, one barrier per step), converting the int8 quants to
// f16 on the way in; each wave owns TM x TN 32x32 output tiles, and with
// KW > 1 the waves split the K blocks and add their sums in wave order (a
// fixed order: results do not depend on timing).
#include "fh_internal.hpp"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // staging registers (a struct copy would go through scratch)
typedef float f4 __attribute__((ext_vector_type(4)));

// Staged rows, in f16 elements.  Activations: 32 h, 32 l, 8 pad (144 B);
// weights: 32 quants, 8 pad (80 B).  Both strides keep the 16 lanes of a
// ds_read_b128 phase (16 consecutive rows) on disjoint banks.
constexpr int kArow = 72;
constexpr int kBrow = 40;

// Four int8 quants to four f16, exactly: bias the bytes to unsigned, place each
// in the mantissa of 1024.0 (0x6400 | u == 1024 + u), subtract 1152.
__device__ __forceinline__ uint2 quants_to_f16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2 off = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const h2 a = __builtin_bit_cast(h2, lo) - off;
    const h2 b = __builtin_bit_cast(h2, hi) - off;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

__device__ __forceinline__ bool finite(float v) { return (__builtin_bit_cast(uint32_t, v) & 0x7F800000u) != 0x7F800000u; }

// activation::gelu (activation.rs:9-12) with every product and sum rounded
// (the kernels here are built with contraction on), so the GEMM epilogues
// give k_gelu's values bit for bit.
__device__ __forceinline__ float gelu_unfused(float v) {
#pragma clang fp contract(off)
    return 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * v * v * v)));
}

// Outputs whose activation row holds inf/NaN (large-m kernel) or whose weight
// row has a non-finite block scale (every kernel) are recomputed this way: the
// reference's own arithmetic (ops.rs:29-126 on the f32 expansion), products
// and sums rounded separately in ascending p, so the inf/NaN pattern (inf * 0
// = NaN, inf - inf = NaN) and the value are the reference's bit for bit.
__device__ __attribute__((noinline)) float exact_dot(const float* __restrict__ x, int k, const int8_t* __restrict__ q,
                                                   const uint16_t* __restrict__ d) {
#pragma clang fp contract(off)  // plain operators: no FMA, each product and sum rounded
    float s = 0.0f;
    for (int b = 0; b < (k >> 5); b++) {
        const float ds = fh_h2f(d[b]);
        for (int t = 0; t < 32; t++)
            s = s + x[b * 32 + t] * (ds * static_cast<float>(q[b * 32 + t]));
    }
    return s;
}

// The outputs of one tile whose activation row is flagged (xbad, may be null)
// or whose weight row has a non-finite scale, recomputed by exact_dot (then
// GELU with act).  Every thread of the workgroup calls; a barrier first
// orders the tile's ordinary stores before these.
__device__ __attribute__((noinline)) void exact_tile(const float* __restrict__ x, const int8_t* __restrict__ qs,
                                                     const uint16_t* __restrict__ dsc, const int8_t* __restrict__ rexp,
                                                     const uint8_t* __restrict__ xbad, const float* __restrict__ bias,
                                                     float* __restrict__ y, int m, int n, int k, int i0, int j0,
                                                     int bm, int bn, int act) {
    __syncthreads();
    for (int o = threadIdx.x; o < bm * bn; o += blockDim.x) {
        const int i = i0 + o / bn, j = j0 + o % bn;
        if (i >= m || j >= n || !((xbad && xbad[i]) || rexp[j] == kFhBadRowExp)) continue;
        const float s = exact_dot(x + static_cast<size_t>(i) * k, k, qs + static_cast<size_t>(j) * k,
                                  dsc + static_cast<size_t>(j) * (k >> 5));
        const float v = bias ? s + bias[j] : s;
        y[static_cast<size_t>(i) * n + j] = act == FH_ACT_GELU ? gelu_unfused(v) : v;
    }
}

// exact_dot on the normalised row (x - mean) * rs * gamma + beta (RmsNorm:
// mean 0, no beta): the rare outputs of a weight row with a non-finite block
// scale when the GEMM normalises its input.
__device__ __attribute__((noinline)) float exact_dot_norm(const float* __restrict__ x, const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, const float* __restrict__ st,
                                                        int groups, int rms, float eps, int k,
                                                        const int8_t* __restrict__ q, const uint16_t* __restrict__ d) {
#pragma clang fp contract(off)
    // the row's statistics from its group statistics (sequential sums)
    float sm = 0.0f;
    for (int g = 0; g < groups; g++) sm += st[2 * g];
    const float mu = rms ? 0.0f : sm / static_cast<float>(groups);
    float m2 = 0.0f;
    for (int g = 0; g < groups; g++) {
        const float dm = st[2 * g] - mu;
        m2 += st[2 * g + 1] + 32.0f * dm * dm;
    }
    const float rsi = 1.0f / sqrtf(m2 / static_cast<float>(k) + eps);
    float s = 0.0f;
    for (int b = 0; b < (k >> 5); b++) {
        const float ds = fh_h2f(d[b]);
        for (int t = 0; t < 32; t++) {
            const int c = b * 32 + t;
            const float a = (x[c] - mu) * rsi * gamma[c] + (beta ? beta[c] : 0.0f);
            s = s + a * (ds * static_cast<float>(q[c]));
        }
    }
    return s;
}

}  // namespace

// One wave per activation row (rows m .. m_pad - 1 are written as zeros).
__global__ void __launch_bounds__(256)
    k_split_rows(const float* __restrict__ x, int m, int m_pad, int k, int bm, uint4* __restrict__ panel,
                 float* __restrict__ xinv, uint8_t* __restrict__ xbad) {
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= m_pad) return;
    const int kb = k >> 5, chunks = k >> 3;
    const bool live = row < m;
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(live ? row : 0) * k);
    float mx = 0.0f;
    bool bad = false;
    if (live) {
        for (int c = lane; c < chunks; c += 64) {
            const float4 a = xr[2 * c], b = xr[2 * c + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                if (finite(v[t])) mx = fmaxf(mx, fabsf(v[t]));
                else bad = true;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) xbad[row] = __ballot(bad) != 0;
    // mx = f * 2^E with f in [0.5, 1): scale by 2^(15 - E).  A subnormal
    // maximum reads E = -126 and clamps like any tiny row.
    int e = 0;
    if (mx > 0.0f) {
        const int E = static_cast<int>((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFF) - 126;
        e = min(max(15 - E, -126), 126);
    }
    const float sc = __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23);
    if (lane == 0) xinv[row] = __builtin_bit_cast(float, static_cast<uint32_t>(127 - e) << 23);
    uint4* dst_row = panel + (static_cast<size_t>(row / bm) * kb * bm + row % bm) * 8;
    for (int c = lane; c < chunks; c += 64) {
        float v[8] = {};
        if (live) {
            const float4 a = xr[2 * c], b = xr[2 * c + 1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
        h8 hv, lv;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float s = v[t] * sc;
            const _Float16 h = static_cast<_Float16>(s);
            hv[t] = h;
            lv[t] = finite(s) ? static_cast<_Float16>(s - static_cast<float>(h)) : static_cast<_Float16>(0.0f);
        }
        uint4* dst = dst_row + static_cast<size_t>(c >> 2) * bm * 8;
        dst[c & 3] = __builtin_bit_cast(uint4, hv);
        dst[4 + (c & 3)] = __builtin_bit_cast(uint4, lv);
    }
}

// The row scales and flags of k_split_rows without the panel: the
// block-scaled GEMM splits the activations itself while staging them (one read of x here
// instead of a read and a write of the whole panel).  Rows m .. m_pad - 1 get
// scale 1 and no flag.
__global__ void __launch_bounds__(256)
    k_row_scales(const float* __restrict__ x, int m, int m_pad, int k, float* __restrict__ xinv,
                 uint8_t* __restrict__ xbad) {
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= m_pad) return;
    const int chunks = k >> 3;
    float mx = 0.0f;
    bool bad = false;
    if (row < m) {
        const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * k);
        for (int c = lane; c < chunks; c += 64) {
            const float4 a = xr[2 * c], b = xr[2 * c + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                if (finite(v[t])) mx = fmaxf(mx, fabsf(v[t]));
                else bad = true;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    const bool any_bad = __ballot(bad) != 0;
    // the same scale as k_split_rows: 2^(15 - E) for mx = f * 2^E, f in [0.5, 1)
    int e = 0;
    if (mx > 0.0f) {
        const int E = static_cast<int>((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFF) - 126;
        e = min(max(15 - E, -126), 126);
    }
    if (lane == 0) {
        xbad[row] = any_bad;
        xinv[row] = __builtin_bit_cast(float, static_cast<uint32_t>(127 - e) << 23);
    }
}

// Workgroup tile BM x BN; NW = WM x WN x KW waves (output sub-tiles x
// K-slices).  Tiles are numbered so that consecutive workgroups on one XCD
// (the hardware deals workgroup ids round-robin over the 8 XCDs) take
// consecutive tiles of one activation row-tile, which then stays in that XCD's L2.
template <int BM, int BN, int WM, int WN, int KW>
__global__ void __launch_bounds__(64 * WM * WN * KW)
    k_gemm_mfma(const uint4* __restrict__ panel, const float* __restrict__ xinv, const float* __restrict__ x,
                const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc, const int8_t* __restrict__ rexp,
                const float* __restrict__ bias, float* __restrict__ y, int m, int n, int k, int tiles_n) {
    constexpr int NW = WM * WN * KW, NT = 64 * NW;
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    constexpr int TM = BM / (32 * WM), TN = BN / (32 * WN);
    static_assert(TM >= 1 && TN >= 1 && TM * 32 * WM == BM && TN * 32 * WN == BN, "tile shape");
    constexpr int A_BYTES = KW * BM * kArow * 2, B_BYTES = KW * BN * kBrow * 2, S_BYTES = KW * BN * 4;
    constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    // 16-byte pieces per thread (the last weight round may leave threads idle)
    constexpr int AP = KW * BM * 8 / NT, BPN = KW * BN * 2, BP = (BPN + NT - 1) / NT;
    static_assert(AP * NT == KW * BM * 8 && KW * BN <= NT, "staging split");
    constexpr int RED = (KW - 1) * WM * WN * TM * TN * 16 * 64 * 4;
    static_assert(RED + BM * 4 <= 2 * STAGE, "reduction and row scales fit the stage buffers");
    __shared__ __attribute__((aligned(16))) char lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kw = wave / (WM * WN), wm = (wave % (WM * WN)) / WN, wn = wave % WN;
    const int tiles = static_cast<int>(gridDim.x), per_xcd = tiles / 8, rem = tiles % 8;
    const int xcd = static_cast<int>(blockIdx.x) % 8, slot = static_cast<int>(blockIdx.x) / 8;
    const int tile = xcd * per_xcd + min(xcd, rem) + slot;  // XCDs 0 .. rem-1 take one extra tile
    const int tile_m = tile / tiles_n, tile_n = tile % tiles_n;
    const int j0 = tile_n * BN;
    const int kb = k >> 5, steps = (kb + KW - 1) / KW;
    const uint4* pan = panel + static_cast<size_t>(tile_m) * kb * BM * 8;

    uint4 ra[AP], rb[BP];
    float rs = 0.0f;
    auto load = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < AP; p++) {
            const int piece = tid + NT * p, blk = piece / (BM * 8), rem = piece % (BM * 8);
            const int b = st * KW + blk;
            ra[p] = b < kb ? pan[static_cast<size_t>(b) * BM * 8 + rem] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int p = 0; p < BP; p++) {
            const int piece = tid + NT * p, blk = piece / (BN * 2), rem = piece % (BN * 2);
            const int b = st * KW + blk, j = j0 + rem / 2;
            rb[p] = (piece < BPN && b < kb && j < n)
                        ? *reinterpret_cast<const uint4*>(qs + static_cast<size_t>(j) * k + b * 32 + (rem & 1) * 16)
                        : make_uint4(0, 0, 0, 0);
        }
        if (tid < KW * BN) {
            const int b = st * KW + tid / BN, j = j0 + tid % BN;
            rs = (b < kb && j < n) ? fh_h2f(dsc[static_cast<size_t>(j) * kb + b]) : 0.0f;
        }
    };
    auto store = [&](int buf) __attribute__((always_inline)) {
        char* st = lds + buf * STAGE;
#pragma unroll
        for (int p = 0; p < AP; p++) {
            const int piece = tid + NT * p, blk = piece / (BM * 8), rem = piece % (BM * 8);
            *reinterpret_cast<uint4*>(st + ((blk * BM + rem / 8) * kArow) * 2 + (rem % 8) * 16) = ra[p];
        }
#pragma unroll
        for (int p = 0; p < BP; p++) {
            const int piece = tid + NT * p, blk = piece / (BN * 2), rem = piece % (BN * 2);
            if (BPN % NT != 0 && piece >= BPN) break;
            char* dst = st + A_BYTES + ((blk * BN + rem / 2) * kBrow) * 2 + (rem & 1) * 32;
            const uint2 a = quants_to_f16(rb[p].x), b = quants_to_f16(rb[p].y);
            const uint2 c = quants_to_f16(rb[p].z), d = quants_to_f16(rb[p].w);
            *reinterpret_cast<uint4*>(dst) = make_uint4(a.x, a.y, b.x, b.y);
            *reinterpret_cast<uint4*>(dst + 16) = make_uint4(c.x, c.y, d.x, d.y);
        }
        if (tid < KW * BN) reinterpret_cast<float*>(st + A_BYTES + B_BYTES)[tid] = rs;
    };

    f16x acc[TM][TN];
#pragma unroll
    for (int r = 0; r < TM; r++)
#pragma unroll
        for (int c = 0; c < TN; c++) acc[r][c] = f16x{};
    const f16x zero = {};

    load(0);
    store(0);
    __syncthreads();
    const int arow = lane % 32, koff = (lane / 32) * 8;
    for (int st = 0; st < steps; st++) {
        const int buf = st & 1;
        if (st + 1 < steps) load(st + 1);
        const char* sb = lds + buf * STAGE;
        const _Float16* As = reinterpret_cast<const _Float16*>(sb) + kw * BM * kArow;
        const _Float16* Bs = reinterpret_cast<const _Float16*>(sb + A_BYTES) + kw * BN * kBrow;
        const float* Ss = reinterpret_cast<const float*>(sb + A_BYTES + B_BYTES) + kw * BN;
        // Weight fragments and scales for all column tiles, then one row tile
        // at a time (its four activation fragments, then its MFMAs).
        h8 bq[TN][2];
        float dw[TN];
#pragma unroll
        for (int c = 0; c < TN; c++) {
            const int col = (wn * TN + c) * 32 + arow;
            const _Float16* b = Bs + col * kBrow + koff;
            bq[c][0] = *reinterpret_cast<const h8*>(b);
            bq[c][1] = *reinterpret_cast<const h8*>(b + 16);
            dw[c] = Ss[col];
        }
#pragma unroll
        for (int r = 0; r < TM; r++) {
            const _Float16* a = As + ((wm * TM + r) * 32 + arow) * kArow + koff;
            const h8 ah0 = *reinterpret_cast<const h8*>(a), ah1 = *reinterpret_cast<const h8*>(a + 16);
            const h8 al0 = *reinterpret_cast<const h8*>(a + 32), al1 = *reinterpret_cast<const h8*>(a + 48);
#pragma unroll
            for (int c = 0; c < TN; c++) {
                f16x p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah0, bq[c][0], zero, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al0, bq[c][0], p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah1, bq[c][1], p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al1, bq[c][1], p, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) acc[r][c][v] = fmaf(dw[c], p[v], acc[r][c][v]);
            }
        }
        if (st + 1 < steps) store(buf ^ 1);
        __syncthreads();
    }

    if (KW > 1) {
        // K-slices 1..KW-1 hand their sums to slice 0 through LDS; slice 0 adds
        // them in slice order.
        float* red = reinterpret_cast<float*>(lds);
        const int sub = wave % (WM * WN);
        if (kw > 0) {
#pragma unroll
            for (int r = 0; r < TM; r++)
#pragma unroll
                for (int c = 0; c < TN; c++)
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        red[((((kw - 1) * WM * WN + sub) * TM + r) * TN + c) * 1024 + v * 64 + lane] = acc[r][c][v];
        }
        __syncthreads();
        if (kw == 0) {
#pragma unroll
            for (int s = 1; s < KW; s++)
#pragma unroll
                for (int r = 0; r < TM; r++)
#pragma unroll
                    for (int c = 0; c < TN; c++)
#pragma unroll
                        for (int v = 0; v < 16; v++)
                            acc[r][c][v] += red[((((s - 1) * WM * WN + sub) * TM + r) * TN + c) * 1024 + v * 64 + lane];
        }
    }

    // Row scales of this tile through LDS (the stage buffers are free).
    const int i0 = tile_m * BM;
    float* s_inv = reinterpret_cast<float*>(lds) + RED / 4;
    __syncthreads();
    for (int t = tid; t < BM; t += NT) s_inv[t] = xinv[i0 + t];  // rows < m_pad
    __syncthreads();
    if (KW == 1 || kw == 0) {  // K-slice 0 holds the totals
#pragma unroll
        for (int c = 0; c < TN; c++) {
            const int j = j0 + (wn * TN + c) * 32 + arow;
            if (j >= n) continue;
            const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
            for (int r = 0; r < TM; r++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int il = (wm * TM + r) * 32 + (v / 4) * 8 + (lane / 32) * 4 + (v % 4), i = i0 + il;
                    if (i >= m) continue;
                    const float s = acc[r][c][v] * s_inv[il];
                    y[static_cast<size_t>(i) * n + j] = bias ? s + bj : s;
                }
        }
    }
    // Rare: weight rows with a non-finite scale are rewritten with the
    // reference's own arithmetic (inf/NaN activations propagate exactly here).
    bool flagged = false;
    for (int t = tid; t < BN; t += NT) flagged |= j0 + t < n && rexp[j0 + t] == kFhBadRowExp;
    if (__syncthreads_or(flagged)) exact_tile(x, qs, dsc, rexp, nullptr, bias, y, m, n, k, i0, j0, BM, BN, FH_ACT_NONE);
}

// ---- large m, block-scaled: the quants as the weight operand -------------------------
// W8A32 for a prompt's linears without folding the block scales into the
// weights: the weight operand is the int8 quants themselves (exact in f16),
// so a Q8_0 block of a 32 x 32 tile is four MFMAs (the activation's h and l
// terms, two K halves) giving the block's partial sum sum_p (h + l) q in f32,
// and one FMA per output adds it times the block scale d_jb to the running
// f32 sum.  Folding the scales into the weights instead (d * q has up to 19
// significant bits: two f16 terms, x_h w_h + x_h w_l + x_l w_h, six MFMAs per
// block) costs half as much again on the matrix cores and a costlier weight
// staging; here the price is 16 FMAs per tile and block on the VALU.  The
// activations are split as in k_gemm_mfma (row scale 2^e_i from
// k_row_scales, h = f16(x 2^e_i), l = f16(x 2^e_i - h)); the sum is scaled by
// 2^-e_i at the end (exact), then the bias is added and GELU applied.  Rows
// with inf/NaN activations and weight rows with a non-finite scale are
// recomputed with the reference's own arithmetic (exact_tile).
// Workgroup tile 256 x 256, eight waves of 128 x 64 (4 x 2 tiles), one Q8_0
// block per stage, two stages of 51 KiB: the activations as [row tile][term
// h|l][MFMA half][lane] (16-byte fragments: lane g * 32 + r holds row r's
// elements 16 g + 8 half .. + 7), the quants as [MFMA half][lane half]
// [column] and the 256 columns' block scales.  Block b + 1 is loaded into
// registers while block b's MFMAs run and is split and stored into the other
// stage between their two halves.
// (each 16-byte-fragment plane is padded by 64 bytes: the two lanes of a
// staging pair write the same slot of neighbouring planes, which then fall on
// different banks)
constexpr int kBsAPlane = 68, kBsBPlane = 260;  // 16-byte entries
constexpr int kBsAOff = 0, kBsBOff = 32 * kBsAPlane * 16, kBsSOff = kBsBOff + 4 * kBsBPlane * 16;
constexpr int kBsStage = kBsSOff + 256 * 4;

__global__ void __launch_bounds__(512)
    k_gemm_bscale(const float* __restrict__ xinv, const uint8_t* __restrict__ xbad, const float* __restrict__ x,
                  const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc, const int8_t* __restrict__ rexp,
                  const float* __restrict__ bias, float* __restrict__ y, int m, int n, int k, int tiles_n, int act) {
    constexpr int TM = 4, TN = 2, BM = 256, BN = 256, NTH = 512;
    __shared__ __attribute__((aligned(16))) char lds[2 * kBsStage];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
    const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves
    const int tiles = static_cast<int>(gridDim.x), per_xcd = tiles / 8, rem = tiles % 8;
    const int xcd = static_cast<int>(blockIdx.x) % 8, slot = static_cast<int>(blockIdx.x) / 8;
    const int tile = xcd * per_xcd + min(xcd, rem) + slot;
    const int tile_m = tile / tiles_n, tile_n = tile % tiles_n;
    const int i0 = tile_m * BM, j0 = tile_n * BN, kb = k >> 5;
    // This thread's activation pieces: row wave * 32 + lane / 2 of the tile,
    // elements 16 s + 8 (lane % 2) .. + 7 for s = 0, 1 (two lanes read 64
    // contiguous bytes of a row).  Rows past m repeat row m - 1 (never stored).
    const int ar = lane >> 1, ahf = lane & 1;
    const float* xsrc = x + static_cast<size_t>(min(i0 + wave * 32 + ar, m - 1)) * k + ahf * 8;
    // 2^e from the stored 2^-e (both exact powers of two)
    const float xsc = __builtin_bit_cast(float, (254u << 23) - __builtin_bit_cast(uint32_t, xinv[i0 + wave * 32 + ar]));
    // Weight half-row (column tid / 2, half tid % 2); waves 0-3 also load the
    // block scale of column tid.  Columns past n repeat column n - 1.
    const int bcol = tid >> 1, bhalf = tid & 1;
    const int8_t* wsrc = qs + static_cast<size_t>(min(j0 + bcol, n - 1)) * k + bhalf * 16;
    const bool scale_loader = __builtin_amdgcn_readfirstlane(wave) < 4;
    const uint16_t* dsrc = dsc + static_cast<size_t>(min(j0 + (tid & 255), n - 1)) * kb;
    u4 ra[2], rb;  // one activation piece in flight at a time
    uint16_t rd = 0;
    auto load_a = [&](int b, int s2) __attribute__((always_inline)) {
        ra[0] = *reinterpret_cast<const u4*>(xsrc + b * 32 + s2 * 16);
        ra[1] = *reinterpret_cast<const u4*>(xsrc + b * 32 + s2 * 16 + 4);
    };
    auto load_b = [&](int b) __attribute__((always_inline)) {
        rb = *reinterpret_cast<const u4*>(wsrc + b * 32);
        if (scale_loader) rd = dsrc[b];
    };
    auto store_a = [&](int buf, int s2) __attribute__((always_inline)) {
        uint4* As = reinterpret_cast<uint4*>(lds + buf * kBsStage + kBsAOff);
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int p2 = 0; p2 < 2; p2++) {
            const f4 sv = __builtin_bit_cast(f4, ra[p2]) * xsc;  // exact (power of two)
            const f2 s01 = {sv.x, sv.y}, s23 = {sv.z, sv.w};
            const h2 h01 = __builtin_convertvector(s01, h2), h23 = __builtin_convertvector(s23, h2);
            // (no guard for inf / NaN: such a row's outputs are recomputed)
            const f2 r01 = {sv.x - static_cast<float>(h01.x), sv.y - static_cast<float>(h01.y)};
            const f2 r23 = {sv.z - static_cast<float>(h23.x), sv.w - static_cast<float>(h23.y)};
            hw[2 * p2] = __builtin_bit_cast(uint32_t, h01);
            hw[2 * p2 + 1] = __builtin_bit_cast(uint32_t, h23);
            lw[2 * p2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r01, h2));
            lw[2 * p2 + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r23, h2));
        }
        const int frag = s2 * 32 + ar;  // lane g * 32 + r of the fragment
        As[((wave * 2) * 2 + ahf) * kBsAPlane + frag] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        As[((wave * 2 + 1) * 2 + ahf) * kBsAPlane + frag] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    };
    auto store_b = [&](int buf) __attribute__((always_inline)) {
        char* st = lds + buf * kBsStage;
        uint4* Bs = reinterpret_cast<uint4*>(st + kBsBOff);
        const uint2 q0 = quants_to_f16(rb[0]), q1 = quants_to_f16(rb[1]), q2 = quants_to_f16(rb[2]),
                    q3 = quants_to_f16(rb[3]);
        Bs[bhalf * kBsBPlane + bcol] = make_uint4(q0.x, q0.y, q1.x, q1.y);
        Bs[(2 + bhalf) * kBsBPlane + bcol] = make_uint4(q2.x, q2.y, q3.x, q3.y);
        if (scale_loader) reinterpret_cast<float*>(st + kBsSOff)[tid] = fh_h2f(rd);
    };
    float acc[TM][TN][16];
#pragma unroll
    for (int r = 0; r < TM; r++)
#pragma unroll
        for (int c = 0; c < TN; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[r][c][v] = 0.0f;

    load_a(0, 0);
    store_a(0, 0);
    load_a(0, 1);
    load_b(0);
    store_a(0, 1);
    store_b(0);
    __syncthreads();
    for (int b = 0; b < kb; b++) {
        const int buf = b & 1;
        const int bn = b + 1 < kb ? b + 1 : b;  // (at the last block: this block again, into the unused stage)
        load_a(bn, 0);
        load_b(bn);
        const char* st = lds + buf * kBsStage;
        const h8* As = reinterpret_cast<const h8*>(st + kBsAOff);
        const h8* Bs = reinterpret_cast<const h8*>(st + kBsBOff);
        const float* Sw = reinterpret_cast<const float*>(st + kBsSOff);
        h8 bf[TN][2];
        float dw[TN];
#pragma unroll
        for (int c = 0; c < TN; c++) {
            const int col = (wn * TN + c) * 32 + l32;
            bf[c][0] = Bs[g * kBsBPlane + col];
            bf[c][1] = Bs[(2 + g) * kBsBPlane + col];
            dw[c] = Sw[col];
        }
        auto rows = [&](int r0, int r1) __attribute__((always_inline)) {
#pragma unroll
            for (int r = r0; r < r1; r++) {
                const int rt = wm * TM + r;
                const h8 ah0 = As[((rt * 2) * 2) * kBsAPlane + lane], ah1 = As[((rt * 2) * 2 + 1) * kBsAPlane + lane];
                const h8 al0 = As[((rt * 2 + 1) * 2) * kBsAPlane + lane],
                         al1 = As[((rt * 2 + 1) * 2 + 1) * kBsAPlane + lane];
#pragma unroll
                for (int c = 0; c < TN; c++) {
                    f16x d = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah0, bf[c][0], f16x{}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah1, bf[c][1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(al0, bf[c][0], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(al1, bf[c][1], d, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        acc[r][c][v] = __builtin_fmaf(d[v], dw[c], acc[r][c][v]);
                        asm volatile("" : "+v"(acc[r][c][v]));  // (keeps the sum before the fence below)
                    }
                }
                __builtin_amdgcn_sched_barrier(0);  // row tiles in order: bounds the live partial sums
            }
        };
        // (the other stage is free since the last barrier)
        rows(0, 1);
        store_a(buf ^ 1, 0);
        load_a(bn, 1);
        rows(1, 3);
        store_a(buf ^ 1, 1);
        store_b(buf ^ 1);
        rows(3, TM);
        __syncthreads();
    }

    // Row scales and flags of this tile through LDS.
    float* s_inv = reinterpret_cast<float*>(lds);
    uint8_t* s_bad = reinterpret_cast<uint8_t*>(lds + BM * 4);
    for (int t = tid; t < BM; t += NTH) {  // rows < m_pad: the arrays cover them
        s_inv[t] = xinv[i0 + t];
        s_bad[t] = xbad[i0 + t];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < TN; c++) {
        const int j = j0 + (wn * TN + c) * 32 + l32;
        if (j >= n) continue;
        const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
        for (int r = 0; r < TM; r++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int il = (wm * TM + r) * 32 + (v >> 2) * 8 + g * 4 + (v & 3), i = i0 + il;
                if (i >= m) continue;
                const float sv = acc[r][c][v] * s_inv[il];
                const float o = bias ? sv + bj : sv;
                y[static_cast<size_t>(i) * n + j] = act == FH_ACT_GELU ? gelu_unfused(o) : o;
            }
    }
    bool flagged = false;
    for (int t = tid; t < BM || t < BN; t += NTH)
        flagged |= (t < BM && s_bad[t]) || (t < BN && j0 + t < n && rexp[j0 + t] == kFhBadRowExp);
    if (__syncthreads_or(flagged)) exact_tile(x, qs, dsc, rexp, xbad, bias, y, m, n, k, i0, j0, BM, BN, act);
}

// ---- W8A8 on the int8 matrix cores ---------------------------------------------------
// llama.cpp numerics (the activations re-quantised to Q8_0 per 32):
//   y[i, j] = sum_b f32(dot_b(i, j)) * (d_w[j, b] * d_x[i, b])  (+ bias[j], last)
// One v_mfma_i32_32x32x32_i8 is one Q8_0 block of a 32 x 32 output tile: the
// int32 block dots are exact; each is scaled and added to the f32 sum in
// ascending b with separately rounded products and sums, the reference's own
// order, so the outputs are the reference's bit for bit.  That per-block VALU
// epilogue (convert, two products, add: 64 instructions per MFMA) bounds the
// kernel, not the matrix cores.  Each wave owns a (32 TM) x 64 output tile and
// reads its fragments straight from global memory: the activation panel
// (fh_k_encode_panel) in MFMA lane order, 1 KiB contiguous per fragment; the
// weight rows 16 bytes per lane.  The next block's operands are loaded while
// the current one is finished.
template <int TM, bool FAST>
__global__ void __launch_bounds__(256)
    k_gemm_w8a8(const uint4* __restrict__ qp, const float* __restrict__ dp, const int8_t* __restrict__ qs,
                const uint16_t* __restrict__ dsc, const float* __restrict__ bias, float* __restrict__ y, int m, int n,
                int k, int tiles_n, int tiles) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    typedef int i16 __attribute__((ext_vector_type(16)));
    constexpr int TN = 2;
    const int lane = threadIdx.x & 63, g = lane >> 5, l32 = lane & 31;
    const int wid = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
    if (wid >= tiles) return;  // no barriers below
    const int tm = wid / tiles_n, tn = wid % tiles_n;
    const int kb = k >> 5;
    const int j0 = tn * 64;
    const int8_t* wrow[TN];
    const uint16_t* drow[TN];
#pragma unroll
    for (int c = 0; c < TN; c++) {
        const int j = min(j0 + c * 32 + l32, n - 1);  // rows past n: computed, never stored
        wrow[c] = qs + static_cast<size_t>(j) * k + g * 16;
        drow[c] = dsc + static_cast<size_t>(j) * kb;
    }
    struct Ops {
        i4 a[TM], w[TN];
        f4 dx[TM][4];
        uint16_t dw[TN];
    };
    auto load = [&](Ops& o, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < TM; r++) {
            const size_t t = static_cast<size_t>(tm * TM + r) * kb + b;
            o.a[r] = __builtin_bit_cast(i4, qp[t * 64 + lane]);
#pragma unroll
            for (int q = 0; q < 4; q++) o.dx[r][q] = *reinterpret_cast<const f4*>(dp + t * 32 + q * 8 + g * 4);
        }
#pragma unroll
        for (int c = 0; c < TN; c++) {
            o.w[c] = *reinterpret_cast<const i4*>(wrow[c] + b * 32);
            o.dw[c] = drow[c][b];
        }
    };
    float acc[TM][TN][16];
#pragma unroll
    for (int r = 0; r < TM; r++)
#pragma unroll
        for (int c = 0; c < TN; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[r][c][v] = 0.0f;
    auto finish = [&](const Ops& o) __attribute__((always_inline)) {
#pragma clang fp contract(off)  // plain operators: separately rounded products and sums
#pragma unroll
        for (int c = 0; c < TN; c++) {
            const float dw = fh_h2f(o.dw[c]);
#pragma unroll
            for (int r = 0; r < TM; r++) {
                const i16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[r], o.w[c], i16{}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    // acc row (v / 4) * 8 + g * 4 + v % 4: its scale is dx[v / 4][v % 4]
                    const float dd = dw * o.dx[r][v >> 2][v & 3];
                    if (FAST) acc[r][c][v] = __builtin_fmaf(static_cast<float>(d[v]), dd, acc[r][c][v]);
                    else acc[r][c][v] = acc[r][c][v] + static_cast<float>(d[v]) * dd;
                }
            }
        }
    };
    Ops o0, o1;
    load(o0, 0);
    for (int b = 0; b < kb; b += 2) {
        if (b + 1 < kb) load(o1, b + 1);
        finish(o0);
        if (b + 1 >= kb) break;
        if (b + 2 < kb) load(o0, b + 2);
        finish(o1);
    }
#pragma unroll
    for (int c = 0; c < TN; c++) {
        const int j = j0 + c * 32 + l32;
        if (j >= n) continue;
        const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
        for (int r = 0; r < TM; r++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = (tm * TM + r) * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
                if (i < m) y[static_cast<size_t>(i) * n + j] = bias ? acc[r][c][v] + bj : acc[r][c][v];
            }
    }
}

// W8A8 for large m (a prompt's linears), the same arithmetic as k_gemm_w8a8
// (every output the same bits), with the operands staged through LDS: a
// workgroup owns a 256 x 256 output tile (eight waves of 128 x 64, 4 x 2
// 32 x 32 tiles) and stages one Q8_0 block of it at a time.  Each operand byte
// crosses from memory once per workgroup instead of once per wave.
// The block terms are formed on the matrix cores, leaving two VALU
// operations per output and block (the product and the sum):
//  * the int8 quants are staged as f16 (exact), and two
//    v_mfma_f32_32x32x16_f16 give the block dot as an f32 that is the exact
//    integer (|dot| <= 32 * 128 * 128 < 2^24, so every partial sum is
//    exact whatever the order inside the MFMA);
//  * d_w * d_x is the product of two f16 values, exact in f32, so one
//    v_mfma_f32_32x32x1_2b_f32 outer product (32 row scales x 64 column
//    scales, no other term) gives it for both 32 x 32 tiles of a row tile, in
//    the accumulators' own register layout; inf and NaN scales propagate as
//    in the scalar product, and a zero's sign cannot reach a sum that
//    starts at +0.
// Then acc = acc + dot * dd with the product and the sum rounded separately,
// in ascending b, as the reference does.  A stage (35 KiB): the eight 32-row
// activation fragments as [row tile][MFMA half][lane] (the panel is in MFMA
// lane order already), the 256 weight half-rows as [MFMA half][lane half]
// [column] (a fragment read is 32 consecutive 16-byte pieces), the rows'
// activation scales and the columns' weight scales.  Two stages: block b + 1
// is loaded into registers while block b's MFMAs and epilogue run, and
// converted and stored into the other stage between the two halves of them.
// Workgroups are dealt to XCDs in contiguous runs of tiles.  The panel covers
// whole 256-row tiles.
constexpr int kW8Rows = 256, kW8Cols = 256, kW8Threads = 512;
constexpr int kW8BPlane = 260;  // 16-byte entries (padded: see the block-scaled kernel)
constexpr int kW8BOff = 16 * 1024, kW8SOff = kW8BOff + 4 * kW8BPlane * 16;
constexpr int kW8StageBytes = kW8SOff + 256 * 4 + 256 * 4;
constexpr size_t kW8LdsMinRows = 1024;  // m from which W8A8 takes the staged kernel

template <bool FAST>
__global__ void __launch_bounds__(kW8Threads)
    k_gemm_w8a8_lds(const uint4* __restrict__ qp, const float* __restrict__ dp, const int8_t* __restrict__ qs,
                    const uint16_t* __restrict__ dsc, const float* __restrict__ bias, float* __restrict__ y, int m,
                    int n, int k, int tiles_n) {
    typedef float f32x __attribute__((ext_vector_type(32)));
    constexpr int TM = 4, TN = 2;
    __shared__ __attribute__((aligned(16))) char lds[2 * kW8StageBytes];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, l32 = lane & 31;
    const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves
    const int tiles = static_cast<int>(gridDim.x), per_xcd = tiles / 8, rem = tiles % 8;
    const int xcd = static_cast<int>(blockIdx.x) % 8, slot = static_cast<int>(blockIdx.x) / 8;
    const int tile = xcd * per_xcd + min(xcd, rem) + slot;
    const int tile_m = tile / tiles_n, tile_n = tile % tiles_n;
    const int j0 = tile_n * kW8Cols, kb = k >> 5;
    // This thread's staging pieces: activation fragment (row tile tid / 64,
    // lane tid % 64), weight half-row (column tid / 2, half tid % 2), and
    // one scale: the row scale of row tid (tid < 256) or the weight scale of
    // column tid - 256.  Columns past n repeat column n - 1 (never stored).
    const int art = tid >> 6, alane = tid & 63;
    const size_t a_base = static_cast<size_t>(tile_m * 8 + art) * kb;
    const int bcol = tid >> 1, bhalf = tid & 1;
    const int8_t* wsrc = qs + static_cast<size_t>(min(j0 + bcol, n - 1)) * k + bhalf * 16;
    // (waves 0-3 hold row scales, 4-7 weight scales: a wave-uniform branch,
    // and the f16 weight scale is widened at the store, so that no wave waits
    // for its loads where it issues them)
    const bool row_scale = __builtin_amdgcn_readfirstlane(wave) < 4;
    const int sc_i = tid & 255;
    const float* dsrc_x = dp + static_cast<size_t>(tile_m * 8 + (sc_i >> 5)) * kb * 32 + (sc_i & 31);
    const uint16_t* dsrc_w = dsc + static_cast<size_t>(min(j0 + sc_i, n - 1)) * kb;
    uint4 ra, rb;
    uint32_t rs;  // the scale's bits: f32 (row scale) or f16 (weight scale)
    auto load = [&](int b) __attribute__((always_inline)) {
        ra = qp[(a_base + b) * 64 + alane];
        rb = *reinterpret_cast<const uint4*>(wsrc + b * 32);
        if (row_scale) rs = __builtin_bit_cast(uint32_t, dsrc_x[static_cast<size_t>(b) * 32]);
        else rs = dsrc_w[b];
    };
    auto store = [&](int buf) __attribute__((always_inline)) {
        char* st = lds + buf * kW8StageBytes;
        uint4* As = reinterpret_cast<uint4*>(st);
        uint4* Bs = reinterpret_cast<uint4*>(st + kW8BOff);
        uint2 q0 = quants_to_f16(ra.x), q1 = quants_to_f16(ra.y), q2 = quants_to_f16(ra.z), q3 = quants_to_f16(ra.w);
        As[(art * 2) * 64 + alane] = make_uint4(q0.x, q0.y, q1.x, q1.y);
        As[(art * 2 + 1) * 64 + alane] = make_uint4(q2.x, q2.y, q3.x, q3.y);
        q0 = quants_to_f16(rb.x), q1 = quants_to_f16(rb.y), q2 = quants_to_f16(rb.z), q3 = quants_to_f16(rb.w);
        Bs[bhalf * kW8BPlane + bcol] = make_uint4(q0.x, q0.y, q1.x, q1.y);
        Bs[(2 + bhalf) * kW8BPlane + bcol] = make_uint4(q2.x, q2.y, q3.x, q3.y);
        // [0, 256): row scales, [256, 512): weight scales
        reinterpret_cast<float*>(st + kW8SOff)[tid] =
            row_scale ? __builtin_bit_cast(float, rs) : fh_h2f(static_cast<uint16_t>(rs));
    };
    float acc[TM][TN][16];
#pragma unroll
    for (int r = 0; r < TM; r++)
#pragma unroll
        for (int c = 0; c < TN; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[r][c][v] = 0.0f;

    load(0);
    store(0);
    __syncthreads();
    for (int b = 0; b < kb; b++) {
        const int buf = b & 1;
        if (b + 1 < kb) load(b + 1);
        const char* st = lds + buf * kW8StageBytes;
        const h8* As = reinterpret_cast<const h8*>(st);
        const h8* Bs = reinterpret_cast<const h8*>(st + kW8BOff);
        const float* Ss = reinterpret_cast<const float*>(st + kW8SOff);
        h8 bf[TN][2];
#pragma unroll
        for (int c = 0; c < TN; c++) {
            const int col = (wn * TN + c) * 32 + l32;
            bf[c][0] = Bs[g * kW8BPlane + col];
            bf[c][1] = Bs[(2 + g) * kW8BPlane + col];
        }
        const float dw = Ss[256 + wn * 64 + lane];  // lane half c: column tile c of this wave
        auto rows = [&](int r0, int r1) __attribute__((always_inline)) {
#pragma clang fp contract(off)  // plain operators: separately rounded products and sums
#pragma unroll
            for (int r = r0; r < r1; r++) {
                const int rt = wm * TM + r;
                const h8 a0 = As[(rt * 2) * 64 + lane], a1 = As[(rt * 2 + 1) * 64 + lane];
                // dd[16 c + v]: d_w * d_x of output v of this lane in column tile c
                const f32x dd = __builtin_amdgcn_mfma_f32_32x32x1f32(Ss[rt * 32 + l32], dw, f32x{}, 0, 0, 0);
#pragma unroll
                for (int c = 0; c < TN; c++) {
                    f16x d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[c][0], f16x{}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[c][1], d, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        if (FAST) acc[r][c][v] = __builtin_fmaf(d[v], dd[c * 16 + v], acc[r][c][v]);
                        else acc[r][c][v] = acc[r][c][v] + d[v] * dd[c * 16 + v];
                    }
                }
            }
        };
        rows(0, TM / 2);
        // (the other stage is free since the last barrier; at the last block
        // it is rewritten with this block's pieces, never read again)
        store(buf ^ 1);
        rows(TM / 2, TM);
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < TN; c++) {
        const int j = j0 + (wn * TN + c) * 32 + l32;
        if (j >= n) continue;
        const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
        for (int r = 0; r < TM; r++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = tile_m * kW8Rows + (wm * TM + r) * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
                if (i < m) y[static_cast<size_t>(i) * n + j] = bias ? acc[r][c][v] + bj : acc[r][c][v];
            }
    }
}

// ---- skinny m (batched decode): m <= 32 * MT ------------------------------------
// Grid: 32-wide weight-row tiles x S splits of the Q8_0 blocks.  A workgroup's
// waves divide its split's blocks and issue every load of a batch of up to BPW
// blocks at once (weights straight into registers: each weight byte is used by
// one workgroup).  Activations are split per (row, block) instead of per row,
// so no pre-pass is needed: the two lanes holding a row's block agree on the
// block's power-of-two scale through one lane swap, and the block partial is
// unscaled exactly (t = P * 2^-e) before the weight-scale FMA.  Inside a block
// the K order is permuted (lane half h holds elements 16h .. 16h + 15; MFMA 0
// takes the first 8 of each half, MFMA 1 the rest) identically for activations
// and weights, so every product still pairs x[i, p] with q[j, p].
// Sums: over the waves in wave order (LDS), then over the splits in split
// order by whichever workgroup of the tile finishes last (a counter per tile,
// left at zero for the next launch) -- a fixed order either way.
namespace {

constexpr int kMaxSplits = 8;  // K splits of the skinny GEMM

// 16 activations (one lane's half of a row's block) times 2^e as h + l; the
// caller has handled blocks whose maximum is not finite (SAFE keeps l = 0 for
// inf and NaN inputs).
template <bool SAFE>
__device__ __forceinline__ void split16(const float* v, float sc, h8& ah0, h8& ah1, h8& al0, h8& al1) {
#pragma unroll
    for (int q = 0; q < 16; q += 2) {
        const f2 s = {v[q] * sc, v[q + 1] * sc};
        const h2 h = __builtin_convertvector(s, h2);
        f2 r = {s.x - static_cast<float>(h.x), s.y - static_cast<float>(h.y)};
        if (SAFE) {
            r.x = finite(s.x) ? r.x : 0.0f;
            r.y = finite(s.y) ? r.y : 0.0f;
        }
        const h2 l = __builtin_convertvector(r, h2);
        if (q < 8) {
            ah0[q] = h.x; ah0[q + 1] = h.y; al0[q] = l.x; al0[q + 1] = l.y;
        } else {
            ah1[q - 8] = h.x; ah1[q - 7] = h.y; al1[q - 8] = l.x; al1[q - 7] = l.y;
        }
    }
}

// Four activations times 2^e as packed f16 h and l (split16's arithmetic).
template <bool SAFE>
__device__ __forceinline__ void split4(const float* v, float sc, uint2& h, uint2& l) {
    uint32_t hw[2], lw[2];
#pragma unroll
    for (int q = 0; q < 4; q += 2) {
        const f2 s = {v[q] * sc, v[q + 1] * sc};
        const h2 hh = __builtin_convertvector(s, h2);
        f2 r = {s.x - static_cast<float>(hh.x), s.y - static_cast<float>(hh.y)};
        if (SAFE) {
            r.x = finite(s.x) ? r.x : 0.0f;
            r.y = finite(s.y) ? r.y : 0.0f;
        }
        hw[q / 2] = __builtin_bit_cast(uint32_t, hh);
        lw[q / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, h2));
    }
    h = make_uint2(hw[0], hw[1]);
    l = make_uint2(lw[0], lw[1]);
}

// Staging row of the skinny kernel: 32 floats + 4 pad, so the 16 lanes of a
// ds_read_b128 pass (16 rows) land on distinct banks.
constexpr int kSkinnyRow = 36;

// What the skinny GEMM does at its edges (k_gemm_skinny's MODE).
// kSkinnyNormGlu: kSkinnyNormIn, and the weight's rows are gate and up
// interleaved in groups of 32, so each workgroup's two column groups are the
// gate and the up of the same 32 outputs, which leave as silu(gate) * up.
enum { kSkinnyPlain = 0, kSkinnyNormIn = 1, kSkinnyResOut = 2, kSkinnyNormGlu = 3 };

__device__ __forceinline__ int block_exponent(float mx) {
    if (!(mx > 0.0f)) return 0;
    const int E = static_cast<int>((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFF) - 126;
    return min(max(15 - E, -126), 126);
}

}  // namespace


// FeedForward's gate (llm.rs:415-421), (g / (1 + exp(-g))) * u, rounded as
// k_swiglu rounds it.
__device__ __forceinline__ float swiglu_unfused(float g, float u) {
#pragma clang fp contract(off)
    return (g / (1.0f + expf(-g))) * u;
}

// MODE kSkinnyPlain: y = act(x W^T + b).  kSkinnyNormIn: the input is
// norm(x) (LayerNorm or RmsNorm), formed as the activations are staged from
// the rows' statistics a kSkinnyResOut launch left (fh_edge).  kSkinnyResOut:
// y = r + (x W^T + b) (y may be r) and, per row and 32-column group of y,
// the group's mean and sum of squared deviations into e.stats.
// kSkinnyNormGlu (NT = 2): as kSkinnyNormIn, y = silu(g) * u, [m][n / 2].
template <int MT, int NT, int BPW, int MODE>
__global__ void __launch_bounds__(512)
    k_gemm_skinny(const float* __restrict__ x, const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc,
                  const int8_t* __restrict__ rexp, const float* __restrict__ bias, float* y, int m, int n,
                  int k, int bps, float* __restrict__ part, unsigned* __restrict__ counters, int act, fh_edge e) {
    constexpr int OUT = MT * NT * 1024;  // outputs of one workgroup
    // Per wave, [SLOT] floats: during the K loop one Q8_0 block of its
    // activation rows ([MT * 32][36]: the rows land there from row-contiguous
    // loads and leave in MFMA lane order), afterwards its OUT sums; then
    // [KW][MT][BPW][32] row scales.
    constexpr int SLOT = OUT > MT * 32 * kSkinnyRow ? OUT : MT * 32 * kSkinnyRow;
    constexpr bool NORM = MODE == kSkinnyNormIn || MODE == kSkinnyNormGlu;
    constexpr bool GLU = MODE == kSkinnyNormGlu;
    static_assert(!GLU || NT == 2, "the gate and up groups are a workgroup's two column groups");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ int last;
    float* sums = lds;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kw = blockDim.x >> 6;
    const int kb = k >> 5, half = lane >> 5, r32 = lane & 31;
    const int tile = blockIdx.x, split = blockIdx.y, splits = gridDim.y;
    const int b_begin = split * bps, b_end = min(kb, b_begin + bps);
    const int8_t* wrow[NT];
    const uint16_t* drow[NT];
    // The outputs this thread stores at the end are all in column r32 of the
    // tiles, so their bias and row flags load now, beside the first weights
    // (loaded per output in the epilogue, each would cost a round trip).
    float bias_c[NT];
    bool bad_c[NT];
#pragma unroll
    for (int c = 0; c < NT; c++) {
        const int j = min((tile * NT + c) * 32 + r32, n - 1);
        wrow[c] = qs + static_cast<size_t>(j) * k + half * 16;
        drow[c] = dsc + static_cast<size_t>(j) * kb;
        bias_c[c] = bias ? bias[j] : 0.0f;
        bad_c[c] = rexp[j] == kFhBadRowExp;
    }
    float* inv_lds = lds + kw * SLOT + wave * (MT * BPW * 32);  // this wave's row scales
    float* xst = lds + wave * SLOT;                              // this wave's staging rows
    const float* nm_beta = NORM && e.beta ? e.beta : e.gamma;
    // kSkinnyNormIn: the mean and 1 / sd of the rows this lane stages (row t *
    // 32 + lane / 8 + 8 q) from their group statistics ([rows][k / 32][2]: per
    // 32-column group its mean and M2).  The eight lanes staging a row split
    // its groups (lane & 7 takes groups lane & 7, + 8, ...) and sum them with
    // an eight-lane tree in a fixed order: mean = the mean of the group means,
    // M2 = sum of (M2_g + 32 (mean_g - mean)^2); LayerNorm: 1 / sqrt(M2 / k +
    // eps); RmsNorm: mean 0, 1 / sqrt(sum of (M2_g + 32 mean_g^2) / k + eps).
    // Kept per wave in LDS, [row] = (mean, 1 / sd) (registers held across the
    // K loop would spill the wider tiles).  (Issuing the K loop's first batch
    // before the statistics are reduced timed no faster and spilled the
    // 64-row, two-group tiles.)
    __shared__ float2 rowf[NORM ? 8 : 1][NORM ? MT * 32 : 1];
    constexpr int kJ = 4;  // groups per lane at most (k <= 1024)
    const int groups = k >> 5, s8 = lane & 7;
    float2 gs[NORM ? MT : 1][4][kJ];
    if constexpr (NORM) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const size_t i = static_cast<size_t>(min(t * 32 + (lane >> 3) + 8 * q, m - 1));
#pragma unroll
                for (int j = 0; j < kJ; j++)
                    if (j * 8 < groups)  // (uniform)
                        gs[t][q][j] = *reinterpret_cast<const float2*>(
                            e.stats + (i * groups + min(s8 + 8 * j, groups - 1)) * 2);
            }
    }
    f16x acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int c = 0; c < NT; c++) acc[t][c] = f16x{};
    const f16x zero = {};

    const int b_first = b_begin + wave * BPW;
    if constexpr (NORM) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float sm = 0.0f;
#pragma unroll
                for (int j = 0; j < kJ; j++)
                    if (j * 8 < groups && s8 + 8 * j < groups) sm += gs[t][q][j].x;
                const float mu = e.rms ? 0.0f : fh::group_sum<8>(sm) / static_cast<float>(groups);
                float m2 = 0.0f;
#pragma unroll
                for (int j = 0; j < kJ; j++)
                    if (j * 8 < groups && s8 + 8 * j < groups) {
                        const float dm = gs[t][q][j].x - mu;
                        m2 += gs[t][q][j].y + 32.0f * dm * dm;
                    }
                m2 = fh::group_sum<8>(m2);
                if (s8 == 0)
                    rowf[wave][t * 32 + (lane >> 3) + 8 * q] =
                        make_float2(mu, 1.0f / sqrtf(m2 / static_cast<float>(k) + e.eps));
            }
        __builtin_amdgcn_wave_barrier();
    }
    for (int b0 = b_first; b0 < b_end; b0 += kw * BPW) {
        // Every load is unconditional (clamped to a block of this split and a
        // valid row) so the batch is in flight at once.  Rows past m compute
        // garbage that is never stored (an MFMA output row depends only on its
        // own activation row); blocks past the split are skipped whole.
        uint4 wq[NT][BPW];
        uint16_t wd[NT][BPW];
        f4 xv[MT][BPW][4];
        f4 gv[NORM ? BPW : 1], bv[NORM ? BPW : 1];
#pragma unroll
        for (int u = 0; u < BPW; u++) {
            const int b = min(b0 + u, b_end - 1);
#pragma unroll
            for (int c = 0; c < NT; c++) {
                wq[c][u] = *reinterpret_cast<const uint4*>(wrow[c] + b * 32);
                wd[c][u] = drow[c][b];
            }
            if constexpr (NORM) {
                gv[u] = *reinterpret_cast<const f4*>(e.gamma + b * 32 + (lane & 7) * 4);
                bv[u] = *reinterpret_cast<const f4*>(nm_beta + b * 32 + (lane & 7) * 4);
            }
            // Activations: eight lanes per row read one block's 128 bytes,
            // eight rows per load (a load in MFMA lane order would touch 64
            // cache lines; this one touches 16).
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int i = min(t * 32 + (lane >> 3) + 8 * q, m - 1);
                    xv[t][u][q] = *reinterpret_cast<const f4*>(x + static_cast<size_t>(i) * k + b * 32 + (lane & 7) * 4);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < BPW; u++) {
            if (b0 + u >= b_end) break;  // wave-uniform
            h8 bq0[NT], bq1[NT];
            float dw[NT];
#pragma unroll
            for (int c = 0; c < NT; c++) {
                const uint2 c0 = quants_to_f16(wq[c][u].x), c1 = quants_to_f16(wq[c][u].y);
                const uint2 c2 = quants_to_f16(wq[c][u].z), c3 = quants_to_f16(wq[c][u].w);
                bq0[c] = __builtin_bit_cast(h8, make_uint4(c0.x, c0.y, c1.x, c1.y));
                bq1[c] = __builtin_bit_cast(h8, make_uint4(c2.x, c2.y, c3.x, c3.y));
                dw[c] = fh_h2f(wd[c][u]);
            }
            // Through this wave's staging rows into MFMA order: lane (r32, half)
            // takes 16 values of row r32.  LDS operations of one wave run in
            // order, so the next block's stores follow these reads.
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    f4 val = xv[t][u][q];
                    if constexpr (NORM) {
                        const float2 f = rowf[wave][t * 32 + (lane >> 3) + 8 * q];
                        val = (val - f.x) * f.y * gv[u];
                        if (e.beta) val = val + bv[u];
                    }
                    *reinterpret_cast<f4*>(xst + (t * 32 + (lane >> 3) + 8 * q) * kSkinnyRow + (lane & 7) * 4) = val;
                }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int t = 0; t < MT; t++) {
                float v[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f4 f = *reinterpret_cast<const f4*>(xst + (t * 32 + r32) * kSkinnyRow + half * 16 + q * 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) v[4 * q + e] = f[e];
                }
                // fmaxf skips NaN; an infinite maximum takes the rare safe path.
                float mx = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) mx = fmaxf(mx, fabsf(v[q]));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                h8 ah0, ah1, al0, al1;
                int e;
                if (__builtin_expect(__ballot(!finite(mx)) != 0, 0)) {
                    float fm = 0.0f;
#pragma unroll
                    for (int q = 0; q < 16; q++)
                        if (finite(v[q])) fm = fmaxf(fm, fabsf(v[q]));
                    fm = fmaxf(fm, __shfl_xor(fm, 32, 64));
                    e = block_exponent(fm);
                    split16<true>(v, __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23), ah0, ah1, al0, al1);
                } else {
                    e = block_exponent(mx);
                    split16<false>(v, __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23), ah0, ah1, al0, al1);
                }
                // The output rows this lane holds are not the row it split:
                // publish 2^-e per row, read back the four groups of four.
                float* sl = inv_lds + (t * BPW + u) * 32;
                if (half == 0) sl[r32] = __builtin_bit_cast(float, static_cast<uint32_t>(127 - e) << 23);
                __builtin_amdgcn_wave_barrier();
                float4 iv[4];
#pragma unroll
                for (int g = 0; g < 4; g++) iv[g] = *reinterpret_cast<const float4*>(sl + g * 8 + half * 4);
#pragma unroll
                for (int c = 0; c < NT; c++) {
                    f16x p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah0, bq0[c], zero, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al0, bq0[c], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah1, bq1[c], p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al1, bq1[c], p, 0, 0, 0);
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        acc[t][c][4 * g + 0] = fmaf(dw[c], p[4 * g + 0] * iv[g].x, acc[t][c][4 * g + 0]);
                        acc[t][c][4 * g + 1] = fmaf(dw[c], p[4 * g + 1] * iv[g].y, acc[t][c][4 * g + 1]);
                        acc[t][c][4 * g + 2] = fmaf(dw[c], p[4 * g + 2] * iv[g].z, acc[t][c][4 * g + 2]);
                        acc[t][c][4 * g + 3] = fmaf(dw[c], p[4 * g + 3] * iv[g].w, acc[t][c][4 * g + 3]);
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    // Wave sums (over the staging rows, once every wave is done with them):
    // every wave stores its own, then each output is added over the waves in
    // wave order.
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int c = 0; c < NT; c++)
#pragma unroll
            for (int v = 0; v < 16; v++) sums[wave * SLOT + ((t * NT + c) * 16 + v) * 64 + lane] = acc[t][c][v];
    __syncthreads();
    // Output o = ((t * NT + c) * 16 + v) * 64 + l  ->  row, column; the loops
    // below walk each (t, c) tile's 1024 outputs, so its bias and flag are
    // picked at compile time, and o & 31 == r32 (blockDim.x is a multiple of 64).
    auto row_of = [](int o) { const int t = o / (NT * 1024), v = (o / 64) % 16, l = o % 64;
                              return t * 32 + (v / 4) * 8 + (l / 32) * 4 + (v % 4); };
    // One output (kSkinnyResOut: every lane of the wave calls together, so the
    // 32 columns of a row group can be reduced across the half-wave).
    auto finish = [&](int o, float s, bool bad, float bv, int jj, float rres = 0.0f, bool have_r = false) {
        const int i = row_of(o);
        const bool live = i < m && jj < n;
        float v = 0.0f;
        if (live) {
            if (__builtin_expect(bad, 0)) {
                if constexpr (NORM)
                    s = exact_dot_norm(x + static_cast<size_t>(i) * k, e.gamma, e.beta, e.stats + 2 * static_cast<size_t>(i) * (k >> 5),
                                       k >> 5, e.rms, e.eps, k,
                                       qs + static_cast<size_t>(jj) * k, dsc + static_cast<size_t>(jj) * kb);
                else
                    s = exact_dot(x + static_cast<size_t>(i) * k, k, qs + static_cast<size_t>(jj) * k,
                                  dsc + static_cast<size_t>(jj) * kb);
            }
            v = bias ? s + bv : s;
            if constexpr (MODE == kSkinnyResOut) {
                v = (have_r ? rres : e.r[static_cast<size_t>(i) * n + jj]) + v;
            } else {
                if (act == FH_ACT_GELU) v = gelu_unfused(v);
            }
            y[static_cast<size_t>(i) * n + jj] = v;
        }
        if constexpr (MODE == kSkinnyResOut) {
            // the row group's 32 columns sit in the 32 lanes of this half-wave
            const float mu = fh::group_total<32>(live ? v : 0.0f) * (1.0f / 32.0f);
            const float dv = live ? v - mu : 0.0f;
            const float m2 = fh::group_total<32>(dv * dv);
            if (r32 == 0 && live) {
                float* st = e.stats + (static_cast<size_t>(i) * (n >> 5) + (jj >> 5)) * 2;
                st[0] = mu;
                st[1] = m2;
            }
        }
    };
    // kSkinnyNormGlu: output o of the gate group (c = 0) and o + 1024 of the
    // up group (c = 1) are the same row and column.
    auto finish_glu = [&](int o, float sg, float su) {
        if constexpr (GLU) {
            const int i = row_of(o), col = tile * 32 + r32, nh = n >> 1;
            if (i >= m || col >= nh) return;
            if (__builtin_expect(bad_c[0] || bad_c[1], 0)) {
                const float* xi = x + static_cast<size_t>(i) * k;
                const float* sti = e.stats + 2 * static_cast<size_t>(i) * (k >> 5);
#pragma unroll
                for (int c = 0; c < 2; c++)
                    if (bad_c[c]) {
                        const int j = tile * 64 + c * 32 + r32;
                        const float v = exact_dot_norm(xi, e.gamma, e.beta, sti, k >> 5, e.rms, e.eps, k,
                                                       qs + static_cast<size_t>(j) * k,
                                                       dsc + static_cast<size_t>(j) * kb);
                        if (c == 0) sg = v; else su = v;
                    }
            }
            const float g = bias ? sg + bias_c[0] : sg, u = bias ? su + bias_c[1] : su;
            y[static_cast<size_t>(i) * nh + col] = swiglu_unfused(g, u);
        }
    };
    const size_t tiles = gridDim.x;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int base = (t * NT + c) * 1024, jj = (tile * NT + c) * 32 + r32;
            for (int o = base + static_cast<int>(threadIdx.x); o < base + 1024; o += blockDim.x) {
                float s = sums[o];
                for (int w = 1; w < kw; w++) s += sums[w * SLOT + o];
                if (GLU && splits == 1) {
                    if (c == 0) {
                        float su = sums[o + 1024];
                        for (int w = 1; w < kw; w++) su += sums[w * SLOT + o + 1024];
                        finish_glu(o, s, su);
                    }
                } else if (splits == 1)
                    finish(o, s, bad_c[c], bias_c[c], jj);
                else
                    __hip_atomic_store(part + (split * tiles + tile) * OUT + o, s, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    if (splits == 1) return;
    // Publish this split; the tile's last workgroup adds all splits in order.
    // The partials go out as device-coherent stores and every thread waits for
    // its own to complete before the arrival count is bumped, so whoever sees
    // the final count reads complete partials (device-coherent loads).  This
    // avoids a release fence, which writes back the whole L2.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(counters + tile, 1u) == static_cast<unsigned>(splits - 1);
    __syncthreads();
    if (!last) return;
    // All splits of two outputs per thread are loaded at once (clamped
    // addresses, unused values skipped in the sum), then added in split order.
    if constexpr (GLU) {
        // gate and up partials of one output per thread at a time, each added in split order
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const int base = t * NT * 1024;
            for (int o = base + static_cast<int>(threadIdx.x); o < base + 1024; o += blockDim.x) {
                float pv[2][kMaxSplits];
#pragma unroll
                for (int q = 0; q < 2; q++)
#pragma unroll
                    for (int sp = 0; sp < kMaxSplits; sp++)
                        pv[q][sp] = __hip_atomic_load(part + (min(sp, splits - 1) * tiles + tile) * OUT + o + q * 1024,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                float sg = pv[0][0], su = pv[1][0];
#pragma unroll
                for (int sp = 1; sp < kMaxSplits; sp++) {
                    sg = sp < splits ? sg + pv[0][sp] : sg;
                    su = sp < splits ? su + pv[1][sp] : su;
                }
                finish_glu(o, sg, su);
            }
        }
        if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int c = 0; c < NT; c++) {
            const int base = (t * NT + c) * 1024, jj = (tile * NT + c) * 32 + r32;
            for (int o0 = base + static_cast<int>(threadIdx.x); o0 < base + 1024; o0 += 2 * blockDim.x) {
                float pv[2][kMaxSplits], rv[2] = {0.0f, 0.0f};
#pragma unroll
                for (int q = 0; q < 2; q++) {
#pragma unroll
                    for (int sp = 0; sp < kMaxSplits; sp++) {
                        const int o = min(o0 + q * static_cast<int>(blockDim.x), base + 1023);
                        pv[q][sp] = __hip_atomic_load(part + (min(sp, splits - 1) * tiles + tile) * OUT + o,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    if constexpr (MODE == kSkinnyResOut) {
                        // the residual with the partials, one round trip for both
                        const int o = min(o0 + q * static_cast<int>(blockDim.x), base + 1023);
                        rv[q] = e.r[static_cast<size_t>(min(row_of(o), m - 1)) * n + min(jj, n - 1)];
                    }
                }
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int o = o0 + q * static_cast<int>(blockDim.x);
                    float s = pv[q][0];
#pragma unroll
                    for (int sp = 1; sp < kMaxSplits; sp++) s = sp < splits ? s + pv[q][sp] : s;
                    // (blockDim.x and 1024 are multiples of 64: the test is the same for the whole wave)
                    if (o < base + 1024) finish(o, s, bad_c[c], bias_c[c], jj, rv[q], MODE == kSkinnyResOut);
                }
            }
        }
    if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wide outputs at m <= 32 (a vocabulary head in a batched decode step), K =
// 32 * KB: one workgroup per CU holding a contiguous run of 32-column tiles,
// one tile per wave over all of K.  The workgroup splits the activations once
// into LDS, [KB][32 rows][kSkinnyRow dwords] (16 of packed f16 h, 16 of l, 4
// pad: the 16-byte fragment reads are conflict-free) with 2^-e per (row,
// block) beside them, so every tile of the workgroup shares one split (the
// skinny kernel redoes it per tile).  Loads, in issue order: every wave's
// activations (a bare barrier keeps them ahead of all weight loads: the split
// waits on them), the row's KB scales, bias and flag, the first kWideLook
// 16-byte quant chunks; then each block issues the chunk kWideLook ahead, so
// block b's MFMAs wait for chunk b only (loads complete in issue order).
// Waves past the workgroup's last tile load that tile (never used) and leave
// after the split.
constexpr int kWideWaves = 8;
// Quant chunks in flight per wave ahead of the MFMAs (4 and 8 time alike; 12
// and 24 slower: the HBM queues fill with the waves' 32-byte row pieces).
constexpr int kWideLook = 8;

template <int KB>
__global__ void __launch_bounds__(64 * kWideWaves)
    k_gemm_wide(const float* __restrict__ x, const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc,
                const int8_t* __restrict__ rexp, const float* __restrict__ bias, float* __restrict__ y, int m, int n,
                int per_wg, int extra) {
    constexpr int k = KB * 32;
    constexpr int kTasks = KB * 32 * 8 / (64 * kWideWaves);  // 4-value groups per thread
    static_assert(KB % 4 == 0 && (KB * 256) % (64 * kWideWaves) == 0, "KB");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds);
    float* ivs = lds + KB * 32 * kSkinnyRow;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    // tiles [t0, t1): per_wg each, one more for the first `extra` workgroups
    const int g = static_cast<int>(blockIdx.x);
    const int t0 = g * per_wg + min(g, extra), t1 = t0 + per_wg + (g < extra ? 1 : 0);
    const int tile = min(t0 + wave, t1 - 1);
    const bool active = t0 + wave < t1;  // wave-uniform
    const int col = tile * 32 + r32, j = min(col, n - 1);

    // Activation groups: task = (block b, row r, 4-value group q), eight
    // consecutive lanes per (b, r) so a load covers 128 contiguous bytes.
    f4 xv[kTasks];
#pragma unroll
    for (int u = 0; u < kTasks; u++) {
        const int task = static_cast<int>(threadIdx.x) + u * 64 * kWideWaves;
        const int b = task >> 8, r = min((task >> 3) & 31, m - 1), q = task & 7;
        xv[u] = *reinterpret_cast<const f4*>(x + static_cast<size_t>(r) * k + b * 32 + q * 4);
    }
    // Every wave's activation loads go out ahead of any weight load (a bare
    // barrier: it does not wait for the loads).
    __builtin_amdgcn_s_barrier();
    // (the scales, bias and flag before the quants: block b's MFMAs then wait
    // for quant chunk b only, loads completing in issue order)
    uint2 sc[KB / 4];
    const uint2* srow = reinterpret_cast<const uint2*>(dsc + static_cast<size_t>(j) * KB);
#pragma unroll
    for (int s = 0; s < KB / 4; s++) sc[s] = srow[s];
    const float bv = bias ? bias[j] : 0.0f;
    const bool bad = rexp[j] == kFhBadRowExp;
    uint4 wq[KB];
    const int8_t* wrow = qs + static_cast<size_t>(j) * k + half * 16;
#pragma unroll
    for (int b = 0; b < kWideLook; b++) wq[b] = *reinterpret_cast<const uint4*>(wrow + b * 32);

    // The split: 2^e from the block's largest finite |x| (eight lanes), then
    // h = f16(x 2^e), l = f16(x 2^e - h); rows past m are zeros.
    auto split_task = [&](int u) __attribute__((always_inline)) {
        const int task = static_cast<int>(threadIdx.x) + u * 64 * kWideWaves;
        const int b = task >> 8, r = (task >> 3) & 31, q = task & 7;
        const f4 z = {};
        const f4 v = r < m ? xv[u] : z;
        float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        mx = fmaxf(mx, fh::dpp<0xB1>(mx));
        mx = fmaxf(mx, fh::dpp<0x4E>(mx));
        mx = fmaxf(mx, fh::dpp<0x141>(mx));
        const float vv[4] = {v.x, v.y, v.z, v.w};
        uint2 h, l;
        int e;
        if (__builtin_expect(__ballot(!finite(mx)) != 0, 0)) {
            float fm = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (finite(vv[i])) fm = fmaxf(fm, fabsf(vv[i]));
            fm = fmaxf(fm, fh::dpp<0xB1>(fm));
            fm = fmaxf(fm, fh::dpp<0x4E>(fm));
            fm = fmaxf(fm, fh::dpp<0x141>(fm));
            e = block_exponent(fm);
            split4<true>(vv, __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23), h, l);
        } else {
            e = block_exponent(mx);
            split4<false>(vv, __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23), h, l);
        }
        uint32_t* dst = xs + (b * 32 + r) * kSkinnyRow + 2 * q;
        *reinterpret_cast<uint2*>(dst) = h;
        *reinterpret_cast<uint2*>(dst + 16) = l;
        if (q == 0) ivs[b * 32 + r] = __builtin_bit_cast(float, static_cast<uint32_t>(127 - e) << 23);
    };

    f16x acc = {};
    const f16x zero = {};
    auto block = [&](int b) __attribute__((always_inline)) {
        if (b + kWideLook < KB) wq[b + kWideLook] = *reinterpret_cast<const uint4*>(wrow + (b + kWideLook) * 32);
        // lane (r32, half) takes x[r32][b*32 + half*16 .. +16] as h and l
        const uint32_t* xr = xs + (b * 32 + r32) * kSkinnyRow + half * 8;
        const h8 ah0 = *reinterpret_cast<const h8*>(xr), ah1 = *reinterpret_cast<const h8*>(xr + 4);
        const h8 al0 = *reinterpret_cast<const h8*>(xr + 16), al1 = *reinterpret_cast<const h8*>(xr + 20);
        float4 iv[4];
#pragma unroll
        for (int g = 0; g < 4; g++) iv[g] = *reinterpret_cast<const float4*>(ivs + b * 32 + g * 8 + half * 4);
        const uint2 c0 = quants_to_f16(wq[b].x), c1 = quants_to_f16(wq[b].y);
        const uint2 c2 = quants_to_f16(wq[b].z), c3 = quants_to_f16(wq[b].w);
        const h8 bq0 = __builtin_bit_cast(h8, make_uint4(c0.x, c0.y, c1.x, c1.y));
        const h8 bq1 = __builtin_bit_cast(h8, make_uint4(c2.x, c2.y, c3.x, c3.y));
        const uint32_t sw = (b & 2) ? sc[b >> 2].y : sc[b >> 2].x;
        const float dw = fh_h2f(static_cast<uint16_t>((b & 1) ? sw >> 16 : sw & 0xFFFFu));
        f16x p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah0, bq0, zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al0, bq0, p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah1, bq1, p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al1, bq1, p, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            acc[4 * g + 0] = fmaf(dw, p[4 * g + 0] * iv[g].x, acc[4 * g + 0]);
            acc[4 * g + 1] = fmaf(dw, p[4 * g + 1] * iv[g].y, acc[4 * g + 1]);
            acc[4 * g + 2] = fmaf(dw, p[4 * g + 2] * iv[g].z, acc[4 * g + 2]);
            acc[4 * g + 3] = fmaf(dw, p[4 * g + 3] * iv[g].w, acc[4 * g + 3]);
        }
        // Each block's sums are formed here, in order: without this the
        // compiler runs every block's MFMAs first and spills their products.
        asm volatile("" : "+v"(acc));
    };

    // Every split first (one barrier), then the blocks in order.  (Splitting
    // and computing chunk by chunk, a barrier per chunk, ran slower.)
#pragma unroll
    for (int u = 0; u < kTasks; u++) split_task(u);
    __syncthreads();
    if (!active) return;
#pragma unroll
    for (int b = 0; b < KB; b++) block(b);
    if (col >= n) return;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = (v >> 2) * 8 + half * 4 + (v & 3);
        if (i >= m) continue;
        float s = acc[v];
        if (__builtin_expect(bad, 0))
            s = exact_dot(x + static_cast<size_t>(i) * k, k, qs + static_cast<size_t>(col) * k,
                          dsc + static_cast<size_t>(col) * KB);
        y[static_cast<size_t>(i) * n + col] = bias ? s + bv : s;
    }
}

namespace {

// The block-scaled GEMM (k_gemm_bscale): row scales first, then the GEMM.
int launch_bscale(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y, int act) {
    const size_t m_pad = (m + 255) / 256 * 256;
    const size_t ibytes = fh_align256(m_pad * 4), fbytes = fh_align256(m_pad);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, ibytes + fbytes, &ws);
    if (rc) return rc;
    float* xinv = static_cast<float*>(ws);
    uint8_t* xbad = reinterpret_cast<uint8_t*>(static_cast<char*>(ws) + ibytes);
    hipLaunchKernelGGL(k_row_scales, dim3(static_cast<unsigned>((m_pad + 3) / 4)), dim3(256), 0, ctx->stream, x,
                       static_cast<int>(m), static_cast<int>(m_pad), static_cast<int>(w->k), xinv, xbad);
    FH_HIP(ctx, hipGetLastError());
    const size_t tiles_n = (w->n + 255) / 256, tiles = tiles_n * (m_pad / 256);
    if (tiles > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: output above 2^31 tiles");
    hipLaunchKernelGGL(k_gemm_bscale, dim3(static_cast<unsigned>(tiles)), dim3(512), 0, ctx->stream, xinv, xbad, x,
                       w->qs, w->d, w->rexp, bias, y, static_cast<int>(m), static_cast<int>(w->n),
                       static_cast<int>(w->k), static_cast<int>(tiles_n), act);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

template <int BM, int BN, int WM, int WN, int KW>
int launch_gemm(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y) {
    const size_t m_pad = (m + BM - 1) / BM * BM;
    const size_t pbytes = fh_align256(m_pad * w->k * 4), ibytes = fh_align256(m_pad * 4), fbytes = fh_align256(m_pad);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, pbytes + ibytes + fbytes, &ws);
    if (rc) return rc;
    uint4* panel = static_cast<uint4*>(ws);
    float* xinv = reinterpret_cast<float*>(static_cast<char*>(ws) + pbytes);
    uint8_t* xbad = reinterpret_cast<uint8_t*>(static_cast<char*>(ws) + pbytes + ibytes);
    hipLaunchKernelGGL(k_split_rows, dim3(static_cast<unsigned>((m_pad + 3) / 4)), dim3(256), 0, ctx->stream, x,
                       static_cast<int>(m), static_cast<int>(m_pad), static_cast<int>(w->k), BM, panel, xinv, xbad);
    FH_HIP(ctx, hipGetLastError());
    const size_t tiles_n = (w->n + BN - 1) / BN, tiles = tiles_n * (m_pad / BM);
    if (tiles > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: output above 2^31 tiles");
    hipLaunchKernelGGL((k_gemm_mfma<BM, BN, WM, WN, KW>), dim3(static_cast<unsigned>(tiles)),
                           dim3(64 * WM * WN * KW), 0, ctx->stream, panel, xinv, x, w->qs, w->d, w->rexp, bias, y,
                           static_cast<int>(m), static_cast<int>(w->n), static_cast<int>(w->k),
                           static_cast<int>(tiles_n));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

// Splits of K only while the column tiles alone leave half the CUs idle, and
// then as few as let one batch of BPW blocks per wave cover a split (each split
// costs a round of partial stores and reloads).  Waves: at most 16 / (MT * NT)
// (their sums fit 64 KiB of LDS, two workgroups per CU) and 8 (256 VGPRs per lane).  Column tiles per
// wave (NT): up to 4 while that still leaves >= 256 workgroups, so wide
// outputs split each activation block once per 128 columns.
__global__ void k_zero_counters(unsigned* __restrict__ c, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) c[i] = 0u;
}

template <int MT, int NT, int BPW>
int launch_skinny_t(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                    const fh_scratch* scratch, int act, const fh_edge* edge = nullptr, int mode = kSkinnyPlain) {
    const size_t kb = w->k / 32, tiles = (w->n + 32 * NT - 1) / (32 * NT);
    // Waves per workgroup: eight, except that a tile of more than two 32 x 32
    // output groups keeps 16 KB of wave sums per wave in LDS, so where the
    // tiles outnumber the CUs it takes four and two workgroups share a CU.
    // (Qwen2-0.5B gate|up at m = 64, 152 tiles: seven blocks per wave with
    // four waves, three or four with eight.)
    const size_t kMaxWaves =
        MT * NT > 2 && tiles > static_cast<size_t>(ctx->num_cus) ? (16 / (MT * NT) < 8 ? 16 / (MT * NT) : 8) : 8;
    size_t splits = 1;
    if (tiles < static_cast<size_t>(ctx->num_cus) / 2) splits = (kb + kMaxWaves * BPW - 1) / (kMaxWaves * BPW);
    if (splits > static_cast<size_t>(kMaxSplits)) splits = kMaxSplits;
    const size_t bps = (kb + splits - 1) / splits;
    splits = (kb + bps - 1) / bps;  // no empty split
    size_t kw = (bps + BPW - 1) / BPW;
    if (kw > kMaxWaves) kw = kMaxWaves;
    constexpr size_t kSlot = MT * NT * 1024 > MT * 32 * kSkinnyRow ? MT * NT * 1024 : MT * 32 * kSkinnyRow;
    const size_t lds = kw * (kSlot + MT * BPW * 32) * sizeof(float);
    float* part = nullptr;
    unsigned* counters = nullptr;
    const fh_edge ed = edge ? *edge : fh_edge{};
    if (splits > 1) {
        const size_t part_bytes = splits * tiles * MT * NT * 1024 * sizeof(float);
        if (scratch) {
            // The caller's fixed scratch: partials, then the arrival counters,
            // which are cleared here (a kernel, not a memset, so the call can
            // be captured into a graph).
            const size_t cnt_at = fh_align256(part_bytes);
            if (cnt_at + tiles * sizeof(unsigned) > scratch->bytes)
                return fh_fail(ctx, FH_ERR_LIMIT,
                               "fh_q8_0_linear_noalloc: this shape needs " +
                                   std::to_string(cnt_at + tiles * sizeof(unsigned)) +
                                   " bytes of scratch, above the fixed " + std::to_string(scratch->bytes));
            part = static_cast<float*>(scratch->ptr);
            counters = reinterpret_cast<unsigned*>(static_cast<char*>(scratch->ptr) + cnt_at);
            hipLaunchKernelGGL(k_zero_counters, dim3(static_cast<unsigned>((tiles + 255) / 256)), dim3(256), 0,
                               ctx->stream, counters, static_cast<int>(tiles));
            FH_HIP(ctx, hipGetLastError());
        } else {
            void* ws = nullptr;
            int rc = fh_workspace(ctx, part_bytes, &ws);
            if (rc) return rc;
            part = static_cast<float*>(ws);
            void* cnt = nullptr;
            rc = fh_counter_area(ctx, tiles * sizeof(unsigned), &cnt);
            if (rc) return rc;
            counters = static_cast<unsigned*>(cnt);
        }
    }
    if (tiles > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: too many output columns");
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits)), block(static_cast<unsigned>(64 * kw));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, x, w->qs, w->d, w->rexp, bias, y, static_cast<int>(m),
                           static_cast<int>(w->n), static_cast<int>(w->k), static_cast<int>(bps), part, counters, act,
                           ed);
    };
    // (the fused edges are built for the tiles of at most two 32-column
    // groups per wave, whose registers hold them without spilling)
    constexpr bool kEdges = NT <= 2 && !(MT == 2 && NT == 2 && BPW == 2);
    if (mode != kSkinnyPlain && !kEdges)
        return fh_fail(ctx, FH_ERR_LIMIT, "skinny GEMM: no fused norm or residual for this tile");
    if constexpr (kEdges && NT == 2) {
        if (mode == kSkinnyNormGlu) {
            go(k_gemm_skinny<MT, NT, BPW, kSkinnyNormGlu>);
            FH_HIP(ctx, hipGetLastError());
            return FH_OK;
        }
    }
    if (mode == kSkinnyNormGlu) return fh_fail(ctx, FH_ERR_LIMIT, "skinny GEMM: no fused SwiGLU for this tile");
    if constexpr (kEdges) {
        if (mode == kSkinnyNormIn) go(k_gemm_skinny<MT, NT, BPW, kSkinnyNormIn>);
        else if (mode == kSkinnyResOut) go(k_gemm_skinny<MT, NT, BPW, kSkinnyResOut>);
        else go(k_gemm_skinny<MT, NT, BPW, kSkinnyPlain>);
    } else {
        go(k_gemm_skinny<MT, NT, BPW, kSkinnyPlain>);
    }
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

// One workgroup per CU (more only past eight tiles per CU), tiles dealt in
// contiguous runs that differ by at most one.
template <int KB>
int launch_wide(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y) {
    const size_t tiles = (w->n + 31) / 32;
    size_t grid = static_cast<size_t>(ctx->num_cus);
    if (grid * kWideWaves < tiles) grid = (tiles + kWideWaves - 1) / kWideWaves;
    if (grid > tiles) grid = tiles;
    if (tiles > 0x7FFFFFFFu / 32) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: too many output columns");
    const size_t lds = KB * (32 * kSkinnyRow + 32) * sizeof(float);
    hipLaunchKernelGGL(k_gemm_wide<KB>, dim3(static_cast<unsigned>(grid)), dim3(64 * kWideWaves), lds, ctx->stream, x,
                       w->qs, w->d, w->rexp, bias, y, static_cast<int>(m), static_cast<int>(w->n),
                       static_cast<int>(tiles / grid), static_cast<int>(tiles % grid));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

// Outputs at least this many 32-column tiles wide take k_gemm_wide, 32 rows per launch.
constexpr size_t kWideMinTiles = 1024;

// Tile rules from timings at m = 32 and 64 over the GPT-2 and Qwen2-0.5B
// shapes: two column tiles per wave pay off from about 256 tiles of 32
// columns (a 9728-wide output: 14.2 -> 11.8 us at m = 32), four only at m <=
// 32 (four at m = 64 ran the 151936-wide head 2.8x slower); at m = 64 two
// blocks per wave batch beat three (small layers 11.4 -> 10.4 us); at m <=
// 32 and 64 outputs narrower than 2048 take one block per wave batch (more K
// splits, so more workgroups: 896 x 896 7.9 -> 6.9 us at m = 32, 10.4 -> 9.2
// us at m = 64; a 3072-wide one slows down).
int launch_skinny(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                  const fh_scratch* scratch = nullptr, int act = FH_ACT_NONE, const fh_edge* edge = nullptr,
                  int mode = kSkinnyPlain) {
    const size_t t32 = (w->n + 31) / 32;
    // the fused SwiGLU needs each workgroup's two column groups to be a gate / up pair
    if (mode == kSkinnyNormGlu)
        return m <= 32 ? launch_skinny_t<1, 2, 3>(ctx, w, x, m, bias, y, scratch, act, edge, mode)
                       : launch_skinny_t<2, 2, 1>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
    if (mode == kSkinnyPlain && t32 >= kWideMinTiles && (w->k == 768 || w->k == 896 || w->k == 1024)) {
        // 32 rows per launch: at m = 64 two launches, each streaming the
        // weight once, beat the skinny kernel's single pass (151936 x 896:
        // 131 -> 114 us), which re-splits the 64-row block per 64 columns
        for (size_t r0 = 0; r0 < m; r0 += 32) {
            const size_t mr = m - r0 < 32 ? m - r0 : 32;
            const float* xr = x + r0 * w->k;
            float* yr = y + r0 * w->n;
            const int rc = w->k == 768   ? launch_wide<24>(ctx, w, xr, mr, bias, yr)
                           : w->k == 896 ? launch_wide<28>(ctx, w, xr, mr, bias, yr)
                                         : launch_wide<32>(ctx, w, xr, mr, bias, yr);
            if (rc) return rc;
        }
        return act == FH_ACT_GELU ? fh_launch_gelu(ctx, y, m * w->n) : FH_OK;
    }
    // (the fused edges never take the 4-group tiles: at t32 >= 1024 they take 2)
    if (m <= 32) {
        if (t32 >= 4 * 256 && mode == kSkinnyPlain) return launch_skinny_t<1, 4, 2>(ctx, w, x, m, bias, y, scratch, act);
        if (t32 >= 256) return launch_skinny_t<1, 2, 3>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
        if (t32 >= 64) return launch_skinny_t<1, 1, 3>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
        return launch_skinny_t<1, 1, 1>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
    }
    if (t32 >= 4 * 256 && mode == kSkinnyPlain) return launch_skinny_t<2, 2, 2>(ctx, w, x, m, bias, y, scratch, act);
    if (t32 >= 256) return launch_skinny_t<2, 2, 1>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
    if (t32 >= 64) return launch_skinny_t<2, 1, 2>(ctx, w, x, m, bias, y, scratch, act, edge, mode);
    return launch_skinny_t<2, 1, 1>(ctx, w, x, m, bias, y, scratch, act, edge, mode);  // 896 x 896: 10.4 -> 9.2 us
}

}  // namespace

template <bool V4>
__global__ void fh_k_encode_panel(const float* __restrict__ x, int m, int m_pad, int kb, uint4* __restrict__ qp,
                                  float* __restrict__ dp);

// W8A8 through the int8 matrix cores: the activations are encoded into the
// lane-order panel, then one wave per (32 TM) x 64 output tile.
int fh_launch_gemm_w8a8(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                        bool fast) {
    // (a prompt's m takes the LDS-staged kernel: its panel covers whole 256-row tiles)
    const bool staged = m >= kW8LdsMinRows;
    const int tm_rows = staged ? kW8Rows : m >= 64 ? 64 : 32;
    const size_t kb = w->k / 32, m_pad = (m + tm_rows - 1) / tm_rows * tm_rows;
    const size_t qbytes = fh_align256(m_pad * w->k), dbytes = fh_align256(m_pad * kb * 4);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, qbytes + dbytes, &ws);
    if (rc) return rc;
    uint4* qp = static_cast<uint4*>(ws);
    float* dp = reinterpret_cast<float*>(static_cast<char*>(ws) + qbytes);
    const size_t frags = m_pad / 32 * kb;  // one wave each
    const dim3 egrid(static_cast<unsigned>((frags + 3) / 4));
    if (reinterpret_cast<uintptr_t>(x) & 15)
        hipLaunchKernelGGL(fh_k_encode_panel<false>, egrid, dim3(256), 0, ctx->stream, x, static_cast<int>(m),
                           static_cast<int>(m_pad), static_cast<int>(kb), qp, dp);
    else
        hipLaunchKernelGGL(fh_k_encode_panel<true>, egrid, dim3(256), 0, ctx->stream, x, static_cast<int>(m),
                           static_cast<int>(m_pad), static_cast<int>(kb), qp, dp);
    FH_HIP(ctx, hipGetLastError());
    if (staged) {
        const size_t tn = (w->n + kW8Cols - 1) / kW8Cols, tl = tn * (m_pad / kW8Rows);
        if (tl > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: output above 2^31 tiles");
        if (fast)
            hipLaunchKernelGGL(k_gemm_w8a8_lds<true>, dim3(static_cast<unsigned>(tl)), dim3(kW8Threads), 0,
                               ctx->stream, qp, dp, w->qs, w->d, bias, y, static_cast<int>(m),
                               static_cast<int>(w->n), static_cast<int>(w->k), static_cast<int>(tn));
        else
            hipLaunchKernelGGL(k_gemm_w8a8_lds<false>, dim3(static_cast<unsigned>(tl)), dim3(kW8Threads), 0,
                               ctx->stream, qp, dp, w->qs, w->d, bias, y, static_cast<int>(m),
                               static_cast<int>(w->n), static_cast<int>(w->k), static_cast<int>(tn));
        FH_HIP(ctx, hipGetLastError());
        return FH_OK;
    }
    const size_t tiles_n = (w->n + 63) / 64, tiles = tiles_n * (m_pad / tm_rows);
    if (tiles > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_q8_0_linear: output above 2^31 tiles");
    const dim3 grid(static_cast<unsigned>((tiles + 3) / 4)), block(256);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, ctx->stream, qp, dp, w->qs, w->d, bias, y, static_cast<int>(m),
                           static_cast<int>(w->n), static_cast<int>(w->k), static_cast<int>(tiles_n),
                           static_cast<int>(tiles));
    };
    if (tm_rows == 64) fast ? go(k_gemm_w8a8<2, true>) : go(k_gemm_w8a8<2, false>);
    else fast ? go(k_gemm_w8a8<1, true>) : go(k_gemm_w8a8<1, false>);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_skinny_norm_in(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_edge& e,
                             const float* bias, float* y, int act) {
    if (m < 3 || m > 64 || w->kind != FH_WEIGHT_Q8_0 || w->k > 1024) return -1;
    if (act == FH_ACT_SWIGLU32) return launch_skinny(ctx, w, x, m, bias, y, nullptr, FH_ACT_NONE, &e, kSkinnyNormGlu);
    return launch_skinny(ctx, w, x, m, bias, y, nullptr, act, &e, kSkinnyNormIn);
}

int fh_launch_skinny_res_out(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const fh_edge& e,
                             const float* bias, float* y) {
    if (m < 3 || m > 64 || w->kind != FH_WEIGHT_Q8_0) return -1;
    return launch_skinny(ctx, w, x, m, bias, y, nullptr, FH_ACT_NONE, &e, kSkinnyResOut);
}

int fh_launch_skinny_scratch(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                             const fh_scratch& scratch) {
    return launch_skinny(ctx, w, x, m, bias, y, &scratch);
}

// Tile choice: m <= 64 takes the skinny kernel; otherwise the 256 x 256
// block-scaled tile (eight waves) once it still yields a tile per CU, the 128 x 128 tile at two
// tiles per CU, else 64 x 64, else 32 x 32 outputs with four waves splitting K.
int fh_launch_gemm_w8a32(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, const float* bias, float* y,
                         int act) {
    const size_t cus = static_cast<size_t>(ctx->num_cus);
    if (m <= 64) return launch_skinny(ctx, w, x, m, bias, y, nullptr, act);  // GELU in its epilogue
    int rc;
    if (((m + 255) / 256) * ((w->n + 255) / 256) >= cus)
        return launch_bscale(ctx, w, x, m, bias, y, act);  // GELU in its epilogue
    else if (((m + 127) / 128) * ((w->n + 127) / 128) >= 2 * cus) rc = launch_gemm<128, 128, 2, 2, 1>(ctx, w, x, m, bias, y);
    else if (((m + 63) / 64) * ((w->n + 63) / 64) >= 2 * cus) rc = launch_gemm<64, 64, 2, 2, 1>(ctx, w, x, m, bias, y);
    else rc = launch_gemm<32, 32, 1, 1, 4>(ctx, w, x, m, bias, y);
    return rc == FH_OK && act == FH_ACT_GELU ? fh_launch_gelu(ctx, y, m * w->n) : rc;
}
