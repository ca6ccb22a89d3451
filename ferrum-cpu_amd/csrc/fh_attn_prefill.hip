// fh_attn_prefill.hip — the attention of a prompt block on the fp32 matrix cores.
//
// What it computes: the attention of TransformerBlock::forward_with_cache
// (layer/transformer.rs:242-279) for every row of a prompt block at once.
// CachedTransformer's prime (slm/cached.rs:129-136) feeds a prompt position by
// position; here row r of sequence s is position pos0 + r and attends over
// cache positions 0 .. pos0 + r of its own sequence, with the scores
// (q . k) * 1/sqrt(hd), their softmax and the weighted sum of v rows.  The
// block's k / v rows go into the caches first (k_kv_store_seqs), so every key
// and value comes from the cache.
//
// How (head width 64): one workgroup per (128 query rows, head, sequence).
// Each of its four waves owns 32 query rows and walks 32-key tiles of the
// sequence's cache up to its last row's position; the tiles are staged in LDS
// once for the four waves (double-buffered, the next tile's loads in flight
// while the current one is used).  Per tile, flash style:
//   S^T = K Q^T   32 v_mfma_f32_32x32x2_f32 (32 keys x 32 queries, K = 64
//                 dims, two dims per step: half h of the wave supplies dim
//                 s + 32 h, so each lane reads one contiguous half row);
//   softmax       lane j of each half holds query j's scores for 16 keys: the
//                 masked max, exp(s - max) and the row sums per query, and the
//                 running max / sum with exact rescaling between tiles;
//   O += P V      32 v_mfma_f32_32x32x2_f32 (32 queries x 2 x 32 dims): the
//                 keys of step s are the ones lane half h holds in accumulator
//                 s, so P goes into the matrix cores straight from the S^T
//                 accumulators, and the outputs come out one query row per
//                 accumulator (coalesced stores).
// All products and sums are f32 (the matrix cores' fp32 path), so the result
// is the reference's within the 1e-5 rule: the same dot products scaled after
// the sum, exp(s - max), a blockwise order of the sums.  A tile holding a
// non-finite v value is finished on the vector units with only the attended
// keys (0 * inf would otherwise turn a masked key's v into NaN); non-finite k
// values of masked keys never reach a score (the mask selects -inf).
#include "fh_internal.hpp"

#pragma clang fp contract(off)

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPT = 256;       // threads: four waves of 32 query rows
constexpr int kQRows = 128;    // query rows per workgroup
constexpr int kKeys = 32;      // keys per tile
constexpr int kHd = 64;        // head width
constexpr int kKPitch = kHd + 4;  // K tile row pitch (floats): 16-byte reads of 8 rows hit distinct banks

struct PrefillArgs {
    const float* qkv;   // row s * rows + r; head h's q at column h * 64
    int ld;             // qkv row stride (floats)
    const float* kc;    // sequence s's caches at kc / vc + s * seq_stride, rows of kv_dim floats
    const float* vc;
    size_t seq_stride;
    int kv_dim;
    int rows, pos0, groups;
    float scale;
    float* out;         // row s * rows + r; head h at column h * 64
    int out_ld;
};

__device__ __forceinline__ bool finite4(float4 v) {
    return __builtin_isfinite(v.x) && __builtin_isfinite(v.y) && __builtin_isfinite(v.z) && __builtin_isfinite(v.w);
}

// Query row of accumulator v in a lane of half `half` (the 32 x 32 MFMA
// output layout: rows 8 (v / 4) + 4 half + v % 4).
__device__ __forceinline__ int acc_row(int v, int half) { return (v >> 2) * 8 + half * 4 + (v & 3); }

__global__ void __launch_bounds__(kPT, 2) k_attn_prefill_mfma(PrefillArgs a) {
    __shared__ __align__(16) float ks[2][kKeys * kKPitch];
    __shared__ __align__(16) float vs[2][kKeys * kHd];     // row kk: position 2 c + t holds v[kk][c + 32 t]
    __shared__ __align__(16) float cx[4][32];               // per wave: one factor per query row
    __shared__ __align__(16) float pt[4][kKeys * 33];       // per wave: P of a tile with non-finite v ([key][query])

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, col = lane & 31;
    const int g = a.groups - 1 - static_cast<int>(blockIdx.x);  // the longest rows first
    const int h = blockIdx.y, s = blockIdx.z;
    const int r0 = g * kQRows + wave * 32;
    const int last_row = min(a.rows - 1, g * kQRows + kQRows - 1);
    const int kmax = a.pos0 + last_row;                         // the last cache row this workgroup reads
    const int ntiles = kmax / kKeys + 1;
    const int my_tiles = r0 < a.rows ? (a.pos0 + min(a.rows - 1, r0 + 31)) / kKeys + 1 : 0;
    const size_t sbase = static_cast<size_t>(s) * a.seq_stride + static_cast<size_t>(h) * kHd;
    const float* kc = a.kc + sbase;
    const float* vc = a.vc + sbase;

    // This lane's half of its query row (rows past the block repeat the last one).
    float q[32];
    {
        const int row = min(r0 + col, a.rows - 1);
        const float4* qp = reinterpret_cast<const float4*>(a.qkv + (static_cast<size_t>(s) * a.rows + row) * a.ld +
                                                           h * kHd + half * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = qp[i];
            q[4 * i] = v.x;
            q[4 * i + 1] = v.y;
            q[4 * i + 2] = v.z;
            q[4 * i + 3] = v.w;
        }
    }
    const int qpos = a.pos0 + r0 + col;  // the position of this lane's query row

    // Tile staging: 512 float4 of k rows and 512 of v rows; thread t takes
    // float4s t and t + 256 of each (row idx / 16, dims 4 (idx % 16) ...).
    float4 pk[2], pv[2];
    auto fetch = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * kPT, row = idx >> 4, c4 = idx & 15;
            const size_t key = static_cast<size_t>(min(t * kKeys + row, kmax));
            pk[i] = *reinterpret_cast<const float4*>(kc + key * a.kv_dim + c4 * 4);
            pv[i] = *reinterpret_cast<const float4*>(vc + key * a.kv_dim + c4 * 4);
        }
    };
    auto stash = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * kPT, row = idx >> 4, c0 = (idx & 15) * 4;
            *reinterpret_cast<float4*>(&ks[buf][row * kKPitch + c0]) = pk[i];
            float* vr = &vs[buf][row * kHd + 2 * (c0 & 31) + (c0 >> 5)];
            vr[0] = pv[i].x;
            vr[2] = pv[i].y;
            vr[4] = pv[i].z;
            vr[6] = pv[i].w;
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x16 o0, o1;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        o0[v] = 0.0f;
        o1[v] = 0.0f;
    }
    fetch(0);
    stash(0);
    bool vbad = __syncthreads_or(!finite4(pv[0]) || !finite4(pv[1]));
    for (int t = 0; t < ntiles; t++) {
        const int buf = t & 1, k0 = t * kKeys;
        if (t + 1 < ntiles) fetch(t + 1);
        if (t < my_tiles) {
            // ---- S^T = K Q^T: accumulator v of lane (half, col) is key acc_row(v, half), query col
            f32x16 sacc;
#pragma unroll
            for (int v = 0; v < 16; v++) sacc[v] = 0.0f;
            const float* krow = &ks[buf][col * kKPitch + half * 32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 kv = *reinterpret_cast<const float4*>(krow + 4 * i);
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, q[4 * i], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, q[4 * i + 1], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, q[4 * i + 2], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, q[4 * i + 3], sacc, 0, 0, 0);
            }
            // ---- scores (scaled after the sum, as the reference), masked past the query's position
            float sv[16];
            float mt = -INFINITY;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                sv[v] = k0 + acc_row(v, half) <= qpos ? sacc[v] * a.scale : -INFINITY;
                mt = fmaxf(mt, sv[v]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float m_new = fmaxf(m_run, mt);
            const float corr = expf(m_run - m_new);  // 0 on the first tile (m_run = -inf)
            float ps = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                sv[v] = expf(sv[v] - m_new);
                ps += sv[v];
            }
            ps += __shfl_xor(ps, 32, 64);
            l_run = l_run * corr + ps;
            m_run = m_new;
            // ---- rescale the output rows (query acc_row(v, half)) by their query's factor
            if (half == 0) cx[wave][col] = corr;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                const float4 c = *reinterpret_cast<const float4*>(&cx[wave][a4 * 8 + half * 4]);
                o0[4 * a4] *= c.x;
                o0[4 * a4 + 1] *= c.y;
                o0[4 * a4 + 2] *= c.z;
                o0[4 * a4 + 3] *= c.w;
                o1[4 * a4] *= c.x;
                o1[4 * a4 + 1] *= c.y;
                o1[4 * a4 + 2] *= c.z;
                o1[4 * a4 + 3] *= c.w;
            }
            __builtin_amdgcn_wave_barrier();
            const float* vt = vs[buf];
            if (!vbad) {
                // ---- O += P V: step st takes key acc_row(st, half) in half `half`
#pragma unroll
                for (int st = 0; st < 16; st++) {
                    const float2 vv = *reinterpret_cast<const float2*>(vt + acc_row(st, half) * kHd + 2 * col);
                    o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(sv[st], vv.x, o0, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(sv[st], vv.y, o1, 0, 0, 0);
                }
            } else {
                // ---- a non-finite v in this tile: only the attended keys, on the vector units
                float* pw = pt[wave];
#pragma unroll
                for (int v = 0; v < 16; v++) pw[acc_row(v, half) * 33 + col] = sv[v];
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int qr = acc_row(v, half), qp = a.pos0 + r0 + qr;
                    float s0 = o0[v], s1 = o1[v];
                    for (int kk = 0; kk < kKeys && k0 + kk <= qp; kk++) {
                        const float p = pw[kk * 33 + qr];
                        s0 += p * vt[kk * kHd + 2 * col];
                        s1 += p * vt[kk * kHd + 2 * col + 1];
                    }
                    o0[v] = s0;
                    o1[v] = s1;
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        bool vbad_next = false;
        if (t + 1 < ntiles) {
            stash(buf ^ 1);
            vbad_next = !finite4(pv[0]) || !finite4(pv[1]);
        }
        vbad = __syncthreads_or(vbad_next);
    }

    // ---- out[row] = O / (sum of the row's exponentials)
    if (r0 >= a.rows) return;
    if (half == 0) cx[wave][col] = l_run;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int qr = acc_row(v, half), row = r0 + qr;
        const float l = cx[wave][qr];
        if (row < a.rows) {
            float* op = a.out + (static_cast<size_t>(s) * a.rows + row) * a.out_ld + h * kHd;
            op[col] = o0[v] / l;
            op[32 + col] = o1[v] / l;
        }
    }
}

// Rows r of each sequence's block: their k and v slices into cache rows
// pos0 + r of that sequence (grid: (column chunks, rows, sequences)).
__global__ void __launch_bounds__(kPT) k_kv_store_seqs(const float* __restrict__ qkv, int ld, int k_off, int v_off,
                                                      int kv_dim, int rows, int pos0, size_t seq_stride,
                                                      float* __restrict__ kc, float* __restrict__ vc) {
    const int r = blockIdx.y, s = blockIdx.z;
    const float* src = qkv + (static_cast<size_t>(s) * rows + r) * ld;
    const size_t dst = static_cast<size_t>(s) * seq_stride + static_cast<size_t>(pos0 + r) * kv_dim;
    for (int c = blockIdx.x * kPT + threadIdx.x; c < kv_dim; c += gridDim.x * kPT) {
        kc[dst + c] = src[k_off + c];
        vc[dst + c] = src[v_off + c];
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int fh_launch_attention_prefill_seqs(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t seq_stride,
                                     size_t d, size_t heads, size_t pos0, size_t rows, size_t seqs, float* out) {
    const size_t hd = d / heads;
    const bool mfma = hd == static_cast<size_t>(kHd) && aligned16(qkv) && aligned16(kc) && aligned16(vc) &&
                      aligned16(out) && seq_stride % 4 == 0;
    if (!mfma) {
        // other head widths: the vector-unit kernel, one sequence at a time
        for (size_t s = 0; s < seqs; s++) {
            const int rc = fh_launch_attention_prefill(ctx, qkv + s * rows * 3 * d, kc + s * seq_stride,
                                                       vc + s * seq_stride, d, heads, pos0, rows, out + s * rows * d);
            if (rc) return rc;
        }
        return FH_OK;
    }
    const unsigned gx = static_cast<unsigned>((d + kPT - 1) / kPT);
    hipLaunchKernelGGL(k_kv_store_seqs, dim3(gx, static_cast<unsigned>(rows), static_cast<unsigned>(seqs)),
                       dim3(kPT), 0, ctx->stream, qkv, static_cast<int>(3 * d), static_cast<int>(d),
                       static_cast<int>(2 * d), static_cast<int>(d), static_cast<int>(rows), static_cast<int>(pos0),
                       seq_stride, kc, vc);
    FH_HIP(ctx, hipGetLastError());
    PrefillArgs a{};
    a.qkv = qkv;
    a.ld = static_cast<int>(3 * d);
    a.kc = kc;
    a.vc = vc;
    a.seq_stride = seq_stride;
    a.kv_dim = static_cast<int>(d);
    a.rows = static_cast<int>(rows);
    a.pos0 = static_cast<int>(pos0);
    a.groups = static_cast<int>((rows + kQRows - 1) / kQRows);
    a.scale = 1.0f / sqrtf(static_cast<float>(hd));
    a.out = out;
    a.out_ld = static_cast<int>(d);
    hipLaunchKernelGGL(k_attn_prefill_mfma,
                       dim3(static_cast<unsigned>(a.groups), static_cast<unsigned>(heads), static_cast<unsigned>(seqs)),
                       dim3(kPT), 0, ctx->stream, a);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
