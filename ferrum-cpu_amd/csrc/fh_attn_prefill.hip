// fh_attn_prefill.hip — the attention of a prompt block on the matrix cores.
//
// What it computes: the attention of TransformerBlock::forward_with_cache
// (layer/transformer.rs:242-279) for every row of a prompt block at once.
// CachedTransformer's prime (slm/cached.rs:129-136) feeds a prompt position by
// position; here row r of sequence s is position pos0 + r and attends over
// cache positions 0 .. pos0 + r of its own sequence, with the scores
// (q . k) * 1/sqrt(hd), their softmax and the weighted sum of v rows.  Keys
// before the block come from the caches, the block's own from its q|k|v rows;
// the same launch writes the block's k / v rows into the caches.
//
// How (head width 64): one workgroup per (128 query rows, head, sequence).
// Each of its four waves owns 32 query rows and walks 32-key tiles of the
// sequence's cache up to its last row's position; the tiles are staged in LDS
// once for the four waves (double-buffered, the next tile's loads in flight
// while the current one is used).  Per tile, flash style: S^T = K Q^T on the
// matrix cores, the masked softmax with a running max and sum per query
// (exact rescaling between tiles), then O += P V on the matrix cores, P
// going in straight from the S^T accumulators and the outputs coming out one
// query row per accumulator (coalesced stores).  The f32 operands ride on the
// f16 matrix cores as two terms each (k_attn_prefill_f16 below).
#include "fh_internal.hpp"

#pragma clang fp contract(off)

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPT = 256;       // threads: four waves of 32 query rows
constexpr int kQRows = 128;    // query rows per workgroup
constexpr int kKeys = 32;      // keys per tile
constexpr int kHd = 64;        // head width

struct PrefillArgs {
    const float* qkv;   // row s * rows + r; head h's q at column h * 64
    int ld;             // qkv row stride (floats)
    float* kc;          // sequence s's caches at kc / vc + s * seq_stride, rows of kv_dim floats
    float* vc;
    size_t seq_stride;
    int kv_dim;
    int rows, pos0, groups;
    float scale;
    float* out;         // row s * rows + r; head h at column h * 64
    int out_ld;
};

// Query row of accumulator v in a lane of half `half` (the 32 x 32 MFMA
// output layout: rows 8 (v / 4) + 4 half + v % 4).
__device__ __forceinline__ int acc_row(int v, int half) { return (v >> 2) * 8 + half * 4 + (v & 3); }

// The products on the f16 matrix cores: every f32 operand is carried as two
// f16 terms, x = h + l with l = f16(x - h) (22 significant bits), and a
// product of two such operands as the three f16 products h h' + h l' + l h'
// (the dropped l l' is 2^-22 of it), summed in f32 by v_mfma_f32_32x32x16_f16:
// 12 MFMAs per 32-key tile for S^T = K Q^T and 12 for O += P V, against 32 +
// 32 v_mfma_f32_32x32x2_f32 on the fp32 path, each of which takes twice an
// f16 one's cycles (measured on the configs[3] prime: 10.6 -> 6.8 ms).
//   q, k: each query row and each key row is scaled by its own power of two
//     (its largest finite |value| into [2^14, 2^15)) before the split, and
//     the score is unscaled exactly afterwards with the 1/sqrt(64) of the
//     reference: s = S' * 2^-eq * 2^-ek / 8.  Non-finite values keep l = 0,
//     so inf and NaN reach the score as the f32 product gives them.
//   P V: P (in [0, 1]) is split as it leaves the score accumulators; a lane's
//     16 keys of its query are the A operand's two K16 steps as they stand
//     (keys 8 a + 4 half + (0..3)), and the v tile is staged transposed,
//     [dim][key] with the keys in that same order, as the B operand.  A tile
//     whose v values are not all finite and below 2^15 in magnitude is
//     finished on the vector units with only the attended keys (0 * inf would
//     otherwise turn a masked key's v into NaN), v read from the cache.
// The error is that of the 22-bit operands, ~2^-22 relative per product,
// well inside the 1e-5 rule.
constexpr int kHPitch = kHd + 8;   // K tile row pitch (halves): 144-byte rows
constexpr int kVPitch = kKeys + 8;  // V tile (transposed) row pitch (halves): 80-byte rows

typedef _Float16 h8f __attribute__((ext_vector_type(8)));
typedef _Float16 h2f __attribute__((ext_vector_type(2)));

// Position of key kk of a tile in the transposed V rows: K16 step s holds,
// per lane half g, the keys 8 (2 s) + 4 g + (0..3) then 8 (2 s + 1) + 4 g + (0..3).
__device__ __forceinline__ int vkey_pos(int kk) {
    const int a = kk >> 3, g = (kk >> 2) & 1, b = kk & 3;
    return 16 * (a >> 1) + 8 * g + 4 * (a & 1) + b;
}

// Offset of (dim, key position kp) in a transposed V tile: the 8-key chunks
// of dim row d are permuted by (d / 16) % 4, so the pair stores of one wave
// (16 dims 4 apart) spread over the banks; a chunk's 8 keys stay contiguous
// for the 16-byte operand loads.
__device__ __forceinline__ int vt_pos(int d, int kp) {
    return d * kVPitch + 8 * ((kp >> 3) ^ ((d >> 4) & 3)) + (kp & 7);
}

// 2^e with |x| 2^e in [2^14, 2^15) for the largest finite |x| (mx; 0 -> e = 0).
__device__ __forceinline__ int pow2_exponent(float mx) {
    if (!(mx > 0.0f)) return 0;
    const int E = static_cast<int>((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFF) - 126;
    return min(max(15 - E, -126), 126);
}
__device__ __forceinline__ float pow2f(int e) { return __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23); }

// e^x for x <= 0 as 2^(x log2 e) on the hardware's exp2 (v_exp_f32, 1 ulp):
// the product's rounding adds |x| 2^-24 relative, ~1e-6 for the x that carry
// weight in a softmax, far inside the 1e-5 rule; -inf gives 0, NaN stays NaN.
__device__ __forceinline__ float exp_approx(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// Two scaled f32 values as f16 h and l terms (l = 0 for a non-finite value).
__device__ __forceinline__ void split2(float x0, float x1, float sc, h2f& h, h2f& l) {
    const float s0 = x0 * sc, s1 = x1 * sc;
    h = h2f{static_cast<_Float16>(s0), static_cast<_Float16>(s1)};
    const float r0 = __builtin_isfinite(s0) ? s0 - static_cast<float>(h.x) : 0.0f;
    const float r1 = __builtin_isfinite(s1) ? s1 - static_cast<float>(h.y) : 0.0f;
    l = h2f{static_cast<_Float16>(r0), static_cast<_Float16>(r1)};
}

__global__ void __launch_bounds__(kPT, 2) k_attn_prefill_f16(PrefillArgs a) {
    __shared__ __align__(16) _Float16 kh[2][kKeys * kHPitch], kl[2][kKeys * kHPitch];
    __shared__ __align__(16) _Float16 vh[2][kHd * kVPitch], vl[2][kHd * kVPitch];
    __shared__ __align__(16) float kinv[2][kKeys];           // 2^-ek per key row
    __shared__ __align__(16) float cx[4][32];                // per wave: one factor per query row
    __shared__ __align__(16) float pt[4][kKeys * 33];        // per wave: P of a tile with unsafe v ([key][query])

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, col = lane & 31;
    const int g = a.groups - 1 - static_cast<int>(blockIdx.x);  // the longest rows first
    const int h = blockIdx.y, s = blockIdx.z;
    const int r0 = g * kQRows + wave * 32;
    const int last_row = min(a.rows - 1, g * kQRows + kQRows - 1);
    const int kmax = a.pos0 + last_row;
    const int ntiles = kmax / kKeys + 1;
    const int my_tiles = r0 < a.rows ? (a.pos0 + min(a.rows - 1, r0 + 31)) / kKeys + 1 : 0;
    const size_t sbase = static_cast<size_t>(s) * a.seq_stride + static_cast<size_t>(h) * kHd;
    float* kc = a.kc + sbase;
    float* vc = a.vc + sbase;

    // This lane's query: dims 16 i + 8 half + (0..7), i = 0..3 (the B
    // operand of step i), scaled by the row's power of two and split.
    h8f qh[4], ql[4];
    float qscale;
    {
        const int row = min(r0 + col, a.rows - 1);
        const float* qp = a.qkv + (static_cast<size_t>(s) * a.rows + row) * a.ld + h * kHd + half * 8;
        float qv[32];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 u = *reinterpret_cast<const float4*>(qp + 16 * i);
            const float4 w = *reinterpret_cast<const float4*>(qp + 16 * i + 4);
            qv[8 * i] = u.x; qv[8 * i + 1] = u.y; qv[8 * i + 2] = u.z; qv[8 * i + 3] = u.w;
            qv[8 * i + 4] = w.x; qv[8 * i + 5] = w.y; qv[8 * i + 6] = w.z; qv[8 * i + 7] = w.w;
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++)
            if (__builtin_isfinite(qv[i])) mx = fmaxf(mx, fabsf(qv[i]));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // the other half of the row
        const int eq = pow2_exponent(mx);
        const float sc = pow2f(eq);
        qscale = pow2f(-eq) * a.scale;  // (a.scale = 1/8: the product stays exact)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                h2f hh, ll;
                split2(qv[8 * i + j], qv[8 * i + j + 1], sc, hh, ll);
                qh[i][j] = hh.x; qh[i][j + 1] = hh.y;
                ql[i][j] = ll.x; ql[i][j + 1] = ll.y;
            }
    }
    const int qpos = a.pos0 + r0 + col;

    // Tile staging: thread t takes float4s t and t + 256 of the k and of the v
    // rows (row idx / 16, dims 4 (idx % 16) ...); the 16 threads of a key row
    // are consecutive lanes, so its exponent is a 16-lane reduction.  Keys of
    // the block itself (pos0 on) come from its q|k|v rows, earlier ones from
    // the cache; workgroup 0 of each (sequence, head), which walks every tile,
    // also writes the block's k and v rows into the cache as it stages them
    // (no other workgroup of the launch reads those cache rows).
    const bool writer = blockIdx.x == 0;
    const float* bq = a.qkv + static_cast<size_t>(s) * a.rows * a.ld + h * kHd;  // this sequence's block rows
    // The v rows go by pairs instead: thread t takes keys 2 (t / 16) and
    // 2 (t / 16) + 1, dims 4 (t % 16) ..., which sit side by side in the
    // transposed tile, so each dim is one 4-byte store per term.
    float4 pk[2], pv[2];
    auto key_row = [&](int key, int off, const float* cache) __attribute__((always_inline)) {
        return key >= a.pos0 ? bq + static_cast<size_t>(key - a.pos0) * a.ld + off
                             : cache + static_cast<size_t>(key) * a.kv_dim;
    };
    auto fetch = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * kPT, c4 = idx & 15;
            const int key = min(t * kKeys + (idx >> 4), kmax);
            const int vkey = min(t * kKeys + 2 * (tid >> 4) + i, kmax);
            pk[i] = *reinterpret_cast<const float4*>(key_row(key, a.kv_dim, kc) + c4 * 4);
            pv[i] = *reinterpret_cast<const float4*>(key_row(vkey, 2 * a.kv_dim, vc) + c4 * 4);
        }
    };
    auto store_block_rows = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * kPT, c4 = idx & 15;
            const int key = t * kKeys + (idx >> 4), vkey = t * kKeys + 2 * (tid >> 4) + i;
            if (key >= a.pos0 && key <= kmax)
                *reinterpret_cast<float4*>(kc + static_cast<size_t>(key) * a.kv_dim + c4 * 4) = pk[i];
            if (vkey >= a.pos0 && vkey <= kmax)
                *reinterpret_cast<float4*>(vc + static_cast<size_t>(vkey) * a.kv_dim + c4 * 4) = pv[i];
        }
    };
    // returns whether this thread's v values are unsafe for the f16 split
    auto stash = [&](int buf) __attribute__((always_inline)) -> bool {
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int idx = tid + i * kPT, row = idx >> 4, c0 = (idx & 15) * 4;
            const float4 k4 = pk[i];
            float mx = 0.0f;
            if (__builtin_isfinite(k4.x)) mx = fmaxf(mx, fabsf(k4.x));
            if (__builtin_isfinite(k4.y)) mx = fmaxf(mx, fabsf(k4.y));
            if (__builtin_isfinite(k4.z)) mx = fmaxf(mx, fabsf(k4.z));
            if (__builtin_isfinite(k4.w)) mx = fmaxf(mx, fabsf(k4.w));
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
            const int ek = pow2_exponent(mx);
            h2f h01, l01, h23, l23;
            split2(k4.x, k4.y, pow2f(ek), h01, l01);
            split2(k4.z, k4.w, pow2f(ek), h23, l23);
            *reinterpret_cast<uint2*>(&kh[buf][row * kHPitch + c0]) =
                make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
            *reinterpret_cast<uint2*>(&kl[buf][row * kHPitch + c0]) =
                make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
            if (c0 == 0) kinv[buf][row] = pow2f(-ek);
        }
        const int c0 = (tid & 15) * 4, kp = vkey_pos(2 * (tid >> 4));  // even; the pair's second key at kp + 1
        const float va[4] = {pv[0].x, pv[0].y, pv[0].z, pv[0].w};
        const float vb[4] = {pv[1].x, pv[1].y, pv[1].z, pv[1].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            bad |= !(fabsf(va[j]) < 32768.0f) || !(fabsf(vb[j]) < 32768.0f);  // (also NaN)
            const h2f hv = h2f{static_cast<_Float16>(va[j]), static_cast<_Float16>(vb[j])};
            const h2f lv = h2f{static_cast<_Float16>(va[j] - static_cast<float>(hv.x)),
                               static_cast<_Float16>(vb[j] - static_cast<float>(hv.y))};
            const int at = vt_pos(c0 + j, kp);
            *reinterpret_cast<uint32_t*>(&vh[buf][at]) = __builtin_bit_cast(uint32_t, hv);
            *reinterpret_cast<uint32_t*>(&vl[buf][at]) = __builtin_bit_cast(uint32_t, lv);
        }
        return bad;
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x16 o0, o1;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        o0[v] = 0.0f;
        o1[v] = 0.0f;
    }
    fetch(0);
    if (writer) store_block_rows(0);
    bool vbad = __syncthreads_or(stash(0));
    for (int t = 0; t < ntiles; t++) {
        const int buf = t & 1, k0 = t * kKeys;
        if (t + 1 < ntiles) fetch(t + 1);
        if (t < my_tiles) {
            // ---- S'^T = K Q^T (scaled terms): accumulator v of lane (half, col) is key acc_row(v, half), query col
            f32x16 sacc;
#pragma unroll
            for (int v = 0; v < 16; v++) sacc[v] = 0.0f;
            const _Float16* khr = &kh[buf][col * kHPitch + half * 8];
            const _Float16* klr = &kl[buf][col * kHPitch + half * 8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const h8f a_h = *reinterpret_cast<const h8f*>(khr + 16 * i);
                const h8f a_l = *reinterpret_cast<const h8f*>(klr + 16 * i);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, qh[i], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, ql[i], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, qh[i], sacc, 0, 0, 0);
            }
            // ---- scores, unscaled exactly, masked past the query's position
            float sv[16];
            float mt = -INFINITY;
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) {
                const float4 ki = *reinterpret_cast<const float4*>(&kinv[buf][a4 * 8 + half * 4]);
                const float kv4[4] = {ki.x, ki.y, ki.z, ki.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int v = 4 * a4 + j;
                    sv[v] = k0 + acc_row(v, half) <= qpos ? sacc[v] * qscale * kv4[j] : -INFINITY;
                    mt = fmaxf(mt, sv[v]);
                }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float m_new = fmaxf(m_run, mt);
            const float corr = exp_approx(m_run - m_new);  // 0 on the first tile (m_run = -inf)
            float ps = 0.0f;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                sv[v] = exp_approx(sv[v] - m_new);
                ps += sv[v];
            }
            ps += __shfl_xor(ps, 32, 64);
            l_run = l_run * corr + ps;
            m_run = m_new;
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
            if (!vbad) {
                // ---- O += P V: step st takes this lane's keys acc_row(8 st + j, half)
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    h8f ph, pl;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float p = sv[8 * st + j];
                        ph[j] = static_cast<_Float16>(p);
                        pl[j] = static_cast<_Float16>(p - static_cast<float>(ph[j]));
                    }
                    const int off = 16 * st + 8 * half, at0 = vt_pos(col, off), at1 = vt_pos(32 + col, off);
                    const h8f v0h = *reinterpret_cast<const h8f*>(&vh[buf][at0]);
                    const h8f v0l = *reinterpret_cast<const h8f*>(&vl[buf][at0]);
                    const h8f v1h = *reinterpret_cast<const h8f*>(&vh[buf][at1]);
                    const h8f v1l = *reinterpret_cast<const h8f*>(&vl[buf][at1]);
                    o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, v0h, o0, 0, 0, 0);
                    o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, v0l, o0, 0, 0, 0);
                    o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, v0h, o0, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, v1h, o1, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, v1l, o1, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, v1h, o1, 0, 0, 0);
                }
            } else {
                // ---- v not safe for the split: only the attended keys, on the vector units
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
                        const int key = k0 + kk;
                        const float* vrow = key_row(key, 2 * a.kv_dim, vc);
                        s0 += p * vrow[col];
                        s1 += p * vrow[32 + col];
                    }
                    o0[v] = s0;
                    o1[v] = s1;
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        bool vbad_next = false;
        if (t + 1 < ntiles) {
            if (writer) store_block_rows(t + 1);
            vbad_next = stash(buf ^ 1);
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
    hipLaunchKernelGGL(k_attn_prefill_f16,
                       dim3(static_cast<unsigned>(a.groups), static_cast<unsigned>(heads), static_cast<unsigned>(seqs)),
                       dim3(kPT), 0, ctx->stream, a);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
