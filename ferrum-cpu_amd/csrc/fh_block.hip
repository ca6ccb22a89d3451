// fh_block.hip — the rest of a GPT-2 decode step on gfx950: token + position
// embedding, LayerNorm, GELU, the residual add and the KV-cache attention of
// one new position.  With the Q8_0 linears (fh_linear.hip) and the fused
// sampler (fh_sampler.hip) a whole decode step stays on the device.
//
//  k_embed_one   Embedding::embed_one (layer/embedding.rs:70-90).
//  k_embed_rows_pos  the same for a batch of sequences, each row at its own
//                position (token and position ids on the device).
//  k_layernorm   LayerNorm::forward (layer/norm.rs:46-82), one workgroup per
//                row; the row sums are tree reductions in a fixed order.
//  k_gelu        activation::gelu (activation.rs:9-12), in place.
//  k_add         the residual adds of forward_with_cache (layer/transformer.rs:
//                281, 288), in place.
//  k_add_layernorm  a residual add and the LayerNorm that follows it (ln2 of
//                the block, or the next block's ln1 / the final LayerNorm) in
//                one pass: the same arithmetic as k_add then k_layernorm.
//  k_attn_chunk  the attention of forward_with_cache (layer/transformer.rs:
//                242-279) for one query: the new k and v rows are written at
//                cache row pos, then each (head, chunk of 32 to 128 positions)
//                workgroup forms its scores, their max, sum of exponentials and
//                the exponential-weighted sum of v rows; with one chunk per head
//                it writes the output, otherwise the last chunk of a head to
//                finish merges the chunks (max, rescaled sums).  The reference sums in position order with one
//                global max; the merge is the same value up to rounding.
// Arithmetic is written without contraction, as the reference has no FMA.
#include "fh_internal.hpp"

#include <type_traits>

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 32;    // cache positions per attention workgroup
constexpr int kMaxHd = 128;   // head width the attention kernel supports

using fh::block_sum;
using fh::wave_sum;

__global__ void __launch_bounds__(kThreads) k_embed_one(const float* __restrict__ tok_w, const float* __restrict__ pos_w,
                                                       int vocab, int d, const uint32_t* __restrict__ token, int pos,
                                                       float* __restrict__ out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= d) return;
    const uint32_t t = *token;
    // An id past the vocabulary (never one the sampler returns) poisons the row.
    out[i] = t < static_cast<uint32_t>(vocab) ? tok_w[static_cast<size_t>(t) * d + i] + pos_w[static_cast<size_t>(pos) * d + i]
                                              : __builtin_nanf("");
}

// Embedding::embed_one for `rows` sequences at once: row r is token tokens[r]
// at position pos[r] (both on the device).  An id past the vocabulary or a
// position past the table poisons the row (the host checks positions before
// the launch).  With hist set, workgroup 0 of each row also records the id at
// hist[r * hist_stride + pos[r]] (a batched decode's per-row penalty window).
__global__ void __launch_bounds__(kThreads) k_embed_rows_pos(const float* __restrict__ tok_w,
                                                            const float* __restrict__ pos_w, int vocab, int max_seq,
                                                            int d, const uint32_t* __restrict__ tokens,
                                                            const uint32_t* __restrict__ pos, uint32_t* hist,
                                                            int hist_stride, float* __restrict__ out) {
    const int r = blockIdx.y, i = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t t = tokens[r], p = pos[r];
    if (hist && blockIdx.x == 0 && threadIdx.x == 0 && p < static_cast<uint32_t>(hist_stride))
        hist[static_cast<size_t>(r) * hist_stride + p] = t;
    if (i >= d) return;
    out[static_cast<size_t>(r) * d + i] =
        t < static_cast<uint32_t>(vocab) && p < static_cast<uint32_t>(max_seq)
            ? tok_w[static_cast<size_t>(t) * d + i] + pos_w[static_cast<size_t>(p) * d + i]
            : __builtin_nanf("");
}

__global__ void __launch_bounds__(kThreads) k_layernorm(const float* __restrict__ x, int d,
                                                       const float* __restrict__ gamma, const float* __restrict__ beta,
                                                       float* __restrict__ y) {
    __shared__ float red[kThreads / 64];
    const float* xr = x + static_cast<size_t>(blockIdx.x) * d;
    float* yr = y + static_cast<size_t>(blockIdx.x) * d;
    float s = 0.0f;
    for (int c = threadIdx.x; c < d; c += kThreads) s += xr[c];
    const float mean = block_sum(s, red) / static_cast<float>(d);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < d; c += kThreads) {
        const float dv = xr[c] - mean;
        ss += dv * dv;
    }
    const float var = block_sum(ss, red) / static_cast<float>(d);
    const float sd = sqrtf(var + 1e-5f);
    for (int c = threadIdx.x; c < d; c += kThreads) yr[c] = ((xr[c] - mean) / sd) * gamma[c] + beta[c];
}

__global__ void __launch_bounds__(kThreads) k_gelu(float* __restrict__ x, size_t n) {
    const size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    x[i] = 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * v * v * v)));
}

__global__ void __launch_bounds__(kThreads) k_add(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    const size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

// Rows r of a prompt block: their k and v slices (qkv + r * ld + k_off / v_off,
// kv_dim values each) into cache rows pos0 + r, before the block's attention
// reads them (one sequence: every row shares the cache).
__global__ void __launch_bounds__(kThreads) k_kv_store(const float* __restrict__ qkv, int ld, int k_off, int v_off,
                                                      int kv_dim, int pos0, float* __restrict__ kc,
                                                      float* __restrict__ vc) {
    const int r = blockIdx.y;
    const float* src = qkv + static_cast<size_t>(r) * ld;
    const size_t dst = static_cast<size_t>(pos0 + r) * kv_dim;
    for (int c = blockIdx.x * kThreads + threadIdx.x; c < kv_dim; c += gridDim.x * kThreads) {
        kc[dst + c] = src[k_off + c];
        vc[dst + c] = src[v_off + c];
    }
}

// Grid (chunks, heads, rows); a workgroup covers S sub-chunks of 32
// positions of one query head of one row (sequence).  Row r's q|k|v sits at
// qkv + r * ld (q heads, then kv heads at k_off and v_off); its caches at
// kc / vc + r * seq_stride, one kv_dim-wide row per position; query head h
// reads kv head h / group (group 1: multi-head, GPT-2).  Row r's position is
// dpos[r] (device) or pos; chunks past it exit at once, and a position at or
// past cap, or past the launch's max_len - 1, gives a NaN output and writes
// nothing.
// Every K, V and q element a thread needs is loaded at entry, so one memory
// latency covers the whole chunk.  With one chunk the workgroup writes the
// head's output itself; otherwise part: [rows][heads][chunks][2 + hd] (max,
// sum, weighted v sum) is written with device-coherent stores and the last
// chunk of a (row, head) to arrive merges them.  counters: [rows][heads], left 0.
struct AttnArgs {
    const float* qkv;
    int ld, k_off, v_off;
    float* kc;
    float* vc;
    size_t seq_stride;
    int kv_dim, group;
    const uint32_t* dpos;
    int pos, cap;
    int pos_step;  // without dpos, row r's position is pos + pos_step * r
    int max_len;   // rows at positions past max_len - 1 get NaN and write nothing
    float scale;
    float* part;
    unsigned* counters;
    float* out;
    int out_ld;
};

template <int S, int HD>
__global__ void __launch_bounds__(kThreads) k_attn_chunk(AttnArgs a) {
    constexpr int kPos = S * kChunk;             // positions per workgroup
    constexpr int hd = HD, per = HD / 8;         // dims per lane of a score
    constexpr int groups = kThreads / HD;        // threads per v column
    constexpr int vper = kChunk / groups;        // v rows per thread and sub-chunk
    __shared__ float sc[kPos];
    __shared__ float acc[kThreads];
    __shared__ float stat[2];
    __shared__ int last;
    const int chunk = blockIdx.x, head = blockIdx.y, row = blockIdx.z;
    const int hs = head * hd, tid = threadIdx.x;
    const int kvs = (head / a.group) * hd;  // this head's kv slice
    const int pos = a.dpos ? static_cast<int>(min(a.dpos[row], 0x7FFFFFFFu)) : a.pos + a.pos_step * row;
    float* out = a.out + static_cast<size_t>(row) * a.out_ld + hs;
    if (pos >= a.cap) {  // a position the cache cannot hold
        if (chunk == 0 && tid < hd) out[tid] = __builtin_nanf("");
        return;
    }
    const int len = pos + 1, chunks = (len + kPos - 1) / kPos;
    if (len > a.max_len) {  // a position past the launch's max_pos
        if (chunk == 0 && tid < hd) out[tid] = __builtin_nanf("");
        return;
    }
    if (chunk >= chunks) return;
    const int j0 = chunk * kPos, jn = min(kPos, len - j0);
    const int jl = tid >> 3, part8 = tid & 7, t = tid % hd, g = tid / hd;
    const float* qkv = a.qkv + static_cast<size_t>(row) * a.ld;
    const int d = a.kv_dim;
    float* kc = a.kc + row * a.seq_stride + kvs;
    float* vc = a.vc + row * a.seq_stride + kvs;
    const float* knew = qkv + a.k_off + kvs;
    const float* vnew = qkv + a.v_off + kvs;
    const float scale = a.scale;
    // loads: this lane's q slice, its K slices (one position per sub-chunk)
    // and its V elements (vper positions per sub-chunk).  Position pos (and
    // any position past it, which is masked) comes from qkv itself, never
    // from the cache, so no workgroup depends on another's store.
    float qr[per], kr[S][per], vr[S][vper];
#pragma unroll
    for (int i = 0; i < per; i++) qr[i] = qkv[hs + part8 * per + i];
#pragma unroll
    for (int u = 0; u < S; u++) {
        const int j = j0 + u * kChunk + jl;
        const float* krow = j >= pos ? knew : kc + static_cast<size_t>(j) * d;
#pragma unroll
        for (int i = 0; i < per; i++) kr[u][i] = krow[part8 * per + i];
#pragma unroll
        for (int i = 0; i < vper; i++) {
            const int jv = j0 + u * kChunk + g + i * groups;
            const float* vrow = jv >= pos ? vnew : vc + static_cast<size_t>(jv) * d;
            vr[u][i] = vrow[t];
        }
    }
    // the new row: chunk 0 of the first query head of each kv head writes
    // that kv head's slice of k and v at row pos
    if (chunk == 0 && head % a.group == 0 && tid < hd) {
        kc[static_cast<size_t>(pos) * d + tid] = knew[tid];
        vc[static_cast<size_t>(pos) * d + tid] = vnew[tid];
    }
    // scores: 8 lanes per position, each over hd / 8 consecutive dims in
    // ascending order, then a fixed 8-lane tree
#pragma unroll
    for (int u = 0; u < S; u++) {
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < per; i++) dot += qr[i] * kr[u][i];
        dot += __shfl_xor(dot, 1, 64);
        dot += __shfl_xor(dot, 2, 64);
        dot += __shfl_xor(dot, 4, 64);
        const int jc = u * kChunk + jl;
        if (part8 == 0) sc[jc] = jc < jn ? dot * scale : -INFINITY;
    }
    __syncthreads();
    // the chunk's max and exponentials, once each (wave 0; position l + 64 i)
    if (tid < 64) {
        constexpr int kL = (kPos + 63) / 64;
        float s[kL];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < kL; i++) {
            const int jc = tid + 64 * i;
            s[i] = jc < kPos ? sc[jc] : -INFINITY;
            mx = fmaxf(mx, s[i]);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float se = 0.0f;
#pragma unroll
        for (int i = 0; i < kL; i++) {
            const int jc = tid + 64 * i;
            const float e = jc < jn ? expf(s[i] - mx) : 0.0f;
            if (jc < kPos) sc[jc] = e;
            se += e;
        }
        se = wave_sum(se);
        if (tid == 0) {
            stat[0] = mx;
            stat[1] = se;
        }
    }
    __syncthreads();
    // weighted v sum: thread (g, t) takes positions g, g + groups, ... of
    // each sub-chunk, in order; positions past the chunk are skipped
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < S; u++)
#pragma unroll
        for (int i = 0; i < vper; i++) {
            const int jc = u * kChunk + g + i * groups;
            if (jc < jn) o += sc[jc] * vr[u][i];
        }
    acc[tid] = o;
    __syncthreads();
    float r = 0.0f;
    if (tid < hd)
        for (int gg = 0; gg < groups; gg++) r += acc[gg * hd + tid];
    if (chunks == 1) {
        if (tid < hd) out[tid] = r / stat[1];
        return;
    }
    const int cmax = gridDim.x;  // partial slots per (row, head)
    const size_t rh = static_cast<size_t>(row) * gridDim.y + head;
    float* mine = a.part + (rh * cmax + chunk) * (2 + hd);
    if (tid < hd) __hip_atomic_store(mine + 2 + tid, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        __hip_atomic_store(mine, stat[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + 1, stat[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Publish: every thread's coherent stores complete before the arrival
    // count moves, so the last arrival reads whole partials.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) last = atomicAdd(a.counters + rh, 1u) == static_cast<unsigned>(chunks - 1);
    __syncthreads();
    if (!last) return;
    // Merge, eight chunks per round with all their loads in flight at once;
    // a running max rescales the sums when a later round raises it.
    const float* hp = a.part + rh * cmax * (2 + hd);
    constexpr int R = 8;
    const int tt = min(tid, hd - 1);
    float M = -INFINITY, Sm = 0.0f, rm = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += R) {
        float mc[R], sc8[R], oc[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float* cp = hp + min(c0 + i, chunks - 1) * (2 + hd);
            mc[i] = __hip_atomic_load(cp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sc8[i] = __hip_atomic_load(cp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            oc[i] = __hip_atomic_load(cp + 2 + tt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        float Mn = M;
#pragma unroll
        for (int i = 0; i < R; i++) Mn = fmaxf(Mn, mc[i]);  // repeats of the last chunk change nothing
        if (Mn != M) {
            const float f = expf(M - Mn);  // 0 on the first round (M = -inf)
            Sm = Sm * f;
            rm = rm * f;
            M = Mn;
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            if (c0 + i >= chunks) break;
            const float f = expf(mc[i] - M);
            Sm += sc8[i] * f;
            rm += oc[i] * f;
        }
    }
    if (tid < hd) out[tid] = rm / Sm;
    if (tid == 0) __hip_atomic_store(a.counters + rh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grouped-query attention: k_attn_chunk for QG query heads that share one kv
// head (QG divides the group), so the workgroup loads the kv head's K and V
// rows once for all of them instead of once per query head.  Grid (chunks,
// heads / QG, rows).  Every query head's arithmetic is k_attn_chunk's, in the
// same order (its scores, the max and exponentials of one wave, the v sums,
// the merge), so the outputs are the same bits; wave w takes the softmax of
// heads w, w + 4, ...  counters: [rows][heads / QG], left 0.
template <int S, int HD, int QG>
__global__ void __launch_bounds__(kThreads) k_attn_group(AttnArgs a) {
    constexpr int kPos = S * kChunk;
    constexpr int hd = HD, per = HD / 8;
    constexpr int groups = kThreads / HD;
    constexpr int vper = kChunk / groups;
    constexpr int kW = kThreads / 64;
    __shared__ float sc[QG][kPos];
    __shared__ float acc[QG][kThreads];
    __shared__ float stat[QG][2];
    __shared__ int last;
    const int chunk = blockIdx.x, hg = blockIdx.y, row = blockIdx.z;
    const int h0 = hg * QG, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvs = (h0 / a.group) * hd;
    const int pos = a.dpos ? static_cast<int>(min(a.dpos[row], 0x7FFFFFFFu)) : a.pos + a.pos_step * row;
    float* out = a.out + static_cast<size_t>(row) * a.out_ld + static_cast<size_t>(h0) * hd;
    const int len = pos + 1, chunks = (len + kPos - 1) / kPos;
    if (pos >= a.cap || len > a.max_len) {  // a position the cache or the launch cannot hold
        if (chunk == 0)
            for (int i = tid; i < QG * hd; i += kThreads) out[i] = __builtin_nanf("");
        return;
    }
    if (chunk >= chunks) return;
    const int j0 = chunk * kPos, jn = min(kPos, len - j0);
    const int jl = tid >> 3, part8 = tid & 7, t = tid % hd, g = tid / hd;
    const float* qkv = a.qkv + static_cast<size_t>(row) * a.ld;
    const int d = a.kv_dim;
    float* kc = a.kc + row * a.seq_stride + kvs;
    float* vc = a.vc + row * a.seq_stride + kvs;
    const float* knew = qkv + a.k_off + kvs;
    const float* vnew = qkv + a.v_off + kvs;
    const float scale = a.scale;
    float qr[QG][per], kr[S][per], vr[S][vper];
#pragma unroll
    for (int qh = 0; qh < QG; qh++)
#pragma unroll
        for (int i = 0; i < per; i++) qr[qh][i] = qkv[(h0 + qh) * hd + part8 * per + i];
#pragma unroll
    for (int u = 0; u < S; u++) {
        const int j = j0 + u * kChunk + jl;
        const float* krow = j >= pos ? knew : kc + static_cast<size_t>(j) * d;
#pragma unroll
        for (int i = 0; i < per; i++) kr[u][i] = krow[part8 * per + i];
#pragma unroll
        for (int i = 0; i < vper; i++) {
            const int jv = j0 + u * kChunk + g + i * groups;
            const float* vrow = jv >= pos ? vnew : vc + static_cast<size_t>(jv) * d;
            vr[u][i] = vrow[t];
        }
    }
    if (chunk == 0 && h0 % a.group == 0 && tid < hd) {
        kc[static_cast<size_t>(pos) * d + tid] = knew[tid];
        vc[static_cast<size_t>(pos) * d + tid] = vnew[tid];
    }
#pragma unroll
    for (int qh = 0; qh < QG; qh++)
#pragma unroll
        for (int u = 0; u < S; u++) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < per; i++) dot += qr[qh][i] * kr[u][i];
            dot += __shfl_xor(dot, 1, 64);
            dot += __shfl_xor(dot, 2, 64);
            dot += __shfl_xor(dot, 4, 64);
            const int jc = u * kChunk + jl;
            if (part8 == 0) sc[qh][jc] = jc < jn ? dot * scale : -INFINITY;
        }
    __syncthreads();
    for (int qh = wave; qh < QG; qh += kW) {  // (wave-uniform)
        constexpr int kL = (kPos + 63) / 64;
        float sv[kL];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < kL; i++) {
            const int jc = lane + 64 * i;
            sv[i] = jc < kPos ? sc[qh][jc] : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float se = 0.0f;
#pragma unroll
        for (int i = 0; i < kL; i++) {
            const int jc = lane + 64 * i;
            const float e = jc < jn ? expf(sv[i] - mx) : 0.0f;
            if (jc < kPos) sc[qh][jc] = e;
            se += e;
        }
        se = wave_sum(se);
        if (lane == 0) {
            stat[qh][0] = mx;
            stat[qh][1] = se;
        }
    }
    __syncthreads();
#pragma unroll
    for (int qh = 0; qh < QG; qh++) {
        float o = 0.0f;
#pragma unroll
        for (int u = 0; u < S; u++)
#pragma unroll
            for (int i = 0; i < vper; i++) {
                const int jc = u * kChunk + g + i * groups;
                if (jc < jn) o += sc[qh][jc] * vr[u][i];
            }
        acc[qh][tid] = o;
    }
    __syncthreads();
    // outputs (query head qh, dim): r over the thread groups in order
    constexpr int kOut = (QG * HD + kThreads - 1) / kThreads;
    float rr[kOut];
#pragma unroll
    for (int q = 0; q < kOut; q++) {
        const int oi = min(tid + q * kThreads, QG * hd - 1), qh = oi / hd, dm = oi % hd;
        float r = 0.0f;
        for (int gg = 0; gg < groups; gg++) r += acc[qh][gg * hd + dm];
        rr[q] = r;
    }
    if (chunks == 1) {
#pragma unroll
        for (int q = 0; q < kOut; q++) {
            const int oi = tid + q * kThreads;
            if (oi < QG * hd) out[oi] = rr[q] / stat[oi / hd][1];
        }
        return;
    }
    const int cmax = gridDim.x;
    const int heads = gridDim.y * QG;
#pragma unroll
    for (int q = 0; q < kOut; q++) {
        const int oi = tid + q * kThreads;
        if (oi >= QG * hd) break;
        const size_t rh = static_cast<size_t>(row) * heads + h0 + oi / hd;
        float* mine = a.part + (rh * cmax + chunk) * (2 + hd);
        __hip_atomic_store(mine + 2 + oi % hd, rr[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (oi % hd == 0) {
            __hip_atomic_store(mine, stat[oi / hd][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(mine + 1, stat[oi / hd][1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const size_t rg = static_cast<size_t>(row) * gridDim.y + hg;
    if (tid == 0) last = atomicAdd(a.counters + rg, 1u) == static_cast<unsigned>(chunks - 1);
    __syncthreads();
    if (!last) return;
    constexpr int R = 8;
#pragma unroll
    for (int q = 0; q < kOut; q++) {
        const int oi = tid + q * kThreads;
        if (oi >= QG * hd) break;
        const size_t rh = static_cast<size_t>(row) * heads + h0 + oi / hd;
        const float* hp = a.part + rh * cmax * (2 + hd);
        const int tt = oi % hd;
        float M = -INFINITY, Sm = 0.0f, rm = 0.0f;
        for (int c0 = 0; c0 < chunks; c0 += R) {
            float mc[R], sc8[R], oc[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float* cp = hp + min(c0 + i, chunks - 1) * (2 + hd);
                mc[i] = __hip_atomic_load(cp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sc8[i] = __hip_atomic_load(cp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                oc[i] = __hip_atomic_load(cp + 2 + tt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            float Mn = M;
#pragma unroll
            for (int i = 0; i < R; i++) Mn = fmaxf(Mn, mc[i]);
            if (Mn != M) {
                const float f = expf(M - Mn);
                Sm = Sm * f;
                rm = rm * f;
                M = Mn;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                if (c0 + i >= chunks) break;
                const float f = expf(mc[i] - M);
                Sm += sc8[i] * f;
                rm += oc[i] * f;
            }
        }
        out[oi] = rm / Sm;
    }
    if (tid == 0) __hip_atomic_store(a.counters + rg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Many rows at once (a batched decode): one workgroup per (row, kv head,
// part of its query-head group) takes up to QS query heads of the kv head's
// group over all of the row's positions and merges them itself, so nothing
// goes through memory between workgroups and each K / V row is read from HBM
// once (the parts of a group read it again from the caches).  Grid (kv heads
// x parts, rows), kRowsThreads threads; head width 64.  A round covers
// kRowsWaves * 32 positions, 32 per wave: lane (g, c) holds dims 4 c .. 4 c +
// 3 of positions g, g + 4, .. of the wave's 32 v rows.  Its k rows: with
// several query heads (QS > 1), lane pair (2 jj, 2 jj + 1) holds position
// jj's k row (32 dims each), so a score is a two-lane sum and the weights go
// to the v lanes through LDS; with one (QS = 1) the k rows are laid out as the
// v rows (16 lanes per 256-byte row, four rows per load instead of 16-byte
// pieces of 64), a score is a 16-lane sum, and every lane of row g then
// holds the weights of exactly the v rows it multiplies (configs[3]'s
// batch-32 run 148.9 -> 146.5 ms; with two or four heads the 16-lane sums per
// head cost more than they save, the 64-row Qwen2-0.5B step 1.877 -> 1.953).
// Each wave keeps an
// online softmax over its rounds (running max, rescaled sums); the waves'
// (max, sum, weighted v sums) then merge through LDS.  Position pos (and the
// masked positions past it) reads the new k / v rows from qkv; part 0 writes
// them to the cache at row pos.  Scores and sums use FMA and sum in another
// order than the reference (position order, one global max): the same value
// up to rounding.  A query head's arithmetic does not depend on QS or on the
// group.  A row past the cache or past max_len gives NaN and writes nothing.
constexpr int kRowsThreads = 512;
constexpr int kRowsWaves = kRowsThreads / 64;
constexpr int kRowsPos = 32;  // positions per wave and round
constexpr size_t kRowsMinGroups = 128;  // workgroups a launch needs to take k_attn_rows (timed at Qwen2-0.5B shapes)

// Max over the 64 lanes of a wave, the same in every lane: DPP within 16-lane
// rows (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then
// the four rows by readlane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, fh::dpp<0xB1>(v));
    v = fmaxf(v, fh::dpp<0x4E>(v));
    v = fmaxf(v, fh::dpp<0x141>(v));
    v = fmaxf(v, fh::dpp<0x140>(v));
    return fmaxf(fmaxf(fh::rdlane(v, 0), fh::rdlane(v, 16)), fmaxf(fh::rdlane(v, 32), fh::rdlane(v, 48)));
}

// apply_rope's parameters for k_attn_rows's own rotation of q and k.
struct RopeArgs {
    int rope_dim, neox;
    float base, linear_factor;
    const float* freq_factors;
};

struct RowsFrag {
    float4 k[8];  // QS > 1: 32 dims of position jj's k row; QS = 1: as v
    float4 v[8];  // dims c4 .. c4 + 3 of positions g, g + 4, .., g + 28 of the wave's 32
};

// With ROPE, q and the new k row are rotated here (fh::rope_rotate, as
// k_rope) as they are read from qkv, which is left as it is.
template <int QS, bool ROPE>
__global__ void __launch_bounds__(kRowsThreads) k_attn_rows(AttnArgs a, RopeArgs ra) {
    constexpr int HD = 64, R = kRowsWaves * kRowsPos;
    __shared__ __align__(16) float qs[QS][2][36];  // q halves, padded onto other banks
    __shared__ __align__(16) float kn[HD];         // the new k row (rotated with ROPE)
    __shared__ __align__(16) float ps[kRowsWaves][QS][kRowsPos];  // position g + 4 q at g * 8 + q
    __shared__ float wm[kRowsWaves][QS], wl[kRowsWaves][QS];
    __shared__ __align__(16) float wo[kRowsWaves][QS][4][HD];  // each lane group's weighted v sums
    const int parts = (a.group + QS - 1) / QS;
    const int kvh = blockIdx.x / parts, hs = (blockIdx.x % parts) * QS, qn = min(QS, a.group - hs);
    const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h0 = kvh * a.group + hs;  // this workgroup's first query head
    const int pos = a.dpos ? static_cast<int>(min(a.dpos[row], 0x7FFFFFFFu)) : a.pos + a.pos_step * row;
    float* out = a.out + static_cast<size_t>(row) * a.out_ld + static_cast<size_t>(h0) * HD;
    if (pos >= a.cap || pos >= a.max_len) {  // a position the cache or the launch cannot hold
        for (int i = tid; i < qn * HD; i += kRowsThreads) out[i] = __builtin_nanf("");
        return;
    }
    const int len = pos + 1, d = a.kv_dim, kvs = kvh * HD;
    const float* qkv = a.qkv + static_cast<size_t>(row) * a.ld;
    float* kc = a.kc + row * a.seq_stride + kvs;
    float* vc = a.vc + row * a.seq_stride + kvs;
    const float* knew = qkv + a.k_off + kvs;
    const float* vnew = qkv + a.v_off + kvs;
    // k: lane pair (2 jj, 2 jj + 1) takes position jj, 32 dims each (rows at
    // or past pos from qkv); v: lane (g, c) takes dims 4 c .. 4 c + 3 of
    // positions g + 4 q, from the cache only, clamped below pos (rows at or
    // past pos are replaced by the new row where they are used)
    const int jj = lane >> 1, half = lane & 1, g = lane >> 4, c4 = (lane & 15) * 4, pm1 = max(pos - 1, 0);
    auto load = [&](RowsFrag& f, int jb) __attribute__((always_inline)) {
        if constexpr (QS == 1) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int jk = jb + g + 4 * q;
                f.k[q] = *reinterpret_cast<const float4*>((jk >= pos ? knew : kc + static_cast<size_t>(jk) * d) + c4);
            }
        } else {
            const int jk = jb + jj;
            const float4* kr =
                reinterpret_cast<const float4*>((jk >= pos ? knew : kc + static_cast<size_t>(jk) * d) + half * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) f.k[i] = kr[i];
        }
#pragma unroll
        for (int q = 0; q < 8; q++)
            f.v[q] = *reinterpret_cast<const float4*>(vc + static_cast<size_t>(min(jb + g + 4 * q, pm1)) * d + c4);
    };
    RowsFrag cur;
    int jb = w * kRowsPos;
    if (jb < len) load(cur, jb);
    const float4 vn = *reinterpret_cast<const float4*>(vnew + c4);
    for (int i = tid; i < qn * HD; i += kRowsThreads) qs[i / HD][(i % HD) / 32][i % 32] = qkv[h0 * HD + i];
    if (tid < HD) kn[tid] = knew[tid];
    if constexpr (ROPE) {
        // pair i of query head h (h == qn: the new k row), in LDS
        __syncthreads();
        const int hr = ra.rope_dim / 2;
        for (int t = tid; t < (qn + 1) * hr; t += kRowsThreads) {
            const int h = t / hr, i = t % hr;
            const int ia = ra.neox ? i : 2 * i, ib = ra.neox ? i + hr : 2 * i + 1;
            float* pa = h < qn ? &qs[h][ia / 32][ia % 32] : &kn[ia];
            float* pb = h < qn ? &qs[h][ib / 32][ib % 32] : &kn[ib];
            float x = *pa, y = *pb;
            fh::rope_rotate(x, y, pos, i, ra.rope_dim, ra.base, ra.freq_factors, ra.linear_factor);
            *pa = x;
            *pb = y;
        }
        __syncthreads();
    }
    // the loads take row pos's k from qkv: with ROPE the rotated row instead
    auto rotated_new_k = [&]() __attribute__((always_inline)) {
        if constexpr (ROPE && QS == 1) {
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (jb + g + 4 * q == pos) cur.k[q] = *reinterpret_cast<const float4*>(&kn[c4]);
        } else if (ROPE && jb + jj == pos) {
            const float4* k4 = reinterpret_cast<const float4*>(&kn[half * 32]);
#pragma unroll
            for (int i = 0; i < 8; i++) cur.k[i] = k4[i];
        }
    };
    rotated_new_k();
    if (hs == 0 && tid < HD) {
        kc[static_cast<size_t>(pos) * d + tid] = kn[tid];
        vc[static_cast<size_t>(pos) * d + tid] = vnew[tid];
    }
    float m[QS], l[QS];
    float4 o[QS];
#pragma unroll
    for (int h = 0; h < QS; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
        o[h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    while (jb < len) {  // (wave-uniform)
      if constexpr (QS == 1) {
        // rows at or past pos: the new v row
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (jb + g + 4 * q >= pos) cur.v[q] = vn;
        asm volatile("" ::: "memory");  // (q from LDS each round)
        const float4 q4 = *reinterpret_cast<const float4*>(&qs[0][c4 >> 5][c4 & 31]);
        float sq[8];
        float mr = -INFINITY;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            float p = q4.x * cur.k[q].x;
            p = fmaf(q4.y, cur.k[q].y, p);
            p = fmaf(q4.z, cur.k[q].z, p);
            p = fmaf(q4.w, cur.k[q].w, p);
            p = fh::group_sum<16>(p);  // every lane of row g: position jb + g + 4 q's score
            sq[q] = jb + g + 4 * q < len ? p * a.scale : -INFINITY;
            mr = fmaxf(mr, sq[q]);
        }
        const float wmx =
            fmaxf(fmaxf(fh::rdlane(mr, 0), fh::rdlane(mr, 16)), fmaxf(fh::rdlane(mr, 32), fh::rdlane(mr, 48)));
        const float mn = fmaxf(m[0], wmx);    // finite: position jb is in range
        const float alpha = expf(m[0] - mn);  // 0 on the wave's first round
        float4 acc = o[0];
        acc.x *= alpha;
        acc.y *= alpha;
        acc.z *= alpha;
        acc.w *= alpha;
        float es = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float e = jb + g + 4 * q < len ? expf(sq[q] - mn) : 0.0f;
            es += e;
            acc.x = fmaf(e, cur.v[q].x, acc.x);
            acc.y = fmaf(e, cur.v[q].y, acc.y);
            acc.z = fmaf(e, cur.v[q].z, acc.z);
            acc.w = fmaf(e, cur.v[q].w, acc.w);
        }
        o[0] = acc;
        l[0] = l[0] * alpha + ((lane & 15) == 0 ? es : 0.0f);  // one lane per row counts its positions
        m[0] = mn;
      } else {
        // (q is read from LDS each round: held in registers across rounds it
        // would take 32 per query head)
        asm volatile("" ::: "memory");
        const bool valid = jb + jj < len;
        float s[QS];
#pragma unroll
        for (int h = 0; h < QS; h++) {
            if (h >= qn) break;  // (wave-uniform)
            asm volatile("" ::: "memory");  // (one head's q in registers at a time)
            const float4* q4 = reinterpret_cast<const float4*>(&qs[h][half][0]);
            float p = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 q = q4[i];
                p = fmaf(q.x, cur.k[i].x, p);
                p = fmaf(q.y, cur.k[i].y, p);
                p = fmaf(q.z, cur.k[i].z, p);
                p = fmaf(q.w, cur.k[i].w, p);
            }
            p = fh::group_sum<2>(p);  // the lane pair's two halves
            s[h] = valid ? p * a.scale : -INFINITY;
        }
#pragma unroll
        for (int h = 0; h < QS; h++) {
            if (h >= qn) break;
            const float mn = fmaxf(m[h], wave_max(s[h]));  // finite: position jb is in range
            const float alpha = expf(m[h] - mn);           // 0 on the wave's first round
            const float e = valid ? expf(s[h] - mn) : 0.0f;
            l[h] = l[h] * alpha + (half == 0 ? e : 0.0f);
            o[h].x *= alpha;
            o[h].y *= alpha;
            o[h].z *= alpha;
            o[h].w *= alpha;
            m[h] = mn;
            if (half == 0) ps[w][h][(jj & 3) * 8 + (jj >> 2)] = e;
        }
        // rows at or past pos: the new v row
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (jb + g + 4 * q >= pos) cur.v[q] = vn;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < QS; h++) {
            if (h >= qn) break;
            const float4* p4 = reinterpret_cast<const float4*>(&ps[w][h][g * 8]);
            const float4 pa = p4[0], pb = p4[1];
            const float pq[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
            float4 acc = o[h];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                acc.x = fmaf(pq[q], cur.v[q].x, acc.x);
                acc.y = fmaf(pq[q], cur.v[q].y, acc.y);
                acc.z = fmaf(pq[q], cur.v[q].z, acc.z);
                acc.w = fmaf(pq[q], cur.v[q].w, acc.w);
            }
            o[h] = acc;
        }
        __builtin_amdgcn_wave_barrier();
      }
        jb += R;
        if (jb < len) {
            load(cur, jb);
            rotated_new_k();
        }
    }
#pragma unroll
    for (int h = 0; h < QS; h++) {
        if (h >= qn) break;
        const float lt = fh::group_total<64>(l[h]);
        if (lane == 0) {
            wm[w][h] = m[h];
            wl[w][h] = lt;
        }
        *reinterpret_cast<float4*>(&wo[w][h][g][c4]) = o[h];
    }
    __syncthreads();
    for (int i = tid; i < qn * HD; i += kRowsThreads) {
        const int h = i / HD, dd = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < kRowsWaves; v++) M = fmaxf(M, wm[v][h]);
        float S = 0.0f, O = 0.0f;
#pragma unroll
        for (int v = 0; v < kRowsWaves; v++) {
            const float f = expf(wm[v][h] - M);  // 0 for a wave with no positions
            S = fmaf(wl[v][h], f, S);
            const float ov = (wo[v][h][0][dd] + wo[v][h][1][dd]) + (wo[v][h][2][dd] + wo[v][h][3][dd]);
            O = fmaf(ov, f, O);
        }
        out[i] = O / S;
    }
}

// x += y, then LayerNorm of the sum into ln (the residual add of
// forward_with_cache followed by the next LayerNorm), one workgroup per row.
// v = x (+ y); s (nullable, may alias x) receives v; ln = LayerNorm(v).
template <bool kAdd>
__global__ void __launch_bounds__(kThreads) k_add_layernorm(const float* x, const float* __restrict__ y, float* s_out,
                                                           int d, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, float* __restrict__ ln) {
    __shared__ float red[kThreads / 64];
    const float* xr = x + static_cast<size_t>(blockIdx.x) * d;
    const float* yr = kAdd ? y + static_cast<size_t>(blockIdx.x) * d : nullptr;
    float* sr = s_out ? s_out + static_cast<size_t>(blockIdx.x) * d : nullptr;
    float* lr = ln + static_cast<size_t>(blockIdx.x) * d;
    constexpr int kPer = 8;  // row elements a thread keeps in registers (d <= 2048 here)
    float v[kPer], gm[kPer], bt[kPer];
    // every load is issued before the first reduction
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        v[i] = c < d ? (kAdd ? xr[c] + yr[c] : xr[c]) : 0.0f;
        gm[i] = c < d ? gamma[c] : 0.0f;
        bt[i] = c < d ? beta[c] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        if (c < d) {
            if (sr) sr[c] = v[i];
            s += v[i];
        }
    }
    const float mean = block_sum(s, red) / static_cast<float>(d);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        if (c < d) {
            const float dv = v[i] - mean;
            ss += dv * dv;
        }
    }
    const float var = block_sum(ss, red) / static_cast<float>(d);
    const float sd = sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int c = threadIdx.x + i * kThreads;
        if (c < d) lr[c] = ((v[i] - mean) / sd) * gm[i] + bt[i];
    }
}

unsigned blocks_for(size_t n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

}  // namespace

int fh_launch_embed_rows_pos(fh_ctx* ctx, const float* tok_w, const float* pos_w, size_t vocab, size_t max_seq,
                             size_t d, const uint32_t* tokens, const uint32_t* pos, size_t rows, uint32_t* hist,
                             size_t hist_stride, float* out) {
    hipLaunchKernelGGL(k_embed_rows_pos, dim3(blocks_for(d), static_cast<unsigned>(rows)), dim3(kThreads), 0,
                       ctx->stream, tok_w, pos_w, static_cast<int>(vocab), static_cast<int>(max_seq),
                       static_cast<int>(d), tokens, pos, hist, static_cast<int>(hist_stride), out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_embed_one(fh_ctx* ctx, const float* tok_w, const float* pos_w, size_t vocab, size_t d,
                        const uint32_t* token, size_t pos, float* out) {
    hipLaunchKernelGGL(k_embed_one, dim3(blocks_for(d)), dim3(kThreads), 0, ctx->stream, tok_w, pos_w,
                       static_cast<int>(vocab), static_cast<int>(d), token, static_cast<int>(pos), out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_layernorm(fh_ctx* ctx, const float* x, size_t rows, size_t d, const float* gamma, const float* beta,
                        float* y) {
    // Rows up to 2048 wide stay in registers (same arithmetic, same order).
    if (d <= 8 * static_cast<size_t>(kThreads))
        hipLaunchKernelGGL(k_add_layernorm<false>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, x,
                           nullptr, nullptr, static_cast<int>(d), gamma, beta, y);
    else
        hipLaunchKernelGGL(k_layernorm, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, x,
                           static_cast<int>(d), gamma, beta, y);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_gelu(fh_ctx* ctx, float* x, size_t n) {
    hipLaunchKernelGGL(k_gelu, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, x, n);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_add(fh_ctx* ctx, float* x, const float* y, size_t n) {
    hipLaunchKernelGGL(k_add, dim3(blocks_for(n)), dim3(kThreads), 0, ctx->stream, x, y, n);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

namespace {

// The residual add after a linear, y = r + t (y may be r), and y's row
// statistics for the next norm: per 32-column group its mean and sum of
// squared deviations (one half-wave per group, fixed-order trees; what the
// skinny GEMM's residual epilogue writes).  One workgroup per row; n % 32 == 0
// when stats is set.
__global__ void __launch_bounds__(kThreads) k_residual_stats(const float* __restrict__ t, const float* r, float* y,
                                                            int n, float* __restrict__ stats) {
    const size_t row = blockIdx.x;
    const int groups = (n + 31) >> 5, tid = threadIdx.x;
    for (int g0 = 0; g0 < groups; g0 += kThreads / 32) {
        const int g = g0 + tid / 32, c = g * 32 + (tid & 31);
        const bool live = c < n;
        float v = 0.0f;
        if (live) {
            v = r[row * n + c] + t[row * n + c];
            y[row * n + c] = v;
        }
        if (stats) {
            const float mu = fh::group_total<32>(live ? v : 0.0f) * (1.0f / 32.0f);
            const float dv = live ? v - mu : 0.0f;
            const float m2 = fh::group_total<32>(dv * dv);
            if ((tid & 31) == 0 && g < groups) {
                stats[(row * groups + g) * 2] = mu;
                stats[(row * groups + g) * 2 + 1] = m2;
            }
        }
    }
}

// out = norm(x) from the rows' group statistics (mean = the mean of the group
// means, M2 = sum of M2_g + 32 (mean_g - mean)^2; LayerNorm: (x - mean) * rs *
// gamma + beta, rs = 1 / sqrt(M2 / k + eps); RmsNorm: mean 0, the same sums
// about 0, x * rs * gamma), the skinny GEMM's normalising staging.  One
// workgroup per row.
__global__ void __launch_bounds__(kThreads) k_norm_from_stats(const float* __restrict__ x, int k,
                                                             const float* __restrict__ stats,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps, int rms,
                                                             float* __restrict__ out) {
    const size_t row = blockIdx.x;
    const int groups = k >> 5;
    __shared__ float mr[2];
    if (threadIdx.x == 0) {
        const float* st = stats + row * groups * 2;
        float sm = 0.0f;
        for (int g = 0; g < groups; g++) sm += st[2 * g];
        const float mu = rms ? 0.0f : sm / static_cast<float>(groups);
        float m2 = 0.0f;
        for (int g = 0; g < groups; g++) {
            const float dm = st[2 * g] - mu;
            m2 += st[2 * g + 1] + 32.0f * dm * dm;
        }
        mr[0] = mu;
        mr[1] = 1.0f / sqrtf(m2 / static_cast<float>(k) + eps);
    }
    __syncthreads();
    const float mu = mr[0], rsi = mr[1];
    for (int c = threadIdx.x; c < k; c += kThreads) {
        float v = (x[row * k + c] - mu) * rsi * gamma[c];
        if (beta) v = v + beta[c];
        out[row * k + c] = v;
    }
}

}  // namespace

int fh_launch_residual_stats(fh_ctx* ctx, const float* t, const float* r, float* y, size_t rows, size_t n,
                             float* stats) {
    if (rows == 0) return FH_OK;
    hipLaunchKernelGGL(k_residual_stats, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, t, r, y,
                       static_cast<int>(n), stats);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_norm_from_stats(fh_ctx* ctx, const float* x, size_t rows, size_t k, const fh_edge& e, float* out) {
    if (rows == 0) return FH_OK;
    hipLaunchKernelGGL(k_norm_from_stats, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, x,
                       static_cast<int>(k), e.stats, e.gamma, e.beta, e.eps, e.rms, out);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

int fh_launch_add_layernorm(fh_ctx* ctx, const float* x, const float* y, float* s, size_t rows, size_t d,
                            const float* gamma, const float* beta, float* ln) {
    if (d > 8 * static_cast<size_t>(kThreads))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_add_layernorm: rows wider than 2048");
    if (y)
        hipLaunchKernelGGL(k_add_layernorm<true>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, x,
                           y, s, static_cast<int>(d), gamma, beta, ln);
    else
        hipLaunchKernelGGL(k_add_layernorm<false>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, x,
                           nullptr, s, static_cast<int>(d), gamma, beta, ln);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

namespace {

// Sub-chunks per workgroup, from timings of 12 heads of 64 at positions 63
// to 1023: one workgroup per head while the head fits in 64 positions, then
// 64 positions per workgroup (enough workgroups in flight to cover the load
// latency; one workgroup per head over 256 positions runs about 1.5x
// slower), 128 past position 767.
size_t attn_sub(size_t len) {
    const size_t need = (len + kChunk - 1) / kChunk;
    return need <= 2 ? need : len > 768 ? 4 : 2;
}

// Query heads per k_attn_rows workgroup for a group size: up to four (a
// group of seven takes two workgroups, four heads and three; all seven in one
// workgroup, each kv row read once, ran the 64-row Qwen2-0.5B step 1.949 ms
// against 1.907: the longer head loop costs more than the second read, which
// the cache serves).
int rows_heads(int group) { return group >= 5 ? 4 : group >= 2 ? 2 : 1; }

// k_attn_rows for a launch of `rows` rows (batched decode only): grouped
// query heads of width 64, float4-aligned k and v rows, and enough
// workgroups to fill the part.  Timings at Qwen2-0.5B shapes (14 heads over 2
// kv heads of 64), 64 rows at positions 63 / 127 / 255 / 511 / 1023: 6.1 /
// 7.5 / 10.4 / 15.0 / 25.4 us against 6.7 / 10.6 / 15.9 / 19.3 / 48.9 for the
// chunked kernels; 32 rows at 255 (128 workgroups) 8.7 against 9.9, 16 rows
// (64) 8.3 against 8.0.  Multi-head rows (group 1, one workgroup per row and
// head) ran slower than the chunked kernel: 32 rows of GPT-2 at 255, 15.4
// against 14.6 us.
bool rows_kernel_fits(const AttnArgs& a, size_t rows, size_t heads, size_t hd) {
    const int g = a.group;
    if (hd != 64 || g < 1) return false;
    const size_t parts = (g + rows_heads(g) - 1) / rows_heads(g);
    if (rows * (heads / g) * parts < kRowsMinGroups) return false;
    const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return al(a.qkv) && al(a.kc) && al(a.vc) && a.ld % 4 == 0 && a.k_off % 4 == 0 && a.v_off % 4 == 0 &&
           a.kv_dim % 4 == 0 && a.seq_stride % 4 == 0;
}

// k_attn_rows over `rows` rows (rows_kernel_fits holds), with the rotation
// of q and the new k rows when rope is set.
int launch_rows(fh_ctx* ctx, AttnArgs a, size_t rows, size_t heads, size_t max_len, const RopeArgs* rope) {
    a.scale = 1.0f / sqrtf(64.0f);
    const int qs = rows_heads(a.group), parts = (a.group + qs - 1) / qs;
    const dim3 grid(static_cast<unsigned>(heads / a.group * parts), static_cast<unsigned>(rows)), block(kRowsThreads);
    a.max_len = static_cast<int>(max_len);
    const RopeArgs ra = rope ? *rope : RopeArgs{};
    if (rope) {
        if (qs == 4) hipLaunchKernelGGL((k_attn_rows<4, true>), grid, block, 0, ctx->stream, a, ra);
        else hipLaunchKernelGGL((k_attn_rows<2, true>), grid, block, 0, ctx->stream, a, ra);
    } else {
        if (qs == 4) hipLaunchKernelGGL((k_attn_rows<4, false>), grid, block, 0, ctx->stream, a, ra);
        else if (qs == 2) hipLaunchKernelGGL((k_attn_rows<2, false>), grid, block, 0, ctx->stream, a, ra);
        else hipLaunchKernelGGL((k_attn_rows<1, false>), grid, block, 0, ctx->stream, a, ra);
    }
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

// max_len: the longest row (positions + 1) the launch may see.
int launch_attention(fh_ctx* ctx, AttnArgs a, size_t rows, size_t heads, size_t hd, size_t max_len,
                     bool batched = false) {
    if (hd > static_cast<size_t>(kMaxHd) || hd % 8 != 0 || kThreads % hd != 0)
        return fh_fail(ctx, FH_ERR_LIMIT, "attention: head width must be 8, 16, 32, 64 or 128");
    // One query head per kv head (GPT-2) takes the one-pass kernel from 256
    // positions on: configs[3]'s batch-32 run (GPT-2-medium, 512-575
    // positions) 151.0 -> 145.0 ms, the GPT-2-124M batch-32 step at position
    // 255 0.670 -> 0.648 ms (shorter rows are not measured: the chunked kernel).
    if (batched && (a.group >= 2 || max_len >= 256) && rows_kernel_fits(a, rows, heads, hd))
        return launch_rows(ctx, a, rows, heads, max_len, nullptr);
    a.max_len = static_cast<int>(max_len);
    const size_t sub = attn_sub(max_len);
    const size_t chunks = (max_len + sub * kChunk - 1) / (sub * kChunk);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, rows * heads * chunks * (2 + hd) * sizeof(float), &ws);
    if (rc) return rc;
    void* cnt = nullptr;
    rc = fh_counter_area(ctx, rows * heads * sizeof(unsigned), &cnt);
    if (rc) return rc;
    a.scale = 1.0f / sqrtf(static_cast<float>(hd));
    a.part = static_cast<float*>(ws);
    a.counters = static_cast<unsigned*>(cnt);
    // Query heads per workgroup: all of a kv head's group (or a divisor of it)
    // while their q slices fit the registers (QG * HD / 8 <= 64 floats), for
    // rows of 384 positions or more.  Timings at 64 rows of Qwen2-0.5B (14
    // heads over 2 kv heads of 64): grouped / per head 11.3 / 7.8 us at
    // position 63, 14.8 / 11.0 at 127, 17.0 / 16.8 at 255, 20.1 / 29.0 at
    // 511 -- the per-head launch re-reads each kv head per query head, mostly
    // from L2, and wins while its many small workgroups fill the CUs.
    int qg = 1;
    for (int c : {8, 7, 4, 3, 2})
        if (max_len >= 384 && a.group % c == 0 && c * static_cast<int>(hd) / 8 <= 64 && hd >= 32) {
            qg = c;
            break;
        }
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(heads / qg), static_cast<unsigned>(rows));
    auto go = [&](auto hdc) {
        constexpr int HD = decltype(hdc)::value;
        auto launch = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, ctx->stream, a); };
        auto grouped = [&](auto qgc) {
            constexpr int QG = decltype(qgc)::value;
            if constexpr (QG * HD / 8 <= 64 && HD >= 32) {
                switch (sub) {
                    case 1: launch(k_attn_group<1, HD, QG>); break;
                    case 2: launch(k_attn_group<2, HD, QG>); break;
                    default: launch(k_attn_group<4, HD, QG>); break;
                }
            }
        };
        switch (qg) {
            case 8: grouped(std::integral_constant<int, 8>{}); return;
            case 7: grouped(std::integral_constant<int, 7>{}); return;
            case 4: grouped(std::integral_constant<int, 4>{}); return;
            case 3: grouped(std::integral_constant<int, 3>{}); return;
            case 2: grouped(std::integral_constant<int, 2>{}); return;
            default: break;
        }
        switch (sub) {
            case 1: launch(k_attn_chunk<1, HD>); break;
            case 2: launch(k_attn_chunk<2, HD>); break;
            default: launch(k_attn_chunk<4, HD>); break;
        }
    };
    switch (hd) {
        case 8: go(std::integral_constant<int, 8>{}); break;
        case 16: go(std::integral_constant<int, 16>{}); break;
        case 32: go(std::integral_constant<int, 32>{}); break;
        case 64: go(std::integral_constant<int, 64>{}); break;
        default: go(std::integral_constant<int, 128>{}); break;
    }
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

}  // namespace

int fh_launch_attention_decode(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t d, size_t heads, size_t pos,
                               float* out) {
    AttnArgs a{};
    a.qkv = qkv;
    a.ld = static_cast<int>(3 * d);
    a.k_off = static_cast<int>(d);
    a.v_off = static_cast<int>(2 * d);
    a.kc = kc;
    a.vc = vc;
    a.seq_stride = 0;
    a.kv_dim = static_cast<int>(d);
    a.group = 1;
    a.dpos = nullptr;
    a.pos = static_cast<int>(pos);
    a.cap = 0x7FFFFFFF;  // checked by the caller
    a.out = out;
    a.out_ld = static_cast<int>(d);
    return launch_attention(ctx, a, 1, heads, d / heads, pos + 1);
}

int fh_launch_attention_prefill(fh_ctx* ctx, const float* qkv, float* kc, float* vc, size_t d, size_t heads,
                                size_t pos0, size_t rows, float* out) {
    // Every row's k and v are in the cache before any row reads them; each
    // attention workgroup then writes its own row again (the same bits).
    const unsigned gx = static_cast<unsigned>((d + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(k_kv_store, dim3(gx, static_cast<unsigned>(rows)), dim3(kThreads), 0, ctx->stream, qkv,
                       static_cast<int>(3 * d), static_cast<int>(d), static_cast<int>(2 * d), static_cast<int>(d),
                       static_cast<int>(pos0), kc, vc);
    FH_HIP(ctx, hipGetLastError());
    AttnArgs a{};
    a.qkv = qkv;
    a.ld = static_cast<int>(3 * d);
    a.k_off = static_cast<int>(d);
    a.v_off = static_cast<int>(2 * d);
    a.kc = kc;
    a.vc = vc;
    a.seq_stride = 0;  // one sequence: the rows share the cache
    a.kv_dim = static_cast<int>(d);
    a.group = 1;
    a.dpos = nullptr;
    a.pos = static_cast<int>(pos0);
    a.pos_step = 1;
    a.cap = 0x7FFFFFFF;  // checked by the caller
    a.out = out;
    a.out_ld = static_cast<int>(d);
    return launch_attention(ctx, a, rows, heads, d / heads, pos0 + rows);
}

namespace {

AttnArgs gqa_args(const float* qkv, size_t ld, size_t n_heads, size_t n_kv, size_t hd, float* kc, float* vc,
                  size_t cap, const uint32_t* dpos, float* out) {
    AttnArgs a{};
    a.qkv = qkv;
    a.ld = static_cast<int>(ld);
    a.k_off = static_cast<int>(n_heads * hd);
    a.v_off = static_cast<int>((n_heads + n_kv) * hd);
    a.kc = kc;
    a.vc = vc;
    a.seq_stride = cap * n_kv * hd;
    a.kv_dim = static_cast<int>(n_kv * hd);
    a.group = static_cast<int>(n_heads / n_kv);
    a.dpos = dpos;
    a.pos = 0;
    a.cap = static_cast<int>(cap);
    a.out = out;
    a.out_ld = static_cast<int>(n_heads * hd);
    return a;
}

}  // namespace

int fh_launch_gqa_attention_decode(fh_ctx* ctx, const float* qkv, size_t ld, size_t rows, size_t n_heads, size_t n_kv,
                                   size_t hd, float* kc, float* vc, size_t cap, const uint32_t* dpos, size_t max_pos,
                                   float* out) {
    const AttnArgs a = gqa_args(qkv, ld, n_heads, n_kv, hd, kc, vc, cap, dpos, out);
    return launch_attention(ctx, a, rows, n_heads, hd, (max_pos < cap ? max_pos : cap - 1) + 1, true);
}

int fh_launch_gqa_attention_rope_decode(fh_ctx* ctx, float* qkv, size_t ld, size_t rows, size_t n_heads, size_t n_kv,
                                        size_t hd, float* kc, float* vc, size_t cap, const uint32_t* dpos,
                                        size_t max_pos, size_t rope_dim, float base, int rope_type,
                                        const float* freq_factors, float linear_factor, float* out) {
    const AttnArgs a = gqa_args(qkv, ld, n_heads, n_kv, hd, kc, vc, cap, dpos, out);
    const size_t max_len = (max_pos < cap ? max_pos : cap - 1) + 1;
    if (a.group >= 2 && rows_kernel_fits(a, rows, n_heads, hd)) {
        const RopeArgs ra{static_cast<int>(rope_dim), rope_type == FH_ROPE_NEOX ? 1 : 0, base, linear_factor,
                          freq_factors};
        return launch_rows(ctx, a, rows, n_heads, max_len, &ra);
    }
    const int rc = fh_launch_rope(ctx, qkv, rows, ld, n_heads + n_kv, hd, rope_dim, dpos, base, rope_type,
                                  freq_factors, linear_factor);
    if (rc) return rc;
    return launch_attention(ctx, a, rows, n_heads, hd, max_len, true);
}
