// fh_decode.hip — a GPT-2 decode position's transformer stack in one launch.
//
// What it computes: CachedTransformer::feed for one new token up to the final
// LayerNorm (slm/cached.rs:100-125): Embedding::embed_one (layer/embedding.rs:
// 70-90), then per block forward_with_cache (layer/transformer.rs:221-290):
// LayerNorm, the fused Q|K|V Q8_0 linear, the KV-cache append and attention
// (scale 1/sqrt(head_dim)), the out projection, residual add, LayerNorm, the up
// projection with GELU, the down projection and the second residual add.  The
// final residual stream goes to x_out; the caller's final LayerNorm + head GEMV
// (fh_q8_0_linear_ln_async) and sampler follow.
//
// Why one launch.  At batch 1 every step of that chain is a tiny GEMV (0.6-2.5
// MB) or an attention over a few hundred cached rows; launched one by one, each
// costs a launch floor (~1.6 us in a HIP graph) plus a memory round trip for
// its weights, and the step is ~64 such launches.  Here G workgroups (one per
// CU, all resident together, checked with the occupancy API) walk the whole
// stack; between dependent phases they exchange data, not barriers:
//  * every phase output element is a 64-bit slot (f32 value | 32-bit tag)
//    written with one device-coherent store; a consumer polls the slots it
//    needs until all carry this launch's tag, so one memory round trip both
//    synchronises and delivers the data.  The tag is the launch count + 1:
//    each workgroup keeps its own counter and bumps it as it ends, so slots
//    are never cleared and graph replays stay valid;
//  * each workgroup keeps its own copy of the residual stream in LDS and forms
//    the embedding and every LayerNorm itself (all copies are bit-identical:
//    same data, same order), so the residual never travels;
//  * while it waits for a phase's inputs, a workgroup already holds the next
//    phase's weights: their loads are issued one phase ahead into registers,
//    and an attention item's cached K/V rows are loaded before the Q|K|V
//    phase's outputs arrive;
//  * attention items (head, 64 cached positions) publish (max, sum of
//    exponentials, weighted V sum); the out-projection phase merges them
//    itself, so attention costs one exchange, not two.
// Phases per block: Q|K|V, attention, out projection, up (+GELU), down — five
// exchanges, each ~2 us on this part (the store reaching the coherence point
// plus one polling round trip across XCDs).
//
// Every wait is bounded: after spin_limit polls the workgroup sets
// FH_STATUS_EXCHANGE in the context's status word (fh_sync reports it) and goes
// on; no index depends on exchanged data, so a failed exchange gives wrong
// values, never an out-of-bounds access, and every workgroup ends.
//
// Numerics: products and sums in f32 as the reference, in a parallel order
// (the GEMV rows with FMA and lane trees, LayerNorm sums by a fixed tree), so
// outputs match ferrum_core within the 1e-5 rule, not bit for bit.
#include <string>

#include "fh_internal.hpp"

#pragma clang fp contract(off)

namespace {

typedef unsigned long long u64;
constexpr int kT = 512;             // threads per workgroup: two waves per SIMD hide the GEMV's VALU latency
constexpr int kWaves = kT / 64;
constexpr int kPos = 64;            // cached positions per attention item
constexpr unsigned kSpinLimit = 1u << 16;  // ~0.1 s of polling: far beyond any legitimate wait

__device__ __forceinline__ u64 cload64(const u64* p) {
    return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore64(u64* p, u64 v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 tagged(float v, unsigned tag) {
    return (static_cast<u64>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float untag(u64 x) { return __builtin_bit_cast(float, static_cast<uint32_t>(x)); }

// Loads and stores through the global address space: the pointers come from
// kernel arguments inside structs, and a generic (flat) access would also
// count against the LDS counter, so every LDS wait would wait for the
// prefetched weights as well.
template <class T>
__device__ __forceinline__ T gload(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
__device__ __forceinline__ uint4 gload4(const int8_t* p) {
    typedef unsigned v4 __attribute__((ext_vector_type(4)));
    const v4 v = *(const __attribute__((address_space(1))) v4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <class T>
__device__ __forceinline__ void gstore(T* p, T v) {
    *(__attribute__((address_space(1))) T*)p = v;
}

__device__ __forceinline__ float gelu(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * v * v * v)));
}

}  // namespace

// Per-block weights and state, on the device (one entry per layer).
struct DecBlock {
    const int8_t* q[4];       // Q|K|V, out, up, down quant planes ([n][k] int8)
    const uint16_t* d[4];     // their f16 block-scale planes
    const float* b[4];        // their biases
    const float* ln1_g;
    const float* ln1_b;
    const float* ln2_g;
    const float* ln2_b;
    float* kc;                // [cap][D]
    float* vc;
};

constexpr int kMaxLayers = 24;  // the block table travels in the kernel arguments (4 KB)

struct DecArgs {
    DecBlock blk[kMaxLayers];
    int layers;
    const float* tok_w;       // [vocab][D]
    const float* pos_w;       // [max_seq][D]
    int vocab;
    const uint32_t* token;    // device
    int pos;
    u64* slots;               // per layer: qkv [3D], attn [H][nch_max][HD + 2], proj [D], up [4D], down [D]
    int nch_max;
    unsigned* epoch;          // [grid + prefetch]: launches each workgroup has finished
    unsigned* status;
    unsigned spin_limit;
    int skip_wg;              // testing hook: this workgroup publishes nothing (-1: none)
    float* x_out;             // [D]
};

namespace {

// One phase's GEMV slice: rows [gw * RPW, (gw + 1) * RPW) of an N x K Q8_0
// weight for global wave gw, LPR lanes per row each holding CPL 16-quant chunks
// (lane gl of a row takes chunks gl, gl + LPR, ...), RPP rows per pass.
constexpr int lanes_for(int k16) {
    int l = 1;
    while (l < (k16 + 2) / 3 && l < 64) l <<= 1;
    return l;
}

template <int N, int K, int G>
struct Slice {
    static constexpr int K16 = K / 16;
    static constexpr int LPR = lanes_for(K16);
    static constexpr int CPL = K16 / LPR;
    static constexpr int RPP = 64 / LPR;
    static constexpr int RPW = (N + G * kWaves - 1) / (G * kWaves);
    static constexpr int PASSES = (RPW + RPP - 1) / RPP;
    static_assert(K16 % LPR == 0, "row chunks must split evenly over the row's lanes");
    uint4 q[PASSES][CPL];
    uint32_t d[PASSES][CPL];
    float b[PASSES];

    // Issue every load of the slice (clamped addresses, no predication).
    __device__ __forceinline__ void issue(const int8_t* __restrict__ qs, const uint16_t* __restrict__ dsc,
                                          const float* __restrict__ bias, int gw) {
        // (the lane index is laundered so the address arithmetic is redone at
        // each issue instead of being hoisted out of the layer loop, where its
        // many live offsets would spill)
        int t = static_cast<int>(threadIdx.x);
        asm volatile("" : "+v"(t));
        const int lane = t & 63, gl = lane % LPR, rs = lane / LPR;
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            // 32-bit offsets from the uniform base pointers (N * K < 2^31 here)
            const uint32_t row = static_cast<uint32_t>(min(gw * RPW + p * RPP + rs, N - 1));
#pragma unroll
            for (int c = 0; c < CPL; c++) {
                const uint32_t ci = static_cast<uint32_t>(gl + c * LPR);
                q[p][c] = gload4(qs + (row * K + ci * 16));
                d[p][c] = gload(dsc + (row * (K / 32) + (ci >> 1)));
            }
            b[p] = gload(bias + row);
        }
    }

    // y = act(x . W^T + b) for the slice's rows, x (K floats) in LDS; each
    // row's value goes to its slot, tagged.
    template <bool kGelu>
    __device__ __forceinline__ void compute(const float* x, u64* __restrict__ out, unsigned tag, int gw,
                                            bool publish) const {
        const int lane = threadIdx.x & 63, gl = lane % LPR, rs = lane / LPR;
        // A lane's activation chunks are the same for every row it visits:
        // each is read from LDS once and used for all of the lane's rows.
        float acc[PASSES];
#pragma unroll
        for (int p = 0; p < PASSES; p++) acc[p] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const float4* xs = reinterpret_cast<const float4*>(x + (gl + c * LPR) * 16);
            float4 xr[4];
#pragma unroll
            for (int v = 0; v < 4; v++) xr[v] = xs[v];
#pragma unroll
            for (int p = 0; p < PASSES; p++) {
                const uint32_t wq[4] = {q[p][c].x, q[p][c].y, q[p][c].z, q[p][c].w};
                float sacc = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float4 f = xr[v];
                    sacc = fmaf(f.x, static_cast<float>(static_cast<int8_t>(wq[v] & 0xFFu)), sacc);
                    sacc = fmaf(f.y, static_cast<float>(static_cast<int8_t>((wq[v] >> 8) & 0xFFu)), sacc);
                    sacc = fmaf(f.z, static_cast<float>(static_cast<int8_t>((wq[v] >> 16) & 0xFFu)), sacc);
                    sacc = fmaf(f.w, static_cast<float>(static_cast<int8_t>(wq[v] >> 24)), sacc);
                }
                acc[p] = fmaf(fh_h2f(static_cast<uint16_t>(d[p][c])), sacc, acc[p]);
            }
        }
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int r = p * RPP + rs, row = gw * RPW + r;
            const float tot = fh::group_total<LPR>(acc[p]);
            if (gl == 0 && r < RPW && row < N && publish) {
                float y = tot + b[p];
                if (kGelu) y = gelu(y);
                cstore64(out + row, tagged(y, tag));
            }
        }
    }
};

struct Waits {
    unsigned* status;
    unsigned limit;
};

// Poll `count` slots (tagged `tag`) into dst (LDS), up to PER per thread per
// round with all of a round's loads in flight; whole-workgroup call, ends with
// a barrier.  A round still stale after the poll limit records
// FH_STATUS_EXCHANGE and takes what it has.
template <int PER>
__device__ __forceinline__ void poll_into(const u64* __restrict__ slots, int count, unsigned tag, float* dst,
                                          const Waits& wt) {
    const int tid = threadIdx.x;
    __syncthreads();  // every thread is done reading dst's previous contents
    for (int base = 0; base < count; base += kT * PER) {
        u64 x[PER];
        unsigned spins = 0;
        while (true) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < PER; i++) x[i] = cload64(slots + min(base + tid + i * kT, count - 1));
#pragma unroll
            for (int i = 0; i < PER; i++) ok &= static_cast<unsigned>(x[i] >> 32) == tag;
            if (ok) break;
            if (++spins >= wt.limit) {
                atomicOr(wt.status, static_cast<unsigned>(FH_STATUS_EXCHANGE));
                break;
            }
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int j = base + tid + i * kT;
            if (j < count) dst[j] = untag(x[i]);
        }
    }
    __syncthreads();
}

// Two sums over the workgroup at once (fixed order: wave DPP trees, then the
// waves in order); red holds 2 * kWaves floats.
__device__ __forceinline__ void block_total2(float& a, float& b, float* red) {
    a = fh::group_total<64>(a);
    b = fh::group_total<64>(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = a;
        red[kWaves + (threadIdx.x >> 6)] = b;
    }
    __syncthreads();
    a = 0.0f;
    b = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) {
        a += red[i];
        b += red[kWaves + i];
    }
}

// A LayerNorm's gamma and beta for this thread's columns, loaded ahead.
template <int D>
struct LnParams {
    static constexpr int PER = (D + kT - 1) / kT;
    float g[PER], b[PER];
    __device__ __forceinline__ void issue(const float* gamma, const float* beta) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int cc = min(static_cast<int>(threadIdx.x) + i * kT, D - 1);
            g[i] = gload(gamma + cc);
            b[i] = gload(beta + cc);
        }
    }
};

// LayerNorm::forward (layer/norm.rs:46-82): ((x - mean) / sqrt(var + 1e-5)) *
// gamma + beta with the biased variance, x and y in LDS.  The reference takes
// the mean, then sum (x - mean)^2; here one reduction forms sum (x - c) and
// sum (x - c)^2 about c = x[0] (a value of the row, so within a few standard
// deviations of the mean): var = S2 / D - (S1 / D)^2 loses no more than a
// couple of bits to cancellation, well inside the 1e-5 rule, and costs one
// workgroup exchange instead of two.
template <int D>
__device__ __forceinline__ void layer_norm(const float* x, const LnParams<D>& lp, float* y, float* red) {
    constexpr int PER = LnParams<D>::PER;
    const int tid = threadIdx.x;
    const float c0 = x[0];
    float v[PER];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = tid + i * kT;
        v[i] = x[min(c, D - 1)];
        if (c < D) {
            const float dv = v[i] - c0;
            s1 += dv;
            s2 += dv * dv;
        }
    }
    block_total2(s1, s2, red);
    const float m1 = s1 / static_cast<float>(D);
    const float mean = c0 + m1;
    const float var = fmaxf(s2 / static_cast<float>(D) - m1 * m1, 0.0f);
    const float sd = sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = tid + i * kT;
        if (c < D) y[c] = ((v[i] - mean) / sd) * lp.g[i] + lp.b[i];
    }
    __syncthreads();
}

// The residual update and LayerNorm in one pass: x += delta, y =
// LayerNorm(x), with the same arithmetic as the residual add followed by
// layer_norm.  Every thread reads its columns of x and delta (and column 0,
// for the shift c0) before the reduction's barriers and writes its updated
// columns of x after them, so no thread reads a column another has already
// updated.  y may be delta (every read of it precedes the barriers).
template <int D>
__device__ __forceinline__ void add_layer_norm(float* x, const float* delta, const LnParams<D>& lp, float* y,
                                               float* red) {
    constexpr int PER = LnParams<D>::PER;
    const int tid = threadIdx.x;
    const float c0 = x[0] + delta[0];
    float v[PER];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = tid + i * kT;
        const int cc = min(c, D - 1);
        v[i] = x[cc] + delta[cc];
        if (c < D) {
            const float dv = v[i] - c0;
            s1 += dv;
            s2 += dv * dv;
        }
    }
    block_total2(s1, s2, red);
    const float m1 = s1 / static_cast<float>(D);
    const float mean = c0 + m1;
    const float var = fmaxf(s2 / static_cast<float>(D) - m1 * m1, 0.0f);
    const float sd = sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = tid + i * kT;
        if (c < D) {
            x[c] = v[i];
            y[c] = ((v[i] - mean) / sd) * lp.g[i] + lp.b[i];
        }
    }
    __syncthreads();
}

// Max over the 64 lanes of a wave, every lane getting it: DPP within 16-lane
// rows (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then
// the four rows by readlane.
__device__ __forceinline__ float group_max64(float v) {
    v = fmaxf(v, fh::dpp<0xB1>(v));
    v = fmaxf(v, fh::dpp<0x4E>(v));
    v = fmaxf(v, fh::dpp<0x141>(v));
    v = fmaxf(v, fh::dpp<0x140>(v));
    return fmaxf(fmaxf(fh::rdlane(v, 0), fh::rdlane(v, 16)), fmaxf(fh::rdlane(v, 32), fh::rdlane(v, 48)));
}

// One attention item: head h, cached positions [j0, j0 + kPos) of 0 .. pos.
// Thread t scores position t / TPP over HD / TPP dims of the head and holds,
// for the V sum, dim t % HD of positions t / HD, t / HD + kT / HD, ...
template <int D, int HD>
struct AttnItem {
    static constexpr int TPP = kT / kPos;      // threads per scored position
    static constexpr int QD = HD / TPP;        // dims per thread of a score
    static constexpr int VG = kT / HD;         // thread groups over positions for V
    static constexpr int VP = kPos / VG;       // V positions per thread
    float kr[QD], vr[VP];

    // Cached rows (positions < pos) of this item; rows at or past pos are
    // taken from the Q|K|V outputs later (clamped loads here, unused).
    __device__ __forceinline__ void issue(const float* __restrict__ kc, const float* __restrict__ vc, int h, int j0,
                                          int pos) {
        int tid = static_cast<int>(threadIdx.x);
        asm volatile("" : "+v"(tid));
        const int jl = j0 + tid / TPP, qt = tid % TPP;
        const uint32_t jk = static_cast<uint32_t>(min(jl, max(pos - 1, 0)));  // (cap * D < 2^31 here)
#pragma unroll
        for (int i = 0; i < QD; i++) kr[i] = gload(kc + (jk * D + h * HD + qt * QD + i));
        const int dv = tid % HD, g = tid / HD;
#pragma unroll
        for (int i = 0; i < VP; i++) {
            const uint32_t jv = static_cast<uint32_t>(min(j0 + g + i * VG, max(pos - 1, 0)));
            vr[i] = gload(vc + (jv * D + h * HD + dv));
        }
    }

    // qkv: this head's [q | k_new | v_new] (3 HD floats, LDS); writes (max,
    // sum of exp, weighted V sum) of the item to `out` (HD + 2 slots).  sc:
    // kPos scores; esc: kWaves x kPos (each wave's own copy of the weights);
    // acc: kT floats.  Two barriers: the scores, then the V partial sums.
    __device__ __forceinline__ void compute(const float* qkv, int j0, int pos, float scale, float* sc, float* esc,
                                            float* acc, u64* __restrict__ out, unsigned tag, bool publish) {
        const int tid = threadIdx.x, lane = tid & 63, len = pos + 1, jn = min(kPos, len - j0);
        const int jl = tid / TPP, qt = tid % TPP;
        const bool fresh = j0 + jl >= pos;  // position pos (or past it, masked): the new k row
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < QD; i++) dot += qkv[qt * QD + i] * (fresh ? qkv[HD + qt * QD + i] : kr[i]);
        dot = fh::group_sum<TPP>(dot);
        if (qt == 0) sc[jl] = jl < jn ? dot * scale : -INFINITY;
        __syncthreads();
        // every wave forms the chunk's max and exponentials itself (no
        // barrier between the softmax and the V sum); kPos == 64: lane j
        // holds position j
        const float s = sc[lane];
        const float mx = group_max64(s);
        const float e = lane < jn ? expf(s - mx) : 0.0f;
        const float se = fh::group_total<64>(e);
        float* ew = esc + (tid >> 6) * kPos;
        ew[lane] = e;
        __builtin_amdgcn_wave_barrier();
        const int dv = tid % HD, g = tid / HD;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < VP; i++) {
            const int jc = g + i * VG;
            const float v = j0 + jc >= pos ? qkv[2 * HD + dv] : vr[i];
            if (jc < jn) o += ew[jc] * v;
        }
        acc[tid] = o;
        __syncthreads();
        if (tid < HD && publish) {
            float r = 0.0f;
#pragma unroll
            for (int gg = 0; gg < VG; gg++) r += acc[gg * HD + tid];
            cstore64(out + 2 + tid, tagged(r, tag));
        }
        if (tid == 0 && publish) {
            cstore64(out, tagged(mx, tag));
            cstore64(out + 1, tagged(se, tag));
        }
        // (no trailing barrier: every later write to sc, esc, acc or the
        // q|k|v buffer comes after at least one more barrier)
    }
};

// Past the stack's own workgroups, up to kPrefetchWGs more read each next
// block's weights (quant and scale planes) and cached K/V rows once the
// current block's Q|K|V outputs are out, so that the stack's own loads of that
// block, issued a phase ahead of their use, find them in the memory-side
// cache instead of HBM.  They only read and never publish; a wait that runs
// out ends their work silently (the stack's own waits report).  Measured,
// HBM-forced GPT-2-124M step at position 255: 229.7 -> 217.4 us with 24; 8
// lag behind and slow the stack (240 us), 16-32 time alike, 64-128 a little
// slower; warming the head as well, or two blocks ahead, did not pay.
constexpr int kPrefetchWGs = 24;
constexpr size_t kPrefetchKvMax = 8u << 20;  // a block's cached K/V bytes still worth warming

template <int D, int HD>
__device__ void prefetch_blocks(const DecArgs& a, int p, int np, size_t stride, unsigned tag) {
    constexpr int F = 4 * D;
    const int tid = threadIdx.x;
    uint32_t sink = 0;
    // this workgroup's share of the 128-byte lines of [base, base + bytes):
    // one word per line brings the whole line in, eight lines in flight per
    // thread (the words are folded into `sink`, kept by an asm).  (Reading
    // every byte warmed as well but cost more where the weights were already
    // cached: 1.3 % of a MALL-resident step against 0.5 %.)
    auto touch = [&](const void* base, size_t bytes) __attribute__((always_inline)) {
        const uint32_t* b1 = static_cast<const uint32_t*>(base);
        const size_t nl = bytes >> 7, step = static_cast<size_t>(np) * kT;
        for (size_t i0 = static_cast<size_t>(p) * kT + tid; i0 < nl; i0 += 8 * step) {
            uint32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = b1[min(i0 + j * step, nl - 1) << 5];
#pragma unroll
            for (int j = 0; j < 8; j++) sink ^= v[j];
        }
    };
    auto touch_block = [&](const DecBlock& B) __attribute__((always_inline)) {
        const size_t n[4] = {3 * D, D, F, D}, k[4] = {D, D, D, F};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            touch(B.q[i], n[i] * k[i]);
            touch(B.d[i], n[i] * (k[i] / 32) * sizeof(uint16_t));
        }
        const size_t kv = static_cast<size_t>(a.pos) * D * sizeof(float);
        if (kv > 0 && 2 * kv <= kPrefetchKvMax) {
            touch(B.kc, kv);
            touch(B.vc, kv);
        }
    };
    __shared__ int go;
    if (a.layers > 1) touch_block(a.blk[1]);
    for (int l = 1; l + 1 < a.layers; l++) {
        // block l's first Q|K|V output (row 0, workgroup 0) carries this launch's tag
        if (tid == 0) {
            const u64* s0 = a.slots + l * stride;
            unsigned spins = 0;
            int ok = 1;
            while (static_cast<unsigned>(cload64(s0) >> 32) != tag) {
                __builtin_amdgcn_s_sleep(2);
                if (++spins >= a.spin_limit) {
                    ok = 0;
                    break;
                }
            }
            go = ok;
        }
        __syncthreads();
        if (!go) break;
        touch_block(a.blk[l + 1]);
        __syncthreads();  // (go is written again next round)
    }
    asm volatile("" ::"v"(sink));
}

template <int D, int HD, int G>
__global__ void __launch_bounds__(kT) k_gpt2_stack(DecArgs a) {
    constexpr int H = D / HD, F = 4 * D;
    constexpr int kAttnSlots = HD + 2;
    using SQkv = Slice<3 * D, D, G>;
    using SOut = Slice<D, D, G>;
    using SUp = Slice<F, D, G>;
    using SDown = Slice<D, F, G>;
    __shared__ __align__(16) float xres[D];  // the residual stream (every workgroup's own copy)
    __shared__ __align__(16) float hbuf[F];  // LayerNorm output / merged attention / up outputs
    __shared__ __align__(16) float hq[3 * HD];
    __shared__ float sc[kPos], esc[kWaves * kPos], acc[kT], red[2 * kWaves];
    static_assert(kPos == 64, "the softmax maps lane j to position j");
    extern __shared__ __align__(16) float part[];  // polled attention partials [H][nch][HD + 2]

    const int tid = threadIdx.x, w = blockIdx.x, gw = w * kWaves + (tid >> 6);
    if (w >= G) {  // a prefetch workgroup (its own epoch counter, like every workgroup)
        const unsigned ptag = a.epoch[w] + 1;
        prefetch_blocks<D, HD>(a, w - G, static_cast<int>(gridDim.x) - G,
                               static_cast<size_t>(3 * D + H * a.nch_max * kAttnSlots + D + F + D), ptag);
        __syncthreads();
        if (tid == 0) a.epoch[w] = ptag;
        return;
    }
    const int pos = a.pos, len = pos + 1, nch = (len + kPos - 1) / kPos, items = H * nch;
    // Each workgroup keeps its own epoch counter and bumps it when it ends,
    // so all counters advance together, one per launch, with no workgroup
    // waiting on another to finish.
    const unsigned tag = a.epoch[w] + 1;
    const Waits wt{a.status, a.spin_limit};
    const size_t stride = static_cast<size_t>(3 * D + H * a.nch_max * kAttnSlots + D + F + D);
    const float scale = 1.0f / sqrtf(static_cast<float>(HD));
    const bool pub = w != a.skip_wg;

    SQkv wqkv;
    SOut wout;
    SUp wup;
    SDown wdown;
    LnParams<D> ln1, ln2;
    wqkv.issue(a.blk[0].q[0], a.blk[0].d[0], a.blk[0].b[0], gw);
    ln1.issue(a.blk[0].ln1_g, a.blk[0].ln1_b);

    // Embedding::embed_one: an id past the vocabulary poisons the row.
    {
        const uint32_t t = *a.token;
        for (int c = tid; c < D; c += kT)
            xres[c] = t < static_cast<uint32_t>(a.vocab)
                          ? gload(a.tok_w + static_cast<size_t>(t) * D + c) + gload(a.pos_w + static_cast<size_t>(pos) * D + c)
                          : __builtin_nanf("");
    }
    __syncthreads();

    for (int l = 0; l < a.layers; l++) {
        const DecBlock& B = a.blk[l];
        u64* s_qkv = a.slots + l * stride;
        u64* s_att = s_qkv + 3 * D;
        u64* s_proj = s_att + H * a.nch_max * kAttnSlots;
        u64* s_up = s_proj + D;
        u64* s_down = s_up + F;

        // ---- Q|K|V: residual += previous block's down projection, LayerNorm 1.
        // This workgroup's first attention item's cached K/V rows are loaded
        // first: they do not depend on this step.
        AttnItem<D, HD> ai0;
        if (w < items) ai0.issue(B.kc, B.vc, w / nch, (w % nch) * kPos, pos);
        if (l > 0) {
            poll_into<(D + kT - 1) / kT>(a.slots + (l - 1) * stride + 3 * D + H * a.nch_max * kAttnSlots + D + F, D,
                                         tag, hbuf, wt);
            add_layer_norm<D>(xres, hbuf, ln1, hbuf, red);
        } else {
            layer_norm<D>(xres, ln1, hbuf, red);
        }
        wqkv.template compute<false>(hbuf, s_qkv, tag, gw, pub);

        // ---- attention items; the out projection's weights are issued first
        wout.issue(B.q[1], B.d[1], B.b[1], gw);
        for (int it = w; it < items; it += G) {
            const int h = it / nch, c = it % nch, j0 = c * kPos;
            AttnItem<D, HD> ai = ai0;
            if (it != w) ai.issue(B.kc, B.vc, h, j0, pos);
            // this head's q, k_new, v_new
            {
                const int i = tid, part_i = i / HD, dd = i % HD;
                const u64* src = s_qkv + part_i * D + h * HD + dd;
                if (i < 3 * HD) {
                    unsigned spins = 0;
                    u64 x;
                    while (static_cast<unsigned>((x = cload64(src)) >> 32) != tag) {
                        if (++spins >= wt.limit) {
                            atomicOr(wt.status, static_cast<unsigned>(FH_STATUS_EXCHANGE));
                            break;
                        }
                    }
                    hq[i] = untag(x);
                }
                __syncthreads();
            }
            // the new row joins the cache (read by later positions only)
            if (c == pos / kPos && tid < HD) {
                gstore(B.kc + static_cast<size_t>(pos) * D + h * HD + tid, hq[HD + tid]);
                gstore(B.vc + static_cast<size_t>(pos) * D + h * HD + tid, hq[2 * HD + tid]);
            }
            ai.compute(hq, j0, pos, scale, sc, esc, acc, s_att + static_cast<size_t>(it) * kAttnSlots, tag, pub);
        }

        // ---- out projection: merge every item (head by head), then the GEMV
        wup.issue(B.q[2], B.d[2], B.b[2], gw);
        ln2.issue(B.ln2_g, B.ln2_b);
        poll_into<8>(s_att, items * kAttnSlots, tag, part, wt);  // item (h, c) at (h * nch + c) * (HD + 2)
        // att[h, d] = (sum_c acc_c[d] e_c) / S_h, e_c = exp(m_c - M_h), S_h =
        // sum_c l_c e_c (M_h the head's largest chunk max).  Each output's
        // thread forms its head's M, e and S itself, four chunks' values
        // loaded at a time, so the merge costs one barrier and a few LDS
        // round trips.
        for (int o = tid; o < D; o += kT) {
            const int h = o / HD, dd = o % HD;
            const float* hp = part + h * nch * kAttnSlots;
            float M = -INFINITY;
            for (int c0 = 0; c0 < nch; c0 += 4) {
                float mv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) mv[i] = hp[min(c0 + i, nch - 1) * kAttnSlots];  // (repeats: same max)
#pragma unroll
                for (int i = 0; i < 4; i++) M = fmaxf(M, mv[i]);
            }
            float S = 0.0f, r = 0.0f;
            for (int c0 = 0; c0 < nch; c0 += 4) {
                float mv[4], lv[4], av[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float* cp = hp + min(c0 + i, nch - 1) * kAttnSlots;
                    mv[i] = cp[0];
                    lv[i] = cp[1];
                    av[i] = cp[2 + dd];
                }
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (c0 + i < nch) {
                        const float e = expf(mv[i] - M);
                        S += lv[i] * e;
                        r += av[i] * e;
                    }
            }
            hbuf[o] = r / S;
        }
        __syncthreads();
        wout.template compute<false>(hbuf, s_proj, tag, gw, pub);

        // ---- up (+GELU): residual += attention output, LayerNorm 2
        wdown.issue(B.q[3], B.d[3], B.b[3], gw);
        poll_into<(D + kT - 1) / kT>(s_proj, D, tag, hbuf, wt);
        add_layer_norm<D>(xres, hbuf, ln2, hbuf, red);
        wup.template compute<true>(hbuf, s_up, tag, gw, pub);

        // ---- down; the next block's Q|K|V weights are issued first
        if (l + 1 < a.layers) {
            const DecBlock& N = a.blk[l + 1];
            wqkv.issue(N.q[0], N.d[0], N.b[0], gw);
            ln1.issue(N.ln1_g, N.ln1_b);
        }
        poll_into<(F + kT - 1) / kT>(s_up, F, tag, hbuf, wt);
        wdown.template compute<false>(hbuf, s_down, tag, gw, pub);
    }

    // the last block's down projection closes the residual stream
    poll_into<(D + kT - 1) / kT>(a.slots + (a.layers - 1) * stride + 3 * D + H * a.nch_max * kAttnSlots + D + F, D,
                                 tag, hbuf, wt);
    if (w == 0)
        for (int c = tid; c < D; c += kT) gstore(a.x_out + c, xres[c] + hbuf[c]);
    __syncthreads();
    if (tid == 0) a.epoch[w] = tag;
}

}  // namespace

// ---- host side ---------------------------------------------------------------------

struct fh_gpt2_stack {
    int device = 0;
    size_t layers = 0, d = 0, heads = 0, cap = 0, vocab = 0, max_seq = 0;
    int nch_max = 0;
    const float* tok_w = nullptr;
    const float* pos_w = nullptr;
    DecBlock blocks[kMaxLayers] = {};  // the block table (it travels in the kernel arguments)
    u64* slots = nullptr;
    unsigned* epoch = nullptr;
    void* base = nullptr;        // one allocation: epoch counters, slots
    int grid = 0;                // the stack's own workgroups
    int prefetch = 0;            // prefetch workgroups launched beside them
    size_t dyn_lds = 0;
    const void* kernel = nullptr;
};

namespace {

// The workgroups one launch uses, all resident at once (one per CU): fewer
// workgroups make each exchange cheaper (fewer pollers), more make each
// phase's GEMV slice smaller.  At d = 768, 48 give every wave whole passes of
// rows (Q|K|V 6 rows, up 8, out and down 2: no more VALU work per lane than
// 64) and one attention item per workgroup at position 255 (12 heads x 4
// items); measured 194 us per position against 204 us with 64 and 294 us with
// 32.  At d = 1024, 48 would add a Q|K|V pass per wave: 64.
constexpr int grid_for(int d) { return d == 768 ? 48 : 64; }

template <int D, int HD>
const void* stack_kernel() {
    return reinterpret_cast<const void*>(k_gpt2_stack<D, HD, grid_for(D)>);
}

}  // namespace

extern "C" {

int fh_gpt2_stack_create(fh_ctx* ctx, const fh_gpt2_block* blocks, size_t layers, size_t d, size_t heads,
                         size_t ffn, size_t capacity, const float* d_tok_w, const float* d_pos_w, size_t vocab,
                         size_t max_seq, fh_gpt2_stack** out) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!out) return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_create: out is NULL");
    *out = nullptr;
    if (!blocks || layers == 0 || !d_tok_w || !d_pos_w)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_create: blocks, token or position table missing");
    if (heads == 0 || d % heads != 0)
        return fh_fail(ctx, FH_ERR_DIM, "fh_gpt2_stack_create: heads (" + std::to_string(heads) +
                                            ") must divide the embedding dim (" + std::to_string(d) + ")");
    const size_t hd = d / heads;
    const void* kern = nullptr;
    if (d == 768 && hd == 64) kern = stack_kernel<768, 64>();
    else if (d == 1024 && hd == 64) kern = stack_kernel<1024, 64>();
    else if (d == 128 && hd == 32) kern = stack_kernel<128, 32>();
    if (!kern || ffn != 4 * d)
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_gpt2_stack_create: shapes d = 768 / 1024 with head width 64, or d = 128 "
                                          "with head width 32, and ffn = 4 d only");
    if (capacity == 0 || capacity > 4096 || vocab == 0 || vocab > 0x7FFFFFFFu || max_seq == 0 ||
        max_seq > 0x7FFFFFFFu || layers > static_cast<size_t>(kMaxLayers))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_gpt2_stack_create: capacity 1 .. 4096, at most 24 blocks, vocab and "
                                          "max_seq below 2^31");
    const size_t shapes[4][2] = {{3 * d, d}, {d, d}, {ffn, d}, {d, ffn}};
    for (size_t l = 0; l < layers; l++) {
        const fh_gpt2_block& b = blocks[l];
        const fh_q8_0* ws[4] = {b.qkv, b.out, b.up, b.down};
        const float* bs[4] = {b.qkv_b, b.out_b, b.up_b, b.down_b};
        for (int i = 0; i < 4; i++) {
            if (!ws[i] || !bs[i])
                return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_create: block " + std::to_string(l) +
                                                        " lacks a weight or a bias");
            if (ws[i]->n != shapes[i][0] || ws[i]->k != shapes[i][1])
                return fh_fail(ctx, FH_ERR_DIM, "fh_gpt2_stack_create: block " + std::to_string(l) + " weight " +
                                                    std::to_string(i) + " is " + std::to_string(ws[i]->n) + " x " +
                                                    std::to_string(ws[i]->k) + ", expected " +
                                                    std::to_string(shapes[i][0]) + " x " + std::to_string(shapes[i][1]));
            if (ws[i]->device != ctx->device)
                return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_create: a weight lives on another device");
            if (ws[i]->kind != FH_WEIGHT_Q8_0)
                return fh_fail(ctx, FH_ERR_LIMIT, "fh_gpt2_stack_create: F32 weights run one op at a time");
        }
        if (!b.ln1_g || !b.ln1_b || !b.ln2_g || !b.ln2_b || !b.k_cache || !b.v_cache)
            return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_create: block " + std::to_string(l) +
                                                    " lacks a LayerNorm parameter or a cache");
    }
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) FH_HIP(ctx, hipSetDevice(ctx->device));
    const int nch = static_cast<int>((capacity + kPos - 1) / kPos);
    const size_t dyn = static_cast<size_t>(heads) * nch * (hd + 2) * sizeof(float);
    const int grid = grid_for(static_cast<int>(d));
    int per_cu = 0;
    FH_HIP(ctx, hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kT, dyn));
    const size_t resident = static_cast<size_t>(per_cu < 0 ? 0 : per_cu) * ctx->num_cus;
    if (per_cu < 1 || resident < static_cast<size_t>(grid))
        return fh_fail(ctx, FH_ERR_LIMIT, "fh_gpt2_stack_create: the device cannot hold the stack kernel's " +
                                              std::to_string(grid) + " workgroups at once");
    // prefetch workgroups only where the device holds them beside the stack's
    // (launched after them, so the stack's are never displaced)
    const int prefetch = static_cast<int>(resident - grid < static_cast<size_t>(kPrefetchWGs) ? resident - grid
                                                                                           : kPrefetchWGs);
    const size_t stride = 3 * d + heads * nch * (hd + 2) + d + ffn + d;
    const size_t ebytes = fh_align256((grid + prefetch) * sizeof(unsigned));
    const size_t sbytes = layers * stride * sizeof(u64);
    fh_gpt2_stack* s = new (std::nothrow) fh_gpt2_stack();
    if (!s) return fh_fail(ctx, FH_ERR_OOM, "fh_gpt2_stack_create: out of host memory");
    hipError_t e = hipMalloc(&s->base, ebytes + sbytes);
    if (e != hipSuccess) {
        delete s;
        return fh_hip_fail(ctx, e, "hipMalloc(stack state)");
    }
    s->epoch = static_cast<unsigned*>(s->base);
    s->slots = reinterpret_cast<u64*>(static_cast<char*>(s->base) + ebytes);
    DecBlock* host = s->blocks;
    for (size_t l = 0; l < layers; l++) {
        const fh_gpt2_block& b = blocks[l];
        const fh_q8_0* ws[4] = {b.qkv, b.out, b.up, b.down};
        const float* bs[4] = {b.qkv_b, b.out_b, b.up_b, b.down_b};
        for (int i = 0; i < 4; i++) {
            host[l].q[i] = ws[i]->qs;
            host[l].d[i] = ws[i]->d;
            host[l].b[i] = bs[i];
        }
        host[l].ln1_g = b.ln1_g;
        host[l].ln1_b = b.ln1_b;
        host[l].ln2_g = b.ln2_g;
        host[l].ln2_b = b.ln2_b;
        host[l].kc = b.k_cache;
        host[l].vc = b.v_cache;
    }
    e = hipMemsetAsync(s->epoch, 0, ebytes + sbytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(s->base);
        delete s;
        return fh_hip_fail(ctx, e, "fh_gpt2_stack_create (state upload)");
    }
    s->device = ctx->device;
    s->layers = layers;
    s->d = d;
    s->heads = heads;
    s->cap = capacity;
    s->vocab = vocab;
    s->max_seq = max_seq;
    s->nch_max = nch;
    s->tok_w = d_tok_w;
    s->pos_w = d_pos_w;
    s->grid = grid;
    s->prefetch = prefetch;
    s->dyn_lds = dyn;
    s->kernel = kern;
    *out = s;
    return FH_OK;
}

void fh_gpt2_stack_free(fh_gpt2_stack* s) {
    if (!s) return;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != s->device) (void)hipSetDevice(s->device);
    if (s->base) (void)hipFree(s->base);
    delete s;
}

int fh_gpt2_stack_forward_async(fh_ctx* ctx, fh_gpt2_stack* s, const uint32_t* d_token, size_t pos, float* d_x) {
    if (!ctx) return FH_ERR_INVALID;
    ctx->err.clear();
    if (!s || !d_token || !d_x) return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_forward: a pointer is NULL");
    if (s->device != ctx->device)
        return fh_fail(ctx, FH_ERR_INVALID, "fh_gpt2_stack_forward: the stack lives on another device");
    if (pos >= s->max_seq)
        return fh_fail(ctx, FH_ERR_DIM, "Position " + std::to_string(pos) + " exceeds max_seq_len " +
                                            std::to_string(s->max_seq));
    if (pos >= s->cap)
        return fh_fail(ctx, FH_ERR_DIM, "KvCache full (" + std::to_string(s->cap) +
                                            " positions): clear and re-prime to continue");
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) FH_HIP(ctx, hipSetDevice(ctx->device));
    DecArgs a;
    static_assert(sizeof(DecArgs) <= 4096, "kernel arguments are limited to 4 KB");
    for (size_t l = 0; l < s->layers; l++) a.blk[l] = s->blocks[l];
    a.layers = static_cast<int>(s->layers);
    a.tok_w = s->tok_w;
    a.pos_w = s->pos_w;
    a.vocab = static_cast<int>(s->vocab);
    a.token = d_token;
    a.pos = static_cast<int>(pos);
    a.slots = s->slots;
    a.nch_max = s->nch_max;
    a.epoch = s->epoch;
    a.status = ctx->status;
    a.spin_limit = ctx->test_spin_limit ? ctx->test_spin_limit : kSpinLimit;
    a.skip_wg = ctx->test_skip_segment;
    a.x_out = d_x;
    void* args[] = {&a};
    FH_HIP(ctx, hipLaunchKernel(s->kernel, dim3(static_cast<unsigned>(s->grid + s->prefetch)), dim3(kT), args, s->dyn_lds,
                                ctx->stream));
    return FH_OK;
}

}  // extern "C"
