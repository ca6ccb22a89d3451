// fh_sampler.hip — the fused logit sampler on gfx950: one 1024-thread
// workgroup per row.
//
// Semantics are those of slm::sampling::sample_with_params
// (ferrum_core/src/slm/sampling.rs:124-210), step by step:
//   0. (GPT-2 input) p = softmax(z) (ops.rs:478-502), l = ln(max(p, 1e-12))
//      (slm/token_stream.rs:134), fused here.
//   1. repetition penalty once per occurrence of an id in `recent`
//      (l > 0 ? l / pen : l * pen), ids >= vocab skipped         (133-144)
//   2. temperature <= 0: argmax_first under f32::total_cmp        (96-104, 147-149)
//   3. t = max(temperature, 0.01); e = exp((l - max) / t); sum; NaN or
//      sum <= 1e-10 -> draw % n; p = e / sum                      (150-169)
//   4. top-k: thr = k-th largest p, p < thr -> 0 (ties kept)      (171-180)
//   5. top-p: walk descending p, keep until cum >= top_p          (183-200)
//   6. p /= sum2 (index order); first i with r <= cumsum          (205-209, 109-122)
//
// Storage.  The row lives in registers: thread t holds ids t, t + 1024, ...
// (up to 50 per thread: vocabularies up to 51,200), loaded once with
// every load in flight, and every later pass runs on registers.  Larger
// vocabularies keep the row in a per-row global buffer (L2-resident) and each
// pass streams it with eight loads in flight per thread.
//
// Steps 4-6.  A 64-bucket histogram of p under the largest p (from the top 12
// bits: 8 buckets per octave for 5 octaves, then 2, then 1 per octave; 21
// octaves in all) finds the bucket where the top-k
// count or the top-p mass is reached; every element at or above it (at most
// kCap) is gathered into LDS, sorted by (p descending, index ascending) with a
// bitonic sort, and one wave replays steps 4-6 in the reference's own order —
// so once the p values agree, the cum / top-p / renormalise / draw arithmetic
// is the reference's bit for bit.  Rows whose survivor set is larger take the
// general path: an exact radix select for the top-k threshold, a radix select
// by mass (64-bit fixed point, order-independent) for the top-p cut, and a
// scan in index order for the draw; those sums are parallel, so they may differ
// from the sequential f32 sums in the last bits (a near-tie only).
// Every reduction has a fixed shape, so results never depend on timing.
#include <cfloat>
#include <climits>

#include "fh_internal.hpp"

// The sequential parts replay the reference's arithmetic, which rounds every
// product and sum (no FMA anywhere in it): no contraction in this file.
#pragma clang fp contract(off)

namespace {

constexpr int kT = 1024;        // threads per row
constexpr int kW = kT / 64;     // waves per row
constexpr int kCap = 4096;      // LDS survivor capacity
constexpr int kBuckets = 64;    // histogram buckets under the max p (bucket_of)
constexpr int kCopies = 16;     // histogram copies (lane & 15) against same-bin conflicts
constexpr int kSlots = 8192;    // repetition-penalty hash table
constexpr int kChunk = 4096;    // recent ids deduplicated per table fill
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr int kMaxItems = 50;   // register-resident rows: vocab <= kMaxItems * kT (51,200; GPT-2's 50,257)

struct Shared {
    union {
        struct {
            uint32_t key[kSlots];
            uint32_t cnt[kSlots];
        } pen;
        unsigned long long cand[kCap];  // sort keys, see cand_key
    } u;
    uint32_t hist[kCopies][kBuckets];
    unsigned long long mass[kCopies][kBuckets];
    uint32_t rhist[256];
    unsigned long long rmass[256];
    alignas(16) float slab[kW][kMaxItems];
    float pa[256], pb[256];  // other workgroups' partials of the split kernel
    int qa[256], qb[256];
    float redf[kW];
    int redi[kW];
    int bi[8];
    unsigned long long bu[2];
    unsigned int n_cand;
};

// ---- wave and block reductions (fixed DPP pattern, deterministic) -------------

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float rl(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: every
// lane of a 16-lane row ends with the same row total; then the four row totals.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return (rl(v, 0) + rl(v, 16)) + (rl(v, 32) + rl(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
}
__device__ __forceinline__ int wave_max_i(int v) {
    v = max(v, dppi<0xB1>(v));
    v = max(v, dppi<0x4E>(v));
    v = max(v, dppi<0x141>(v));
    v = max(v, dppi<0x140>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, dppi<0xB1>(v));
    v = min(v, dppi<0x4E>(v));
    v = min(v, dppi<0x141>(v));
    v = min(v, dppi<0x140>(v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += dppi<0xB1>(v);
    v += dppi<0x4E>(v);
    v += dppi<0x141>(v);
    v += dppi<0x140>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float block_sum(Shared& s, float v) {
    v = wave_sum(v);
    __syncthreads();
    if (lane_id() == 0) s.redf[wave_id()] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < kW; i++) r += s.redf[i];
    return r;
}
__device__ __forceinline__ float block_max(Shared& s, float v) {
    v = wave_max(v);
    __syncthreads();
    if (lane_id() == 0) s.redf[wave_id()] = v;
    __syncthreads();
    float r = -INFINITY;
#pragma unroll
    for (int i = 0; i < kW; i++) r = fmaxf(r, s.redf[i]);
    return r;
}
__device__ __forceinline__ int block_max_i(Shared& s, int v) {
    v = wave_max_i(v);
    __syncthreads();
    if (lane_id() == 0) s.redi[wave_id()] = v;
    __syncthreads();
    int r = INT_MIN;
#pragma unroll
    for (int i = 0; i < kW; i++) r = max(r, s.redi[i]);
    return r;
}
__device__ __forceinline__ int block_min_i(Shared& s, int v) {
    v = wave_min_i(v);
    __syncthreads();
    if (lane_id() == 0) s.redi[wave_id()] = v;
    __syncthreads();
    int r = INT_MAX;
#pragma unroll
    for (int i = 0; i < kW; i++) r = min(r, s.redi[i]);
    return r;
}
__device__ __forceinline__ int block_sum_i(Shared& s, int v) {
    v = wave_sum_i(v);
    __syncthreads();
    if (lane_id() == 0) s.redi[wave_id()] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < kW; i++) r += s.redi[i];
    return r;
}
// Exclusive prefix over threads in thread order; also returns the total.
__device__ __forceinline__ float block_exclusive_scan(Shared& s, float v, float* total) {
    const int lane = lane_id(), wv = wave_id();
    float incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    __syncthreads();
    if (lane == 63) s.redf[wv] = incl;
    __syncthreads();
    float before = 0.0f, all = 0.0f;
#pragma unroll
    for (int i = 0; i < kW; i++) {
        if (i < wv) before += s.redf[i];
        all += s.redf[i];
    }
    *total = all;
    return before + (incl - v);
}

// ---- row storage ---------------------------------------------------------------------

// Register-resident row (or row segment): thread t holds ids
// base + t + j * kT < n, j < ITEMS (n is the end of the ids held here).
template <int ITEMS>
struct RegRow {
    float v[ITEMS];
    int n;
    int base = 0;
    __device__ __forceinline__ void load(const float* __restrict__ src) {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = base + threadIdx.x + j * kT;
            v[j] = i < n ? src[i] : 0.0f;
        }
    }
    template <class F>
    __device__ __forceinline__ void map(F f) {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = base + threadIdx.x + j * kT;
            if (i < n) v[j] = f(v[j], i);
        }
    }
    template <class F>
    __device__ __forceinline__ void visit(F f) const {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = base + threadIdx.x + j * kT;
            if (i < n) f(v[j], i);
        }
    }
};

// Global-buffer row for vocabularies beyond the register file: same id-to-thread
// mapping, streamed eight ids per thread at a time.
struct GlobalRow {
    static constexpr int U = 8;
    float* w;
    int n;
    __device__ __forceinline__ void load(const float* __restrict__ src) {
        for (int base = threadIdx.x; base < n; base += kT * U) {
            float t[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                t[u] = i < n ? src[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                if (i < n) w[i] = t[u];
            }
        }
    }
    template <class F>
    __device__ __forceinline__ void map(F f) {
        for (int base = threadIdx.x; base < n; base += kT * U) {
            float t[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                t[u] = i < n ? w[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                if (i < n) w[i] = f(t[u], i);
            }
        }
    }
    template <class F>
    __device__ __forceinline__ void visit(F f) const {
        for (int base = threadIdx.x; base < n; base += kT * U) {
            float t[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                t[u] = i < n ? w[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + u * kT;
                if (i < n) f(t[u], i);
            }
        }
    }
};

// ---- helpers -------------------------------------------------------------------------

__device__ __forceinline__ int total_key(float v) {
    const int b = __builtin_bit_cast(int, v);
    return b ^ static_cast<int>(static_cast<unsigned>(b >> 31) >> 1);
}

// Sort key: (bits(p) << 32) | ~index; descending order = p descending, then
// index ascending.  p >= 0 here, so its bits order like its values.
__device__ __forceinline__ unsigned long long cand_key(float p, int i) {
    return (static_cast<unsigned long long>(__builtin_bit_cast(uint32_t, p)) << 32) |
           static_cast<unsigned long long>(~static_cast<uint32_t>(i));
}
__device__ __forceinline__ float key_p(unsigned long long k) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(k >> 32));
}
__device__ __forceinline__ int key_i(unsigned long long k) {
    return static_cast<int>(~static_cast<uint32_t>(k & 0xFFFFFFFFull));
}

// 12-bit bucket key of a non-negative float: 8 exponent bits and the top 3
// mantissa bits (8 buckets per octave).
__device__ __forceinline__ int key12(float p) { return static_cast<int>(__builtin_bit_cast(uint32_t, p) >> 20); }

// Histogram bucket of p under the largest p (ktop = key12(pmax)), coarser with
// depth: 8 buckets per octave for the first 5 octaves, 2 per octave for the
// next 8, one per octave for the next 8 (21 octaves; kBuckets past them).
// Monotone in p, so "bucket <= depth" gathers every id at or above a bucket.
__device__ __forceinline__ int bucket_of(int ktop, float p) {
    const int d = ktop - key12(p);
    return d < 40 ? d : d < 104 ? 40 + ((d - 40) >> 2) : d < 168 ? 56 + ((d - 104) >> 3) : kBuckets;
}

// Fixed-point image of a probability, for order-independent mass sums.
__device__ __forceinline__ unsigned long long fix40(float p) {
    return static_cast<unsigned long long>(static_cast<double>(p) * 1099511627776.0 + 0.5);
}

// Bitonic sort of s.u.cand[0..n2) descending; n2 a power of two <= kCap.
__device__ __forceinline__ void sort_desc(Shared& s, int n2) {
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < n2 / 2; t += kT) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const unsigned long long a = s.u.cand[lo], b = s.u.cand[hi];
                if ((a < b) == desc) {
                    s.u.cand[lo] = b;
                    s.u.cand[hi] = a;
                }
            }
        }
    }
    __syncthreads();
}

// Append (key) to the LDS list, one LDS atomic per wave.
__device__ __forceinline__ void append(Shared& s, bool take, unsigned long long key) {
    const unsigned long long mask = __ballot(take);
    if (mask == 0) return;
    const int lane = lane_id();
    const int leader = __ffsll(static_cast<long long>(mask)) - 1;
    unsigned base = 0;
    if (lane == leader) base = atomicAdd(&s.n_cand, static_cast<unsigned>(__popcll(mask)));
    base = __builtin_amdgcn_readlane(base, leader);
    if (take) {
        const unsigned before = __popcll(mask & ((1ull << lane) - 1ull));
        s.u.cand[base + before] = key;
    }
}

// Radix select over the bit patterns of the non-negative values (bit order =
// value order): the k-th largest (1-based), exactly.  Histograms count in LDS.
template <class Row>
__device__ __forceinline__ float radix_kth_largest(Shared& s, const Row& row, int k) {
    uint32_t prefix = 0, pmask = 0;
    int kr = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kT) s.rhist[i] = 0;
        __syncthreads();
        row.visit([&](float p, int) {
            const uint32_t u = __builtin_bit_cast(uint32_t, p);
            if ((u & pmask) == prefix) atomicAdd(&s.rhist[(u >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (threadIdx.x == 0) {
            int above = 0, dg = 0;
            for (int d = 255; d >= 0; d--) {
                if (above + static_cast<int>(s.rhist[d]) >= kr) {
                    dg = d;
                    break;
                }
                above += static_cast<int>(s.rhist[d]);
            }
            s.bi[0] = dg;
            s.bi[1] = kr - above;
        }
        __syncthreads();
        prefix |= static_cast<uint32_t>(s.bi[0]) << shift;
        pmask |= 255u << shift;
        kr = s.bi[1];
    }
    return __builtin_bit_cast(float, prefix);
}

// The c-th smallest index (1-based) among ids whose value equals `tau`.
template <class Row>
__device__ __forceinline__ int radix_kth_smallest_index_of(Shared& s, const Row& row, float tau, int c) {
    uint32_t prefix = 0, pmask = 0;
    int kr = c;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kT) s.rhist[i] = 0;
        __syncthreads();
        row.visit([&](float p, int i) {
            const uint32_t u = static_cast<uint32_t>(i);
            if (p == tau && (u & pmask) == prefix) atomicAdd(&s.rhist[(u >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (threadIdx.x == 0) {
            int below = 0, dg = 255;
            for (int d = 0; d < 256; d++) {
                if (below + static_cast<int>(s.rhist[d]) >= kr) {
                    dg = d;
                    break;
                }
                below += static_cast<int>(s.rhist[d]);
            }
            s.bi[0] = dg;
            s.bi[1] = kr - below;
        }
        __syncthreads();
        prefix |= static_cast<uint32_t>(s.bi[0]) << shift;
        pmask |= 255u << shift;
        kr = s.bi[1];
    }
    return static_cast<int>(prefix);
}

// The top-p cut over the whole row by mass (general path): the largest value
// tau with mass(p >= tau) >= top_p in 64-bit fixed point; keeps p > tau and,
// of the p == tau ties, the lowest indices until the mass is reached.
template <class Row>
__device__ __forceinline__ void topp_by_mass(Shared& s, Row& row, float top_p) {
    const unsigned long long target = fix40(top_p);
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above = 0;
    bool cut = true;
#pragma unroll
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kT) s.rmass[i] = 0;
        __syncthreads();
        row.visit([&](float p, int) {
            const uint32_t u = __builtin_bit_cast(uint32_t, p);
            if (p > 0.0f && (u & pmask) == prefix) atomicAdd(&s.rmass[(u >> shift) & 255u], fix40(p));
        });
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long acc = above;
            int dg = -1;
            for (int d = 255; d >= 0; d--) {
                if (acc + s.rmass[d] >= target) {
                    dg = d;
                    break;
                }
                acc += s.rmass[d];
            }
            s.bi[0] = dg;
            s.bu[0] = acc;
        }
        __syncthreads();
        const int dg = s.bi[0];
        above = s.bu[0];
        __syncthreads();
        if (dg < 0) {  // the whole mass stays under top_p: everything is kept
            cut = false;
            break;
        }
        prefix |= static_cast<uint32_t>(dg) << shift;
        pmask |= 255u << shift;
    }
    if (!cut) return;
    const float tau = __builtin_bit_cast(float, prefix);
    const unsigned long long ft = fix40(tau);
    const unsigned long long need = target > above ? target - above : 0;
    int ties = 0;
    row.visit([&](float p, int) { ties += p == tau; });
    ties = block_sum_i(s, ties);
    long long keep = ft ? static_cast<long long>((need + ft - 1) / ft) : 1;
    if (keep < 1) keep = 1;
    int last_tie = INT_MAX;
    if (keep < ties) last_tie = radix_kth_smallest_index_of(s, row, tau, static_cast<int>(keep));
    row.map([&](float p, int i) { return (p > tau || (p == tau && i <= last_tie)) ? p : 0.0f; });
    __syncthreads();
}

// The first id in index order whose running mass cum0 + sum of p / sum2
// reaches r, or INT_MAX.  Slab j = the kT ids base + [j * kT, (j + 1) * kT):
// slab totals (wave sums, then waves in order) find the slab, one block scan
// finds the id.
template <int ITEMS>
__device__ __forceinline__ int draw_scan_from(Shared& s, const RegRow<ITEMS>& row, float sum2, float r, float cum0) {
    const int lane = lane_id(), wv = wave_id();
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const int i = row.base + threadIdx.x + j * kT;
        const float q = (i < row.n && row.v[j] > 0.0f) ? row.v[j] / sum2 : 0.0f;
        const float t = wave_sum(q);
        if (lane == 0) s.slab[wv][j] = t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float cum = cum0;
        int js = -1;
        for (int j = 0; j < ITEMS; j++) {
            float t = 0.0f;
            for (int w = 0; w < kW; w++) t += s.slab[w][j];
            if (js < 0 && r <= cum + t) {
                js = j;
                s.redf[0] = cum;
            }
            cum += t;
        }
        s.bi[0] = js;
    }
    __syncthreads();
    const int js = s.bi[0];
    const float base = s.redf[0];
    __syncthreads();
    if (js < 0) return INT_MAX;
    float q = 0.0f;
    int mine = -1;
#pragma unroll
    for (int j = 0; j < ITEMS; j++)
        if (j == js) {
            const int i = row.base + threadIdx.x + j * kT;
            if (i < row.n && row.v[j] > 0.0f) {
                q = row.v[j] / sum2;
                mine = i;
            }
        }
    float total;
    const float before = block_exclusive_scan(s, q, &total);
    const bool hit = mine >= 0 && r <= base + before + q;
    return block_min_i(s, hit ? mine : INT_MAX);
}

// The first id in index order whose running mass of p / sum2 reaches r, else
// the last id with mass (pick_by_mass, sampling.rs:109-122).
template <int ITEMS>
__device__ __forceinline__ int draw_scan(Shared& s, const RegRow<ITEMS>& row, float sum2, float r) {
    const int first = draw_scan_from(s, row, sum2, r, 0.0f);
    if (first != INT_MAX) return first;
    int last = -1;
    row.visit([&](float p, int i) {
        if (p > 0.0f) last = i;
    });
    last = block_max_i(s, last);
    return last >= 0 ? last : 0;
}

__device__ __forceinline__ int draw_scan(Shared& s, const GlobalRow& row, float sum2, float r) {
    const int seg = (row.n + kT - 1) / kT;
    const int b0 = min(row.n, static_cast<int>(threadIdx.x) * seg), b1 = min(row.n, b0 + seg);
    float local = 0.0f;
    int last = -1;
    for (int i = b0; i < b1; i++) {
        const float p = row.w[i];
        if (p > 0.0f) {
            local += p / sum2;
            last = i;
        }
    }
    float total;
    float cum = block_exclusive_scan(s, local, &total);
    int pick = INT_MAX;
    for (int i = b0; i < b1; i++) {
        const float p = row.w[i];
        if (p > 0.0f) {
            cum += p / sum2;
            if (r <= cum) {
                pick = i;
                break;
            }
        }
    }
    const int first = block_min_i(s, pick);
    const int lastg = block_max_i(s, last);
    return first != INT_MAX ? first : (lastg >= 0 ? lastg : 0);
}

__device__ __forceinline__ unsigned long long shfl_xor64(unsigned long long v, int m) {
    const unsigned lo = __shfl_xor(static_cast<unsigned>(v), m, 64);
    const unsigned hi = __shfl_xor(static_cast<unsigned>(v >> 32), m, 64);
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ __forceinline__ unsigned rlu(unsigned v, int lane) {
    return static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ unsigned long long rl64(unsigned long long v, int lane) {
    return (static_cast<unsigned long long>(rlu(static_cast<unsigned>(v >> 32), lane)) << 32) |
           rlu(static_cast<unsigned>(v), lane);
}

// Sort one wave's keys (lanes < nc, distinct) descending: each lane counts the
// keys above its own (readlane broadcasts, no LDS round trips), then the keys
// are scattered to their ranks through `tmp` (64 entries of LDS).
// Lane exchange with lane ^ S inside the wave, without LDS: DPP quad_perm for
// 1 and 2, DPP row shifts left/right for 4 and 8, and the gfx950 half-row /
// half-wave swaps (v_permlane16_swap, v_permlane32_swap) for 16 and 32.
template <int S>
__device__ __forceinline__ unsigned xor_lane(unsigned v) {
    const int lane = lane_id();
    if constexpr (S == 1) return static_cast<unsigned>(dppi<0xB1>(static_cast<int>(v)));
    else if constexpr (S == 2) return static_cast<unsigned>(dppi<0x4E>(static_cast<int>(v)));
    else if constexpr (S == 4 || S == 8) {
        const unsigned up = static_cast<unsigned>(dppi<0x100 + S>(static_cast<int>(v)));  // row_shl: lane + S
        const unsigned dn = static_cast<unsigned>(dppi<0x110 + S>(static_cast<int>(v)));  // row_shr: lane - S
        return (lane & S) ? dn : up;
    } else if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        static_assert(S == 32, "lane distance");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}

// One compare-exchange of a bitonic network over the 64 lanes: blocks of SIZE
// lanes alternate direction so the whole wave ends descending.
template <int SIZE, int S>
__device__ __forceinline__ unsigned long long bitonic_step(unsigned long long k) {
    const int lane = lane_id();
    const unsigned long long p = (static_cast<unsigned long long>(xor_lane<S>(static_cast<unsigned>(k >> 32))) << 32) |
                                 xor_lane<S>(static_cast<unsigned>(k));
    const bool keep_max = ((lane & S) == 0) == (SIZE == 64 || (lane & SIZE) == 0);
    return keep_max == (p > k) ? p : k;
}
template <int SIZE>
__device__ __forceinline__ unsigned long long bitonic_merge(unsigned long long k) {
    if constexpr (SIZE >= 64) k = bitonic_step<SIZE, 32>(k);
    if constexpr (SIZE >= 32) k = bitonic_step<SIZE, 16>(k);
    if constexpr (SIZE >= 16) k = bitonic_step<SIZE, 8>(k);
    if constexpr (SIZE >= 8) k = bitonic_step<SIZE, 4>(k);
    if constexpr (SIZE >= 4) k = bitonic_step<SIZE, 2>(k);
    return bitonic_step<SIZE, 1>(k);
}

// The wave's keys (lanes >= nc contribute 0, which is above no key) sorted
// descending across the lanes, in registers: 21 compare-exchange steps.
__device__ __forceinline__ unsigned long long wave_sort_desc(unsigned long long k, int nc) {
    k = lane_id() < nc ? k : 0ull;
    k = bitonic_merge<2>(k);
    k = bitonic_merge<4>(k);
    k = bitonic_merge<8>(k);
    k = bitonic_merge<16>(k);
    k = bitonic_merge<32>(k);
    return bitonic_merge<64>(k);
}

// The 64 largest of two waves of keys, sorted descending: a descending and an
// ascending run form a bitonic sequence whose lane-wise maxima are its upper
// half (the 64 largest), and one bitonic merge sorts them.
__device__ __forceinline__ unsigned long long wave_top64(unsigned long long a, unsigned long long b) {
    a = wave_sort_desc(a, 64);
    b = ~wave_sort_desc(~b, 64);  // ascending (complements reverse the order)
    return bitonic_merge<64>(a > b ? a : b);
}

// Running f32 sum over lanes 0..len-1 in lane order (the reference's
// sequential order): lane c gets the sum of lanes 0..c.  Each step is one
// readlane and one dependent add; no branches.
__device__ __forceinline__ float lane_running_sum(float v, int len) {
    const int lane = lane_id();
    // lanes >= len add +0.0, which leaves a non-negative sum unchanged: all
    // 64 steps, unrolled, no branches
    const unsigned vb = __builtin_bit_cast(unsigned, lane < len ? v : 0.0f);
    float cum = 0.0f, mine = 0.0f;
#pragma unroll
    for (int c = 0; c < 64; c++) {
        cum += __builtin_bit_cast(float, rlu(vb, c));
        mine = lane == c ? cum : mine;
    }
    return mine;
}

// Steps 4-6 for at most 64 gathered ids, in one wave and in registers: sort
// by (p desc, index asc), the reference's top-k threshold and sequential
// top-p walk, back to index order, sequential sum2 and pick_by_mass
// (sampling.rs:171-209, 109-122).  Every lane of the wave calls with the same
// arguments; lane 0 writes *out.  Returns false, writing nothing, when the
// top-p cut lies below the gathered ids.
__device__ __forceinline__ bool wave_tail(unsigned long long key, int nc, int top_k, float top_p, bool use_k,
                                          bool use_p, float r, uint32_t* __restrict__ out) {
    const int lane = lane_id();
    unsigned long long k = lane < nc ? key : 0ull;
    k = wave_sort_desc(k, nc);
    int len = nc;
    if (use_k) {
        const float thr = __builtin_bit_cast(float, rlu(static_cast<unsigned>(k >> 32), top_k - 1));
        len = __popcll(__ballot(lane < nc && key_p(k) >= thr));  // a prefix: the keys are sorted
    }
    if (use_p) {
        // cum after each survivor in descending order; keep up to the first >= top_p
        const float cum = lane_running_sum(lane < len ? key_p(k) : 0.0f, len);
        const unsigned long long crossed = __ballot(lane < len && cum >= top_p);
        if (crossed) len = __ffsll(static_cast<long long>(crossed));
        else if (!use_k) return false;
    }
    unsigned long long k2 =
        lane < len ? (static_cast<unsigned long long>(~static_cast<uint32_t>(key_i(k))) << 32) | (k >> 32) : 0ull;
    k2 = wave_sort_desc(k2, len);  // descending ~index = ascending index
    const float pl = lane < len ? __builtin_bit_cast(float, static_cast<unsigned>(k2)) : 0.0f;
    const int idx = static_cast<int>(~static_cast<unsigned>(k2 >> 32));
    // sum2 in index order, sequentially
    const unsigned pb = __builtin_bit_cast(unsigned, pl);
    float sum2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; i++) sum2 += __builtin_bit_cast(float, rlu(pb, i));  // lanes >= len hold +0.0
    // p / sum2 per lane, the running cumsum in index order, then the first
    // id with mass whose cumsum reaches r, else the last id with mass
    const float q = pl / sum2;
    const float cumsum = lane_running_sum(q, len);
    const unsigned long long live = __ballot(lane < len && q > 0.0f);
    const unsigned long long hit = __ballot(lane < len && q > 0.0f && r <= cumsum);
    const int pick_lane = hit ? __ffsll(static_cast<long long>(hit)) - 1 : (live ? 63 - __clzll(live) : 0);
    const int pick = __builtin_amdgcn_readlane(idx, pick_lane);
    if (lane == 0) *out = static_cast<uint32_t>(live ? pick : 0);
    return true;
}

// The shallowest bucket depth whose cumulative count reaches k (top-k) or
// whose fixed-point mass reaches top_p, plus one bucket of margin (top-p
// only); -1 when not found or when more than kCap ids would be gathered.
// One wave (lane = bucket): inclusive prefix sums of the counts and the
// fixed-point masses (exact integer sums, so the order does not matter), the
// first bucket that reaches the target by ballot.  Every lane of the wave
// calls and gets the result.
__device__ __forceinline__ int bucket_depth(const uint32_t* hist, const unsigned long long* mass, int top_k,
                                            float top_p, bool use_k, bool use_p) {
    static_assert(kBuckets == 64, "one bucket per lane");
    const int lane = lane_id();
    unsigned cnt = hist[lane];
    unsigned long long acc = use_k ? 0ull : mass[lane];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned c_up = static_cast<unsigned>(__shfl_up(static_cast<int>(cnt), off, 64));
        const unsigned lo = static_cast<unsigned>(__shfl_up(static_cast<int>(static_cast<unsigned>(acc)), off, 64));
        const unsigned hi = static_cast<unsigned>(__shfl_up(static_cast<int>(static_cast<unsigned>(acc >> 32)), off, 64));
        if (lane >= off) {
            cnt += c_up;
            acc += (static_cast<unsigned long long>(hi) << 32) | lo;
        }
    }
    const unsigned long long target = use_p ? fix40(top_p) : 0;
    const unsigned long long reached =
        __ballot(use_k ? static_cast<int>(cnt) >= top_k : acc >= target);
    if (!reached) return -1;
    int depth = __ffsll(static_cast<long long>(reached)) - 1;
    if (!use_k && depth + 1 < kBuckets) depth++;
    const int total = static_cast<int>(rlu(cnt, depth));
    return total <= kCap ? depth : -1;
}

// Sort s.u.cand[0..nc) by (p desc, index asc) and replay top-k then top-p in
// the reference's order (sampling.rs:171-200).  Returns the survivor count,
// or -1 when the top-p cut lies below the gathered ids.  Every thread calls.
__device__ __forceinline__ int replay_list(Shared& s, int nc, int top_k, float top_p, bool use_k, bool use_p) {
    const int tid = threadIdx.x;
    int n2 = 1;
    while (n2 < nc) n2 <<= 1;
    for (int i = nc + tid; i < n2; i += kT) s.u.cand[i] = 0ull;  // p = 0 sorts last
    sort_desc(s, n2);
    if (tid < 64) {  // wave 0, every lane the same
        int len = nc;
        bool ok = true;
        if (use_k) {
            const float thr = key_p(s.u.cand[top_k - 1]);
            len = top_k;
            while (len < nc && key_p(s.u.cand[len]) >= thr) len++;
        }
        if (use_p) {
            float cum = 0.0f;
            bool crossed = false;
            int c = 0;
            for (; c < len; c++) {
                cum += key_p(s.u.cand[c]);
                if (cum >= top_p) {
                    crossed = true;
                    break;
                }
            }
            if (crossed) len = c + 1;
            else if (!use_k) ok = false;
        }
        if (tid == 0) s.bi[1] = ok ? len : -1;
    }
    __syncthreads();
    const int n_list = s.bi[1];
    __syncthreads();
    return n_list;
}

// Renormalise the survivors s.u.cand[0..n_list) (p-descending on entry) and
// draw: back into index order, then one wave replays sum2 and pick_by_mass
// sequentially (sampling.rs:205-209, 109-122).  Every thread calls; thread 0
// writes *out.
__device__ __forceinline__ void finish_list(Shared& s, int n_list, float r, uint32_t* __restrict__ out) {
    const int tid = threadIdx.x;
    for (int i = tid; i < n_list; i += kT) {  // key (~index << 32) | bits(p)
        const unsigned long long k = s.u.cand[i];
        s.u.cand[i] = (static_cast<unsigned long long>(~static_cast<uint32_t>(key_i(k))) << 32) | (k >> 32);
    }
    int n2 = 1;
    while (n2 < n_list) n2 <<= 1;
    for (int i = n_list + tid; i < n2; i += kT) s.u.cand[i] = 0ull;
    sort_desc(s, n2);  // descending ~index = ascending index
    if (tid < 64) {
        float sum2 = 0.0f;
        for (int i = 0; i < n_list; i++) sum2 += __builtin_bit_cast(float, static_cast<uint32_t>(s.u.cand[i]));
        float cumsum = 0.0f;
        int pick = -1, last = 0;
        for (int i = 0; i < n_list; i++) {
            const unsigned long long k = s.u.cand[i];
            const float p = __builtin_bit_cast(float, static_cast<uint32_t>(k)) / sum2;
            const int idx = static_cast<int>(~static_cast<uint32_t>(k >> 32));
            if (p > 0.0f) {
                last = idx;
                cumsum += p;
                if (r <= cumsum) {
                    pick = idx;
                    break;
                }
            }
        }
        if (tid == 0) *out = static_cast<uint32_t>(pick >= 0 ? pick : last);
    }
}

// The general path over a whole row: exact top-k threshold, top-p cut by mass,
// then the block-wide draw.  Every thread calls; thread 0 writes *out.
template <class Row>
__device__ __forceinline__ void general_tail(Shared& s, Row& row, int top_k, float top_p, bool use_k, bool use_p,
                                             float r, uint32_t* __restrict__ out) {
    if (use_k) {
        const float thr = radix_kth_largest(s, row, top_k);
        row.map([&](float p, int) { return p < thr ? 0.0f : p; });
        __syncthreads();
    }
    if (use_p) topp_by_mass(s, row, top_p);
    float s2 = 0.0f;
    row.visit([&](float p, int) { s2 += p; });
    const float sum2 = block_sum(s, s2);
    const int pick = draw_scan(s, row, sum2, r);
    if (threadIdx.x == 0) *out = static_cast<uint32_t>(pick);
}

struct Params {
    float temperature;
    int top_k;
    float top_p;
    float pen;
    int kind;
    int n;
    // Recent lists as (begin, end) pairs per row (FH_RECENT_RANGES) rather
    // than rows + 1 running offsets.
    bool ranges;
    // Cross-workgroup waits of the split kernel give up after this many polls
    // (kSpinLimit unless a test lowers it).
    unsigned spin_limit;
    // Testing hook: the segment whose workgroup publishes nothing (-1: none),
    // so its readers' bounded waits give up and report FH_STATUS_EXCHANGE.
    int skip_seg;
};

// The recent list of a row: offsets[row] .. offsets[row + 1], or with ranges
// offsets[2 row] .. offsets[2 row + 1].  Decreasing offsets are recorded in
// the status word (and the row gets no penalty).
__device__ __forceinline__ int recent_len(const uint32_t* __restrict__ offsets, size_t row, bool ranges,
                                          unsigned* status, const uint32_t** rec, const uint32_t* __restrict__ recent) {
    const uint32_t r0 = ranges ? offsets[2 * row] : offsets[row], r1 = ranges ? offsets[2 * row + 1] : offsets[row + 1];
    *rec = recent + r0;
    if (r1 < r0) {
        if (threadIdx.x == 0) atomicOr(status, static_cast<unsigned>(FH_STATUS_BAD_OFFSETS));
        return 0;
    }
    return static_cast<int>(min(r1 - r0, 0x7FFFFFFFu));
}

template <class Row>
__device__ __forceinline__ void sample_row(Shared& s, Row& row, const Params& P, const float* __restrict__ z,
                           const uint32_t* __restrict__ recent, int nrec, uint64_t draw_u64, bool has_draw,
                           uint32_t* __restrict__ out) {
    const int tid = threadIdx.x;
    const int n = P.n;

    // ---- 0. sampler input ------------------------------------------------------------
    row.load(z);
    if (P.kind == FH_LOGITS_GPT2_SOFTMAX) {
        float m = -INFINITY;
        row.visit([&](float x, int) { m = fmaxf(m, x); });
        const float zmax = block_max(s, m);
        float sm = 0.0f;
        row.visit([&](float x, int) { sm += expf(x - zmax); });
        const float zsum = block_sum(s, sm);
        row.map([&](float x, int) { return logf(fmaxf(expf(x - zmax) / zsum, 1e-12f)); });
    }

    // ---- 1. repetition penalty ---------------------------------------------------------
    const float pen = P.pen;
    if (fabsf(pen - 1.0f) > FLT_EPSILON && pen > 0.0f && nrec > 0) {
        for (int base = 0; base < nrec; base += kChunk) {
            for (int i = tid; i < kSlots; i += kT) {
                s.u.pen.key[i] = kEmpty;
                s.u.pen.cnt[i] = 0;
            }
            __syncthreads();
            const int end = min(nrec, base + kChunk);
            for (int r = base + tid; r < end; r += kT) {
                const uint32_t tok = recent[r];
                if (tok >= static_cast<uint32_t>(n)) continue;
                uint32_t h = (tok * 2654435761u) & (kSlots - 1);
                while (true) {
                    const uint32_t prev = atomicCAS(&s.u.pen.key[h], kEmpty, tok);
                    if (prev == kEmpty || prev == tok) {
                        atomicAdd(&s.u.pen.cnt[h], 1u);
                        break;
                    }
                    h = (h + 1) & (kSlots - 1);
                }
            }
            __syncthreads();
            row.map([&](float l, int i) {
                uint32_t h = (static_cast<uint32_t>(i) * 2654435761u) & (kSlots - 1);
                while (true) {
                    const uint32_t key = s.u.pen.key[h];
                    if (key == kEmpty) return l;
                    if (key == static_cast<uint32_t>(i)) {
                        for (uint32_t c = s.u.pen.cnt[h]; c > 0; c--) l = l > 0.0f ? l / pen : l * pen;
                        return l;
                    }
                    h = (h + 1) & (kSlots - 1);
                }
            });
            __syncthreads();
        }
    }

    // ---- 2. greedy -----------------------------------------------------------------------
    if (P.temperature <= 0.0f) {
        int bk = INT_MIN, bi = INT_MAX;
        row.visit([&](float x, int i) {
            const int k = total_key(x);
            if (k > bk || (k == bk && i < bi)) {
                bk = k;
                bi = i;
            }
        });
        const int best = block_max_i(s, bk);
        const int first = block_min_i(s, bk == best ? bi : INT_MAX);
        if (tid == 0) *out = static_cast<uint32_t>(first == INT_MAX ? 0 : first);
        return;
    }
    (void)has_draw;
    const float t = fmaxf(P.temperature, 0.01f);

    // ---- 3. temperature softmax ---------------------------------------------------------
    float m = -INFINITY;
    row.visit([&](float l, int) { m = fmaxf(m, l); });
    const float mx = block_max(s, m);
    float se = 0.0f;
    row.map([&](float l, int) {
        const float e = expf((l - mx) / t);
        se += e;
        return e;
    });
    const float sum = block_sum(s, se);
    if (sum != sum || sum <= 1e-10f) {
        if (tid == 0) *out = static_cast<uint32_t>(draw_u64 % static_cast<uint64_t>(n));
        return;
    }
    float pm = 0.0f;
    row.map([&](float e, int) {
        const float p = e / sum;
        pm = fmaxf(pm, p);
        return p;
    });
    const float pmax = block_max(s, pm);
    const float r = static_cast<float>(draw_u64 >> 40) / static_cast<float>(1u << 24);

    // ---- 4./5./6. top-k, top-p, renormalise and draw --------------------------------------
    const bool use_k = P.top_k > 0 && P.top_k < n;
    const bool use_p = P.top_p < 1.0f;
    if (use_k || use_p) {
        const int ktop = key12(pmax);
        const int copy = tid & (kCopies - 1);
        for (int i = tid; i < kCopies * kBuckets; i += kT) {
            (&s.hist[0][0])[i] = 0;
            (&s.mass[0][0])[i] = 0;
        }
        __syncthreads();
        row.visit([&](float p, int) {
            const int b = bucket_of(ktop, p);
            if (p > 0.0f && b < kBuckets) {
                atomicAdd(&s.hist[copy][b], 1u);
                if (!use_k) atomicAdd(&s.mass[copy][b], fix40(p));
            }
        });
        __syncthreads();
        if (tid < kBuckets) {  // fold the copies
            uint32_t c = 0;
            unsigned long long ms = 0;
            for (int k = 0; k < kCopies; k++) {
                c += s.hist[k][tid];
                ms += s.mass[k][tid];
            }
            s.hist[0][tid] = c;
            s.mass[0][tid] = ms;
        }
        __syncthreads();
        if (tid < 64) {
            const int d = bucket_depth(s.hist[0], s.mass[0], P.top_k, P.top_p, use_k, use_p);
            if (tid == 0) {
                s.bi[0] = d;
                s.n_cand = 0;
            }
        }
        __syncthreads();
        const int depth = s.bi[0];
        int n_list = -1;
        if (depth >= 0) {
            row.visit([&](float p, int i) { append(s, p > 0.0f && bucket_of(ktop, p) <= depth, cand_key(p, i)); });
            __syncthreads();
            const int nc = static_cast<int>(s.n_cand);
            if (nc <= 64) {
                if (tid < 64) {
                    const bool ok = wave_tail(s.u.cand[tid < nc ? tid : 0], nc, P.top_k, P.top_p, use_k, use_p, r, out);
                    if (tid == 0) s.bi[2] = ok;
                }
                __syncthreads();
                if (s.bi[2]) return;
            } else {
                n_list = replay_list(s, nc, P.top_k, P.top_p, use_k, use_p);
            }
        }
        if (n_list >= 0) {
            finish_list(s, n_list, r, out);
            return;
        }
    }
    general_tail(s, row, P.top_k, P.top_p, use_k, use_p, r, out);
}

template <int ITEMS>
__global__ void __launch_bounds__(kT)
    k_sample_regs(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
                  const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws,
                  uint32_t* __restrict__ out, unsigned* __restrict__ status) {
    __shared__ Shared s;
    const size_t row = blockIdx.x;
    int nrec = 0;
    const uint32_t* rec = nullptr;
    if (offsets && recent) nrec = recent_len(offsets, row, P.ranges, status, &rec, recent);
    RegRow<ITEMS> st;
    st.n = P.n;
    const bool has_draw = draws != nullptr;
    sample_row(s, st, P, logits + row * static_cast<size_t>(P.n), rec, nrec, has_draw ? draws[row] : 0ull,
               has_draw, out + row);
}

__global__ void __launch_bounds__(kT)
    k_sample_global(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
                    const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws,
                    uint32_t* __restrict__ out, float* __restrict__ work, unsigned* __restrict__ status) {
    __shared__ Shared s;
    const size_t row = blockIdx.x;
    int nrec = 0;
    const uint32_t* rec = nullptr;
    if (offsets && recent) nrec = recent_len(offsets, row, P.ranges, status, &rec, recent);
    GlobalRow st;
    st.n = P.n;
    st.w = work + row * static_cast<size_t>(P.n);
    const bool has_draw = draws != nullptr;
    sample_row(s, st, P, logits + row * static_cast<size_t>(P.n), rec, nrec, has_draw ? draws[row] : 0ull,
               has_draw, out + row);
}

// ---- one row over several workgroups ---------------------------------------------------
//
// Vocabulary rows split into S segments of kT * ITEMS ids, one workgroup each,
// so the per-id exp/log/divide work of steps 0-3 spreads over S CUs.  The
// workgroups of a row exchange small per-segment results (softmax max/sum
// pairs, bucket histograms, segment masses) and workgroup 0 finishes the row
// (sorting the gathered survivors, or the general path over the row's p values
// in `pbuf`).  Partial results are combined in segment order, so the result
// does not depend on timing.
//
// Exchange.  Every value crosses workgroups in a 64-bit slot (32-bit payload,
// 32-bit tag) written with one device-coherent store (a relaxed agent-scope
// atomic: it bypasses the XCD-private L2, so no cache write-back or invalidate
// is needed); a reader polls the slots until each carries this launch's tag,
// so one memory round trip both synchronises and delivers the data.  The tag
// is the row's generation + 1: every workgroup reads `gen` at its start and
// workgroup 0 bumps it when the row is done, so no slot is ever cleared and a
// stale slot (the previous launch's tag) is never taken for a fresh one — which
// keeps the state valid across HIP graph replays.  The launcher keeps rows * S
// <= the number of CUs with one workgroup per CU (the kernel's LDS allows no
// more, and checks that with the occupancy API), so every workgroup of a row
// is resident together; every poll is bounded: a slot still stale after
// P.spin_limit polls sets FH_STATUS_EXCHANGE in the context's status word
// (which fh_sync and the blocking call report) and the workgroup goes on with
// what it has.  Every index derived from exchanged data is clamped, so a
// failed exchange gives a wrong id, never an out-of-bounds access.

constexpr int kSMax = 64;
constexpr unsigned kSpinLimit = 1u << 20;
enum { kPhGpt2 = 0, kPhTemp = 1, kPhGreedy = 2, kPhSeg = 3, kPhDone = 4, kPhases = 5 };

struct RowSync {
    unsigned gen;
    unsigned unused;
    unsigned n_cand;  // survivors appended so far (workgroup 0 zeroes it when done)
    unsigned pad[13];
    unsigned long long a[kPhases][kSMax];  // payload A | tag
    unsigned long long b[kPhases][kSMax];  // payload B | tag
    unsigned long long hist[kSMax][kBuckets];  // bucket count | tag
    unsigned long long mass[kSMax][kBuckets];  // bucket mass, stored before its count
    unsigned long long cand[kCap];
};

template <class T>
__device__ __forceinline__ void cstore(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T cload(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's own earlier stores are complete (so a later store
// of a tag cannot overtake them).
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ unsigned long long tagf(float v, unsigned tag) {
    return (static_cast<unsigned long long>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ unsigned long long tagi(int v, unsigned tag) {
    return (static_cast<unsigned long long>(tag) << 32) | static_cast<uint32_t>(v);
}
__device__ __forceinline__ float untagf(unsigned long long x) { return __builtin_bit_cast(float, static_cast<uint32_t>(x)); }
__device__ __forceinline__ int untagi(unsigned long long x) { return static_cast<int>(static_cast<uint32_t>(x)); }

// Where a bounded wait reports that it gave up, and after how many polls.
struct Waits {
    unsigned* status;
    unsigned limit;
};

// Poll one slot until it carries `tag` (bounded).
__device__ __forceinline__ unsigned long long poll(const Waits& wt, const unsigned long long* slot, unsigned tag) {
    unsigned spins = 0;
    while (true) {
        const unsigned long long x = cload(slot);
        if (static_cast<unsigned>(x >> 32) == tag) return x;
        __builtin_amdgcn_s_sleep(1);
        if (++spins >= wt.limit) {
            atomicOr(wt.status, static_cast<unsigned>(FH_STATUS_EXCHANGE));
            return x;
        }
    }
}
// Poll two slots at once (both loads in flight per round).
__device__ __forceinline__ void poll2(const Waits& wt, const unsigned long long* p, const unsigned long long* q,
                                      unsigned tag, unsigned long long* x, unsigned long long* y) {
    unsigned spins = 0;
    while (true) {
        *x = cload(p);
        *y = cload(q);
        if (static_cast<unsigned>(*x >> 32) == tag && static_cast<unsigned>(*y >> 32) == tag) return;
        __builtin_amdgcn_s_sleep(1);
        if (++spins >= wt.limit) {
            atomicOr(wt.status, static_cast<unsigned>(FH_STATUS_EXCHANGE));
            return;
        }
    }
}

// Thread 0 publishes this workgroup's pair for `phase` (the testing hook
// P.skip_seg silences one segment).
__device__ __forceinline__ void publish(RowSync* rs, int phase, int w, unsigned long long a, unsigned long long b,
                                        int skip_seg) {
    if (threadIdx.x == 0 && w != skip_seg) {
        cstore(&rs->a[phase][w], a);
        cstore(&rs->b[phase][w], b);
    }
}

// Every workgroup's pair for `phase` into s.pa / s.pb (float view) and
// s.qa / s.qb (int view); whole-workgroup call.
__device__ __forceinline__ void gather(Shared& s, const Waits& wt, RowSync* rs, int phase, int S, unsigned tag) {
    const int tid = threadIdx.x;
    if (tid < S) {
        unsigned long long x, y;
        poll2(wt, &rs->a[phase][tid], &rs->b[phase][tid], tag, &x, &y);
        s.pa[tid] = untagf(x);
        s.pb[tid] = untagf(y);
        s.qa[tid] = untagi(x);
        s.qb[tid] = untagi(y);
    }
    __syncthreads();
}

// Softmax statistics of one segment: its max m and sum of exp((x - m) / t),
// two block reductions.  The reference's NaN and -inf behaviour is kept: a
// NaN term makes the sum NaN; a segment whose max is -inf adds nothing (or
// NaN, if it holds a NaN) once merged.
template <class Row>
__device__ __forceinline__ void block_softmax_stats(Shared& s, const Row& row, float t, bool divide, float* m_out,
                                                    float* s_out) {
    float m = -INFINITY;
    row.visit([&](float x, int) { m = fmaxf(m, x); });
    m = block_max(s, m);
    float sum = 0.0f;
    if (m != -INFINITY) row.visit([&](float x, int) { sum += expf(divide ? (x - m) / t : x - m); });
    else row.visit([&](float x, int) { sum += x != x ? NAN : 0.0f; });
    *m_out = m;
    *s_out = block_sum(s, sum);
}

// The gathered per-segment pairs (s.pa = max, s.pb = sum) merged: the row max
// M, then Z = sum_w s_w exp((m_w - M) / t), one segment per lane of every wave
// (a fixed reduction pattern, so every wave gets the same M and Z).
__device__ __forceinline__ void merge_segments(const Shared& s, int S, float t, bool divide, float* M, float* Z) {
    const int lane = lane_id();
    const float mw = lane < S ? s.pa[lane] : -INFINITY;
    const float sw = lane < S ? s.pb[lane] : 0.0f;
    const float m = wave_max(mw);
    float term = 0.0f;
    if (lane < S) term = mw == -INFINITY ? sw * 0.0f : sw * expf(divide ? (mw - m) / t : mw - m);
    *M = m;
    *Z = wave_sum(term);
}

template <int ITEMS>
__global__ void __launch_bounds__(kT)
    k_sample_split(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
                   const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws,
                   uint32_t* __restrict__ out, RowSync* __restrict__ sync, float* __restrict__ pbuf, int S,
                   unsigned* __restrict__ status) {
    __shared__ Shared s;
    const int tid = threadIdx.x;
    const int row = blockIdx.x / S, w = blockIdx.x % S;
    const int n = P.n;
    RowSync* rs = sync + row;
    const Waits wt{status, P.spin_limit};
    const unsigned gen = cload(&rs->gen);
    const unsigned tag = gen + 1;
    const float* z = logits + static_cast<size_t>(row) * n;
    uint32_t* o = out + row;
    RegRow<ITEMS> st;
    st.base = w * kT * ITEMS;
    st.n = min(n, st.base + kT * ITEMS);
    st.load(z);
    // workgroup 0 finishes the row: zero the survivor count, bump the generation
    auto finish = [&]() __attribute__((always_inline)) {
        __syncthreads();
        if (tid == 0) {
            cstore(&rs->n_cand, 0u);
            cstore(&rs->gen, tag);
        }
    };

    // ---- 1. repetition penalty on this segment's ids: the table of (id, count)
    // is built before the first exchange so its loads overlap the wait; it is
    // applied after the GPT-2 bridge, as the reference orders them.
    const float pen = P.pen;
    int nrec = 0;
    const uint32_t* rec = nullptr;
    if (offsets && recent) nrec = recent_len(offsets, row, P.ranges, status, &rec, recent);
    const bool use_pen = fabsf(pen - 1.0f) > FLT_EPSILON && pen > 0.0f && nrec > 0;
    auto fill = [&](int b0) __attribute__((always_inline)) {
        for (int i = tid; i < kSlots; i += kT) {
            s.u.pen.key[i] = kEmpty;
            s.u.pen.cnt[i] = 0;
        }
        __syncthreads();
        const int end = min(nrec, b0 + kChunk);
        for (int r = b0 + tid; r < end; r += kT) {
            const uint32_t tok = rec[r];
            if (tok < static_cast<uint32_t>(st.base) || tok >= static_cast<uint32_t>(st.n)) continue;
            uint32_t h = (tok * 2654435761u) & (kSlots - 1);
            while (true) {
                const uint32_t prev = atomicCAS(&s.u.pen.key[h], kEmpty, tok);
                if (prev == kEmpty || prev == tok) {
                    atomicAdd(&s.u.pen.cnt[h], 1u);
                    break;
                }
                h = (h + 1) & (kSlots - 1);
            }
        }
        __syncthreads();
    };
    auto apply = [&]() __attribute__((always_inline)) {
        st.map([&](float l, int i) {
            uint32_t h = (static_cast<uint32_t>(i) * 2654435761u) & (kSlots - 1);
            while (true) {
                const uint32_t key = s.u.pen.key[h];
                if (key == kEmpty) return l;
                if (key == static_cast<uint32_t>(i)) {
                    for (uint32_t c = s.u.pen.cnt[h]; c > 0; c--) l = l > 0.0f ? l / pen : l * pen;
                    return l;
                }
                h = (h + 1) & (kSlots - 1);
            }
        });
        __syncthreads();
    };
    if (use_pen) fill(0);

    // ---- 0. GPT-2 bridge, with the row's softmax max and sum --------------------------
    if (P.kind == FH_LOGITS_GPT2_SOFTMAX) {
        float m, sm;
        block_softmax_stats(s, st, 1.0f, false, &m, &sm);
        publish(rs, kPhGpt2, w, tagf(m, tag), tagf(sm, tag), P.skip_seg);
        gather(s, wt, rs, kPhGpt2, S, tag);
        float M, Z;
        merge_segments(s, S, 1.0f, false, &M, &Z);
        st.map([&](float x, int) { return logf(fmaxf(expf(x - M) / Z, 1e-12f)); });
    }
    if (use_pen) {
        apply();
        for (int b0 = kChunk; b0 < nrec; b0 += kChunk) {
            fill(b0);
            apply();
        }
    }

    // ---- 2. greedy ---------------------------------------------------------------------
    if (P.temperature <= 0.0f) {
        int bk = INT_MIN, bi = INT_MAX;
        st.visit([&](float x, int i) {
            const int k = total_key(x);
            if (k > bk || (k == bk && i < bi)) {
                bk = k;
                bi = i;
            }
        });
        const int best = block_max_i(s, bk);
        const int first = block_min_i(s, bk == best ? bi : INT_MAX);
        publish(rs, kPhGreedy, w, tagi(best, tag), tagi(first, tag), P.skip_seg);
        if (w != 0) return;
        gather(s, wt, rs, kPhGreedy, S, tag);
        if (tid == 0) {
            int gk = INT_MIN, gi = INT_MAX;
            for (int v = 0; v < S; v++) {  // segments in index order: strict '>' keeps the first
                const int k = s.qa[v], i = s.qb[v];
                if (i != INT_MAX && (gi == INT_MAX || k > gk)) {
                    gk = k;
                    gi = i;
                }
            }
            *o = static_cast<uint32_t>(gi == INT_MAX ? 0 : gi);
        }
        finish();
        return;
    }
    const float t = fmaxf(P.temperature, 0.01f);
    const uint64_t draw = draws[row];
    const float r = static_cast<float>(draw >> 40) / static_cast<float>(1u << 24);

    // ---- 3. temperature softmax over the row --------------------------------------------
    {
        float m, sm;
        block_softmax_stats(s, st, t, true, &m, &sm);
        publish(rs, kPhTemp, w, tagf(m, tag), tagf(sm, tag), P.skip_seg);
    }
    gather(s, wt, rs, kPhTemp, S, tag);
    float mx, sum;
    merge_segments(s, S, t, true, &mx, &sum);
    if (sum != sum || sum <= 1e-10f) {
        if (w == 0) {
            if (tid == 0) *o = static_cast<uint32_t>(draw % static_cast<uint64_t>(n));
            finish();
        }
        return;
    }
    st.map([&](float l, int) { return expf((l - mx) / t) / sum; });
    const float pmax = 1.0f / sum;  // the max id has e = exp(0) = 1
    float* prow = pbuf + static_cast<size_t>(row) * n;

    const bool use_k = P.top_k > 0 && P.top_k < n;
    const bool use_p = P.top_p < 1.0f;
    if (use_k || use_p) {
        // ---- 4./5. bucket histograms, then the gathered survivors --------------------
        const int ktop = key12(pmax);
        const int copy = tid & (kCopies - 1);
        for (int i = tid; i < kCopies * kBuckets; i += kT) {
            (&s.hist[0][0])[i] = 0;
            (&s.mass[0][0])[i] = 0;
        }
        __syncthreads();
        st.visit([&](float p, int) {
            const int b = bucket_of(ktop, p);
            if (p > 0.0f && b < kBuckets) {
                atomicAdd(&s.hist[copy][b], 1u);
                if (!use_k) atomicAdd(&s.mass[copy][b], fix40(p));
            }
        });
        __syncthreads();
        if (tid < kBuckets) {
            uint32_t c = 0;
            unsigned long long ms = 0;
            for (int k = 0; k < kCopies; k++) {
                c += s.hist[k][tid];
                ms += s.mass[k][tid];
            }
            if (w != P.skip_seg) {
                if (!use_k) {
                    cstore(&rs->mass[w][tid], ms);
                    stores_done();
                }
                cstore(&rs->hist[w][tid], tagi(static_cast<int>(c), tag));
            }
        }
        // every segment's histogram, summed in segment order
        uint32_t* hc = reinterpret_cast<uint32_t*>(s.u.cand);                     // [S][kBuckets]
        unsigned long long* hm = s.u.cand + (kSMax * kBuckets) / 2;                 // [S][kBuckets]
        for (int i = tid; i < S * kBuckets; i += kT) {
            const int v = i / kBuckets, b = i % kBuckets;
            hc[i] = static_cast<uint32_t>(poll(wt, &rs->hist[v][b], tag));
            if (!use_k) hm[i] = cload(&rs->mass[v][b]);
        }
        __syncthreads();
        if (tid < kBuckets) {
            uint32_t c = 0;
            unsigned long long ms = 0;
            for (int v = 0; v < S; v++) {
                c += hc[v * kBuckets + tid];
                if (!use_k) ms += hm[v * kBuckets + tid];
            }
            s.hist[0][tid] = c;
            s.mass[0][tid] = ms;
        }
        __syncthreads();
        if (tid < 64) {
            const int d = bucket_depth(s.hist[0], s.mass[0], P.top_k, P.top_p, use_k, use_p);
            if (tid == 0) s.bi[0] = d;
        }
        __syncthreads();
        const int depth = s.bi[0];
        // The row's p values (pbuf) feed workgroup 0's general path, which
        // runs when no bucket qualifies (depth < 0, known to every segment)
        // or, with top-p alone, when the cut lies below the gathered ids;
        // with top-k the gathered survivors always suffice (after a failed
        // exchange the general path may read stale values: a wrong id, never
        // an out-of-bounds read, and the failure is reported).  So they are
        // written only when they may be read -- not before the histogram
        // exchange, where 200 KB of device-coherent stores delayed it.
        if (depth < 0 || !use_k) st.visit([&](float p, int i) { cstore(&prow[i], p); });
        if (depth >= 0) {
            // append this segment's survivors to the row's list, one atomic per wave
            st.visit([&](float p, int i) {
                const bool take = p > 0.0f && bucket_of(ktop, p) <= depth;
                const unsigned long long mask = __ballot(take);
                if (mask == 0) return;
                const int lane = lane_id();
                const int leader = __ffsll(static_cast<long long>(mask)) - 1;
                unsigned base = 0;
                if (lane == leader) base = atomicAdd(&rs->n_cand, static_cast<unsigned>(__popcll(mask)));
                base = __builtin_amdgcn_readlane(base, leader);
                // (at most kCap survivors when the histograms were exchanged
                // intact; the bound only matters after a failed exchange)
                const unsigned at = base + static_cast<unsigned>(__popcll(mask & ((1ull << lane) - 1ull)));
                if (take && at < static_cast<unsigned>(kCap)) cstore(&rs->cand[at], cand_key(p, i));
            });
        }
        stores_done();
        __syncthreads();
        publish(rs, kPhDone, w, tagi(0, tag), tagi(0, tag), P.skip_seg);
        if (w != 0) return;
        gather(s, wt, rs, kPhDone, S, tag);
        int n_list = -1;
        bool done = false;
        if (depth >= 0) {
            // the count and the first 64 keys in one round trip
            unsigned long long key = 0;
            if (tid < 64) key = cload(&rs->cand[tid]);
            const unsigned nc_all = cload(&rs->n_cand);
            const int nc = static_cast<int>(min(nc_all, static_cast<unsigned>(kCap)));
            if (nc_all > static_cast<unsigned>(kCap)) {
                // only after a failed exchange: the list is incomplete, take
                // the general path over the row
            } else if (nc <= 64) {
                if (tid < 64) {
                    const bool ok = wave_tail(key, nc, P.top_k, P.top_p, use_k, use_p, r, o);
                    if (tid == 0) s.bi[2] = ok;
                }
                __syncthreads();
                done = s.bi[2];
            } else if (use_k && P.top_k <= 64 && nc <= 256) {
                // Top-k keeps only ids at or above the k-th largest p, so the
                // 64 largest keys suffice unless the 64th still ties that p:
                // reduce up to 256 gathered keys to their top 64 in one wave
                // (registers, no barriers) and finish there; else the block
                // path below.
                if (tid < 64) {
                    unsigned long long q1 = tid + 64 < nc ? cload(&rs->cand[tid + 64]) : 0ull;
                    unsigned long long t = wave_top64(key, q1);
                    if (nc > 128) {
                        const unsigned long long q2 = tid + 128 < nc ? cload(&rs->cand[tid + 128]) : 0ull;
                        const unsigned long long q3 = tid + 192 < nc ? cload(&rs->cand[tid + 192]) : 0ull;
                        t = wave_top64(t, wave_top64(q2, q3));
                    }
                    const float thr = __builtin_bit_cast(float, rlu(static_cast<unsigned>(t >> 32), P.top_k - 1));
                    const bool fits = __builtin_bit_cast(float, rlu(static_cast<unsigned>(t >> 32), 63)) < thr;
                    const bool ok = fits && wave_tail(t, 64, P.top_k, P.top_p, use_k, use_p, r, o);
                    if (tid == 0) s.bi[2] = ok;
                }
                __syncthreads();
                done = s.bi[2];
                if (!done) {
                    for (int i = tid; i < nc; i += kT) s.u.cand[i] = cload(&rs->cand[i]);
                    __syncthreads();
                    n_list = replay_list(s, nc, P.top_k, P.top_p, use_k, use_p);
                }
            } else {
                for (int i = tid; i < nc; i += kT) s.u.cand[i] = cload(&rs->cand[i]);
                __syncthreads();
                n_list = replay_list(s, nc, P.top_k, P.top_p, use_k, use_p);
            }
        }
        if (!done) {
            if (n_list >= 0) {
                finish_list(s, n_list, r, o);
            } else {
                __threadfence();  // the general path reads prow with ordinary loads
                GlobalRow g;
                g.w = prow;
                g.n = n;
                general_tail(s, g, P.top_k, P.top_p, use_k, use_p, r, o);
            }
        }
        finish();
        return;
    }

    // ---- 6. no top-k / top-p: segment masses, then the segment holding r ------------------
    {
        float loc = 0.0f;
        int lastid = -1;
        st.visit([&](float p, int i) {
            loc += p;
            if (p > 0.0f) lastid = i;
        });
        loc = block_sum(s, loc);
        lastid = block_max_i(s, lastid);
        publish(rs, kPhSeg, w, tagf(loc, tag), tagi(lastid, tag), P.skip_seg);
    }
    gather(s, wt, rs, kPhSeg, S, tag);
    float sum2 = 0.0f, before = 0.0f;
    for (int v = 0; v < S; v++) {
        if (v == w) before = sum2;
        sum2 += s.pa[v];
    }
    // Every segment at or past the crossing scans itself; the smallest id found
    // wins.  (A crossing that rounding pushes past a segment's end is then
    // taken by the next segment's first id with mass; past the row's end, by
    // the last id with mass, as pick_by_mass does.)
    const float cum0 = before / sum2;
    const float mine = s.pa[w] / sum2;
    int first = INT_MAX;
    if (r <= cum0 + mine || w == S - 1) first = draw_scan_from(s, st, sum2, r, cum0);
    publish(rs, kPhDone, w, tagi(first, tag), tagi(0, tag), P.skip_seg);
    if (w != 0) return;
    // s.qb still holds every segment's last id with mass (gathered above)
    int lastg = -1;
    for (int v = 0; v < S; v++) lastg = max(lastg, s.qb[v]);
    __syncthreads();
    gather(s, wt, rs, kPhDone, S, tag);
    if (tid == 0) {
        int pick = INT_MAX;
        for (int v = 0; v < S; v++) pick = min(pick, s.qa[v]);
        *o = static_cast<uint32_t>(pick != INT_MAX ? pick : (lastg >= 0 ? lastg : 0));
    }
    finish();
}

template <int ITEMS>
int launch_split(fh_ctx* ctx, size_t rows, int S, const float* logits, const Params& P, const uint32_t* recent,
                 const uint32_t* offsets, const uint64_t* draws, uint32_t* out, void* sync, float* pbuf) {
    hipLaunchKernelGGL(k_sample_split<ITEMS>, dim3(static_cast<unsigned>(rows * S)), dim3(kT), 0, ctx->stream,
                       logits, P, recent, offsets, draws, out, static_cast<RowSync*>(sync), pbuf, S, ctx->status);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

template <int ITEMS>
int launch_regs(fh_ctx* ctx, size_t rows, const float* logits, const Params& P, const uint32_t* recent,
                const uint32_t* offsets, const uint64_t* draws, uint32_t* out) {
    hipLaunchKernelGGL(k_sample_regs<ITEMS>, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, ctx->stream, logits, P,
                       recent, offsets, draws, out, ctx->status);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}

}  // namespace

int fh_launch_sample(fh_ctx* ctx, const float* logits, size_t rows, size_t vocab, int kind,
                     const fh_sampling_params* p, const uint32_t* recent, const uint32_t* offsets,
                     const uint64_t* draws, uint32_t* out) {
    if (rows > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_sample_rows: too many rows");
    Params P;
    P.temperature = p->temperature;
    P.top_k = p->top_k > 0x7FFFFFFFu ? 0x7FFFFFFF : static_cast<int>(p->top_k);
    P.top_p = p->top_p;
    P.pen = p->repetition_penalty;
    P.kind = kind & ~FH_RECENT_RANGES;
    P.ranges = (kind & FH_RECENT_RANGES) != 0;
    P.n = static_cast<int>(vocab);
    P.spin_limit = ctx->test_spin_limit ? ctx->test_spin_limit : kSpinLimit;
    P.skip_seg = ctx->test_skip_segment;
    // Split rows over S workgroups while a launch's rows * S fit the device
    // at once: the occupancy API gives how many of the split kernel's
    // workgroups a CU holds (one: its LDS allows no more), so all workgroups
    // of a launch are resident together and their exchanges cannot wait on an
    // undispatched one.  For rows of at least 8192 ids, the fewest ids per
    // thread that fits all rows in one launch; when none does, consecutive
    // launches of as many rows as fit (fewest launches, at most 8), each row
    // keeping its own exchange slots.  (Fewer, fuller segments time worse:
    // the GPT-2-124M b1 step with 13 / 7 / 4 segments per row instead of 25
    // ran 0.2192 / 0.2244 / 0.2355 ms against 0.2169; the b32 step with 4
    // instead of 7, 0.682 against 0.672 ms.)
    const size_t items = (vocab + kT - 1) / kT;
    if (ctx->split_per_cu < 0) {  // the least over the instances below
        const void* ks[] = {reinterpret_cast<const void*>(k_sample_split<2>), reinterpret_cast<const void*>(k_sample_split<4>),
                            reinterpret_cast<const void*>(k_sample_split<8>), reinterpret_cast<const void*>(k_sample_split<16>),
                            reinterpret_cast<const void*>(k_sample_split<32>), reinterpret_cast<const void*>(k_sample_split<40>)};
        int least = 1 << 30;
        for (const void* k : ks) {
            int per = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, kT, 0) != hipSuccess) per = 0;
            least = per < least ? per : least;
        }
        ctx->split_per_cu = least;
    }
    if (vocab >= 8192 && rows <= 1024 && ctx->split_per_cu > 0) {
        // (40: a 151936-id row in four segments, so that 64 rows take one launch)
        static const int kOpts[] = {2, 4, 8, 16, 32, 40};
        const size_t cus = static_cast<size_t>(ctx->num_cus) * static_cast<size_t>(ctx->split_per_cu);
        int pick = 0;
        size_t pick_rows = 0, pick_launches = 9;
        for (int it : kOpts) {
            const size_t S = (vocab + static_cast<size_t>(kT) * it - 1) / (static_cast<size_t>(kT) * it);
            if (S < 2 || S > static_cast<size_t>(kSMax) || S > cus) continue;
            const size_t per = cus / S, launches = (rows + per - 1) / per;
            if (launches < pick_launches) {
                pick = it, pick_rows = per, pick_launches = launches;
                if (launches == 1) break;
            }
        }
        if (pick) {
            const size_t S = (vocab + static_cast<size_t>(kT) * pick - 1) / (static_cast<size_t>(kT) * pick);
            void* sync = nullptr;
            int rc = fh_sync_area(ctx, rows * sizeof(RowSync), &sync);
            if (rc) return rc;
            void* ws = nullptr;
            rc = fh_workspace(ctx, rows * vocab * sizeof(float), &ws);
            if (rc) return rc;
            const int s32 = static_cast<int>(S);
            for (size_t r0 = 0; r0 < rows; r0 += pick_rows) {
                const size_t nr = rows - r0 < pick_rows ? rows - r0 : pick_rows;
                const float* lg = logits + r0 * vocab;
                const uint32_t* of = offsets ? offsets + (P.ranges ? 2 * r0 : r0) : nullptr;
                const uint64_t* dr = draws ? draws + r0 : nullptr;
                void* sy = static_cast<RowSync*>(sync) + r0;
                float* pb = static_cast<float*>(ws) + r0 * vocab;
                switch (pick) {
                    case 2: rc = launch_split<2>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                    case 4: rc = launch_split<4>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                    case 8: rc = launch_split<8>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                    case 16: rc = launch_split<16>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                    case 32: rc = launch_split<32>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                    default: rc = launch_split<40>(ctx, nr, s32, lg, P, recent, of, dr, out + r0, sy, pb); break;
                }
                if (rc) return rc;
            }
            return FH_OK;
        }
    }
    if (items <= 1) return launch_regs<1>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 4) return launch_regs<4>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 16) return launch_regs<16>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 32) return launch_regs<32>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= kMaxItems) return launch_regs<kMaxItems>(ctx, rows, logits, P, recent, offsets, draws, out);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, rows * vocab * sizeof(float), &ws);
    if (rc) return rc;
    hipLaunchKernelGGL(k_sample_global, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, ctx->stream, logits, P, recent,
                       offsets, draws, out, static_cast<float*>(ws), ctx->status);
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
