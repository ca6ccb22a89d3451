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
// Steps 4-6.  A 64-bucket histogram of the top 12 bits of p (8 buckets per
// octave, the 8 octaves under the largest p) finds the bucket where the top-k
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

namespace {

constexpr int kT = 1024;        // threads per row
constexpr int kW = kT / 64;     // waves per row
constexpr int kCap = 4096;      // LDS survivor capacity
constexpr int kBuckets = 64;    // 8 octaves x 8 sub-buckets under the max p
constexpr int kCopies = 16;     // histogram copies (lane & 15) against same-bin conflicts
constexpr int kSlots = 8192;    // repetition-penalty hash table
constexpr int kChunk = 4096;    // recent ids deduplicated per table fill
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr int kMaxRecent = 16384;
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
    float slab[kW][kMaxItems];
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

// Register-resident row: thread t holds ids t + j * kT, j < ITEMS.
template <int ITEMS>
struct RegRow {
    static constexpr bool kRegs = true;
    float v[ITEMS];
    int n;
    __device__ __forceinline__ void load(const float* __restrict__ src) {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = threadIdx.x + j * kT;
            v[j] = i < n ? src[i] : 0.0f;
        }
    }
    template <class F>
    __device__ __forceinline__ void map(F f) {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = threadIdx.x + j * kT;
            if (i < n) v[j] = f(v[j], i);
        }
    }
    template <class F>
    __device__ __forceinline__ void visit(F f) const {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const int i = threadIdx.x + j * kT;
            if (i < n) f(v[j], i);
        }
    }
};

// Global-buffer row for vocabularies beyond the register file: same id-to-thread
// mapping, streamed eight ids per thread at a time.
struct GlobalRow {
    static constexpr bool kRegs = false;
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

// The first id in index order whose running mass of p / sum2 reaches r (the
// last id with mass if none does): register rows scan slab by slab (slab j =
// ids [j * kT, (j + 1) * kT)), global rows by contiguous per-thread segments.
template <int ITEMS>
__device__ __forceinline__ int draw_scan(Shared& s, const RegRow<ITEMS>& row, float sum2, float r) {
    const int lane = lane_id(), wv = wave_id();
    // per-slab totals: wave sums, then over waves in wave order
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const int i = threadIdx.x + j * kT;
        const float q = (i < row.n && row.v[j] > 0.0f) ? row.v[j] / sum2 : 0.0f;
        const float t = wave_sum(q);
        if (lane == 0) s.slab[wv][j] = t;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float cum = 0.0f;
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
    if (js >= 0) {
        float q = 0.0f;
        int mine = -1;
#pragma unroll
        for (int j = 0; j < ITEMS; j++)
            if (j == js) {
                const int i = threadIdx.x + j * kT;
                if (i < row.n && row.v[j] > 0.0f) {
                    q = row.v[j] / sum2;
                    mine = i;
                }
            }
        float total;
        const float before = block_exclusive_scan(s, q, &total);
        const bool hit = mine >= 0 && r <= base + before + q;
        const int first = block_min_i(s, hit ? mine : INT_MAX);
        if (first != INT_MAX) return first;
    }
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

struct Params {
    float temperature;
    int top_k;
    float top_p;
    float pen;
    int kind;
    int n;
};

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

    // ---- 4./5. top-k and top-p ------------------------------------------------------------
    const bool use_k = P.top_k > 0 && P.top_k < n;
    const bool use_p = P.top_p < 1.0f;
    int n_list = -1;  // >= 0: the survivors are s.u.cand[0..n_list), p descending
    if (use_k || use_p) {
        const int ktop = key12(pmax);
        const int copy = tid & (kCopies - 1);
        for (int i = tid; i < kCopies * kBuckets; i += kT) {
            (&s.hist[0][0])[i] = 0;
            (&s.mass[0][0])[i] = 0;
        }
        __syncthreads();
        row.visit([&](float p, int) {
            const int b = ktop - key12(p);
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
        if (tid == 0) {
            // The shallowest bucket depth whose cumulative count reaches k (top-k)
            // or whose mass reaches top_p, plus one bucket of margin (top-p only).
            int depth = -1, cnt = 0;
            unsigned long long acc = 0;
            const unsigned long long target = use_p ? fix40(P.top_p) : 0;
            for (int b = 0; b < kBuckets; b++) {
                cnt += static_cast<int>(s.hist[0][b]);
                acc += s.mass[0][b];
                if (use_k ? cnt >= P.top_k : acc >= target) {
                    depth = b;
                    break;
                }
            }
            if (depth >= 0 && !use_k && depth + 1 < kBuckets) {
                depth++;
                cnt += static_cast<int>(s.hist[0][depth]);
            }
            s.bi[0] = (depth >= 0 && cnt <= kCap) ? depth : -1;
            s.n_cand = 0;
        }
        __syncthreads();
        const int depth = s.bi[0];
        if (depth >= 0) {
            row.visit([&](float p, int i) { append(s, p > 0.0f && ktop - key12(p) <= depth, cand_key(p, i)); });
            // RegRow::visit skips ids >= n per item, so append's ballot may run
            // with some lanes inactive; the list is complete after the barrier.
            __syncthreads();
            const int nc = static_cast<int>(s.n_cand);
            int n2 = 1;
            while (n2 < nc) n2 <<= 1;
            for (int i = nc + tid; i < n2; i += kT) s.u.cand[i] = 0ull;  // p = 0 sorts last
            sort_desc(s, n2);
            if (tid < 64) {  // wave 0 replays top-k / top-p in the reference's order
                int len = nc;
                bool ok = true;
                if (use_k) {
                    const float thr = key_p(s.u.cand[P.top_k - 1]);
                    len = P.top_k;
                    while (len < nc && key_p(s.u.cand[len]) >= thr) len++;
                }
                if (use_p) {
                    float cum = 0.0f;
                    bool crossed = false;
                    int c = 0;
                    for (; c < len; c++) {
                        cum += key_p(s.u.cand[c]);
                        if (cum >= P.top_p) {
                            crossed = true;
                            break;
                        }
                    }
                    if (crossed) len = c + 1;
                    else if (!use_k) ok = false;  // the cut lies below the gathered set
                }
                if (tid == 0) s.bi[1] = ok ? len : -1;
            }
            __syncthreads();
            n_list = s.bi[1];
            __syncthreads();
        }
        if (n_list < 0) {
            if (use_k) {
                const float thr = radix_kth_largest(s, row, P.top_k);
                row.map([&](float p, int) { return p < thr ? 0.0f : p; });
                __syncthreads();
            }
            if (use_p) topp_by_mass(s, row, P.top_p);
        }
    }

    // ---- 6. renormalise and draw -------------------------------------------------------
    if (n_list >= 0) {
        // survivors back into index order: key (~index << 32) | bits(p), descending
        for (int i = tid; i < n_list; i += kT) {
            const unsigned long long k = s.u.cand[i];
            s.u.cand[i] = (static_cast<unsigned long long>(~static_cast<uint32_t>(key_i(k))) << 32) | (k >> 32);
        }
        int n2 = 1;
        while (n2 < n_list) n2 <<= 1;
        for (int i = n_list + tid; i < n2; i += kT) s.u.cand[i] = 0ull;
        sort_desc(s, n2);
        if (tid < 64) {  // wave 0: sum2, then pick_by_mass, sequentially in index order
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
        return;
    }
    float s2 = 0.0f;
    row.visit([&](float p, int) { s2 += p; });
    const float sum2 = block_sum(s, s2);
    const int pick = draw_scan(s, row, sum2, r);
    if (tid == 0) *out = static_cast<uint32_t>(pick);
}

template <int ITEMS>
__global__ void __launch_bounds__(kT)
    k_sample_regs(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
                  const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws,
                  uint32_t* __restrict__ out) {
    __shared__ Shared s;
    const size_t row = blockIdx.x;
    int nrec = 0;
    const uint32_t* rec = nullptr;
    if (offsets && recent) {
        const uint32_t r0 = offsets[row], r1 = offsets[row + 1];
        nrec = r1 > r0 ? static_cast<int>(min(r1 - r0, static_cast<uint32_t>(kMaxRecent))) : 0;
        rec = recent + r0;
    }
    RegRow<ITEMS> st;
    st.n = P.n;
    const bool has_draw = draws != nullptr;
    sample_row(s, st, P, logits + row * static_cast<size_t>(P.n), rec, nrec, has_draw ? draws[row] : 0ull,
               has_draw, out + row);
}

__global__ void __launch_bounds__(kT)
    k_sample_global(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
                    const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws,
                    uint32_t* __restrict__ out, float* __restrict__ work) {
    __shared__ Shared s;
    const size_t row = blockIdx.x;
    int nrec = 0;
    const uint32_t* rec = nullptr;
    if (offsets && recent) {
        const uint32_t r0 = offsets[row], r1 = offsets[row + 1];
        nrec = r1 > r0 ? static_cast<int>(min(r1 - r0, static_cast<uint32_t>(kMaxRecent))) : 0;
        rec = recent + r0;
    }
    GlobalRow st;
    st.n = P.n;
    st.w = work + row * static_cast<size_t>(P.n);
    const bool has_draw = draws != nullptr;
    sample_row(s, st, P, logits + row * static_cast<size_t>(P.n), rec, nrec, has_draw ? draws[row] : 0ull,
               has_draw, out + row);
}

template <int ITEMS>
int launch_regs(fh_ctx* ctx, size_t rows, const float* logits, const Params& P, const uint32_t* recent,
                const uint32_t* offsets, const uint64_t* draws, uint32_t* out) {
    hipLaunchKernelGGL(k_sample_regs<ITEMS>, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, ctx->stream, logits, P,
                       recent, offsets, draws, out);
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
    P.kind = kind;
    P.n = static_cast<int>(vocab);
    const size_t items = (vocab + kT - 1) / kT;
    if (items <= 1) return launch_regs<1>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 4) return launch_regs<4>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 16) return launch_regs<16>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= 32) return launch_regs<32>(ctx, rows, logits, P, recent, offsets, draws, out);
    if (items <= kMaxItems) return launch_regs<kMaxItems>(ctx, rows, logits, P, recent, offsets, draws, out);
    void* ws = nullptr;
    int rc = fh_workspace(ctx, rows * vocab * sizeof(float), &ws);
    if (rc) return rc;
    hipLaunchKernelGGL(k_sample_global, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, ctx->stream, logits, P, recent,
                       offsets, draws, out, static_cast<float*>(ws));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
