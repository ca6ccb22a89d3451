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
// Parallel structure.  Steps 0-3 are block-wide passes over the row (kept in
// a per-row global buffer, L2-resident).  For steps 4-6 the kernel gathers the
// few elements that can survive into LDS: a 64-bucket histogram of the top 12
// bits of p (one octave = 8 buckets, counted only for the 8 octaves under the
// largest p) finds the bucket where the top-k count (or the top-p mass) is
// reached; every element at or above it is gathered (at most kCap), sorted by
// (p descending, index ascending) with a bitonic sort, and then one lane
// replays steps 4-6 sequentially in the reference's own order — so once the p
// values agree, the cum/top-p/renormalise/draw arithmetic is the reference's
// bit for bit.  Rows where that set would exceed kCap take a general path:
// an exact radix select for the top-k threshold, a radix select by mass
// (64-bit fixed-point, order-independent) for the top-p cut, and a block scan
// for the draw; those sums are parallel, so they may differ from the
// sequential f32 sums in the last bits (a near-tie only; see the tests).
// Every reduction has a fixed shape, so results never depend on timing.
#include <cfloat>

#include "fh_internal.hpp"

namespace {

constexpr int kT = 1024;        // threads per row
constexpr int kW = kT / 64;     // waves per row
constexpr int kCap = 4096;      // LDS survivor capacity
constexpr int kBuckets = 64;    // 8 octaves x 8 sub-buckets under the max p
constexpr int kSlots = 8192;    // repetition-penalty hash table
constexpr int kChunk = 4096;    // recent ids deduplicated per table fill
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr int kMaxRecent = 16384;

struct Shared {
    union {
        struct {
            uint32_t key[kSlots];
            uint32_t cnt[kSlots];
        } pen;
        struct {
            unsigned long long key[kCap];  // (bits(p) << 32) | ~index, sorted descending
        } cand;
    } u;
    uint32_t hist[256];
    unsigned long long mass[256];
    float redf[kW];
    int redi[kW];
    unsigned long long redu[kW];
    int bcast_i[4];
    float bcast_f[4];
    unsigned int n_cand;
};

__device__ __forceinline__ int total_key(float v) {
    int b = __builtin_bit_cast(int, v);
    return b ^ static_cast<int>(static_cast<unsigned>(b >> 31) >> 1);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Block reductions: a fixed tree (wave butterfly, then wave 0 over the kW
// partials), so the result is the same on every run.
__device__ float block_sum(Shared& s, float v) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s.redf[wv] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < kW; i++) r += s.redf[i];
    return r;
}
__device__ float block_max(Shared& s, float v) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s.redf[wv] = v;
    __syncthreads();
    float r = -INFINITY;
#pragma unroll
    for (int i = 0; i < kW; i++) r = fmaxf(r, s.redf[i]);
    return r;
}
__device__ int block_sum_i(Shared& s, int v) {
    v = wave_sum_i(v);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s.redi[wv] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int i = 0; i < kW; i++) r += s.redi[i];
    return r;
}
__device__ int block_min_i(Shared& s, int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s.redi[wv] = v;
    __syncthreads();
    int r = s.redi[0];
#pragma unroll
    for (int i = 1; i < kW; i++) r = min(r, s.redi[i]);
    return r;
}
__device__ int block_max_i(Shared& s, int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s.redi[wv] = v;
    __syncthreads();
    int r = s.redi[0];
#pragma unroll
    for (int i = 1; i < kW; i++) r = max(r, s.redi[i]);
    return r;
}
// Exclusive prefix over threads of a float, in thread order (wave scan then
// an LDS scan of the wave totals).  Returns this thread's exclusive prefix.
__device__ float block_exclusive_scan(Shared& s, float v, float* total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    float incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        float t = __shfl_up(incl, o, 64);
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

// Bitonic sort of s.u.cand.key[0..n2) descending, n2 a power of two.
__device__ void sort_desc(Shared& s, int n2) {
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < n2 / 2; t += kT) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                unsigned long long a = s.u.cand.key[lo], b = s.u.cand.key[hi];
                if ((a < b) == desc) {
                    s.u.cand.key[lo] = b;
                    s.u.cand.key[hi] = a;
                }
            }
        }
    }
    __syncthreads();
}

__device__ __forceinline__ unsigned long long cand_key(float p, int i) {
    return (static_cast<unsigned long long>(__builtin_bit_cast(uint32_t, p)) << 32) |
           static_cast<unsigned long long>(~static_cast<uint32_t>(i));
}
__device__ __forceinline__ float cand_p(unsigned long long key) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(key >> 32));
}
__device__ __forceinline__ int cand_i(unsigned long long key) {
    return static_cast<int>(~static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

// 12-bit bucket key of a non-negative float: 8 exponent bits and the top 3
// mantissa bits, so 8 buckets per octave.
__device__ __forceinline__ int key12(float p) { return static_cast<int>(__builtin_bit_cast(uint32_t, p) >> 20); }

// Radix select over the bit patterns of the non-negative w[i] (order of bits
// = order of values): the k-th largest value (1-based), exactly.
__device__ float radix_kth_largest(Shared& s, const float* w, int n, int k) {
    uint32_t prefix = 0, pmask = 0;
    int kr = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kT) s.hist[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kT) {
            const uint32_t u = __builtin_bit_cast(uint32_t, w[i]);
            if ((u & pmask) == prefix) atomicAdd(&s.hist[(u >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int above = 0, dg = 0;
            for (int d = 255; d >= 0; d--) {
                if (above + static_cast<int>(s.hist[d]) >= kr) {
                    dg = d;
                    break;
                }
                above += static_cast<int>(s.hist[d]);
            }
            s.bcast_i[0] = dg;
            s.bcast_i[1] = kr - above;
        }
        __syncthreads();
        prefix |= static_cast<uint32_t>(s.bcast_i[0]) << shift;
        pmask |= 255u << shift;
        kr = s.bcast_i[1];
        __syncthreads();
    }
    return __builtin_bit_cast(float, prefix);
}

// Fixed-point image of a probability, for order-independent mass sums.
__device__ __forceinline__ unsigned long long fix40(float p) {
    return static_cast<unsigned long long>(static_cast<double>(p) * 1099511627776.0 + 0.5);
}

// The top-p cut over all of w by mass, when too many elements would survive
// to sort in LDS: finds the largest value tau with mass(p >= tau) >= top_p
// (64-bit fixed point), then keeps p > tau and, of the p == tau ties, the
// lowest indices until the mass is reached.  Zeroes the rest in w.
__device__ void topp_by_mass(Shared& s, float* w, int n, float top_p) {
    const unsigned long long target = fix40(top_p);
    uint32_t prefix = 0, pmask = 0;
    unsigned long long above_mass = 0;
    bool found = true;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = threadIdx.x; i < 256; i += kT) s.mass[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kT) {
            const float p = w[i];
            const uint32_t u = __builtin_bit_cast(uint32_t, p);
            if (p > 0.0f && (u & pmask) == prefix) atomicAdd(&s.mass[(u >> shift) & 255u], fix40(p));
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long acc = above_mass;
            int dg = -1;
            for (int d = 255; d >= 0; d--) {
                if (acc + s.mass[d] >= target) {
                    dg = d;
                    break;
                }
                acc += s.mass[d];
            }
            s.bcast_i[0] = dg;
            s.redu[0] = acc;
        }
        __syncthreads();
        if (s.bcast_i[0] < 0) {  // the whole mass stays under top_p: keep everything
            found = false;
            __syncthreads();
            break;
        }
        prefix |= static_cast<uint32_t>(s.bcast_i[0]) << shift;
        pmask |= 255u << shift;
        above_mass = s.redu[0];
        __syncthreads();
    }
    if (!found) return;
    const float tau = __builtin_bit_cast(float, prefix);
    // Ties at tau: keep them in index order until above_mass + c * tau >= target.
    const unsigned long long ft = fix40(tau);
    const unsigned long long need = target > above_mass ? target - above_mass : 0;
    const long long keep_ties = ft ? static_cast<long long>((need + ft - 1) / ft) : 1;
    // Rank of each tie by index: per-thread contiguous segments, block scan.
    const int seg = (n + kT - 1) / kT;
    const int b0 = min(n, static_cast<int>(threadIdx.x) * seg), b1 = min(n, b0 + seg);
    int mine = 0;
    for (int i = b0; i < b1; i++) mine += w[i] == tau;
    float tot;
    int rank = static_cast<int>(block_exclusive_scan(s, static_cast<float>(mine), &tot));
    for (int i = b0; i < b1; i++) {
        const float p = w[i];
        if (p > tau) continue;
        if (p == tau) {
            if (rank >= keep_ties) w[i] = 0.0f;
            rank++;
        } else {
            w[i] = 0.0f;
        }
    }
    __syncthreads();
}

struct Params {
    float temperature;
    int top_k;
    float top_p;
    float pen;
    int kind;
    int n;
};

__global__ void __launch_bounds__(kT)
    k_sample(const float* __restrict__ logits, Params P, const uint32_t* __restrict__ recent,
             const uint32_t* __restrict__ offsets, const uint64_t* __restrict__ draws, uint32_t* __restrict__ out,
             float* __restrict__ work) {
    __shared__ Shared s;
    const int n = P.n;
    const size_t row = blockIdx.x;
    const float* z = logits + row * static_cast<size_t>(n);
    float* w = work + row * static_cast<size_t>(n);
    const int tid = threadIdx.x;

    // ---- 0. sampler input --------------------------------------------------------
    if (P.kind == FH_LOGITS_GPT2_SOFTMAX) {
        float m = -INFINITY;
        for (int i = tid; i < n; i += kT) m = fmaxf(m, z[i]);
        const float zmax = block_max(s, m);
        float sm = 0.0f;
        for (int i = tid; i < n; i += kT) sm += expf(z[i] - zmax);
        const float zsum = block_sum(s, sm);
        for (int i = tid; i < n; i += kT) w[i] = logf(fmaxf(expf(z[i] - zmax) / zsum, 1e-12f));
    } else {
        for (int i = tid; i < n; i += kT) w[i] = z[i];
    }
    __syncthreads();

    // ---- 1. repetition penalty ------------------------------------------------
    const float pen = P.pen;
    if (fabsf(pen - 1.0f) > FLT_EPSILON && pen > 0.0f && offsets && recent) {
        const uint32_t r0 = offsets[row], r1 = offsets[row + 1];
        const int nrec = r1 > r0 ? static_cast<int>(min(r1 - r0, static_cast<uint32_t>(kMaxRecent))) : 0;
        for (int base = 0; base < nrec; base += kChunk) {
            for (int i = tid; i < kSlots; i += kT) {
                s.u.pen.key[i] = kEmpty;
                s.u.pen.cnt[i] = 0;
            }
            __syncthreads();
            const int end = min(nrec, base + kChunk);
            for (int r = base + tid; r < end; r += kT) {
                const uint32_t tok = recent[r0 + r];
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
            for (int i = tid; i < kSlots; i += kT) {
                const uint32_t tok = s.u.pen.key[i];
                if (tok == kEmpty) continue;
                float l = w[tok];
                for (uint32_t c = s.u.pen.cnt[i]; c > 0; c--) l = l > 0.0f ? l / pen : l * pen;
                w[tok] = l;
            }
            __syncthreads();
        }
    }

    // ---- 2. greedy ---------------------------------------------------------------
    if (P.temperature <= 0.0f) {
        // Per thread: ascending indices, strict '>' keeps the first maximum.
        int bk = INT_MIN, bi = INT_MAX;
        if (tid < n) {
            bk = total_key(w[tid]);
            bi = tid;
        }
        for (int i = tid + kT; i < n; i += kT) {
            const int kk = total_key(w[i]);
            if (kk > bk) {
                bk = kk;
                bi = i;
            }
        }
        // the largest key, then the first index holding it
        int best = bk;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) best = max(best, __shfl_xor(best, o, 64));
        const int lane = tid & 63, wv = tid >> 6;
        __syncthreads();
        if (lane == 0) s.redi[wv] = best;
        __syncthreads();
        int gbest = s.redi[0];
        for (int i = 1; i < kW; i++) gbest = max(gbest, s.redi[i]);
        const int first = block_min_i(s, bk == gbest ? bi : INT_MAX);
        if (tid == 0) out[row] = static_cast<uint32_t>(first);
        return;
    }
    const float t = fmaxf(P.temperature, 0.01f);

    // ---- 3. temperature softmax --------------------------------------------------
    float m = -INFINITY;
    for (int i = tid; i < n; i += kT) m = fmaxf(m, w[i]);
    const float mx = block_max(s, m);
    float se = 0.0f;
    for (int i = tid; i < n; i += kT) {
        const float e = expf((w[i] - mx) / t);
        w[i] = e;
        se += e;
    }
    const float sum = block_sum(s, se);
    if (sum != sum || sum <= 1e-10f) {
        if (tid == 0) out[row] = static_cast<uint32_t>(draws[row] % static_cast<uint64_t>(n));
        return;
    }
    float pmax = 0.0f;
    for (int i = tid; i < n; i += kT) {
        const float p = w[i] / sum;
        w[i] = p;
        pmax = fmaxf(pmax, p);
    }
    pmax = block_max(s, pmax);
    const float r = static_cast<float>(draws[row] >> 40) / static_cast<float>(1u << 24);

    // ---- 4./5. top-k and top-p -------------------------------------------------------
    const bool use_k = P.top_k > 0 && P.top_k < n;
    const bool use_p = P.top_p < 1.0f;
    int n_list = -1;  // >= 0: survivors are s.u.cand.key[0..n_list), sorted by p desc
    if (use_k || use_p) {
        // Bucket histogram under the max p: count (top-k) and fixed-point mass (top-p).
        const int ktop = key12(pmax);
        for (int i = tid; i < kBuckets; i += kT) {
            s.hist[i] = 0;
            s.mass[i] = 0;
        }
        __syncthreads();
        for (int i = tid; i < n; i += kT) {
            const float p = w[i];
            const int b = ktop - key12(p);
            if (p > 0.0f && b < kBuckets) {
                atomicAdd(&s.hist[b], 1u);
                if (!use_k) atomicAdd(&s.mass[b], fix40(p));
            }
        }
        __syncthreads();
        if (tid == 0) {
            // Smallest bucket depth whose cumulative count reaches k (top-k) or
            // whose mass clears top_p by a margin of one more bucket (top-p only).
            int depth = -1, cnt = 0;
            unsigned long long acc = 0;
            const unsigned long long target = use_p ? fix40(P.top_p) : 0;
            for (int b = 0; b < kBuckets; b++) {
                cnt += static_cast<int>(s.hist[b]);
                acc += s.mass[b];
                if (use_k ? cnt >= P.top_k : acc >= target) {
                    depth = b;
                    break;
                }
            }
            if (depth >= 0 && !use_k && depth + 1 < kBuckets) {  // mass margin for the f32 replay
                depth++;
                cnt += static_cast<int>(s.hist[depth]);
            }
            s.bcast_i[0] = (depth >= 0 && cnt <= kCap) ? depth : -1;
            s.n_cand = 0;
        }
        __syncthreads();
        const int depth = s.bcast_i[0];
        if (depth >= 0) {
            for (int i = tid; i < n; i += kT) {
                const float p = w[i];
                if (p > 0.0f && ktop - key12(p) <= depth) {
                    const unsigned slot = atomicAdd(&s.n_cand, 1u);
                    s.u.cand.key[slot] = cand_key(p, i);
                }
            }
            __syncthreads();
            const int nc = static_cast<int>(s.n_cand);
            int n2 = 1;
            while (n2 < nc) n2 <<= 1;
            for (int i = nc + tid; i < n2; i += kT) s.u.cand.key[i] = 0ull;  // p = 0 sorts last
            sort_desc(s, n2);
            if (tid == 0) {
                int len = nc;
                bool ok = true;
                if (use_k) {
                    const float thr = cand_p(s.u.cand.key[P.top_k - 1]);
                    len = P.top_k;
                    while (len < nc && cand_p(s.u.cand.key[len]) >= thr) len++;
                }
                if (use_p) {
                    float cum = 0.0f;
                    int c = 0;
                    bool crossed = false;
                    for (; c < len; c++) {
                        cum += cand_p(s.u.cand.key[c]);
                        if (cum >= P.top_p) {
                            crossed = true;
                            break;
                        }
                    }
                    if (crossed) len = c + 1;
                    else if (!use_k) ok = false;  // the cut lies below the gathered set
                }
                s.bcast_i[1] = ok ? len : -1;
            }
            __syncthreads();
            n_list = s.bcast_i[1];
            __syncthreads();
        }
        if (n_list < 0) {
            // General path: exact top-k threshold, then the top-p cut by mass.
            if (use_k) {
                const float thr = radix_kth_largest(s, w, n, P.top_k);
                for (int i = tid; i < n; i += kT)
                    if (w[i] < thr) w[i] = 0.0f;
                __syncthreads();
            }
            if (use_p) topp_by_mass(s, w, n, P.top_p);
        }
    }

    // ---- 6. renormalise and draw -------------------------------------------------
    if (n_list >= 0) {
        // Survivors back into index order; one lane replays the reference's loop.
        if (tid == 0) {
            for (int i = 0; i < n_list; i++) {
                const unsigned long long kk = s.u.cand.key[i];
                s.u.cand.key[i] = (static_cast<unsigned long long>(~static_cast<uint32_t>(cand_i(kk))) << 32) |
                                  (kk >> 32);
            }
            s.bcast_i[2] = n_list;
        }
        __syncthreads();
        int n2 = 1;
        while (n2 < n_list) n2 <<= 1;
        for (int i = n_list + tid; i < n2; i += kT) s.u.cand.key[i] = 0ull;
        sort_desc(s, n2);  // descending ~index = ascending index
        if (tid == 0) {
            float sum2 = 0.0f;
            for (int i = 0; i < n_list; i++) sum2 += __builtin_bit_cast(float, static_cast<uint32_t>(s.u.cand.key[i]));
            float cumsum = 0.0f;
            int pick = -1, last = 0;
            for (int i = 0; i < n_list; i++) {
                const unsigned long long kk = s.u.cand.key[i];
                const float p = __builtin_bit_cast(float, static_cast<uint32_t>(kk)) / sum2;
                const int idx = static_cast<int>(~static_cast<uint32_t>(kk >> 32));
                if (p > 0.0f) {
                    last = idx;
                    cumsum += p;
                    if (r <= cumsum) {
                        pick = idx;
                        break;
                    }
                }
            }
            out[row] = static_cast<uint32_t>(pick >= 0 ? pick : last);
        }
        return;
    }
    // Block-wide: sum2, then the first index whose running mass reaches r.
    float s2 = 0.0f;
    for (int i = tid; i < n; i += kT) s2 += w[i];
    const float sum2 = block_sum(s, s2);
    const int seg = (n + kT - 1) / kT;
    const int b0 = min(n, tid * seg), b1 = min(n, b0 + seg);
    float local = 0.0f;
    int last = -1;
    for (int i = b0; i < b1; i++) {
        const float p = w[i] / sum2;
        if (p > 0.0f) {
            local += p;
            last = i;
        }
    }
    float total;
    float cum = block_exclusive_scan(s, local, &total);
    int pick = INT_MAX;
    for (int i = b0; i < b1; i++) {
        const float p = w[i] / sum2;
        if (p > 0.0f) {
            cum += p;
            if (r <= cum) {
                pick = i;
                break;
            }
        }
    }
    const int first = block_min_i(s, pick);
    const int lastg = block_max_i(s, last);
    if (tid == 0) out[row] = static_cast<uint32_t>(first != INT_MAX ? first : (lastg >= 0 ? lastg : 0));
}

}  // namespace

int fh_launch_sample(fh_ctx* ctx, const float* logits, size_t rows, size_t vocab, int kind,
                     const fh_sampling_params* p, const uint32_t* recent, const uint32_t* offsets,
                     const uint64_t* draws, uint32_t* out) {
    if (rows > 0x7FFFFFFFu) return fh_fail(ctx, FH_ERR_LIMIT, "fh_sample_rows: too many rows");
    void* ws = nullptr;
    int rc = fh_workspace(ctx, rows * vocab * sizeof(float), &ws);
    if (rc) return rc;
    Params P;
    P.temperature = p->temperature;
    P.top_k = p->top_k > 0x7FFFFFFFu ? 0x7FFFFFFF : static_cast<int>(p->top_k);
    P.top_p = p->top_p;
    P.pen = p->repetition_penalty;
    P.kind = kind;
    P.n = static_cast<int>(vocab);
    hipLaunchKernelGGL(k_sample, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, ctx->stream, logits, P, recent,
                       offsets, draws, out, static_cast<float*>(ws));
    FH_HIP(ctx, hipGetLastError());
    return FH_OK;
}
