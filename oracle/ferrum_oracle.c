/*
 * ferrum_oracle.c — CPU restatement of ferrum_core's Q8_0 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline ("port") of bench.py.  Nothing in the product library links or calls
 * this file.  Build: oracle/Makefile (-O3 -ffp-contract=off, no fast-math, the
 * default x86-64 ISA like a default `cargo build --release`).
 *
 * Each function follows the reference file:line given in ferrum_oracle.h.  The
 * reference is pure Rust and cannot be built here (no Rust toolchain), so this
 * restatement is pinned by the reference's own known-answer tests, re-encoded
 * under tests/, and by library/closed-form checks (numpy's IEEE half cast,
 * numpy's sequential float32 cumsum, brute force on small inputs).
 */
#define _GNU_SOURCE
#include "ferrum_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* IEEE half codec                                                           */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

/* gguf_write/blocks.rs:12-61 */
uint16_t fo_f32_to_f16(float value) {
    uint32_t x = f32_bits(value);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int32_t exp32 = (int32_t)((x >> 23) & 0xFFu);
    uint32_t mant32 = x & 0x007FFFFFu;
    if (exp32 == 0xFF) return mant32 != 0 ? (uint16_t)(sign | 0x7E00u) : (uint16_t)(sign | 0x7C00u);
    int32_t exp16 = exp32 - 127 + 15;
    if (exp16 >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (exp16 <= 0) {
        if (exp16 < -10) return sign;
        uint32_t mant = mant32 | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - exp16); /* 14..24 */
        uint32_t half = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half & 1u) == 1u)) half += 1u;
        return (uint16_t)(sign | (uint16_t)half);
    }
    uint16_t mant16 = (uint16_t)(mant32 >> 13);
    uint32_t rem = mant32 & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (mant16 & 1u) == 1u)) {
        mant16 = (uint16_t)(mant16 + 1u);
        if (mant16 == 0x0400u) {
            mant16 = 0;
            exp16 += 1;
            if (exp16 >= 0x1F) return (uint16_t)(sign | 0x7C00u);
        }
    }
    return (uint16_t)(sign | (uint16_t)((uint32_t)exp16 << 10) | mant16);
}

/* gguf/dequant.rs:7-35 */
float fo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)((h >> 15) & 1u);
    int32_t exp = (int32_t)((h >> 10) & 0x1Fu);
    uint32_t mant = (uint32_t)(h & 0x3FFu);
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t m = mant;
            int32_t e = -14;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(e + 127) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    }
    return bits_f32(bits);
}

void fo_f32_to_f16_n(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = fo_f32_to_f16(x[i]);
}

void fo_f16_to_f32_n(const uint16_t* h, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = fo_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                       */
/* ------------------------------------------------------------------------ */

/* Rust `f32::round(v) as i8`: half away from zero, saturating, NaN -> 0. */
static int8_t round_sat_i8(float v) {
    float r = roundf(v);
    if (isnan(r)) return 0;
    if (r >= 127.0f) return 127;
    if (r <= -128.0f) return -128;
    return (int8_t)r;
}

/* quant.rs:271-280 */
void fo_q8_0_block(const float* x, uint16_t* d16, int8_t* q) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i])); /* f32::max ignores NaN */
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) q[i] = round_sat_i8(x[i] * id);
    *d16 = fo_f32_to_f16(d);
}

/* gguf_write/blocks.rs:65-92 (length check), 132-140 */
int fo_q8_0_encode(const float* data, size_t n, uint8_t* out) {
    if (n % 32 != 0) return -1;
    for (size_t b = 0; b < n / 32; b++) {
        uint16_t d16;
        int8_t q[32];
        fo_q8_0_block(data + b * 32, &d16, q);
        out[b * 34 + 0] = (uint8_t)(d16 & 0xFFu);
        out[b * 34 + 1] = (uint8_t)(d16 >> 8);
        memcpy(out + b * 34 + 2, q, 32);
    }
    return 0;
}

static float q8_0_weight(const uint8_t* blk, int t) {
    uint16_t d16 = (uint16_t)(blk[0] | ((uint16_t)blk[1] << 8));
    return fo_f16_to_f32(d16) * (float)(int8_t)blk[2 + t];
}

/* gguf/dequant.rs:37-49 */
int fo_q8_0_dequant(const uint8_t* raw, size_t raw_len, size_t n, float* out) {
    size_t nb = n / 32;
    if (raw_len < nb * 34) return -1;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = raw + b * 34;
        for (int t = 0; t < 32; t++) out[b * 32 + (size_t)t] = q8_0_weight(blk, t);
    }
    return 0;
}

/* quant.rs:283-291 */
static void snap_block(float* x) {
    uint16_t d16;
    int8_t q[32];
    fo_q8_0_block(x, &d16, q);
    float d = fo_f16_to_f32(d16);
    for (int i = 0; i < 32; i++) x[i] = (float)q[i] * d;
}

/* quant.rs:298-305 */
void fo_fake_quantize_q8_0_rows(float* data, size_t len, size_t ne0) {
    if (ne0 == 0 || ne0 % 32 != 0) return;
    for (size_t b = 0; b + 32 <= len; b += 32) snap_block(data + b);
}

/* quant.rs:309-325 */
void fo_fake_quantize_q8_0_cols(float* data, size_t rows_in, size_t cols_out) {
    if (rows_in == 0 || rows_in % 32 != 0) return;
    float buf[32];
    for (size_t j = 0; j < cols_out; j++) {
        for (size_t i0 = 0; i0 < rows_in; i0 += 32) {
            for (size_t t = 0; t < 32; t++) buf[t] = data[(i0 + t) * cols_out + j];
            snap_block(buf);
            for (size_t t = 0; t < 32; t++) data[(i0 + t) * cols_out + j] = buf[t];
        }
    }
}

/* gguf/tensors.rs:58-87 + gguf/llama.rs:342-350 */
int fo_q8_0_to_ferrum_weight(const uint8_t* raw, size_t n_rows, size_t k, float* w_kn) {
    if (k % 32 != 0) return -1;
    size_t row_bytes = k / 32 * 34;
    for (size_t r = 0; r < n_rows; r++) {
        const uint8_t* row = raw + r * row_bytes;
        for (size_t p = 0; p < k; p++) w_kn[p * n_rows + r] = q8_0_weight(row + (p / 32) * 34, (int)(p % 32));
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Linear layer: ops.rs:29-256 with the parallel.rs row split                 */
/* ------------------------------------------------------------------------ */

enum { KC = 256, NC = 256, MR = 4, NR = 8 };

/* ops.rs:99-126 */
static void edge_rows(const float* a, const float* b, size_t k, size_t n, size_t ia, size_t ib,
                      size_t r0, size_t ja, size_t jb, size_t pp, size_t p1, float* out) {
    for (size_t i = ia; i < ib; i++) {
        const float* arow = a + i * k;
        float* o = out + (i - r0) * n;
        for (size_t p = pp; p < p1; p++) {
            float aip = arow[p];
            const float* brow = b + p * n;
            for (size_t j = ja; j < jb; j++) o[j] += aip * brow[j];
        }
    }
}

/* ops.rs:63-94 */
static void micro_tile(const float* a, const float* b, size_t k, size_t n, size_t i, size_t r0,
                       size_t j, size_t pp, size_t p1, float* out) {
    float acc[MR][NR];
    for (int r = 0; r < MR; r++)
        for (int c = 0; c < NR; c++) acc[r][c] = out[(i + (size_t)r - r0) * n + j + (size_t)c];
    for (size_t p = pp; p < p1; p++) {
        const float* bs = b + p * n + j;
        for (int r = 0; r < MR; r++) {
            float av = a[(i + (size_t)r) * k + p];
            for (int c = 0; c < NR; c++) acc[r][c] += av * bs[c];
        }
    }
    for (int r = 0; r < MR; r++)
        for (int c = 0; c < NR; c++) out[(i + (size_t)r - r0) * n + j + (size_t)c] = acc[r][c];
}

/* ops.rs:29-55 */
static void matmul_block(const float* a, const float* b, size_t k, size_t n, size_t r0, size_t r1,
                         float* out) {
    for (size_t jj = 0; jj < n;) {
        size_t j1 = jj + NC < n ? jj + NC : n;
        for (size_t pp = 0; pp < k;) {
            size_t p1 = pp + KC < k ? pp + KC : k;
            size_t i = r0;
            for (; i + MR <= r1; i += MR) {
                size_t j = jj;
                for (; j + NR <= j1; j += NR) micro_tile(a, b, k, n, i, r0, j, pp, p1, out);
                if (j < j1) edge_rows(a, b, k, n, i, i + MR, r0, j, j1, pp, p1, out);
            }
            if (i < r1) edge_rows(a, b, k, n, i, r1, r0, jj, j1, pp, p1, out);
            pp = p1;
        }
        jj = j1;
    }
}

/* ops.rs:132-148 */
static void matmul_bias_block(const float* a, const float* b, const float* bias, size_t k, size_t n,
                              size_t r0, size_t r1, float* block) {
    matmul_block(a, b, k, n, r0, r1, block);
    if (bias && n > 0)
        for (size_t i = r0; i < r1; i++) {
            float* row = block + (i - r0) * n;
            for (size_t j = 0; j < n; j++) row[j] += bias[j];
        }
}

typedef struct {
    const float *a, *b, *bias;
    size_t k, n, r0, r1;
    float* out;
} row_job;

static void* row_job_run(void* arg) {
    row_job* j = (row_job*)arg;
    matmul_bias_block(j->a, j->b, j->bias, j->k, j->n, j->r0, j->r1, j->out + j->r0 * j->n);
    return NULL;
}

int fo_linear_forward(const float* x, size_t m, size_t k, const float* w_kn, size_t n,
                      const float* bias, float* y, int threads) {
    memset(y, 0, m * n * sizeof(float));
    size_t cost = m * k * n;
    /* parallel.rs:90-92: rows >= 2 && cost >= 1<<16 && threads > 1 */
    if (threads <= 1 || m < 2 || cost < (1u << 16)) {
        matmul_bias_block(x, w_kn, bias, k, n, 0, m, y);
        return 0;
    }
    size_t t = (size_t)threads < m ? (size_t)threads : m;
    size_t rows_per = (m + t - 1) / t; /* parallel.rs:190, 280 */
    row_job jobs[256];
    pthread_t tids[256];
    size_t nj = 0;
    for (size_t r0 = 0; r0 < m && nj < 256; r0 += rows_per) {
        jobs[nj] = (row_job){x, w_kn, bias, k, n, r0, r0 + rows_per < m ? r0 + rows_per : m, y};
        nj++;
    }
    int started[256];
    for (size_t i = 1; i < nj; i++) started[i] = pthread_create(&tids[i], NULL, row_job_run, &jobs[i]) == 0;
    row_job_run(&jobs[0]);
    for (size_t i = 1; i < nj; i++) {
        if (started[i])
            pthread_join(tids[i], NULL);
        else
            row_job_run(&jobs[i]); /* parallel.rs:285-291: a failed spawn leaves its share to the caller */
    }
    return 0;
}

int fo_q8_0_linear_rows(const float* x, size_t m, size_t k, const uint8_t* raw, size_t n,
                        const float* bias, float* y) {
    if (k % 32 != 0) return -1;
    size_t row_bytes = k / 32 * 34;
    for (size_t i = 0; i < m; i++) {
        const float* xr = x + i * k;
        for (size_t j = 0; j < n; j++) {
            const uint8_t* row = raw + j * row_bytes;
            float acc = 0.0f;
            for (size_t b = 0; b < k / 32; b++) {
                const uint8_t* blk = row + b * 34;
                float d = fo_f16_to_f32((uint16_t)(blk[0] | ((uint16_t)blk[1] << 8)));
                for (int t = 0; t < 32; t++) {
                    float w = d * (float)(int8_t)blk[2 + t];
                    acc += xr[b * 32 + (size_t)t] * w;
                }
            }
            if (bias) acc += bias[j];
            y[i * n + j] = acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Packed per-row int8 / int4 weights: QWeight and ops::qlinear               */
/* ------------------------------------------------------------------------ */

/* f32 -> integer level as Rust's `(v * inv).round().clamp(-lim, lim) as i8/i32`:
 * round half away from zero, saturating, NaN -> 0. */
static int q_level(float v, float lim) {
    if (v != v) return 0;
    float r = roundf(v);
    if (r < -lim) r = -lim;
    if (r > lim) r = lim;
    return (int)r;
}

/* quant.rs:17-19 int8_scale / the int4 amax: fold max(abs) from 0 (NaN ignored). */
static float row_amax(const float* row, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(row[i]);
        if (a > m) m = a; /* a NaN compares false: skipped, as f32::max does */
    }
    return m;
}

size_t fo_qweight_row_bytes(size_t cols, int kind) { return kind == 0 ? cols : (cols + 1) / 2; }

void fo_qweight_from_f32(const float* data, size_t rows, size_t cols, int kind, float* scales, uint8_t* q) {
    size_t rb = fo_qweight_row_bytes(cols, kind), half = (cols + 1) / 2;
    memset(q, 0, rows * rb);
    for (size_t r = 0; r < rows; r++) {
        const float* row = data + r * cols;
        float scale = row_amax(row, cols) / (kind == 0 ? 127.0f : 7.0f);
        scales[r] = scale;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        uint8_t* dst = q + r * rb;
        for (size_t c = 0; c < cols; c++) {
            if (kind == 0) {
                dst[c] = (uint8_t)(int8_t)q_level(row[c] * inv, 127.0f);
            } else {
                uint8_t nib = (uint8_t)(q_level(row[c] * inv, 7.0f) & 0x0F);
                if (c < half)
                    dst[c] = (uint8_t)((dst[c] & 0xF0) | nib);
                else
                    dst[c - half] = (uint8_t)((dst[c - half] & 0x0F) | (nib << 4));
            }
        }
    }
}

static float qweight_level(const uint8_t* row, size_t c, size_t half, int kind) {
    if (kind == 0) return (float)(int8_t)row[c];
    uint8_t nib = c < half ? (uint8_t)(row[c] & 0x0F) : (uint8_t)(row[c - half] >> 4);
    return (float)(int8_t)((int8_t)(nib << 4) >> 4); /* quant.rs:222-225 nibble_to_i8 */
}

void fo_qweight_to_f32(const float* scales, const uint8_t* q, size_t rows, size_t cols, int kind, float* out) {
    size_t rb = fo_qweight_row_bytes(cols, kind), half = (cols + 1) / 2;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = qweight_level(q + r * rb, c, half, kind) * scales[r];
}

/* ops.rs:268-305 qaccum_cols: out[j - j0] += a[p] * level(p, j), p ascending.
 * Int8 walks each weight row as one contiguous i8 run; int4 as the two
 * contiguous nibble lanes of the split-half layout (a low-nibble pass over
 * [j0, min(j1, half)), a high-nibble pass over [max(j0, half), j1)), the same
 * order and arithmetic, written so the compiler vectorises them. */
static void qaccum_cols(const float* a, size_t k, const uint8_t* q, size_t cols, int kind, size_t j0, size_t j1,
                        float* out) {
    size_t rb = fo_qweight_row_bytes(cols, kind), half = (cols + 1) / 2;
    for (size_t p = 0; p < k; p++) {
        const uint8_t* row = q + p * rb;
        const float ap = a[p];
        if (kind == 0) {
            const int8_t* r8 = (const int8_t*)row;
            for (size_t j = j0; j < j1; j++) out[j - j0] += ap * (float)r8[j];
        } else {
            size_t lo_end = j1 < half ? j1 : half, hi_start = j0 > half ? j0 : half;
            for (size_t j = j0; j < lo_end; j++) out[j - j0] += ap * (float)(int8_t)((int8_t)(row[j] << 4) >> 4);
            for (size_t j = hi_start; j < j1; j++) out[j - j0] += ap * (float)((int8_t)row[j - half] >> 4);
        }
    }
}

/* A persistent worker pool, as the reference keeps one (parallel.rs:94-166):
 * workers are created once and wait on a condition variable; a parallel call
 * hands job i to worker i - 1 and runs job 0 itself.  The partition (and so
 * the result) is the caller's; the pool only saves creating threads per call. */
typedef void* (*pool_fn)(void*);
static struct {
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    pthread_t tids[256];
    int n;                 /* workers started */
    unsigned long gen;     /* bumps once per dispatch */
    int pending;
    pool_fn fn;
    char* args;
    size_t stride;
    int njobs;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};

static void* pool_worker(void* arg) {
    const int id = (int)(intptr_t)arg; /* runs job id + 1 */
    unsigned long seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.gen == seen) pthread_cond_wait(&g_pool.go, &g_pool.mu);
        seen = g_pool.gen;
        if (id + 1 < g_pool.njobs) {
            pool_fn fn = g_pool.fn;
            void* a = g_pool.args + (size_t)(id + 1) * g_pool.stride;
            pthread_mutex_unlock(&g_pool.mu);
            fn(a);
            pthread_mutex_lock(&g_pool.mu);
            if (--g_pool.pending == 0) pthread_cond_signal(&g_pool.done);
        }
    }
    return NULL;
}

/* Run fn over njobs job records (stride bytes apart); returns when all are done. */
static void pool_run(pool_fn fn, void* args, size_t stride, int njobs) {
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.n < njobs - 1 && g_pool.n < 256) {
        if (pthread_create(&g_pool.tids[g_pool.n], NULL, pool_worker, (void*)(intptr_t)g_pool.n) != 0) break;
        pthread_detach(g_pool.tids[g_pool.n]);
        g_pool.n++;
    }
    int remote = njobs - 1 < g_pool.n ? njobs - 1 : g_pool.n;
    g_pool.fn = fn;
    g_pool.args = (char*)args;
    g_pool.stride = stride;
    g_pool.njobs = remote + 1;
    g_pool.pending = remote;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.go);
    pthread_mutex_unlock(&g_pool.mu);
    fn(args);
    for (int i = remote + 1; i < njobs; i++) fn((char*)args + (size_t)i * stride); /* no worker: run here */
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.pending > 0) pthread_cond_wait(&g_pool.done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

typedef struct {
    const float* a;
    size_t k, n, r0, r1, j0, j1;
    const uint8_t* q;
    int kind;
    const float* bias;
    float* y;
} q_job;

static void* q_job_run(void* arg) {
    q_job* j = (q_job*)arg;
    for (size_t i = j->r0; i < j->r1; i++) {
        float* o = j->y + i * j->n;
        for (size_t c = j->j0; c < j->j1; c++) o[c] = j->bias[c];
        qaccum_cols(j->a + i * j->k, j->k, j->q, j->n, j->kind, j->j0, j->j1, o + j->j0);
    }
    return NULL;
}

int fo_qlinear(const float* x, size_t m, size_t k, const float* scales, const uint8_t* q, size_t n, int kind,
               const float* bias, float* y, int threads) {
    /* a'[i, p] = x[i, p] * scale[p] (ops.rs:331-339) */
    float* a = (float*)malloc((m * k > 0 ? m * k : 1) * sizeof(float));
    if (!a) return -1;
    for (size_t i = 0; i < m; i++)
        for (size_t p = 0; p < k; p++) a[i * k + p] = x[i * k + p] * scales[p];
    q_job jobs[256];
    size_t nj = 0;
    if (m == 1 && threads > 1 && n >= 2 && n * k >= (1u << 16)) {
        /* parallel.rs:313-366, 370-372: column split, min chunk 64 */
        size_t t = (size_t)threads, cap = (n + 63) / 64;
        if (t > cap) t = cap;
        if (t > 256) t = 256;
        size_t per = (n + t - 1) / t;
        for (size_t j0 = 0; j0 < n; j0 += per)
            jobs[nj++] = (q_job){a, k, n, 0, 1, j0, j0 + per < n ? j0 + per : n, q, kind, bias, y};
    } else if (m >= 2 && threads > 1 && m * k * n >= (1u << 16)) {
        /* parallel.rs:90-92, 168-297: row split */
        size_t t = (size_t)threads < m ? (size_t)threads : m;
        if (t > 256) t = 256;
        size_t per = (m + t - 1) / t;
        for (size_t r0 = 0; r0 < m; r0 += per)
            jobs[nj++] = (q_job){a, k, n, r0, r0 + per < m ? r0 + per : m, 0, n, q, kind, bias, y};
    } else {
        jobs[nj++] = (q_job){a, k, n, 0, m, 0, n, q, kind, bias, y};
    }
    pool_run(q_job_run, jobs, sizeof(q_job), (int)nj);
    free(a);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* W8A8                                                                       */
/* ------------------------------------------------------------------------ */

void fo_q8_0_quantize_rows(const float* x, size_t m, size_t k, uint16_t* d16, int8_t* q) {
    size_t kb = k / 32;
    for (size_t i = 0; i < m; i++)
        for (size_t b = 0; b < kb; b++) fo_q8_0_block(x + i * k + b * 32, d16 + i * kb + b, q + i * k + b * 32);
}

void fo_q8_0_block_dots(const int8_t* qx, size_t m, size_t k, const uint8_t* raw, size_t n,
                        int32_t* dots) {
    size_t kb = k / 32, row_bytes = kb * 34;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++)
            for (size_t b = 0; b < kb; b++) {
                const uint8_t* blk = raw + j * row_bytes + b * 34;
                int32_t s = 0;
                for (int t = 0; t < 32; t++) s += (int32_t)qx[i * k + b * 32 + (size_t)t] * (int32_t)(int8_t)blk[2 + t];
                dots[(i * n + j) * kb + b] = s;
            }
}

int fo_q8_0_linear_w8a8(const float* x, size_t m, size_t k, const uint8_t* raw, size_t n,
                        const float* bias, float* y) {
    if (k % 32 != 0) return -1;
    size_t kb = k / 32, row_bytes = kb * 34;
    uint16_t* dx = (uint16_t*)malloc((m * kb + 1) * sizeof(uint16_t));
    int8_t* qx = (int8_t*)malloc(m * k + 1);
    if (!dx || !qx) {
        free(dx);
        free(qx);
        return -2;
    }
    fo_q8_0_quantize_rows(x, m, k, dx, qx);
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float sumf = 0.0f;
            for (size_t b = 0; b < kb; b++) {
                const uint8_t* blk = raw + j * row_bytes + b * 34;
                int32_t s = 0;
                for (int t = 0; t < 32; t++) s += (int32_t)qx[i * k + b * 32 + (size_t)t] * (int32_t)(int8_t)blk[2 + t];
                float dw = fo_f16_to_f32((uint16_t)(blk[0] | ((uint16_t)blk[1] << 8)));
                float dd = dw * fo_f16_to_f32(dx[i * kb + b]);
                sumf += (float)s * dd;
            }
            if (bias) sumf += bias[j];
            y[i * n + j] = sumf;
        }
    free(dx);
    free(qx);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* softmax + ln bridge                                                        */
/* ------------------------------------------------------------------------ */

/* ops.rs:478-502 */
void fo_softmax_rows(const float* z, size_t rows, size_t cols, float* out) {
    for (size_t r = 0; r < rows; r++) {
        const float* zr = z + r * cols;
        float* o = out + r * cols;
        float mx = -INFINITY;
        for (size_t c = 0; c < cols; c++) mx = fmaxf(mx, zr[c]);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            float e = expf(zr[c] - mx);
            o[c] = e;
            sum += e;
        }
        for (size_t c = 0; c < cols; c++) o[c] /= sum;
    }
}

/* slm/token_stream.rs:134 */
void fo_ln_bridge(const float* p, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = logf(fmaxf(p[i], 1e-12f));
}

/* ------------------------------------------------------------------------ */
/* the rest of a GPT-2 decode step                                            */
/* ------------------------------------------------------------------------ */

/* LayerNorm::forward (layer/norm.rs:46-82): per row the mean and the biased
 * variance as sequential sums over the row divided by cols, std =
 * sqrt(var + 1e-5), out = ((x - mean) / std) * gamma + beta. */
void fo_layernorm(const float* x, size_t rows, size_t cols, const float* gamma, const float* beta, float* out) {
    for (size_t r = 0; r < rows; r++) {
        const float* xr = x + r * cols;
        float sum = 0.0f;
        for (size_t c = 0; c < cols; c++) sum += xr[c];
        const float mean = sum / (float)cols;
        float ss = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            const float dv = xr[c] - mean;
            ss += dv * dv;
        }
        const float var = ss / (float)cols;
        const float sd = sqrtf(var + 1e-5f);
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = ((xr[c] - mean) / sd) * gamma[c] + beta[c];
    }
}

/* activation::gelu (activation.rs:9-12), tanh approximation, in place. */
void fo_gelu(float* x, size_t n) {
    const float k = 0.7978846f;
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        x[i] = 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
    }
}

/* Embedding::embed_one (layer/embedding.rs:70-90): token row + position row.
 * token >= vocab or pos >= max_seq -> -1 (the reference's DimMismatch). */
int fo_embed_one(const float* tok_w, const float* pos_w, size_t vocab, size_t max_seq, size_t d, size_t token,
                 size_t pos, float* out) {
    if (token >= vocab || pos >= max_seq) return -1;
    for (size_t i = 0; i < d; i++) out[i] = tok_w[token * d + i] + pos_w[pos * d + i];
    return 0;
}

/* The attention of TransformerBlock::forward_with_cache (layer/transformer.rs:
 * 242-279): the new k, v (qkv[d .. 2d), qkv[2d .. 3d)) are written at cache row
 * pos, then per head h the query qkv[h hd ..] attends over rows 0..pos:
 * s_j = (sum_d q k_j) * (1 / sqrt(hd)), e_j = exp(s_j - max), sum in j order,
 * out_h += (e_j / sum) * v_j in j order.  pos >= capacity -> -1 (cache full);
 * d % heads != 0 -> -2. */
int fo_attention_decode(const float* qkv, float* k_cache, float* v_cache, size_t capacity, size_t d, size_t heads,
                        size_t pos, float* out) {
    if (pos >= capacity) return -1;
    if (heads == 0 || d % heads != 0) return -2;
    for (size_t i = 0; i < d; i++) {
        k_cache[pos * d + i] = qkv[d + i];
        v_cache[pos * d + i] = qkv[2 * d + i];
    }
    const size_t len = pos + 1, hd = d / heads;
    const float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(len * sizeof(float));
    if (!sc) return -3;
    for (size_t i = 0; i < d; i++) out[i] = 0.0f;
    for (size_t h = 0; h < heads; h++) {
        const size_t hs = h * hd;
        for (size_t j = 0; j < len; j++) {
            float dot = 0.0f;
            for (size_t t = 0; t < hd; t++) dot += qkv[hs + t] * k_cache[j * d + hs + t];
            sc[j] = dot * scale;
        }
        float mx = -INFINITY;
        for (size_t j = 0; j < len; j++) mx = fmaxf(mx, sc[j]);
        float sum = 0.0f;
        for (size_t j = 0; j < len; j++) {
            sc[j] = expf(sc[j] - mx);
            sum += sc[j];
        }
        for (size_t j = 0; j < len; j++) {
            const float pj = sc[j] / sum;
            for (size_t t = 0; t < hd; t++) out[hs + t] += pj * v_cache[j * d + hs + t];
        }
    }
    free(sc);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Llama / Qwen block pieces                                                  */
/* ------------------------------------------------------------------------ */

void fo_rmsnorm(const float* x, size_t rows, size_t dim, const float* w, float eps, float* out) {
    for (size_t r = 0; r < rows; r++) {
        const float* xr = x + r * dim;
        float* o = out + r * dim;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; i++) ss += xr[i] * xr[i];
        const float ms = ss / (float)dim;
        const float inv = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < dim; i++) o[i] = xr[i] * inv * w[i];
    }
}

void fo_rope(float* x, size_t n_heads, size_t head_dim, size_t rope_dim, size_t pos, float base, int rope_type,
             const float* freq_factors, float linear_factor) {
    const size_t half = rope_dim / 2;
    for (size_t h = 0; h < n_heads; h++) {
        const size_t off = h * head_dim;
        for (size_t i = 0; i < half; i++) {
            const float freq = (float)pow((double)base, -2.0 * (double)i / (double)rope_dim);
            const float ff = freq_factors ? freq_factors[i] : 1.0f;
            const float theta = (float)pos * freq / ff * (1.0f / linear_factor);
            const float sn = sinf(theta), cs = cosf(theta);
            const size_t ia = rope_type == 0 ? off + 2 * i : off + i;
            const size_t ib = rope_type == 0 ? off + 2 * i + 1 : off + i + half;
            const float a = x[ia], b = x[ib];
            x[ia] = a * cs - b * sn;
            x[ib] = a * sn + b * cs;
        }
    }
}

int fo_gqa_attention_decode(const float* qkv, float* k_cache, float* v_cache, size_t capacity, size_t n_heads,
                            size_t n_kv, size_t head_dim, size_t pos, float* out) {
    if (pos >= capacity) return -1;
    if (n_kv == 0 || n_heads % n_kv != 0 || head_dim == 0) return -2;
    const size_t hd = head_dim, q_dim = n_heads * hd, kv_dim = n_kv * hd, group = n_heads / n_kv;
    for (size_t i = 0; i < kv_dim; i++) {
        k_cache[pos * kv_dim + i] = qkv[q_dim + i];
        v_cache[pos * kv_dim + i] = qkv[q_dim + kv_dim + i];
    }
    const size_t len = pos + 1;
    const float scale = 1.0f / sqrtf((float)hd);
    float* sc = (float*)malloc(len * sizeof(float));
    if (!sc) return -3;
    for (size_t h = 0; h < n_heads; h++) {
        const size_t kvh = h / group;
        const float* qh = qkv + h * hd;
        for (size_t j = 0; j < len; j++) {
            const float* kj = k_cache + j * kv_dim + kvh * hd;
            float dot = 0.0f;
            for (size_t t = 0; t < hd; t++) dot += qh[t] * kj[t];
            sc[j] = dot * scale;
        }
        float mx = -INFINITY;
        for (size_t j = 0; j < len; j++) mx = fmaxf(mx, sc[j]);
        float sum = 0.0f;
        for (size_t j = 0; j < len; j++) {
            sc[j] = expf(sc[j] - mx);
            sum += sc[j];
        }
        float* oh = out + h * hd;
        for (size_t t = 0; t < hd; t++) oh[t] = 0.0f;
        for (size_t j = 0; j < len; j++) {
            const float p = sc[j] / sum;
            const float* vj = v_cache + j * kv_dim + kvh * hd;
            for (size_t t = 0; t < hd; t++) oh[t] += p * vj[t];
        }
    }
    free(sc);
    return 0;
}

void fo_swiglu(const float* g, const float* u, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* ------------------------------------------------------------------------ */
/* RNG                                                                        */
/* ------------------------------------------------------------------------ */

uint64_t fo_rng_new(uint64_t seed) { return seed == 0 ? 0x9E3779B97F4A7C15ull : seed; }

uint64_t fo_rng_next_u64(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

float fo_draw_to_f32(uint64_t draw) { return (float)(draw >> 40) / (float)(1u << 24); }

float fo_rng_next_f32(uint64_t* state) { return fo_draw_to_f32(fo_rng_next_u64(state)); }

/* ------------------------------------------------------------------------ */
/* Sampler: slm/sampling.rs:96-210                                            */
/* ------------------------------------------------------------------------ */

/* f32::total_cmp as a signed integer key. */
static int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* sampling.rs:96-104 */
static size_t argmax_first(const float* xs, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (total_key(xs[i]) > total_key(xs[best])) best = i;
    return best;
}

size_t fo_argmax_first(const float* xs, size_t n) { return n ? argmax_first(xs, n) : 0; }

/* sampling.rs:109-122 */
size_t fo_pick_by_mass(const float* probs, size_t n, float r) {
    float cumsum = 0.0f;
    size_t last = 0;
    for (size_t i = 0; i < n; i++)
        if (probs[i] > 0.0f) {
            last = i;
            cumsum += probs[i];
            if (r <= cumsum) return i;
        }
    return last;
}

static int cmp_desc_f32(const void* a, const void* b) {
    int32_t ka = total_key(*(const float*)a), kb = total_key(*(const float*)b);
    return ka < kb ? 1 : (ka > kb ? -1 : 0);
}

static int cmp_idx_desc(const void* a, const void* b, void* ctx) {
    const float* probs = (const float*)ctx;
    uint32_t ia = *(const uint32_t*)a, ib = *(const uint32_t*)b;
    int32_t ka = total_key(probs[ia]), kb = total_key(probs[ib]);
    if (ka != kb) return ka < kb ? 1 : -1;
    return ia < ib ? -1 : (ia > ib ? 1 : 0);
}

static float rel_gap(float hi, float lo) {
    float den = fabsf(hi) > 1e-30f ? fabsf(hi) : 1e-30f;
    return (hi - lo) / den;
}

uint32_t fo_sample(const float* logits, size_t n, const fo_sampling_params* params,
                   const uint32_t* recent, size_t n_recent, uint64_t draw, fo_sample_info* info) {
    fo_sample_info local;
    if (!info) info = &local;
    memset(info, 0, sizeof(*info));
    info->margin = info->greedy_gap = info->topk_gap = info->topp_gap = info->draw_gap = 1.0f;
    if (n == 0) return 0;

    float* work = (float*)malloc(n * sizeof(float));
    memcpy(work, logits, n * sizeof(float));
    float pen = params->repetition_penalty;
    /* 1. repetition penalty, once per occurrence (sampling.rs:133-144) */
    if (fabsf(pen - 1.0f) > FLT_EPSILON && pen > 0.0f)
        for (size_t r = 0; r < n_recent; r++) {
            uint32_t tok = recent[r];
            if (tok < n) work[tok] = work[tok] > 0.0f ? work[tok] / pen : work[tok] * pen;
        }

    /* greedy (sampling.rs:147-149) */
    if (params->temperature <= 0.0f) {
        size_t best = argmax_first(work, n);
        float second = -INFINITY;
        for (size_t i = 0; i < n; i++)
            if (i != best && total_key(work[i]) > total_key(second)) second = work[i];
        info->path = FO_PATH_GREEDY;
        info->greedy_gap = n > 1 ? rel_gap(work[best], second) : 1.0f;
        info->margin = info->greedy_gap;
        free(work);
        return (uint32_t)best;
    }
    float t = fmaxf(params->temperature, 0.01f);

    /* 2. temperature softmax (sampling.rs:150-169) */
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, work[i]);
    float* probs = work; /* in place: work is not read again */
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        probs[i] = expf((probs[i] - mx) / t);
        sum += probs[i];
    }
    if (isnan(sum) || sum <= 1e-10f) {
        info->path = FO_PATH_FALLBACK;
        free(work);
        return (uint32_t)(draw % (uint64_t)n);
    }
    for (size_t i = 0; i < n; i++) probs[i] /= sum;
    info->path = FO_PATH_SAMPLED;

    /* 3. top-k (sampling.rs:171-180) */
    if (params->top_k > 0 && params->top_k < n) {
        float* sorted = (float*)malloc(n * sizeof(float));
        memcpy(sorted, probs, n * sizeof(float));
        qsort(sorted, n, sizeof(float), cmp_desc_f32);
        float thr = sorted[params->top_k - 1];
        float below = 0.0f;
        for (size_t i = params->top_k; i < n; i++)
            if (sorted[i] < thr) {
                below = sorted[i];
                break;
            }
        info->topk_gap = thr > 0.0f ? rel_gap(thr, below) : 1.0f;
        for (size_t i = 0; i < n; i++)
            if (probs[i] < thr) probs[i] = 0.0f;
        free(sorted);
    }

    /* 4. top-p (sampling.rs:183-200) */
    if (params->top_p < 1.0f) {
        uint32_t* order = (uint32_t*)malloc(n * sizeof(uint32_t));
        unsigned char* keep = (unsigned char*)calloc(n, 1);
        for (size_t i = 0; i < n; i++) order[i] = (uint32_t)i;
        qsort_r(order, n, sizeof(uint32_t), cmp_idx_desc, probs);
        float cum = 0.0f, prev = 0.0f;
        size_t c = 0;
        int crossed = 0;
        for (; c < n; c++) {
            keep[order[c]] = 1;
            prev = cum;
            cum += probs[order[c]];
            if (cum >= params->top_p) {
                crossed = 1;
                break;
            }
        }
        float tp = params->top_p;
        if (crossed) {
            float g1 = (tp - prev) / tp, g2 = (cum - tp) / tp;
            info->topp_gap = g1 < g2 ? g1 : g2;
            if (c + 1 < n) {
                float pc = probs[order[c]], pn = probs[order[c + 1]];
                if (pn == pc && pc > 0.0f) info->topp_tie = 1;
                float g3 = pc > 0.0f ? rel_gap(pc, pn) : 1.0f;
                if (g3 < info->topp_gap) info->topp_gap = g3;
            }
        } else {
            info->topp_gap = (tp - cum) / tp;
        }
        for (size_t i = 0; i < n; i++)
            if (!keep[i]) probs[i] = 0.0f;
        free(order);
        free(keep);
    }

    /* 5. renormalise and draw (sampling.rs:205-209, 109-122) */
    float sum2 = 0.0f;
    for (size_t i = 0; i < n; i++) sum2 += probs[i];
    for (size_t i = 0; i < n; i++) probs[i] /= sum2;
    float r = fo_draw_to_f32(draw);
    float cumsum = 0.0f, before = 0.0f;
    size_t last = 0, pick = n;
    int first_survivor = 1, pick_first = 0;
    uint32_t kept = 0;
    for (size_t i = 0; i < n; i++) {
        if (probs[i] > 0.0f) {
            kept++;
            last = i;
            before = cumsum;
            cumsum += probs[i];
            if (pick == n && r <= cumsum) {
                pick = i;
                pick_first = first_survivor;
                float g_hi = cumsum - r, g_lo = r - before;
                info->draw_gap = pick_first ? g_hi : (g_hi < g_lo ? g_hi : g_lo);
            }
            first_survivor = 0;
        }
    }
    if (pick == n) {
        pick = last;
        info->draw_gap = r - cumsum;
    }
    info->n_kept = kept;
    float m = info->topk_gap;
    if (info->topp_gap < m) m = info->topp_gap;
    if (info->draw_gap < m) m = info->draw_gap;
    if (info->topp_tie) m = 0.0f;
    info->margin = m;
    free(work);
    return (uint32_t)pick;
}

uint32_t fo_sample_with_params(const float* logits, size_t n, const fo_sampling_params* params,
                               const uint32_t* recent, size_t n_recent, uint64_t* rng_state,
                               fo_sample_info* info) {
    uint64_t draw = 0;
    if (params->temperature > 0.0f || isnan(params->temperature)) draw = fo_rng_next_u64(rng_state);
    return fo_sample(logits, n, params, recent, n_recent, draw, info);
}
