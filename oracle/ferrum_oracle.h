/*
 * ferrum_oracle — CPU restatement of ferrum_core's Q8_0 decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against, and the timed CPU baseline of bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (libferrum_hip) never links, calls or falls back to it.
 *
 * Every function restates one piece of the reference (Rust, CPU-only, not
 * buildable here: no Rust toolchain in the image).  The reference file:line it
 * follows is cited beside each declaration.  Arithmetic is plain IEEE binary32
 * with no contraction (built with -ffp-contract=off), so the linear layer is
 * bit-identical to ferrum_core's `ops::linear_forward`.
 */
#ifndef FERRUM_ORACLE_H
#define FERRUM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE half codec ---------------------------------------------------- */
/* ferrum_core/src/gguf_write/blocks.rs:12-61 (round-to-nearest-even encode). */
uint16_t fo_f32_to_f16(float value);
/* ferrum_core/src/gguf/dequant.rs:7-35 (exact decode incl. subnormals). */
float fo_f16_to_f32(uint16_t h);

/* Element-wise array forms of the two codecs above (same arithmetic). */
void fo_f32_to_f16_n(const float* x, size_t n, uint16_t* out);
void fo_f16_to_f32_n(const uint16_t* h, size_t n, float* out);

/* ---- Q8_0 block codec --------------------------------------------------- */
/* ferrum_core/src/quant.rs:271-280: amax fold (NaN ignored), d = amax/127,
 * id = d != 0 ? 1/d : 0, q = round-half-away(x*id) saturating (NaN -> 0),
 * stored scale f16(d). */
void fo_q8_0_block(const float* x32, uint16_t* d16, int8_t* q32);
/* ferrum_core/src/gguf_write/blocks.rs:65-92,132-140: n floats -> n/32 blocks
 * of 34 bytes (little-endian f16 scale then 32 int8).  Returns -1 when n is
 * not a multiple of 32 (the reference's Format error), else 0. */
int fo_q8_0_encode(const float* data, size_t n, uint8_t* out);
/* ferrum_core/src/gguf/dequant.rs:37-49: w[b*32+j] = f16_to_f32(d_b) * q_j.
 * Returns -1 when raw_len < n/32*34 (the reference's cursor error). */
int fo_q8_0_dequant(const uint8_t* raw, size_t raw_len, size_t n, float* out);
/* ferrum_core/src/quant.rs:298-305 (in-place snap of ne0-long rows). */
void fo_fake_quantize_q8_0_rows(float* data, size_t len, size_t ne0);
/* ferrum_core/src/quant.rs:309-325 (snap of a Ferrum [rows_in, cols_out]
 * weight whose Q8_0 blocks run down each column). */
void fo_fake_quantize_q8_0_cols(float* data, size_t rows_in, size_t cols_out);

/* GGUF Q8_0 tensor [n_rows x k] (GGML ne0 = k) -> Ferrum row-major [k, n_rows]
 * f32 weight: dequantize (gguf/tensors.rs:58-87, gguf/dequant.rs:37-49) then
 * transpose (gguf/llama.rs:342-350; loader/decode.rs:57-81).  Returns -1 when
 * k % 32 != 0. */
int fo_q8_0_to_ferrum_weight(const uint8_t* raw, size_t n_rows, size_t k, float* w_kn);

/* ---- linear layer ------------------------------------------------------- */
/* ferrum_core/src/ops.rs:233-256 -> matmul_rows (159-177) -> matmul_bias_block
 * (132-148) -> matmul_block / micro_tile / edge_rows (29-126):
 *   y[i,j] = fl( fl( sum_{p ascending} fl(x[i,p] * W[p,j]) ) + b[j] )
 * W is Ferrum's [k, n] row-major weight.  bias may be NULL (ops::matmul,
 * ops.rs:197).  threads follows parallel.rs:84-92,168-297: m == 1 or
 * m*k*n < 65536 runs serially; otherwise ceil(m/threads)-row blocks.  The
 * result is bit-identical at every thread count.  Returns 0. */
int fo_linear_forward(const float* x, size_t m, size_t k, const float* w_kn, size_t n,
                      const float* bias, float* y, int threads);

/* Same contraction taken straight from GGUF Q8_0 rows (no [k, n] expansion):
 * the products and their order are those of fo_linear_forward on
 * fo_q8_0_to_ferrum_weight's output, so the result is bit-identical. */
int fo_q8_0_linear_rows(const float* x, size_t m, size_t k, const uint8_t* raw, size_t n,
                        const float* bias, float* y);

/* ---- packed per-row int8 / int4 weights (adjacent path, not GGUF Q8_0) ---- */
/* quant.rs:130-217 QWeight::from_f32: row-major [rows, cols], one symmetric
 * scale per row (amax/127 int8, amax/7 int4), levels round-half-away
 * saturating (NaN -> 0); int4 in the split-half nibble layout (column c < half
 * in the low nibble of byte c, else the high nibble of byte c - half).
 * kind 0 = int8, 1 = int4. */
size_t fo_qweight_row_bytes(size_t cols, int kind);
void fo_qweight_from_f32(const float* data, size_t rows, size_t cols, int kind, float* scales, uint8_t* q);
/* quant.rs:228-254 dequant_row over all rows. */
void fo_qweight_to_f32(const float* scales, const uint8_t* q, size_t rows, size_t cols, int kind, float* out);
/* ops.rs:268-377 qlinear: y[i, j] = bias[j] + sum_p (x[i, p] * scale[p]) * level(p, j),
 * p ascending, no FMA, bias FIRST; k = rows, n = cols.  m == 1 splits columns
 * over threads (min chunk 64, parallel.rs:313-372), m >= 2 splits rows; the
 * result does not depend on the thread count. */
int fo_qlinear(const float* x, size_t m, size_t k, const float* scales, const uint8_t* q, size_t n, int kind,
               const float* bias, float* y, int threads);

/* ---- W8A8 (activation re-quantization, llama.cpp semantics) ------------- */
/* Activations are Q8_0-encoded with fo_q8_0_block per 32 (quant.rs:271-280).
 * d16: [m, k/32], q: [m, k]. */
void fo_q8_0_quantize_rows(const float* x, size_t m, size_t k, uint16_t* d16, int8_t* q);
/* int32 block dot products dots[i, j, b] = sum_{t<32} qx[i, 32b+t] * qw[j, 32b+t],
 * qw taken from GGUF rows raw [n x k].  Exact integers. */
void fo_q8_0_block_dots(const int8_t* qx, size_t m, size_t k, const uint8_t* raw, size_t n,
                        int32_t* dots);
/* y[i,j] = fl(sum_b fl((float)dots * fl(dw_b * dx_b))) + b[j], blocks in
 * ascending order (llama.cpp ggml_vec_dot_q8_0_q8_0 generic form; the
 * reference names it as the llama.cpp behaviour, MANUAL.md:1609-1611). */
int fo_q8_0_linear_w8a8(const float* x, size_t m, size_t k, const uint8_t* raw, size_t n,
                        const float* bias, float* y);

/* ---- softmax and the GPT-2 pre-sampler bridge --------------------------- */
/* ferrum_core/src/ops.rs:478-502: p = exp(z - max) / sum, sequential sum. */
void fo_softmax_rows(const float* z, size_t rows, size_t cols, float* out);
/* ferrum_core/src/slm/token_stream.rs:134: l = ln(max(p, 1e-12)). */
void fo_ln_bridge(const float* p, size_t n, float* out);

/* ---- RNG (xorshift64*) -------------------------------------------------- */
/* ferrum_core/src/rng.rs:10-14 (seed 0 remap), 29-36, 39-41. */
uint64_t fo_rng_new(uint64_t seed);
uint64_t fo_rng_next_u64(uint64_t* state);
float fo_rng_next_f32(uint64_t* state);
/* The f32 draw derived from one next_u64 output: (x >> 40) / 2^24. */
float fo_draw_to_f32(uint64_t draw);

/* ---- sampler ------------------------------------------------------------ */
typedef struct {
    float temperature;        /* <= 0: greedy */
    uint32_t top_k;           /* 0 disables */
    float top_p;              /* >= 1 disables */
    float repetition_penalty; /* 1 disables */
} fo_sampling_params;

enum { FO_PATH_GREEDY = 0, FO_PATH_FALLBACK = 1, FO_PATH_SAMPLED = 2 };

typedef struct {
    int32_t path;        /* FO_PATH_* */
    uint32_t n_kept;     /* tokens with p > 0 after top-k/top-p (sampled path) */
    float margin;        /* smallest relative decision margin (see fo_sample) */
    float greedy_gap;    /* (top1 - top2) / max(|top1|, 1e-30) over the penalized row */
    float topk_gap;      /* (thr - largest p below thr) / thr, 1 when not applied */
    float topp_gap;      /* min |cum - top_p| / top_p at the cutoff, 1 when not applied */
    float draw_gap;      /* min |r - cumsum boundary| of the chosen token */
    uint32_t topp_tie;   /* 1 when a tie group of p straddles the top-p cutoff */
} fo_sample_info;

/* slm/sampling.rs:96-104: index of the first maximum under f32::total_cmp. */
size_t fo_argmax_first(const float* xs, size_t n);
/* slm/sampling.rs:109-122: inverse-CDF draw over index order, skipping p == 0. */
size_t fo_pick_by_mass(const float* probs, size_t n, float r);

/* ferrum_core/src/slm/sampling.rs:124-210 with argmax_first (96-104) and
 * pick_by_mass (109-122).  `draw` is the one next_u64 the reference consumes
 * for temperature > 0 (the fallback uses draw % n, the normal path
 * fo_draw_to_f32(draw)); it is ignored for greedy.  Ties of p in the top-p sort
 * are broken by ascending index (the reference's sort_unstable leaves that
 * order unspecified; info->topp_tie reports when it matters).  info may be
 * NULL.  Returns the token id. */
uint32_t fo_sample(const float* logits, size_t n, const fo_sampling_params* params,
                   const uint32_t* recent, size_t n_recent, uint64_t draw, fo_sample_info* info);

/* The reference signature: draws from *rng_state exactly as sample_with_params
 * does (nothing for greedy, one next_u64 otherwise). */
uint32_t fo_sample_with_params(const float* logits, size_t n, const fo_sampling_params* params,
                               const uint32_t* recent, size_t n_recent, uint64_t* rng_state,
                               fo_sample_info* info);

/* The rest of a GPT-2 decode step: LayerNorm::forward (layer/norm.rs:46-82),
 * activation::gelu in place (activation.rs:9-12), Embedding::embed_one
 * (layer/embedding.rs:70-90; -1 when token or pos is out of range) and the
 * attention of TransformerBlock::forward_with_cache (layer/transformer.rs:
 * 242-279; appends k, v from qkv = [q | k | v] at row pos, -1 when the cache is
 * full, -2 when heads does not divide d). */
void fo_layernorm(const float* x, size_t rows, size_t cols, const float* gamma, const float* beta, float* out);
void fo_gelu(float* x, size_t n);
int fo_embed_one(const float* tok_w, const float* pos_w, size_t vocab, size_t max_seq, size_t d, size_t token,
                 size_t pos, float* out);
int fo_attention_decode(const float* qkv, float* k_cache, float* v_cache, size_t capacity, size_t d, size_t heads,
                        size_t pos, float* out);

/* ---- Llama / Qwen block pieces (llm.rs) ---------------------------------- */
/* RmsNorm::forward_row (llm.rs:58-65), every row: ms = sequential sum of v*v
 * divided by dim, inv = 1 / sqrt(ms + eps), out = x * inv * w. */
void fo_rmsnorm(const float* x, size_t rows, size_t dim, const float* w, float eps, float* out);
/* apply_rope (llm.rs:146-175) with RopeScaling::angle (llm.rs:118-121):
 * freq_i = (f32) pow((f64) base, -2 i / rope_dim), theta = pos * freq / ff_i
 * * (1 / linear_factor), pairs (2i, 2i+1) for NORM (rope_type 0) or
 * (i, i + rope_dim/2) for NEOX (1); channels past rope_dim pass through.
 * freq_factors may be NULL (none) or hold rope_dim / 2 values. */
void fo_rope(float* x, size_t n_heads, size_t head_dim, size_t rope_dim, size_t pos, float base, int rope_type,
             const float* freq_factors, float linear_factor);
/* Attention::forward_one's cache append + attend (llm.rs:285-358) for one
 * query row: qkv = [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)], already
 * RoPE'd; k and v are written at row pos of the [capacity, n_kv*hd] caches,
 * then every head h attends over rows 0..pos with kv head h / (n_heads/n_kv),
 * p = exp(s - max) / sum applied before the v sum.  Returns -1 when the cache
 * is full, -2 on a bad head split. */
int fo_gqa_attention_decode(const float* qkv, float* k_cache, float* v_cache, size_t capacity, size_t n_heads,
                            size_t n_kv, size_t head_dim, size_t pos, float* out);
/* FeedForward::forward's gate (llm.rs:415-421): out = (g / (1 + exp(-g))) * u. */
void fo_swiglu(const float* g, const float* u, size_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
