/*
 * ferrum_hip.h — C ABI of libferrum_hip, the MI355X (gfx950) implementation of
 * ferrum_core's decode-step hot path: GGUF Q8_0 linear layers and the logit
 * sampler.
 *
 * The reference (thomascherickal/ferrum-cpu, Rust, CPU-only) has no plugin
 * registry: the path is reached through two Rust source APIs, which these
 * entry points replace one for one:
 *
 *   ops::linear_forward(input, weight, bias)     ferrum_core/src/ops.rs:233-256
 *   ops::matmul(a, b)  (the bias-free form)      ferrum_core/src/ops.rs:197-223
 *     called only from Linear::forward           ferrum_core/src/layer/linear.rs:177-210
 *   slm::sampling::sample_with_params(logits, params, recent, rng)
 *                                                ferrum_core/src/slm/sampling.rs:124-210
 *
 * plus the Q8_0 block codec they are specified by:
 *
 *   quant::q8_0_block                            ferrum_core/src/quant.rs:271-280
 *   gguf_write enc_q8_0                          ferrum_core/src/gguf_write/blocks.rs:132-140
 *   gguf dequant_q8_0                            ferrum_core/src/gguf/dequant.rs:37-49
 *
 * Conventions.
 *  - Every entry point returns an int status (FH_OK = 0); the message of the
 *    last failure is fh_last_error(ctx).  Nothing aborts the process.
 *  - A context owns one HIP stream on one device (or borrows a caller's stream,
 *    fh_ctx_set_stream).  A context is not thread-safe; use one per thread.
 *  - Entry points without the _async suffix take HOST pointers, copy in, run,
 *    copy out and synchronise before returning (the reference's blocking call).
 *    _async entry points take DEVICE pointers, enqueue on the context stream
 *    and return at once; fh_sync waits.
 *  - Shapes follow the reference: an input x is [m, k] row-major, a weight is
 *    the GGUF Q8_0 tensor with ne0 = k (the reduction axis) and ne1 = n rows,
 *    and y = x . W^T + b is [m, n] — the same product ferrum_core computes on
 *    its transposed [k, n] f32 expansion (gguf/llama.rs:342-350).
 *  - Results are deterministic run to run: no reduction depends on the order
 *    in which atomics land.
 */
#ifndef FERRUM_HIP_H
#define FERRUM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
enum {
    FH_OK = 0,
    FH_ERR_DIM = 1,     /* shape mismatch: ferrum_core's InferError::DimMismatch (ops.rs:236-246) */
    FH_ERR_INVALID = 2, /* null pointer, unknown enum value, k % 32 != 0 */
    FH_ERR_OOM = 3,     /* device or host allocation failed */
    FH_ERR_HIP = 4,     /* a HIP runtime call failed (message carries hipGetErrorString) */
    FH_ERR_LIMIT = 5,   /* a size beyond a documented kernel limit */
    FH_ERR_FORMAT = 6,  /* a malformed GGUF file: ferrum_core's InferError::Format (gguf/cursor.rs) */
    FH_ERR_EXCHANGE = 7 /* a kernel's bounded cross-workgroup wait gave up (its workgroups were not all
                           resident at once, e.g. the GPU was shared): the results of the calls since
                           the last fh_sync are unreliable; no reference counterpart */
};

/* Bits kernels record in a context's device status word, reported (and
 * cleared) by fh_sync and by the blocking calls. */
enum {
    FH_STATUS_EXCHANGE = 1,   /* -> FH_ERR_EXCHANGE */
    FH_STATUS_BAD_OFFSETS = 2 /* a device recent_offsets list decreased -> FH_ERR_INVALID */
};

/* Numerics of a Q8_0 linear.
 *  FH_W8A32: ferrum_core's own semantics — weights dequantized exactly
 *            (f16(d) * q is exact in f32), activations stay f32, products and
 *            sums in f32 (loader/decode.rs:97-100; ops.rs:233-256).  Judged
 *            against the reference at 1e-5 relative.
 *  FH_W8A8:  llama.cpp's semantics, which the reference names as the
 *            behaviour it does NOT follow (MANUAL.md:1609-1611): activations
 *            Q8_0-encoded per 32 with q8_0_block, exact int32 block dots,
 *            then y = sum_b f32(dot_b) * (d_w * d_x) + bias.
 *  FH_W8A32_EXACT: FH_W8A32 bit for bit as ferrum_core computes it over the
 *            expanded weights: each output is 0 + x[0] w[0] + x[1] w[1] + ...
 *            in ascending k, every product and add rounded (no FMA), then
 *            + bias (ops.rs:29-148, 233-256) — the contract the reference's
 *            roadmap names q8_0_packed_forward_equals_expanded.  K is never
 *            split, so it runs at a fraction of FH_W8A32's speed; opt-in.
 *  FH_W8A8_FAST: FH_W8A8's quantisation and exact int32 block dots, with each
 *            block's term fused into the running sum (one rounding for
 *            f32(dot_b) * (d_w * d_x) + s instead of two): within 1e-5 of
 *            FH_W8A8's outputs (componentwise, relative to the sum of the
 *            terms' magnitudes), not bit-identical to them.  The prefill
 *            speed mode of the W8A8 semantics; no reference counterpart. */
enum { FH_W8A32 = 0, FH_W8A8 = 1, FH_W8A32_EXACT = 2, FH_W8A8_FAST = 3 };

/* What fh_sample_* receives in `logits`.
 *  FH_LOGITS_RAW:          the sampler input itself (the Llama/Qwen path,
 *                          llm.rs:745).
 *  FH_LOGITS_GPT2_SOFTMAX: the GPT-2 head's raw scores z; the sampler first
 *                          forms p = softmax(z) (ops.rs:478-502) and the bridge
 *                          l = ln(max(p, 1e-12)) (slm/token_stream.rs:134),
 *                          fused into the same kernel. */
enum { FH_LOGITS_RAW = 0, FH_LOGITS_GPT2_SOFTMAX = 1 };
/* OR'd into logits_kind: recent_offsets holds a (begin, end) pair per row
 * (2 * rows entries: row r's recent list is recent[recent_offsets[2r] ..
 * recent_offsets[2r + 1]]) instead of rows + 1 running offsets, so each row's
 * window can sit in its own stretch of a [rows, L] buffer (a batched decode,
 * fh_embed_rows_pos_async).  No reference counterpart: the reference samples
 * one row at a time (slm/sampling.rs:124).  fh_sample_rows_async only. */
enum { FH_RECENT_RANGES = 0x100 };

/* slm/sampling.rs:27-38 (SamplingParams without its cancel flag, which is a
 * host-side control checked between tokens, slm/token_stream.rs:126-131). */
typedef struct {
    float temperature;        /* <= 0: greedy argmax_first, no draw consumed */
    uint32_t top_k;           /* 0 or >= vocab: off */
    float top_p;              /* >= 1: off */
    float repetition_penalty; /* |pen - 1| <= f32::EPSILON or pen <= 0: off */
} fh_sampling_params;

typedef struct fh_ctx fh_ctx;
typedef struct fh_q8_0 fh_q8_0; /* a device-resident Q8_0 weight [n rows x k] */

/* ---- context ------------------------------------------------------------ */
/* No reference counterpart (the reference has no device); creates a context on
 * HIP device `device` with its own non-blocking stream. */
int fh_ctx_create(int device, fh_ctx** out);
void fh_ctx_destroy(fh_ctx* ctx);
/* Enqueue on `hip_stream`, a hipStream_t of the same device, instead of the
 * context's own stream.  NULL is HIP's legacy default stream (it is what
 * PyTorch's default stream handle is).  fh_ctx_reset_stream goes back to the
 * context's own stream. */
int fh_ctx_set_stream(fh_ctx* ctx, void* hip_stream);
int fh_ctx_reset_stream(fh_ctx* ctx);
/* Wait for all work enqueued on the context stream, then report what its
 * kernels recorded since the last fh_sync (and clear it): FH_ERR_EXCHANGE when a
 * bounded wait gave up, FH_ERR_INVALID when a device-form sampler call found
 * decreasing recent_offsets; FH_OK otherwise. */
int fh_sync(fh_ctx* ctx);
/* Message of the last failed call on `ctx` ("" if none); valid until the next
 * call on `ctx`.  fh_ctx_create failures are reported with ctx == NULL. */
const char* fh_last_error(const fh_ctx* ctx);
/* Number of HIP devices visible (0 when none), for hosts that probe first. */
int fh_device_count(void);

/* ---- Q8_0 weights ------------------------------------------------------- */
/* Upload the raw bytes of a GGUF Q8_0 tensor (ne0 = k, ne1 = n_rows; n_rows
 * rows of k/32 blocks, each block a little-endian f16 scale then 32 int8)
 * and repack it on the device for the kernels.  Replaces the reference's
 * load-time f32 expansion Gguf::dequantize -> dequant_q8_0 -> transpose_2d
 * (gguf/tensors.rs:58-87, gguf/dequant.rs:37-49, gguf/llama.rs:342-350,
 * loader/decode.rs:57-81) without expanding: the weight stays 34 B per 32
 * values in HBM.  k % 32 != 0 -> FH_ERR_INVALID (the reference stores such a
 * tensor as F32, loader/mod.rs:147-152). */
int fh_q8_0_upload(fh_ctx* ctx, const uint8_t* gguf_bytes, size_t n_rows, size_t k, fh_q8_0** out);
/* The same from a device buffer holding the GGUF bytes. */
int fh_q8_0_upload_device(fh_ctx* ctx, const uint8_t* d_gguf_bytes, size_t n_rows, size_t k,
                          fh_q8_0** out);
/* An F32 weight [n_rows x k] behind the same handle, from host rows (GGUF
 * order: k = ne0 values per row, any k): a matrix the reference stores as F32
 * (loader/mod.rs:147-152: ne0 % 32 != 0, or an unquantized save), read back
 * by Gguf::dequantize.  Every linear entry point takes it and computes the
 * reference's f32 linear_forward bit for bit (the FH_W8A32_EXACT kernel, for
 * FH_W8A32 too); FH_W8A8, the block dots, download, the no-allocation linear
 * and the one-launch GPT-2 stack need Q8_0 (FH_ERR_INVALID / FH_ERR_LIMIT). */
int fh_weight_upload_f32(fh_ctx* ctx, const float* rows, size_t n_rows, size_t k, fh_q8_0** out);
/* 0 for a Q8_0 weight, 1 for F32, -1 for NULL. */
int fh_weight_kind(const fh_q8_0* w);
/* Write the tensor back as GGUF bytes (host buffer of n_rows * k / 32 * 34). */
int fh_q8_0_download(fh_ctx* ctx, const fh_q8_0* w, uint8_t* gguf_bytes);
int fh_q8_0_dims(const fh_q8_0* w, size_t* n_rows, size_t* k);
void fh_q8_0_free(fh_q8_0* w);

/* ---- Q8_0 linear -------------------------------------------------------- */
/* y[m, n] = x[m, k] . W^T (+ bias[n]).  Replaces ops::linear_forward
 * (ops.rs:233-256; bias_len == n) and ops::matmul (ops.rs:197-223; bias NULL,
 * bias_len 0) on a Q8_0-backed Linear (layer/linear.rs:191-194).
 * k != W's k, or bias_len not in {0 (with bias NULL), n} -> FH_ERR_DIM, with the
 * reference's message.  m == 0 is a valid empty call.  numerics: FH_W8A32,
 * FH_W8A8, FH_W8A32_EXACT or FH_W8A8_FAST.  Host pointers; blocks until y is written. */
int fh_q8_0_linear(fh_ctx* ctx, const fh_q8_0* w, const float* x, size_t m, size_t k,
                   const float* bias, size_t bias_len, float* y, int numerics);
/* Device-pointer form of fh_q8_0_linear, enqueued on the context stream. */
int fh_q8_0_linear_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                         const float* d_bias, size_t bias_len, float* d_y, int numerics);

/* No reference counterpart: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  fh_q8_0_linear_async for FH_W8A32 at m <= 64 (the decode and
 * batched-decode shapes: the same kernels, the same results bit for bit), with
 * no allocation of any kind: the skinny GEMM's split-K partial sums and
 * arrival counters live in a fixed 12 MiB device array that each GPU holds
 * for the life of the process.  m > 64, FH_W8A8, or a shape whose K split
 * would need more than 12 MiB -> FH_ERR_LIMIT.  All calls on one GPU share that
 * array: calls that overlap on one GPU (two streams, two threads) race;
 * calls in one stream order are safe. */
int fh_q8_0_linear_noalloc_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                 const float* d_bias, size_t bias_len, float* d_y, int numerics);

/* ---- Q8_0 encode -------------------------------------------------------- */
/* n floats -> n/32 GGUF Q8_0 blocks of 34 bytes, bit-exact with enc_q8_0
 * (gguf_write/blocks.rs:132-140) over q8_0_block (quant.rs:271-280) and
 * f32_to_f16 (gguf_write/blocks.rs:12-61).  n % 32 != 0 -> FH_ERR_INVALID
 * (encode_tensor's length check, gguf_write/blocks.rs:65-92). */
int fh_q8_0_encode(fh_ctx* ctx, const float* x, size_t n, uint8_t* out);
int fh_q8_0_encode_async(fh_ctx* ctx, const float* d_x, size_t n, uint8_t* d_out);
/* GGUF Q8_0 bytes -> f32, bit-exact with dequant_q8_0 (gguf/dequant.rs:37-49). */
int fh_q8_0_dequant_async(fh_ctx* ctx, const uint8_t* d_gguf_bytes, size_t n, float* d_out);
/* The exact int32 block dot products of the W8A8 path:
 * dots[i, j, b] = sum_{t<32} qx[i, 32b+t] * q_w[j, 32b+t] for int8 activations
 * qx [m, k] (as fh_q8_0_encode lays them out, scales stripped).  A checking
 * hook for the integer core of FH_W8A8; no reference counterpart. */
int fh_q8_0_block_dots_async(fh_ctx* ctx, const fh_q8_0* w, const int8_t* d_qx, size_t m,
                             int32_t* d_dots);

/* ---- sampler ------------------------------------------------------------ */
/* One token id per row of `logits` [rows, vocab], each row sampled exactly as
 * sample_with_params does (slm/sampling.rs:124-210): repetition penalty once
 * per occurrence of an id in the row's `recent` list (ids >= vocab skipped),
 * greedy argmax_first when temperature <= 0, else temperature softmax, top-k
 * (ties at the k-th probability kept), top-p over the descending order,
 * renormalise and the inverse-CDF draw pick_by_mass (sampling.rs:109-122).
 *
 * Row r's recent ids are recent[recent_offsets[r] .. recent_offsets[r+1]]
 * (recent_offsets has rows + 1 entries; recent may be NULL when all are empty),
 * or with FH_RECENT_RANGES recent[recent_offsets[2r] .. recent_offsets[2r+1]].
 * draws[r] is the one u64 the reference's Rng::next_u64 yields for the row
 * (rng.rs:29-36): the draw is r = (draws[r] >> 40) / 2^24 (Rng::next_f32,
 * rng.rs:39-41), or draws[r] % vocab on the degenerate-softmax fallback
 * (sampling.rs:156-168).  The RNG stays on the host so the sequence is exactly
 * the reference's; draws may be NULL for greedy.  logits_kind: FH_LOGITS_*.
 * A recent list may be of any length (the Llama path passes the whole prompt
 * and everything generated, llm.rs:740-750).  vocab == 0 or decreasing
 * recent_offsets -> FH_ERR_INVALID.  Rows of 8192 ids or more are split over
 * several workgroups that exchange partial results; if a bounded wait of that
 * exchange gives up (the GPU did not hold all of a launch's workgroups at
 * once), the call returns FH_ERR_EXCHANGE.  Host pointers; blocks until
 * out_ids is written. */
int fh_sample_rows(fh_ctx* ctx, const float* logits, size_t rows, size_t vocab, int logits_kind,
                   const fh_sampling_params* params, const uint32_t* recent,
                   const uint32_t* recent_offsets, const uint64_t* draws, uint32_t* out_ids);
/* Device-pointer form of fh_sample_rows (params by value, on the host).  The
 * offsets are not read on the host: decreasing offsets and a failed exchange
 * are recorded on the device and reported by the next fh_sync. */
int fh_sample_rows_async(fh_ctx* ctx, const float* d_logits, size_t rows, size_t vocab,
                         int logits_kind, const fh_sampling_params* params,
                         const uint32_t* d_recent, const uint32_t* d_recent_offsets,
                         const uint64_t* d_draws, uint32_t* d_out_ids);
/* Testing hook, no reference counterpart: for later calls on ctx, the split
 * sampler's segment `skip_segment` and workgroup `skip_segment` of
 * fh_gpt2_stack_forward_async publish nothing (-1: none), and their bounded
 * waits give up after `spin_limit` polls (0: the default, 2^20), so a test can
 * drive the failure path from the host while every kernel still ends. */
int fh_debug_sampler_faults(fh_ctx* ctx, int skip_segment, uint32_t spin_limit);

/* ---- the rest of a GPT-2 decode step ------------------------------------- */
/* Activation applied to a linear's output before it is stored.
 * FH_ACT_SWIGLU32 (fh_q8_0_linear_normed_async only): the weight's n rows are
 * a gate and an up projection interleaved in groups of 32 (rows 64g .. 64g + 31
 * are gate rows 32g .. 32g + 31, rows 64g + 32 .. 64g + 63 the up rows of the
 * same outputs), and y[i][j] = silu(gate[i][j]) * up[i][j] is stored,
 * [m][n / 2]: FeedForward's gate (llm.rs:415-421) inside the linear. */
enum { FH_ACT_NONE = 0, FH_ACT_GELU = 1, FH_ACT_SWIGLU32 = 2 };
/* Device pointers, enqueued on the context's stream.  With fh_q8_0_linear_async
 * and fh_sample_rows_async these keep a whole decode step on the device.
 *
 * Embedding::embed_one (ferrum_core/src/layer/embedding.rs:70-90):
 * out[i] = token_w[token, i] + pos_w[pos, i].  The token id is read from device
 * memory (so a sampled id feeds the next step without a copy); an id >= vocab
 * makes the row NaN.  pos >= max_seq -> FH_ERR_DIM, the reference's message. */
int fh_embed_one_async(fh_ctx* ctx, const float* d_token_w, const float* d_pos_w, size_t vocab, size_t max_seq,
                       size_t d, const uint32_t* d_token, size_t pos, float* d_out);
/* Embedding::embed_one (layer/embedding.rs:70-90) for `rows` sequences decoded
 * together: out[r, i] = token_w[tokens[r], i] + pos_w[pos[r], i], token and
 * position ids on the device (a batched step's sampled ids feed the next step
 * without a copy).  An id >= vocab or a position >= max_seq makes the row NaN
 * (the caller checks positions: the reference's error is the host's).  With
 * d_hist set, each row's id is also recorded at d_hist[r * hist_stride +
 * pos[r]] (skipped when pos[r] >= hist_stride): the per-row token windows a
 * batched decode's sampler reads as its recent lists (FH_RECENT_RANGES).
 * rows <= 65535. */
int fh_embed_rows_pos_async(fh_ctx* ctx, const float* d_token_w, const float* d_pos_w, size_t vocab, size_t max_seq,
                            size_t d, const uint32_t* d_tokens, const uint32_t* d_pos, size_t rows, uint32_t* d_hist,
                            size_t hist_stride, float* d_out);
/* LayerNorm::forward (layer/norm.rs:46-82) over `rows` rows of width d:
 * ((x - mean) / sqrt(var + 1e-5)) * gamma + beta, biased variance. */
int fh_layernorm_async(fh_ctx* ctx, const float* d_x, size_t rows, size_t d, const float* d_gamma,
                       const float* d_beta, float* d_y);
/* activation::gelu (activation.rs:9-12, tanh approximation), in place. */
int fh_gelu_async(fh_ctx* ctx, float* d_x, size_t n);
/* fh_q8_0_linear_async followed by an activation (FH_ACT_*) on its output:
 * Linear::forward then `.map(gelu)` as the block's ffn1 does
 * (layer/transformer.rs:286).  The decode GEMV (m <= 2, W8A32) applies it in
 * its epilogue, other paths in a second kernel; the result is the same. */
int fh_q8_0_linear_act_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                             const float* d_bias, size_t bias_len, float* d_y, int numerics, int activation);
/* x += y, then LayerNorm of the sum into ln (forward_with_cache's residual add
 * and the LayerNorm that follows it: layer/transformer.rs:281-285, or the next
 * block's ln1 after line 288), rows of width d <= 2048.  Same arithmetic as
 * fh_add_async then fh_layernorm_async. */
int fh_add_layernorm_async(fh_ctx* ctx, float* d_x, const float* d_y, size_t rows, size_t d,
                           const float* d_gamma, const float* d_beta, float* d_ln);
/* A residual add, the LayerNorm after it and the Q8_0 linear that reads the
 * LayerNorm's output, as one call (forward_with_cache's `x + attn` -> ln2 ->
 * ffn1 -> gelu, layer/transformer.rs:281-286; `x + ffn` -> the next block's
 * ln1 -> qkv, or the final LayerNorm -> the head, slm/cached.rs:118-124):
 *   s = x + r (written to s when s is not NULL; r NULL means s = x),
 *   y = act(LayerNorm(s; gamma, beta) . W^T + bias).
 * s must not alias x or r.  Rows of width k <= 2048.  The decode GEMV
 * (m <= 2, W8A32) forms each row's mean and variance inside every wave, so
 * the whole step is one launch; other shapes run fh_add_layernorm's kernel
 * into a context buffer, then the linear. */
int fh_q8_0_linear_ln_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, const float* d_r, float* d_s,
                            size_t m, size_t k, const float* d_gamma, const float* d_beta, const float* d_bias,
                            size_t bias_len, float* d_y, int numerics, int activation);

/* ---- a GPT-2 decode position's block stack in one launch --------------------
 * CachedTransformer::feed for one token up to the final LayerNorm
 * (slm/cached.rs:100-125): embed_one (layer/embedding.rs:70-90), then every
 * block's forward_with_cache (layer/transformer.rs:221-290: LayerNorm, fused
 * Q|K|V, KV-cache append and attention, out projection, residual, LayerNorm,
 * up + GELU, down, residual), as ONE kernel launch whose workgroups exchange
 * each phase's outputs through device memory (bounded waits; a wait that gives
 * up is FH_ERR_EXCHANGE at the next fh_sync).  The same arithmetic as the
 * separate calls above, within the 1e-5 rule.  The final LayerNorm, the head
 * (fh_q8_0_linear_ln_async) and the sampler follow as usual. */
typedef struct {
    const fh_q8_0* qkv;   /* [3d x d] */
    const fh_q8_0* out;   /* [d x d] */
    const fh_q8_0* up;    /* [ffn x d] */
    const fh_q8_0* down;  /* [d x ffn] */
    const float *qkv_b, *out_b, *up_b, *down_b;  /* device */
    const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;  /* device, d each */
    float* k_cache;       /* device, [capacity, d] */
    float* v_cache;
} fh_gpt2_block;
typedef struct fh_gpt2_stack fh_gpt2_stack;
/* Builds the device state of a stack of `layers` blocks (the block table,
 * exchange slots, launch counters); weights, caches and the token / position
 * tables stay the caller's and must outlive the stack.  d = 768 or 1024 with
 * head width 64, or d = 128 with head width 32; ffn = 4 d; capacity <= 4096
 * (and within the device's LDS: 1024 at d = 768) -> else FH_ERR_LIMIT; a
 * weight of the wrong shape -> FH_ERR_DIM. */
int fh_gpt2_stack_create(fh_ctx* ctx, const fh_gpt2_block* blocks, size_t layers, size_t d, size_t heads,
                         size_t ffn, size_t capacity, const float* d_tok_w, const float* d_pos_w, size_t vocab,
                         size_t max_seq, fh_gpt2_stack** out);
void fh_gpt2_stack_free(fh_gpt2_stack* s);
/* One position: the token id is read from device memory (a sampled id feeds
 * the next step without a copy); k and v of every block are written at cache
 * row pos; the final residual stream [d] goes to d_x.  pos >= max_seq or pos >=
 * capacity -> FH_ERR_DIM with the reference's messages.  Calls on one stack
 * must not overlap. */
int fh_gpt2_stack_forward_async(fh_ctx* ctx, fh_gpt2_stack* s, const uint32_t* d_token, size_t pos, float* d_x);

/* ---- Llama / Qwen block pieces (ferrum_core llm.rs), batched over rows ------
 * Each row is one sequence of a batched decode.  Positions live on the device
 * (d_pos[r] for row r), so a decode loop can run without the host. */
enum { FH_ROPE_NORM = 0, FH_ROPE_NEOX = 1 };
/* RmsNorm::forward_row (llm.rs:58-65), x * (1 / sqrt(mean(x^2) + eps)) * w,
 * over rows of width d <= 8192.  With d_r (nullable) the residual add in front
 * of it: h = x + r is normalised and, when d_s is not NULL (it may be d_x),
 * written there (LlamaBlock::forward_one, llm.rs:445-456). */
int fh_rmsnorm_async(fh_ctx* ctx, const float* d_x, const float* d_r, float* d_s, size_t rows, size_t d,
                     const float* d_w, float eps, float* d_out);
/* apply_rope (llm.rs:146-175, angle llm.rs:118-121) in place on n_heads
 * consecutive heads of head_dim starting at d_x + r * ld, row r at position
 * d_pos[r]: FH_ROPE_NORM rotates pairs (2i, 2i+1), FH_ROPE_NEOX (i, i +
 * rope_dim/2); channels past rope_dim pass through.  d_freq_factors: NULL or
 * rope_dim / 2 divisors on the device.  Errors as Attention::new and
 * RopeScaling::check (llm.rs:123-139, 239-246): rope_dim odd or above
 * head_dim, linear_factor not finite and > 0. */
int fh_rope_async(fh_ctx* ctx, float* d_x, size_t rows, size_t ld, size_t n_heads, size_t head_dim, size_t rope_dim,
                  const uint32_t* d_pos, float base, int rope_type, const float* d_freq_factors, float linear_factor);
/* Attention::forward_one's cache append and attend (llm.rs:285-358) for
 * `rows` sequences: row r's RoPE'd [q (n_heads heads) | k (n_kv) | v (n_kv)]
 * at d_qkv + r * ld; its caches at d_k_cache / d_v_cache + r * capacity *
 * n_kv * head_dim ([capacity, n_kv * head_dim] each); k and v go to cache row
 * d_pos[r], then each query head h attends over rows 0..d_pos[r] with kv head
 * h / (n_heads / n_kv).  Output [rows, n_heads * head_dim].  max_pos bounds the
 * positions (it sizes the launch); a row whose position is above max_pos or
 * at or past capacity gets NaN and its cache is not touched.  head_dim 8, 16,
 * 32, 64 or 128.  n_heads not a multiple of n_kv is FH_ERR_DIM (llm.rs:233-238). */
int fh_gqa_attention_decode_async(fh_ctx* ctx, const float* d_qkv, size_t ld, size_t rows, size_t n_heads,
                                  size_t n_kv, size_t head_dim, float* d_k_cache, float* d_v_cache, size_t capacity,
                                  const uint32_t* d_pos, size_t max_pos, float* d_out);
/* fh_rope_async on each row's q and k heads (n_heads + n_kv heads from d_qkv
 * + r * ld), then fh_gqa_attention_decode_async: Attention::forward_one with
 * its apply_rope calls (llm.rs:285-358, 146-175) in one call.  The outputs
 * and caches are those of the two calls, bit for bit.  Many rows at head
 * width 64 take one launch that rotates q and the new k row as it reads them;
 * otherwise the two launches run.  d_qkv's q and k values are scratch: on
 * return they hold the input or its rotation.  Errors as the two calls. */
int fh_gqa_attention_rope_decode_async(fh_ctx* ctx, float* d_qkv, size_t ld, size_t rows, size_t n_heads,
                                       size_t n_kv, size_t head_dim, float* d_k_cache, float* d_v_cache,
                                       size_t capacity, const uint32_t* d_pos, size_t max_pos, size_t rope_dim,
                                       float base, int rope_type, const float* d_freq_factors, float linear_factor,
                                       float* d_out);
/* FeedForward::forward's gate (llm.rs:415-421): out[r, j] = (g / (1 +
 * exp(-g))) * u, g = d_g[r * ld + j], u = d_u[r * ld + j], j < n. */
int fh_swiglu_async(fh_ctx* ctx, const float* d_g, const float* d_u, size_t rows, size_t n, size_t ld, float* d_out);
/* LlamaModel::embed (llm.rs:588-596) for `rows` token ids on the device; an id
 * at or past vocab gives a NaN row (the sampler never returns one). */
int fh_embed_rows_async(fh_ctx* ctx, const float* d_tok_w, size_t vocab, size_t d, const uint32_t* d_tokens,
                        size_t rows, float* d_out);
/* x += y, the residual adds of TransformerBlock::forward_with_cache
 * (layer/transformer.rs:281, 288). */
int fh_add_async(fh_ctx* ctx, float* d_x, const float* d_y, size_t n);
/* The attention of TransformerBlock::forward_with_cache (layer/transformer.rs:
 * 242-279) for one new position: qkv = [q | k | v] (3d floats, the fused
 * attn_qkv output); k and v are written at row pos of the caches
 * ([capacity, d] each), then every head attends over rows 0 .. pos with scale
 * 1/sqrt(d / heads).  pos >= capacity -> FH_ERR_DIM (the reference's "KvCache
 * full" error); heads not dividing d -> FH_ERR_DIM; head widths other than 8,
 * 16, 32, 64, 128 -> FH_ERR_LIMIT. */
int fh_attention_decode_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                              size_t capacity, size_t d, size_t heads, size_t pos, float* d_out);
/* The same for a block of `rows` consecutive positions pos0 .. pos0 + rows - 1
 * of one sequence (a prompt fed at once instead of position by position, as
 * CachedTransformer::feed does one token at a time, slm/cached.rs:100-125):
 * row r of qkv ([rows, 3d]) is position pos0 + r; every row's k and v go to
 * the caches first, then row r attends over rows 0 .. pos0 + r.  The same
 * per-row arithmetic as fh_attention_decode_async (within the 1e-5 rule: the
 * chunking of the positions may differ).  pos0 + rows > capacity ->
 * FH_ERR_DIM ("KvCache full"); rows <= 65535. */
int fh_attention_prefill_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                               size_t capacity, size_t d, size_t heads, size_t pos0, size_t rows, float* d_out);
/* fh_attention_prefill_async for `seqs` independent sequences in one call: the
 * prime of each sequence's CachedTransformer (slm/cached.rs:129-136) through
 * forward_with_cache's attention (layer/transformer.rs:242-279), every
 * sequence's block at positions pos0 .. pos0 + rows - 1.  Sequence s's rows are
 * rows s * rows .. s * rows + rows - 1 of d_qkv ([seqs * rows, 3d]) and d_out
 * ([seqs * rows, d]); its caches start at d_k_cache / d_v_cache + s *
 * seq_stride (floats; seq_stride >= capacity * d when seqs > 1).  Head width
 * 64 runs on the f16 matrix cores with every f32 operand as two f16 terms
 * (three f16 products per product); within the 1e-5 rule of the reference.
 * Errors as fh_attention_prefill_async; seqs <= 65535. */
int fh_attention_prefill_seqs_async(fh_ctx* ctx, const float* d_qkv, float* d_k_cache, float* d_v_cache,
                                    size_t seq_stride, size_t capacity, size_t d, size_t heads, size_t pos0,
                                    size_t rows, size_t seqs, float* d_out);

/* ---- a batched decode step's residual adds and norms, fused into the linears ---
 * The block of forward_with_cache (layer/transformer.rs:221-294; Llama:
 * LlamaBlock::forward_one, llm.rs:445-456) adds each projection to the
 * residual stream and normalises the sum before the next linear.  These two
 * entry points carry that between two linears without a norm launch:
 *   fh_q8_0_linear_residual_async  y = r + (x W^T + b) (y may be r: the
 *       residual stream updated in place) and, with d_stats, y's row
 *       statistics: per row i and 32-column group g of the n outputs, the
 *       group's mean and sum of squared deviations at d_stats[(i * n/32 + g) * 2]
 *       (n % 32 == 0);
 *   fh_q8_0_linear_normed_async    y = act(norm(x) W^T + b), norm formed
 *       from such statistics of x: LayerNorm::forward (layer/norm.rs:46-82:
 *       rms = 0, gamma, beta, eps 1e-5 there) or RmsNorm::forward_row
 *       (llm.rs:58-65: rms = 1, gamma = its weight, beta NULL).
 * W8A32 numerics (the 1e-5 rule); 3 <= m <= 64 runs each as one skinny-GEMM
 * launch, other shapes as the linear plus a small kernel.  k % 32 == 0 for the
 * normed form.  The normed form's activation may be FH_ACT_SWIGLU32 (a Llama
 * block's gate|up: y is [m][n / 2]) for Q8_0 weights with n % 64 == 0 at
 * 3 <= m <= 64 and k <= 1024, FH_ERR_LIMIT elsewhere.  Errors as
 * fh_q8_0_linear_async ("linear_forward: ..."), FH_ERR_INVALID for a missing
 * pointer or y aliasing x. */
int fh_q8_0_linear_residual_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                  const float* d_bias, size_t bias_len, const float* d_r, float* d_y,
                                  float* d_stats);
int fh_q8_0_linear_normed_async(fh_ctx* ctx, const fh_q8_0* w, const float* d_x, size_t m, size_t k,
                                const float* d_stats, const float* d_gamma, const float* d_beta, float eps, int rms,
                                const float* d_bias, size_t bias_len, float* d_y, int activation);

/* ---- packed per-row int8 / int4 weights: ops::qlinear (ops.rs:268-377) ------
 * QWeight (quant.rs:130-217): k rows (input features) x n columns (outputs),
 * one f32 scale per row, int8 levels ([k][n] bytes) or int4 levels in the
 * split-half nibble layout ([k][ceil(n/2)] bytes: column c < half in the low
 * nibble of byte c, else the high nibble of byte c - half). */
enum { FH_QINT8 = 0, FH_QINT4 = 1 };
typedef struct fh_qweight fh_qweight;
/* Host scales [k] and levels as the reference stores them; the device copy pads
 * each row to 64 bytes.  Blocks until the copy is done. */
int fh_qweight_upload(fh_ctx* ctx, const float* scales, const uint8_t* q, size_t k, size_t n, int kind,
                      fh_qweight** out);
void fh_qweight_free(fh_qweight* w);
/* y[i, j] = b[j] + sum over p ascending of (x[i, p] * scale[p]) * level(p, j),
 * bias first and no FMA, as qaccum_cols: the reference's outputs bit for bit.
 * d_x [m, k], d_y [m, n] device pointers; bias NULL (bias_len 0) means zeros.
 * Errors as qlinear: "qlinear: input width K ≠ weight rows R", "qlinear: bias
 * length B ≠ out_features N" (FH_ERR_DIM). */
int fh_qlinear_async(fh_ctx* ctx, const fh_qweight* w, const float* d_x, size_t m, size_t k, const float* d_bias,
                     size_t bias_len, float* d_y);

/* ---- GGUF reader (gguf/mod.rs:208-310, gguf/header.rs, gguf/tensors.rs:26-87) ----
 * The file is memory-mapped read-only and parsed as ferrum_core's parse_header
 * does: magic "GGUF", version 2 or 3, metadata table, tensor directory, data
 * at the next multiple of general.alignment (default 32); every sized tensor
 * must lie inside the file and no two may overlap.  Host-only calls, no GPU
 * needed, except fh_gguf_upload_q8_0. */
typedef struct fh_gguf fh_gguf;
/* Always sets *out (even on failure, so fh_gguf_error can say why); close it
 * with fh_gguf_close.  A malformed file is FH_ERR_FORMAT with the reference's
 * messages ("not a GGUF file (bad magic)", "unsupported GGUF version N (need 2
 * or 3)", "GGUF truncated at +P: need N bytes, file has T", "tensor 'X' data
 * runs past EOF", "tensors 'X' and 'Y' overlap", ...). */
int fh_gguf_open(const char* path, fh_gguf** out);
void fh_gguf_close(fh_gguf* g);
const char* fh_gguf_error(const fh_gguf* g);
uint32_t fh_gguf_version(const fh_gguf* g);
size_t fh_gguf_tensor_count(const fh_gguf* g);
/* Index of the first tensor called name, or -1 (Gguf::tensor). */
long fh_gguf_find_tensor(const fh_gguf* g, const char* name);
/* dims: room for 8 (GGML order: dims[0] = ne0, the contiguous one); nbytes 0
 * for a type the reader cannot size (gguf/format.rs:87-129). */
int fh_gguf_tensor_info(const fh_gguf* g, size_t i, const char** name, uint32_t* n_dims, uint64_t* dims,
                        uint32_t* ggml_type, uint64_t* nbytes);
/* Host pointer to the tensor's bytes inside the mapping (valid until close). */
const void* fh_gguf_tensor_data(const fh_gguf* g, size_t i);
/* Metadata: the value type (GGUF value type codes), the element type and
 * length of an array; integer / bool values as u64; numbers as f64; a string
 * or element `index` of a string array. */
int fh_gguf_meta_type(const fh_gguf* g, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* count);
int fh_gguf_meta_u64(const fh_gguf* g, const char* key, uint64_t* out);
int fh_gguf_meta_f64(const fh_gguf* g, const char* key, double* out);
int fh_gguf_meta_str(const fh_gguf* g, const char* key, size_t index, const char** out, size_t* len);
/* Raw little-endian elements of a numeric array. */
int fh_gguf_meta_array_data(const fh_gguf* g, const char* key, const void** data, size_t* elem_size);
/* An F32 or F16 tensor of n elements into host floats (F16 decoded exactly,
 * gguf/dequant.rs:7-35).  ctx may be NULL (the message is then not kept). */
int fh_gguf_read_f32(fh_ctx* ctx, const fh_gguf* g, const char* name, float* out, size_t n);
/* A Q8_0 tensor [ne0 = k, ne1 = n] straight from the mapping to the device, as
 * fh_q8_0_upload (GgufIn::rows/matrix/linear, loader/decode.rs:57-81, without
 * the f32 expansion). */
int fh_gguf_upload_q8_0(fh_ctx* ctx, const fh_gguf* g, const char* name, fh_q8_0** out);

#ifdef __cplusplus
}
#endif
#endif /* FERRUM_HIP_H */
