//! Safe Rust binding of `libferrum_hip`, the MI355X (gfx950) implementation of
//! ferrum_core's decode-step hot path: GGUF Q8_0 linears (`ops::linear_forward`,
//! `ops.rs:233-256`, reached from `Linear::forward`, `layer/linear.rs:177-210`)
//! and the fused logit sampler (`sample_with_params`, `slm/sampling.rs:124-210`).
//!
//! All `unsafe` code a device-backed ferrum_core needs lives here, so
//! ferrum_core keeps `#![forbid(unsafe_code)]`.  [`sys`] declares every entry
//! point of `include/ferrum_hip.h` one to one; the safe types wrap the host-
//! pointer calls and own the handles:
//!
//! * [`Device`]: one context (a HIP device and stream).  The library's context
//!   is single-threaded, so every call holds the context's mutex for the whole
//!   foreign call (the guard is bound to a local that outlives the call).
//! * [`Weight`]: a device-resident Q8_0 (or F32) weight, freed on drop.
//! * [`Gguf`]: the library's memory-mapped GGUF reader.
//!
//! Device-pointer (`*_async`) entry points are reached through
//! [`Device::with_raw`], which hands a closure the raw context while the lock
//! is held.
#![deny(unsafe_op_in_unsafe_fn)]

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::{c_char, c_int};
use std::path::Path;
use std::sync::{Mutex, MutexGuard};

/// The C ABI, one declaration per entry point of `include/ferrum_hip.h`.
#[allow(non_camel_case_types)]
pub mod sys {
    use std::os::raw::{c_char, c_int, c_long, c_void};

    #[repr(C)]
    pub struct fh_ctx {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct fh_q8_0 {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct fh_gpt2_stack {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct fh_qweight {
        _p: [u8; 0],
    }
    #[repr(C)]
    pub struct fh_gguf {
        _p: [u8; 0],
    }

    /// `slm/sampling.rs:27-38` without the cancel flag (a host-side control).
    #[repr(C)]
    #[derive(Clone, Copy, Debug, PartialEq)]
    pub struct fh_sampling_params {
        pub temperature: f32,
        pub top_k: u32,
        pub top_p: f32,
        pub repetition_penalty: f32,
    }

    /// One GPT-2 block for `fh_gpt2_stack_create` (device pointers).
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct fh_gpt2_block {
        pub qkv: *const fh_q8_0,
        pub out: *const fh_q8_0,
        pub up: *const fh_q8_0,
        pub down: *const fh_q8_0,
        pub qkv_b: *const f32,
        pub out_b: *const f32,
        pub up_b: *const f32,
        pub down_b: *const f32,
        pub ln1_g: *const f32,
        pub ln1_b: *const f32,
        pub ln2_g: *const f32,
        pub ln2_b: *const f32,
        pub k_cache: *mut f32,
        pub v_cache: *mut f32,
    }

    pub const FH_OK: c_int = 0;
    pub const FH_ERR_DIM: c_int = 1;
    pub const FH_ERR_INVALID: c_int = 2;
    pub const FH_ERR_OOM: c_int = 3;
    pub const FH_ERR_HIP: c_int = 4;
    pub const FH_ERR_LIMIT: c_int = 5;
    pub const FH_ERR_FORMAT: c_int = 6;
    pub const FH_ERR_EXCHANGE: c_int = 7;
    pub const FH_STATUS_EXCHANGE: c_int = 1;
    pub const FH_STATUS_BAD_OFFSETS: c_int = 2;
    pub const FH_W8A32: c_int = 0;
    pub const FH_W8A8: c_int = 1;
    pub const FH_W8A32_EXACT: c_int = 2;
    pub const FH_W8A8_FAST: c_int = 3;
    pub const FH_LOGITS_RAW: c_int = 0;
    pub const FH_LOGITS_GPT2_SOFTMAX: c_int = 1;
    pub const FH_RECENT_RANGES: c_int = 0x100;
    pub const FH_ACT_NONE: c_int = 0;
    pub const FH_ACT_GELU: c_int = 1;
    pub const FH_ACT_SWIGLU32: c_int = 2;
    pub const FH_ROPE_NORM: c_int = 0;
    pub const FH_ROPE_NEOX: c_int = 1;
    pub const FH_QINT8: c_int = 0;
    pub const FH_QINT4: c_int = 1;

    #[link(name = "ferrum_hip")]
    extern "C" {
        pub fn fh_ctx_create(device: c_int, out: *mut *mut fh_ctx) -> c_int;
        pub fn fh_ctx_destroy(ctx: *mut fh_ctx);
        pub fn fh_ctx_set_stream(ctx: *mut fh_ctx, hip_stream: *mut c_void) -> c_int;
        pub fn fh_ctx_reset_stream(ctx: *mut fh_ctx) -> c_int;
        pub fn fh_sync(ctx: *mut fh_ctx) -> c_int;
        pub fn fh_last_error(ctx: *const fh_ctx) -> *const c_char;
        pub fn fh_device_count() -> c_int;
        pub fn fh_q8_0_upload(ctx: *mut fh_ctx, gguf_bytes: *const u8, n_rows: usize, k: usize, out: *mut *mut fh_q8_0) -> c_int;
        pub fn fh_q8_0_upload_device(ctx: *mut fh_ctx, d_gguf_bytes: *const u8, n_rows: usize, k: usize, out: *mut *mut fh_q8_0) -> c_int;
        pub fn fh_weight_upload_f32(ctx: *mut fh_ctx, rows: *const f32, n_rows: usize, k: usize, out: *mut *mut fh_q8_0) -> c_int;
        pub fn fh_weight_kind(w: *const fh_q8_0) -> c_int;
        pub fn fh_q8_0_download(ctx: *mut fh_ctx, w: *const fh_q8_0, gguf_bytes: *mut u8) -> c_int;
        pub fn fh_q8_0_dims(w: *const fh_q8_0, n_rows: *mut usize, k: *mut usize) -> c_int;
        pub fn fh_q8_0_free(w: *mut fh_q8_0);
        pub fn fh_q8_0_linear(ctx: *mut fh_ctx, w: *const fh_q8_0, x: *const f32, m: usize, k: usize, bias: *const f32, bias_len: usize, y: *mut f32, numerics: c_int) -> c_int;
        pub fn fh_q8_0_linear_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, m: usize, k: usize, d_bias: *const f32, bias_len: usize, d_y: *mut f32, numerics: c_int) -> c_int;
        pub fn fh_q8_0_linear_noalloc_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, m: usize, k: usize, d_bias: *const f32, bias_len: usize, d_y: *mut f32, numerics: c_int) -> c_int;
        pub fn fh_q8_0_encode(ctx: *mut fh_ctx, x: *const f32, n: usize, out: *mut u8) -> c_int;
        pub fn fh_q8_0_encode_async(ctx: *mut fh_ctx, d_x: *const f32, n: usize, d_out: *mut u8) -> c_int;
        pub fn fh_q8_0_dequant_async(ctx: *mut fh_ctx, d_gguf_bytes: *const u8, n: usize, d_out: *mut f32) -> c_int;
        pub fn fh_q8_0_block_dots_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_qx: *const i8, m: usize, d_dots: *mut i32) -> c_int;
        pub fn fh_sample_rows(ctx: *mut fh_ctx, logits: *const f32, rows: usize, vocab: usize, logits_kind: c_int, params: *const fh_sampling_params, recent: *const u32, recent_offsets: *const u32, draws: *const u64, out_ids: *mut u32) -> c_int;
        pub fn fh_sample_rows_async(ctx: *mut fh_ctx, d_logits: *const f32, rows: usize, vocab: usize, logits_kind: c_int, params: *const fh_sampling_params, d_recent: *const u32, d_recent_offsets: *const u32, d_draws: *const u64, d_out_ids: *mut u32) -> c_int;
        pub fn fh_debug_sampler_faults(ctx: *mut fh_ctx, skip_segment: c_int, spin_limit: u32) -> c_int;
        pub fn fh_embed_one_async(ctx: *mut fh_ctx, d_token_w: *const f32, d_pos_w: *const f32, vocab: usize, max_seq: usize, d: usize, d_token: *const u32, pos: usize, d_out: *mut f32) -> c_int;
        pub fn fh_layernorm_async(ctx: *mut fh_ctx, d_x: *const f32, rows: usize, d: usize, d_gamma: *const f32, d_beta: *const f32, d_y: *mut f32) -> c_int;
        pub fn fh_gelu_async(ctx: *mut fh_ctx, d_x: *mut f32, n: usize) -> c_int;
        pub fn fh_q8_0_linear_act_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, m: usize, k: usize, d_bias: *const f32, bias_len: usize, d_y: *mut f32, numerics: c_int, activation: c_int) -> c_int;
        pub fn fh_add_layernorm_async(ctx: *mut fh_ctx, d_x: *mut f32, d_y: *const f32, rows: usize, d: usize, d_gamma: *const f32, d_beta: *const f32, d_ln: *mut f32) -> c_int;
        pub fn fh_q8_0_linear_ln_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, d_r: *const f32, d_s: *mut f32, m: usize, k: usize, d_gamma: *const f32, d_beta: *const f32, d_bias: *const f32, bias_len: usize, d_y: *mut f32, numerics: c_int, activation: c_int) -> c_int;
        pub fn fh_gpt2_stack_create(ctx: *mut fh_ctx, blocks: *const fh_gpt2_block, layers: usize, d: usize, heads: usize, ffn: usize, capacity: usize, d_tok_w: *const f32, d_pos_w: *const f32, vocab: usize, max_seq: usize, out: *mut *mut fh_gpt2_stack) -> c_int;
        pub fn fh_gpt2_stack_free(s: *mut fh_gpt2_stack);
        pub fn fh_gpt2_stack_forward_async(ctx: *mut fh_ctx, s: *mut fh_gpt2_stack, d_token: *const u32, pos: usize, d_x: *mut f32) -> c_int;
        pub fn fh_rmsnorm_async(ctx: *mut fh_ctx, d_x: *const f32, d_r: *const f32, d_s: *mut f32, rows: usize, d: usize, d_w: *const f32, eps: f32, d_out: *mut f32) -> c_int;
        pub fn fh_rope_async(ctx: *mut fh_ctx, d_x: *mut f32, rows: usize, ld: usize, n_heads: usize, head_dim: usize, rope_dim: usize, d_pos: *const u32, base: f32, rope_type: c_int, d_freq_factors: *const f32, linear_factor: f32) -> c_int;
        pub fn fh_gqa_attention_decode_async(ctx: *mut fh_ctx, d_qkv: *const f32, ld: usize, rows: usize, n_heads: usize, n_kv: usize, head_dim: usize, d_k_cache: *mut f32, d_v_cache: *mut f32, capacity: usize, d_pos: *const u32, max_pos: usize, d_out: *mut f32) -> c_int;
        pub fn fh_gqa_attention_rope_decode_async(ctx: *mut fh_ctx, d_qkv: *mut f32, ld: usize, rows: usize, n_heads: usize, n_kv: usize, head_dim: usize, d_k_cache: *mut f32, d_v_cache: *mut f32, capacity: usize, d_pos: *const u32, max_pos: usize, rope_dim: usize, base: f32, rope_type: c_int, d_freq_factors: *const f32, linear_factor: f32, d_out: *mut f32) -> c_int;
        pub fn fh_swiglu_async(ctx: *mut fh_ctx, d_g: *const f32, d_u: *const f32, rows: usize, n: usize, ld: usize, d_out: *mut f32) -> c_int;
        pub fn fh_embed_rows_async(ctx: *mut fh_ctx, d_tok_w: *const f32, vocab: usize, d: usize, d_tokens: *const u32, rows: usize, d_out: *mut f32) -> c_int;
        pub fn fh_embed_rows_pos_async(ctx: *mut fh_ctx, d_token_w: *const f32, d_pos_w: *const f32, vocab: usize, max_seq: usize, d: usize, d_tokens: *const u32, d_pos: *const u32, rows: usize, d_hist: *mut u32, hist_stride: usize, d_out: *mut f32) -> c_int;
        pub fn fh_add_async(ctx: *mut fh_ctx, d_x: *mut f32, d_y: *const f32, n: usize) -> c_int;
        pub fn fh_attention_decode_async(ctx: *mut fh_ctx, d_qkv: *const f32, d_k_cache: *mut f32, d_v_cache: *mut f32, capacity: usize, d: usize, heads: usize, pos: usize, d_out: *mut f32) -> c_int;
        pub fn fh_attention_prefill_async(ctx: *mut fh_ctx, d_qkv: *const f32, d_k_cache: *mut f32, d_v_cache: *mut f32, capacity: usize, d: usize, heads: usize, pos0: usize, rows: usize, d_out: *mut f32) -> c_int;
        pub fn fh_q8_0_linear_residual_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, m: usize, k: usize, d_bias: *const f32, bias_len: usize, d_r: *const f32, d_y: *mut f32, d_stats: *mut f32) -> c_int;
        pub fn fh_q8_0_linear_normed_async(ctx: *mut fh_ctx, w: *const fh_q8_0, d_x: *const f32, m: usize, k: usize, d_stats: *const f32, d_gamma: *const f32, d_beta: *const f32, eps: f32, rms: c_int, d_bias: *const f32, bias_len: usize, d_y: *mut f32, activation: c_int) -> c_int;
        pub fn fh_attention_prefill_seqs_async(ctx: *mut fh_ctx, d_qkv: *const f32, d_k_cache: *mut f32, d_v_cache: *mut f32, seq_stride: usize, capacity: usize, d: usize, heads: usize, pos0: usize, rows: usize, seqs: usize, d_out: *mut f32) -> c_int;
        pub fn fh_qweight_upload(ctx: *mut fh_ctx, scales: *const f32, q: *const u8, k: usize, n: usize, kind: c_int, out: *mut *mut fh_qweight) -> c_int;
        pub fn fh_qweight_free(w: *mut fh_qweight);
        pub fn fh_qlinear_async(ctx: *mut fh_ctx, w: *const fh_qweight, d_x: *const f32, m: usize, k: usize, d_bias: *const f32, bias_len: usize, d_y: *mut f32) -> c_int;
        pub fn fh_gguf_open(path: *const c_char, out: *mut *mut fh_gguf) -> c_int;
        pub fn fh_gguf_close(g: *mut fh_gguf);
        pub fn fh_gguf_error(g: *const fh_gguf) -> *const c_char;
        pub fn fh_gguf_version(g: *const fh_gguf) -> u32;
        pub fn fh_gguf_tensor_count(g: *const fh_gguf) -> usize;
        pub fn fh_gguf_find_tensor(g: *const fh_gguf, name: *const c_char) -> c_long;
        pub fn fh_gguf_tensor_info(g: *const fh_gguf, i: usize, name: *mut *const c_char, n_dims: *mut u32, dims: *mut u64, ggml_type: *mut u32, nbytes: *mut u64) -> c_int;
        pub fn fh_gguf_tensor_data(g: *const fh_gguf, i: usize) -> *const c_void;
        pub fn fh_gguf_meta_type(g: *const fh_gguf, key: *const c_char, type_: *mut u32, elem_type: *mut u32, count: *mut u64) -> c_int;
        pub fn fh_gguf_meta_u64(g: *const fh_gguf, key: *const c_char, out: *mut u64) -> c_int;
        pub fn fh_gguf_meta_f64(g: *const fh_gguf, key: *const c_char, out: *mut f64) -> c_int;
        pub fn fh_gguf_meta_str(g: *const fh_gguf, key: *const c_char, index: usize, out: *mut *const c_char, len: *mut usize) -> c_int;
        pub fn fh_gguf_meta_array_data(g: *const fh_gguf, key: *const c_char, data: *mut *const c_void, elem_size: *mut usize) -> c_int;
        pub fn fh_gguf_read_f32(ctx: *mut fh_ctx, g: *const fh_gguf, name: *const c_char, out: *mut f32, n: usize) -> c_int;
        pub fn fh_gguf_upload_q8_0(ctx: *mut fh_ctx, g: *const fh_gguf, name: *const c_char, out: *mut *mut fh_q8_0) -> c_int;
    }
}

/// A failed call: the library's status code and its message
/// (`fh_last_error`).  `Dim` is ferrum_core's `InferError::DimMismatch`
/// (the message is the reference's own text), `Format` its
/// `InferError::Format`.
#[derive(Clone, Debug, PartialEq, Eq)]
pub enum Error {
    Dim(String),
    Invalid(String),
    OutOfMemory(String),
    Hip(String),
    Limit(String),
    Format(String),
    /// A kernel's bounded cross-workgroup wait gave up (the GPU was shared):
    /// results since the last sync are unreliable.
    Exchange(String),
    Other(i32, String),
}

impl Error {
    fn from_code(code: c_int, msg: String) -> Error {
        match code {
            sys::FH_ERR_DIM => Error::Dim(msg),
            sys::FH_ERR_INVALID => Error::Invalid(msg),
            sys::FH_ERR_OOM => Error::OutOfMemory(msg),
            sys::FH_ERR_HIP => Error::Hip(msg),
            sys::FH_ERR_LIMIT => Error::Limit(msg),
            sys::FH_ERR_FORMAT => Error::Format(msg),
            sys::FH_ERR_EXCHANGE => Error::Exchange(msg),
            c => Error::Other(c, msg),
        }
    }
    /// The message without the kind.
    pub fn message(&self) -> &str {
        match self {
            Error::Dim(m) | Error::Invalid(m) | Error::OutOfMemory(m) | Error::Hip(m) | Error::Limit(m)
            | Error::Format(m) | Error::Exchange(m) | Error::Other(_, m) => m,
        }
    }
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            Error::Other(c, m) => write!(f, "ferrum_hip status {c}: {m}"),
            e => write!(f, "ferrum_hip: {}", e.message()),
        }
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

/// Numerics of a Q8_0 linear (`FH_W8A32` ...; see the header).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Numerics {
    /// ferrum_core's semantics (exact dequantisation, f32 products and sums),
    /// within the 1e-5 rule.
    W8A32,
    /// llama.cpp's (activations re-quantised to Q8_0 per 32).
    W8A8,
    /// ferrum_core's sums bit for bit (ascending k, no FMA, bias last).
    W8A32Exact,
    /// `W8A8` with each block's term fused into the sum (one rounding),
    /// within the 1e-5 rule of `W8A8`'s outputs: the prefill speed mode.
    W8A8Fast,
}

/// The drop-in default is the bit-exact mode: `ops::linear_forward`'s bits on
/// the f32 expansion, which the reference plan's packed-Q8_0 contract
/// (`q8_0_packed_forward_equals_expanded`) asserts.  `W8A32` is the opt-in
/// fast mode (within the 1e-5 rule, not bit-identical).
impl Default for Numerics {
    fn default() -> Self {
        Numerics::W8A32Exact
    }
}

impl Numerics {
    fn code(self) -> c_int {
        match self {
            Numerics::W8A32 => sys::FH_W8A32,
            Numerics::W8A8 => sys::FH_W8A8,
            Numerics::W8A32Exact => sys::FH_W8A32_EXACT,
            Numerics::W8A8Fast => sys::FH_W8A8_FAST,
        }
    }
}

/// What the sampler receives.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Logits {
    /// The sampler input itself (the Llama / Qwen path, `llm.rs:745`).
    Raw,
    /// The GPT-2 head's raw scores: softmax and the `ln(max(p, 1e-12))` bridge
    /// are fused in (`slm/token_stream.rs:134`).
    Gpt2Softmax,
}

impl Logits {
    fn code(self) -> c_int {
        match self {
            Logits::Raw => sys::FH_LOGITS_RAW,
            Logits::Gpt2Softmax => sys::FH_LOGITS_GPT2_SOFTMAX,
        }
    }
}

pub use sys::fh_sampling_params as SamplingParams;

impl SamplingParams {
    pub fn new(temperature: f32, top_k: u32, top_p: f32, repetition_penalty: f32) -> SamplingParams {
        SamplingParams { temperature, top_k, top_p, repetition_penalty }
    }
}

/// The raw context pointer, owned by a [`Device`].
struct Ctx(*mut sys::fh_ctx);
// The context is used by one thread at a time: every access goes through the
// Device's mutex.
unsafe impl Send for Ctx {}

/// One HIP device and stream (an `fh_ctx`).  `Send + Sync`: calls from several
/// threads are serialised on the context's mutex, held across each foreign call.
pub struct Device {
    ctx: Mutex<Ctx>,
}

/// Number of HIP devices visible (0 when none).
pub fn device_count() -> usize {
    // SAFETY: takes no arguments and touches no caller memory.
    let n = unsafe { sys::fh_device_count() };
    n.max(0) as usize
}

fn last_error(ctx: *const sys::fh_ctx) -> String {
    // SAFETY: fh_last_error returns a NUL-terminated string owned by the
    // context (or the library, for ctx NULL) that stays valid until the next
    // call on that context; it is copied out before the lock is released.
    unsafe { CStr::from_ptr(sys::fh_last_error(ctx)).to_string_lossy().into_owned() }
}

impl Device {
    /// `fh_ctx_create`: a context on HIP device `device` with its own stream.
    pub fn new(device: i32) -> Result<Device> {
        let mut c: *mut sys::fh_ctx = std::ptr::null_mut();
        // SAFETY: `c` is a valid out-pointer.
        let rc = unsafe { sys::fh_ctx_create(device, &mut c) };
        if rc != sys::FH_OK {
            return Err(Error::from_code(rc, last_error(std::ptr::null())));
        }
        Ok(Device { ctx: Mutex::new(Ctx(c)) })
    }

    fn lock(&self) -> MutexGuard<'_, Ctx> {
        // A panic while the lock was held leaves no broken invariant on the
        // Rust side (the context only holds device state), so take it anyway.
        self.ctx.lock().unwrap_or_else(|p| p.into_inner())
    }

    /// Run `f` with the raw context while the context's lock is held; the
    /// status `f` returns is turned into a Result with the context's message.
    /// This is the door to the device-pointer (`*_async`) entry points.
    ///
    /// # Safety
    /// `f` calls into [`sys`] with the given context: every pointer it passes
    /// must be valid for the call as the header documents it (device pointers
    /// for the `_async` forms), and work it enqueues must not outlive the
    /// buffers it names (call [`Device::sync`] first).
    pub unsafe fn with_raw<F: FnOnce(*mut sys::fh_ctx) -> c_int>(&self, f: F) -> Result<()> {
        let guard = self.lock();
        let c = guard.0;
        let rc = f(c);
        let out = if rc == sys::FH_OK { Ok(()) } else { Err(Error::from_code(rc, last_error(c))) };
        drop(guard);
        out
    }

    /// Call a blocking entry point with the lock held for the whole call.
    fn call<F: FnOnce(*mut sys::fh_ctx) -> c_int>(&self, f: F) -> Result<()> {
        let guard = self.lock();
        let c = guard.0;
        let rc = f(c);
        let out = if rc == sys::FH_OK { Ok(()) } else { Err(Error::from_code(rc, last_error(c))) };
        drop(guard);
        out
    }

    /// `fh_sync`: wait for the context's stream; reports a failed exchange or
    /// decreasing device-form offsets recorded since the last sync.
    pub fn sync(&self) -> Result<()> {
        // SAFETY: the context pointer is valid while `self` lives.
        self.call(|c| unsafe { sys::fh_sync(c) })
    }

    /// `fh_q8_0_upload`: the raw bytes of a GGUF Q8_0 tensor with ne0 = k and
    /// ne1 = n_rows (`Gguf::tensor_bytes`), kept as Q8_0 on the device.
    pub fn upload_q8_0(&self, gguf_bytes: &[u8], n_rows: usize, k: usize) -> Result<Weight> {
        if k % 32 == 0 && gguf_bytes.len() != n_rows * (k / 32) * 34 {
            return Err(Error::Invalid(format!(
                "fh_q8_0_upload: expected {} bytes, got {}",
                n_rows * (k / 32) * 34,
                gguf_bytes.len()
            )));
        }
        let mut w: *mut sys::fh_q8_0 = std::ptr::null_mut();
        // SAFETY: gguf_bytes holds n_rows * k / 32 * 34 bytes (checked above;
        // the library refuses k % 32 != 0 before reading), `w` is an out-pointer.
        self.call(|c| unsafe { sys::fh_q8_0_upload(c, gguf_bytes.as_ptr(), n_rows, k, &mut w) })?;
        Ok(Weight { w, n_rows, k })
    }

    /// `fh_weight_upload_f32`: an F32 matrix [n_rows x k] (GGUF row order),
    /// for tensors the reference stores as F32 (`loader/mod.rs:147-152`).
    pub fn upload_f32(&self, rows: &[f32], n_rows: usize, k: usize) -> Result<Weight> {
        if rows.len() != n_rows * k {
            return Err(Error::Invalid(format!("fh_weight_upload_f32: expected {} values, got {}", n_rows * k, rows.len())));
        }
        let mut w: *mut sys::fh_q8_0 = std::ptr::null_mut();
        // SAFETY: rows holds n_rows * k floats; `w` is an out-pointer.
        self.call(|c| unsafe { sys::fh_weight_upload_f32(c, rows.as_ptr(), n_rows, k, &mut w) })?;
        Ok(Weight { w, n_rows, k })
    }

    /// `ops::linear_forward` (`bias` of length n_rows) or `ops::matmul`
    /// (`bias` empty): x [m, k] row-major -> y [m, n_rows].  Host slices; the
    /// call blocks until y is written.  A width or bias length that does not
    /// fit is `Error::Dim` with the reference's message.
    pub fn linear_forward(&self, x: &[f32], m: usize, w: &Weight, bias: &[f32], numerics: Numerics) -> Result<Vec<f32>> {
        let k = if m == 0 { w.k } else { x.len() / m };
        if m != 0 && x.len() != m * k {
            return Err(Error::Invalid(format!("linear_forward: {} inputs do not form {m} rows", x.len())));
        }
        let mut y = vec![0.0f32; m * w.n_rows];
        let b = if bias.is_empty() { std::ptr::null() } else { bias.as_ptr() };
        // SAFETY: x holds m * k floats, bias bias.len() (NULL when empty), y
        // m * n_rows; the weight handle is alive for the call.
        self.call(|c| unsafe {
            sys::fh_q8_0_linear(c, w.w, x.as_ptr(), m, k, b, bias.len(), y.as_mut_ptr(), numerics.code())
        })?;
        Ok(y)
    }

    /// `fh_q8_0_encode`: f32 values (a multiple of 32) to GGUF Q8_0 bytes with
    /// `q8_0_block` (`quant.rs:271-280`), bit for bit.
    pub fn encode_q8_0(&self, x: &[f32]) -> Result<Vec<u8>> {
        let mut out = vec![0u8; x.len() / 32 * 34];
        // SAFETY: out holds len / 32 * 34 bytes (the library refuses lengths
        // off the block grid before writing).
        self.call(|c| unsafe { sys::fh_q8_0_encode(c, x.as_ptr(), x.len(), out.as_mut_ptr()) })?;
        Ok(out)
    }

    /// `sample_with_params` for `rows` rows of `vocab` logits, each with its
    /// penalty history (`recent[r]`) and its draw (`rng.next_u64()`, taken by
    /// the caller once per row, none when greedy): the ids, as the reference
    /// picks them.
    pub fn sample_rows(&self, logits: &[f32], vocab: usize, kind: Logits, params: &SamplingParams,
                       recent: &[&[u32]], draws: Option<&[u64]>) -> Result<Vec<u32>> {
        let rows = recent.len();
        if logits.len() != rows * vocab {
            return Err(Error::Invalid(format!("fh_sample_rows: {} logits are not {rows} rows of {vocab}", logits.len())));
        }
        if let Some(d) = draws {
            if d.len() != rows {
                return Err(Error::Invalid(format!("fh_sample_rows: {} draws for {rows} rows", d.len())));
            }
        }
        let mut flat: Vec<u32> = Vec::new();
        let mut offsets: Vec<u32> = Vec::with_capacity(rows + 1);
        offsets.push(0);
        for r in recent {
            flat.extend_from_slice(r);
            offsets.push(u32::try_from(flat.len()).map_err(|_| Error::Limit("fh_sample_rows: more than 2^32 recent ids".into()))?);
        }
        let mut out = vec![0u32; rows];
        let rec = if flat.is_empty() { std::ptr::null() } else { flat.as_ptr() };
        let dr = draws.map_or(std::ptr::null(), |d| d.as_ptr());
        // SAFETY: logits holds rows * vocab floats, offsets rows + 1 entries
        // into `flat`, draws (when given) rows values, out rows ids.
        self.call(|c| unsafe {
            sys::fh_sample_rows(c, logits.as_ptr(), rows, vocab, kind.code(), params, rec, offsets.as_ptr(), dr,
                                out.as_mut_ptr())
        })?;
        Ok(out)
    }
}

impl Drop for Device {
    fn drop(&mut self) {
        let c = self.ctx.get_mut().unwrap_or_else(|p| p.into_inner()).0;
        // SAFETY: the context was created by fh_ctx_create and is destroyed
        // once; `&mut self` means no call is in flight on it.
        unsafe { sys::fh_ctx_destroy(c) }
    }
}

/// A device-resident weight (`fh_q8_0`): Q8_0 rows, or F32 rows for a tensor
/// the reference stores as F32.  Freed on drop.
pub struct Weight {
    w: *mut sys::fh_q8_0,
    pub n_rows: usize,
    pub k: usize,
}

// The library never writes a weight after its upload, and frees it only
// through Drop (exclusive access): sharing it between threads is sound.
unsafe impl Send for Weight {}
unsafe impl Sync for Weight {}

impl Weight {
    /// The raw handle, for [`Device::with_raw`] calls (valid while `self` lives).
    pub fn as_ptr(&self) -> *const sys::fh_q8_0 {
        self.w
    }
    /// True for an F32 weight.
    pub fn is_f32(&self) -> bool {
        // SAFETY: the handle is alive.
        unsafe { sys::fh_weight_kind(self.w) == 1 }
    }
    /// `fh_q8_0_download`: the GGUF Q8_0 bytes back (Q8_0 weights only).
    pub fn download(&self, dev: &Device) -> Result<Vec<u8>> {
        let mut out = vec![0u8; self.n_rows * (self.k / 32) * 34];
        // SAFETY: out holds the tensor's byte count; the handle is alive.
        dev.call(|c| unsafe { sys::fh_q8_0_download(c, self.w, out.as_mut_ptr()) })?;
        Ok(out)
    }
}

impl Drop for Weight {
    fn drop(&mut self) {
        // SAFETY: freed once; fh_q8_0_free waits for the device's queued work.
        unsafe { sys::fh_q8_0_free(self.w) }
    }
}

/// Information about one tensor of a [`Gguf`] file.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct TensorInfo {
    pub name: String,
    /// GGML order: ne0 first.
    pub dims: Vec<u64>,
    pub ggml_type: u32,
    pub nbytes: u64,
}

/// The library's GGUF reader (`fh_gguf_open`: memory-mapped, one pass over the
/// header; the reference's `InferError::Format` texts on malformed files).
pub struct Gguf {
    g: *mut sys::fh_gguf,
}

// A parsed file is read-only after open.
unsafe impl Send for Gguf {}
unsafe impl Sync for Gguf {}

fn cstring(s: &str) -> Result<CString> {
    CString::new(s).map_err(|_| Error::Invalid(format!("{s:?} holds a NUL byte")))
}

impl Gguf {
    pub fn open(path: &Path) -> Result<Gguf> {
        let p = cstring(&path.to_string_lossy())?;
        let mut g: *mut sys::fh_gguf = std::ptr::null_mut();
        // SAFETY: p is NUL-terminated; `g` is an out-pointer the library always sets.
        let rc = unsafe { sys::fh_gguf_open(p.as_ptr(), &mut g) };
        if rc != sys::FH_OK {
            // SAFETY: the handle carries the message even on failure.
            let msg = unsafe { CStr::from_ptr(sys::fh_gguf_error(g)).to_string_lossy().into_owned() };
            // SAFETY: closed once.
            unsafe { sys::fh_gguf_close(g) };
            return Err(Error::from_code(rc, msg));
        }
        Ok(Gguf { g })
    }

    pub fn version(&self) -> u32 {
        // SAFETY: the handle is alive.
        unsafe { sys::fh_gguf_version(self.g) }
    }

    pub fn tensor_count(&self) -> usize {
        // SAFETY: the handle is alive.
        unsafe { sys::fh_gguf_tensor_count(self.g) }
    }

    /// The i-th tensor of the directory.
    pub fn tensor(&self, i: usize) -> Option<TensorInfo> {
        if i >= self.tensor_count() {
            return None;
        }
        let mut name: *const c_char = std::ptr::null();
        let (mut nd, mut ty, mut nb) = (0u32, 0u32, 0u64);
        let mut dims = [0u64; 8];
        // SAFETY: i is in range; the out-pointers are valid and dims holds the
        // header's maximum of 8 dimensions.
        let rc = unsafe { sys::fh_gguf_tensor_info(self.g, i, &mut name, &mut nd, dims.as_mut_ptr(), &mut ty, &mut nb) };
        if rc != sys::FH_OK {
            return None;
        }
        // SAFETY: the name points into the mapping, valid while self lives.
        let name = unsafe { CStr::from_ptr(name).to_string_lossy().into_owned() };
        Some(TensorInfo { name, dims: dims[..(nd as usize).min(8)].to_vec(), ggml_type: ty, nbytes: nb })
    }

    /// The directory index of a tensor by name.
    pub fn find(&self, name: &str) -> Option<usize> {
        let n = cstring(name).ok()?;
        // SAFETY: n is NUL-terminated.
        let i = unsafe { sys::fh_gguf_find_tensor(self.g, n.as_ptr()) };
        usize::try_from(i).ok()
    }

    /// An unsigned integer metadata value (any integer type holding a
    /// non-negative value).
    pub fn meta_u64(&self, key: &str) -> Option<u64> {
        let k = cstring(key).ok()?;
        let mut v = 0u64;
        // SAFETY: k is NUL-terminated; v is an out-pointer.
        (unsafe { sys::fh_gguf_meta_u64(self.g, k.as_ptr(), &mut v) } == sys::FH_OK).then_some(v)
    }

    /// A floating-point (or integer) metadata value.
    pub fn meta_f64(&self, key: &str) -> Option<f64> {
        let k = cstring(key).ok()?;
        let mut v = 0f64;
        // SAFETY: k is NUL-terminated; v is an out-pointer.
        (unsafe { sys::fh_gguf_meta_f64(self.g, k.as_ptr(), &mut v) } == sys::FH_OK).then_some(v)
    }

    /// A string value, or element `index` of a string array.
    pub fn meta_str(&self, key: &str, index: usize) -> Option<String> {
        let k = cstring(key).ok()?;
        let mut p: *const c_char = std::ptr::null();
        let mut len = 0usize;
        // SAFETY: k is NUL-terminated; p / len are out-pointers.
        if unsafe { sys::fh_gguf_meta_str(self.g, k.as_ptr(), index, &mut p, &mut len) } != sys::FH_OK {
            return None;
        }
        // SAFETY: p points at len bytes inside the mapping, valid while self lives.
        let bytes = unsafe { std::slice::from_raw_parts(p as *const u8, len) };
        Some(String::from_utf8_lossy(bytes).into_owned())
    }

    /// An F32 or F16 tensor as f32 values (`Gguf::dequantize` for those types).
    pub fn read_f32(&self, dev: &Device, name: &str) -> Result<Vec<f32>> {
        let i = self.find(name).ok_or_else(|| Error::Format(format!("missing tensor '{name}'")))?;
        let info = self.tensor(i).ok_or_else(|| Error::Format(format!("missing tensor '{name}'")))?;
        let n: u64 = info.dims.iter().product();
        let n = usize::try_from(n).map_err(|_| Error::Limit(format!("tensor '{name}' is too large")))?;
        let mut out = vec![0f32; n];
        let key = cstring(name)?;
        // SAFETY: out holds the tensor's element count.
        dev.call(|c| unsafe { sys::fh_gguf_read_f32(c, self.g, key.as_ptr(), out.as_mut_ptr(), n) })?;
        Ok(out)
    }

    /// A Q8_0 tensor straight from the mapping to the device (no f32 expansion).
    pub fn upload_q8_0(&self, dev: &Device, name: &str) -> Result<Weight> {
        let i = self.find(name).ok_or_else(|| Error::Format(format!("missing tensor '{name}'")))?;
        let info = self.tensor(i).ok_or_else(|| Error::Format(format!("missing tensor '{name}'")))?;
        let key = cstring(name)?;
        let mut w: *mut sys::fh_q8_0 = std::ptr::null_mut();
        // SAFETY: key is NUL-terminated; `w` is an out-pointer.
        dev.call(|c| unsafe { sys::fh_gguf_upload_q8_0(c, self.g, key.as_ptr(), &mut w) })?;
        let k = *info.dims.first().unwrap_or(&0) as usize;
        let n_rows = info.dims.get(1).copied().unwrap_or(1) as usize;
        Ok(Weight { w, n_rows, k })
    }
}

impl Drop for Gguf {
    fn drop(&mut self) {
        // SAFETY: closed once.
        unsafe { sys::fh_gguf_close(self.g) }
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn the_library_links_and_counts_devices() {
        let _ = device_count();
    }

    #[test]
    fn error_codes_map_to_kinds() {
        assert_eq!(Error::from_code(sys::FH_ERR_DIM, "m".into()), Error::Dim("m".into()));
        assert_eq!(Error::from_code(sys::FH_ERR_FORMAT, "m".into()), Error::Format("m".into()));
        assert_eq!(Error::from_code(42, "m".into()), Error::Other(42, "m".into()));
    }

    /// Needs a GPU: `cargo test -- --ignored`.
    #[test]
    #[ignore]
    fn a_linear_and_a_greedy_pick_on_the_device() {
        let dev = Device::new(0).expect("a HIP device");
        let k = 64;
        let x: Vec<f32> = (0..k).map(|i| (i as f32 - 32.0) / 16.0).collect();
        let q = dev.encode_q8_0(&x).unwrap();
        let w = dev.upload_q8_0(&q, 1, k).unwrap();
        let y = dev.linear_forward(&x, 1, &w, &[], Numerics::W8A32Exact).unwrap();
        assert_eq!(y.len(), 1);
        let err = dev.linear_forward(&x[..32], 1, &w, &[], Numerics::W8A32).unwrap_err();
        assert!(matches!(err, Error::Dim(_)), "{err}");
        let no_history: &[u32] = &[];
        let ids = dev
            .sample_rows(&[0.1, 0.9, 0.3], 3, Logits::Raw, &SamplingParams::new(0.0, 0, 1.0, 1.0), &[no_history], None)
            .unwrap();
        assert_eq!(ids, vec![1]);
        dev.sync().unwrap();
    }
}
