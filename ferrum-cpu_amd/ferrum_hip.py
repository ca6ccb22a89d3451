"""Host-side face of libferrum_hip: ferrum_core's matmul-engine and sampler API
on an MI355X, through the library's C ABI (include/ferrum_hip.h).

The names mirror the reference's Rust API one for one, so code written against
ferrum_core reads the same here:

    ops::linear_forward(input, weight, bias)   ferrum_core/src/ops.rs:233-256
    ops::matmul(a, b)                          ferrum_core/src/ops.rs:197-223
    Linear::forward (Q8_0-backed)              ferrum_core/src/layer/linear.rs:177-210
    SamplingParams                             ferrum_core/src/slm/sampling.rs:27-83
    sample_with_params(logits, params, recent, rng)
                                               ferrum_core/src/slm/sampling.rs:124-210
    Rng (xorshift64*)                          ferrum_core/src/rng.rs:1-41
    q8_0_block / enc_q8_0 / dequant_q8_0       quant.rs:271-280, gguf_write/blocks.rs:132-140,
                                               gguf/dequant.rs:37-49

Errors: a shape mismatch raises ``DimMismatch`` (the reference's
``InferError::DimMismatch``, same message); every other failure raises
``FerrumHipError`` carrying the library's status code and message.

The library must be built (``make -C ferrum-cpu_amd``); there is no CPU
fallback: importing this module without the built library raises.
PyTorch is only plumbing here (device buffers and streams for the _async
forms); the computation is the HIP library's.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libferrum_hip.so")

FH_OK, FH_ERR_DIM, FH_ERR_INVALID, FH_ERR_OOM, FH_ERR_HIP, FH_ERR_LIMIT, FH_ERR_FORMAT, FH_ERR_EXCHANGE = range(8)
W8A32, W8A8, W8A32_EXACT, W8A8_FAST = 0, 1, 2, 3  # FH_W8A32 ... (W8A8_FAST: W8A8 with each block term fused, 1e-5)
LOGITS_RAW, LOGITS_GPT2_SOFTMAX = 0, 1
RECENT_RANGES = 0x100  # OR'd into the logits kind: recent offsets as (begin, end) pairs per row

EXPORTS = (
    "fh_ctx_create", "fh_ctx_destroy", "fh_ctx_set_stream", "fh_ctx_reset_stream", "fh_sync", "fh_last_error",
    "fh_device_count", "fh_q8_0_upload", "fh_q8_0_upload_device", "fh_q8_0_download",
    "fh_q8_0_dims", "fh_q8_0_free", "fh_weight_upload_f32", "fh_weight_kind", "fh_q8_0_linear", "fh_q8_0_linear_async",
    "fh_q8_0_linear_noalloc_async",
    "fh_q8_0_encode", "fh_q8_0_encode_async", "fh_q8_0_dequant_async",
    "fh_q8_0_block_dots_async", "fh_sample_rows", "fh_sample_rows_async", "fh_debug_sampler_faults",
    "fh_embed_one_async", "fh_layernorm_async", "fh_gelu_async", "fh_add_async", "fh_attention_decode_async",
    "fh_attention_prefill_async", "fh_attention_prefill_seqs_async",
    "fh_q8_0_linear_act_async", "fh_add_layernorm_async", "fh_q8_0_linear_ln_async",
    "fh_q8_0_linear_residual_async", "fh_q8_0_linear_normed_async",
    "fh_gpt2_stack_create", "fh_gpt2_stack_free", "fh_gpt2_stack_forward_async",
    "fh_rmsnorm_async", "fh_rope_async", "fh_gqa_attention_decode_async", "fh_gqa_attention_rope_decode_async",
    "fh_swiglu_async", "fh_embed_rows_async",
    "fh_embed_rows_pos_async",
    "fh_gguf_open", "fh_gguf_close", "fh_gguf_error", "fh_gguf_version", "fh_gguf_tensor_count", "fh_gguf_find_tensor",
    "fh_gguf_tensor_info", "fh_gguf_tensor_data", "fh_gguf_meta_type", "fh_gguf_meta_u64", "fh_gguf_meta_f64",
    "fh_gguf_meta_str", "fh_gguf_meta_array_data", "fh_gguf_read_f32", "fh_gguf_upload_q8_0",
    "fh_qweight_upload", "fh_qweight_free", "fh_qlinear_async",
)


class FerrumHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[ferrum_hip status {code}] {msg}")
        self.code = code
        self.msg = msg


class DimMismatch(FerrumHipError, ValueError):
    """ferrum_core's InferError::DimMismatch (error.rs:5-27)."""


class SamplingParams(C.Structure):
    """slm/sampling.rs:27-38 (the cancel flag is a host-side control checked
    between tokens, so it is not part of the device call)."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("repetition_penalty", C.c_float),
    ]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0):
        super().__init__(float(temperature), int(top_k), float(top_p), float(repetition_penalty))

    @classmethod
    def with_temperature(cls, temperature: float) -> "SamplingParams":
        """SamplingParams::with_temperature (slm/sampling.rs:76-82)."""
        return cls(temperature=temperature)

    def __repr__(self):
        return (f"SamplingParams(temperature={self.temperature}, top_k={self.top_k}, "
                f"top_p={self.top_p}, repetition_penalty={self.repetition_penalty})")


class Rng:
    """rng::Rng, the reference's seeded xorshift64* (rng.rs:10-41).  The draws
    stay on the host so the sequence is exactly the reference's."""

    _M = (1 << 64) - 1

    def __init__(self, seed: int = 0):
        self.state = 0x9E3779B97F4A7C15 if seed == 0 else seed & self._M

    @classmethod
    def from_state(cls, state: int) -> "Rng":
        r = cls(1)
        r.state = state & cls._M
        return r

    def next_u64(self) -> int:
        x = self.state
        x ^= (x << 13) & self._M
        x ^= x >> 7
        x ^= (x << 17) & self._M
        self.state = x
        return (x * 0x2545F4914F6CDD1D) & self._M

    def next_f32(self) -> float:
        return float(np.float32(self.next_u64() >> 40) / np.float32(1 << 24))


class GPT2Block(C.Structure):
    """fh_gpt2_block: one transformer block's device weights and caches."""

    _fields_ = [(n, C.c_void_p) for n in ("qkv", "out", "up", "down", "qkv_b", "out_b", "up_b", "down_b", "ln1_g",
                                           "ln1_b", "ln2_g", "ln2_b", "k_cache", "v_cache")]


_lib = None


def _share_torch_hip_runtime():
    """PyTorch wheels ship their own libamdhip64.so and load it by that file
    name, so a process that loads this library (which needs the soname
    libamdhip64.so.7) before torch ends up with two HIP runtimes, and torch then
    sees no GPU.  Importing torch first makes both share torch's runtime, and
    torch streams and device pointers stay valid here.  Without torch, the
    system ROCm runtime is used."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    """The loaded libferrum_hip (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FerrumHipError(FH_ERR_INVALID, f"{LIB_PATH} is not built (run make -C {HERE})")
        _share_torch_hip_runtime()
        L = C.CDLL(LIB_PATH)
        vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
        L.fh_ctx_create.argtypes = [i32, C.POINTER(vp)]
        L.fh_ctx_destroy.argtypes = [vp]
        L.fh_ctx_destroy.restype = None
        L.fh_ctx_set_stream.argtypes = [vp, vp]
        L.fh_ctx_reset_stream.argtypes = [vp]
        L.fh_sync.argtypes = [vp]
        L.fh_last_error.argtypes = [vp]
        L.fh_last_error.restype = C.c_char_p
        L.fh_device_count.argtypes = []
        L.fh_q8_0_upload.argtypes = [vp, vp, sz, sz, C.POINTER(vp)]
        L.fh_q8_0_upload_device.argtypes = [vp, vp, sz, sz, C.POINTER(vp)]
        L.fh_q8_0_download.argtypes = [vp, vp, vp]
        L.fh_q8_0_dims.argtypes = [vp, C.POINTER(sz), C.POINTER(sz)]
        L.fh_weight_upload_f32.argtypes = [vp, vp, sz, sz, C.POINTER(vp)]
        L.fh_weight_kind.argtypes = [vp]
        L.fh_q8_0_free.argtypes = [vp]
        L.fh_q8_0_free.restype = None
        L.fh_q8_0_linear.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp, i32]
        L.fh_q8_0_linear_async.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp, i32]
        L.fh_q8_0_linear_noalloc_async.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp, i32]
        L.fh_q8_0_encode.argtypes = [vp, vp, sz, vp]
        L.fh_q8_0_encode_async.argtypes = [vp, vp, sz, vp]
        L.fh_q8_0_dequant_async.argtypes = [vp, vp, sz, vp]
        L.fh_q8_0_block_dots_async.argtypes = [vp, vp, vp, sz, vp]
        L.fh_sample_rows.argtypes = [vp, vp, sz, sz, i32, C.POINTER(SamplingParams), vp, vp, vp, vp]
        L.fh_sample_rows_async.argtypes = [vp, vp, sz, sz, i32, C.POINTER(SamplingParams), vp, vp, vp, vp]
        L.fh_debug_sampler_faults.argtypes = [vp, i32, C.c_uint32]
        L.fh_embed_one_async.argtypes = [vp, vp, vp, sz, sz, sz, vp, sz, vp]
        L.fh_layernorm_async.argtypes = [vp, vp, sz, sz, vp, vp, vp]
        L.fh_gelu_async.argtypes = [vp, vp, sz]
        L.fh_add_async.argtypes = [vp, vp, vp, sz]
        L.fh_attention_decode_async.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, vp]
        L.fh_attention_prefill_async.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, sz, vp]
        L.fh_attention_prefill_seqs_async.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, vp]
        L.fh_q8_0_linear_act_async.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp, i32, i32]
        L.fh_add_layernorm_async.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp]
        L.fh_q8_0_linear_ln_async.argtypes = [vp, vp, vp, vp, vp, sz, sz, vp, vp, vp, sz, vp, i32, i32]
        L.fh_q8_0_linear_residual_async.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp, vp, vp]
        L.fh_q8_0_linear_normed_async.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp, C.c_float, i32, vp, sz, vp, i32]
        L.fh_gpt2_stack_create.argtypes = [vp, C.POINTER(GPT2Block), sz, sz, sz, sz, sz, vp, vp, sz, sz,
                                           C.POINTER(vp)]
        L.fh_gpt2_stack_free.argtypes = [vp]
        L.fh_gpt2_stack_free.restype = None
        L.fh_gpt2_stack_forward_async.argtypes = [vp, vp, vp, sz, vp]
        f32 = C.c_float
        L.fh_rmsnorm_async.argtypes = [vp, vp, vp, vp, sz, sz, vp, f32, vp]
        L.fh_rope_async.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp, f32, i32, vp, f32]
        L.fh_gqa_attention_decode_async.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp, vp, sz, vp, sz, vp]
        L.fh_gqa_attention_rope_decode_async.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp, vp, sz, vp, sz, sz, f32, i32,
                                                         vp, f32, vp]
        L.fh_swiglu_async.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        L.fh_embed_rows_async.argtypes = [vp, vp, sz, sz, vp, sz, vp]
        L.fh_embed_rows_pos_async.argtypes = [vp, vp, vp, sz, sz, sz, vp, vp, sz, vp, sz, vp]
        u32, u64 = C.c_uint32, C.c_uint64
        L.fh_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp)]
        L.fh_gguf_close.argtypes = [vp]
        L.fh_gguf_close.restype = None
        L.fh_gguf_error.argtypes = [vp]
        L.fh_gguf_error.restype = C.c_char_p
        L.fh_gguf_version.argtypes = [vp]
        L.fh_gguf_version.restype = u32
        L.fh_gguf_tensor_count.argtypes = [vp]
        L.fh_gguf_tensor_count.restype = sz
        L.fh_gguf_find_tensor.argtypes = [vp, C.c_char_p]
        L.fh_gguf_find_tensor.restype = C.c_long
        L.fh_gguf_tensor_info.argtypes = [vp, sz, C.POINTER(C.c_char_p), C.POINTER(u32), C.POINTER(u64),
                                          C.POINTER(u32), C.POINTER(u64)]
        L.fh_gguf_tensor_data.argtypes = [vp, sz]
        L.fh_gguf_tensor_data.restype = vp
        L.fh_gguf_meta_type.argtypes = [vp, C.c_char_p, C.POINTER(u32), C.POINTER(u32), C.POINTER(u64)]
        L.fh_gguf_meta_u64.argtypes = [vp, C.c_char_p, C.POINTER(u64)]
        L.fh_gguf_meta_f64.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double)]
        L.fh_gguf_meta_str.argtypes = [vp, C.c_char_p, sz, C.POINTER(C.c_char_p), C.POINTER(sz)]
        L.fh_gguf_meta_array_data.argtypes = [vp, C.c_char_p, C.POINTER(vp), C.POINTER(sz)]
        L.fh_gguf_read_f32.argtypes = [vp, vp, C.c_char_p, vp, sz]
        L.fh_gguf_upload_q8_0.argtypes = [vp, vp, C.c_char_p, C.POINTER(vp)]
        L.fh_qweight_upload.argtypes = [vp, vp, vp, sz, sz, i32, C.POINTER(vp)]
        L.fh_qweight_free.argtypes = [vp]
        L.fh_qweight_free.restype = None
        L.fh_qlinear_async.argtypes = [vp, vp, vp, sz, sz, vp, sz, vp]
        _lib = L
    return _lib


def device_count() -> int:
    return int(lib().fh_device_count())


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()  # a torch tensor on the device


class Context:
    """One HIP device and stream (fh_ctx)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        rc = lib().fh_ctx_create(int(device), C.byref(h))
        if rc != FH_OK:
            raise FerrumHipError(rc, lib().fh_last_error(None).decode())
        self.h = h
        self.device = device

    def check(self, rc: int):
        if rc == FH_OK:
            return
        msg = lib().fh_last_error(self.h).decode()
        raise (DimMismatch if rc == FH_ERR_DIM else FerrumHipError)(rc, msg)

    def set_stream(self, stream_handle: int | None):
        """Enqueue on a caller's hipStream_t, e.g. torch.cuda.current_stream().cuda_stream
        (0 is the legacy default stream); None goes back to the context's own stream."""
        if stream_handle is None:
            self.check(lib().fh_ctx_reset_stream(self.h))
        else:
            self.check(lib().fh_ctx_set_stream(self.h, stream_handle))

    def sync(self):
        """Wait for the context's stream; raises what its kernels recorded since
        the last sync (FH_ERR_EXCHANGE for a bounded wait that gave up)."""
        self.check(lib().fh_sync(self.h))

    def debug_sampler_faults(self, skip_segment: int = -1, spin_limit: int = 0):
        """Testing hook: one split-sampler segment publishes nothing and the
        bounded waits give up after spin_limit polls (0: the default)."""
        self.check(lib().fh_debug_sampler_faults(self.h, int(skip_segment), int(spin_limit)))

    def close(self):
        if getattr(self, "h", None):
            lib().fh_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Q8_0Weight:
    """A device-resident GGUF Q8_0 weight [n_rows x k] (fh_q8_0): the backing of
    a Q8_0 Linear, uploaded straight from the GGUF bytes (no f32 expansion)."""

    def __init__(self, ctx: Context, handle, n_rows: int, k: int):
        self.ctx, self.h, self.n_rows, self.k = ctx, handle, n_rows, k

    @classmethod
    def upload(cls, ctx: Context, gguf_bytes, n_rows: int, k: int) -> "Q8_0Weight":
        raw = np.ascontiguousarray(gguf_bytes, dtype=np.uint8)
        if k % 32 == 0 and raw.size != n_rows * (k // 32) * 34:
            raise FerrumHipError(FH_ERR_INVALID, f"expected {n_rows * (k // 32) * 34} bytes, got {raw.size}")
        h = C.c_void_p()
        ctx.check(lib().fh_q8_0_upload(ctx.h, raw.ctypes.data, n_rows, k, C.byref(h)))
        return cls(ctx, h, n_rows, k)

    @classmethod
    def upload_f32(cls, ctx: Context, rows) -> "Q8_0Weight":
        """An F32 weight [n_rows, k] (host rows, GGUF order: k = ne0) behind the
        same handle: a tensor the reference stores as F32 (ne0 % 32 != 0, or an
        unquantized file).  Linears on it run the reference's f32 sums bit for
        bit (the exact kernel)."""
        a = np.ascontiguousarray(rows, dtype=np.float32)
        if a.ndim != 2:
            raise FerrumHipError(FH_ERR_INVALID, f"expected a matrix, got shape {a.shape}")
        h = C.c_void_p()
        ctx.check(lib().fh_weight_upload_f32(ctx.h, a.ctypes.data, a.shape[0], a.shape[1], C.byref(h)))
        return cls(ctx, h, a.shape[0], a.shape[1])

    @property
    def is_f32(self) -> bool:
        return lib().fh_weight_kind(self.h) == 1

    @classmethod
    def upload_device(cls, ctx: Context, d_bytes, n_rows: int, k: int) -> "Q8_0Weight":
        h = C.c_void_p()
        ctx.check(lib().fh_q8_0_upload_device(ctx.h, _ptr(d_bytes), n_rows, k, C.byref(h)))
        return cls(ctx, h, n_rows, k)

    def download(self) -> np.ndarray:
        out = np.empty(self.n_rows * (self.k // 32) * 34, np.uint8)
        self.ctx.check(lib().fh_q8_0_download(self.ctx.h, self.h, out.ctypes.data))
        return out

    def dims(self):
        n, k = C.c_size_t(), C.c_size_t()
        lib().fh_q8_0_dims(self.h, C.byref(n), C.byref(k))
        return int(n.value), int(k.value)

    def free(self):
        if self.h:
            lib().fh_q8_0_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def linear_forward(ctx: Context, x, weight: Q8_0Weight, bias=None, numerics: int = W8A32) -> np.ndarray:
    """ops::linear_forward(input [m, k], weight, bias [n]) -> [m, n] on the GPU
    (bias None = ops::matmul).  Host arrays in, host array out."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim != 2:
        raise FerrumHipError(FH_ERR_INVALID, f"expected a matrix, got shape {x.shape}")
    m, k = x.shape
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).ravel()
    y = np.empty((m, weight.n_rows), np.float32)
    ctx.check(lib().fh_q8_0_linear(ctx.h, weight.h, x.ctypes.data, m, k,
                                   None if b is None else b.ctypes.data, 0 if b is None else b.size,
                                   y.ctypes.data, numerics))
    return y


def matmul(ctx: Context, x, weight: Q8_0Weight, numerics: int = W8A32) -> np.ndarray:
    return linear_forward(ctx, x, weight, None, numerics)


def linear_forward_async(ctx: Context, weight: Q8_0Weight, x, m: int, k: int, bias, bias_len: int, y,
                         numerics: int = W8A32):
    """Device-pointer form (torch tensors or raw addresses), enqueued on the context stream."""
    ctx.check(lib().fh_q8_0_linear_async(ctx.h, weight.h, _ptr(x), m, k, _ptr(bias), bias_len, _ptr(y),
                                         numerics))


def q8_0_encode(ctx: Context, x) -> np.ndarray:
    """enc_q8_0 over q8_0_block: f32 -> GGUF Q8_0 bytes, on the GPU."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(max(x.size // 32 * 34, 1), np.uint8)
    ctx.check(lib().fh_q8_0_encode(ctx.h, x.ctypes.data if x.size else None, x.size, out.ctypes.data))
    return out[: x.size // 32 * 34]


def q8_0_encode_async(ctx: Context, x, n: int, out):
    ctx.check(lib().fh_q8_0_encode_async(ctx.h, _ptr(x), n, _ptr(out)))


def q8_0_dequant_async(ctx: Context, raw, n: int, out):
    ctx.check(lib().fh_q8_0_dequant_async(ctx.h, _ptr(raw), n, _ptr(out)))


def q8_0_block_dots_async(ctx: Context, weight: Q8_0Weight, qx, m: int, dots):
    ctx.check(lib().fh_q8_0_block_dots_async(ctx.h, weight.h, _ptr(qx), m, _ptr(dots)))


def _recent_lists(recents, rows):
    if recents is None:
        return None, None
    if len(recents) != rows:
        raise FerrumHipError(FH_ERR_INVALID, f"{len(recents)} recent lists for {rows} rows")
    lens = [len(r) for r in recents]
    off = np.zeros(rows + 1, np.uint32)
    off[1:] = np.cumsum(lens, dtype=np.uint64).astype(np.uint32)
    flat = np.concatenate([np.asarray(r, dtype=np.uint64).ravel() for r in recents]) if sum(lens) else np.zeros(0)
    # ids beyond u32 are out of any vocab; the reference skips them (sampling.rs:136)
    flat = np.minimum(flat, 0xFFFFFFFF).astype(np.uint32)
    return np.ascontiguousarray(flat), off


def sample_rows(ctx: Context, logits, params: SamplingParams, recents=None, draws=None,
                logits_kind: int = LOGITS_RAW) -> np.ndarray:
    """sample_with_params for every row of logits [rows, vocab] (host arrays).
    recents: one id list per row; draws: one u64 per row (Rng::next_u64)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    if lg.ndim == 1:
        lg = lg[None, :]
    rows, vocab = lg.shape
    flat, off = _recent_lists(recents, rows)
    dr = None if draws is None else np.ascontiguousarray(np.asarray(draws, dtype=np.uint64).ravel())
    out = np.zeros(max(rows, 1), np.uint32)
    ctx.check(lib().fh_sample_rows(ctx.h, lg.ctypes.data, rows, vocab, logits_kind, C.byref(params),
                                   None if flat is None or flat.size == 0 else flat.ctypes.data,
                                   None if off is None else off.ctypes.data,
                                   None if dr is None else dr.ctypes.data, out.ctypes.data))
    return out[:rows]


def sample_rows_async(ctx: Context, d_logits, rows: int, vocab: int, params: SamplingParams, d_recent=None,
                      d_offsets=None, d_draws=None, d_out=None, logits_kind: int = LOGITS_RAW):
    ctx.check(lib().fh_sample_rows_async(ctx.h, _ptr(d_logits), rows, vocab, logits_kind, C.byref(params),
                                         _ptr(d_recent), _ptr(d_offsets), _ptr(d_draws), _ptr(d_out)))


def sample_with_params(ctx: Context, logits, params: SamplingParams, recent, rng: Rng,
                       logits_kind: int = LOGITS_RAW) -> int:
    """slm::sampling::sample_with_params (sampling.rs:124): one row, drawing from
    rng exactly as the reference does (nothing when greedy, one next_u64 otherwise)."""
    draw = None if params.temperature <= 0.0 else [rng.next_u64()]
    return int(sample_rows(ctx, np.asarray(logits, np.float32)[None, :], params, [list(recent)], draw,
                           logits_kind)[0])


# ---- decode loops at the token level (the callers of the hot path) -------------------
# The model between two samples (embedding, attention, norms, GELU) belongs to
# the caller: `forward` hands back the next position's raw head scores.

class GPT2Window:
    """The token window of GenerativeSLM::token_stream / stream_next
    (slm/token_stream.rs:66-111, 150-168): capacity = the model's context
    (at least 1), keep = capacity / 2 (at least 1).  The prompt (or [bos] when
    empty) is cut to its last `capacity` ids; every sampled id that is not EOS
    is appended, and a window that outgrows the capacity is cut to its last
    `keep` ids and re-primed.  The window is also the penalty history."""

    def __init__(self, capacity: int, prompt, bos: int = 0):
        self.cap = max(int(capacity), 1)
        self.keep = max(self.cap // 2, 1)
        ids = [int(t) for t in prompt] or [int(bos)]
        self.ids = ids[-self.cap:] if len(ids) > self.cap else ids

    def push(self, tok: int) -> bool:
        """Append a sampled id; True when the window was cut and must be re-primed."""
        self.ids.append(int(tok))
        if len(self.ids) > self.cap:
            self.ids = self.ids[len(self.ids) - self.keep:]
            return True
        return False


def cancelled(cancel) -> bool:
    """SamplingParams::is_cancelled (slm/sampling.rs:55-60) for the host-side
    flag: None (never cancelled), an object with is_set() (threading.Event,
    settable from any thread), a callable returning a bool, or a bool."""
    if cancel is None:
        return False
    if hasattr(cancel, "is_set"):
        return bool(cancel.is_set())
    if callable(cancel):
        return bool(cancel())
    return bool(cancel)


def gpt2_decode(ctx: Context, forward, prompt, max_tokens: int, params: SamplingParams, rng: Rng,
                capacity: int, eos=None, bos: int = 0, cancel=None):
    """Token-level stream_next loop (slm/token_stream.rs:121-190).
    forward(window_ids, reprime) -> raw head scores z of the next position
    (reprime: the whole window was (re)fed, else only its last id).  Each step
    checks `cancel` first (stopping before it draws), then samples with the
    softmax -> ln(max(p, 1e-12)) bridge fused into the sampler, the window as
    the penalty history, and one draw from rng unless greedy.  Stops at
    max_tokens or EOS (drawn, not appended).  Returns the ids."""
    win = GPT2Window(capacity, prompt, bos)
    z = forward(list(win.ids), True)
    out = []
    while len(out) < max_tokens:
        if cancelled(cancel):
            break
        nxt = sample_with_params(ctx, z, params, win.ids, rng, LOGITS_GPT2_SOFTMAX)
        if eos is not None and nxt == eos:
            break
        out.append(nxt)
        reprime = win.push(nxt)
        z = forward(list(win.ids), reprime)
    return out


def llama_decode(ctx: Context, forward_one, prompt, max_new: int, params: SamplingParams, rng: Rng,
                 context_len: int, stops=(), cancel=None):
    """LlamaModel::generate_inner at the token level (llm.rs:706-754): a
    non-empty prompt shorter than the context, max_new clipped to
    context - prompt, every prompt and generated id as the penalty history, a
    stop id returned but not fed.  `cancel` (see cancelled) is checked before
    every prompt position (a cancel there returns nothing) and before every
    draw.  forward_one(token) -> raw logits."""
    prompt = [int(t) for t in prompt]
    if not prompt:
        raise DimMismatch(FH_ERR_DIM, "prompt must be non-empty")
    if len(prompt) >= context_len:
        raise DimMismatch(FH_ERR_DIM, f"prompt of {len(prompt)} tokens does not fit the model's "
                                      f"{context_len}-token context window")
    max_new = min(int(max_new), context_len - len(prompt))
    logits = None
    for tok in prompt:
        if cancelled(cancel):
            return []
        logits = forward_one(tok)
    out, recent = [], list(prompt)
    for _ in range(max_new):
        if cancelled(cancel):
            break
        nxt = sample_with_params(ctx, logits, params, recent, rng, LOGITS_RAW)
        out.append(nxt)
        if nxt in stops:
            break
        recent.append(nxt)
        logits = forward_one(nxt)
    return out


# ---- the rest of a GPT-2 decode step (device pointers) -----------------------------

def embed_one_async(ctx: Context, token_w, pos_w, vocab: int, max_seq: int, d: int, d_token, pos: int, out):
    """Embedding::embed_one (layer/embedding.rs:70-90); the token id is read on the device."""
    ctx.check(lib().fh_embed_one_async(ctx.h, _ptr(token_w), _ptr(pos_w), vocab, max_seq, d, _ptr(d_token), pos,
                                       _ptr(out)))


def layernorm_async(ctx: Context, x, rows: int, d: int, gamma, beta, y):
    """LayerNorm::forward (layer/norm.rs:46-82)."""
    ctx.check(lib().fh_layernorm_async(ctx.h, _ptr(x), rows, d, _ptr(gamma), _ptr(beta), _ptr(y)))


def gelu_async(ctx: Context, x, n: int):
    """activation::gelu (activation.rs:9-12), in place."""
    ctx.check(lib().fh_gelu_async(ctx.h, _ptr(x), n))


def add_async(ctx: Context, x, y, n: int):
    """x += y (the residual adds of layer/transformer.rs:281, 288)."""
    ctx.check(lib().fh_add_async(ctx.h, _ptr(x), _ptr(y), n))


ACT_NONE, ACT_GELU = 0, 1
# linear_normed_async only: the weight's rows are gate / up interleaved in
# groups of 32 (interleave_gate_up), the output silu(gate) * up ([m, n / 2])
ACT_SWIGLU32 = 2


def interleave_gate_up(gate: np.ndarray, up: np.ndarray, rows: int) -> np.ndarray:
    """Two row-major matrices of `rows` rows each (Q8_0 bytes or any per-row
    layout) as one, gate and up rows interleaved in groups of 32: the weight
    ACT_SWIGLU32 reads."""
    g, u = np.asarray(gate).reshape(rows // 32, 32, -1), np.asarray(up).reshape(rows // 32, 32, -1)
    return np.stack([g, u], axis=1).reshape(-1)


def linear_act_async(ctx: Context, weight: "Q8_0Weight", x, m: int, k: int, bias, bias_len: int, y, act: int,
                     numerics: int = W8A32):
    """Linear::forward followed by an activation (ACT_GELU: the block's ffn1 + gelu)."""
    ctx.check(lib().fh_q8_0_linear_act_async(ctx.h, weight.h, _ptr(x), m, k, _ptr(bias), bias_len, _ptr(y),
                                             numerics, act))


def add_layernorm_async(ctx: Context, x, y, rows: int, d: int, gamma, beta, ln):
    """x += y, then LayerNorm(x) into ln (a residual add and the LayerNorm after it)."""
    ctx.check(lib().fh_add_layernorm_async(ctx.h, _ptr(x), _ptr(y), rows, d, _ptr(gamma), _ptr(beta), _ptr(ln)))


def linear_ln_async(ctx: Context, weight: "Q8_0Weight", x, r, s, m: int, k: int, gamma, beta, bias, bias_len: int,
                    y, act: int = ACT_NONE, numerics: int = W8A32):
    """y = act(LayerNorm(x + r) . W^T + b), with x + r written to s when s is
    given (r may be None: LayerNorm(x)): a residual add, the LayerNorm after it
    and the Linear that reads it, as one call."""
    ctx.check(lib().fh_q8_0_linear_ln_async(ctx.h, weight.h, _ptr(x), _ptr(r), _ptr(s), m, k, _ptr(gamma), _ptr(beta),
                                            _ptr(bias), bias_len, _ptr(y), numerics, act))


def linear_residual_async(ctx: Context, weight: "Q8_0Weight", x, m: int, k: int, bias, bias_len: int, r, y,
                          stats=None):
    """y = r + linear_forward(x) (y may be r), and with `stats` ([m, n / 32,
    2]) y's row statistics (per 32-column group: mean, sum of squared
    deviations) for a following linear_normed_async: the residual adds of
    forward_with_cache (layer/transformer.rs:281, 288) without a launch of
    their own."""
    ctx.check(lib().fh_q8_0_linear_residual_async(ctx.h, weight.h, _ptr(x), m, k, _ptr(bias), bias_len, _ptr(r),
                                                  _ptr(y), _ptr(stats)))


def linear_normed_async(ctx: Context, weight: "Q8_0Weight", x, m: int, k: int, stats, gamma, beta, eps: float,
                        rms: bool, bias, bias_len: int, y, act: int = ACT_NONE):
    """y = act(norm(x) W^T + b), norm (LayerNorm, or RmsNorm with rms) formed
    from the row statistics linear_residual_async left for x."""
    ctx.check(lib().fh_q8_0_linear_normed_async(ctx.h, weight.h, _ptr(x), m, k, _ptr(stats), _ptr(gamma), _ptr(beta),
                                                float(eps), 1 if rms else 0, _ptr(bias), bias_len, _ptr(y), act))


def attention_decode_async(ctx: Context, qkv, k_cache, v_cache, capacity: int, d: int, heads: int, pos: int, out):
    """The KV-cache attention of forward_with_cache (layer/transformer.rs:242-279)."""
    ctx.check(lib().fh_attention_decode_async(ctx.h, _ptr(qkv), _ptr(k_cache), _ptr(v_cache), capacity, d, heads,
                                              pos, _ptr(out)))


def attention_prefill_async(ctx: Context, qkv, k_cache, v_cache, capacity: int, d: int, heads: int, pos0: int,
                            rows: int, out):
    """The same attention for `rows` consecutive positions pos0 .. pos0 + rows - 1
    of one sequence at once (row r of qkv is position pos0 + r)."""
    ctx.check(lib().fh_attention_prefill_async(ctx.h, _ptr(qkv), _ptr(k_cache), _ptr(v_cache), capacity, d, heads,
                                               pos0, rows, _ptr(out)))


def attention_prefill_seqs_async(ctx: Context, qkv, k_cache, v_cache, seq_stride: int, capacity: int, d: int,
                                 heads: int, pos0: int, rows: int, seqs: int, out):
    """attention_prefill_async for `seqs` sequences in one call: sequence s's
    rows are rows s * rows .. of qkv and out, its caches start seq_stride
    floats after sequence s - 1's (the primes of a batch of sequences)."""
    ctx.check(lib().fh_attention_prefill_seqs_async(ctx.h, _ptr(qkv), _ptr(k_cache), _ptr(v_cache), seq_stride,
                                                    capacity, d, heads, pos0, rows, seqs, _ptr(out)))


# ---- packed per-row int8 / int4 weights: ops::qlinear ---------------------------

QINT8, QINT4 = 0, 1


class QWeight:
    """A device-resident QWeight (quant.rs:130-217): k input rows x n outputs,
    one scale per row, int8 or split-half int4 levels as the reference stores
    them (fh_qweight)."""

    def __init__(self, ctx: Context, scales, q, k: int, n: int, kind: int):
        s = np.ascontiguousarray(scales, np.float32)
        b = np.ascontiguousarray(q, np.uint8)
        row = n if kind == QINT8 else (n + 1) // 2
        if kind in (QINT8, QINT4) and (s.size != k or b.size != k * row):
            raise FerrumHipError(FH_ERR_INVALID, f"QWeight: expected {k} scales and {k * row} level bytes")
        h = C.c_void_p()
        ctx.check(lib().fh_qweight_upload(ctx.h, s.ctypes.data, b.ctypes.data, k, n, kind, C.byref(h)))
        self.ctx, self.h, self.k, self.n, self.kind = ctx, h, k, n, kind

    def free(self):
        if self.h:
            lib().fh_qweight_free(self.h)
            self.h = None


def qlinear_async(ctx: Context, w: QWeight, x, m: int, k: int, bias, bias_len: int, y):
    """ops::qlinear on device pointers: y = x . W + b, the reference's bits."""
    ctx.check(lib().fh_qlinear_async(ctx.h, w.h, _ptr(x), m, k, _ptr(bias), bias_len, _ptr(y)))


# ---- GGUF files (the library's native reader) ----------------------------------

class GGUFFormatError(FerrumHipError):
    """A malformed GGUF file (ferrum_core's InferError::Format)."""


class GGUFFile:
    """A GGUF file opened by the library's reader (memory-mapped; Gguf::open,
    gguf/mod.rs:208-310).  Tensors: name -> (dims in GGML order, GGML type,
    byte count); metadata through meta(); Q8_0 tensors go straight to the
    device with upload_q8_0."""

    def __init__(self, path):
        h = C.c_void_p()
        rc = lib().fh_gguf_open(os.fsencode(path), C.byref(h))
        if rc != FH_OK:
            msg = lib().fh_gguf_error(h).decode(errors="replace")
            lib().fh_gguf_close(h)
            raise (GGUFFormatError if rc == FH_ERR_FORMAT else FerrumHipError)(rc, msg)
        self.h = h
        self.version = lib().fh_gguf_version(h)
        self.tensors = {}
        for i in range(lib().fh_gguf_tensor_count(h)):
            name, nd, ty, nb = C.c_char_p(), C.c_uint32(), C.c_uint32(), C.c_uint64()
            dims = (C.c_uint64 * 8)()
            lib().fh_gguf_tensor_info(h, i, C.byref(name), C.byref(nd), dims, C.byref(ty), C.byref(nb))
            key = name.value.decode(errors="replace")
            self.tensors.setdefault(key, (tuple(dims[:nd.value]), ty.value, nb.value, i))

    def close(self):
        if self.h:
            lib().fh_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def meta_kind(self, key: str):
        """(GGUF value type, array element type, array length) of a key, None if absent."""
        ty, el, cnt = C.c_uint32(), C.c_uint32(), C.c_uint64()
        if lib().fh_gguf_meta_type(self.h, key.encode(), C.byref(ty), C.byref(el), C.byref(cnt)) != FH_OK:
            return None
        return ty.value, el.value, cnt.value

    def meta(self, key: str):
        """The value of a metadata key (int, float, str, or list), None if absent."""
        k = key.encode()
        ty, el, cnt = C.c_uint32(), C.c_uint32(), C.c_uint64()
        if lib().fh_gguf_meta_type(self.h, k, C.byref(ty), C.byref(el), C.byref(cnt)) != FH_OK:
            return None
        ty, el, cnt = ty.value, el.value, cnt.value
        if ty == 8:  # string
            out, n = C.c_char_p(), C.c_size_t()
            lib().fh_gguf_meta_str(self.h, k, 0, C.byref(out), C.byref(n))
            return C.string_at(out, n.value).decode(errors="replace")
        if ty == 9:  # array
            if el == 8:
                vals = []
                for i in range(cnt):
                    out, n = C.c_char_p(), C.c_size_t()
                    lib().fh_gguf_meta_str(self.h, k, i, C.byref(out), C.byref(n))
                    vals.append(C.string_at(out, n.value).decode(errors="replace"))
                return vals
            data, es = C.c_void_p(), C.c_size_t()
            lib().fh_gguf_meta_array_data(self.h, k, C.byref(data), C.byref(es))
            dt = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "<u1", 10: "<u8",
                  11: "<i8", 12: "<f8"}[el]
            if cnt == 0:
                return []
            return list(np.frombuffer(C.string_at(data, cnt * es.value), dtype=dt))
        if ty in (6, 12):
            v = C.c_double()
            lib().fh_gguf_meta_f64(self.h, k, C.byref(v))
            return v.value
        if ty in (1, 3, 5, 11):  # signed
            v = C.c_double()
            lib().fh_gguf_meta_f64(self.h, k, C.byref(v))
            return int(v.value)
        v = C.c_uint64()
        lib().fh_gguf_meta_u64(self.h, k, C.byref(v))
        return v.value

    def raw(self, name: str) -> bytes:
        """The tensor's bytes (a copy)."""
        dims, ty, nb, i = self.tensors[name]
        return C.string_at(lib().fh_gguf_tensor_data(self.h, i), nb)

    def read_f32(self, ctx, name: str) -> np.ndarray:
        """An F32 / F16 tensor as float32 (numpy, GGML order reversed: [ne1, ne0]).
        ctx may be None (host-only; errors then carry no message)."""
        dims = self.tensors[name][0]
        n = int(np.prod(dims)) if dims else 1
        out = np.empty(n, np.float32)
        rc = lib().fh_gguf_read_f32(ctx.h if ctx else None, self.h, name.encode(), out.ctypes.data, n)
        if ctx:
            ctx.check(rc)
        elif rc != FH_OK:
            raise FerrumHipError(rc, f"fh_gguf_read_f32 '{name}' failed")
        return out.reshape(tuple(reversed(dims))) if len(dims) > 1 else out

    def upload_q8_0(self, ctx: "Context", name: str) -> "Q8_0Weight":
        """A Q8_0 tensor [ne0 = k, ne1 = n] straight from the mapping to the device."""
        dims = self.tensors[name][0]
        h = C.c_void_p()
        ctx.check(lib().fh_gguf_upload_q8_0(ctx.h, self.h, name.encode(), C.byref(h)))
        k, n = int(dims[0]), int(dims[1]) if len(dims) > 1 else 1
        return Q8_0Weight(ctx, h, n, k)


# ---- GGUF import: the reference's loader checks, before anything is uploaded ----

GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
_VT_INTS = {0: False, 1: True, 2: False, 3: True, 4: False, 5: True, 10: False, 11: True}  # type -> signed
_VT_F32, _VT_BOOL, _VT_STRING, _VT_ARRAY, _VT_F64 = 6, 7, 8, 9, 12
LN_EPS = 1e-5  # GPT-2's LayerNorm epsilon, which ferrum_core's LayerNorm uses (loader/mod.rs:135-136)


def _fmt(msg: str) -> "GGUFFormatError":
    return GGUFFormatError(FH_ERR_FORMAT, msg)


def _rust_str(s: str) -> str:
    """A string as Rust's {:?} prints it (quoted, with its escapes)."""
    esc = {'"': '\\"', "\\": "\\\\", "\n": "\\n", "\r": "\\r", "\t": "\\t", "\0": "\\0"}
    return '"' + "".join(esc.get(ch, ch) for ch in s) + '"'


def _rust_f32(v: float) -> str:
    """An f32 as Rust's {} prints it (shortest round trip, no exponent)."""
    return np.format_float_positional(np.float32(v), trim="-")


def _dims(dims) -> str:
    return "[" + ", ".join(str(int(x)) for x in dims) + "]"


class GgufMeta:
    """Typed metadata reads as ferrum_core's MetaValue converts them
    (gguf/mod.rs:96-116): as_usize takes any integer type holding a
    non-negative value, as_f32 takes F32/F64 or such an integer; booleans
    and strings are neither."""

    def __init__(self, g: "GGUFFile"):
        self.g = g

    def usize(self, key: str):
        k = self.g.meta_kind(key)
        if k is None or k[0] not in _VT_INTS:
            return None
        v = int(self.g.meta(key))
        return v if v >= 0 else None

    def f32(self, key: str):
        k = self.g.meta_kind(key)
        if k is None:
            return None
        if k[0] in (_VT_F32, _VT_F64):
            return float(np.float32(self.g.meta(key)))
        u = self.usize(key)
        return None if u is None else float(np.float32(u))

    def string(self, key: str):
        k = self.g.meta_kind(key)
        return self.g.meta(key) if k is not None and k[0] == _VT_STRING else None

    def array(self, key: str, elem: int):
        k = self.g.meta_kind(key)
        if k is None or k[0] != _VT_ARRAY or k[1] != elem:
            return None
        return self.g.meta(key)


def ferrum_vocab(tokens, merges, types):
    """loader/gpt2.rs:149-191: map a GGUF BPE vocabulary onto ferrum_core's id
    layout -- the 256 byte tokens in byte order, one token per merge in rank
    order, then every other token in file order -- so a foreign GPT-2 file
    (which orders its byte tokens differently) loads too.  Returns perm with
    perm[ferrum_id] = file_id."""
    from ferrum_gguf import byte_to_unicode

    if len(types) != len(tokens):
        raise _fmt(f"gguf vocab: {len(tokens)} tokens but {len(types)} token types")
    ids = {}
    for i, t in enumerate(tokens):  # (a repeated token keeps its last id, as a HashMap collect does)
        ids[t] = i
    b2u = byte_to_unicode()
    used = [False] * len(tokens)
    perm = []
    for w in [b2u[b] for b in range(256)] + [m.replace(" ", "", 1) for m in merges]:
        i = ids.get(w)
        if i is None or used[i]:
            raise _fmt(f"gguf vocab: no unique token {_rust_str(w)}")
        used[i] = True
        perm.append(i)
    perm.extend(i for i in range(len(tokens)) if not used[i])
    return perm


def _check_dims(g: "GGUFFile", name: str, want):
    """GgufIn::tensor's checks (loader/decode.rs:44-56)."""
    if name not in g.tensors:
        raise _fmt(f"missing tensor '{name}'")
    dims = g.tensors[name][0]
    if tuple(int(x) for x in dims) != tuple(int(x) for x in want):
        raise _fmt(f"tensor '{name}' has dims {_dims(dims)}, expected {_dims(want)}")


def gpt2_gguf_plan(g: "GGUFFile"):
    """gpt2_from's reading of a GPT-2 GGUF (loader/gpt2.rs:201-232 and the
    tensor shapes it asks for, 233-275), before any upload: the
    hyperparameters, the layer_norm_epsilon check, the vocabulary permutation
    and every tensor's dims.  Returns (cfg dict, perm, tied)."""
    meta = GgufMeta(g)
    arch = meta.string("general.architecture")
    if arch != "gpt2":
        shown = "None" if arch is None else f"Some({_rust_str(arch)})"
        raise _fmt(f"not a GPT-2 model: architecture {shown} (need gpt2)")

    def usize(key):
        v = meta.usize(key)
        if v is None:
            raise _fmt(f"GGUF key '{key}' missing or not an integer")
        return v

    ctx_len, d, n_layer = usize("gpt2.context_length"), usize("gpt2.embedding_length"), usize("gpt2.block_count")
    ff, heads = usize("gpt2.feed_forward_length"), usize("gpt2.attention.head_count")
    eps = meta.f32("gpt2.attention.layer_norm_epsilon")
    if eps is None:
        raise _fmt("GGUF key 'gpt2.attention.layer_norm_epsilon' missing or not a number")
    if np.abs(np.float32(eps) - np.float32(LN_EPS)) > np.float32(1e-9):
        raise _fmt(f"gpt2.attention.layer_norm_epsilon is {_rust_f32(eps)}; Ferrum's LayerNorm uses "
                   f"{_rust_f32(LN_EPS)}")
    arrays = {}
    for key, elem in (("tokenizer.ggml.tokens", _VT_STRING), ("tokenizer.ggml.merges", _VT_STRING),
                      ("tokenizer.ggml.token_type", 5)):
        arrays[key] = meta.array(key, elem)
        if arrays[key] is None:
            raise _fmt(f"GGUF key '{key}' missing or of the wrong type")
    perm = ferrum_vocab(arrays["tokenizer.ggml.tokens"], arrays["tokenizer.ggml.merges"],
                        [int(t) for t in arrays["tokenizer.ggml.token_type"]])
    v = len(perm)
    _check_dims(g, "token_embd.weight", (d, v))
    tied = "output.weight" not in g.tensors
    if not tied:
        _check_dims(g, "output.weight", (d, v))
    _check_dims(g, "position_embd.weight", (d, ctx_len))
    for i in range(n_layer):
        for stem, dims in (("attn_norm.weight", (d,)), ("attn_norm.bias", (d,)), ("attn_qkv.weight", (d, 3 * d)),
                           ("attn_qkv.bias", (3 * d,)), ("attn_output.weight", (d, d)), ("attn_output.bias", (d,)),
                           ("ffn_norm.weight", (d,)), ("ffn_norm.bias", (d,)), ("ffn_up.weight", (d, ff)),
                           ("ffn_up.bias", (ff,)), ("ffn_down.weight", (ff, d)), ("ffn_down.bias", (d,))):
            _check_dims(g, f"blk.{i}.{stem}", dims)
    _check_dims(g, "output_norm.weight", (d,))
    _check_dims(g, "output_norm.bias", (d,))
    return dict(vocab=v, d=d, heads=heads, layers=n_layer, ffn=ff, context=ctx_len), perm, tied


def llama_gguf_plan(g: "GGUFFile"):
    """Gguf::load_llama_prec's reading of a llama / qwen2 GGUF
    (gguf/llama.rs:171-340, rope scaling 51-103), before any upload: the
    architecture and its rope type, the hyperparameters with the reference's
    defaults, the rope scaling rules, the bias rules and every tensor's dims.
    Returns (cfg dict for LlamaDevice, {name: (n_out, n_in)} of the matrices,
    tied)."""
    meta = GgufMeta(g)
    arch = meta.string("general.architecture")
    if arch is None:
        raise _fmt("GGUF missing general.architecture")
    if arch not in ("llama", "qwen2"):
        raise _fmt(f"architecture '{arch}' is not supported by load_llama (llama / qwen2 only)")
    rope_type = ROPE_NEOX if arch == "qwen2" else ROPE_NORM

    def req(key):
        v = meta.usize(key)
        if v is None:
            raise _fmt(f"GGUF missing/invalid metadata '{key}'")
        return v

    def opt(key, default):
        v = meta.usize(key)
        return default if v is None else v

    def f32_or(key, default):
        v = meta.f32(key)
        return float(np.float32(default)) if v is None else v

    dim = req(f"{arch}.embedding_length")
    n_layers = req(f"{arch}.block_count")
    if n_layers > len(g.tensors):
        raise _fmt(f"GGUF block_count = {n_layers} exceeds what the file can hold ({len(g.tensors)})")
    n_heads = req(f"{arch}.attention.head_count")
    n_kv = opt(f"{arch}.attention.head_count_kv", n_heads)
    ffn = req(f"{arch}.feed_forward_length")
    head_dim = opt(f"{arch}.attention.key_length", dim // max(n_heads, 1))
    rope_dim = opt(f"{arch}.rope.dimension_count", head_dim)
    rope_base = f32_or(f"{arch}.rope.freq_base", 10000.0)
    # rope scaling (gguf/llama.rs:51-103)
    key = lambda k: f"{arch}.rope.{k}"  # noqa: E731
    if g.meta_kind(key("scaling.factor")) is not None:
        factor = meta.f32(key("scaling.factor"))
    else:
        factor = meta.f32(key("scale_linear"))
    if g.meta_kind(key("scaling.type")) is not None:
        ty = meta.string(key("scaling.type"))
        if ty is None:
            raise _fmt(f"'{key('scaling.type')}' is not a string")
    else:
        ty = "linear"
    factor = factor if factor is not None and factor != 0.0 else 1.0
    if ty == "linear":
        linear_factor = factor
    elif ty == "none":
        if factor != 1.0:
            raise _fmt(f"'{key('scaling.type')}' is \"none\" but the scaling factor is {_rust_f32(factor)}")
        linear_factor = 1.0
    else:
        raise _fmt(f"RoPE scaling type '{ty}' is not supported: Ferrum implements none, linear and "
                   "rope_freqs.weight (yarn and longrope are refused)")
    attn = f32_or(key("scaling.attn_factor"), 1.0)
    if attn != 1.0:
        raise _fmt(f"RoPE scaling attn_factor {_rust_f32(attn)} is not supported (only 1.0)")
    has_freqs = "rope_freqs.weight" in g.tensors
    if has_freqs and tuple(int(x) for x in g.tensors["rope_freqs.weight"][0]) != (rope_dim // 2,):
        raise _fmt(f"rope_freqs.weight has dims {_dims(g.tensors['rope_freqs.weight'][0])}, expected "
                   f"[{rope_dim // 2}] (rope_dim / 2)")
    eps = f32_or(f"{arch}.attention.layer_norm_rms_epsilon", 1e-5)
    ctx_len = opt(f"{arch}.context_length", 2048)
    if "token_embd.weight" not in g.tensors:
        raise _fmt("GGUF missing token_embd.weight")
    edims = tuple(int(x) for x in g.tensors["token_embd.weight"][0])
    vocab = edims[1] if len(edims) == 2 else req(f"{arch}.vocab_size")
    n_el = int(np.prod(edims)) if edims else 1
    emb_ok = edims == (dim, vocab) if len(edims) == 2 else vocab * dim == n_el
    if not emb_ok or vocab == 0 or dim == 0:
        raise _fmt("token_embd.weight size does not match vocab × dim")
    q_dim, kv_dim = n_heads * head_dim, n_kv * head_dim
    mats = {}

    def norm(name):
        if name not in g.tensors:
            raise _fmt(f"GGUF tensor '{name}' not found")
        n = int(np.prod(g.tensors[name][0])) if g.tensors[name][0] else 1
        if n != dim:
            raise _fmt(f"tensor '{name}' length is not {dim}")

    def linear(name, n_in, n_out, bias=None):
        if name not in g.tensors:
            raise _fmt(f"GGUF tensor '{name}' not found")
        dims = tuple(int(x) for x in g.tensors[name][0])
        if dims != (n_in, n_out):
            raise _fmt(f"tensor '{name}' has dims {_dims(dims)}, expected [{n_in}, {n_out}] from the metadata")
        if bias is not None and bias in g.tensors:
            nb = int(np.prod(g.tensors[bias][0])) if g.tensors[bias][0] else 1
            if nb != n_out:
                raise _fmt(f"bias for '{name}' has wrong length")
        mats[name] = (n_out, n_in)

    for i in range(n_layers):
        p = f"blk.{i}"
        for stem in ("attn_output", "ffn_gate", "ffn_up", "ffn_down"):
            if f"{p}.{stem}.bias" in g.tensors:
                raise _fmt(f"GGUF tensor '{p}.{stem}.bias' is not supported: Ferrum loads biases only for "
                           "attn_q/attn_k/attn_v")
        norm(f"{p}.attn_norm.weight")
        linear(f"{p}.attn_q.weight", dim, q_dim, f"{p}.attn_q.bias")
        linear(f"{p}.attn_k.weight", dim, kv_dim, f"{p}.attn_k.bias")
        linear(f"{p}.attn_v.weight", dim, kv_dim, f"{p}.attn_v.bias")
        linear(f"{p}.attn_output.weight", q_dim, dim)
        norm(f"{p}.ffn_norm.weight")
        linear(f"{p}.ffn_gate.weight", dim, ffn)
        linear(f"{p}.ffn_up.weight", dim, ffn)
        linear(f"{p}.ffn_down.weight", ffn, dim)
    norm("output_norm.weight")
    if "output.bias" in g.tensors:
        raise _fmt("GGUF tensor 'output.bias' is not supported: Ferrum loads biases only for attn_q/attn_k/attn_v")
    tied = "output.weight" not in g.tensors
    if not tied:
        linear("output.weight", dim, vocab)
    cfg = dict(arch=arch, vocab=vocab, d=dim, n_heads=n_heads, n_kv=n_kv, head_dim=head_dim, layers=n_layers,
               ffn=ffn, context=ctx_len, rope_dim=rope_dim, rope_base=rope_base, rope_type=rope_type, eps=eps,
               rope_linear=linear_factor, rope_freqs=has_freqs)
    return cfg, mats, tied


# ---- Llama / Qwen block pieces (llm.rs), batched over rows --------------------

ROPE_NORM, ROPE_NEOX = 0, 1


def rmsnorm_async(ctx: Context, x, r, s, rows: int, d: int, w, eps: float, out):
    """RmsNorm::forward_row over rows; with r, the residual add in front of it
    (x + r is normalised and written to s when s is given)."""
    ctx.check(lib().fh_rmsnorm_async(ctx.h, _ptr(x), _ptr(r), _ptr(s), rows, d, _ptr(w), eps, _ptr(out)))


def rope_async(ctx: Context, x, rows: int, ld: int, n_heads: int, head_dim: int, rope_dim: int, pos, base: float,
               rope_type: int, freq_factors=None, linear_factor: float = 1.0):
    """apply_rope in place on n_heads heads of each row (row r at x + r * ld,
    position pos[r] on the device)."""
    ctx.check(lib().fh_rope_async(ctx.h, _ptr(x), rows, ld, n_heads, head_dim, rope_dim, _ptr(pos), base, rope_type,
                                  _ptr(freq_factors), linear_factor))


def gqa_attention_decode_async(ctx: Context, qkv, ld: int, rows: int, n_heads: int, n_kv: int, head_dim: int, k_cache,
                               v_cache, capacity: int, pos, max_pos: int, out):
    """Attention::forward_one's cache append + attend for `rows` sequences."""
    ctx.check(lib().fh_gqa_attention_decode_async(ctx.h, _ptr(qkv), ld, rows, n_heads, n_kv, head_dim, _ptr(k_cache),
                                                  _ptr(v_cache), capacity, _ptr(pos), max_pos, _ptr(out)))


def gqa_attention_rope_decode_async(ctx: Context, qkv, ld: int, rows: int, n_heads: int, n_kv: int, head_dim: int,
                                    k_cache, v_cache, capacity: int, pos, max_pos: int, rope_dim: int, base: float,
                                    rope_type: int, freq_factors, linear_factor: float, out):
    """rope_async on each row's q and k heads, then gqa_attention_decode_async,
    in one call (one launch for many rows at head width 64); qkv's q and k
    values are scratch afterwards."""
    ctx.check(lib().fh_gqa_attention_rope_decode_async(ctx.h, _ptr(qkv), ld, rows, n_heads, n_kv, head_dim,
                                                       _ptr(k_cache), _ptr(v_cache), capacity, _ptr(pos), max_pos,
                                                       rope_dim, base, rope_type, _ptr(freq_factors), linear_factor,
                                                       _ptr(out)))


def swiglu_async(ctx: Context, g, u, rows: int, n: int, ld: int, out):
    """(g / (1 + exp(-g))) * u per row (row r of g and u at r * ld)."""
    ctx.check(lib().fh_swiglu_async(ctx.h, _ptr(g), _ptr(u), rows, n, ld, _ptr(out)))


def embed_rows_pos_async(ctx: Context, tok_w, pos_w, vocab: int, max_seq: int, d: int, tokens, pos, rows: int, out,
                         hist=None, hist_stride: int = 0):
    """Embedding::embed_one for `rows` sequences (token and position ids on the
    device); with hist, each row's id is also recorded at hist[r, pos[r]]."""
    ctx.check(lib().fh_embed_rows_pos_async(ctx.h, _ptr(tok_w), _ptr(pos_w), vocab, max_seq, d, _ptr(tokens), _ptr(pos),
                                            rows, _ptr(hist), hist_stride, _ptr(out)))


def embed_rows_async(ctx: Context, tok_w, vocab: int, d: int, tokens, rows: int, out):
    """LlamaModel::embed for token ids on the device."""
    ctx.check(lib().fh_embed_rows_async(ctx.h, _ptr(tok_w), vocab, d, _ptr(tokens), rows, _ptr(out)))


class LlamaDevice:
    """A Llama / Qwen2 decoder on the device for `rows` independent sequences
    (a batched decode step), the way LlamaModel::forward_one walks it
    (llm.rs:606-616): embed, then per LlamaBlock::forward_one (llm.rs:445-456)
    RmsNorm, the q|k|v Q8_0 linear (one weight: the three GGUF tensors' rows
    stacked, with the q/k/v biases a Qwen2 file carries), RoPE on q and k,
    grouped-query attention over the row's KV cache, the output projection,
    residual, RmsNorm, the gate|up Q8_0 linear (stacked the same way), SwiGLU,
    down, residual; the final RmsNorm and the head (the tied token table or
    output.weight).  Each row's token and position live on the device
    (self.tokens, self.pos), so a step can be captured in one graph.

    from_weights takes numpy arrays keyed as a GGUF file names them
    (gguf/llama.rs:171-340): token_embd (Q8_0 bytes [vocab, d]), output
    (optional, Q8_0 [vocab, d]), output_norm [d], and per block i
    blk.i.attn_norm, attn_q / attn_k / attn_v (Q8_0) with optional .bias,
    attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down (Q8_0)."""

    def __init__(self, ctx: Context, cfg: dict, rows: int):
        import torch

        self.ctx, self.cfg, self.rows = ctx, dict(cfg), rows
        c = self.cfg
        self.vocab, self.d, self.nh, self.nkv, self.hd = c["vocab"], c["d"], c["n_heads"], c["n_kv"], c["head_dim"]
        self.layers, self.ffn, self.cap = c["layers"], c["ffn"], c["context"]
        self.rope_dim, self.rope_base = c.get("rope_dim", self.hd), c.get("rope_base", 10000.0)
        self.rope_type, self.eps = c.get("rope_type", ROPE_NEOX), c.get("eps", 1e-5)
        # RopeScaling (llm.rs): a linear position factor and optional per-pair
        # frequency factors (a device tensor of rope_dim / 2 floats, or None)
        self.rope_linear, self.rope_freqs = float(c.get("rope_linear", 1.0)), None
        self.q_dim, self.kv_dim = self.nh * self.hd, self.nkv * self.hd
        self.qkv_dim = self.q_dim + 2 * self.kv_dim
        dev, B = torch.device("cuda"), rows
        self.x = torch.zeros((B, self.d), device=dev)
        self.x2 = torch.zeros((B, self.d), device=dev)  # the residual stream alternates between x and x2
        self.h = torch.empty((B, self.d), device=dev)
        self.qkv = torch.empty((B, self.qkv_dim), device=dev)
        self.att = torch.empty((B, self.q_dim), device=dev)
        self.proj = torch.empty((B, self.d), device=dev)
        self.gu = torch.empty((B, 2 * self.ffn), device=dev)
        self.mid = torch.empty((B, self.ffn), device=dev)
        self.z = torch.empty((B, self.vocab), device=dev)
        self.tokens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.blocks = []
        # the residual stream's row statistics between a projection and the next RmsNorm
        self.fused = 3 <= B <= 64 and self.d % 32 == 0
        self.st = torch.empty((B, self.d // 32, 2), device=dev) if self.fused else None
        # SwiGLU inside the gate|up GEMM (a Q8_0 gate|up stored interleaved, ACT_SWIGLU32)
        self.glu = self.fused and self.ffn % 32 == 0 and self.d <= 1024

    def _alloc_cache(self):
        import torch

        n = self.rows * self.cap * self.kv_dim
        return torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda")

    @classmethod
    def from_weights(cls, ctx: Context, weights: dict, cfg: dict, rows: int) -> "LlamaDevice":
        import torch

        m = cls(ctx, cfg, rows)
        d, f = m.d, (lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda())
        raw = lambda name: np.asarray(weights[name], np.uint8).ravel()  # noqa: E731
        tok = raw("token_embd")
        m.tok_w = torch.empty((m.vocab, d), device="cuda")
        traw = torch.from_numpy(tok.copy()).cuda()
        torch.cuda.synchronize()
        q8_0_dequant_async(ctx, traw, m.vocab * d, m.tok_w)
        m.head = Q8_0Weight.upload(ctx, raw("output") if "output" in weights else tok, m.vocab, d)
        for i in range(m.layers):
            p = f"blk.{i}."
            qkv = np.concatenate([raw(p + "attn_q"), raw(p + "attn_k"), raw(p + "attn_v")])
            bias = np.concatenate([np.asarray(weights.get(p + f"attn_{s}.bias", np.zeros(n, np.float32)), np.float32)
                                   for s, n in (("q", m.q_dim), ("k", m.kv_dim), ("v", m.kv_dim))])
            gate, up = raw(p + "ffn_gate"), raw(p + "ffn_up")
            gate_up = interleave_gate_up(gate, up, m.ffn) if m.glu else np.concatenate([gate, up])
            k, v = m._alloc_cache()
            m.blocks.append({
                "attn_norm": f(weights[p + "attn_norm"]), "ffn_norm": f(weights[p + "ffn_norm"]),
                "qkv": Q8_0Weight.upload(ctx, qkv, m.qkv_dim, d), "qkv_b": f(bias),
                "o": Q8_0Weight.upload(ctx, raw(p + "attn_output"), d, m.q_dim),
                "gate_up": Q8_0Weight.upload(ctx, gate_up, 2 * m.ffn, d),
                "down": Q8_0Weight.upload(ctx, raw(p + "ffn_down"), d, m.ffn), "k": k, "v": v, "glu": m.glu})
        m.out_norm = f(weights["output_norm"])
        torch.cuda.synchronize()
        ctx.sync()
        return m

    @classmethod
    def from_gguf(cls, ctx: Context, path, rows: int = 1, capacity=None) -> "LlamaDevice":
        """A llama / qwen2 GGUF read as Gguf::load_llama_prec(None) reads it
        (gguf/llama.rs:171-340; the checks, llama_gguf_plan): rope type by
        architecture (NORM for llama, NEOX for qwen2), the metadata defaults,
        linear rope scaling and rope_freqs.weight, q/k/v biases when present,
        the head tied to the token table when output.weight is absent.  The
        q|k|v and gate|up matrices are stacked into one weight each (row
        concatenation: Q8_0 rows stay Q8_0 bytes; a group holding an F32 / F16
        matrix becomes one F32 weight, the Q8_0 rows expanded exactly).  Each
        row's KV cache holds `capacity` positions (default: the file's
        context_length)."""
        import torch

        with GGUFFile(path) as g:
            cfg, mats, tied = llama_gguf_plan(g)
            if capacity is not None:
                cfg["context"] = int(capacity)
            m = cls(ctx, cfg, rows)
            d = m.d
            f = lambda name: torch.from_numpy(np.ascontiguousarray(g.read_f32(ctx, name), np.float32).ravel()).cuda()  # noqa: E731

            def kind(name):
                ty = g.tensors[name][1]
                if ty not in (GGML_Q8_0, GGML_F32, GGML_F16):
                    raise FerrumHipError(FH_ERR_LIMIT, f"tensor '{name}' is GGML type {ty}; the device path takes "
                                                       "Q8_0, F32 or F16 matrices")
                return ty

            def shape(name):
                """(rows, row length) of a 2-D tensor: GGML dims are (ne0, ne1)."""
                dims = g.tensors[name][0]
                return int(dims[1]), int(dims[0])

            def dense(name):
                """The matrix's rows as f32 (Q8_0 expanded exactly: f16 scale times int8)."""
                n_out, n_in = shape(name)
                if kind(name) == GGML_Q8_0:
                    blk = np.frombuffer(g.raw(name), np.uint8).reshape(-1, 34)
                    sc = blk[:, :2].copy().view(np.float16).astype(np.float32)
                    return (sc * blk[:, 2:].copy().view(np.int8).astype(np.float32)).reshape(n_out, n_in)
                return g.read_f32(ctx, name).reshape(n_out, n_in)

            def weight(names, glu=False):
                """One device weight holding the rows of `names` in order (glu:
                gate and up interleaved for ACT_SWIGLU32, Q8_0 only)."""
                shapes = [shape(n) for n in names]
                n_in = shapes[0][1]
                if all(kind(n) == GGML_Q8_0 for n in names):
                    parts = [np.frombuffer(g.raw(n), np.uint8) for n in names]
                    raw = interleave_gate_up(parts[0], parts[1], shapes[0][0]) if glu else np.concatenate(parts)
                    return Q8_0Weight.upload(ctx, raw, sum(s[0] for s in shapes), n_in)
                return Q8_0Weight.upload_f32(ctx, np.concatenate([dense(n) for n in names]))

            if kind("token_embd.weight") == GGML_Q8_0:
                traw = torch.from_numpy(np.frombuffer(g.raw("token_embd.weight"), np.uint8).copy()).cuda()
                m.tok_w = torch.empty((m.vocab, d), device="cuda")
                torch.cuda.synchronize()
                q8_0_dequant_async(ctx, traw, m.vocab * d, m.tok_w)
                ctx.sync()
            else:
                m.tok_w = f("token_embd.weight").reshape(m.vocab, d)
            m.head = weight(["token_embd.weight" if tied else "output.weight"])
            for i in range(m.layers):
                p = f"blk.{i}."
                names = [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"]
                biases = [p + f"attn_{s}.bias" for s in "qkv"]
                qkv_b = None
                if any(b in g.tensors for b in biases):
                    qkv_b = torch.cat([f(b) if b in g.tensors else torch.zeros(n, device="cuda")
                                       for b, n in zip(biases, (m.q_dim, m.kv_dim, m.kv_dim))])
                k, v = m._alloc_cache()
                gu_names = [p + "ffn_gate.weight", p + "ffn_up.weight"]
                glu = m.glu and all(kind(n) == GGML_Q8_0 for n in gu_names)
                m.blocks.append({
                    "attn_norm": f(p + "attn_norm.weight"), "ffn_norm": f(p + "ffn_norm.weight"),
                    "qkv": weight(names), "qkv_b": qkv_b, "o": weight([p + "attn_output.weight"]),
                    "gate_up": weight(gu_names, glu), "down": weight([p + "ffn_down.weight"]), "k": k, "v": v,
                    "glu": glu})
            m.out_norm = f("output_norm.weight")
            if cfg["rope_freqs"]:
                m.rope_freqs = f("rope_freqs.weight")
            torch.cuda.synchronize()
            ctx.sync()
        return m

    @classmethod
    def random(cls, ctx: Context, cfg: dict, rows: int, gen) -> "LlamaDevice":
        """N(0, 0.02) Q8_0 weights generated and encoded on the device (for timing)."""
        import torch

        m = cls(ctx, cfg, rows)
        d = m.d

        def q8(n, k):
            w = torch.randn((n, k), generator=gen, device="cuda") * 0.02
            raw = torch.empty(n * k // 32 * 34, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            q8_0_encode_async(ctx, w, n * k, raw)
            q = Q8_0Weight.upload_device(ctx, raw, n, k)
            ctx.sync()
            return q, raw

        vec = lambda n, base=0.0: torch.randn(n, generator=gen, device="cuda") * 0.02 + base  # noqa: E731
        m.head, raw = q8(m.vocab, d)
        m.tok_w = torch.empty((m.vocab, d), device="cuda")
        q8_0_dequant_async(ctx, raw, m.vocab * d, m.tok_w)
        ctx.sync()
        for _ in range(m.layers):
            k, v = m._alloc_cache()
            m.blocks.append({"attn_norm": vec(d, 1.0), "ffn_norm": vec(d, 1.0), "qkv": q8(m.qkv_dim, d)[0],
                             "qkv_b": vec(m.qkv_dim), "o": q8(d, m.q_dim)[0], "gate_up": q8(2 * m.ffn, d)[0],
                             "down": q8(d, m.ffn)[0], "k": k, "v": v, "glu": m.glu})
        m.out_norm = vec(d, 1.0)
        torch.cuda.synchronize()
        ctx.sync()
        return m

    def launches_per_step(self) -> int:
        """Kernel launches of feed_async (the sampler not included): at 3 .. 64
        rows the o and down projections add themselves to the residual stream
        and leave its row statistics, and the q|k|v and gate|up GEMMs form the
        RmsNorm from them as they stage their inputs (seven launches per
        block, six with SwiGLU in the gate|up GEMM, one fewer again where the
        attention rotates q and k itself); otherwise each RmsNorm is a launch
        of its own (nine).  The head counts as one call (a wide head at more
        than 32 rows takes one launch per 32 rows)."""
        per = (6 if all(b.get("glu") for b in self.blocks) else 7) if self.fused else 9
        if self.fused and self._rope_in_attention():
            per -= 1
        return 1 + per * self.layers + 2 + (1 if self.fused else 0)

    def _rope_in_attention(self) -> bool:
        """Whether fh_gqa_attention_rope_decode_async rotates inside its one
        attention launch here (the library's rule for its batched kernel: head
        width 64, grouped heads, at least 128 workgroups of up to four query
        heads), rather than launching fh_rope first."""
        g = self.nh // self.nkv
        per = 4 if g >= 5 else 2
        return self.hd == 64 and g >= 2 and self.rows * self.nkv * -(-g // per) >= 128

    def forward_one(self, token: int):
        """LlamaModel::forward_one (llm.rs:606-616) for a single sequence (rows
        == 1): feed `token` at the next position and return the logits (host)
        — the callback llama_decode drives.  A full cache is FH_ERR_DIM."""
        import torch

        if self.rows != 1:
            raise FerrumHipError(FH_ERR_INVALID, "forward_one drives a single-row LlamaDevice")
        nxt = getattr(self, "next_pos", 0)
        if nxt >= self.cap:
            raise DimMismatch(FH_ERR_DIM, f"KvCache full ({self.cap} positions): clear and re-prime to continue")
        self.ctx.sync()
        self.tokens.fill_(int(token))
        self.pos.fill_(nxt)
        torch.cuda.current_stream().synchronize()
        self.feed_async(nxt)
        self.next_pos = nxt + 1
        self.ctx.sync()
        return self.z[0].cpu().numpy()

    def feed_async(self, max_pos: int):
        """One decode step of every row: token self.tokens[r] at position
        self.pos[r] (both on the device; max_pos bounds the positions).  The
        head's scores land in self.z; positions are not advanced."""
        ctx, d, B = self.ctx, self.d, self.rows
        embed_rows_async(ctx, self.tok_w, self.vocab, d, self.tokens, B, self.x)
        if self.fused:
            # x is updated in place by the o and down projections, which leave
            # its row statistics in self.st for the RmsNorm the next GEMM forms
            x, st = self.x, self.st
            for i, b in enumerate(self.blocks):
                qkv_b = b.get("qkv_b")
                if i == 0:
                    rmsnorm_async(ctx, x, None, None, B, d, b["attn_norm"], self.eps, self.h)
                    linear_forward_async(ctx, b["qkv"], self.h, B, d, qkv_b, 0 if qkv_b is None else self.qkv_dim,
                                         self.qkv)
                else:
                    linear_normed_async(ctx, b["qkv"], x, B, d, st, b["attn_norm"], None, self.eps, True, qkv_b,
                                        0 if qkv_b is None else self.qkv_dim, self.qkv)
                gqa_attention_rope_decode_async(ctx, self.qkv, self.qkv_dim, B, self.nh, self.nkv, self.hd, b["k"],
                                                b["v"], self.cap, self.pos, max_pos, self.rope_dim, self.rope_base,
                                                self.rope_type, self.rope_freqs, self.rope_linear, self.att)
                linear_residual_async(ctx, b["o"], self.att, B, self.q_dim, None, 0, x, x, st)
                if b.get("glu"):
                    linear_normed_async(ctx, b["gate_up"], x, B, d, st, b["ffn_norm"], None, self.eps, True, None, 0,
                                        self.mid, ACT_SWIGLU32)
                else:
                    linear_normed_async(ctx, b["gate_up"], x, B, d, st, b["ffn_norm"], None, self.eps, True, None, 0,
                                        self.gu)
                    swiglu_async(ctx, self.gu, self.gu[:, self.ffn:], B, self.ffn, 2 * self.ffn, self.mid)
                linear_residual_async(ctx, b["down"], self.mid, B, self.ffn, None, 0, x, x, st)
            rmsnorm_async(ctx, x, None, None, B, d, self.out_norm, self.eps, self.h)
            linear_forward_async(ctx, self.head, self.h, B, d, None, 0, self.z)
            return
        cur, other = self.x, self.x2
        for i, b in enumerate(self.blocks):
            if i == 0:
                rmsnorm_async(ctx, cur, None, None, B, d, b["attn_norm"], self.eps, self.h)
            else:  # the previous block's second residual add, then attn_norm
                rmsnorm_async(ctx, cur, self.proj, other, B, d, b["attn_norm"], self.eps, self.h)
                cur, other = other, cur
            qkv_b = b.get("qkv_b")  # (None: a file without q/k/v biases, whose linears are bias-free)
            linear_forward_async(ctx, b["qkv"], self.h, B, d, qkv_b, 0 if qkv_b is None else self.qkv_dim, self.qkv)
            rope_async(ctx, self.qkv, B, self.qkv_dim, self.nh + self.nkv, self.hd, self.rope_dim, self.pos,
                       self.rope_base, self.rope_type, self.rope_freqs, self.rope_linear)
            gqa_attention_decode_async(ctx, self.qkv, self.qkv_dim, B, self.nh, self.nkv, self.hd, b["k"], b["v"],
                                       self.cap, self.pos, max_pos, self.att)
            linear_forward_async(ctx, b["o"], self.att, B, self.q_dim, None, 0, self.proj)
            rmsnorm_async(ctx, cur, self.proj, other, B, d, b["ffn_norm"], self.eps, self.h)
            cur, other = other, cur
            linear_forward_async(ctx, b["gate_up"], self.h, B, d, None, 0, self.gu)
            swiglu_async(ctx, self.gu, self.gu[:, self.ffn:], B, self.ffn, 2 * self.ffn, self.mid)
            linear_forward_async(ctx, b["down"], self.mid, B, self.ffn, None, 0, self.proj)
        rmsnorm_async(ctx, cur, self.proj, None, B, d, self.out_norm, self.eps, self.h)
        linear_forward_async(ctx, self.head, self.h, B, d, None, 0, self.z)

    def free(self):
        self.head.free()
        for b in self.blocks:
            for key in ("qkv", "o", "gate_up", "down"):
                b[key].free()


class GPT2Device:
    """A GPT-2 decoder on the device, the way CachedTransformer::feed walks it
    (slm/cached.rs:100-125): embed_one, then per block forward_with_cache
    (layer/transformer.rs:221-290: LayerNorm, fused Q|K|V Q8_0 linear, KV-cache
    attention, out projection, residual, LayerNorm, up, GELU, down, residual),
    the final LayerNorm and the tied Q8_0 head.  The head's scores go to the
    fused sampler (softmax -> ln bridge inside it).

    from_weights takes a dict of numpy arrays -- token_embd_q8 (GGUF Q8_0
    bytes of the [vocab, d] token table; the embedding uses its f32 expansion
    and the head the Q8_0 rows, as the reference ties them), position_embd
    [ctx, d] f32, and per block i: ln1_g/ln1_b/ln2_g/ln2_b [d], qkv_q8
    ([3d, d] Q8_0) / qkv_b [3d], out_q8 / out_b, up_q8 ([ffn, d]) / up_b,
    down_q8 ([d, ffn]) / down_b; lnf_g / lnf_b.  random builds the same on the
    device from a torch generator (N(0, 0.02) weights, for timing)."""

    def __init__(self, ctx: Context, vocab: int, d: int, heads: int, layers: int, ffn: int, context: int):
        import torch

        self.ctx, self.vocab, self.d, self.heads, self.layers, self.ffn, self.cap = ctx, vocab, d, heads, layers, ffn, context
        dev = torch.device("cuda")
        self.x = torch.empty(d, device=dev)
        self.x2 = torch.empty(d, device=dev)  # the residual stream ping-pongs between x and x2
        self.h = torch.empty(d, device=dev)
        self.qkv = torch.empty(3 * d, device=dev)
        self.att = torch.empty(d, device=dev)
        self.proj = torch.empty(d, device=dev)
        self.mid = torch.empty(ffn, device=dev)
        self.z = torch.empty(vocab, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = 0
        self.blocks = []
        self.stack = None  # fh_gpt2_stack: the whole block stack as one launch (when the shape has a kernel)
        self.fused = True

    def _make_stack(self):
        """The one-launch block stack (fh_gpt2_stack_create); shapes without a
        kernel keep the one-launch-per-op path (FH_ERR_LIMIT)."""
        blocks = (GPT2Block * self.layers)()
        for i, b in enumerate(self.blocks):
            blocks[i] = GPT2Block(b["qkv"].h, b["out"].h, b["up"].h, b["down"].h, _ptr(b["qkv_b"]), _ptr(b["out_b"]),
                                  _ptr(b["up_b"]), _ptr(b["down_b"]), _ptr(b["ln1_g"]), _ptr(b["ln1_b"]),
                                  _ptr(b["ln2_g"]), _ptr(b["ln2_b"]), _ptr(b["k"]), _ptr(b["v"]))
        h = C.c_void_p()
        rc = lib().fh_gpt2_stack_create(self.ctx.h, blocks, self.layers, self.d, self.heads, self.ffn, self.cap,
                                        _ptr(self.tok_w), _ptr(self.pos_w), self.vocab, self.pos_w.shape[0],
                                        C.byref(h))
        if rc == FH_ERR_LIMIT:
            return
        self.ctx.check(rc)
        self.stack = h

    def _block(self, ln, qkv, qkv_b, out, out_b, up, up_b, down, down_b):
        import torch

        return dict(ln1_g=ln[0], ln1_b=ln[1], ln2_g=ln[2], ln2_b=ln[3], qkv=qkv, qkv_b=qkv_b, out=out, out_b=out_b,
                    up=up, up_b=up_b, down=down, down_b=down_b,
                    k=torch.zeros((self.cap, self.d), device="cuda"), v=torch.zeros((self.cap, self.d), device="cuda"))

    @classmethod
    def from_weights(cls, ctx: Context, weights: dict, vocab: int, d: int, heads: int, layers: int, ffn: int,
                     context: int) -> "GPT2Device":
        import torch

        m = cls(ctx, vocab, d, heads, layers, ffn, context)
        f = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()  # noqa: E731
        tok = np.frombuffer(bytes(np.asarray(weights["token_embd_q8"], np.uint8)), np.uint8)
        m.head = Q8_0Weight.upload(ctx, tok, vocab, d)
        m.tok_w = torch.empty((vocab, d), device="cuda")
        raw = torch.from_numpy(tok.copy()).cuda()
        torch.cuda.synchronize()
        q8_0_dequant_async(ctx, raw, vocab * d, m.tok_w)
        m.pos_w = f(weights["position_embd"])
        for i in range(layers):
            g = lambda name: weights[f"blk{i}.{name}"]  # noqa: E731
            up = lambda name, n, k: Q8_0Weight.upload(ctx, np.asarray(g(name), np.uint8), n, k)  # noqa: E731
            m.blocks.append(m._block([f(g(n)) for n in ("ln1_g", "ln1_b", "ln2_g", "ln2_b")],
                                     up("qkv_q8", 3 * d, d), f(g("qkv_b")), up("out_q8", d, d), f(g("out_b")),
                                     up("up_q8", ffn, d), f(g("up_b")), up("down_q8", d, ffn), f(g("down_b"))))
        m.lnf_g, m.lnf_b = f(weights["lnf_g"]), f(weights["lnf_b"])
        torch.cuda.synchronize()  # uploads ran on torch's stream
        ctx.sync()
        m._make_stack()
        return m

    @classmethod
    def from_gguf(cls, ctx: Context, path) -> "GPT2Device":
        """A GPT-2 GGUF read as gpt2_from reads it (loader/gpt2.rs:201-295;
        the checks, gpt2_gguf_plan): hyperparameters from the gpt2.* keys, the
        layer_norm_epsilon check, the token table's rows (and an untied
        output.weight's) reordered to ferrum_core's vocabulary order
        (ferrum_vocab / permute_rows, loader/gpt2.rs:149-199); Q8_0 matrices
        uploaded straight from the file's mapping (a row permutation of Q8_0
        rows is exact), F32 / F16 ones (the reference's writer stores a matrix
        as F32 when ne0 % 32 != 0, loader/mod.rs:147-152) as F32 weights; the
        head is output.weight when present, else the token table (tied).  A
        model with an F32 matrix runs one op at a time (the one-launch stack
        takes Q8_0 only)."""
        import torch

        with GGUFFile(path) as g:
            cfg, perm, tied = gpt2_gguf_plan(g)
            vocab, d = cfg["vocab"], cfg["d"]
            m = cls(ctx, vocab, d, cfg["heads"], cfg["layers"], cfg["ffn"], cfg["context"])
            identity = perm == list(range(vocab))
            f = lambda name: torch.from_numpy(g.read_f32(ctx, name).copy()).cuda()  # noqa: E731

            def rows_q8(name):
                raw = np.frombuffer(g.raw(name), np.uint8).reshape(vocab, -1)
                return raw if identity else raw[perm]

            def rows_f32(name):
                a = g.read_f32(ctx, name).reshape(vocab, d)
                return a if identity else a[perm]

            def table(name):
                """(device Q8_0-or-F32 weight of the vocab rows, f32 rows on the device)."""
                ty = g.tensors[name][1]
                if ty == GGML_Q8_0:
                    raw = np.ascontiguousarray(rows_q8(name))
                    w = Q8_0Weight.upload(ctx, raw, vocab, d)
                    dense = torch.empty((vocab, d), device="cuda")
                    traw = torch.from_numpy(raw.ravel().copy()).cuda()
                    torch.cuda.synchronize()
                    q8_0_dequant_async(ctx, traw, vocab * d, dense)
                    ctx.sync()
                    return w, dense
                if ty in (GGML_F32, GGML_F16):
                    a = np.ascontiguousarray(rows_f32(name))
                    return Q8_0Weight.upload_f32(ctx, a), torch.from_numpy(a.copy()).cuda()
                raise FerrumHipError(FH_ERR_LIMIT, f"tensor '{name}' is GGML type {ty}; the device path takes "
                                                   "Q8_0, F32 or F16 matrices")

            def mat(name):
                ty = g.tensors[name][1]
                if ty == GGML_Q8_0:
                    return g.upload_q8_0(ctx, name)
                if ty in (GGML_F32, GGML_F16):
                    return Q8_0Weight.upload_f32(ctx, g.read_f32(ctx, name))
                raise FerrumHipError(FH_ERR_LIMIT, f"tensor '{name}' is GGML type {ty}; the device path takes "
                                                   "Q8_0, F32 or F16 matrices")

            tok_w, m.tok_w = table("token_embd.weight")
            if tied:
                m.head = tok_w
            else:
                tok_w.free()
                m.head = table("output.weight")[0]
            m.pos_w = f("position_embd.weight")
            for i in range(cfg["layers"]):
                n = lambda s: f"blk.{i}.{s}"  # noqa: E731
                m.blocks.append(m._block([f(n("attn_norm.weight")), f(n("attn_norm.bias")), f(n("ffn_norm.weight")),
                                          f(n("ffn_norm.bias"))],
                                         mat(n("attn_qkv.weight")), f(n("attn_qkv.bias")),
                                         mat(n("attn_output.weight")), f(n("attn_output.bias")),
                                         mat(n("ffn_up.weight")), f(n("ffn_up.bias")),
                                         mat(n("ffn_down.weight")), f(n("ffn_down.bias"))))
            m.lnf_g, m.lnf_b = f("output_norm.weight"), f("output_norm.bias")
            m.vocab_perm = None if identity else perm
            torch.cuda.synchronize()
            ctx.sync()
        m._make_stack()
        return m

    @classmethod
    def random(cls, ctx: Context, vocab: int, d: int, heads: int, layers: int, ffn: int, context: int,
               gen) -> "GPT2Device":
        import torch

        m = cls(ctx, vocab, d, heads, layers, ffn, context)

        def q8(n, k):
            w = torch.randn((n, k), generator=gen, device="cuda") * 0.02
            raw = torch.empty(n * k // 32 * 34, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            q8_0_encode_async(ctx, w, n * k, raw)
            q = Q8_0Weight.upload_device(ctx, raw, n, k)
            ctx.sync()
            return q, raw

        vec = lambda n, base=0.0: torch.randn(n, generator=gen, device="cuda") * 0.02 + base  # noqa: E731
        m.head, raw = q8(vocab, d)
        m.tok_w = torch.empty((vocab, d), device="cuda")
        q8_0_dequant_async(ctx, raw, vocab * d, m.tok_w)
        ctx.sync()
        m.pos_w = vec(context * d).reshape(context, d)
        for _ in range(layers):
            m.blocks.append(m._block([vec(d, 1.0), vec(d), vec(d, 1.0), vec(d)], q8(3 * d, d)[0], vec(3 * d),
                                     q8(d, d)[0], vec(d), q8(ffn, d)[0], vec(ffn), q8(d, ffn)[0], vec(d)))
        m.lnf_g, m.lnf_b = vec(d, 1.0), vec(d)
        torch.cuda.synchronize()
        ctx.sync()
        m._make_stack()
        return m

    def feed_async(self, d_token, pos: int):
        """One position: the head's scores for the next token land in self.z.
        With the one-launch stack: the stack (embedding and every block) into
        self.x, then the final LayerNorm fused into the head GEMV (two
        launches); otherwise one launch per op."""
        ctx, d = self.ctx, self.d
        if self.stack is not None and self.fused:
            ctx.check(lib().fh_gpt2_stack_forward_async(ctx.h, self.stack, _ptr(d_token), int(pos), _ptr(self.x)))
            linear_ln_async(ctx, self.head, self.x, None, None, 1, d, self.lnf_g, self.lnf_b, None, 0, self.z)
            return
        embed_one_async(ctx, self.tok_w, self.pos_w, self.vocab, self.pos_w.shape[0], d, d_token, pos, self.x)
        cur, other = self.x, self.x2
        for i, b in enumerate(self.blocks):
            # Each residual add runs inside the linear after it, together with
            # the LayerNorm: the sum lands in `other`, which becomes `cur`.
            if i == 0:
                layernorm_async(ctx, cur, 1, d, b["ln1_g"], b["ln1_b"], self.h)
                linear_forward_async(ctx, b["qkv"], self.h, 1, d, b["qkv_b"], 3 * d, self.qkv)
            else:
                linear_ln_async(ctx, b["qkv"], cur, self.proj, other, 1, d, b["ln1_g"], b["ln1_b"], b["qkv_b"], 3 * d,
                                self.qkv)
                cur, other = other, cur
            attention_decode_async(ctx, self.qkv, b["k"], b["v"], self.cap, d, self.heads, pos, self.att)
            linear_forward_async(ctx, b["out"], self.att, 1, d, b["out_b"], d, self.proj)
            linear_ln_async(ctx, b["up"], cur, self.proj, other, 1, d, b["ln2_g"], b["ln2_b"], b["up_b"], self.ffn,
                            self.mid, ACT_GELU)
            cur, other = other, cur
            linear_forward_async(ctx, b["down"], self.mid, 1, self.ffn, b["down_b"], d, self.proj)
        linear_ln_async(ctx, self.head, cur, self.proj, None, 1, d, self.lnf_g, self.lnf_b, None, 0, self.z)

    def launches_per_step(self) -> int:
        """Kernel launches of feed_async (the sampler not included)."""
        if self.stack is not None and self.fused:
            return 2
        return 2 + 5 * self.layers + 1

    def prefill_async(self, d_tokens, pos0: int, n: int):
        """Positions pos0 .. pos0 + n - 1 (tokens on the device) through every
        block at once, as n rows of one sequence: the same ops as feed_async's
        per-op path with m = n (GEMMs for the linears, the block's attention
        with every row's k / v in the cache first), the final LayerNorm and
        the head for the last position only.  What CachedTransformer::feed
        computes one token at a time (slm/cached.rs:100-125), within the 1e-5
        rule (the GEMMs and the attention chunks sum in another order).  The
        last position's scores land in self.z; the caches hold every row."""
        import torch

        ctx, d, ffn = self.ctx, self.d, self.ffn
        if n <= 0:
            return
        if pos0 + n > self.cap:
            raise DimMismatch(FH_ERR_DIM, f"KvCache full ({self.cap} positions): clear and re-prime to continue")
        dev = "cuda"
        x, x2, h = (torch.empty((n, d), device=dev) for _ in range(3))
        qkv, att, proj = torch.empty((n, 3 * d), device=dev), torch.empty((n, d), device=dev), \
            torch.empty((n, d), device=dev)
        mid = torch.empty((n, ffn), device=dev)
        embed_rows_async(ctx, self.tok_w, self.vocab, d, d_tokens, n, x)
        add_async(ctx, x, self.pos_w[pos0:pos0 + n], n * d)  # tok + pos, as embed_one adds them
        cur, other = x, x2
        for i, b in enumerate(self.blocks):
            if i == 0:
                layernorm_async(ctx, cur, n, d, b["ln1_g"], b["ln1_b"], h)
                linear_forward_async(ctx, b["qkv"], h, n, d, b["qkv_b"], 3 * d, qkv)
            else:
                linear_ln_async(ctx, b["qkv"], cur, proj, other, n, d, b["ln1_g"], b["ln1_b"], b["qkv_b"], 3 * d, qkv)
                cur, other = other, cur
            attention_prefill_async(ctx, qkv, b["k"], b["v"], self.cap, d, self.heads, pos0, n, att)
            linear_forward_async(ctx, b["out"], att, n, d, b["out_b"], d, proj)
            linear_ln_async(ctx, b["up"], cur, proj, other, n, d, b["ln2_g"], b["ln2_b"], b["up_b"], ffn, mid, ACT_GELU)
            cur, other = other, cur
            linear_forward_async(ctx, b["down"], mid, n, ffn, b["down_b"], d, proj)
        linear_ln_async(ctx, self.head, cur[n - 1:], proj[n - 1:], None, 1, d, self.lnf_g, self.lnf_b, None, 0, self.z)
        self._keep = (x, x2, h, qkv, att, proj, mid)  # alive until the stream has used them

    def generate(self, prompt, max_tokens: int, params: SamplingParams, rng: Rng, eos=None, bos: int = 0,
                 prefill: bool = False, cancel=None, chunk: int = 32, timings=None):
        """GenerativeSLM::token_stream + stream_next (slm/token_stream.rs:66-190)
        with every step on the device: the prompt is primed, then each step
        runs the block stack, the head and the fused sampler, which writes its
        id straight into the device history (the penalty window) where the
        next step's embedding reads it.  Same kernels and order as gpt2_decode
        over forward(), so the same ids.

        The steps run in chunks of `chunk`; between chunks the host reads the
        chunk's ids and stops at the first EOS (drawn, not returned, as
        stream_next does) and checks `cancel` (see cancelled): a set flag ends
        the run before the next chunk, which is where a device-resident loop
        can see it (the reference checks once per token; a flag set before
        the call returns nothing).  Steps a chunk computed past an EOS are
        discarded.  The draws are rng's (one next_u64 per sampled step, none
        when greedy): they are taken from a copy of rng up front, and rng
        itself is then advanced by exactly the draws of the steps returned
        plus the EOS step, so it ends in ferrum_core's state.  A run that
        would outgrow the window (prompt + max_tokens > context: the reference
        cuts and re-primes) takes the host loop instead.

        prefill=True primes the prompt in one pass (prefill_async: its
        positions as rows of GEMMs) instead of position by position: much
        faster for long prompts, and the same run within the 1e-5 rule
        rather than bit for bit.

        timings (a list, optional) receives the wall-clock milliseconds from
        the call's start to the end of the prime and of each chunk."""
        import time

        import torch

        t_start = time.perf_counter()
        win = GPT2Window(self.cap, prompt, bos)
        n0 = len(win.ids)
        if n0 + max_tokens > self.cap or self.stack is None or not self.fused:
            return gpt2_decode(self.ctx, self.forward, prompt, max_tokens, params, rng, self.cap, eos, bos, cancel)
        if max_tokens <= 0 or cancelled(cancel):
            return []
        ctx, dev = self.ctx, "cuda"
        chunk = max(int(chunk), 1)
        greedy = params.temperature <= 0.0
        hist = torch.zeros(n0 + max_tokens, dtype=torch.int32, device=dev)
        hist[:n0] = torch.tensor(win.ids, dtype=torch.int32, device=dev)
        # step j's penalty window is hist[0 : n0 + j], built on the device (a
        # nested Python list of max_tokens pairs can set off a full garbage
        # collection of the host process, tens of ms, inside the run)
        offs = torch.zeros((max_tokens, 2), dtype=torch.int32, device=dev)
        offs[:, 1] = torch.arange(n0, n0 + max_tokens, dtype=torch.int32, device=dev)
        draws = None
        if not greedy:
            probe = Rng.from_state(rng.state)
            d = np.array([probe.next_u64() for _ in range(max_tokens)], dtype=np.uint64)
            draws = torch.from_numpy(d.view(np.int64)).to(dev)
        torch.cuda.synchronize()
        ctx.sync()
        # prime: positions 0 .. n0 - 2 (the last prompt position is the first step's)
        if prefill and n0 > 1:
            self.prefill_async(hist, 0, n0 - 1)
        else:
            for p in range(n0 - 1):
                ctx.check(lib().fh_gpt2_stack_forward_async(ctx.h, self.stack, hist.data_ptr() + 4 * p, p,
                                                            _ptr(self.x)))
        if timings is not None:
            ctx.sync()
            timings.append(round((time.perf_counter() - t_start) * 1e3, 3))
        out, used, k = [], 0, 0
        while k < max_tokens:
            if k > 0 and cancelled(cancel):
                break
            c = min(chunk, max_tokens - k)
            for j in range(k, k + c):
                p = n0 - 1 + j
                self.feed_async(hist.data_ptr() + 4 * p, p)
                sample_rows_async(ctx, self.z, 1, self.vocab, params, hist, offs[j], None if greedy else draws[j:],
                                  hist.data_ptr() + 4 * (n0 + j), LOGITS_GPT2_SOFTMAX)
            ctx.sync()
            if timings is not None:
                timings.append(round((time.perf_counter() - t_start) * 1e3, 3))
            got = [int(t) for t in hist[n0 + k:n0 + k + c].cpu().numpy()]
            k += c
            stop = False
            for t in got:
                used += 1
                if eos is not None and t == eos:
                    stop = True
                    break
                out.append(t)
            if stop:
                break
        if not greedy:
            for _ in range(used):
                rng.next_u64()
        self.pos = n0 - 1 + k
        return out

    def forward(self, ids, reprime: bool):
        """gpt2_decode's forward: re-feed the whole window from position 0, or
        feed its last id at the next position.  Returns the scores (host)."""
        import torch

        ids = list(ids)
        if reprime:
            self.pos = 0
            todo = ids
        else:
            todo = ids[-1:]
        for t in todo:
            self.ctx.sync()
            self.token.fill_(int(t))
            torch.cuda.current_stream().synchronize()
            self.feed_async(self.token, self.pos)
            self.pos += 1
        self.ctx.sync()
        return self.z.cpu().numpy()

    def free(self):
        if self.stack is not None:
            lib().fh_gpt2_stack_free(self.stack)
            self.stack = None
        self.head.free()
        for b in self.blocks:
            for key in ("qkv", "out", "up", "down"):
                b[key].free()


class GPT2Batch:
    """`rows` GPT-2 sequences decoded together on one GPT2Device's weights.
    Each row is its own CachedTransformer (slm/cached.rs:100-137) with its own
    KV caches ([rows, capacity, d] per block) and token window; one step feeds
    every row's token at its own position through the same ops as
    GPT2Device's per-op path with the linears as GEMMs over the rows (the
    batched decode of BASELINE's b32 figure and configs[3]), then the final
    LayerNorm, the head and the fused sampler over the rows.  prefill_async
    primes equal-length prompts of all rows in one pass (rows x positions as
    the GEMMs' rows, one attention launch per block for all sequences).  Per row the
    arithmetic is GPT2Device's, so a row matches ferrum_core's single-sequence
    decode within the same 1e-5 rule.  Token and position ids live on the
    device, so a step can be captured in one graph."""

    def __init__(self, model: GPT2Device, rows: int, capacity: int):
        import torch

        if rows < 1 or rows > 65535 or capacity < 1:
            raise FerrumHipError(FH_ERR_INVALID, "GPT2Batch: rows in 1 .. 65535 and capacity >= 1")
        if capacity > model.pos_w.shape[0]:
            raise DimMismatch(FH_ERR_DIM, f"GPT2Batch: capacity {capacity} exceeds max_seq_len {model.pos_w.shape[0]}")
        m, dev, B, d = model, "cuda", rows, model.d
        self.m, self.ctx, self.rows, self.cap = m, m.ctx, rows, capacity
        self.k = [torch.zeros(B * capacity * d, device=dev) for _ in range(m.layers)]
        self.v = [torch.zeros(B * capacity * d, device=dev) for _ in range(m.layers)]
        self.x, self.x2, self.h, self.att, self.proj = (torch.empty((B, d), device=dev) for _ in range(5))
        self.qkv = torch.empty((B, 3 * d), device=dev)
        self.mid = torch.empty((B, m.ffn), device=dev)
        self.z = torch.empty((B, m.vocab), device=dev)
        self.tokens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        # the residual stream's row statistics between a projection and the next LayerNorm
        self.fused = 3 <= B <= 64 and d % 32 == 0
        self.st = torch.empty((B, d // 32, 2), device=dev) if self.fused else None

    def launches_per_step(self) -> int:
        """Kernel launches of feed_async (the sampler not included).  At 3 ..
        64 rows the out and down projections add themselves to the residual
        stream and leave its row statistics, and the Q|K|V and up GEMMs
        normalise from those as they stage their inputs: five launches per
        block, plus the embedding, block 0's LayerNorm, the final LayerNorm and
        the head.  At one or two rows the decode GEMV forms each LayerNorm
        itself (the residual add inside it); past 64 rows each linear after a
        LayerNorm takes two launches."""
        L = self.m.layers
        if self.fused:
            return 4 + 5 * L
        return 3 + 5 * L if self.rows <= 2 else 3 + 7 * L

    def _cache(self, i, b):
        n = self.cap * self.m.d
        return self.k[i][b * n:(b + 1) * n], self.v[i][b * n:(b + 1) * n]

    def feed_async(self, d_tokens, d_pos, max_pos: int, hist=None, hist_stride: int = 0):
        """One decode step of every row: token d_tokens[r] at position d_pos[r]
        (device ids; max_pos bounds the positions and must be below the
        capacity).  With hist, each row's id is recorded at hist[r, pos[r]].
        The head's scores land in self.z; nothing is advanced."""
        m, ctx, B, d = self.m, self.ctx, self.rows, self.m.d
        if max_pos >= self.cap:
            raise DimMismatch(FH_ERR_DIM, f"KvCache full ({self.cap} positions): clear and re-prime to continue")
        embed_rows_pos_async(ctx, m.tok_w, m.pos_w, m.vocab, m.pos_w.shape[0], d, d_tokens, d_pos, B, self.x, hist,
                             hist_stride)
        if self.fused:
            # the residual stream x is updated in place by the out and down
            # projections, which leave its row statistics in self.st for the
            # LayerNorm the next GEMM forms as it stages x
            x, st, H = self.x, self.st, m.heads
            for i, b in enumerate(m.blocks):
                if i == 0:
                    layernorm_async(ctx, x, B, d, b["ln1_g"], b["ln1_b"], self.h)
                    linear_forward_async(ctx, b["qkv"], self.h, B, d, b["qkv_b"], 3 * d, self.qkv)
                else:
                    linear_normed_async(ctx, b["qkv"], x, B, d, st, b["ln1_g"], b["ln1_b"], 1e-5, False, b["qkv_b"],
                                        3 * d, self.qkv)
                gqa_attention_decode_async(ctx, self.qkv, 3 * d, B, H, H, d // H, self.k[i], self.v[i], self.cap,
                                           d_pos, max_pos, self.att)
                linear_residual_async(ctx, b["out"], self.att, B, d, b["out_b"], d, x, x, st)
                linear_normed_async(ctx, b["up"], x, B, d, st, b["ln2_g"], b["ln2_b"], 1e-5, False, b["up_b"], m.ffn,
                                    self.mid, ACT_GELU)
                linear_residual_async(ctx, b["down"], self.mid, B, m.ffn, b["down_b"], d, x, x, st)
            layernorm_async(ctx, x, B, d, m.lnf_g, m.lnf_b, self.h)
            linear_forward_async(ctx, m.head, self.h, B, d, None, 0, self.z)
            return
        cur, other = self.x, self.x2
        for i, b in enumerate(m.blocks):
            if i == 0:
                layernorm_async(ctx, cur, B, d, b["ln1_g"], b["ln1_b"], self.h)
                linear_forward_async(ctx, b["qkv"], self.h, B, d, b["qkv_b"], 3 * d, self.qkv)
            else:
                linear_ln_async(ctx, b["qkv"], cur, self.proj, other, B, d, b["ln1_g"], b["ln1_b"], b["qkv_b"], 3 * d,
                                self.qkv)
                cur, other = other, cur
            gqa_attention_decode_async(ctx, self.qkv, 3 * d, B, m.heads, m.heads, d // m.heads, self.k[i], self.v[i],
                                       self.cap, d_pos, max_pos, self.att)
            linear_forward_async(ctx, b["out"], self.att, B, d, b["out_b"], d, self.proj)
            linear_ln_async(ctx, b["up"], cur, self.proj, other, B, d, b["ln2_g"], b["ln2_b"], b["up_b"], m.ffn,
                            self.mid, ACT_GELU)
            cur, other = other, cur
            linear_forward_async(ctx, b["down"], self.mid, B, m.ffn, b["down_b"], d, self.proj)
        linear_ln_async(ctx, m.head, cur, self.proj, None, B, d, m.lnf_g, m.lnf_b, None, 0, self.z)

    def prefill_async(self, d_tokens, n: int, pos0: int = 0):
        """Positions pos0 .. pos0 + n - 1 of every row at once: d_tokens holds
        rows x n ids (row-major), the GEMMs run over all rows x n of them and
        each sequence's attention reads and fills its own caches (GPT2Device.
        prefill_async per sequence, batched).  Nothing reaches the head: the
        first decode step feeds the next position."""
        import torch

        m, ctx, B, d = self.m, self.ctx, self.rows, self.m.d
        if n <= 0:
            return
        if pos0 + n > self.cap:
            raise DimMismatch(FH_ERR_DIM, f"KvCache full ({self.cap} positions): clear and re-prime to continue")
        N = B * n
        if N > 65535:
            raise FerrumHipError(FH_ERR_LIMIT, f"GPT2Batch.prefill_async: rows x positions = {N} above 65535")
        dev = "cuda"
        x, x2, h, att, proj = (torch.empty((N, d), device=dev) for _ in range(5))
        qkv, mid = torch.empty((N, 3 * d), device=dev), torch.empty((N, m.ffn), device=dev)
        pos = torch.arange(pos0, pos0 + n, dtype=torch.int32, device=dev).repeat(B)
        torch.cuda.synchronize()
        embed_rows_pos_async(ctx, m.tok_w, m.pos_w, m.vocab, m.pos_w.shape[0], d, d_tokens, pos, N, x)
        cur, other = x, x2
        for i, b in enumerate(m.blocks):
            if i == 0:
                layernorm_async(ctx, cur, N, d, b["ln1_g"], b["ln1_b"], h)
                linear_forward_async(ctx, b["qkv"], h, N, d, b["qkv_b"], 3 * d, qkv)
            else:
                linear_ln_async(ctx, b["qkv"], cur, proj, other, N, d, b["ln1_g"], b["ln1_b"], b["qkv_b"], 3 * d, qkv)
                cur, other = other, cur
            attention_prefill_seqs_async(ctx, qkv, self.k[i], self.v[i], self.cap * d, self.cap, d, m.heads, pos0, n,
                                         B, att)
            linear_forward_async(ctx, b["out"], att, N, d, b["out_b"], d, proj)
            linear_ln_async(ctx, b["up"], cur, proj, other, N, d, b["ln2_g"], b["ln2_b"], b["up_b"], m.ffn, mid,
                            ACT_GELU)
            cur, other = other, cur
            linear_forward_async(ctx, b["down"], mid, N, m.ffn, b["down_b"], d, proj)
        # the last block's down projection is not added in: no position here reaches the head
        self._keep = (x, x2, h, att, proj, qkv, mid, pos)  # alive until the stream has used them

    def generate(self, prompts, max_tokens: int, params: SamplingParams, rngs, eos=None, prefill: bool = True,
                 cancel=None, chunk: int = 32):
        """GenerativeSLM::token_stream + stream_next (slm/token_stream.rs:66-190)
        for every row at once, each step on the device: row r's prompt
        (all of equal length), then up to max_tokens steps sampled with
        `params` over row r's window (its prompt and everything sampled so
        far), the draws from rngs[r] (one next_u64 per sampled step, none when
        greedy), the sampler's ids feeding the next step's embedding on the
        device.  The prompt is primed in one pass (prefill=True) or position
        by position.  Windows never outgrow the capacity here (prompt +
        max_tokens <= capacity; the reference would cut and re-prime).

        Each row is its own stream: it stops at its first EOS (drawn, not
        returned).  The steps run in chunks of `chunk`; between chunks the
        host reads the ids, and the run ends once every row has stopped or
        `cancel` (see cancelled) is set (checked before each chunk: the
        granularity at which a device-resident loop sees the flag).  A row
        that has stopped is still computed with the others until the run ends
        and those steps are discarded (rows are independent, so the other
        rows do not change).  rngs[r] is advanced by exactly the draws of row
        r's returned steps plus its EOS step, so each ends in ferrum_core's
        state.  Returns one id list per row."""
        import torch

        B, ctx = self.rows, self.ctx
        P = np.asarray(prompts, np.int64)
        if P.ndim != 2 or P.shape[0] != B or P.shape[1] < 1:
            raise FerrumHipError(FH_ERR_INVALID, f"GPT2Batch.generate: {B} prompts of one length >= 1")
        if (P < 0).any() or (P >= 2 ** 32).any():
            raise FerrumHipError(FH_ERR_INVALID, "GPT2Batch.generate: ids must fit u32")
        if len(rngs) != B and params.temperature > 0.0:
            raise FerrumHipError(FH_ERR_INVALID, f"GPT2Batch.generate: {len(rngs)} generators for {B} rows")
        n0 = P.shape[1]
        L = n0 + max_tokens
        if max_tokens < 1 or cancelled(cancel):
            return [[] for _ in range(B)]
        if L > self.cap:
            raise DimMismatch(FH_ERR_DIM, f"GPT2Batch.generate: prompt + max_tokens = {L} above the capacity "
                                          f"{self.cap}")
        dev, greedy = "cuda", params.temperature <= 0.0
        chunk = max(int(chunk), 1)
        hist = torch.zeros((B, L), dtype=torch.int32, device=dev)
        hist[:, :n0] = torch.from_numpy(P.astype(np.uint32).view(np.int32)).to(dev)
        ids = torch.zeros((max_tokens + 1, B), dtype=torch.int32, device=dev)  # ids[k]: the ids step k feeds
        ids[0] = hist[:, n0 - 1]
        steps = torch.arange(max_tokens, dtype=torch.int32, device=dev)
        pos = (n0 - 1 + steps)[:, None].repeat(1, B).contiguous()
        starts = torch.arange(B, dtype=torch.int32, device=dev) * L
        ranges = torch.stack([starts[None, :].repeat(max_tokens, 1),
                              starts[None, :] + (n0 + steps)[:, None]], dim=2).contiguous()  # [steps, B, 2]
        draws = None
        if not greedy:
            probes = [Rng.from_state(r.state) for r in rngs]
            dr = np.empty((max_tokens, B), dtype=np.uint64)  # (filled in place: no per-step Python lists)
            for t in range(max_tokens):
                for r in range(B):
                    dr[t, r] = probes[r].next_u64()
            draws = torch.from_numpy(dr.view(np.int64)).to(dev)
        toks = hist[:, :n0 - 1].contiguous()
        torch.cuda.synchronize()
        ctx.sync()
        if n0 > 1:
            if prefill:
                self.prefill_async(toks, n0 - 1)
            else:
                for p in range(n0 - 1):
                    col = toks[:, p].contiguous()
                    pp = torch.full((B,), p, dtype=torch.int32, device=dev)
                    torch.cuda.synchronize()
                    self.feed_async(col, pp, p)
                    ctx.sync()
        kind = LOGITS_GPT2_SOFTMAX | RECENT_RANGES
        res = [[] for _ in range(B)]
        used = [0] * B
        live = [True] * B
        k = 0
        while k < max_tokens and any(live):
            if k > 0 and cancelled(cancel):
                break
            c = min(chunk, max_tokens - k)
            for j in range(k, k + c):
                self.feed_async(ids[j], pos[j], n0 - 1 + j, hist, L)
                sample_rows_async(ctx, self.z, B, self.m.vocab, params, hist, ranges[j],
                                  None if greedy else draws[j], ids[j + 1], kind)
            ctx.sync()
            got = ids[k + 1:k + 1 + c].cpu().numpy().astype(np.int64)  # [c, B]
            k += c
            for r in range(B):
                for t in got[:, r]:
                    if not live[r]:
                        break
                    used[r] += 1
                    if eos is not None and int(t) == eos:
                        live[r] = False
                    else:
                        res[r].append(int(t))
        if not greedy:
            for r in range(B):
                for _ in range(used[r]):
                    rngs[r].next_u64()
        return res
