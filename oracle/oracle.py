"""ctypes/numpy face of the CPU oracle (oracle/ferrum_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg may import this module, and only as the checker
(or the timed CPU baseline) -- never as the thing measured or shipped.  The
product path (ferrum-cpu_amd/ferrum_hip) does not import it.

Each wrapper names the ferrum_core function it restates; the file:line
citations live beside the C declarations in oracle/ferrum_oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libferrum_oracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


class _f32p_or_null:
    """A float32 array argument that may be None (NULL)."""

    @classmethod
    def from_param(cls, obj):
        return None if obj is None else _f32p.from_param(obj)
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class SamplingParams(C.Structure):
    """slm/sampling.rs:27-38 without the cancel flag (a control, not a setting)."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("repetition_penalty", C.c_float),
    ]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0):
        super().__init__(float(temperature), int(top_k), float(top_p), float(repetition_penalty))


class SampleInfo(C.Structure):
    _fields_ = [
        ("path", C.c_int32),
        ("n_kept", C.c_uint32),
        ("margin", C.c_float),
        ("greedy_gap", C.c_float),
        ("topk_gap", C.c_float),
        ("topp_gap", C.c_float),
        ("draw_gap", C.c_float),
        ("topp_tie", C.c_uint32),
    ]


PATH_GREEDY, PATH_FALLBACK, PATH_SAMPLED = 0, 1, 2


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, seconds)."""
    if force or not os.path.exists(LIB_PATH):
        cmd = ["make", "-s", "-C", HERE] + (["-B"] if force else [])
        subprocess.run(cmd, check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.fo_f32_to_f16.argtypes = [C.c_float]
        L.fo_f32_to_f16.restype = C.c_uint16
        L.fo_f16_to_f32.argtypes = [C.c_uint16]
        L.fo_f16_to_f32.restype = C.c_float
        L.fo_f32_to_f16_n.argtypes = [_f32p, C.c_size_t, _u16p]
        L.fo_f16_to_f32_n.argtypes = [_u16p, C.c_size_t, _f32p]
        L.fo_argmax_first.argtypes = [_f32p, C.c_size_t]
        L.fo_argmax_first.restype = C.c_size_t
        L.fo_pick_by_mass.argtypes = [_f32p, C.c_size_t, C.c_float]
        L.fo_pick_by_mass.restype = C.c_size_t
        L.fo_q8_0_block.argtypes = [_f32p, C.POINTER(C.c_uint16), _i8p]
        L.fo_q8_0_encode.argtypes = [_f32p, C.c_size_t, _u8p]
        L.fo_q8_0_encode.restype = C.c_int
        L.fo_q8_0_dequant.argtypes = [_u8p, C.c_size_t, C.c_size_t, _f32p]
        L.fo_q8_0_dequant.restype = C.c_int
        L.fo_fake_quantize_q8_0_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t]
        L.fo_fake_quantize_q8_0_cols.argtypes = [_f32p, C.c_size_t, C.c_size_t]
        L.fo_q8_0_to_ferrum_weight.argtypes = [_u8p, C.c_size_t, C.c_size_t, _f32p]
        L.fo_q8_0_to_ferrum_weight.restype = C.c_int
        L.fo_linear_forward.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, C.c_size_t,
                                        C.c_void_p, _f32p, C.c_int]
        L.fo_linear_forward.restype = C.c_int
        L.fo_q8_0_linear_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t, _u8p, C.c_size_t,
                                          C.c_void_p, _f32p]
        L.fo_q8_0_linear_rows.restype = C.c_int
        L.fo_q8_0_quantize_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t, _u16p, _i8p]
        L.fo_q8_0_block_dots.argtypes = [_i8p, C.c_size_t, C.c_size_t, _u8p, C.c_size_t, _i32p]
        L.fo_q8_0_linear_w8a8.argtypes = [_f32p, C.c_size_t, C.c_size_t, _u8p, C.c_size_t,
                                          C.c_void_p, _f32p]
        L.fo_q8_0_linear_w8a8.restype = C.c_int
        L.fo_qweight_row_bytes.argtypes = [C.c_size_t, C.c_int]
        L.fo_qweight_row_bytes.restype = C.c_size_t
        L.fo_qweight_from_f32.argtypes = [_f32p, C.c_size_t, C.c_size_t, C.c_int, _f32p, _u8p]
        L.fo_qweight_to_f32.argtypes = [_f32p, _u8p, C.c_size_t, C.c_size_t, C.c_int, _f32p]
        L.fo_qlinear.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, _u8p, C.c_size_t, C.c_int, _f32p, _f32p,
                                 C.c_int]
        L.fo_qlinear.restype = C.c_int
        L.fo_softmax_rows.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p]
        L.fo_layernorm.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, _f32p, _f32p]
        L.fo_gelu.argtypes = [_f32p, C.c_size_t]
        L.fo_embed_one.argtypes = [_f32p, _f32p] + [C.c_size_t] * 5 + [_f32p]
        L.fo_embed_one.restype = C.c_int
        L.fo_attention_decode.argtypes = [_f32p, _f32p, _f32p] + [C.c_size_t] * 4 + [_f32p]
        L.fo_attention_decode.restype = C.c_int
        L.fo_ln_bridge.argtypes = [_f32p, C.c_size_t, _f32p]
        L.fo_rmsnorm.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, C.c_float, _f32p]
        L.fo_rope.argtypes = [_f32p] + [C.c_size_t] * 4 + [C.c_float, C.c_int, _f32p_or_null, C.c_float]
        L.fo_gqa_attention_decode.argtypes = [_f32p, _f32p, _f32p] + [C.c_size_t] * 5 + [_f32p]
        L.fo_gqa_attention_decode.restype = C.c_int
        L.fo_swiglu.argtypes = [_f32p, _f32p, C.c_size_t, _f32p]
        L.fo_rng_new.argtypes = [C.c_uint64]
        L.fo_rng_new.restype = C.c_uint64
        L.fo_rng_next_u64.argtypes = [C.POINTER(C.c_uint64)]
        L.fo_rng_next_u64.restype = C.c_uint64
        L.fo_rng_next_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.fo_rng_next_f32.restype = C.c_float
        L.fo_draw_to_f32.argtypes = [C.c_uint64]
        L.fo_draw_to_f32.restype = C.c_float
        L.fo_sample.argtypes = [_f32p, C.c_size_t, C.POINTER(SamplingParams), C.c_void_p,
                                C.c_size_t, C.c_uint64, C.POINTER(SampleInfo)]
        L.fo_sample.restype = C.c_uint32
        L.fo_sample_with_params.argtypes = [_f32p, C.c_size_t, C.POINTER(SamplingParams),
                                            C.c_void_p, C.c_size_t, C.POINTER(C.c_uint64),
                                            C.POINTER(SampleInfo)]
        L.fo_sample_with_params.restype = C.c_uint32
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- half codec ------------------------------------------------------------

def f32_to_f16(v: float) -> int:
    return int(lib().fo_f32_to_f16(v))


def f16_to_f32(h: int) -> float:
    return float(lib().fo_f16_to_f32(h))


def f32_to_f16_array(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.zeros(max(x.size, 1), np.uint16)
    lib().fo_f32_to_f16_n(x if x.size else np.zeros(1, np.float32), x.size, out)
    return out[: x.size]


def f16_to_f32_array(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.zeros(max(h.size, 1), np.float32)
    lib().fo_f16_to_f32_n(h if h.size else np.zeros(1, np.uint16), h.size, out)
    return out[: h.size]


# ---- Q8_0 ------------------------------------------------------------------

def q8_0_block(x):
    """quant::q8_0_block -> (d16, int8[32])."""
    x = _f32(x)
    assert x.size == 32
    d16 = C.c_uint16()
    q = np.zeros(32, np.int8)
    lib().fo_q8_0_block(x, C.byref(d16), q)
    return int(d16.value), q


def q8_0_encode(data) -> np.ndarray:
    """gguf_write enc_q8_0: raw GGUF bytes (34 per 32 values)."""
    data = _f32(data).ravel()
    out = np.zeros(max(data.size // 32 * 34, 1), np.uint8)
    if lib().fo_q8_0_encode(data, data.size, out) != 0:
        raise ValueError(f"tensor length {data.size} is not a multiple of block size 32")
    return out[: data.size // 32 * 34]


def q8_0_dequant(raw, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros(max(n, 1), np.float32)
    if lib().fo_q8_0_dequant(raw if raw.size else np.zeros(1, np.uint8), raw.size, n, out) != 0:
        raise ValueError("Q8_0 data shorter than the element count")
    return out[:n]


def fake_quantize_q8_0_rows(data, ne0: int) -> np.ndarray:
    d = _f32(data).copy()
    lib().fo_fake_quantize_q8_0_rows(d, d.size, ne0)
    return d


def fake_quantize_q8_0_cols(data, rows_in: int, cols_out: int) -> np.ndarray:
    d = _f32(data).copy()
    lib().fo_fake_quantize_q8_0_cols(d, rows_in, cols_out)
    return d


def q8_0_to_ferrum_weight(raw, n_rows: int, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    w = np.zeros((k, n_rows), np.float32)
    if lib().fo_q8_0_to_ferrum_weight(raw, n_rows, k, w) != 0:
        raise ValueError("k must be a multiple of 32")
    return w


def quantize_weight(n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Config-2 weights: W [n, k] ~ N(0, std) -> raw GGUF Q8_0 bytes [n rows]."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return q8_0_encode(w).reshape(n, k // 32 * 34)


# ---- linear ----------------------------------------------------------------

def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def linear_forward(x, w_kn, bias=None, threads: int = 1) -> np.ndarray:
    """ops::linear_forward (bias None = ops::matmul): x [m,k] . W [k,n] + b."""
    x = _f32(x)
    w_kn = _f32(w_kn)
    m, k = x.shape
    kb, n = w_kn.shape
    if k != kb:
        raise ValueError(f"linear_forward: input width {k} != weight rows {kb}")
    b = None if bias is None else _f32(bias)
    if b is not None and b.size != n:
        raise ValueError(f"linear_forward: bias length {b.size} != out_features {n}")
    y = np.zeros((m, n), np.float32)
    lib().fo_linear_forward(x, m, k, w_kn, n, _ptr(b), y, int(threads))
    return y


def q8_0_linear(x, raw, n: int, bias=None) -> np.ndarray:
    """Q8_0 Linear as ferrum_core executes it (W8A32), straight from GGUF rows.
    Bit-identical to linear_forward(x, q8_0_to_ferrum_weight(raw), bias)."""
    x = _f32(x)
    m, k = x.shape
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    b = None if bias is None else _f32(bias)
    y = np.zeros((m, n), np.float32)
    if lib().fo_q8_0_linear_rows(x, m, k, raw.ravel(), n, _ptr(b), y) != 0:
        raise ValueError("k must be a multiple of 32")
    return y


def q8_0_quantize_rows(x):
    x = _f32(x)
    m, k = x.shape
    d16 = np.zeros((m, k // 32), np.uint16)
    q = np.zeros((m, k), np.int8)
    lib().fo_q8_0_quantize_rows(x, m, k, d16, q)
    return d16, q


def q8_0_block_dots(qx, raw, n: int) -> np.ndarray:
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    m, k = qx.shape
    dots = np.zeros((m, n, k // 32), np.int32)
    lib().fo_q8_0_block_dots(qx, m, k, np.ascontiguousarray(raw, np.uint8).ravel(), n, dots)
    return dots


def q8_0_linear_w8a8(x, raw, n: int, bias=None) -> np.ndarray:
    x = _f32(x)
    m, k = x.shape
    b = None if bias is None else _f32(bias)
    y = np.zeros((m, n), np.float32)
    lib().fo_q8_0_linear_w8a8(x, m, k, np.ascontiguousarray(raw, np.uint8).ravel(), n, _ptr(b), y)
    return y


# ---- packed per-row int8 / int4 weights (QWeight, ops::qlinear) ------------

INT8, INT4 = 0, 1


class QWeight:
    """quant.rs:130-217: [rows = in_features, cols = out_features], one scale per row."""

    def __init__(self, data, rows: int, cols: int, kind: int):
        data = _f32(np.asarray(data).reshape(rows, cols))
        self.rows, self.cols, self.kind = rows, cols, kind
        self.scales = np.zeros(rows, np.float32)
        self.q = np.zeros(rows * int(lib().fo_qweight_row_bytes(cols, kind)), np.uint8)
        lib().fo_qweight_from_f32(data, rows, cols, kind, self.scales, self.q)

    def row_bytes(self) -> int:
        return int(lib().fo_qweight_row_bytes(self.cols, self.kind))

    def to_f32(self) -> np.ndarray:
        out = np.zeros((self.rows, self.cols), np.float32)
        lib().fo_qweight_to_f32(self.scales, self.q, self.rows, self.cols, self.kind, out)
        return out


def qlinear(x, w: QWeight, bias, threads: int = 1) -> np.ndarray:
    """ops::qlinear (ops.rs:316-377): bias first, then (x * scale) . level, p ascending."""
    x = _f32(np.atleast_2d(x))
    m, k = x.shape
    if k != w.rows:
        raise ValueError(f"qlinear: input width {k} != weight rows {w.rows}")
    b = _f32(bias)
    if b.size != w.cols:
        raise ValueError(f"qlinear: bias length {b.size} != out_features {w.cols}")
    y = np.zeros((m, w.cols), np.float32)
    lib().fo_qlinear(x, m, k, w.scales, w.q, w.cols, w.kind, b, y, int(threads))
    return y


# ---- softmax / ln bridge ---------------------------------------------------

def softmax_rows(z) -> np.ndarray:
    z = _f32(np.atleast_2d(z))
    out = np.zeros_like(z)
    lib().fo_softmax_rows(z, z.shape[0], z.shape[1], out)
    return out


def layernorm(x, gamma, beta) -> np.ndarray:
    """LayerNorm::forward (layer/norm.rs:46-82) over the rows of x."""
    x = _f32(np.atleast_2d(x))
    out = np.zeros_like(x)
    lib().fo_layernorm(x, x.shape[0], x.shape[1], _f32(gamma), _f32(beta), out)
    return out


def gelu(x) -> np.ndarray:
    """activation::gelu (activation.rs:9-12), elementwise."""
    out = _f32(x).copy()
    lib().fo_gelu(out.ravel(), out.size)
    return out


def embed_one(tok_w, pos_w, token: int, pos: int) -> np.ndarray:
    """Embedding::embed_one (layer/embedding.rs:70-90)."""
    tok_w, pos_w = _f32(tok_w), _f32(pos_w)
    d = tok_w.shape[1]
    out = np.zeros(d, np.float32)
    if lib().fo_embed_one(tok_w, pos_w, tok_w.shape[0], pos_w.shape[0], d, token, pos, out) != 0:
        raise ValueError(f"token {token} or position {pos} out of range")
    return out


def attention_decode(qkv, k_cache, v_cache, heads: int, pos: int) -> np.ndarray:
    """The attention of TransformerBlock::forward_with_cache
    (layer/transformer.rs:242-279): appends k, v at row pos of the caches
    (updated in place) and returns the attention output for the new position."""
    d = k_cache.shape[1]
    out = np.zeros(d, np.float32)
    rc = lib().fo_attention_decode(_f32(qkv), k_cache, v_cache, k_cache.shape[0], d, heads, pos, out)
    if rc != 0:
        raise ValueError(f"attention_decode: status {rc}")
    return out


# ---- Llama / Qwen block pieces ---------------------------------------------

ROPE_NORM, ROPE_NEOX = 0, 1


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """RmsNorm::forward_row (llm.rs:58-65) over every row."""
    x = _f32(x)
    w = _f32(w)
    out = np.zeros_like(x)
    dim = x.shape[-1]
    lib().fo_rmsnorm(x, x.size // dim, dim, w, C.c_float(eps), out)
    return out


def rope(x, n_heads: int, head_dim: int, rope_dim: int, pos: int, base: float, rope_type: int,
         freq_factors=None, linear_factor: float = 1.0) -> np.ndarray:
    """apply_rope (llm.rs:146-175) on a copy of x ([n_heads * head_dim])."""
    out = _f32(x).copy()
    ff = None if freq_factors is None else _f32(freq_factors)
    lib().fo_rope(out, n_heads, head_dim, rope_dim, pos, C.c_float(base), rope_type, ff, C.c_float(linear_factor))
    return out


def gqa_attention_decode(qkv, k_cache, v_cache, n_heads: int, n_kv: int, head_dim: int, pos: int) -> np.ndarray:
    """Attention::forward_one's cache append and attend (llm.rs:285-358) for one
    RoPE'd q|k|v row; the caches ([capacity, n_kv*head_dim]) are updated in place."""
    out = np.zeros(n_heads * head_dim, np.float32)
    rc = lib().fo_gqa_attention_decode(_f32(qkv), k_cache, v_cache, k_cache.shape[0], n_heads, n_kv, head_dim, pos,
                                       out)
    if rc != 0:
        raise ValueError(f"gqa_attention_decode: status {rc}")
    return out


def swiglu(g, u) -> np.ndarray:
    """(g / (1 + exp(-g))) * u (llm.rs:415-421)."""
    g, u = _f32(g), _f32(u)
    out = np.zeros_like(g)
    lib().fo_swiglu(g.ravel(), u.ravel(), g.size, out.ravel())
    return out


def ln_bridge(p) -> np.ndarray:
    p = _f32(p)
    out = np.zeros_like(p)
    lib().fo_ln_bridge(p.ravel(), p.size, out.ravel())
    return out


# ---- RNG -------------------------------------------------------------------

class Rng:
    """rng::Rng (xorshift64*)."""

    def __init__(self, seed: int = 0, state: int | None = None):
        self.state = C.c_uint64(lib().fo_rng_new(seed) if state is None else state)

    def next_u64(self) -> int:
        return int(lib().fo_rng_next_u64(C.byref(self.state)))

    def next_f32(self) -> float:
        return float(lib().fo_rng_next_f32(C.byref(self.state)))


def draw_to_f32(draw: int) -> float:
    return float(lib().fo_draw_to_f32(draw))


# ---- sampler ---------------------------------------------------------------

def argmax_first(xs) -> int:
    xs = _f32(xs).ravel()
    return int(lib().fo_argmax_first(xs if xs.size else np.zeros(1, np.float32), xs.size))


def pick_by_mass(probs, r: float) -> int:
    probs = _f32(probs).ravel()
    return int(lib().fo_pick_by_mass(probs if probs.size else np.zeros(1, np.float32), probs.size, r))


def sample(logits, params: SamplingParams, recent=(), draw: int = 0):
    """sample_with_params with an explicit u64 draw -> (id, SampleInfo)."""
    logits = _f32(logits).ravel()
    rec = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32).ravel())
    info = SampleInfo()
    tok = lib().fo_sample(logits, logits.size, C.byref(params),
                          rec.ctypes.data_as(C.c_void_p) if rec.size else None, rec.size,
                          C.c_uint64(draw), C.byref(info))
    return int(tok), info


def sample_with_params(logits, params: SamplingParams, recent, rng: Rng):
    """slm::sampling::sample_with_params: draws from rng as the reference does."""
    logits = _f32(logits).ravel()
    rec = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32).ravel())
    info = SampleInfo()
    tok = lib().fo_sample_with_params(logits, logits.size, C.byref(params),
                                      rec.ctypes.data_as(C.c_void_p) if rec.size else None,
                                      rec.size, C.byref(rng.state), C.byref(info))
    return int(tok)
