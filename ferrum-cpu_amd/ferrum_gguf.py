"""GGUF writing for ferrum_hip: a GGUF v3 builder (gguf_write/builder.rs:26-121)
and the GPT-2 export layout of ferrum_core's GgufOut::gpt2
(loader/gpt2.rs:61-146) with a byte-level BPE tokenizer table in ferrum's
order (tokenizer/gguf_io.rs: 256 byte tokens, one token per merge in rank
order, then control tokens).  Host-side file writing only; reading goes
through the library's native reader (ferrum_hip.GGUFFile)."""
import struct

import numpy as np

GGUF_MAGIC = 0x46554747
ALIGNMENT = 32
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STRING, VT_ARRAY, VT_U64, VT_I64, VT_F64 = range(13)
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
TOK_EOS = "<|endoftext|>"
_NUM = {VT_U8: "<B", VT_I8: "<b", VT_U16: "<H", VT_I16: "<h", VT_U32: "<I", VT_I32: "<i", VT_F32: "<f",
        VT_BOOL: "<B", VT_U64: "<Q", VT_I64: "<q", VT_F64: "<d"}


def _str(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == VT_STRING:
        return _str(v)
    if vtype == VT_ARRAY:
        elem, items = v
        out = struct.pack("<IQ", elem, len(items))
        if elem == VT_STRING:
            return out + b"".join(_str(x) for x in items)
        return out + np.asarray(items, dtype=np.dtype(_NUM[elem][1:]).newbyteorder("<")).tobytes()
    return struct.pack(_NUM[vtype], v)


class GGUFBuilder:
    """Metadata in insertion order, tensors at 32-byte-aligned offsets of the
    data section, which starts at the next multiple of 32 after the directory."""

    def __init__(self, alignment: int = ALIGNMENT):
        self.meta, self.tensors, self.alignment = [], [], alignment

    def kv(self, key: str, vtype: int, value):
        self.meta.append((key, vtype, value))
        return self

    def u32(self, key, v):
        return self.kv(key, VT_U32, int(v))

    def f32(self, key, v):
        return self.kv(key, VT_F32, float(v))

    def str(self, key, v):
        return self.kv(key, VT_STRING, v)

    def bool(self, key, v):
        return self.kv(key, VT_BOOL, 1 if v else 0)

    def tensor(self, name: str, dims, ggml_type: int, data: bytes):
        if any(t[0] == name for t in self.tensors):
            raise ValueError(f"GGUFBuilder: duplicate tensor name '{name}'")
        self.tensors.append((name, [int(d) for d in dims], ggml_type, bytes(data)))
        return self

    def to_bytes(self) -> bytes:
        a = self.alignment
        up = lambda x: (x + a - 1) // a * a  # noqa: E731
        out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.meta)))
        for key, vtype, value in self.meta:
            out += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        offsets, running = [], 0
        for _, _, _, data in self.tensors:
            off = up(running)
            offsets.append(off)
            running = off + len(data)
        for (name, dims, ty, _), off in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", ty, off)
        start = up(len(out))
        out += b"\0" * (start - len(out))
        for (_, _, _, data), off in zip(self.tensors, offsets):
            out += b"\0" * (start + off - len(out))
            out += data
        return bytes(out)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.to_bytes())


def byte_to_unicode():
    """GPT-2's byte <-> printable-character table: printable Latin-1 bytes map
    to themselves, the other 68 to U+0100 onwards in byte order."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    table, extra = {}, 0
    for b in range(256):
        if b in keep:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + extra)
            extra += 1
    return table


def synthetic_bpe(vocab: int):
    """A byte-level BPE vocabulary of `vocab` tokens in ferrum's order: the 256
    byte tokens, vocab - 257 merges (pairs of byte tokens, each a new token),
    and the end-of-text control token.  Returns (tokens, merges, token_types)."""
    n_merges = vocab - 257
    if not 0 <= n_merges <= 256 * 256:
        raise ValueError(f"synthetic_bpe: vocab {vocab} outside 257 .. 65793")
    b2u = byte_to_unicode()
    base = [b2u[b] for b in range(256)]
    merges = [f"{base[i // 256]} {base[i % 256]}" for i in range(n_merges)]
    tokens = base + [m.replace(" ", "", 1) for m in merges] + [TOK_EOS]
    types = [1] * (256 + n_merges) + [3]
    return tokens, merges, types


def q8_0_rows_to_f32(raw, n_rows: int, k: int) -> np.ndarray:
    """GGUF Q8_0 bytes [n_rows of k] expanded to f32 [n_rows, k] (exact: an f16
    scale times an 8-bit integer)."""
    blk = np.asarray(raw, np.uint8).reshape(-1, 34)
    sc = blk[:, :2].copy().view(np.float16).astype(np.float32)
    return (sc * blk[:, 2:].copy().view(np.int8).astype(np.float32)).reshape(n_rows, k)


def gpt2_gguf(weights: dict, vocab: int, d: int, heads: int, layers: int, ffn: int, ctx: int,
              eps: float = 1e-5, name: str = "synthetic", file_order=None, output=None) -> GGUFBuilder:
    """GgufOut::gpt2's layout (loader/gpt2.rs:61-146, loader/encode.rs:60-93)
    from Q8_0 bytes and f32 arrays keyed as tests/gpt2_tiny.make_weights makes
    them: token_embd_q8 [vocab rows of d], position_embd [ctx, d], per block
    ln1/ln2 gamma and beta, qkv_q8 [3d rows] + qkv_b, out_q8 [d rows] + out_b,
    up_q8 [ffn rows] + up_b, down_q8 [d rows of ffn] + down_b; lnf_g / lnf_b.
    A matrix may instead be given as f32 rows under the same name with _f32
    for _q8 (token_embd_f32, blk{i}.qkv_f32, ...): it is written as F32, as the
    reference's writer stores a matrix whose ne0 is not a multiple of 32
    (loader/mod.rs:147-152).  The head is tied (no output.weight) unless
    `output` (Q8_0 bytes of [vocab rows of d]) is given.

    file_order (a permutation of the vocabulary, ferrum ids in file order)
    writes the tokens, their types and the token-table (and output) rows in
    that order instead of ferrum's -- a foreign GPT-2 vocab, as a llama.cpp
    conversion orders it."""
    tokens, merges, types = synthetic_bpe(vocab)
    order = list(range(vocab)) if file_order is None else [int(i) for i in file_order]
    if sorted(order) != list(range(vocab)):
        raise ValueError("file_order must be a permutation of the vocabulary")
    tokens, types = [tokens[i] for i in order], [types[i] for i in order]
    b = GGUFBuilder()
    b.str("general.architecture", "gpt2").str("general.name", name)
    for k, v in (("context_length", ctx), ("embedding_length", d), ("block_count", layers),
                 ("feed_forward_length", ffn), ("attention.head_count", heads)):
        b.u32(f"gpt2.{k}", v)
    b.f32("gpt2.attention.layer_norm_epsilon", eps)
    b.str("tokenizer.ggml.model", "gpt2").str("tokenizer.ggml.pre", "gpt-2")
    b.kv("tokenizer.ggml.tokens", VT_ARRAY, (VT_STRING, tokens))
    b.kv("tokenizer.ggml.merges", VT_ARRAY, (VT_STRING, merges))
    b.kv("tokenizer.ggml.token_type", VT_ARRAY, (VT_I32, types))
    eos = vocab - 1
    b.u32("tokenizer.ggml.bos_token_id", eos).u32("tokenizer.ggml.eos_token_id", eos)
    b.bool("tokenizer.ggml.add_bos_token", False).bool("tokenizer.ggml.add_eos_token", False)
    b.u32("general.file_type", 7).u32("general.quantization_version", 2)
    f32 = lambda a: np.ascontiguousarray(a, np.float32).tobytes()  # noqa: E731
    q8 = lambda a: np.asarray(a, np.uint8).tobytes()  # noqa: E731

    def matrix(tname, key, rows, ne0, perm=None):
        """A [rows x ne0] matrix, Q8_0 from key_q8 or F32 from key_f32, rows
        optionally reordered."""
        if key + "_f32" in weights:
            a = np.asarray(weights[key + "_f32"], np.float32).reshape(rows, ne0)
            b.tensor(tname, [ne0, rows], GGML_F32, f32(a if perm is None else a[perm]))
        else:
            a = np.asarray(weights[key + "_q8"], np.uint8).reshape(rows, -1)
            b.tensor(tname, [ne0, rows], GGML_Q8_0, q8(a if perm is None else a[perm]))

    matrix("token_embd.weight", "token_embd", vocab, d, order)
    if output is not None:
        b.tensor("output.weight", [d, vocab], GGML_Q8_0, q8(np.asarray(output, np.uint8).reshape(vocab, -1)[order]))
    b.tensor("position_embd.weight", [d, ctx], GGML_F32, f32(weights["position_embd"]))
    for i in range(layers):
        w = lambda k: weights[f"blk{i}.{k}"]  # noqa: E731
        n = lambda s: f"blk.{i}.{s}"  # noqa: E731
        b.tensor(n("attn_norm.weight"), [d], GGML_F32, f32(w("ln1_g")))
        b.tensor(n("attn_norm.bias"), [d], GGML_F32, f32(w("ln1_b")))
        matrix(n("attn_qkv.weight"), f"blk{i}.qkv", 3 * d, d)
        b.tensor(n("attn_qkv.bias"), [3 * d], GGML_F32, f32(w("qkv_b")))
        matrix(n("attn_output.weight"), f"blk{i}.out", d, d)
        b.tensor(n("attn_output.bias"), [d], GGML_F32, f32(w("out_b")))
        b.tensor(n("ffn_norm.weight"), [d], GGML_F32, f32(w("ln2_g")))
        b.tensor(n("ffn_norm.bias"), [d], GGML_F32, f32(w("ln2_b")))
        matrix(n("ffn_up.weight"), f"blk{i}.up", ffn, d)
        b.tensor(n("ffn_up.bias"), [ffn], GGML_F32, f32(w("up_b")))
        matrix(n("ffn_down.weight"), f"blk{i}.down", d, ffn)
        b.tensor(n("ffn_down.bias"), [d], GGML_F32, f32(w("down_b")))
    b.tensor("output_norm.weight", [d], GGML_F32, f32(weights["lnf_g"]))
    b.tensor("output_norm.bias", [d], GGML_F32, f32(weights["lnf_b"]))
    return b


def llama_gguf(weights: dict, cfg: dict, arch: str = "qwen2", f32_names=(), extra=None) -> GGUFBuilder:
    """A llama.cpp-layout llama / qwen2 GGUF (the keys and tensor names
    Gguf::load_llama_prec reads, gguf/llama.rs:171-340) from a weights dict
    keyed as LlamaDevice.from_weights takes it (token_embd, optional output,
    output_norm, blk.i.attn_norm / attn_q / attn_k / attn_v (+ .bias) /
    attn_output / ffn_norm / ffn_gate / ffn_up / ffn_down; matrices as Q8_0
    bytes) and its cfg.  Matrices named in f32_names (dict keys) are written
    as F32 (their Q8_0 rows expanded exactly).  extra(builder) adds further
    metadata or tensors (rope scaling keys, rope_freqs.weight)."""
    d, nh, nkv, hd, L, ffn = cfg["d"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["layers"], cfg["ffn"]
    qd, kvd, V = nh * hd, nkv * hd, cfg["vocab"]
    b = GGUFBuilder()
    b.str("general.architecture", arch).str("general.name", "synthetic")
    for k, v in (("embedding_length", d), ("block_count", L), ("attention.head_count", nh),
                 ("attention.head_count_kv", nkv), ("feed_forward_length", ffn), ("context_length", cfg["context"]),
                 ("attention.key_length", hd), ("rope.dimension_count", cfg.get("rope_dim", hd))):
        b.u32(f"{arch}.{k}", v)
    b.f32(f"{arch}.rope.freq_base", cfg["rope_base"])
    b.f32(f"{arch}.attention.layer_norm_rms_epsilon", cfg["eps"])
    f32 = lambda a: np.ascontiguousarray(a, np.float32).tobytes()  # noqa: E731

    def mat(tname, key, rows, ne0):
        raw = np.asarray(weights[key], np.uint8)
        if key in f32_names:
            b.tensor(tname, [ne0, rows], GGML_F32, f32(q8_0_rows_to_f32(raw, rows, ne0)))
        else:
            b.tensor(tname, [ne0, rows], GGML_Q8_0, raw.tobytes())

    mat("token_embd.weight", "token_embd", V, d)
    if "output" in weights:
        mat("output.weight", "output", V, d)
    b.tensor("output_norm.weight", [d], GGML_F32, f32(weights["output_norm"]))
    for i in range(L):
        p = f"blk.{i}."
        b.tensor(p + "attn_norm.weight", [d], GGML_F32, f32(weights[p + "attn_norm"]))
        for s, n in (("q", qd), ("k", kvd), ("v", kvd)):
            mat(p + f"attn_{s}.weight", p + f"attn_{s}", n, d)
            if p + f"attn_{s}.bias" in weights:
                b.tensor(p + f"attn_{s}.bias", [n], GGML_F32, f32(weights[p + f"attn_{s}.bias"]))
        mat(p + "attn_output.weight", p + "attn_output", d, qd)
        b.tensor(p + "ffn_norm.weight", [d], GGML_F32, f32(weights[p + "ffn_norm"]))
        mat(p + "ffn_gate.weight", p + "ffn_gate", ffn, d)
        mat(p + "ffn_up.weight", p + "ffn_up", ffn, d)
        mat(p + "ffn_down.weight", p + "ffn_down", d, ffn)
    if extra is not None:
        extra(b)
    return b
