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


def gpt2_gguf(weights: dict, vocab: int, d: int, heads: int, layers: int, ffn: int, ctx: int,
              eps: float = 1e-5, name: str = "synthetic") -> GGUFBuilder:
    """GgufOut::gpt2's layout (loader/gpt2.rs:61-146, loader/encode.rs:60-93)
    from Q8_0 bytes and f32 arrays keyed as tests/gpt2_tiny.make_weights makes
    them: token_embd_q8 [vocab rows of d], position_embd [ctx, d], per block
    ln1/ln2 gamma and beta, qkv_q8 [3d rows] + qkv_b, out_q8 [d rows] + out_b,
    up_q8 [ffn rows] + up_b, down_q8 [d rows of ffn] + down_b; lnf_g / lnf_b.
    The head is tied (no output.weight)."""
    tokens, merges, types = synthetic_bpe(vocab)
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
    b.tensor("token_embd.weight", [d, vocab], GGML_Q8_0, q8(weights["token_embd_q8"]))
    b.tensor("position_embd.weight", [d, ctx], GGML_F32, f32(weights["position_embd"]))
    for i in range(layers):
        w = lambda k: weights[f"blk{i}.{k}"]  # noqa: E731
        n = lambda s: f"blk.{i}.{s}"  # noqa: E731
        b.tensor(n("attn_norm.weight"), [d], GGML_F32, f32(w("ln1_g")))
        b.tensor(n("attn_norm.bias"), [d], GGML_F32, f32(w("ln1_b")))
        b.tensor(n("attn_qkv.weight"), [d, 3 * d], GGML_Q8_0, q8(w("qkv_q8")))
        b.tensor(n("attn_qkv.bias"), [3 * d], GGML_F32, f32(w("qkv_b")))
        b.tensor(n("attn_output.weight"), [d, d], GGML_Q8_0, q8(w("out_q8")))
        b.tensor(n("attn_output.bias"), [d], GGML_F32, f32(w("out_b")))
        b.tensor(n("ffn_norm.weight"), [d], GGML_F32, f32(w("ln2_g")))
        b.tensor(n("ffn_norm.bias"), [d], GGML_F32, f32(w("ln2_b")))
        b.tensor(n("ffn_up.weight"), [d, ffn], GGML_Q8_0, q8(w("up_q8")))
        b.tensor(n("ffn_up.bias"), [ffn], GGML_F32, f32(w("up_b")))
        b.tensor(n("ffn_down.weight"), [ffn, d], GGML_Q8_0, q8(w("down_q8")))
        b.tensor(n("ffn_down.bias"), [d], GGML_F32, f32(w("down_b")))
    b.tensor("output_norm.weight", [d], GGML_F32, f32(weights["lnf_g"]))
    b.tensor("output_norm.bias", [d], GGML_F32, f32(weights["lnf_b"]))
    return b
