"""GGUF import rules, host side (no GPU): the checks gpt2_from
(loader/gpt2.rs:149-232) and Gguf::load_llama_prec (gguf/llama.rs:51-340)
make before anything is uploaded, with the reference's messages, and the
library's reader pinned on the two GGUF v3 files the reference's own tests
hold (train_transformer/testdata/pre_epoch_rng.ckpt.gguf and
llm_train/testdata/pre_epoch_rng.flck, copied under tests/golden/gguf as data).

The reader's expectations for those files come from the reference's tests
(checkpoint.rs:390-401: vocab 3, context 2, step 3, rng state
3354630805809648812; run.rs:452, 494-496: step 3) and, for the tensor
directory and data, from an independent parse of the published GGUF v3 layout
written here in plain Python."""
import os
import struct

import numpy as np
import pytest

import gpt2_tiny
import llama_tiny

HERE = os.path.dirname(os.path.abspath(__file__))
REF_FILES = {
    "pre_epoch_rng.ckpt.gguf": dict(arch="ferrum-checkpoint", tensors=63, keys=12,
                                    ints={"ferrum.ckpt.vocab": 3, "ferrum.ckpt.context": 2, "ferrum.ckpt.step": 3,
                                          "ferrum.ckpt.rng": 3354630805809648812}),
    "pre_epoch_rng.flck": dict(arch="ferrum-llama-checkpoint", tensors=60, keys=12,
                               ints={"ferrum.ckpt.vocab": 6, "ferrum.ckpt.model_dim": 8, "ferrum.ckpt.layers": 1,
                                     "ferrum.ckpt.heads": 2, "ferrum.ckpt.ffn": 16, "ferrum.ckpt.step": 3}),
}


@pytest.fixture(scope="module")
def fhm():
    import ferrum_hip

    ferrum_hip.lib()
    return ferrum_hip


@pytest.fixture(scope="module")
def gg():
    import ferrum_gguf

    return ferrum_gguf


def write(tmp_path, builder, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(builder.to_bytes())
    return str(p)


# ---- the reference's own files ----------------------------------------------------

def parse_gguf(data: bytes):
    """GGUF v3, straight from the format: magic, version, tensor count, key
    count, the keys, the tensor directory, then the data at the next multiple
    of general.alignment (32 by default)."""
    o = 0

    def rd(fmt):
        nonlocal o
        v = struct.unpack_from("<" + fmt, data, o)
        o += struct.calcsize("<" + fmt)
        return v[0]

    def rstr():
        nonlocal o
        n = rd("Q")
        s = data[o:o + n].decode()
        o += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t == 8:
            return rstr()
        if t == 9:
            et, n = rd("I"), rd("Q")
            return [value(et) for _ in range(n)]
        return rd(scalar[t])

    assert data[:4] == b"GGUF"
    o = 4
    version, n_t, n_kv = rd("I"), rd("Q"), rd("Q")
    kv = {}
    for _ in range(n_kv):
        k = rstr()
        t = rd("I")
        kv[k] = (t, value(t))
    tensors = []
    for _ in range(n_t):
        name = rstr()
        nd = rd("I")
        dims = tuple(rd("Q") for _ in range(nd))
        tensors.append((name, dims, rd("I"), rd("Q")))
    align = kv.get("general.alignment", (4, 32))[1]
    start = (o + align - 1) // align * align
    return version, kv, tensors, start


@pytest.mark.parametrize("fname", sorted(REF_FILES))
def test_reader_on_the_reference_files(fhm, fname):
    want = REF_FILES[fname]
    path = os.path.join(HERE, "golden", "gguf", fname)
    data = open(path, "rb").read()
    version, kv, tensors, start = parse_gguf(data)
    assert (version, len(tensors), len(kv)) == (3, want["tensors"], want["keys"])
    with fhm.GGUFFile(path) as g:
        assert g.version == 3
        assert len(g.tensors) == want["tensors"]
        assert g.meta("general.architecture") == want["arch"]
        for key, v in want["ints"].items():  # the reference's asserted values
            assert g.meta(key) == v, key
        for key, (t, v) in kv.items():  # and every key as the format gives it
            got = g.meta(key)
            if t == 6:
                assert got == pytest.approx(v, rel=0, abs=0) or np.float32(got) == np.float32(v)
            else:
                assert got == v, key
            assert g.meta_kind(key)[0] == t
        for name, dims, ty, off in tensors:
            gd, gt, nb, _ = g.tensors[name]
            assert (tuple(gd), gt) == (dims, ty), name
            assert ty == 0 and nb == 4 * int(np.prod(dims))
            assert g.raw(name) == data[start + off:start + off + nb]
            got = g.read_f32(None, name)
            assert np.array_equal(got.view(np.uint32).ravel(),
                                  np.frombuffer(data, np.uint32, int(np.prod(dims)), start + off))
    # the u64 above 2^63 in the second file survives the reader
    if fname == "pre_epoch_rng.flck":
        with fhm.GGUFFile(path) as g:
            assert g.meta("ferrum.ckpt.rng") == 17830752068367197595


# ---- GPT-2: vocabulary order, epsilon, dims -----------------------------------------

def test_ferrum_vocab_of_a_ferrum_ordered_vocab_is_the_identity(fhm, gg):
    toks, merges, types = gg.synthetic_bpe(600)
    assert fhm.ferrum_vocab(toks, merges, types) == list(range(600))


def test_ferrum_vocab_undoes_a_foreign_order(fhm, gg):
    toks, merges, types = gg.synthetic_bpe(600)
    order = np.random.default_rng(4).permutation(600)  # file position -> ferrum id
    perm = fhm.ferrum_vocab([toks[i] for i in order], merges, [types[i] for i in order])
    # perm[ferrum_id] = file_id: the file token at perm[f] is ferrum token f
    assert [int(order[p]) for p in perm] == list(range(600))


def test_ferrum_vocab_keeps_extra_tokens_in_file_order(fhm, gg):
    toks, merges, types = gg.synthetic_bpe(300)
    extra = ["<a>", "<b>", "<c>"]
    file_toks = extra[:1] + toks[:-1] + extra[1:] + toks[-1:]
    perm = fhm.ferrum_vocab(file_toks, merges, [1] * len(file_toks))
    ordered = [file_toks[i] for i in perm]
    assert ordered[:299] == toks[:299] and ordered[299:] == ["<a>", "<b>", "<c>", toks[-1]]


def test_ferrum_vocab_errors(fhm, gg):
    toks, merges, types = gg.synthetic_bpe(300)
    with pytest.raises(fhm.GGUFFormatError, match="gguf vocab: 300 tokens but 299 token types"):
        fhm.ferrum_vocab(toks, merges, types[:-1])
    missing = [t if t != "a" else "zz" for t in toks]
    with pytest.raises(fhm.GGUFFormatError, match='gguf vocab: no unique token "a"'):
        fhm.ferrum_vocab(missing, merges, types)
    # two merges with one result: the second finds its token taken
    toks2 = toks[:256] + ["ab", "<|endoftext|>"]
    with pytest.raises(fhm.GGUFFormatError) as e:
        fhm.ferrum_vocab(toks2, ["a b", "a b"], [1] * len(toks2))
    assert e.value.msg == 'gguf vocab: no unique token "ab"'
    # Rust's {:?} quoting of a token with a quote and a backslash
    toks3 = toks[:256] + ["<|endoftext|>"]
    with pytest.raises(fhm.GGUFFormatError) as e:
        fhm.ferrum_vocab(toks3, ['" \\'], [1] * len(toks3))
    assert e.value.msg == 'gguf vocab: no unique token "\\"\\\\"'


def tiny_file(gg, orc, tmp_path, **kw):
    w = gpt2_tiny.make_weights(orc, seed=3)
    V, D, H, L, F, CTX = gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX
    return write(tmp_path, gg.gpt2_gguf(w, V, D, H, L, F, CTX, **kw)), w


def test_gpt2_plan_reads_the_hyperparameters(fhm, gg, orc, tmp_path):
    path, _ = tiny_file(gg, orc, tmp_path)
    with fhm.GGUFFile(path) as g:
        cfg, perm, tied = fhm.gpt2_gguf_plan(g)
    assert cfg == dict(vocab=gpt2_tiny.VOCAB, d=gpt2_tiny.D, heads=gpt2_tiny.HEADS, layers=gpt2_tiny.LAYERS,
                       ffn=gpt2_tiny.FFN, context=gpt2_tiny.CTX)
    assert perm == list(range(gpt2_tiny.VOCAB)) and tied


def test_gpt2_plan_finds_a_foreign_order(fhm, gg, orc, tmp_path):
    order = np.random.default_rng(8).permutation(gpt2_tiny.VOCAB)
    path, _ = tiny_file(gg, orc, tmp_path, file_order=order)
    with fhm.GGUFFile(path) as g:
        _, perm, _ = fhm.gpt2_gguf_plan(g)
    assert [int(order[p]) for p in perm] == list(range(gpt2_tiny.VOCAB))


@pytest.mark.parametrize("eps,msg", [
    (1e-3, "gpt2.attention.layer_norm_epsilon is 0.001; Ferrum's LayerNorm uses 0.00001"),
    (1e-6, "gpt2.attention.layer_norm_epsilon is 0.000001; Ferrum's LayerNorm uses 0.00001")])
def test_gpt2_plan_refuses_another_epsilon(fhm, gg, orc, tmp_path, eps, msg):
    path, _ = tiny_file(gg, orc, tmp_path, eps=eps)
    with fhm.GGUFFile(path) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.gpt2_gguf_plan(g)
    assert e.value.msg == msg


def test_gpt2_plan_accepts_an_epsilon_within_1e9(fhm, gg, orc, tmp_path):
    path, _ = tiny_file(gg, orc, tmp_path, eps=1e-5 + 5e-10)
    with fhm.GGUFFile(path) as g:
        fhm.gpt2_gguf_plan(g)


def test_gpt2_plan_errors(fhm, gg, orc, tmp_path):
    D, H, L, F, CTX = gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX
    # missing epsilon key
    b2 = gg.GGUFBuilder()
    b2.str("general.architecture", "gpt2")
    for k, v in (("context_length", CTX), ("embedding_length", D), ("block_count", L), ("feed_forward_length", F),
                 ("attention.head_count", H)):
        b2.u32(f"gpt2.{k}", v)
    with fhm.GGUFFile(write(tmp_path, b2, "noeps.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.gpt2_gguf_plan(g)
    assert e.value.msg == "GGUF key 'gpt2.attention.layer_norm_epsilon' missing or not a number"
    b3 = gg.GGUFBuilder()
    b3.str("general.architecture", "gpt2")
    with fhm.GGUFFile(write(tmp_path, b3, "nokeys.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.gpt2_gguf_plan(g)
    assert e.value.msg == "GGUF key 'gpt2.context_length' missing or not an integer"
    b4 = gg.GGUFBuilder()
    b4.str("general.architecture", "llama")
    with fhm.GGUFFile(write(tmp_path, b4, "llama.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.gpt2_gguf_plan(g)
    assert e.value.msg == 'not a GPT-2 model: architecture Some("llama") (need gpt2)'


def test_gpt2_plan_checks_tensor_dims(fhm, gg, orc, tmp_path):
    w = gpt2_tiny.make_weights(orc, seed=3)
    V, D, H, L, F, CTX = gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX
    # a file claiming a wider feed-forward than its tensors hold
    path = write(tmp_path, gg.gpt2_gguf(w, V, D, H, L, F, CTX))
    data = bytearray(open(path, "rb").read())
    key = b"gpt2.feed_forward_length"
    i = data.index(key) + len(key) + 4  # past the value type
    struct.pack_into("<I", data, i, F + 32)
    p2 = tmp_path / "wide.gguf"
    p2.write_bytes(bytes(data))
    with fhm.GGUFFile(str(p2)) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.gpt2_gguf_plan(g)
    assert e.value.msg == f"tensor 'blk.0.ffn_up.weight' has dims [{D}, {F}], expected [{D}, {F + 32}]"


# ---- Llama / Qwen2 ------------------------------------------------------------------

def llama_file(gg, orc, tmp_path, name="QWEN", arch="qwen2", biases=True, tied=True, extra=None, f32_names=(),
               fname="l.gguf"):
    cfg = getattr(llama_tiny, name)
    w = llama_tiny.make_weights(orc, cfg, 21, biases, tied)
    return write(tmp_path, gg.llama_gguf(w, cfg, arch, f32_names, extra), fname), w, cfg


def test_llama_plan_reads_a_qwen2_file(fhm, gg, orc, tmp_path):
    path, _, c = llama_file(gg, orc, tmp_path)
    with fhm.GGUFFile(path) as g:
        cfg, mats, tied = fhm.llama_gguf_plan(g)
    assert tied and cfg["arch"] == "qwen2" and cfg["rope_type"] == fhm.ROPE_NEOX
    for k in ("vocab", "d", "n_heads", "n_kv", "head_dim", "layers", "ffn", "context"):
        assert cfg[k] == c[k], k
    assert cfg["eps"] == np.float32(c["eps"]) and cfg["rope_base"] == np.float32(c["rope_base"])
    assert cfg["rope_linear"] == 1.0 and not cfg["rope_freqs"]
    assert mats["blk.1.attn_k.weight"] == (c["n_kv"] * c["head_dim"], c["d"])


def test_llama_plan_reads_a_llama_file(fhm, gg, orc, tmp_path):
    path, _, c = llama_file(gg, orc, tmp_path, "LLAMA", "llama", False, False)
    with fhm.GGUFFile(path) as g:
        cfg, mats, tied = fhm.llama_gguf_plan(g)
    assert not tied and cfg["rope_type"] == fhm.ROPE_NORM and cfg["rope_dim"] == c["rope_dim"]
    assert mats["output.weight"] == (c["vocab"], c["d"])


def test_llama_plan_defaults(fhm, gg, tmp_path):
    """Absent keys take the reference's defaults: head_count_kv = head_count,
    key_length = d / heads, rope dims = head dim, freq_base 10000, eps 1e-5,
    context 2048."""
    b = gg.GGUFBuilder()
    b.str("general.architecture", "llama")
    for k, v in (("embedding_length", 64), ("block_count", 0), ("attention.head_count", 4),
                 ("feed_forward_length", 96)):
        b.u32(f"llama.{k}", v)
    b.tensor("token_embd.weight", [64, 10], gg.GGML_F32, np.zeros(640, np.float32).tobytes())
    b.tensor("output_norm.weight", [64], gg.GGML_F32, np.ones(64, np.float32).tobytes())
    with fhm.GGUFFile(write(tmp_path, b)) as g:
        cfg, _, tied = fhm.llama_gguf_plan(g)
    assert (cfg["n_kv"], cfg["head_dim"], cfg["rope_dim"], cfg["rope_base"], cfg["context"]) == (4, 16, 16, 1e4, 2048)
    assert cfg["eps"] == np.float32(1e-5) and tied and cfg["vocab"] == 10


def with_meta(*pairs):
    def extra(b):
        for kind, key, value in pairs:
            getattr(b, kind)(key, value)
    return extra


@pytest.mark.parametrize("pairs,msg", [
    ((("str", "qwen2.rope.scaling.type", "yarn"),),
     "RoPE scaling type 'yarn' is not supported: Ferrum implements none, linear and rope_freqs.weight "
     "(yarn and longrope are refused)"),
    ((("str", "qwen2.rope.scaling.type", "none"), ("f32", "qwen2.rope.scaling.factor", 2.0)),
     "'qwen2.rope.scaling.type' is \"none\" but the scaling factor is 2"),
    ((("f32", "qwen2.rope.scaling.attn_factor", 0.5),),
     "RoPE scaling attn_factor 0.5 is not supported (only 1.0)"),
    ((("u32", "qwen2.rope.scaling.type", 3),), "'qwen2.rope.scaling.type' is not a string"),
])
def test_llama_plan_rope_scaling_errors(fhm, gg, orc, tmp_path, pairs, msg):
    path, _, _ = llama_file(gg, orc, tmp_path, extra=with_meta(*pairs))
    with fhm.GGUFFile(path) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == msg


@pytest.mark.parametrize("pairs,factor", [
    ((("str", "qwen2.rope.scaling.type", "linear"), ("f32", "qwen2.rope.scaling.factor", 4.0)), 4.0),
    ((("f32", "qwen2.rope.scale_linear", 2.0),), 2.0),            # legacy key, no type: linear
    ((("f32", "qwen2.rope.scaling.factor", 0.0),), 1.0),          # factor 0: no scaling
    ((("str", "qwen2.rope.scaling.type", "none"),), 1.0)])
def test_llama_plan_rope_scaling_factors(fhm, gg, orc, tmp_path, pairs, factor):
    path, _, _ = llama_file(gg, orc, tmp_path, extra=with_meta(*pairs))
    with fhm.GGUFFile(path) as g:
        cfg, _, _ = fhm.llama_gguf_plan(g)
    assert cfg["rope_linear"] == factor


def test_llama_plan_rope_freqs_dims(fhm, gg, orc, tmp_path):
    c = llama_tiny.QWEN
    good = lambda b: b.tensor("rope_freqs.weight", [c["head_dim"] // 2], gg.GGML_F32,  # noqa: E731
                              np.ones(c["head_dim"] // 2, np.float32).tobytes())
    path, _, _ = llama_file(gg, orc, tmp_path, extra=good)
    with fhm.GGUFFile(path) as g:
        assert fhm.llama_gguf_plan(g)[0]["rope_freqs"]
    bad = lambda b: b.tensor("rope_freqs.weight", [5], gg.GGML_F32, np.ones(5, np.float32).tobytes())  # noqa: E731
    path, _, _ = llama_file(gg, orc, tmp_path, extra=bad, fname="bad.gguf")
    with fhm.GGUFFile(path) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == f"rope_freqs.weight has dims [5], expected [{c['head_dim'] // 2}] (rope_dim / 2)"


def test_llama_plan_refuses_biases_outside_qkv(fhm, gg, orc, tmp_path):
    c = llama_tiny.QWEN
    extra = lambda b: b.tensor("blk.1.ffn_up.bias", [c["ffn"]], gg.GGML_F32,  # noqa: E731
                               np.zeros(c["ffn"], np.float32).tobytes())
    path, _, _ = llama_file(gg, orc, tmp_path, extra=extra)
    with fhm.GGUFFile(path) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == ("GGUF tensor 'blk.1.ffn_up.bias' is not supported: Ferrum loads biases only for "
                           "attn_q/attn_k/attn_v")
    extra = lambda b: b.tensor("output.bias", [c["vocab"]], gg.GGML_F32,  # noqa: E731
                               np.zeros(c["vocab"], np.float32).tobytes())
    path, _, _ = llama_file(gg, orc, tmp_path, extra=extra, fname="ob.gguf")
    with fhm.GGUFFile(path) as g, pytest.raises(fhm.GGUFFormatError, match="'output.bias' is not supported"):
        fhm.llama_gguf_plan(g)


def test_llama_plan_other_errors(fhm, gg, orc, tmp_path):
    b = gg.GGUFBuilder()
    b.str("general.architecture", "mistral")
    with fhm.GGUFFile(write(tmp_path, b, "a.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == "architecture 'mistral' is not supported by load_llama (llama / qwen2 only)"
    b = gg.GGUFBuilder()
    b.u32("llama.embedding_length", 8)
    with fhm.GGUFFile(write(tmp_path, b, "b.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == "GGUF missing general.architecture"
    b = gg.GGUFBuilder()
    b.str("general.architecture", "llama").u32("llama.embedding_length", 8).u32("llama.block_count", 1000)
    with fhm.GGUFFile(write(tmp_path, b, "c.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == "GGUF block_count = 1000 exceeds what the file can hold (0)"
    b = gg.GGUFBuilder()
    b.str("general.architecture", "llama")
    for k, v in (("embedding_length", 64), ("block_count", 0), ("attention.head_count", 4),
                 ("feed_forward_length", 96)):
        b.u32(f"llama.{k}", v)
    b.tensor("token_embd.weight", [32, 10], gg.GGML_F32, np.zeros(320, np.float32).tobytes())
    with fhm.GGUFFile(write(tmp_path, b, "d.gguf")) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == "token_embd.weight size does not match vocab × dim"
    c = llama_tiny.QWEN
    path, w, _ = llama_file(gg, orc, tmp_path, fname="e.gguf")
    data = bytearray(open(path, "rb").read())
    key = b"qwen2.feed_forward_length"
    i = data.index(key) + len(key) + 4
    struct.pack_into("<I", data, i, c["ffn"] + 32)
    p2 = tmp_path / "f.gguf"
    p2.write_bytes(bytes(data))
    with fhm.GGUFFile(str(p2)) as g, pytest.raises(fhm.GGUFFormatError) as e:
        fhm.llama_gguf_plan(g)
    assert e.value.msg == (f"tensor 'blk.0.ffn_gate.weight' has dims [{c['d']}, {c['ffn']}], expected "
                           f"[{c['d']}, {c['ffn'] + 32}] from the metadata")


def test_interleave_gate_up_layout(fhm):
    """The gate|up weight ACT_SWIGLU32 reads: rows 64g .. 64g + 31 are gate rows
    32g .. 32g + 31 and the next 32 the up rows of the same outputs, each row's
    bytes (a Q8_0 row, or one bias value) kept whole."""
    rows, width = 96, 34 * 4
    gate = np.arange(rows * width, dtype=np.int64).reshape(rows, width)
    up = -gate - 1
    out = fhm.interleave_gate_up(gate.ravel(), up.ravel(), rows).reshape(2 * rows, width)
    for g in range(rows // 32):
        assert np.array_equal(out[64 * g:64 * g + 32], gate[32 * g:32 * g + 32])
        assert np.array_equal(out[64 * g + 32:64 * g + 64], up[32 * g:32 * g + 32])
    bias = fhm.interleave_gate_up(np.arange(rows), np.arange(rows) + 1000, rows)
    assert bias.tolist()[:64] == list(range(32)) + list(range(1000, 1032))
