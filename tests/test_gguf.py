"""The library's GGUF reader and the GGUF writer (host-only, no GPU): a GPT-2
file in ferrum_core's export layout read back field by field, the reference's
synthetic tensors (gguf/test_support.rs:52-73), an exhaustive F16 decode
check, and the malformed-file errors of gguf/header.rs and gguf/cursor.rs."""
import struct

import numpy as np
import pytest

import gpt2_tiny


@pytest.fixture(scope="module")
def fhm():
    import ferrum_hip

    ferrum_hip.lib()
    return ferrum_hip


@pytest.fixture(scope="module")
def gg():
    import ferrum_gguf

    return ferrum_gguf


def write(tmp_path, data, name="t.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_gpt2_file_reads_back(fhm, gg, orc, tmp_path):
    w = gpt2_tiny.make_weights(orc, seed=3)
    V, D, H, L, F, CTX = gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX
    path = write(tmp_path, gg.gpt2_gguf(w, V, D, H, L, F, CTX).to_bytes())
    with fhm.GGUFFile(path) as g:
        assert g.version == 3
        assert g.meta("general.architecture") == "gpt2"
        assert [g.meta(f"gpt2.{k}") for k in ("context_length", "embedding_length", "block_count",
                                               "feed_forward_length", "attention.head_count")] == [CTX, D, L, F, H]
        assert g.meta("gpt2.attention.layer_norm_epsilon") == pytest.approx(1e-5, rel=1e-7)
        toks, merges, types = g.meta("tokenizer.ggml.tokens"), g.meta("tokenizer.ggml.merges"), \
            g.meta("tokenizer.ggml.token_type")
        assert len(toks) == V and len(merges) == V - 257 and len(types) == V
        assert toks[ord("a")] == "a" and toks[ord(" ")] == "Ġ" and toks[-1] == "<|endoftext|>"
        assert merges[0] == "Ā Ā" and toks[256] == "ĀĀ"
        assert types[:256 + len(merges)] == [1] * (256 + len(merges)) and types[-1] == 3
        assert g.meta("tokenizer.ggml.eos_token_id") == V - 1 and g.meta("tokenizer.ggml.add_bos_token") == 0
        assert g.meta("no.such.key") is None
        dims, ty, nb, _ = g.tensors["token_embd.weight"]
        assert dims == (D, V) and ty == 8 and nb == V * D // 32 * 34
        assert g.raw("token_embd.weight") == np.asarray(w["token_embd_q8"], np.uint8).tobytes()
        assert g.tensors["blk.2.ffn_down.weight"][0] == (F, D)
        assert g.raw("blk.2.ffn_down.weight") == np.asarray(w["blk2.down_q8"], np.uint8).tobytes()
        assert np.array_equal(g.read_f32(None, "position_embd.weight"), w["position_embd"])
        assert np.array_equal(g.read_f32(None, "blk.1.attn_qkv.bias"), w["blk1.qkv_b"])
        assert "output.weight" not in g.tensors  # tied head


def test_reference_synthetic_tensors(fhm, gg, orc, tmp_path):
    """gguf/test_support.rs:52-73: an F32 tensor (i - 16) * 0.25 and a Q8_0
    block with d = 0.5, q = i - 16; their values read back exactly."""
    b = gg.GGUFBuilder()
    b.u32("general.alignment", 32)
    f32_vals = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.25)
    b.tensor("f32", [32], gg.GGML_F32, f32_vals.tobytes())
    q8 = struct.pack("<H", 0x3800) + bytes(((i - 16) & 0xFF) for i in range(32))  # f16(0.5) = 0x3800
    b.tensor("q8", [32], gg.GGML_Q8_0, q8)
    path = write(tmp_path, b.to_bytes())
    with fhm.GGUFFile(path) as g:
        assert np.array_equal(g.read_f32(None, "f32"), f32_vals)
        assert g.raw("q8") == q8
        assert np.array_equal(orc.q8_0_dequant(np.frombuffer(g.raw("q8"), np.uint8), 32),
                              0.5 * (np.arange(32, dtype=np.float32) - 16))


def test_f16_tensor_decodes_every_code_exactly(fhm, gg, tmp_path):
    codes = np.arange(65536, dtype=np.uint16)
    b = gg.GGUFBuilder()
    b.tensor("h", [65536], gg.GGML_F16, codes.tobytes())
    with fhm.GGUFFile(write(tmp_path, b.to_bytes())) as g:
        got = g.read_f32(None, "h")
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_alignment_and_offsets(fhm, gg, tmp_path):
    b = gg.GGUFBuilder(alignment=64)
    b.u32("general.alignment", 64)
    b.tensor("a", [3], gg.GGML_F32, np.array([1, 2, 3], np.float32).tobytes())
    b.tensor("b", [2], gg.GGML_F32, np.array([4, 5], np.float32).tobytes())
    raw = b.to_bytes()
    with fhm.GGUFFile(write(tmp_path, raw)) as g:
        assert list(g.read_f32(None, "b")) == [4.0, 5.0]
    start = raw.index(np.array([1, 2, 3], np.float32).tobytes())
    assert start % 64 == 0 and raw.index(np.array([4, 5], np.float32).tobytes()) == start + 64


def test_repeated_key_keeps_the_last_value_and_first_tensor_wins(fhm, gg, tmp_path):
    b = gg.GGUFBuilder()
    b.u32("k", 1).u32("k", 2)
    raw = bytearray(b.to_bytes())
    with fhm.GGUFFile(write(tmp_path, bytes(raw))) as g:
        assert g.meta("k") == 2


def header(n_tensors=0, n_kv=0, version=3, magic=0x46554747):
    return struct.pack("<IIQQ", magic, version, n_tensors, n_kv)


def kv_u32(key, v):
    return struct.pack("<Q", len(key)) + key.encode() + struct.pack("<II", 4, v)


def tinfo(name, dims, ty, off):
    return (struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims)) +
            b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off))


@pytest.mark.parametrize("data,msg", [
    (b"GGUX" + b"\0" * 40, "bad magic"),
    (header(version=1), "unsupported GGUF version 1"),
    (header(version=4), "unsupported GGUF version 4"),
    (header(n_kv=1)[:-3], "truncated"),
    (header(n_kv=1) + struct.pack("<Q", 1) + b"k" + struct.pack("<II", 9, 9), "nested arrays"),
    (header(n_kv=1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 77), "unknown metadata value type 77"),
    (header(n_kv=1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 4, 10**9), "array count exceeds"),
    (header(n_tensors=1) + tinfo("t", [1] * 9, 0, 0), "implausible 9 dims"),
])
def test_malformed_headers(fhm, tmp_path, data, msg):
    with pytest.raises(fhm.GGUFFormatError, match=msg):
        fhm.GGUFFile(write(tmp_path, data))


def test_tensor_extents(fhm, tmp_path):
    def file(infos, payload):
        body = header(n_tensors=len(infos)) + b"".join(infos)
        body += b"\0" * (-len(body) % 32)
        return body + payload

    with pytest.raises(fhm.GGUFFormatError, match="data runs past EOF"):
        fhm.GGUFFile(write(tmp_path, file([tinfo("t", [16], 0, 0)], b"\0" * 32)))
    with pytest.raises(fhm.GGUFFormatError, match="'a' and 'b' overlap"):
        fhm.GGUFFile(write(tmp_path, file([tinfo("a", [8], 0, 0), tinfo("b", [8], 0, 16)], b"\0" * 64)))
    with fhm.GGUFFile(write(tmp_path, file([tinfo("a", [8], 0, 0), tinfo("b", [8], 0, 32)], b"\0" * 64))) as g:
        assert set(g.tensors) == {"a", "b"}


def test_missing_file_and_wrong_type(fhm, gg, tmp_path):
    with pytest.raises(fhm.FerrumHipError, match="cannot open"):
        fhm.GGUFFile(str(tmp_path / "nope.gguf"))
    b = gg.GGUFBuilder()
    b.tensor("q", [32], gg.GGML_Q8_0, b"\0" * 34)
    with fhm.GGUFFile(write(tmp_path, b.to_bytes())) as g:
        with pytest.raises(fhm.FerrumHipError):
            g.read_f32(None, "q")
