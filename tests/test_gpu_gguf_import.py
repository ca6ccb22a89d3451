"""GGUF import on the device: F32 weights (the matrices the reference stores
as F32), GPT-2 files in a foreign vocabulary order, and llama / qwen2 files
(Gguf::load_llama_prec), each against the model built from the same arrays or
against the CPU oracle."""
import numpy as np
import pytest

import gpt2_tiny
import llama_tiny

pytestmark = pytest.mark.gpu


def bits_equal(got, want):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} of {same.size} differ; first at {np.argwhere(~same)[0].tolist()}"


def close(got, want, atol):
    np.testing.assert_allclose(np.asarray(got, np.float64), np.asarray(want, np.float64), rtol=0, atol=atol)


# ---- F32 weights ----------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 70, 48), (3, 130, 100), (2, 33, 7), (1, 2000, 768), (5, 50, 1),
                                   (4, 300, 333)])
def test_f32_weight_linear_is_the_reference_bit_for_bit(fh, orc, m, n, k):
    import ferrum_hip

    rng = np.random.default_rng(m * 100 + n + k)
    w = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    wt = ferrum_hip.Q8_0Weight.upload_f32(fh, w)
    assert wt.is_f32 and wt.dims() == (n, k)
    want = orc.linear_forward(x, np.ascontiguousarray(w.T), b)
    for numerics in (ferrum_hip.W8A32, ferrum_hip.W8A32_EXACT):
        bits_equal(ferrum_hip.linear_forward(fh, x, wt, b, numerics=numerics), want)
    bits_equal(ferrum_hip.matmul(fh, x, wt), orc.linear_forward(x, np.ascontiguousarray(w.T), None))
    wt.free()


def test_f32_weight_fused_forms_equal_their_parts(fh, orc):
    """linear + GELU and LayerNorm + linear on an F32 weight: the same bits as
    the separate device ops."""
    import torch

    import ferrum_hip

    m, n, k = 3, 200, 48
    rng = np.random.default_rng(2)
    w = ferrum_hip.Q8_0Weight.upload_f32(fh, (rng.standard_normal((n, k)) * 0.2).astype(np.float32))
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    r = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(k)).astype(np.float32)).cuda()
    be = torch.from_numpy((0.1 * rng.standard_normal(k)).astype(np.float32)).cuda()
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    y1, y2 = torch.empty((m, n), device="cuda"), torch.empty((m, n), device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.linear_act_async(fh, w, x, m, k, bias, n, y1, ferrum_hip.ACT_GELU)
    ferrum_hip.linear_forward_async(fh, w, x, m, k, bias, n, y2)
    ferrum_hip.gelu_async(fh, y2, m * n)
    fh.sync()
    bits_equal(y1.cpu().numpy(), y2.cpu().numpy())
    h, s1, xs = torch.empty((m, k), device="cuda"), torch.empty((m, k), device="cuda"), x.clone()
    torch.cuda.synchronize()
    ferrum_hip.linear_ln_async(fh, w, x, r, s1, m, k, g, be, bias, n, y1)
    ferrum_hip.add_layernorm_async(fh, xs, r, m, k, g, be, h)
    fh.sync()
    ferrum_hip.linear_forward_async(fh, w, h, m, k, bias, n, y2)
    fh.sync()
    bits_equal(y1.cpu().numpy(), y2.cpu().numpy())
    bits_equal(s1.cpu().numpy(), xs.cpu().numpy())
    w.free()


def test_f32_weight_refusals(fh):
    import torch

    import ferrum_hip

    w = ferrum_hip.Q8_0Weight.upload_f32(fh, np.ones((64, 64), np.float32))
    x = np.ones((1, 64), np.float32)
    with pytest.raises(ferrum_hip.FerrumHipError, match="FH_W8A8 needs a Q8_0 weight"):
        ferrum_hip.linear_forward(fh, x, w, None, numerics=ferrum_hip.W8A8)
    with pytest.raises(ferrum_hip.FerrumHipError, match="the weight is F32"):
        w.download()
    dx, dy = torch.ones((1, 64), device="cuda"), torch.empty((1, 64), device="cuda")
    rc = ferrum_hip.lib().fh_q8_0_linear_noalloc_async(fh.h, w.h, dx.data_ptr(), 1, 64, None, 0, dy.data_ptr(),
                                                       ferrum_hip.W8A32)
    assert rc == ferrum_hip.FH_ERR_LIMIT
    w.free()


# ---- GPT-2 files ------------------------------------------------------------------------

def gpt2_file(tmp_path, w, name, **kw):
    import ferrum_gguf

    path = str(tmp_path / name)
    ferrum_gguf.gpt2_gguf(w, gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN,
                          gpt2_tiny.CTX, **kw).write(path)
    return path


@pytest.mark.parametrize("untied", [False, True])
def test_gpt2_foreign_vocab_order_loads_as_ferrum_order(fh, orc, tmp_path, untied):
    """The same model written with its vocabulary in ferrum's order and in a
    shuffled (foreign) order: loading undoes the shuffle (ferrum_vocab +
    permute_rows on the token table and an untied output.weight), so the
    same ids give the same scores, bit for bit."""
    import ferrum_hip

    w = gpt2_tiny.make_weights(orc, seed=12)
    out = orc.q8_0_encode((np.random.default_rng(3).standard_normal(gpt2_tiny.VOCAB * gpt2_tiny.D) * 0.1)
                          .astype(np.float32)) if untied else None
    order = np.random.default_rng(99).permutation(gpt2_tiny.VOCAB)
    a = ferrum_hip.GPT2Device.from_gguf(fh, gpt2_file(tmp_path, w, "ferrum.gguf", output=out))
    b = ferrum_hip.GPT2Device.from_gguf(fh, gpt2_file(tmp_path, w, "foreign.gguf", file_order=order, output=out))
    try:
        assert a.vocab_perm is None and b.vocab_perm is not None
        assert [int(order[p]) for p in b.vocab_perm] == list(range(gpt2_tiny.VOCAB))
        ids = list(np.random.default_rng(5).integers(0, gpt2_tiny.VOCAB, 10))
        for i in range(len(ids)):
            za = a.forward(ids[: i + 1], reprime=(i == 0))
            zb = b.forward(ids[: i + 1], reprime=(i == 0))
            bits_equal(zb, za)
    finally:
        a.free()
        b.free()


def f32_gpt2_weights(orc, vocab, d, layers, ffn, ctx, seed):
    """A GPT-2 whose d-wide matrices have ne0 = d = 48 (not a multiple of 32):
    the reference's writer stores those as F32, and ffn_down (ne0 = ffn) as
    Q8_0."""
    rng = np.random.default_rng(seed)
    f = lambda *s, sc=0.1, base=0.0: (base + rng.standard_normal(s) * sc).astype(np.float32)  # noqa: E731
    w = {"token_embd_f32": f(vocab, d, sc=0.3), "position_embd": f(ctx, d), "lnf_g": f(d, base=1.0), "lnf_b": f(d)}
    for i in range(layers):
        w.update({f"blk{i}.ln1_g": f(d, base=1.0), f"blk{i}.ln1_b": f(d, sc=0.05), f"blk{i}.ln2_g": f(d, base=1.0),
                  f"blk{i}.ln2_b": f(d, sc=0.05), f"blk{i}.qkv_f32": f(3 * d, d, sc=0.15), f"blk{i}.qkv_b": f(3 * d),
                  f"blk{i}.out_f32": f(d, d, sc=0.08), f"blk{i}.out_b": f(d), f"blk{i}.up_f32": f(ffn, d),
                  f"blk{i}.up_b": f(ffn), f"blk{i}.down_q8": orc.q8_0_encode(f(d * ffn, sc=0.05)),
                  f"blk{i}.down_b": f(d)})
    return w


def test_gpt2_with_f32_matrices_matches_the_oracle(fh, orc, tmp_path):
    import ferrum_gguf
    import ferrum_hip

    V, D, H, L, F, CTX = 300, 48, 3, 2, 192, 32
    w = f32_gpt2_weights(orc, V, D, L, F, CTX, 4)
    path = str(tmp_path / "f32.gguf")
    ferrum_gguf.gpt2_gguf(w, V, D, H, L, F, CTX).write(path)
    with ferrum_hip.GGUFFile(path) as g:
        assert g.tensors["blk.0.attn_qkv.weight"][1] == ferrum_gguf.GGML_F32
        assert g.tensors["blk.0.ffn_down.weight"][1] == ferrum_gguf.GGML_Q8_0
    m = ferrum_hip.GPT2Device.from_gguf(fh, path)
    ref = gpt2_tiny.OracleGPT2(orc, w, V, D, H, L, F, CTX)
    try:
        assert m.stack is None and m.head.is_f32 and not m.blocks[0]["down"].is_f32
        ids = list(np.random.default_rng(6).integers(0, V, 12))
        for i in range(len(ids)):
            got = m.forward(ids[: i + 1], reprime=(i == 0))
            want = ref.forward(ids[: i + 1], reprime=(i == 0))
            close(got, want, 2e-5 * max(1.0, float(np.abs(want).max())))
    finally:
        m.free()


# ---- llama / qwen2 files ----------------------------------------------------------------

def llama_path(tmp_path, w, cfg, arch, name="m.gguf", **kw):
    import ferrum_gguf

    path = str(tmp_path / name)
    ferrum_gguf.llama_gguf(w, cfg, arch, **kw).write(path)
    return path


def step(m, toks, pos):
    import torch

    m.tokens.copy_(torch.from_numpy(np.asarray(toks, np.int32)).cuda())
    m.pos.copy_(torch.from_numpy(np.asarray(pos, np.int32)).cuda())
    torch.cuda.synchronize()
    m.feed_async(int(max(pos)))
    m.ctx.sync()
    return m.z.cpu().numpy()


@pytest.mark.parametrize("rows", [2, 3])
@pytest.mark.parametrize("name,arch,biases,tied", [("QWEN", "qwen2", True, True), ("LLAMA", "llama", False, False)])
def test_llama_gguf_equals_the_model_built_from_arrays(fh, orc, tmp_path, name, arch, biases, tied, rows):
    """Two rows (one launch per op) and three (the fused edges, with the
    gate|up rows interleaved for the SwiGLU epilogue), 10 steps: the
    file-loaded model's scores are the array-built model's, bit for bit (same
    kernels on the same Q8_0 bytes)."""
    import ferrum_hip

    cfg = dict(getattr(llama_tiny, name))
    w = llama_tiny.make_weights(orc, cfg, 33, biases, tied)
    a = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, rows)
    b = ferrum_hip.LlamaDevice.from_gguf(fh, llama_path(tmp_path, w, cfg, arch), rows=rows)
    try:
        assert (b.rope_type, b.nkv, b.hd, b.rope_dim, b.cap) == (cfg["rope_type"], cfg["n_kv"], cfg["head_dim"],
                                                                 cfg.get("rope_dim", cfg["head_dim"]), cfg["context"])
        assert all(blk["glu"] for blk in a.blocks + b.blocks) == (rows == 3)
        toks = np.random.default_rng(1).integers(0, cfg["vocab"], (10, rows))
        for t in range(10):
            pos = [t + 3 * r for r in range(rows)]
            bits_equal(step(b, toks[t], pos), step(a, toks[t], pos))
    finally:
        a.free()
        b.free()


def test_qwen_gguf_with_f32_matrices_and_rope_scaling_matches_the_oracle(fh, orc, tmp_path):
    """A qwen2 file with some matrices stored F32 (the token table among them,
    so the tied head is F32), linear rope scaling 2 and rope_freqs.weight."""
    import ferrum_gguf
    import ferrum_hip

    cfg = dict(llama_tiny.QWEN)
    w = llama_tiny.make_weights(orc, cfg, 7, True, True)
    freqs = np.random.default_rng(2).uniform(0.5, 4.0, cfg["head_dim"] // 2).astype(np.float32)

    def extra(b):
        b.str("qwen2.rope.scaling.type", "linear").f32("qwen2.rope.scaling.factor", 2.0)
        b.tensor("rope_freqs.weight", [cfg["head_dim"] // 2], ferrum_gguf.GGML_F32, freqs.tobytes())

    path = llama_path(tmp_path, w, cfg, "qwen2", f32_names=("token_embd", "blk.0.attn_k", "blk.1.ffn_down"),
                      extra=extra)
    m = ferrum_hip.LlamaDevice.from_gguf(fh, path, rows=1)
    rcfg = dict(cfg, rope_linear=2.0, rope_freqs=freqs)
    ref = llama_tiny.OracleLlamaRow(orc, w, rcfg)
    try:
        assert m.head.is_f32 and m.blocks[0]["qkv"].is_f32 and not m.blocks[0]["gate_up"].is_f32
        assert m.rope_linear == 2.0 and m.rope_freqs is not None
        toks = np.random.default_rng(4).integers(0, cfg["vocab"], 12)
        for t in range(12):
            got = step(m, [toks[t]], [t])[0]
            want = ref.feed(toks[t])
            close(got, want, 2e-5 * max(1.0, float(np.abs(want).max())))
    finally:
        m.free()


def test_llama_gguf_capacity_override(fh, orc, tmp_path):
    import ferrum_hip

    cfg = dict(llama_tiny.LLAMA)
    w = llama_tiny.make_weights(orc, cfg, 3, False, False)
    m = ferrum_hip.LlamaDevice.from_gguf(fh, llama_path(tmp_path, w, cfg, "llama"), rows=1, capacity=16)
    try:
        assert m.cap == 16 and m.blocks[0]["k"].numel() == 16 * cfg["n_kv"] * cfg["head_dim"]
    finally:
        m.free()
