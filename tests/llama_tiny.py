"""Small random Llama / Qwen2 models for the batched decode tests, and their
decode on the CPU oracle, composed the way LlamaModel::forward_one walks the
model (llm.rs:606-616) with LlamaBlock::forward_one (llm.rs:445-456) and
Attention::forward_one (llm.rs:345-358): separate q, k, v, gate and up linears,
as the reference holds them."""
import numpy as np

# Qwen2-shaped: NEOX rope, q/k/v biases, tied head (gguf/llama.rs:181-185, 250-262, 301-306)
QWEN = dict(vocab=512, d=128, n_heads=4, n_kv=2, head_dim=32, layers=2, ffn=256, context=48, rope_type=1,
            rope_base=1e6, eps=1e-6)
# Llama-shaped: NORM rope on 8 of 16 channels, no biases, its own output.weight
LLAMA = dict(vocab=384, d=96, n_heads=6, n_kv=2, head_dim=16, layers=2, ffn=160, context=40, rope_type=0,
             rope_base=10000.0, eps=1e-5, rope_dim=8)


# the Qwen2-0.5B shape (d 896, 14 q-heads / 2 kv-heads of 64, SwiGLU 4864, vocabulary
# 151936, 24 blocks, NEOX rope with base 1e6, q/k/v biases, tied head)
QWEN05 = dict(vocab=151936, d=896, n_heads=14, n_kv=2, head_dim=64, layers=24, ffn=4864, context=320, rope_type=1,
              rope_base=1e6, eps=1e-6)


def make_weights(orc, cfg, seed, biases, tied, std=None):
    """Random weights keyed as a GGUF file names them.  std=None gives each
    matrix its own spread; a number draws every Q8_0 matrix from N(0, std)
    (float32 draws), as BASELINE's configs do (0.02)."""
    rng = np.random.default_rng(seed)
    d, qd, kvd, ffn = cfg["d"], cfg["n_heads"] * cfg["head_dim"], cfg["n_kv"] * cfg["head_dim"], cfg["ffn"]

    def q8(n, k, scale):
        if std is not None:
            return orc.q8_0_encode(rng.standard_normal(n * k, dtype=np.float32) * np.float32(std))
        return orc.q8_0_encode((rng.standard_normal(n * k) * scale).astype(np.float32))

    def vec(n, scale, base=0.0):
        return (base + rng.standard_normal(n) * scale).astype(np.float32)

    w = {"token_embd": q8(cfg["vocab"], d, 0.5), "output_norm": vec(d, 0.1, 1.0)}
    if not tied:
        w["output"] = q8(cfg["vocab"], d, 0.1)
    for i in range(cfg["layers"]):
        p = f"blk.{i}."
        w.update({p + "attn_norm": vec(d, 0.1, 1.0), p + "ffn_norm": vec(d, 0.1, 1.0),
                  p + "attn_q": q8(qd, d, 0.12), p + "attn_k": q8(kvd, d, 0.12), p + "attn_v": q8(kvd, d, 0.12),
                  p + "attn_output": q8(d, qd, 0.08), p + "ffn_gate": q8(ffn, d, 0.1), p + "ffn_up": q8(ffn, d, 0.1),
                  p + "ffn_down": q8(d, ffn, 0.06)})
        if biases:
            w.update({p + "attn_q.bias": vec(qd, 0.05), p + "attn_k.bias": vec(kvd, 0.05),
                      p + "attn_v.bias": vec(kvd, 0.05)})
    return w


class OracleLlamaRow:
    """One sequence decoded on the oracle; its caches start zeroed, like the
    device's, so a row may start at any position."""

    def __init__(self, orc, w, cfg, pos0=0):
        self.orc, self.w, self.c = orc, w, cfg
        kvd = cfg["n_kv"] * cfg["head_dim"]
        self.tok_w = orc.q8_0_dequant(w["token_embd"], cfg["vocab"] * cfg["d"]).reshape(cfg["vocab"], cfg["d"])
        self.k = [np.zeros((cfg["context"], kvd), np.float32) for _ in range(cfg["layers"])]
        self.v = [np.zeros((cfg["context"], kvd), np.float32) for _ in range(cfg["layers"])]
        self.pos = pos0

    def feed(self, token):
        orc, w, c = self.orc, self.w, self.c
        d, nh, nkv, hd = c["d"], c["n_heads"], c["n_kv"], c["head_dim"]
        rd, base, rt, eps = c.get("rope_dim", hd), c["rope_base"], c["rope_type"], c["eps"]
        lin = lambda x, name, n: orc.q8_0_linear(x[None, :], w[name], n, w.get(name + ".bias"))[0]  # noqa: E731
        x = self.tok_w[int(token)].copy()
        for i in range(c["layers"]):
            p = f"blk.{i}."
            h = orc.rmsnorm(x, w[p + "attn_norm"], eps)
            ff, lf = c.get("rope_freqs"), c.get("rope_linear", 1.0)  # RopeScaling (gguf/llama.rs:51-103)
            q = orc.rope(lin(h, p + "attn_q", nh * hd), nh, hd, rd, self.pos, base, rt, ff, lf)
            k = orc.rope(lin(h, p + "attn_k", nkv * hd), nkv, hd, rd, self.pos, base, rt, ff, lf)
            v = lin(h, p + "attn_v", nkv * hd)
            att = orc.gqa_attention_decode(np.concatenate([q, k, v]), self.k[i], self.v[i], nh, nkv, hd, self.pos)
            x = (x + lin(att, p + "attn_output", d)).astype(np.float32)
            h = orc.rmsnorm(x, w[p + "ffn_norm"], eps)
            m = orc.swiglu(lin(h, p + "ffn_gate", c["ffn"]), lin(h, p + "ffn_up", c["ffn"]))
            x = (x + lin(m, p + "ffn_down", d)).astype(np.float32)
        self.pos += 1
        h = orc.rmsnorm(x, w["output_norm"], eps)
        return orc.q8_0_linear(h[None, :], w.get("output", w["token_embd"]), c["vocab"], None)[0]


def step_f64(orc, w, cfg, tokens, positions, kc, vc):
    """One decode position of several sequences in float64 (exact arithmetic
    on the dequantised weights; the exp, sin and cos of numpy's float64):
    token tokens[r] at position positions[r], attending over the float64
    caches kc[i][r] / vc[i][r] ([capacity, n_kv * head_dim] per layer and
    row), whose row positions[r] it writes.  Returns the logits [rows, vocab]."""
    d, nh, nkv, hd = cfg["d"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"]
    rd, base, rt, eps = cfg.get("rope_dim", hd), cfg["rope_base"], cfg["rope_type"], cfg["eps"]
    qd, kvd, group = nh * hd, nkv * hd, nh // nkv
    f64 = lambda a: np.asarray(a, np.float64)  # noqa: E731

    def W(name, n, k):
        return f64(orc.q8_0_dequant(w[name], n * k).reshape(n, k))

    def rms(x, g):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * f64(g)

    def rope(x, nheads):
        x = x.copy()
        half = rd // 2
        for r in range(x.shape[0]):
            ang = positions[r] * base ** (-2.0 * np.arange(half) / rd)
            sn, cs = np.sin(ang), np.cos(ang)
            for h in range(nheads):
                o = h * hd
                ia = o + (2 * np.arange(half) if rt == 0 else np.arange(half))
                ib = ia + (1 if rt == 0 else half)
                a, b = x[r, ia].copy(), x[r, ib].copy()
                x[r, ia], x[r, ib] = a * cs - b * sn, a * sn + b * cs
        return x

    rows = len(tokens)
    tok = W("token_embd", cfg["vocab"], d)
    x = tok[np.asarray(tokens)]
    for i in range(cfg["layers"]):
        p = f"blk.{i}."
        h = rms(x, w[p + "attn_norm"])
        bias = lambda s, n: f64(w.get(p + f"attn_{s}.bias", np.zeros(n)))  # noqa: E731
        q = rope(h @ W(p + "attn_q", qd, d).T + bias("q", qd), nh)
        k = rope(h @ W(p + "attn_k", kvd, d).T + bias("k", kvd), nkv)
        v = h @ W(p + "attn_v", kvd, d).T + bias("v", kvd)
        att = np.zeros((rows, qd))
        for r in range(rows):
            pos = positions[r]
            kc[i][r][pos], vc[i][r][pos] = k[r], v[r]
            for hh in range(nh):
                kv = slice((hh // group) * hd, (hh // group + 1) * hd)
                sc = kc[i][r][:pos + 1, kv] @ q[r, hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                e = np.exp(sc - sc.max())
                att[r, hh * hd:(hh + 1) * hd] = (e / e.sum()) @ vc[i][r][:pos + 1, kv]
        x = x + att @ W(p + "attn_output", d, qd).T
        h = rms(x, w[p + "ffn_norm"])
        g, u = h @ W(p + "ffn_gate", cfg["ffn"], d).T, h @ W(p + "ffn_up", cfg["ffn"], d).T
        x = x + (g / (1.0 + np.exp(-g)) * u) @ W(p + "ffn_down", d, cfg["ffn"]).T
    h = rms(x, w["output_norm"])
    return h @ W("output" if "output" in w else "token_embd", cfg["vocab"], d).T
