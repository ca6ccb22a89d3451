"""A small random GPT-2 (the shape of the tiny configuration: d = 128, 4
blocks, 4 heads, FFN 512, vocabulary 4096, context 256) for the decode-step
tests, and its decode on the CPU oracle, composed the way
CachedTransformer::feed walks the model (slm/cached.rs:100-125) with
TransformerBlock::forward_with_cache (layer/transformer.rs:221-290)."""
import numpy as np

VOCAB, D, HEADS, LAYERS, FFN, CTX = 4096, 128, 4, 4, 512, 256


def make_weights(orc, seed=11, vocab=VOCAB, d=D, layers=LAYERS, ffn=FFN, ctx=CTX, std=None):
    """Random weights in GgufOut::gpt2's naming.  std=None gives each matrix its
    own spread (0.05-0.3, so the tiny model's scores are not flat); a number
    draws every Q8_0 matrix from N(0, std), as BASELINE's configs do (0.02)."""
    rng = np.random.default_rng(seed)

    def q8(n, k, scale):
        return orc.q8_0_encode((rng.standard_normal(n * k) * (scale if std is None else std)).astype(np.float32))

    def vec(n, scale, base=0.0):
        return (base + rng.standard_normal(n) * scale).astype(np.float32)

    w = {"token_embd_q8": q8(vocab, d, 0.3), "position_embd": vec(ctx * d, 0.1).reshape(ctx, d),
         "lnf_g": vec(d, 0.1, 1.0), "lnf_b": vec(d, 0.05)}
    for i in range(layers):
        w.update({f"blk{i}.ln1_g": vec(d, 0.1, 1.0), f"blk{i}.ln1_b": vec(d, 0.05),
                  f"blk{i}.ln2_g": vec(d, 0.1, 1.0), f"blk{i}.ln2_b": vec(d, 0.05),
                  f"blk{i}.qkv_q8": q8(3 * d, d, 0.15), f"blk{i}.qkv_b": vec(3 * d, 0.05),
                  f"blk{i}.out_q8": q8(d, d, 0.08), f"blk{i}.out_b": vec(d, 0.05),
                  f"blk{i}.up_q8": q8(ffn, d, 0.1), f"blk{i}.up_b": vec(ffn, 0.05),
                  f"blk{i}.down_q8": q8(d, ffn, 0.05), f"blk{i}.down_b": vec(d, 0.05)})
    return w


def make_config1_weights(orc, seed=1):
    """BASELINE configs[0] as its random init: every matrix (Q8_0, including
    the tied token table) and the position table from N(0, 0.02), LayerNorm
    gamma 1 and beta 0, biases 0."""
    rng = np.random.default_rng(seed)

    def q8(n, k):
        return orc.q8_0_encode((rng.standard_normal(n * k) * 0.02).astype(np.float32))

    ones, zeros = (lambda n: np.ones(n, np.float32)), (lambda n: np.zeros(n, np.float32))
    w = {"token_embd_q8": q8(VOCAB, D),
         "position_embd": (rng.standard_normal((CTX, D)) * 0.02).astype(np.float32),
         "lnf_g": ones(D), "lnf_b": zeros(D)}
    for i in range(LAYERS):
        w.update({f"blk{i}.ln1_g": ones(D), f"blk{i}.ln1_b": zeros(D), f"blk{i}.ln2_g": ones(D),
                  f"blk{i}.ln2_b": zeros(D), f"blk{i}.qkv_q8": q8(3 * D, D), f"blk{i}.qkv_b": zeros(3 * D),
                  f"blk{i}.out_q8": q8(D, D), f"blk{i}.out_b": zeros(D), f"blk{i}.up_q8": q8(FFN, D),
                  f"blk{i}.up_b": zeros(FFN), f"blk{i}.down_q8": q8(D, FFN), f"blk{i}.down_b": zeros(D)})
    return w


class OracleGPT2:
    """The decode on the oracle: every piece is the C restatement."""

    def __init__(self, orc, w, vocab=VOCAB, d=D, heads=HEADS, layers=LAYERS, ffn=FFN, ctx=CTX):
        self.orc, self.w, self.vocab, self.d, self.heads, self.layers, self.ffn, self.cap = (
            orc, w, vocab, d, heads, layers, ffn, ctx)
        self.tok_w = (np.asarray(w["token_embd_f32"], np.float32).reshape(vocab, d) if "token_embd_f32" in w
                      else orc.q8_0_dequant(w["token_embd_q8"], vocab * d).reshape(vocab, d))
        self.k = [np.zeros((ctx, d), np.float32) for _ in range(layers)]
        self.v = [np.zeros((ctx, d), np.float32) for _ in range(layers)]
        self.pos = 0

    def lin(self, x, key, n, bias):
        """ops::linear_forward on the key's matrix: Q8_0 rows (key_q8) as the
        reference expands them, or F32 rows (key_f32) as stored."""
        x = np.atleast_2d(np.asarray(x, np.float32))
        if key + "_f32" in self.w:
            rows = np.asarray(self.w[key + "_f32"], np.float32).reshape(n, -1)
            return self.orc.linear_forward(x, np.ascontiguousarray(rows.T), bias)
        return self.orc.q8_0_linear(x, self.w[key + "_q8"], n, bias)

    def feed(self, token):
        orc, w, d = self.orc, self.w, self.d
        x = orc.embed_one(self.tok_w, w["position_embd"], int(token), self.pos)
        for i in range(self.layers):
            g = lambda name: w[f"blk{i}.{name}"]  # noqa: E731
            h = orc.layernorm(x, g("ln1_g"), g("ln1_b"))
            qkv = self.lin(h, f"blk{i}.qkv", 3 * d, g("qkv_b"))[0]
            att = orc.attention_decode(qkv, self.k[i], self.v[i], self.heads, self.pos)
            x = (x + self.lin(att, f"blk{i}.out", d, g("out_b"))[0]).astype(np.float32)
            h = orc.layernorm(x, g("ln2_g"), g("ln2_b"))
            up = orc.gelu(self.lin(h, f"blk{i}.up", self.ffn, g("up_b")))
            x = (x + self.lin(up, f"blk{i}.down", d, g("down_b"))[0]).astype(np.float32)
        self.pos += 1
        h = orc.layernorm(x, w["lnf_g"], w["lnf_b"])
        return self.lin(h, "token_embd", self.vocab, None)[0]

    def forward(self, ids, reprime):
        """gpt2_decode's forward: reprime re-feeds the window from position 0."""
        ids = list(ids)
        if reprime:
            self.pos = 0
            for kk, vv in zip(self.k, self.v):
                kk[:] = 0.0
                vv[:] = 0.0
            todo = ids
        else:
            todo = ids[-1:]
        z = None
        for t in todo:
            z = self.feed(t)
        return z


def full_forward_f64(orc, w, ids, vocab=VOCAB, d=D, heads=HEADS, layers=LAYERS, ffn=FFN):
    """The whole sequence at once in float64 with matrix attention and a causal
    mask (the non-cached formulation; slm/cached.rs:153-230 pins the cached
    path against it).  Returns the scores of every position."""
    f64 = lambda a: np.asarray(a, np.float64)  # noqa: E731
    tok = f64(orc.q8_0_dequant(w["token_embd_q8"], vocab * d).reshape(vocab, d))
    W = lambda raw, n, k: f64(orc.q8_0_dequant(raw, n * k).reshape(n, k))  # noqa: E731 (rows = outputs)

    def ln(x, g, b):
        mu = x.mean(axis=1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
        return (x - mu) / np.sqrt(var + 1e-5) * f64(g) + f64(b)

    def gelu(x):
        return 0.5 * x * (1.0 + np.tanh(0.7978846 * (x + 0.044715 * x ** 3)))

    T = len(ids)
    x = tok[ids] + f64(w["position_embd"])[:T]
    hd = d // heads
    mask = np.triu(np.full((T, T), -np.inf), 1)
    for i in range(layers):
        g = lambda name: w[f"blk{i}.{name}"]  # noqa: E731
        h = ln(x, g("ln1_g"), g("ln1_b"))
        qkv = h @ W(g("qkv_q8"), 3 * d, d).T + f64(g("qkv_b"))
        q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
        att = np.zeros((T, d))
        for hh in range(heads):
            s = slice(hh * hd, (hh + 1) * hd)
            sc = q[:, s] @ k[:, s].T / np.sqrt(hd) + mask
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            att[:, s] = (p / p.sum(axis=1, keepdims=True)) @ v[:, s]
        x = x + att @ W(g("out_q8"), d, d).T + f64(g("out_b"))
        h = ln(x, g("ln2_g"), g("ln2_b"))
        x = x + gelu(h @ W(g("up_q8"), ffn, d).T + f64(g("up_b"))) @ W(g("down_q8"), d, ffn).T + f64(g("down_b"))
    return ln(x, w["lnf_g"], w["lnf_b"]) @ tok.T
