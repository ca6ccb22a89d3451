"""Pins for the oracle's restatement of the rest of a GPT-2 decode step
(layer/norm.rs:46-82, activation.rs:9-12, layer/embedding.rs:70-90,
layer/transformer.rs:221-290), CPU only: the reference's own tests re-run on
it, and the cached decode against a float64 full-sequence forward."""
import numpy as np
import pytest

import gpt2_tiny


def test_gelu_known_values_and_saturation(orc):
    # activation.rs:183-195, 170-180, 166
    got = orc.gelu(np.array([1.0, -1.0, 0.5], np.float32))
    assert np.all(np.abs(got - np.array([0.8411919, -0.1588081, 0.345714], np.float32)) < 2e-6)
    assert orc.gelu(np.zeros(1, np.float32))[0] == 0.0
    big = np.array([10.0, 12.5, 30.0, 1e4, 1e10, 1e20, 3e38], np.float32)
    assert np.array_equal(orc.gelu(big), big)
    assert np.all(np.abs(orc.gelu(-big)) == 0.0)


def test_gelu_is_the_tanh_form_in_float64(orc):
    x = np.linspace(-8, 8, 2001).astype(np.float32)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(orc.gelu(x) - want) <= 1e-6 * np.maximum(1.0, np.abs(want)))


def test_layernorm_mean_var_and_constant_rows(orc):
    # layer/norm.rs:99-124
    x = np.array([[1, 2, 3, 4], [10, -10, 20, -20]], np.float32)
    y = orc.layernorm(x, np.ones(4), np.zeros(4))
    assert np.all(np.abs(y.mean(axis=1)) < 1e-4) and np.all(np.abs(y.var(axis=1) - 1.0) < 1e-3)
    y = orc.layernorm(np.full((1, 4), 5.0, np.float32), np.full(4, 2.0), np.ones(4))
    assert np.all(np.abs(y - 1.0) < 1e-3)


def test_layernorm_against_float64(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 768)) * rng.choice([1e-2, 1.0, 30.0], (7, 1))).astype(np.float32)
    g, b = rng.standard_normal(768).astype(np.float32), rng.standard_normal(768).astype(np.float32)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + b
    assert np.all(np.abs(orc.layernorm(x, g, b) - want) <= 2e-5 * np.maximum(1.0, np.abs(want)))


def test_embed_one_sums_rows_and_rejects_out_of_range(orc):
    rng = np.random.default_rng(4)
    tok, pos = rng.standard_normal((10, 8)).astype(np.float32), rng.standard_normal((5, 8)).astype(np.float32)
    assert np.array_equal(orc.embed_one(tok, pos, 7, 3), (tok[7] + pos[3]).astype(np.float32))
    with pytest.raises(ValueError):
        orc.embed_one(tok, pos, 10, 0)
    with pytest.raises(ValueError):
        orc.embed_one(tok, pos, 0, 5)


def test_attention_decode_equals_full_causal_attention(orc):
    """transformer.rs:670 (kv_cache_matches_full_forward): feeding positions
    one by one equals softmax(Q K^T / sqrt(hd) + causal mask) V."""
    rng = np.random.default_rng(5)
    T, d, heads = 40, 96, 3
    hd = d // heads
    qkv = rng.standard_normal((T, 3 * d)).astype(np.float32)
    kc, vc = np.zeros((64, d), np.float32), np.zeros((64, d), np.float32)
    got = np.stack([orc.attention_decode(qkv[t], kc, vc, heads, t) for t in range(T)])
    q, k, v = (qkv[:, :d].astype(np.float64), qkv[:, d:2 * d].astype(np.float64), qkv[:, 2 * d:].astype(np.float64))
    want = np.zeros((T, d))
    for h in range(heads):
        s = slice(h * hd, (h + 1) * hd)
        sc = q[:, s] @ k[:, s].T / np.sqrt(hd) + np.triu(np.full((T, T), -np.inf), 1)
        p = np.exp(sc - sc.max(1, keepdims=True))
        want[:, s] = (p / p.sum(1, keepdims=True)) @ v[:, s]
    assert np.all(np.abs(got - want) <= 1e-5 * np.maximum(1.0, np.abs(want)))
    assert np.array_equal(kc[:T], qkv[:, d:2 * d]) and np.array_equal(vc[:T], qkv[:, 2 * d:])


def test_attention_decode_rejects_a_full_cache_and_bad_heads(orc):
    kc, vc = np.zeros((4, 8), np.float32), np.zeros((4, 8), np.float32)
    with pytest.raises(ValueError, match="status -1"):
        orc.attention_decode(np.zeros(24, np.float32), kc, vc, 2, 4)
    with pytest.raises(ValueError, match="status -2"):
        orc.attention_decode(np.zeros(24, np.float32), kc, vc, 3, 0)


def test_cached_decode_matches_the_full_forward(orc):
    """slm/cached.rs:153-230: the cached decode's scores at every position equal
    the full non-cached forward of the prefix (float64, matrix attention)."""
    w = gpt2_tiny.make_weights(orc, seed=2, layers=2, vocab=512, ctx=32)
    ids = list(np.random.default_rng(9).integers(0, 512, 12))
    m = gpt2_tiny.OracleGPT2(orc, w, vocab=512, layers=2, ctx=32)
    got = np.stack([m.feed(t) for t in ids])
    want = gpt2_tiny.full_forward_f64(orc, w, ids, vocab=512, layers=2)
    assert np.all(np.abs(got - want) <= 2e-4 * np.maximum(1.0, np.abs(want).max()))
