"""Pins for the oracle's restatement of the Llama / Qwen block pieces
(ferrum_core/src/llm.rs): RmsNorm, RoPE (NORM and NEOX pairings, frequency
factors, linear scaling, partial rotary), grouped-query attention with a KV
cache, and the SwiGLU gate.  Known answers are the reference's own tests
(llm.rs:791-1051); the rest is checked against float64 closed forms written
independently of the oracle's loops."""
import numpy as np
import pytest


def det(n, seed):
    """The reference tests' input generator (llm.rs:775-788): xorshift64 on
    seed | 1, each value (x >> 40) / 2^23 - 1."""
    x = (seed | 1) & 0xFFFFFFFFFFFFFFFF
    out = []
    for _ in range(n):
        x ^= (x << 13) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 7
        x ^= (x << 17) & 0xFFFFFFFFFFFFFFFF
        out.append(np.float32(x >> 40) / np.float32(1 << 23) - np.float32(1.0))
    return np.array(out, np.float32)


# ---- RmsNorm ----------------------------------------------------------------

def test_rmsnorm_matches_formula(orc):
    """llm.rs:791-803."""
    w = np.array([2.0, 0.5, 1.0, 1.5], np.float32)
    x = np.array([1.0, -2.0, 3.0, 0.5], np.float32)
    got = orc.rmsnorm(x, w, 1e-6)
    ms = np.float32(np.sum(x * x, dtype=np.float32) / np.float32(4))
    inv = np.float32(1.0) / np.sqrt(ms + np.float32(1e-6))
    assert np.max(np.abs(got - x * inv * w)) < 1e-6
    # float64 closed form, several rows
    rng = np.random.default_rng(1)
    xs = (rng.standard_normal((5, 896)) * 3).astype(np.float32)
    ws = rng.standard_normal(896).astype(np.float32)
    want = xs / np.sqrt(np.mean(xs.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-5) * ws
    np.testing.assert_allclose(orc.rmsnorm(xs, ws, 1e-5), want, rtol=2e-5, atol=1e-6)


def test_rmsnorm_unit_weight_gives_unit_rms(orc):
    """llm.rs:805-812."""
    out = orc.rmsnorm(det(8, 5), np.ones(8, np.float32), 1e-6)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-3


# ---- RoPE -------------------------------------------------------------------

def rope64(x, n_heads, head_dim, rope_dim, pos, base, rope_type, ff=None, lf=1.0):
    """float64 rotation written from the definition.  The angle is formed as
    the reference forms it, in float32 (pos * freq / ff_i * (1 / lf), with
    freq = f32(base^(-2i/rope_dim)) in float64): its rounding (an ulp of
    pos * freq) is part of the reference's result."""
    x = x.astype(np.float64).copy()
    half = rope_dim // 2
    f32 = np.float32
    for h in range(n_heads):
        off = h * head_dim
        for i in range(half):
            freq = f32(float(base) ** (-2.0 * i / rope_dim))
            th = float(f32(f32(f32(pos) * freq) / f32(1.0 if ff is None else ff[i])) * (f32(1.0) / f32(lf)))
            a, b = (off + 2 * i, off + 2 * i + 1) if rope_type == 0 else (off + i, off + i + half)
            xa, xb = x[a], x[b]
            x[a], x[b] = xa * np.cos(th) - xb * np.sin(th), xa * np.sin(th) + xb * np.cos(th)
    return x


@pytest.mark.parametrize("rt", [0, 1])
def test_rope_at_position_zero_is_identity(orc, rt):
    """llm.rs:816-826."""
    x = det(16, 9)
    assert np.max(np.abs(orc.rope(x, 2, 8, 8, 0, 10000.0, rt) - x)) < 1e-6


@pytest.mark.parametrize("rt", [0, 1])
def test_rope_preserves_per_pair_norm(orc, rt):
    """llm.rs:828-841."""
    x = det(8, 3)
    y = orc.rope(x, 1, 8, 8, 5, 10000.0, rt)
    assert abs(np.sum(x * x) - np.sum(y * y)) < 1e-4


def test_rope_norm_and_neox_differ(orc):
    """llm.rs:843-877."""
    x = det(8, 7)
    assert np.max(np.abs(orc.rope(x, 1, 8, 8, 3, 10000.0, 0) - orc.rope(x, 1, 8, 8, 3, 10000.0, 1))) > 1e-3


@pytest.mark.parametrize("rt", [0, 1])
def test_rope_with_unit_factors_is_bit_identical_to_unscaled(orc, rt):
    """llm.rs:878-891."""
    for pos in (0, 1, 5, 17, 300):
        x = det(16, 3)
        a = orc.rope(x, 2, 8, 8, pos, 10000.0, rt)
        b = orc.rope(x, 2, 8, 8, pos, 10000.0, rt, np.ones(4, np.float32), 1.0)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rope_freq_factors_divide_each_frequency_as_hand_computed(orc):
    """llm.rs:893-918: the reference's own values (libm, f64)."""
    want = {2: [-0.41614684, 0.9092974, 0.9999875, 0.004999979], 7: [0.75390225, 0.6569866, 0.9998469, 0.017499107]}
    ff = np.array([1.0, 4.0], np.float32)
    for pos, w in want.items():
        got = orc.rope(np.array([1, 0, 1, 0], np.float32), 1, 4, 4, pos, 10000.0, 0, ff)
        assert np.max(np.abs(got - np.array(w, np.float32))) < 1e-6
        got = orc.rope(np.array([1, 1, 0, 0], np.float32), 1, 4, 4, pos, 10000.0, 1, ff)
        assert np.max(np.abs(got - np.array([w[0], w[2], w[1], w[3]], np.float32))) < 1e-6


@pytest.mark.parametrize("rt", [0, 1])
def test_linear_factor_two_halves_the_effective_position(orc, rt):
    """llm.rs:920-933: exact equality."""
    for pos in (2, 6, 10, 64):
        x = det(8, 9)
        assert np.array_equal(orc.rope(x, 1, 8, 8, pos, 10000.0, rt, None, 2.0),
                              orc.rope(x, 1, 8, 8, pos // 2, 10000.0, rt))


@pytest.mark.parametrize("rt", [0, 1])
@pytest.mark.parametrize("pos", [1, 37, 1023, 4095])
def test_rope_matches_float64_and_partial_rotary_passes_through(orc, rt, pos):
    x = (np.random.default_rng(pos).standard_normal(3 * 64) * 2).astype(np.float32)
    got = orc.rope(x, 3, 64, 48, pos, 1e6, rt)
    want = rope64(x, 3, 64, 48, pos, 1e6, rt)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    for h in range(3):  # channels past rope_dim are untouched
        assert np.array_equal(got[h * 64 + 48:(h + 1) * 64], x[h * 64 + 48:(h + 1) * 64])


# ---- grouped-query attention --------------------------------------------------

def full_causal_gqa64(q_rows, k_rows, v_rows, n_heads, n_kv, hd):
    """float64 softmax(q K^T / sqrt(hd)) V with the causal mask, query head h
    reading kv head h // (n_heads / n_kv) (llm.rs:305-341)."""
    T = q_rows.shape[0]
    out = np.zeros((T, n_heads * hd))
    group = n_heads // n_kv
    for t in range(T):
        for h in range(n_heads):
            kvh = h // group
            q = q_rows[t, h * hd:(h + 1) * hd].astype(np.float64)
            K = k_rows[:t + 1, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            V = v_rows[:t + 1, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            s = K @ q / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd,T", [(4, 4, 4, 5), (6, 2, 4, 6), (14, 2, 64, 40), (8, 1, 16, 33)])
def test_cached_gqa_attention_matches_full_causal(orc, n_heads, n_kv, hd, T):
    """llm.rs:973-1010 (cached equals full, MHA and GQA), against float64."""
    rng = np.random.default_rng(n_heads * T)
    qd, kvd = n_heads * hd, n_kv * hd
    qkv = (rng.standard_normal((T, qd + 2 * kvd)) * 1.5).astype(np.float32)
    kc, vc = np.zeros((T + 2, kvd), np.float32), np.zeros((T + 2, kvd), np.float32)
    want = full_causal_gqa64(qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], n_heads, n_kv, hd)
    for t in range(T):
        got = orc.gqa_attention_decode(qkv[t], kc, vc, n_heads, n_kv, hd, t)
        np.testing.assert_allclose(got, want[t], rtol=1e-4, atol=1e-5)
    assert np.array_equal(kc[:T], qkv[:, qd:qd + kvd]) and np.array_equal(vc[:T], qkv[:, qd + kvd:])


def test_gqa_attention_rejects_a_full_cache_and_bad_split(orc):
    kc = np.zeros((2, 8), np.float32)
    with pytest.raises(ValueError, match="-1"):
        orc.gqa_attention_decode(np.zeros(24, np.float32), kc, kc.copy(), 2, 2, 4, 2)
    with pytest.raises(ValueError, match="-2"):
        orc.gqa_attention_decode(np.zeros(24, np.float32), kc, kc.copy(), 3, 2, 4, 0)


# ---- SwiGLU -----------------------------------------------------------------

def test_swiglu_matches_the_closed_form(orc):
    """llm.rs:1031-1051's gate: (g / (1 + exp(-g))) * u."""
    rng = np.random.default_rng(4)
    g = (rng.standard_normal(4864) * 4).astype(np.float32)
    u = rng.standard_normal(4864).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(orc.swiglu(g, u), want, rtol=2e-6, atol=1e-30)
    edge = orc.swiglu(np.array([0.0, 100.0, -100.0, -1e30], np.float32), np.ones(4, np.float32))
    assert edge[0] == 0.0 and edge[1] == 100.0 and edge[2] <= 0.0 and edge[3] == 0.0


def test_float64_step_agrees_with_the_oracle(orc):
    """llama_tiny.step_f64 (the float64 anchor of the whole-model GPU tests) is
    an independent restatement of LlamaModel::forward_one: on the tiny Qwen2
    and Llama shapes (NEOX and partial NORM rope, biases, tied and untied
    heads) it agrees with the oracle's f32 decode to f32 rounding over three
    positions, and a planted mistake (the rope pairs of the other type) does
    not."""
    import llama_tiny

    for cfg, biases, tied in ((llama_tiny.QWEN, True, True), (llama_tiny.LLAMA, False, False)):
        w = llama_tiny.make_weights(orc, cfg, 5, biases, tied)
        kvd = cfg["n_kv"] * cfg["head_dim"]
        ref = llama_tiny.OracleLlamaRow(orc, w, cfg, 0)
        kc = [[np.zeros((cfg["context"], kvd))] for _ in range(cfg["layers"])]
        vc = [[np.zeros((cfg["context"], kvd))] for _ in range(cfg["layers"])]
        bad = dict(cfg, rope_type=1 - cfg["rope_type"])
        kb = [[np.zeros((cfg["context"], kvd))] for _ in range(cfg["layers"])]
        vb = [[np.zeros((cfg["context"], kvd))] for _ in range(cfg["layers"])]
        worst_bad = 0.0
        for pos, tok in enumerate((3, 77, 5)):
            want = ref.feed(tok)
            got = llama_tiny.step_f64(orc, w, cfg, [tok], [pos], kc, vc)[0]
            scale = np.abs(want).max()
            assert np.abs(got - want).max() <= 2e-5 * scale, (cfg["vocab"], pos)
            worst_bad = max(worst_bad, float(np.abs(llama_tiny.step_f64(orc, w, bad, [tok], [pos], kb, vb)[0]
                                                    - want).max() / scale))
        assert worst_bad > 1e-3
