"""The rest of a GPT-2 decode step on the GPU (fh_block.hip through the C ABI)
against the oracle: LayerNorm, GELU, the residual add, embed_one and the
KV-cache attention one op at a time, then a small GPT-2 decoded on the device
against the same model on the oracle (scores per position, and greedy and
sampled token ids with the reference's tie rule)."""
import numpy as np
import pytest

import gpt2_tiny

pytestmark = pytest.mark.gpu


def dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def host(fh, t):
    import torch

    fh.sync()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ready():
    import torch

    torch.cuda.synchronize()


def close(got, want, rtol):
    want = np.asarray(want, np.float64)
    err = np.abs(np.asarray(got, np.float64) - want)
    assert np.all(err <= rtol * np.maximum(1.0, np.abs(want))), float(err.max())


@pytest.mark.parametrize("rows,d", [(1, 768), (5, 1024), (3, 128), (2, 3)])
def test_layernorm_matches_oracle(fh, orc, rows, d):
    import ferrum_hip

    rng = np.random.default_rng(rows * d)
    x = (rng.standard_normal((rows, d)) * rng.choice([1e-3, 1.0, 50.0], (rows, 1))).astype(np.float32)
    x[0, :] += np.float32(7.0)
    g, b = rng.standard_normal(d).astype(np.float32), rng.standard_normal(d).astype(np.float32)
    y = dev(np.zeros((rows, d), np.float32))
    xs, gs, bs = dev(x), dev(g), dev(b)
    ready()
    ferrum_hip.layernorm_async(fh, xs, rows, d, gs, bs, y)
    close(host(fh, y), orc.layernorm(x, g, b), 2e-5)


def test_layernorm_constant_row_gives_beta(fh, orc):
    import ferrum_hip

    x, g, b = dev(np.full((1, 4), 5.0, np.float32)), dev(np.full(4, 2.0, np.float32)), dev(np.ones(4, np.float32))
    y = dev(np.zeros((1, 4), np.float32))
    ready()
    ferrum_hip.layernorm_async(fh, x, 1, 4, g, b, y)
    assert np.array_equal(host(fh, y), np.ones((1, 4), np.float32))


def test_gelu_matches_oracle_including_saturation(fh, orc):
    import ferrum_hip

    x = np.concatenate([np.linspace(-12, 12, 4801), [0.0, -0.0, 1e4, -1e4, 1e20, 3e38, -3e38]]).astype(np.float32)
    t = dev(x)
    ready()
    ferrum_hip.gelu_async(fh, t, x.size)
    got, want = host(fh, t), orc.gelu(x)
    close(got, want, 2e-6)
    assert got[4801] == 0.0 and np.array_equal(got[-5:-2], want[-5:-2])


def test_add_is_exact(fh):
    import ferrum_hip

    rng = np.random.default_rng(1)
    a, b = rng.standard_normal(3001).astype(np.float32), rng.standard_normal(3001).astype(np.float32)
    ta, tb = dev(a), dev(b)
    ready()
    ferrum_hip.add_async(fh, ta, tb, a.size)
    assert np.array_equal(host(fh, ta), (a + b).astype(np.float32))


def test_embed_one_reads_the_token_on_the_device(fh, orc):
    import torch

    import ferrum_hip

    rng = np.random.default_rng(2)
    tok, pos = rng.standard_normal((50, 96)).astype(np.float32), rng.standard_normal((20, 96)).astype(np.float32)
    tt, tp, out = dev(tok), dev(pos), dev(np.zeros(96, np.float32))
    token = torch.tensor([37], dtype=torch.int32, device="cuda")
    ready()
    ferrum_hip.embed_one_async(fh, tt, tp, 50, 20, 96, token, 19, out)
    assert np.array_equal(host(fh, out), orc.embed_one(tok, pos, 37, 19))
    with pytest.raises(ferrum_hip.DimMismatch, match="Position 20 exceeds max_seq_len 20"):
        ferrum_hip.embed_one_async(fh, tt, tp, 50, 20, 96, token, 20, out)
    token.fill_(50)                                   # past the vocabulary: a NaN row
    ready()
    ferrum_hip.embed_one_async(fh, tt, tp, 50, 20, 96, token, 0, out)
    assert np.isnan(host(fh, out)).all()


@pytest.mark.parametrize(
    "d,heads,T",
    [(768, 12, 70), (128, 4, 33), (96, 3, 5), (256, 2, 40),
     # several workgroups per head (merge through the partials): 256
     # positions per workgroup at head width <= 64, 128 at 128; the last two
     # need more than one merge round of eight chunks
     (768, 12, 600), (64, 8, 300), (256, 2, 1100), (64, 8, 2100)])
def test_attention_decode_matches_oracle(fh, orc, d, heads, T):
    import ferrum_hip

    rng = np.random.default_rng(d + T)
    cap = T + 3
    qkv = (rng.standard_normal((T, 3 * d)) * 1.5).astype(np.float32)
    # rows at and past the position have never been written: NaN there must
    # not reach the output
    kc, vc = dev(np.full((cap, d), np.nan, np.float32)), dev(np.full((cap, d), np.nan, np.float32))
    ko, vo = np.full((cap, d), np.nan, np.float32), np.full((cap, d), np.nan, np.float32)
    out = dev(np.zeros(d, np.float32))
    edges = {31, 32, 33, 63, 64, 65, 95, 96, 97, 127, 128, 129, 255, 256, 257, 511, 512, 1023, 1024, 1025, 2047, 2048}
    for t in range(T):
        q = dev(qkv[t])
        ready()
        ferrum_hip.attention_decode_async(fh, q, kc, vc, cap, d, heads, t, out)
        if t < 40 or t % 97 == 0 or t in edges or t >= T - 2:
            close(host(fh, out), orc.attention_decode(qkv[t], ko, vo, heads, t), 1e-5)
        else:
            orc.attention_decode(qkv[t], ko, vo, heads, t)  # keeps the oracle's cache in step
    assert np.array_equal(host(fh, kc), ko, equal_nan=True) and np.array_equal(host(fh, vc), vo, equal_nan=True)


@pytest.mark.parametrize(
    "d,heads,blocks",
    [(1024, 16, [(0, 511), (511, 1)]),      # configs[3]'s prime: 511 prompt positions, then the first step's row
     (768, 12, [(0, 128), (128, 200)]),     # a second block reading the first block's cache rows
     (128, 4, [(0, 33), (33, 64), (97, 3)]),
     (64, 1, [(0, 70)])])
def test_attention_prefill_matches_oracle(fh, orc, d, heads, blocks):
    """fh_attention_prefill_async: a block of consecutive positions of one
    sequence at once (row r of qkv is position pos0 + r; every row's k and v go
    into the cache first, then row r attends over positions 0 .. pos0 + r).
    Each row against the oracle's attention for that one position
    (layer/transformer.rs:242-279, fed position by position), and the caches
    bit-equal."""
    import ferrum_hip

    T = blocks[-1][0] + blocks[-1][1]
    cap = T + 5
    rng = np.random.default_rng(d * 3 + T)
    qkv = (rng.standard_normal((T, 3 * d)) * 1.5).astype(np.float32)
    kc, vc = dev(np.full((cap, d), np.nan, np.float32)), dev(np.full((cap, d), np.nan, np.float32))
    ko, vo = np.full((cap, d), np.nan, np.float32), np.full((cap, d), np.nan, np.float32)
    for pos0, n in blocks:
        tq = dev(qkv[pos0:pos0 + n])
        out = dev(np.zeros((n, d), np.float32))
        ready()
        ferrum_hip.attention_prefill_async(fh, tq, kc, vc, cap, d, heads, pos0, n, out)
        got = host(fh, out)
        for r in range(n):
            close(got[r], orc.attention_decode(qkv[pos0 + r], ko, vo, heads, pos0 + r), 1e-5)
    assert np.array_equal(host(fh, kc), ko, equal_nan=True) and np.array_equal(host(fh, vc), vo, equal_nan=True)


@pytest.mark.parametrize("d,heads,seqs,rows,pos0", [(1024, 16, 3, 300, 0), (768, 12, 2, 100, 40), (128, 4, 3, 50, 7)])
def test_attention_prefill_seqs_matches_oracle(fh, orc, d, heads, seqs, rows, pos0):
    """fh_attention_prefill_seqs_async: several sequences' prompt blocks in one
    call (each with its own caches, seq_stride apart; rows before pos0 already
    cached): every row of every sequence against the oracle's attention for
    that position, and the caches bit-equal."""
    import ferrum_hip

    cap = pos0 + rows + 3
    rng = np.random.default_rng(d + seqs * 7 + pos0)
    qkv = (rng.standard_normal((seqs * rows, 3 * d)) * 1.5).astype(np.float32)
    kc = np.full((seqs, cap, d), np.nan, np.float32)
    vc = np.full((seqs, cap, d), np.nan, np.float32)
    kc[:, :pos0] = rng.standard_normal((seqs, pos0, d)).astype(np.float32)
    vc[:, :pos0] = rng.standard_normal((seqs, pos0, d)).astype(np.float32)
    tk, tv = dev(kc), dev(vc)
    out = dev(np.zeros((seqs * rows, d), np.float32))
    ready()
    ferrum_hip.attention_prefill_seqs_async(fh, dev(qkv), tk, tv, cap * d, cap, d, heads, pos0, rows, seqs, out)
    got = host(fh, out)
    for s in range(seqs):
        ko, vo = kc[s].copy(), vc[s].copy()
        for r in range(rows):
            want = orc.attention_decode(qkv[s * rows + r], ko, vo, heads, pos0 + r)
            close(got[s * rows + r], want, 1e-5)
        assert np.array_equal(host(fh, tk)[s], ko, equal_nan=True) and np.array_equal(host(fh, tv)[s], vo,
                                                                                      equal_nan=True)


def test_attention_prefill_with_non_finite_values(fh, orc):
    """A NaN v value at position 50 (head 0) and an inf at position 70 (head
    3): rows before them attend only finite values and stay finite, later rows
    of those heads turn NaN / inf exactly where the oracle's do; every other
    output within 1e-5."""
    import ferrum_hip

    d, heads, rows = 768, 12, 100
    rng = np.random.default_rng(99)
    qkv = (rng.standard_normal((rows, 3 * d)) * 1.5).astype(np.float32)
    qkv[50, 2 * d + 5] = np.nan
    qkv[70, 2 * d + 3 * 64 + 9] = np.inf
    kc, vc = dev(np.zeros((rows, d), np.float32)), dev(np.zeros((rows, d), np.float32))
    out = dev(np.zeros((rows, d), np.float32))
    ready()
    ferrum_hip.attention_prefill_async(fh, dev(qkv), kc, vc, rows, d, heads, 0, rows, out)
    got = host(fh, out)
    ko, vo = np.zeros((rows, d), np.float32), np.zeros((rows, d), np.float32)
    for r in range(rows):
        want = orc.attention_decode(qkv[r], ko, vo, heads, r)
        assert np.array_equal(np.isnan(got[r]), np.isnan(want)), r
        assert np.array_equal(np.isposinf(got[r]), np.isposinf(want)), r
        fin = np.isfinite(want)
        close(got[r][fin], want[fin], 1e-5)
    assert np.isfinite(got[:50]).all() and np.isnan(got[50:, 5]).all()


def test_attention_decode_errors(fh):
    import ferrum_hip

    q, kc, vc, out = (dev(np.zeros(n, np.float32)) for n in (24, 32, 32, 8))
    ready()
    with pytest.raises(ferrum_hip.DimMismatch, match="KvCache full"):
        ferrum_hip.attention_decode_async(fh, q, kc, vc, 4, 8, 2, 4, out)
    with pytest.raises(ferrum_hip.DimMismatch, match="must divide"):
        ferrum_hip.attention_decode_async(fh, q, kc, vc, 4, 8, 3, 0, out)
    with pytest.raises(ferrum_hip.FerrumHipError):
        ferrum_hip.attention_decode_async(fh, dev(np.zeros(3 * 12, np.float32)), dev(np.zeros(48, np.float32)),
                                          dev(np.zeros(48, np.float32)), 4, 12, 1, 0, dev(np.zeros(12, np.float32)))


@pytest.mark.parametrize("m,n,k", [(1, 3072, 768), (2, 512, 256), (5, 640, 768),
                                   (32, 3072, 768), (32, 768, 3072), (64, 4864, 896),  # skinny GEMM epilogue
                                   (7, 50257, 768), (100, 640, 768)])  # wide head, tiled GEMM: GELU kernel after
def test_linear_with_gelu_equals_linear_then_gelu(fh, orc, m, n, k):
    """The fused epilogues (decode GEMV; skinny GEMM at m <= 64, also after
    its K splits are summed) and the two-kernel paths give the separate ops'
    values bit for bit; both track the oracle."""
    import torch

    import ferrum_hip

    raw = orc.quantize_weight(n, k, m + n, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    b = (np.random.default_rng(n).standard_normal(n) * 0.1).astype(np.float32)
    tx, tb = dev(x), dev(b)
    fused, plain = (torch.empty((m, n), device="cuda") for _ in range(2))
    ready()
    ferrum_hip.linear_act_async(fh, w, tx, m, k, tb, n, fused, ferrum_hip.ACT_GELU)
    ferrum_hip.linear_forward_async(fh, w, tx, m, k, tb, n, plain)
    ferrum_hip.gelu_async(fh, plain, m * n)
    got, sep = host(fh, fused), host(fh, plain)
    w.free()
    assert np.array_equal(got, sep)
    # the linear's 1e-5 rule (against max(|y|, sum_p |x_p w_p|)), carried
    # through GELU, whose slope stays below 1.13
    want = np.asarray(orc.gelu(orc.q8_0_linear(x, raw, n, b)), np.float64)
    mass = np.abs(x.astype(np.float64)) @ np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 1.13e-5 * np.maximum(np.abs(want), mass + np.abs(b))), float(err.max())
    with pytest.raises(ferrum_hip.FerrumHipError, match="unknown activation"):
        ferrum_hip.linear_act_async(fh, w, tx, m, k, tb, n, fused, 7)


def test_prefill_gemm_gelu_equals_gemm_then_gelu(fh, orc):
    """At prefill depth (the block-scaled MFMA GEMM, one tile per CU or more)
    GELU runs in the GEMM's epilogue: bit for bit the GEMM followed by the
    GELU kernel, including the rows recomputed by the reference's own
    arithmetic (a weight row with an infinite block scale, an activation row
    holding inf)."""
    import torch

    import ferrum_hip

    m, n, k = 4096, 4096, 256
    raw = np.array(orc.quantize_weight(n, k, 17, 0.05)).reshape(n, k // 32 * 34)
    raw[5, 34:36] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)  # row 5, block 1: scale inf
    w = ferrum_hip.Q8_0Weight.upload(fh, raw.ravel(), n, k)
    x = np.random.default_rng(3).standard_normal((m, k)).astype(np.float32)
    x[7, 3] = np.inf
    b = (np.random.default_rng(4).standard_normal(n) * 0.1).astype(np.float32)
    tx, tb = dev(x), dev(b)
    fused, plain = (torch.empty((m, n), device="cuda") for _ in range(2))
    ready()
    ferrum_hip.linear_act_async(fh, w, tx, m, k, tb, n, fused, ferrum_hip.ACT_GELU)
    ferrum_hip.linear_forward_async(fh, w, tx, m, k, tb, n, plain)
    ferrum_hip.gelu_async(fh, plain, m * n)
    got, sep = host(fh, fused), host(fh, plain)
    w.free()
    assert np.array_equal(got, sep, equal_nan=True)
    assert not np.isfinite(got[:, 5]).all() and not np.isfinite(got[7]).all()
    rows = [0, 7, 4095]
    want = orc.gelu(orc.q8_0_linear(x[rows], raw.ravel(), n, b))
    assert np.array_equal(got[rows], want, equal_nan=True) or np.allclose(got[rows][np.isfinite(want)],
                                                                          want[np.isfinite(want)], rtol=2e-5,
                                                                          atol=2e-5)


@pytest.mark.parametrize(
    "m,n,k,res,act,numerics",
    [(1, 2304, 768, True, 0, 0), (1, 3072, 768, True, 1, 0), (1, 50257, 768, True, 0, 0),  # GPT-2 shapes (G = 16)
     (2, 640, 1024, True, 1, 0), (1, 512, 2048, True, 0, 0),   # 64 lanes per row, 1 and 2 chunks per lane
     (1, 96, 128, True, 0, 0), (2, 100, 896, True, 1, 0),      # narrow rows, ragged group tails
     (5, 640, 768, True, 1, 0), (1, 384, 768, False, 0, 0),    # m > 2: the norm fused into the skinny GEMM
     (32, 2304, 768, True, 0, 0), (32, 3072, 768, True, 1, 0),  # the batch-32 step's QKV and up (+GELU)
     (64, 1152, 896, True, 0, 0), (40, 4096, 1024, False, 1, 0),  # 64-row tiles, no residual
     (17, 9728, 1024, True, 0, 0), (100, 640, 768, True, 1, 0),  # two column tiles per wave; m > 64: two kernels
     (3, 256, 512, True, 1, 1)])                              # W8A8
def test_linear_ln_matches_oracle(fh, orc, m, n, k, res, act, numerics):
    """y = act(LayerNorm(x + r) W^T + b) and s = x + r, against the oracle's
    add, layernorm, Q8_0 linear and gelu (m <= 2: the GEMV's prologue;
    3 <= m <= 64: the skinny GEMM normalising as it stages; else two
    kernels)."""
    import torch

    import ferrum_hip

    rng = np.random.default_rng(m * n + k)
    raw = orc.quantize_weight(n, k, n + k, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = (rng.standard_normal((m, k)) * 2 + 0.5).astype(np.float32)
    r = rng.standard_normal((m, k)).astype(np.float32)
    g, be = rng.standard_normal(k).astype(np.float32), (rng.standard_normal(k) * 0.1).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    tx, tr, tg, tbe, tb = dev(x), dev(r), dev(g), dev(be), dev(b)
    ts = dev(np.full((m, k), np.nan, np.float32))
    y = torch.empty((m, n), device="cuda")
    ready()
    ferrum_hip.linear_ln_async(fh, w, tx, tr if res else None, ts, m, k, tg, tbe, tb, n, y, act, numerics)
    got, s_got = host(fh, y), host(fh, ts)
    sm = (x + r).astype(np.float32) if res else x
    assert np.array_equal(s_got, sm)
    if numerics == 0:
        want = orc.q8_0_linear(orc.layernorm(sm, g, be), raw, n, b)
        close(got, orc.gelu(want) if act else want, 1e-5)
    else:
        # W8A8 re-quantises the LayerNorm output, so a last-bit difference
        # in it can move a quant: compare with the same steps as separate calls.
        tx2, th = dev(x), dev(np.zeros((m, k), np.float32))
        y2 = torch.empty((m, n), device="cuda")
        ready()
        ferrum_hip.add_layernorm_async(fh, tx2, tr, m, k, tg, tbe, th)
        ferrum_hip.linear_act_async(fh, w, th, m, k, tb, n, y2, act, numerics)
        assert np.array_equal(got, host(fh, y2))
    w.free()


def test_fused_layernorm_with_non_finite_scales(fh, orc):
    """The skinny GEMM with the fused LayerNorm (m = 32): weight rows with an
    inf or NaN block scale are recomputed on the normalised row in the
    reference's order, so their inf / NaN pattern is the oracle's; the other
    outputs within 1e-5."""
    import torch

    import ferrum_hip

    m, n, k = 32, 768, 768
    rng = np.random.default_rng(5)
    raw = orc.quantize_weight(n, k, 77, 0.05).reshape(n, k // 32, 34).copy()
    raw[2, 0, :2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)   # +inf scale
    raw[9, 5, :2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)   # NaN scale
    raw = raw.ravel()
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    r = rng.standard_normal((m, k)).astype(np.float32)
    g, be = rng.standard_normal(k).astype(np.float32), (rng.standard_normal(k) * 0.1).astype(np.float32)
    y = torch.empty((m, n), device="cuda")
    ready()
    ferrum_hip.linear_ln_async(fh, w, dev(x), dev(r), None, m, k, dev(g), dev(be), None, 0, y, 0, 0)
    got = host(fh, y)
    want = orc.q8_0_linear(orc.layernorm((x + r).astype(np.float32), g, be), raw, n, None)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want)) and np.array_equal(np.isneginf(got), np.isneginf(want))
    assert not np.isfinite(want[:, 2]).any() and np.isnan(want[:, 9]).all()
    fin = np.isfinite(want)
    close(got[fin], want[fin], 1e-5)
    w.free()


def group_stats(y):
    """Per row and 32-column group: mean and sum of squared deviations (float64)."""
    g = np.asarray(y, np.float64).reshape(y.shape[0], -1, 32)
    mu = g.mean(axis=2)
    return np.stack([mu, ((g - mu[..., None]) ** 2).sum(axis=2)], axis=2)


@pytest.mark.parametrize("m,n,k,inplace", [(32, 768, 768, True), (32, 768, 3072, True), (3, 768, 768, False),
                                           (64, 896, 4864, True), (40, 128, 512, False),
                                           (1, 768, 768, True), (100, 256, 768, False)])  # other shapes: two kernels
def test_linear_residual_matches_oracle(fh, orc, m, n, k, inplace):
    """fh_q8_0_linear_residual_async: y = r + (x W^T + b) (in place: y is r)
    against the oracle's linear and add, and y's row statistics (per 32-column
    group: mean, sum of squared deviations) against float64."""
    import torch

    import ferrum_hip

    rng = np.random.default_rng(m * 7 + n + k)
    raw = orc.quantize_weight(n, k, n + 3 * k, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    r = (rng.standard_normal((m, n)) * 3 + 1).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    tr = dev(r)
    y = tr if inplace else torch.empty((m, n), device="cuda")
    st = dev(np.full((m, n // 32, 2), np.nan, np.float32))
    ready()
    ferrum_hip.linear_residual_async(fh, w, dev(x), m, k, dev(b), n, tr, y, st)
    got = host(fh, y)
    lin = orc.q8_0_linear(x, raw, n, b)
    want = (r + lin).astype(np.float32)
    # the linear's 1e-5 rule (relative to its terms' mass, as every linear
    # test), plus the add's half ulp
    mass = np.abs(x.astype(np.float64)) @ np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= 1e-5 * np.maximum(np.abs(lin), mass) + 6e-8 * np.abs(want)).all(), float(err.max())
    gs, ws = host(fh, st), group_stats(got)
    np.testing.assert_allclose(gs[..., 0], ws[..., 0], rtol=1e-5, atol=1e-6 * np.abs(got).max())
    np.testing.assert_allclose(gs[..., 1], ws[..., 1], rtol=2e-5)
    w.free()


@pytest.mark.parametrize("m,n,k,rms,act", [(32, 2304, 768, False, 0), (32, 3072, 768, False, 1),
                                           (64, 9728, 896, True, 0), (5, 1152, 896, True, 0),
                                           (17, 9728, 1024, False, 0), (2, 640, 768, False, 1),
                                           (80, 384, 256, True, 0)])  # m <= 2 or > 64: two kernels
def test_linear_normed_matches_oracle(fh, orc, m, n, k, rms, act):
    """fh_q8_0_linear_normed_async: act(norm(x) W^T + b) with LayerNorm or
    RmsNorm formed from the rows' group statistics (per 32 columns: mean, sum
    of squared deviations), against the oracle's layernorm / rmsnorm, Q8_0
    linear and gelu."""
    import torch

    import ferrum_hip

    rng = np.random.default_rng(m + n * 3 + k)
    raw = orc.quantize_weight(n, k, n + k, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = (rng.standard_normal((m, k)) * 2 + 0.5).astype(np.float32)
    g = rng.standard_normal(k).astype(np.float32)
    be = (rng.standard_normal(k) * 0.1).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    st = group_stats(x).astype(np.float32)
    y = torch.empty((m, n), device="cuda")
    ready()
    ferrum_hip.linear_normed_async(fh, w, dev(x), m, k, dev(st), dev(g), None if rms else dev(be), 1e-6 if rms else 1e-5,
                                   rms, dev(b), n, y, act)
    h = orc.rmsnorm(x, g, 1e-6) if rms else orc.layernorm(x, g, be)
    want = orc.q8_0_linear(h, raw, n, b)
    close(host(fh, y), orc.gelu(want) if act else want, 1e-5)
    w.free()


@pytest.mark.parametrize("m,ffn,k,rms,bias", [(64, 4864, 896, True, False), (32, 4864, 896, True, False),
                                               (5, 256, 128, True, False), (40, 160, 1024, True, False),
                                               (3, 96, 64, False, True), (33, 4864, 896, False, True)])
def test_linear_normed_swiglu_matches_oracle(fh, orc, m, ffn, k, rms, bias):
    """ACT_SWIGLU32: silu(norm(x) G^T + bg) * (norm(x) U^T + bu) from one
    gate|up weight interleaved in groups of 32 rows, against the oracle's
    rmsnorm / layernorm, two Q8_0 linears and swiglu (the error the two
    linears may carry, 1e-5 of their terms' size, carried through silu and the
    product); where the gate|up GEMM picks the same tile unfused, the result
    equals the unfused GEMM followed by fh_swiglu bit for bit."""
    import torch

    import ferrum_hip

    rng = np.random.default_rng(m * 7 + ffn + k)
    g_raw = orc.quantize_weight(ffn, k, ffn + k, 0.05)
    u_raw = orc.quantize_weight(ffn, k, ffn + k + 1, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, ferrum_hip.interleave_gate_up(g_raw, u_raw, ffn), 2 * ffn, k)
    x = (rng.standard_normal((m, k)) * 2 + 0.5).astype(np.float32)
    gam = rng.standard_normal(k).astype(np.float32)
    be = (rng.standard_normal(k) * 0.1).astype(np.float32)
    bg = (rng.standard_normal(ffn) * 0.1).astype(np.float32) if bias else None
    bu = (rng.standard_normal(ffn) * 0.1).astype(np.float32) if bias else None
    b_il = ferrum_hip.interleave_gate_up(bg, bu, ffn).astype(np.float32) if bias else None
    st = group_stats(x).astype(np.float32)
    eps = 1e-6 if rms else 1e-5
    y = torch.empty((m, ffn), device="cuda")
    ready()
    ferrum_hip.linear_normed_async(fh, w, dev(x), m, k, dev(st), dev(gam), None if rms else dev(be), eps, rms,
                                   dev(b_il) if bias else None, 2 * ffn if bias else 0, y, ferrum_hip.ACT_SWIGLU32)
    got = host(fh, y)
    h = orc.rmsnorm(x, gam, eps) if rms else orc.layernorm(x, gam, be)
    gate, up = orc.q8_0_linear(h, g_raw, ffn, bg), orc.q8_0_linear(h, u_raw, ffn, bu)
    want = orc.swiglu(gate, up)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g64))
    dsilu = np.abs(sig * (1.0 + g64 * (1.0 - sig)))
    tol = 1e-5 * (dsilu * np.maximum(1.0, np.abs(g64)) * np.abs(u64) + np.abs(g64 * sig) * np.maximum(1.0, np.abs(u64)))
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol + 1e-6 * np.maximum(1.0, np.abs(want))), float((err - tol).max())
    if 2 * ffn // 32 >= 256:  # the same tile as the unfused gate|up GEMM
        gu = torch.empty((m, 2 * ffn), device="cuda")
        ferrum_hip.linear_normed_async(fh, w, dev(x), m, k, dev(st), dev(gam), None if rms else dev(be), eps, rms,
                                       dev(b_il) if bias else None, 2 * ffn if bias else 0, gu)
        gu_h = host(fh, gu).reshape(m, ffn // 32, 2, 32)
        sep = torch.empty((m, ffn), device="cuda")
        gg = dev(np.ascontiguousarray(gu_h[:, :, 0].reshape(m, ffn)))
        uu = dev(np.ascontiguousarray(gu_h[:, :, 1].reshape(m, ffn)))
        ready()
        ferrum_hip.swiglu_async(fh, gg, uu, m, ffn, ffn, sep)
        assert np.array_equal(host(fh, sep).view(np.uint32), got.view(np.uint32))
    w.free()


def test_linear_normed_swiglu_limits(fh, orc):
    """ACT_SWIGLU32 is the skinny GEMM's epilogue: m outside 3 .. 64, a weight
    whose rows are not whole gate / up pairs of 32, or k > 1024 is
    FH_ERR_LIMIT; the other linear entry points refuse the activation."""
    import torch

    import ferrum_hip

    k = 128
    for m, n, kk in ((2, 128, k), (65, 128, k), (4, 96, k), (4, 128, 2048)):
        raw = orc.quantize_weight(n, kk, 5, 0.05)
        w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, kk)
        x, st = torch.zeros((m, kk), device="cuda"), torch.zeros((m, kk // 32, 2), device="cuda")
        gam, y = torch.ones(kk, device="cuda"), torch.empty((m, n), device="cuda")
        with pytest.raises(ferrum_hip.FerrumHipError) as e:
            ferrum_hip.linear_normed_async(fh, w, x, m, kk, st, gam, None, 1e-6, True, None, 0, y,
                                           ferrum_hip.ACT_SWIGLU32)
        assert e.value.code == ferrum_hip.FH_ERR_LIMIT and "SWIGLU32" in str(e.value)
        w.free()
    raw = orc.quantize_weight(128, k, 6, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, 128, k)
    with pytest.raises(ferrum_hip.FerrumHipError) as e:
        ferrum_hip.linear_act_async(fh, w, torch.zeros((4, k), device="cuda"), 4, k, None, 0,
                                    torch.empty((4, 128), device="cuda"), ferrum_hip.ACT_SWIGLU32)
    assert e.value.code == ferrum_hip.FH_ERR_INVALID
    w.free()


def test_residual_then_normed_is_add_then_layernorm(fh, orc):
    """A block's chain at 32 rows: x += attn W_out^T + b (statistics left),
    then up(LayerNorm(x)) with GELU from them, against the oracle's add,
    layernorm, linear and gelu; the residual stream equals the oracle's sum."""
    import torch

    import ferrum_hip

    m, d, f = 32, 768, 3072
    rng = np.random.default_rng(3)
    wo_raw, wu_raw = orc.quantize_weight(d, d, 1, 0.05), orc.quantize_weight(f, d, 2, 0.05)
    wo, wu = ferrum_hip.Q8_0Weight.upload(fh, wo_raw, d, d), ferrum_hip.Q8_0Weight.upload(fh, wu_raw, f, d)
    x = rng.standard_normal((m, d)).astype(np.float32)
    att = rng.standard_normal((m, d)).astype(np.float32)
    bo, bu = (rng.standard_normal(d) * 0.1).astype(np.float32), (rng.standard_normal(f) * 0.1).astype(np.float32)
    g, be = rng.standard_normal(d).astype(np.float32), (rng.standard_normal(d) * 0.1).astype(np.float32)
    tx, st, y = dev(x), torch.empty((m, d // 32, 2), device="cuda"), torch.empty((m, f), device="cuda")
    ready()
    ferrum_hip.linear_residual_async(fh, wo, dev(att), m, d, dev(bo), d, tx, tx, st)
    ferrum_hip.linear_normed_async(fh, wu, tx, m, d, st, dev(g), dev(be), 1e-5, False, dev(bu), f, y,
                                   ferrum_hip.ACT_GELU)
    s_want = (x + orc.q8_0_linear(att, wo_raw, d, bo)).astype(np.float32)
    s_got = host(fh, tx)
    close(s_got, s_want, 1e-5)
    want = orc.gelu(orc.q8_0_linear(orc.layernorm(s_got, g, be), wu_raw, f, bu))
    close(host(fh, y), want, 1e-5)
    wo.free()
    wu.free()


def test_linear_ln_errors(fh, orc):
    import torch

    import ferrum_hip

    raw = orc.quantize_weight(64, 256, 1, 0.05)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, 64, 256)
    x, r, g = (dev(np.ones((1, 256), np.float32)) for _ in range(3))
    y = torch.empty(64, device="cuda")
    with pytest.raises(ferrum_hip.FerrumHipError, match="must not alias"):
        ferrum_hip.linear_ln_async(fh, w, x, r, x, 1, 256, g, g, None, 0, y)
    with pytest.raises(ferrum_hip.FerrumHipError, match="must not alias"):
        ferrum_hip.linear_ln_async(fh, w, x, r, r, 1, 256, g, g, None, 0, y)
    with pytest.raises(ferrum_hip.FerrumHipError, match="gamma"):
        ferrum_hip.linear_ln_async(fh, w, x, r, None, 1, 256, None, g, None, 0, y)
    with pytest.raises(ferrum_hip.FerrumHipError, match="unknown activation"):
        ferrum_hip.linear_ln_async(fh, w, x, r, None, 1, 256, g, g, None, 0, y, 9)
    w.free()


def test_add_layernorm_equals_add_then_layernorm(fh, orc):
    import ferrum_hip

    rng = np.random.default_rng(8)
    x, y = rng.standard_normal((3, 768)).astype(np.float32), rng.standard_normal((3, 768)).astype(np.float32)
    g, b = rng.standard_normal(768).astype(np.float32), rng.standard_normal(768).astype(np.float32)
    x1, x2, ty, tg, tb = dev(x), dev(x), dev(y), dev(g), dev(b)
    l1, l2 = dev(np.zeros((3, 768), np.float32)), dev(np.zeros((3, 768), np.float32))
    ready()
    ferrum_hip.add_layernorm_async(fh, x1, ty, 3, 768, tg, tb, l1)
    ferrum_hip.add_async(fh, x2, ty, 3 * 768)
    ferrum_hip.layernorm_async(fh, x2, 3, 768, tg, tb, l2)
    assert np.array_equal(host(fh, x1), host(fh, x2)) and np.array_equal(host(fh, l1), host(fh, l2))
    close(host(fh, l1), orc.layernorm((x + y).astype(np.float32), g, b), 2e-5)


@pytest.fixture(scope="module")
def tiny(fh, orc):
    import ferrum_hip

    w = gpt2_tiny.make_weights(orc, seed=11)
    model = ferrum_hip.GPT2Device.from_weights(fh, w, gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS,
                                  gpt2_tiny.FFN, gpt2_tiny.CTX)
    yield w, model
    model.free()


def test_tiny_gpt2_scores_match_the_oracle_per_position(orc, tiny):
    w, model = tiny
    ref = gpt2_tiny.OracleGPT2(orc, w)
    ids = list(np.random.default_rng(4).integers(0, gpt2_tiny.VOCAB, 24))
    for i, t in enumerate(ids):
        got = model.forward(ids[: i + 1], reprime=(i == 0))
        want = ref.forward(ids[: i + 1], reprime=(i == 0))
        close(got, want, 2e-5 * max(1.0, float(np.abs(want).max())))


def test_gpt2_from_gguf_equals_the_model_built_from_arrays(fh, orc, tiny, tmp_path):
    """The tiny model written as a GPT-2 GGUF (the reference's export layout)
    and loaded through the library's reader, Q8_0 tensors uploaded from the
    file mapping: scores bit-identical to the model built from the arrays."""
    import ferrum_gguf
    import ferrum_hip

    w, model = tiny
    path = str(tmp_path / "tiny.gguf")
    ferrum_gguf.gpt2_gguf(w, gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN,
                          gpt2_tiny.CTX).write(path)
    m2 = ferrum_hip.GPT2Device.from_gguf(fh, path)
    try:
        assert (m2.vocab, m2.d, m2.heads, m2.layers, m2.ffn, m2.cap) == (
            gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX)
        ids = list(np.random.default_rng(8).integers(0, gpt2_tiny.VOCAB, 12))
        for i in range(len(ids)):
            z1 = model.forward(ids[: i + 1], reprime=(i == 0))
            z2 = m2.forward(ids[: i + 1], reprime=(i == 0))
            assert np.array_equal(z1, z2)
    finally:
        m2.free()


def test_tiny_gpt2_greedy_decode_matches_the_oracle(fh, orc, tiny):
    """The tiny configuration's run: 16-token prompt, 64 greedy tokens.  Each
    step's id must be the oracle's greedy id on the same window unless the
    oracle's top-2 gap there is below 1e-5 (then the runs may part)."""
    import ferrum_hip

    w, model = tiny
    prompt = list(np.random.default_rng(6).integers(0, gpt2_tiny.VOCAB, 16))
    scores = []

    def fwd(ids, reprime):
        z = model.forward(ids, reprime)
        scores.append(z)
        return z

    got = ferrum_hip.gpt2_decode(fh, fwd, prompt, 64, ferrum_hip.SamplingParams(temperature=0.0),
                                 ferrum_hip.Rng(1), gpt2_tiny.CTX)
    assert len(got) == 64
    ref = gpt2_tiny.OracleGPT2(orc, w)
    win = ferrum_hip.GPT2Window(gpt2_tiny.CTX, prompt)
    z = ref.forward(win.ids, True)
    for step, tok in enumerate(got):
        p = orc.ln_bridge(orc.softmax_rows(z)[0])
        want = int(np.argmax(p))
        if want != tok:
            top2 = np.sort(p)[-2:]
            assert top2[1] - top2[0] < 1e-5, (step, tok, want)
            break
        reprime = win.push(tok)
        z = ref.forward(win.ids, reprime)


def test_tiny_gpt2_sampled_decode_replays_on_the_oracle(fh, orc, tiny):
    import ferrum_hip

    w, model = tiny
    kw = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    prompt = list(np.random.default_rng(7).integers(0, gpt2_tiny.VOCAB, 16))
    got = ferrum_hip.gpt2_decode(fh, model.forward, prompt, 48, ferrum_hip.SamplingParams(**kw),
                                 ferrum_hip.Rng(5), gpt2_tiny.CTX)
    ref = gpt2_tiny.OracleGPT2(orc, w)
    win, rng, op = ferrum_hip.GPT2Window(gpt2_tiny.CTX, prompt), orc.Rng(5), orc.SamplingParams(**kw)
    z = ref.forward(win.ids, True)
    for step, tok in enumerate(got):
        want, info = orc.sample(orc.ln_bridge(orc.softmax_rows(z)[0]), op, win.ids, rng.next_u64())
        if want != tok:
            assert info.margin < 1e-4, (step, tok, want, info.margin)
            break
        reprime = win.push(tok)
        z = ref.forward(win.ids, reprime)


def test_config1_greedy_run_on_the_device(fh, orc):
    """BASELINE configs[0] as configured: the tiny GPT-2 with N(0, 0.02) random
    init (gpt2_tiny.make_config1_weights), a 16-token prompt of uniform random
    ids, 64 greedy tokens -- run with every step on the device
    (GPT2Device.generate: the one-launch stack, the head and the fused
    sampler) and through the host loop over forward().  Both runs agree, and
    every step's id is the oracle's greedy id on the same window unless the
    oracle's top-2 gap there is below 1e-5 (then the runs may part; the steps
    checked before that are counted)."""
    import ferrum_hip

    w = gpt2_tiny.make_config1_weights(orc, seed=1)
    model = ferrum_hip.GPT2Device.from_weights(fh, w, gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS,
                                               gpt2_tiny.LAYERS, gpt2_tiny.FFN, gpt2_tiny.CTX)
    try:
        assert model.stack is not None
        prompt = [int(t) for t in np.random.default_rng(16).integers(0, gpt2_tiny.VOCAB, 16)]
        greedy = ferrum_hip.SamplingParams(temperature=0.0)
        dev = model.generate(prompt, 64, greedy, ferrum_hip.Rng(1))
        host = ferrum_hip.gpt2_decode(fh, model.forward, prompt, 64, greedy, ferrum_hip.Rng(1), gpt2_tiny.CTX)
        assert len(dev) == 64 and dev == host
        ref = gpt2_tiny.OracleGPT2(orc, w)
        win = ferrum_hip.GPT2Window(gpt2_tiny.CTX, prompt)
        z = ref.forward(win.ids, True)
        checked = 0
        for step, tok in enumerate(dev):
            p = orc.ln_bridge(orc.softmax_rows(z)[0])
            want = int(np.argmax(p))
            if want != tok:
                top2 = np.sort(p)[-2:]
                assert top2[1] - top2[0] < 1e-5, (step, tok, want)
                break
            checked += 1
            reprime = win.push(tok)
            z = ref.forward(win.ids, reprime)
        print(f"config-1 greedy run: {checked} of 64 steps equal to the oracle's before any near-tie")
        assert checked >= 8
    finally:
        model.free()
