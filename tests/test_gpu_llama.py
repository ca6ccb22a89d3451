"""The Llama / Qwen block pieces on the GPU against the oracle: RmsNorm (with
the residual add), RoPE (NORM / NEOX, partial rotary, frequency factors,
linear scaling, a position per row), grouped-query attention over per-row KV
caches, SwiGLU, the row embedding, and a whole batched decode of tiny
Qwen2- and Llama-shaped models (ferrum_core llm.rs)."""
import numpy as np
import pytest

import llama_tiny

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


@pytest.mark.parametrize("rows,d,res", [(1, 896, False), (64, 896, True), (3, 4096, True), (2, 100, False)])
def test_rmsnorm_matches_oracle(fh, orc, rows, d, res):
    import torch

    import ferrum_hip

    rng = np.random.default_rng(rows + d)
    x = (rng.standard_normal((rows, d)) * rng.choice([1e-3, 1.0, 40.0], (rows, 1))).astype(np.float32)
    r = rng.standard_normal((rows, d)).astype(np.float32)
    w = rng.standard_normal(d).astype(np.float32)
    tx, tr, tw = dev(x), dev(r), dev(w)
    ts, out = dev(np.full((rows, d), np.nan, np.float32)), torch.empty((rows, d), device="cuda")
    ready()
    ferrum_hip.rmsnorm_async(fh, tx, tr if res else None, ts if res else None, rows, d, tw, 1e-6, out)
    h = (x + r).astype(np.float32) if res else x
    if res:
        assert np.array_equal(host(fh, ts), h)
    close(host(fh, out), orc.rmsnorm(h, w, 1e-6), 1e-5)


@pytest.mark.parametrize("rt", [0, 1])
@pytest.mark.parametrize("hd,rope_dim,ff,lf", [(64, 64, False, 1.0), (32, 16, False, 1.0), (16, 16, True, 1.0),
                                               (64, 64, False, 4.0)])
def test_rope_matches_oracle(fh, orc, rt, hd, rope_dim, ff, lf):
    import ferrum_hip

    rows, nh, ld = 3, 6, 6 * hd + 40  # rows of a wider q|k|v buffer
    rng = np.random.default_rng(hd * 7 + rope_dim + rt)
    x = (rng.standard_normal((rows, ld)) * 2).astype(np.float32)
    pos = np.array([0, 17, 1000], np.uint32)
    fac = (rng.uniform(0.5, 8.0, rope_dim // 2)).astype(np.float32) if ff else None
    tx = dev(x)
    ready()
    ferrum_hip.rope_async(fh, tx, rows, ld, nh, hd, rope_dim, dev(pos.view(np.int32)), 1e4, rt,
                          None if fac is None else dev(fac), lf)
    got = host(fh, tx)
    for r in range(rows):
        want = orc.rope(x[r, :nh * hd], nh, hd, rope_dim, int(pos[r]), 1e4, rt, fac, lf)
        np.testing.assert_allclose(got[r, :nh * hd], want, rtol=0, atol=2e-6 * 4)
        assert np.array_equal(got[r, nh * hd:], x[r, nh * hd:])  # past the heads: untouched


def test_rope_errors(fh):
    import ferrum_hip

    x, p = dev(np.zeros(64, np.float32)), dev(np.zeros(1, np.int32))
    ready()
    with pytest.raises(ferrum_hip.DimMismatch, match="must be even"):
        ferrum_hip.rope_async(fh, x, 1, 64, 2, 32, 7, p, 1e4, 0)
    with pytest.raises(ferrum_hip.DimMismatch, match="must be even"):
        ferrum_hip.rope_async(fh, x, 1, 64, 2, 32, 34, p, 1e4, 0)
    with pytest.raises(ferrum_hip.DimMismatch, match="finite and > 0"):
        ferrum_hip.rope_async(fh, x, 1, 64, 2, 32, 32, p, 1e4, 0, None, 0.0)
    with pytest.raises(ferrum_hip.FerrumHipError, match="rope_type"):
        ferrum_hip.rope_async(fh, x, 1, 64, 2, 32, 32, p, 1e4, 2)


@pytest.mark.parametrize("nh,nkv,hd,T", [(14, 2, 64, 140), (4, 4, 32, 40), (8, 1, 128, 300), (6, 2, 16, 70)])
def test_gqa_attention_matches_oracle(fh, orc, nh, nkv, hd, T):
    """Three sequences at different positions (starting at 0, 60 and 129 with
    zeroed caches), every step checked against the oracle."""
    import torch

    import ferrum_hip

    rows, cap = 3, T + 140
    qd, kvd = nh * hd, nkv * hd
    ld = qd + 2 * kvd
    start = [0, 60, 129]
    rng = np.random.default_rng(nh * T + hd)
    kc, vc = torch.zeros(rows * cap * kvd, device="cuda"), torch.zeros(rows * cap * kvd, device="cuda")
    ko = [np.zeros((cap, kvd), np.float32) for _ in range(rows)]
    vo = [np.zeros((cap, kvd), np.float32) for _ in range(rows)]
    out = torch.empty((rows, qd), device="cuda")
    for t in range(T):
        qkv = (rng.standard_normal((rows, ld)) * 1.5).astype(np.float32)
        pos = np.array([s + t for s in start], np.uint32)
        ready()
        ferrum_hip.gqa_attention_decode_async(fh, dev(qkv), ld, rows, nh, nkv, hd, kc, vc, cap,
                                              dev(pos.view(np.int32)), int(pos.max()), out)
        got = host(fh, out)
        for r in range(rows):
            close(got[r], orc.gqa_attention_decode(qkv[r], ko[r], vo[r], nh, nkv, hd, int(pos[r])), 1e-5)
    kh, vh = host(fh, kc).reshape(rows, cap, kvd), host(fh, vc).reshape(rows, cap, kvd)
    for r in range(rows):
        assert np.array_equal(kh[r], ko[r]) and np.array_equal(vh[r], vo[r])


@pytest.mark.parametrize("nh,nkv,rows", [(14, 2, 40), (32, 8, 10), (16, 2, 40), (6, 2, 40), (16, 16, 40),
                                         (12, 12, 10)])
def test_batched_gqa_attention_matches_oracle(fh, orc, nh, nkv, rows):
    """Launches with many (row, kv head) workgroups take the batched kernel
    (one workgroup per row, kv head and up to four query heads, every position
    merged inside it): groups of 7 (split 4 + 3), 4, 8 and 3 (split 2 + 1),
    and one query head per kv head (GPT-2's batched decode, which takes it
    for rows of 256 positions or more; 12 x 10 workgroups are too few and take
    the chunked kernel).
    Positions span the wave (32) and round (256) edges, 0 and the last cache
    row; two rows sit past max_pos and one at capacity (NaN, cache untouched).
    Cache rows from pos on hold NaN, so a row read past the position shows."""
    import torch

    import ferrum_hip

    hd, cap, max_pos = 64, 600, 580
    qd, kvd = nh * hd, nkv * hd
    ld = qd + 2 * kvd
    rng = np.random.default_rng(nh * 10 + nkv + rows)
    edges = [0, 1, 2, 30, 31, 32, 33, 63, 64, 255, 256, 257, 300, 511, 512, 513, 579, 580]
    pos = np.array([edges[r] if r < len(edges) else int(rng.integers(0, max_pos + 1)) for r in range(rows)], np.uint32)
    pos[rows - 3], pos[rows - 2], pos[rows - 1] = max_pos + 1, 599, cap  # past max_pos (twice), at capacity
    qkv = (rng.standard_normal((rows, ld)) * 1.5).astype(np.float32)
    kc0 = rng.standard_normal((rows, cap, kvd)).astype(np.float32)
    vc0 = rng.standard_normal((rows, cap, kvd)).astype(np.float32)
    for r in range(rows):
        kc0[r, min(int(pos[r]), cap):] = np.nan
        vc0[r, min(int(pos[r]), cap):] = np.nan
    kc, vc = dev(kc0.ravel()), dev(vc0.ravel())
    out = torch.empty((rows, qd), device="cuda")
    ready()
    ferrum_hip.gqa_attention_decode_async(fh, dev(qkv), ld, rows, nh, nkv, hd, kc, vc, cap, dev(pos.view(np.int32)),
                                          max_pos, out)
    got = host(fh, out)
    kh, vh = host(fh, kc).reshape(rows, cap, kvd), host(fh, vc).reshape(rows, cap, kvd)
    for r in range(rows):
        p = int(pos[r])
        if p > max_pos:
            assert np.isnan(got[r]).all()
            assert np.array_equal(kh[r].view(np.uint32), kc0[r].view(np.uint32))
            assert np.array_equal(vh[r].view(np.uint32), vc0[r].view(np.uint32))
            continue
        ko, vo = kc0[r].copy(), vc0[r].copy()
        want = orc.gqa_attention_decode(qkv[r], ko, vo, nh, nkv, hd, p)
        close(got[r], want, 1e-5)
        assert np.array_equal(kh[r, p], qkv[r, qd:qd + kvd]) and np.array_equal(vh[r, p], qkv[r, qd + kvd:])
        keep = np.arange(cap) != p
        assert np.array_equal(kh[r, keep].view(np.uint32), kc0[r, keep].view(np.uint32))


@pytest.mark.parametrize("nh,nkv,hd,rows,rt,rope_dim,ff,lf", [
    (14, 2, 64, 40, 1, 64, False, 1.0),   # one launch, rotation inside (group 7: 4 + 3 heads)
    (32, 8, 64, 10, 0, 48, True, 2.0),    # one launch, NORM pairs, partial rotary, factors, scaling
    (6, 2, 64, 40, 0, 64, False, 1.0),    # one launch, group 3 (2 + 1 heads)
    (14, 2, 64, 3, 1, 64, False, 1.0),    # few rows: fh_rope, then the attention
    (8, 2, 32, 50, 1, 32, False, 1.0),    # head width 32: fh_rope, then the attention
])
def test_attention_with_rope_equals_rope_then_attention(fh, orc, nh, nkv, hd, rows, rt, rope_dim, ff, lf):
    """fh_gqa_attention_rope_decode_async gives the bits of fh_rope_async on
    the q and k heads followed by fh_gqa_attention_decode_async, outputs and
    caches, whichever form it takes; a row past max_pos is NaN in both and
    leaves its cache alone."""
    import torch

    import ferrum_hip

    cap, max_pos = 600, 560
    qd, kvd = nh * hd, nkv * hd
    ld = qd + 2 * kvd + 8  # rows of a wider buffer
    rng = np.random.default_rng(nh + rows * 3 + rt)
    edges = [0, 1, 31, 32, 255, 256, 300, 511, 512, 560]
    pos = np.array([edges[r] if r < len(edges) else int(rng.integers(0, max_pos + 1)) for r in range(rows)], np.uint32)
    pos[-1] = max_pos + 3
    qkv = (rng.standard_normal((rows, ld)) * 1.5).astype(np.float32)
    kc0 = rng.standard_normal(rows * cap * kvd).astype(np.float32)
    vc0 = rng.standard_normal(rows * cap * kvd).astype(np.float32)
    fac = dev(rng.uniform(0.5, 8.0, rope_dim // 2).astype(np.float32)) if ff else None
    dpos = dev(pos.view(np.int32))
    outs, caches = [], []
    for fused in (False, True):
        x, kc, vc = dev(qkv), dev(kc0), dev(vc0)
        out = torch.empty((rows, qd), device="cuda")
        ready()
        if fused:
            ferrum_hip.gqa_attention_rope_decode_async(fh, x, ld, rows, nh, nkv, hd, kc, vc, cap, dpos, max_pos,
                                                       rope_dim, 1e6, rt, fac, lf, out)
        else:
            ferrum_hip.rope_async(fh, x, rows, ld, nh + nkv, hd, rope_dim, dpos, 1e6, rt, fac, lf)
            ferrum_hip.gqa_attention_decode_async(fh, x, ld, rows, nh, nkv, hd, kc, vc, cap, dpos, max_pos, out)
        outs.append(host(fh, out))
        caches.append((host(fh, kc), host(fh, vc)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for a, b in zip(caches[0], caches[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.isnan(outs[1][-1]).all() and not np.isnan(outs[1][:-1]).any()
    kh = caches[1][0].reshape(rows, cap, kvd)
    assert np.array_equal(kh[-1], kc0.reshape(rows, cap, kvd)[-1])
    # row 1 against the oracle: RoPE'd q|k, then the attention
    q = qkv[1, :qd + 2 * kvd].copy()
    f = None if fac is None else host(fh, fac)
    q[:qd + kvd] = orc.rope(q[:qd + kvd], nh + nkv, hd, rope_dim, int(pos[1]), 1e6, rt, f, lf)
    ko, vo = kc0.reshape(rows, cap, kvd)[1].copy(), vc0.reshape(rows, cap, kvd)[1].copy()
    close(outs[1][1], orc.gqa_attention_decode(q, ko, vo, nh, nkv, hd, int(pos[1])), 1e-5)


def test_attention_with_rope_errors(fh):
    import ferrum_hip

    x, c, p, o = (dev(np.zeros(n, np.float32)) for n in (256, 4096, 1, 256))
    ready()
    call = ferrum_hip.gqa_attention_rope_decode_async
    with pytest.raises(ferrum_hip.DimMismatch, match="must be even"):
        call(fh, x, 192, 1, 2, 1, 64, c, c, 8, p, 0, 63, 1e4, 0, None, 1.0, o)
    with pytest.raises(ferrum_hip.DimMismatch, match="finite and > 0"):
        call(fh, x, 192, 1, 2, 1, 64, c, c, 8, p, 0, 64, 1e4, 0, None, float("inf"), o)
    with pytest.raises(ferrum_hip.DimMismatch, match="multiple of n_kv_heads"):
        call(fh, x, 192, 1, 3, 2, 32, c, c, 8, p, 0, 32, 1e4, 0, None, 1.0, o)
    with pytest.raises(ferrum_hip.FerrumHipError, match="rope_type"):
        call(fh, x, 192, 1, 2, 1, 64, c, c, 8, p, 0, 64, 1e4, 5, None, 1.0, o)


@pytest.mark.parametrize("nh,nkv,hd", [(14, 2, 64), (32, 8, 128), (4, 2, 32), (12, 2, 64), (16, 2, 32)])
def test_grouped_attention_equals_the_per_head_kernel(fh, orc, nh, nkv, hd):
    """The grouped-query kernel (one workgroup per kv head's query heads, K
    and V loaded once) gives the per-head kernel's bits: the same query heads
    run with every kv head repeated for each of its query heads (n_kv =
    n_heads).  Rows at positions 0, 40, 200 and 700 (a launch reaching 384
    positions takes the grouped kernel: one chunk, several, the merge over
    many), cache rows seeded below them; the new k / v rows land in the cache
    as the expanded run writes them."""
    import torch

    import ferrum_hip

    rows, cap, grp = 4, 720, nh // nkv
    qd, kvd = nh * hd, nkv * hd
    rng = np.random.default_rng(nh * hd + nkv)
    qkv = (rng.standard_normal((rows, qd + 2 * kvd)) * 1.5).astype(np.float32)
    kc0 = rng.standard_normal((rows, cap, nkv, hd)).astype(np.float32)
    vc0 = rng.standard_normal((rows, cap, nkv, hd)).astype(np.float32)
    pos = np.array([0, 40, 200, 700], np.uint32)
    # the same inputs with kv head j repeated for its query heads j * grp ..
    k_new = qkv[:, qd:qd + kvd].reshape(rows, nkv, hd)
    v_new = qkv[:, qd + kvd:].reshape(rows, nkv, hd)
    qkv_e = np.concatenate([qkv[:, :qd], np.repeat(k_new, grp, axis=1).reshape(rows, qd),
                            np.repeat(v_new, grp, axis=1).reshape(rows, qd)], axis=1)
    kc, vc = dev(kc0.ravel()), dev(vc0.ravel())
    kce, vce = dev(np.repeat(kc0, grp, axis=2).ravel()), dev(np.repeat(vc0, grp, axis=2).ravel())
    out, out_e = torch.empty((rows, qd), device="cuda"), torch.empty((rows, qd), device="cuda")
    dpos = dev(pos.view(np.int32))
    ready()
    ferrum_hip.gqa_attention_decode_async(fh, dev(qkv), qd + 2 * kvd, rows, nh, nkv, hd, kc, vc, cap, dpos,
                                          int(pos.max()), out)
    ferrum_hip.gqa_attention_decode_async(fh, dev(qkv_e), 3 * qd, rows, nh, nh, hd, kce, vce, cap, dpos,
                                          int(pos.max()), out_e)
    got, want = host(fh, out), host(fh, out_e)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    kh = host(fh, kc).reshape(rows, cap, nkv, hd)
    keh = host(fh, kce).reshape(rows, cap, nh, hd)
    for r in range(rows):
        assert np.array_equal(kh[r, pos[r]], k_new[r]) and np.array_equal(keh[r, pos[r]], np.repeat(k_new[r], grp, 0))
        close(got[r], orc.gqa_attention_decode(qkv[r], kc0[r].reshape(cap, kvd), vc0[r].reshape(cap, kvd),
                                               nh, nkv, hd, int(pos[r])), 1e-5)


def test_gqa_attention_bad_positions_give_nan_and_leave_the_cache(fh, orc):
    import torch

    import ferrum_hip

    rows, nh, nkv, hd, cap = 3, 4, 2, 32, 100
    qd, kvd = nh * hd, nkv * hd
    ld = qd + 2 * kvd
    qkv = np.random.default_rng(1).standard_normal((rows, ld)).astype(np.float32)
    kc, vc = torch.zeros(rows * cap * kvd, device="cuda"), torch.zeros(rows * cap * kvd, device="cuda")
    out = torch.empty((rows, qd), device="cuda")
    pos = np.array([5, 100, 70], np.uint32)  # fine, at capacity, above max_pos
    ready()
    ferrum_hip.gqa_attention_decode_async(fh, dev(qkv), ld, rows, nh, nkv, hd, kc, vc, cap, dev(pos.view(np.int32)),
                                          40, out)
    got = host(fh, out)
    ko, vo = np.zeros((cap, kvd), np.float32), np.zeros((cap, kvd), np.float32)
    close(got[0], orc.gqa_attention_decode(qkv[0], ko, vo, nh, nkv, hd, 5), 1e-5)
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()
    kh = host(fh, kc).reshape(rows, cap, kvd)
    assert not kh[1].any() and not kh[2].any()
    with pytest.raises(ferrum_hip.DimMismatch, match="multiple of n_kv_heads"):
        ferrum_hip.gqa_attention_decode_async(fh, dev(qkv), ld, rows, 3, 2, hd, kc, vc, cap, dev(pos.view(np.int32)),
                                              40, out)


@pytest.mark.parametrize("rows,n,ld", [(1, 4864, 4864), (64, 4864, 9728), (3, 100, 256)])
def test_swiglu_matches_oracle(fh, orc, rows, n, ld):
    import torch

    import ferrum_hip

    rng = np.random.default_rng(n + rows)
    g = (rng.standard_normal((rows, ld)) * 4).astype(np.float32)
    u = rng.standard_normal((rows, ld)).astype(np.float32)
    out = torch.empty((rows, n), device="cuda")
    ready()
    ferrum_hip.swiglu_async(fh, dev(g), dev(u), rows, n, ld, out)
    close(host(fh, out), orc.swiglu(g[:, :n], u[:, :n]), 1e-5)


def test_embed_rows_copies_rows_and_poisons_bad_ids(fh):
    import torch

    import ferrum_hip

    tw = np.random.default_rng(2).standard_normal((50, 24)).astype(np.float32)
    toks = np.array([3, 49, 50, 0], np.uint32)
    out = torch.empty((4, 24), device="cuda")
    ready()
    ferrum_hip.embed_rows_async(fh, dev(tw), 50, 24, dev(toks.view(np.int32)), 4, out)
    got = host(fh, out)
    assert np.array_equal(got[[0, 1, 3]], tw[[3, 49, 0]]) and np.isnan(got[2]).all()


@pytest.mark.parametrize("name,biases,tied", [("QWEN", True, True), ("LLAMA", False, False)])
def test_tiny_model_batched_decode_matches_the_oracle(fh, orc, name, biases, tied):
    """Three sequences starting at positions 0, 5 and 11 (zeroed caches), 14
    teacher-forced steps: every row's scores at every step against the oracle."""
    import ferrum_hip

    cfg = getattr(llama_tiny, name)
    w = llama_tiny.make_weights(orc, cfg, 21, biases, tied)
    rows, start = 3, [0, 5, 11]
    m = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, rows)
    refs = [llama_tiny.OracleLlamaRow(orc, w, cfg, s) for s in start]
    toks = np.random.default_rng(5).integers(0, cfg["vocab"], (14, rows))
    try:
        for t in range(14):
            m.tokens.copy_(dev(toks[t].astype(np.int32)))
            m.pos.copy_(dev(np.array([s + t for s in start], np.int32)))
            ready()
            m.feed_async(start[-1] + t)
            got = host(fh, m.z)
            for r in range(rows):
                want = refs[r].feed(toks[t, r])
                close(got[r], want, 2e-5 * max(1.0, float(np.abs(want).max())))
    finally:
        m.free()


def test_tiny_qwen_greedy_batch_runs_on_the_device(fh, orc):
    """A batch of 4 greedy decodes with the token and position fed back on the
    device (sampler -> tokens, pos + 1) replays on the oracle: each id is the
    oracle's argmax unless its top-2 gap is below 1e-5."""
    import torch

    import ferrum_hip

    cfg = llama_tiny.QWEN
    w = llama_tiny.make_weights(orc, cfg, 23, True, True)
    rows = 4
    m = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, rows)
    refs = [llama_tiny.OracleLlamaRow(orc, w, cfg, 0) for _ in range(rows)]
    first = np.random.default_rng(9).integers(0, cfg["vocab"], rows)
    m.tokens.copy_(dev(first.astype(np.int32)))
    off = dev(np.zeros(rows + 1, np.int32))
    greedy = ferrum_hip.SamplingParams(temperature=0.0)
    out = torch.zeros(rows, dtype=torch.int32, device="cuda")
    want_tok = [int(t) for t in first]
    live = [True] * rows
    try:
        for t in range(20):
            ready()
            m.feed_async(t)
            ferrum_hip.sample_rows_async(fh, m.z, rows, cfg["vocab"], greedy, None, off, None, out)
            got = host(fh, out).astype(np.int64)
            for r in range(rows):
                if not live[r]:
                    continue
                z = refs[r].feed(want_tok[r])
                want = int(np.argmax(z))
                if want != got[r]:
                    top2 = np.sort(z)[-2:]
                    assert top2[1] - top2[0] < 1e-5, (t, r, int(got[r]), want)
                    live[r] = False
                want_tok[r] = want
            m.tokens.copy_(out)
            m.pos.add_(1)
    finally:
        m.free()


def test_tiny_qwen_generate_replays_on_the_oracle(fh, orc):
    """LlamaModel::generate_inner's loop (llm.rs:706-754, ferrum_hip.llama_decode)
    driving the device decoder: a 6-token prompt, sampled ids (temperature,
    top-k, top-p, repetition penalty over every prompt and generated id) with
    draws from the reference's Rng.  Replayed on the oracle model and sampler
    with the same draws: the same scores at every position (2e-5 of the row's
    largest) and the same ids unless the oracle reports a near-tie margin."""
    import ferrum_hip

    cfg = llama_tiny.QWEN
    w = llama_tiny.make_weights(orc, cfg, 29, True, True)
    m = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, 1)
    scores = []

    def fwd(tok):
        z = m.forward_one(tok)
        scores.append(z)
        return z

    kw = dict(temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.05)
    prompt = list(np.random.default_rng(12).integers(0, cfg["vocab"], 6))
    try:
        got = ferrum_hip.llama_decode(fh, fwd, prompt, 30, ferrum_hip.SamplingParams(**kw), ferrum_hip.Rng(4),
                                      context_len=cfg["context"])
    finally:
        m.free()
    assert len(got) == 30
    ref = llama_tiny.OracleLlamaRow(orc, w, cfg, 0)
    for i, t in enumerate(prompt[:-1]):
        close(scores[i], ref.feed(t), 2e-5 * max(1.0, float(np.abs(scores[i]).max())))
    recent, op, rng = list(prompt), orc.SamplingParams(**kw), orc.Rng(4)
    z = ref.feed(prompt[-1])
    for step, tok in enumerate(got):
        zg = scores[len(prompt) - 1 + step]
        close(zg, z, 2e-5 * max(1.0, float(np.abs(z).max())))
        want, info = orc.sample(z, op, recent, rng.next_u64())
        if want != tok:
            assert info.margin < 1e-5, (step, tok, want, info.margin)
            break
        recent.append(tok)
        if step + 1 < len(got):
            z = ref.feed(tok)


def test_qwen2_05b_step_matches_oracle(fh, orc):
    """BASELINE configs[4] at its own depth: the Qwen2-0.5B shape (24 blocks,
    d 896, 14 / 2 heads of 64, SwiGLU 4864, vocabulary 151936, q/k/v biases,
    tied head; N(0, 0.02) Q8_0 weights) as LlamaModel::forward_one walks it
    (llm.rs:606-616) for three sequences at positions 0, 97 and 255 whose
    caches hold seeded rows before that position, two steps each (the second
    reads the row the first wrote).  Every row's logits against the oracle's
    within 1e-5 of the row's largest, and all of them anchored to the float64
    step (accuracy_against_f64)."""
    import torch

    import ferrum_hip
    from accuracy import accuracy_against_f64

    cfg = llama_tiny.QWEN05
    w = llama_tiny.make_weights(orc, cfg, 31, True, True, std=0.02)
    rows, start, cap = 3, [0, 97, 255], cfg["context"]
    kvd = cfg["n_kv"] * cfg["head_dim"]
    m = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, rows)
    try:
        refs = [llama_tiny.OracleLlamaRow(orc, w, cfg, s) for s in start]
        kc = [[np.zeros((cap, kvd)) for _ in range(rows)] for _ in range(cfg["layers"])]
        vc = [[np.zeros((cap, kvd)) for _ in range(rows)] for _ in range(cfg["layers"])]
        rng = np.random.default_rng(77)
        for i, b in enumerate(m.blocks):
            kd, vd = b["k"].view(rows, cap, kvd), b["v"].view(rows, cap, kvd)
            for r, s in enumerate(start):
                kk = rng.standard_normal((s, kvd), dtype=np.float32)
                vv = rng.standard_normal((s, kvd), dtype=np.float32)
                refs[r].k[i][:s], refs[r].v[i][:s] = kk, vv
                kc[i][r][:s], vc[i][r][:s] = kk, vv
                kd[r, :s] = torch.from_numpy(kk).cuda()
                vd[r, :s] = torch.from_numpy(vv).cuda()
        got_all, want_all, exact_all = [], [], []
        for t in range(2):
            toks = rng.integers(0, cfg["vocab"], rows)
            pos = [s + t for s in start]
            m.tokens.copy_(dev(toks.astype(np.int32)))
            m.pos.copy_(dev(np.array(pos, np.int32)))
            ready()
            m.feed_async(max(pos))
            got = host(fh, m.z)
            exact = llama_tiny.step_f64(orc, w, cfg, toks, pos, kc, vc)
            for r in range(rows):
                want = refs[r].feed(toks[r])
                err = float(np.abs(got[r].astype(np.float64) - want).max())
                print(f"qwen2-0.5b step {t} row {r} (position {pos[r]}): max |diff| {err:.3e}, "
                      f"max |logit| {np.abs(want).max():.3e}")
                assert err <= 1e-5 * np.abs(want).max(), (t, r, err)
                got_all.append(got[r])
                want_all.append(want)
                exact_all.append(exact[r])
        accuracy_against_f64(np.stack(got_all), np.stack(want_all), np.stack(exact_all), "qwen2-0.5b step")
    finally:
        m.free()
