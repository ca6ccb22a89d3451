"""Batched GPT-2 decode (ferrum_hip.GPT2Batch): `rows` sequences, each its own
CachedTransformer (slm/cached.rs:100-137) with its own KV caches and token
window, stepped together with the linears as GEMMs over the rows -- the
batched decode behind BASELINE's b32 figure and configs[3].  Each row must
replay on the oracle's single-sequence model and sampler
(slm/token_stream.rs:66-190, slm/sampling.rs:124-210) with the row's own
draws; the batched embedding (fh_embed_rows_pos_async) against embed_one."""
import numpy as np
import pytest

import gpt2_tiny

pytestmark = pytest.mark.gpu

CONFIG3 = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
G124 = dict(vocab=50257, d=768, heads=12, layers=12, ffn=3072, ctx=1024)


def device_model(fh, w, cfg):
    import ferrum_hip

    return ferrum_hip.GPT2Device.from_weights(fh, w, cfg["vocab"], cfg["d"], cfg["heads"], cfg["layers"], cfg["ffn"],
                                              cfg["ctx"])


TINY = dict(vocab=gpt2_tiny.VOCAB, d=gpt2_tiny.D, heads=gpt2_tiny.HEADS, layers=gpt2_tiny.LAYERS, ffn=gpt2_tiny.FFN,
            ctx=gpt2_tiny.CTX)


@pytest.fixture(scope="module")
def tiny(fh, orc):
    w = gpt2_tiny.make_weights(orc)
    m = device_model(fh, w, TINY)
    yield w, m
    m.free()


def replay_rows(orc, w, cfg, prompts, ids, params_kw, seeds):
    """Every row's run replayed on the oracle: its own window and Rng(seed).
    A differing id must lie within the sampler's margins; the replay goes on
    from the device's id.  Returns the number of such steps."""
    import ferrum_hip
    from sampler_margins import exempt

    greedy = params_kw.get("temperature", 1.0) <= 0.0
    op = orc.SamplingParams(**params_kw)
    n_exempt = 0
    for r, prompt in enumerate(prompts):
        ref = gpt2_tiny.OracleGPT2(orc, w, **{k: cfg[k] for k in ("vocab", "d", "heads", "layers", "ffn")},
                                   ctx=cfg["ctx"])
        win, rng = ferrum_hip.GPT2Window(cfg["ctx"], list(prompt)), orc.Rng(seeds[r])
        z = ref.forward(win.ids, True)
        for step, tok in enumerate(ids[r]):
            draw = 0 if greedy else rng.next_u64()
            want, info = orc.sample(orc.ln_bridge(orc.softmax_rows(z)[0]), op, win.ids, draw)
            if want != tok:
                assert exempt(info, greedy), (r, step, tok, want)
                n_exempt += 1
            win.push(tok)
            z = ref.forward(win.ids, False)
    return n_exempt


def test_embed_rows_pos_matches_embed_one(fh, orc, tiny):
    """Rows at their own positions against embed_one; an id past the
    vocabulary poisons its row; the history records each row's id at its
    position and skips a position past the stride."""
    import torch

    import ferrum_hip

    w, m = tiny
    toks = np.array([3, 4095, 0, 4096, 17], np.int32)
    pos = np.array([0, 255, 7, 3, 200], np.int32)
    out = torch.empty((5, m.d), device="cuda")
    hist = torch.full((5, 201), -1, dtype=torch.int32, device="cuda")
    d_t, d_p = torch.from_numpy(toks).cuda(), torch.from_numpy(pos).cuda()
    torch.cuda.synchronize()
    ferrum_hip.embed_rows_pos_async(fh, m.tok_w, m.pos_w, m.vocab, m.pos_w.shape[0], m.d, d_t, d_p, 5, out, hist, 201)
    fh.sync()
    got, h = out.cpu().numpy(), hist.cpu().numpy()
    tok_w = m.tok_w.cpu().numpy()
    pos_w = np.asarray(w["position_embd"], np.float32).reshape(-1, m.d)
    for r in range(5):
        if toks[r] >= m.vocab:
            assert np.isnan(got[r]).all()
        else:
            assert np.array_equal(got[r], orc.embed_one(tok_w, pos_w, int(toks[r]), int(pos[r])))
    for r in range(5):
        marks = np.flatnonzero(h[r] != -1)
        if pos[r] < 201:
            assert list(marks) == [pos[r]] and h[r, pos[r]] == toks[r]
        else:
            assert marks.size == 0


def test_tiny_batch_runs_replay_on_the_oracle(fh, orc, tiny):
    """Four rows, 24-token prompts, eight steps: sampled with config-3
    parameters (each row its own Rng) and greedy; primed in one pass and
    position by position (the same ids); every row replays on the oracle."""
    import ferrum_hip

    w, m = tiny
    B = 4
    rng = np.random.default_rng(40)
    prompts = rng.integers(0, gpt2_tiny.VOCAB, size=(B, 24))
    batch = ferrum_hip.GPT2Batch(m, B, 64)
    seeds = [101 + r for r in range(B)]
    params = ferrum_hip.SamplingParams(**CONFIG3)
    ids = batch.generate(prompts, 8, params, [ferrum_hip.Rng(s) for s in seeds])
    assert all(len(r) == 8 for r in ids)
    slow = batch.generate(prompts, 8, params, [ferrum_hip.Rng(s) for s in seeds], prefill=False)
    assert replay_rows(orc, w, TINY, prompts, ids, CONFIG3, seeds) <= 1
    assert replay_rows(orc, w, TINY, prompts, slow, CONFIG3, seeds) <= 1
    g = batch.generate(prompts, 8, ferrum_hip.SamplingParams(0.0), [])
    assert replay_rows(orc, w, TINY, prompts, g, dict(temperature=0.0), seeds) <= 1


def test_batch_rows_equal_the_single_sequence_path(fh, orc, tiny):
    """A row of a batch and the same sequence through GPT2Device.generate
    (the one-launch stack): same ids (both replay on the oracle), and a
    one-row batch (the m = 1 GEMV path) as well."""
    import ferrum_hip

    w, m = tiny
    rng = np.random.default_rng(41)
    prompts = rng.integers(0, gpt2_tiny.VOCAB, size=(3, 12))
    params = ferrum_hip.SamplingParams(**CONFIG3)
    batch = ferrum_hip.GPT2Batch(m, 3, 40)
    ids = batch.generate(prompts, 6, params, [ferrum_hip.Rng(7 + r) for r in range(3)])
    one = ferrum_hip.GPT2Batch(m, 1, 40)
    for r in range(3):
        single = m.generate([int(t) for t in prompts[r]], 6, params, ferrum_hip.Rng(7 + r))
        solo = one.generate(prompts[r:r + 1], 6, params, [ferrum_hip.Rng(7 + r)])[0]
        assert single == ids[r] == solo, (r, single, ids[r], solo)


def test_batch_errors(fh, tiny):
    import ferrum_hip

    _, m = tiny
    batch = ferrum_hip.GPT2Batch(m, 2, 16)
    with pytest.raises(ferrum_hip.DimMismatch, match="capacity"):
        batch.generate(np.zeros((2, 10), np.int64), 7, ferrum_hip.SamplingParams(0.0), [])
    with pytest.raises(ferrum_hip.FerrumHipError, match="prompts"):
        batch.generate(np.zeros((3, 4), np.int64), 2, ferrum_hip.SamplingParams(0.0), [])
    with pytest.raises(ferrum_hip.DimMismatch, match="max_seq_len"):
        ferrum_hip.GPT2Batch(m, 2, gpt2_tiny.CTX + 1)
    fh.sync()


def test_gpt2_124m_batch_replays_on_the_oracle(fh, orc):
    """GPT-2-124M shape (N(0, 0.02) Q8_0 weights): three rows with 40-token
    prompts primed in one pass, then five config-3 steps; every row replays
    on the oracle."""
    import ferrum_hip

    w = gpt2_tiny.make_weights(orc, seed=3, vocab=G124["vocab"], d=G124["d"], layers=G124["layers"],
                               ffn=G124["ffn"], ctx=G124["ctx"], std=0.02)
    m = device_model(fh, w, G124)
    try:
        prompts = np.random.default_rng(42).integers(0, G124["vocab"], size=(3, 40))
        batch = ferrum_hip.GPT2Batch(m, 3, 64)
        seeds = [51, 52, 53]
        ids = batch.generate(prompts, 5, ferrum_hip.SamplingParams(**CONFIG3), [ferrum_hip.Rng(s) for s in seeds])
        n = replay_rows(orc, w, G124, prompts, ids, CONFIG3, seeds)
        print(f"124M batch: 3 rows x 5 steps, {n} exempt")
        assert n <= 1
    finally:
        m.free()


def test_gpt2_medium_batch32_rows_equal_single_runs(fh):
    """configs[3]'s shape (GPT-2-medium: 24 blocks, d = 1024, 16 heads, FFN
    4096; N(0, 0.02) weights made on the device) at batch 32: 32 prompts of
    48 ids primed in one pass (GEMMs at m = 32 x 47), then six greedy steps;
    rows 0, 13 and 31 equal the same prompts run alone through
    GPT2Device.generate."""
    import torch

    import ferrum_hip

    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    m = ferrum_hip.GPT2Device.random(fh, 50257, 1024, 16, 24, 4096, 128, gen)
    try:
        prompts = np.random.default_rng(43).integers(0, 50257, size=(32, 48))
        batch = ferrum_hip.GPT2Batch(m, 32, 64)
        ids = batch.generate(prompts, 6, ferrum_hip.SamplingParams(0.0), [])
        assert len(ids) == 32 and all(len(r) == 6 for r in ids)
        for r in (0, 13, 31):
            assert ids[r] == m.generate([int(t) for t in prompts[r]], 6, ferrum_hip.SamplingParams(0.0),
                                        ferrum_hip.Rng(1)), r
    finally:
        m.free()
