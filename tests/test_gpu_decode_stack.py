"""The one-launch GPT-2 block stack (fh_gpt2_stack_*, csrc/fh_decode.hip)
against the oracle's CachedTransformer::feed (slm/cached.rs:100-125,
layer/transformer.rs:221-290) and against the one-launch-per-op device path:
the tiny configuration and the GPT-2-124M shape (12
blocks, d = 768, 12 heads, N(0, 0.02) Q8_0 weights) across positions that
span several 64-position attention items per head; HIP graph replays (the
stack's launch counters); the reference's position errors; a failed exchange
forced from the host, reported and recovered from."""
import numpy as np
import pytest

import gpt2_tiny
from accuracy import accuracy_against_f64

pytestmark = pytest.mark.gpu

G124 = dict(vocab=50257, d=768, heads=12, layers=12, ffn=3072, ctx=1024)


def device_model(fh, w, cfg):
    import ferrum_hip

    return ferrum_hip.GPT2Device.from_weights(fh, w, cfg["vocab"], cfg["d"], cfg["heads"], cfg["layers"], cfg["ffn"],
                                              cfg["ctx"])


def feed(model, tok, pos, fused):
    import torch

    model.fused = fused
    model.token.fill_(int(tok))
    torch.cuda.synchronize()
    model.feed_async(model.token, pos)
    model.ctx.sync()
    torch.cuda.synchronize()
    return model.z.cpu().numpy().copy()


def assert_scores_close(got, want, what, rel=2e-5):
    """|got - want| <= rel * max|want| over the row (the device sums in other
    orders than the oracle, through every block)."""
    err = np.abs(np.asarray(got, np.float64) - want).max()
    scale = np.abs(want).max()
    assert err <= rel * scale, f"{what}: max |diff| {err:.3e} against max |score| {scale:.3e}"


@pytest.fixture(scope="module")
def tiny_pair(fh, orc):
    w = gpt2_tiny.make_weights(orc)
    m = device_model(fh, w, dict(vocab=gpt2_tiny.VOCAB, d=gpt2_tiny.D, heads=gpt2_tiny.HEADS,
                                 layers=gpt2_tiny.LAYERS, ffn=gpt2_tiny.FFN, ctx=gpt2_tiny.CTX))
    yield w, m
    m.free()


def test_tiny_stack_matches_oracle_and_per_op_path(fh, orc, tiny_pair):
    """Positions 0 .. 149 (three attention items per head at the end): the
    stack's scores against the oracle's, and against the one-launch-per-op
    path fed the same tokens into its own cache."""
    w, m = tiny_pair
    assert m.stack is not None and m.launches_per_step() == 2
    ref = gpt2_tiny.OracleGPT2(orc, w)
    ids = np.random.default_rng(21).integers(0, gpt2_tiny.VOCAB, 150)
    per_op = [feed(m, t, p, False) for p, t in enumerate(ids)]  # fills the cache the per-op way
    for p, t in enumerate(ids):
        z = feed(m, t, p, True)                                   # rewrites row p, reads rows < p
        want = ref.feed(t)
        assert_scores_close(z, want, f"stack at position {p}")
        assert_scores_close(z, per_op[p], f"stack vs per-op at position {p}")


@pytest.fixture(scope="module")
def g124(fh, orc):
    w = gpt2_tiny.make_weights(orc, seed=3, vocab=G124["vocab"], d=G124["d"], layers=G124["layers"],
                               ffn=G124["ffn"], ctx=G124["ctx"], std=0.02)
    m = device_model(fh, w, G124)
    yield w, m
    m.free()


def test_gpt2_124m_stack_matches_oracle(fh, orc, g124):
    """GPT-2-124M shape with N(0, 0.02) weights: 300 positions through the
    stack (up to five 64-position attention items per head, so past position
    256 some of the 48 workgroups take two), every position's scores against
    the oracle's within 1e-5 of the row's largest score, and all 300 x 50257
    scores anchored to the float64 forward (accuracy_against_f64)."""
    w, m = g124
    assert m.stack is not None
    cfg = {k: G124[k] for k in ("vocab", "d", "heads", "layers", "ffn")}
    ref = gpt2_tiny.OracleGPT2(orc, w, **cfg, ctx=G124["ctx"])
    ids = np.random.default_rng(5).integers(0, G124["vocab"], 300)
    got, want = [], []
    worst = 0.0
    for p, t in enumerate(ids):
        z, zr = feed(m, t, p, True), ref.feed(t)
        worst = max(worst, float(np.abs(z.astype(np.float64) - zr).max() / np.abs(zr).max()))
        assert_scores_close(z, zr, f"124M stack at position {p}", 1e-5)
        got.append(z)
        want.append(zr)
    print(f"124M stack: largest |diff| / max|score| over 300 positions {worst:.3e}")
    exact = gpt2_tiny.full_forward_f64(orc, w, [int(t) for t in ids], **cfg)
    accuracy_against_f64(np.stack(got), np.stack(want), exact, "124M stack, positions 0-299")


def test_gpt2_124m_stack_agrees_with_per_op_path(fh, orc, g124):
    """300 positions through both device paths (each re-primed from 0): past
    position 256 a head has five attention items and some of the stack's 48
    workgroups take two (the second item forms its head's q on the spot)."""
    w, m = g124
    ids = np.random.default_rng(6).integers(0, G124["vocab"], 300)
    a = [feed(m, t, p, True) for p, t in enumerate(ids)]
    b = [feed(m, t, p, False) for p, t in enumerate(ids)]
    for p in (0, 1, 63, 64, 65, 69, 191, 192, 255, 256, 257, 299):
        assert_scores_close(a[p], b[p], f"position {p}")


def test_gpt2_medium_stack_matches_oracle(fh, orc):
    """The d = 1024 instance (GPT-2-medium, BASELINE configs[3]'s shape: 24
    blocks, 16 heads, FFN 4096, vocabulary 50257; N(0, 0.02) Q8_0 weights):
    70 positions through the stack (two attention items per head at the end),
    every position's scores against the oracle's within 1e-5 of the row's
    largest, all of them anchored to the float64 forward, and the stack
    against the one-launch-per-op path at item boundaries."""
    cfg = dict(vocab=50257, d=1024, heads=16, layers=24, ffn=4096)
    w = gpt2_tiny.make_weights(orc, seed=17, ctx=128, std=0.02, **{k: cfg[k] for k in ("vocab", "d", "layers", "ffn")})
    m = device_model(fh, w, dict(cfg, ctx=128))
    try:
        assert m.stack is not None
        ref = gpt2_tiny.OracleGPT2(orc, w, **cfg, ctx=128)
        ids = np.random.default_rng(8).integers(0, cfg["vocab"], 70)
        got, want = [], []
        for p, t in enumerate(ids):
            z, zr = feed(m, t, p, True), ref.feed(t)
            assert_scores_close(z, zr, f"medium stack at position {p}", 1e-5)
            got.append(z)
            want.append(zr)
        exact = gpt2_tiny.full_forward_f64(orc, w, [int(t) for t in ids], **cfg)
        accuracy_against_f64(np.stack(got), np.stack(want), exact, "medium stack, positions 0-69")
        b = [feed(m, t, p, False) for p, t in enumerate(ids)]
        for p in (0, 1, 31, 63, 64, 65, 69):
            assert_scores_close(got[p], b[p], f"medium stack vs per-op, position {p}")
    finally:
        m.free()


def test_stack_replays_in_a_graph(fh, orc, tiny_pair):
    """The launch counters advance per replay: replays of a captured step give
    the eager result, with eager work between them."""
    import torch

    import ferrum_hip

    w, m = tiny_pair
    ids = np.random.default_rng(8).integers(0, gpt2_tiny.VOCAB, 40)
    for p, t in enumerate(ids[:-1]):
        feed(m, t, p, True)
    pos = len(ids) - 1
    want = feed(m, ids[-1], pos, True)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    m.token.fill_(int(ids[-1]))
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fh.set_stream(torch.cuda.current_stream().cuda_stream)
        m.feed_async(m.token, pos)
    fh.set_stream(None)
    try:
        for rep in range(4):
            m.z.zero_()
            g.replay()
            torch.cuda.synchronize()
            fh.sync()
            assert np.array_equal(m.z.cpu().numpy(), want), rep
            feed(m, ids[-1], pos, True)  # eager launches between replays
    finally:
        del g
    assert isinstance(ferrum_hip.GPT2Device, type)


def test_stack_position_errors(fh, tiny_pair):
    import ferrum_hip

    _, m = tiny_pair
    with pytest.raises(ferrum_hip.DimMismatch, match="exceeds max_seq_len|KvCache full"):
        m.feed_async(m.token, gpt2_tiny.CTX)


def test_a_failed_stack_exchange_is_reported_and_recovered(fh, orc, tiny_pair):
    """Workgroup 5 publishes none of its outputs (testing hook) and the waits
    give up after 64 polls: every workgroup ends, fh_sync reports
    FH_ERR_EXCHANGE, and a re-primed run is exact again."""
    import ferrum_hip

    w, m = tiny_pair
    ids = np.random.default_rng(9).integers(0, gpt2_tiny.VOCAB, 6)
    fh.debug_sampler_faults(5, 64)
    try:
        m.fused = True
        m.token.fill_(int(ids[0]))
        import torch

        torch.cuda.synchronize()
        m.feed_async(m.token, 0)
        with pytest.raises(ferrum_hip.FerrumHipError) as e:
            fh.sync()
        assert e.value.code == ferrum_hip.FH_ERR_EXCHANGE
    finally:
        fh.debug_sampler_faults(-1, 0)
    fh.sync()
    ref = gpt2_tiny.OracleGPT2(orc, w)
    for p, t in enumerate(ids):
        assert_scores_close(feed(m, t, p, True), ref.feed(t), f"after recovery, position {p}")


CONFIG3 = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)


def replay_config3(orc, w, prompt, ids):
    """Every step of a config-3 run replayed on the oracle's model and sampler
    with the same window and draw; a differing id must be one the oracle
    reports within the sampler's margins, and the replay continues from the
    device's id.  Returns the number of such steps."""
    import ferrum_hip
    from sampler_margins import exempt

    ref = gpt2_tiny.OracleGPT2(orc, w, **{k: G124[k] for k in ("vocab", "d", "heads", "layers", "ffn")},
                               ctx=G124["ctx"])
    win, rng, op = ferrum_hip.GPT2Window(G124["ctx"], prompt), orc.Rng(11), orc.SamplingParams(**CONFIG3)
    z = ref.forward(win.ids, True)
    n_exempt = 0
    for step, tok in enumerate(ids):
        want, info = orc.sample(orc.ln_bridge(orc.softmax_rows(z)[0]), op, win.ids, rng.next_u64())
        if want != tok:
            assert exempt(info, False), (step, tok, want, info.topk_gap, info.topp_gap, info.draw_gap)
            n_exempt += 1
        win.push(tok)
        z = ref.forward(win.ids, False)
    return n_exempt


CONFIG3_RUNS = {}  # the position-by-position run's ids, once replayed on the oracle


def test_config3_run_replays_on_the_oracle(fh, orc, g124):
    """BASELINE configs[2] end to end: GPT-2-124M (N(0, 0.02) Q8_0 weights), a
    128-token random prompt, then all 256 steps sampled with temperature 0.8,
    top-k 40, top-p 0.95 and repetition penalty 1.1 over the window, the draws
    from Rng (slm/token_stream.rs:66-190, slm/cached.rs:100-137).  The
    device-resident run (GPT2Device.generate: the sampler's id feeds the next
    step on the device) equals the host loop over forward() id for id and
    leaves the Rng in the same state, and every one of the 256 steps replays
    on the oracle (replay_config3); the exempt count is reported."""
    import ferrum_hip

    w, m = g124
    prompt = [int(t) for t in np.random.default_rng(128).integers(0, G124["vocab"], 128)]
    params = ferrum_hip.SamplingParams(**CONFIG3)
    rng_dev, rng_host = ferrum_hip.Rng(11), ferrum_hip.Rng(11)
    ids = m.generate(prompt, 256, params, rng_dev)
    assert len(ids) == 256
    host = ferrum_hip.gpt2_decode(fh, m.forward, prompt, 256, params, rng_host, G124["ctx"])
    assert host == ids and rng_dev.state == rng_host.state
    n_exempt = replay_config3(orc, w, prompt, ids)
    print(f"config-3 run: 256 steps, {n_exempt} exempt")
    assert n_exempt <= 4
    CONFIG3_RUNS["ids"] = ids


def test_config3_run_with_prefill_replays_on_the_oracle(fh, orc, g124):
    """The same 256-step run with the prompt primed in one pass
    (generate(prefill=True): 127 positions as rows of GEMMs and one attention
    launch per block): the ids equal the position-by-position run's (already
    replayed on the oracle), or else every step replays on the oracle within
    the sampler's margins."""
    import ferrum_hip

    w, m = g124
    prompt = [int(t) for t in np.random.default_rng(128).integers(0, G124["vocab"], 128)]
    ids = m.generate(prompt, 256, ferrum_hip.SamplingParams(**CONFIG3), ferrum_hip.Rng(11), prefill=True)
    assert len(ids) == 256
    if ids == CONFIG3_RUNS.get("ids"):
        print("config-3 run with prefill: the same 256 ids as the position-by-position run")
        return
    n_exempt = replay_config3(orc, w, prompt, ids)
    print(f"config-3 run with prefill: 256 steps, {n_exempt} exempt")
    assert n_exempt <= 4


def prefill(model, ids, pos0):
    import torch

    d_ids = torch.tensor(np.asarray(ids, np.int32), device="cuda")
    torch.cuda.synchronize()
    model.prefill_async(d_ids, pos0, len(ids))
    model.ctx.sync()
    torch.cuda.synchronize()
    return model.z.cpu().numpy().copy()


def test_tiny_prefill_matches_oracle(fh, orc, tiny_pair):
    """A 150-position prompt as one block of rows, and as two (100 + 50: the
    second block's attention reads the first's cache rows): the last
    position's scores against the oracle fed position by position
    (CachedTransformer::feed), and the next position through the stack and
    through the per-op path, reading the caches the prefill filled."""
    w, m = tiny_pair
    ref = gpt2_tiny.OracleGPT2(orc, w)
    ids = np.random.default_rng(31).integers(0, gpt2_tiny.VOCAB, 151)
    want = [ref.feed(t) for t in ids]
    assert_scores_close(prefill(m, ids[:150], 0), want[149], "one block of 150")
    assert_scores_close(feed(m, ids[150], 150, True), want[150], "stack after the prefill")
    assert_scores_close(prefill(m, ids[:100], 0), want[99], "first block of 100")
    assert_scores_close(prefill(m, ids[100:150], 100), want[149], "second block of 50")
    assert_scores_close(feed(m, ids[150], 150, False), want[150], "per-op after two blocks")
    assert_scores_close(prefill(m, ids[:1], 0), want[0], "a block of one")


def test_prefill_errors(fh, tiny_pair):
    import torch

    import ferrum_hip

    _, m = tiny_pair
    d_ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(ferrum_hip.DimMismatch, match="KvCache full"):
        m.prefill_async(d_ids, gpt2_tiny.CTX - 4, 8)
    with pytest.raises(ferrum_hip.DimMismatch, match="KvCache full"):
        ferrum_hip.attention_prefill_async(fh, m.qkv, m.blocks[0]["k"], m.blocks[0]["v"], gpt2_tiny.CTX,
                                           gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.CTX - 1, 2, m.att)
    with pytest.raises(ferrum_hip.DimMismatch, match="must divide"):
        ferrum_hip.attention_prefill_async(fh, m.qkv, m.blocks[0]["k"], m.blocks[0]["v"], gpt2_tiny.CTX,
                                           gpt2_tiny.D, 3, 0, 1, m.att)
    m.prefill_async(d_ids, 0, 0)  # nothing to do
    fh.sync()


def test_gpt2_124m_prefill_matches_oracle(fh, orc, g124):
    """GPT-2-124M: a 128-position prompt in one block (every GEMM at m = 128,
    two attention items per head for the last rows), its last scores against
    the oracle's, then three stack positions on from the prefilled caches."""
    w, m = g124
    ref = gpt2_tiny.OracleGPT2(orc, w, **{k: G124[k] for k in ("vocab", "d", "heads", "layers", "ffn")},
                               ctx=G124["ctx"])
    ids = np.random.default_rng(12).integers(0, G124["vocab"], 131)
    want = [ref.feed(t) for t in ids]
    assert_scores_close(prefill(m, ids[:128], 0), want[127], "124M prefill of 128")
    for p in range(128, 131):
        assert_scores_close(feed(m, ids[p], p, True), want[p], f"124M stack at {p} after the prefill")
