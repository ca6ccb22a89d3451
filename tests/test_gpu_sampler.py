"""The fused sampler on the GPU against the oracle's sample_with_params
(slm/sampling.rs:124-210).

Parity rule: tests/sampler_margins.py (ids identical given the same draws
except at a decision within the precision both sides carry: 1e-5 top-2 gap
for greedy, 1e-6 at the k-th place or the draw, 2e-5 at the top-p cut).
Every call prints how many rows fall within these margins and how many were
exempt (ids differ); each test bounds the exempt share.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from sampler_margins import exempt  # noqa: E402


def run_and_compare(fh, orc, logits, params_kw, recents=None, draws=None, kind=0, max_exempt=0.01):
    import ferrum_hip

    logits = np.ascontiguousarray(logits, np.float32)
    rows, vocab = logits.shape
    if recents is None:
        recents = [[] for _ in range(rows)]
    if draws is None:
        rng = np.random.default_rng(rows * 977 + vocab)
        draws = rng.integers(0, 2**64, size=rows, dtype=np.uint64)
    gp = ferrum_hip.SamplingParams(**params_kw)
    got = ferrum_hip.sample_rows(fh, logits, gp, recents, draws, kind)
    op = orc.SamplingParams(**params_kw)
    greedy = params_kw.get("temperature", 1.0) <= 0.0
    n_exempt, near, bad = 0, 0, []
    for r in range(rows):
        row = logits[r]
        if kind == ferrum_hip.LOGITS_GPT2_SOFTMAX:
            row = orc.ln_bridge(orc.softmax_rows(row)[0])
        want, info = orc.sample(row, op, recents[r], int(draws[r]))
        near += exempt(info, greedy)
        if got[r] != want:
            if exempt(info, greedy):
                n_exempt += 1
            else:
                bad.append(f"row {r}: gpu {got[r]} vs oracle {want}; gaps greedy {info.greedy_gap:.2e} top-k "
                           f"{info.topk_gap:.2e} top-p {info.topp_gap:.2e} draw {info.draw_gap:.2e}, "
                           f"path {info.path}, kept {info.n_kept}")
    print(f"sampler parity {params_kw} kind {kind}: {rows} rows, {near} within the margins, "
          f"{n_exempt} exempt (ids differ)")
    assert not bad, "; ".join(bad)
    assert n_exempt <= max(1, int(max_exempt * rows)), f"{n_exempt} exempt rows of {rows}"
    return got


def normal_logits(rows, vocab, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal((rows, vocab)) * scale).astype(np.float32)


# ---- the reference's own known answers (sampling.rs:219-422) --------------------------

def test_greedy_known_answers(fh):
    import ferrum_hip

    g = ferrum_hip.SamplingParams(temperature=0.0)
    s = lambda lg, rec=(): ferrum_hip.sample_with_params(fh, np.array(lg, np.float32), g, list(rec), ferrum_hip.Rng(1))
    assert s([0.1, 2.0, 2.0, 1.0]) == 1 and s([3.0, 3.0, 3.0]) == 0 and s([-1.0, -0.5, -0.5]) == 1
    assert s([float("-inf"), float("-inf")]) == 0 and s([1.0, 5.0, 5.0]) == 1 and s([1.0]) == 0
    # repetition penalty flips the argmax (sampling.rs:235-262); out-of-vocab ids ignored (219-232)
    pen = ferrum_hip.SamplingParams(temperature=0.0, repetition_penalty=2.0)
    t = lambda lg, rec: ferrum_hip.sample_with_params(fh, np.array(lg, np.float32), pen, rec, ferrum_hip.Rng(1))
    assert t([2.0, 1.5], [0]) == 1 and t([2.0, 1.5], [99]) == 0 and t([-1.0, -1.5], [0, 0]) == 1


def test_greedy_draws_no_rng(fh):
    # sampling.rs:365-389: greedy consumes nothing from the generator
    import ferrum_hip

    rng = ferrum_hip.Rng(7)
    before = rng.state
    ferrum_hip.sample_with_params(fh, np.arange(10, dtype=np.float32), ferrum_hip.SamplingParams(0.0), [], rng)
    assert rng.state == before


def test_top_k_one_is_argmax_and_nan_fallback(fh, orc):
    import ferrum_hip

    lg = normal_logits(16, 1000, 3)
    got = ferrum_hip.sample_rows(fh, lg, ferrum_hip.SamplingParams(0.9, 1), None, np.arange(16, dtype=np.uint64) << 40)
    assert np.array_equal(got, lg.argmax(axis=1))
    # a NaN or +inf logit makes the softmax sum NaN: the reference draws next_u64 % n (sampling.rs:156-168)
    bad = lg.copy()
    bad[0, 5] = np.nan
    bad[1, 9] = np.inf
    draws = np.array([123456789, 987654321] + [0] * 14, np.uint64)
    got = ferrum_hip.sample_rows(fh, bad, ferrum_hip.SamplingParams(1.0), None, draws)
    assert got[0] == 123456789 % 1000 and got[1] == 987654321 % 1000


def test_pick_by_mass_boundaries(fh, orc):
    """Draws on both sides of every cumulative boundary of a small distribution
    (sampling.rs:408-422 behaviour through the whole sampler)."""
    lg = np.log(np.array([[0.1, 0.2, 0.3, 0.4]], np.float32))
    rs = np.arange(0, 1 << 24, 1 << 14, dtype=np.uint64) << 40
    for d in rs[:256]:
        run_and_compare(fh, orc, lg, dict(temperature=1.0), draws=np.array([d], np.uint64))


# ---- seeded parity sweeps -------------------------------------------------------------

PARAMS = {
    "greedy": dict(temperature=0.0),
    "greedy_pen": dict(temperature=0.0, repetition_penalty=1.3),
    "temp": dict(temperature=0.8),
    "topk": dict(temperature=0.8, top_k=40),
    "topp": dict(temperature=0.8, top_p=0.95),
    "topk_topp_pen": dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
    "hot_topp": dict(temperature=2.5, top_p=0.6),
    "bigk": dict(temperature=1.0, top_k=6000),
    "tiny_t": dict(temperature=0.001, top_k=5),
}


@pytest.mark.parametrize("name", sorted(PARAMS))
@pytest.mark.parametrize("vocab", [2, 7, 4096, 50257])
def test_raw_logits_parity(fh, orc, name, vocab):
    rows = 24 if vocab > 1000 else 64
    lg = normal_logits(rows, vocab, vocab + len(name))
    rng = np.random.default_rng(vocab)
    recents = [list(rng.integers(0, vocab + 3, size=rng.integers(0, 300))) for _ in range(rows)]
    run_and_compare(fh, orc, lg, PARAMS[name], recents)


@pytest.mark.parametrize("name", ["greedy", "topk_topp_pen", "topp", "temp"])
def test_gpt2_softmax_bridge_parity(fh, orc, name):
    import ferrum_hip

    rows, vocab = 16, 50257
    lg = normal_logits(rows, vocab, 99, scale=2.0)
    rng = np.random.default_rng(5)
    recents = [list(rng.integers(0, vocab, size=256)) for _ in range(rows)]
    # GPT-2-bridged rows are flat (|z| ~ 2): with top-p alone the kept set is
    # ~10,000 ids at nearly equal p, so almost every row's top-p cut falls
    # between ids whose p differ by ~1e-6 relative (all 16 rows are within
    # the top-p margin); each mismatch must still be such a row.
    run_and_compare(fh, orc, lg, PARAMS[name], recents, kind=ferrum_hip.LOGITS_GPT2_SOFTMAX,
                    max_exempt=0.25 if name == "topp" else 0.1)


def test_repeated_ids_penalised_once_per_occurrence(fh, orc):
    rows, vocab = 8, 4096
    lg = normal_logits(rows, vocab, 12)
    rec = [[7] * 50 + [9] * 3 + list(range(100, 140)) * 4 for _ in range(rows)]
    lg[:, 7] = 9.0
    run_and_compare(fh, orc, lg, dict(temperature=0.0, repetition_penalty=1.05), rec)
    run_and_compare(fh, orc, lg, dict(temperature=0.7, top_k=20, repetition_penalty=1.05), rec)


def test_long_history_chunks(fh, orc):
    """More recent ids than one LDS table fill (4096), with heavy repetition."""
    rows, vocab = 4, 50257
    lg = normal_logits(rows, vocab, 21)
    rng = np.random.default_rng(3)
    rec = [list(rng.integers(0, 64, size=9000)) + list(rng.integers(0, vocab, size=3000)) for _ in range(rows)]
    run_and_compare(fh, orc, lg, dict(temperature=0.0, repetition_penalty=1.01), rec)
    run_and_compare(fh, orc, lg, dict(temperature=0.9, top_k=50, repetition_penalty=1.01), rec)


def test_flat_top_p_takes_the_general_path(fh, orc):
    """Nearly flat logits: the top-p set is thousands of ids (beyond the LDS
    list), so the cut is found by the mass radix select."""
    rows, vocab = 12, 50257
    lg = (np.random.default_rng(8).standard_normal((rows, vocab)) * 0.05).astype(np.float32)
    run_and_compare(fh, orc, lg, dict(temperature=1.0, top_p=0.5), max_exempt=0.1)
    run_and_compare(fh, orc, lg, dict(temperature=1.0, top_k=10000, top_p=0.9), max_exempt=0.1)


@pytest.mark.parametrize("rows", [16, 64])
def test_qwen_config5_rows(fh, orc, rows):
    """Config 5: 151936-wide logits ~N(0,3) plus 5 planted peaks (+12), top-k 50,
    top-p 0.9, repetition penalty 1.05 over a 1024-token random history.  At 64
    rows the split sampler takes four segments of 40 ids per thread, so every
    row fits the CUs together in one launch."""
    vocab = 151936
    rng = np.random.default_rng(55)
    lg = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    peaks = rng.integers(0, vocab, size=5)
    lg[:, peaks] += 12.0
    rec = [list(rng.integers(0, vocab, size=1024)) + list(peaks[:2]) for _ in range(rows)]
    run_and_compare(fh, orc, lg, dict(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.05), rec)


def test_many_rows_run_as_consecutive_split_launches(fh, orc):
    """600 rows of 8192 ids: more rows than one split launch holds."""
    lg = normal_logits(600, 8192, 31)
    rng = np.random.default_rng(32)
    rec = [list(rng.integers(0, 8192, size=64)) for _ in range(600)]
    run_and_compare(fh, orc, lg, dict(temperature=0.9, top_k=40, top_p=0.95, repetition_penalty=1.1), rec)


def test_sampler_errors(fh):
    import ferrum_hip

    with pytest.raises(ferrum_hip.FerrumHipError, match="vocab is 0"):
        ferrum_hip.sample_rows(fh, np.zeros((1, 0), np.float32), ferrum_hip.SamplingParams(0.0))
    with pytest.raises(ferrum_hip.FerrumHipError, match="draws is NULL"):
        ferrum_hip.sample_rows(fh, np.zeros((1, 10), np.float32), ferrum_hip.SamplingParams(0.5))


@pytest.mark.parametrize("vocab", [4096, 50257])
def test_histories_longer_than_any_table(fh, orc, vocab):
    """A Llama-path history is the whole prompt plus every generated id
    (llm.rs:740-750): 40,000 recent ids, no cut-off, through the blocking call
    and through the device form."""
    import torch

    import ferrum_hip

    rows = 3
    lg = normal_logits(rows, vocab, 17)
    rng = np.random.default_rng(18)
    rec = [list(rng.integers(0, 300, size=40000)) for _ in range(rows)]
    lg[:, :300] += 1.0
    kw = dict(temperature=0.7, top_k=30, top_p=0.9, repetition_penalty=1.0005)
    got = run_and_compare(fh, orc, lg, kw, rec)
    run_and_compare(fh, orc, lg, dict(temperature=0.0, repetition_penalty=1.0005), rec)
    flat, off = ferrum_hip._recent_lists(rec, rows)
    draws = np.random.default_rng(rows * 977 + vocab).integers(0, 2**64, size=rows, dtype=np.uint64)
    d_out = torch.zeros(rows, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.sample_rows_async(fh, torch.from_numpy(lg).cuda(), rows, vocab, ferrum_hip.SamplingParams(**kw),
                                 torch.from_numpy(flat.astype(np.int32)).cuda(),
                                 torch.from_numpy(off.astype(np.int32)).cuda(),
                                 torch.from_numpy(draws.view(np.int64)).cuda(), d_out)
    fh.sync()
    assert np.array_equal(d_out.cpu().numpy().astype(np.uint32), got)


def test_decreasing_device_offsets_are_reported(fh):
    """The device form cannot read its offsets on the host: a decreasing list
    is recorded by the kernel and raised by the next sync."""
    import torch

    import ferrum_hip

    rows, vocab = 2, 50257
    lg = torch.from_numpy(normal_logits(rows, vocab, 4)).cuda()
    rec = torch.zeros(8, dtype=torch.int32, device="cuda")
    off = torch.tensor([4, 2, 6], dtype=torch.int32, device="cuda")
    out = torch.zeros(rows, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for params in (ferrum_hip.SamplingParams(0.0, repetition_penalty=1.2),
                   ferrum_hip.SamplingParams(0.8, 40, 0.95, 1.2)):
        draws = torch.zeros(rows, dtype=torch.int64, device="cuda")
        ferrum_hip.sample_rows_async(fh, lg, rows, vocab, params, rec, off, draws, out)
        with pytest.raises(ferrum_hip.FerrumHipError, match="recent_offsets decrease") as e:
            fh.sync()
        assert e.value.code == ferrum_hip.FH_ERR_INVALID
    fh.sync()  # cleared


@pytest.mark.parametrize("params", [dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
                                    dict(temperature=0.0), dict(temperature=0.9)])
def test_a_failed_exchange_is_reported_and_recovered(fh, orc, params):
    """One segment of a split row publishes nothing (a host-set testing hook)
    and the bounded waits give up after 64 polls: every workgroup still ends,
    the blocking call returns FH_ERR_EXCHANGE, the device form reports it at
    the next sync, and later calls are exact again."""
    import torch

    import ferrum_hip

    rows, vocab = 3, 50257
    lg = normal_logits(rows, vocab, 61)
    rng = np.random.default_rng(62)
    rec = [list(rng.integers(0, vocab, size=128)) for _ in range(rows)]
    draws = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    gp = ferrum_hip.SamplingParams(**params)
    fh.debug_sampler_faults(1, 64)
    try:
        with pytest.raises(ferrum_hip.FerrumHipError) as e:
            ferrum_hip.sample_rows(fh, lg, gp, rec, draws)
        assert e.value.code == ferrum_hip.FH_ERR_EXCHANGE
        flat, off = ferrum_hip._recent_lists(rec, rows)
        out = torch.zeros(rows, dtype=torch.int32, device="cuda")
        d_lg = torch.from_numpy(lg).cuda()
        d_rec = torch.from_numpy(flat.astype(np.int32)).cuda()
        d_off = torch.from_numpy(off.astype(np.int32)).cuda()
        d_dr = torch.from_numpy(draws.view(np.int64)).cuda()
        torch.cuda.synchronize()
        ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, gp, d_rec, d_off, d_dr, out)
        with pytest.raises(ferrum_hip.FerrumHipError) as e:
            fh.sync()
        assert e.value.code == ferrum_hip.FH_ERR_EXCHANGE
    finally:
        fh.debug_sampler_faults(-1, 0)
    fh.sync()
    run_and_compare(fh, orc, lg, params, rec, draws=draws)


def test_split_rows_replay_in_a_graph(fh, orc):
    """The multi-workgroup sampler keeps per-row barrier state on the device and
    zeroes it when a row finishes, so back-to-back launches and HIP graph
    replays must give the same ids as the first eager call."""
    import torch

    import ferrum_hip

    rows, vocab = 3, 50257
    lg = normal_logits(rows, vocab, 31)
    rng = np.random.default_rng(2)
    recents = [list(rng.integers(0, vocab, size=128)) for _ in range(rows)]
    flat, off = ferrum_hip._recent_lists(recents, rows)
    draws = rng.integers(0, 2**63, size=rows, dtype=np.uint64)
    cases = [dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1), dict(temperature=0.0),
             dict(temperature=0.9), dict(temperature=1.0, top_p=0.5)]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        d_lg = torch.from_numpy(lg).cuda()
        d_rec = torch.from_numpy(flat.astype(np.int32)).cuda()
        d_off = torch.from_numpy(off.astype(np.int32)).cuda()
        d_dr = torch.from_numpy(draws.view(np.int64)).cuda()
        d_out = torch.zeros(rows, dtype=torch.int32, device="cuda")
        for kind in (ferrum_hip.LOGITS_RAW, ferrum_hip.LOGITS_GPT2_SOFTMAX):
            for kw in cases:
                params = ferrum_hip.SamplingParams(**kw)
                want = ferrum_hip.sample_rows(fh, lg, params, recents, draws, kind)
                fh.set_stream(s.cuda_stream)
                try:
                    ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, params, d_rec, d_off, d_dr, d_out, kind)
                    s.synchronize()
                    assert np.array_equal(d_out.cpu().numpy().astype(np.uint32), want), (kind, kw)
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=s):
                        fh.set_stream(torch.cuda.current_stream().cuda_stream)
                        ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, params, d_rec, d_off, d_dr, d_out, kind)
                    fh.set_stream(s.cuda_stream)
                    for rep in range(4):
                        d_out.zero_()
                        g.replay()
                        s.synchronize()
                        assert np.array_equal(d_out.cpu().numpy().astype(np.uint32), want), (kind, kw, rep)
                        ferrum_hip.sample_rows(fh, lg, params, recents, draws, kind)  # eager work between replays
                finally:
                    fh.set_stream(None)


@pytest.mark.parametrize("crowd,spread", [(100, 0.04), (200, 0.04), (400, 0.005)])
def test_top_k_with_a_crowded_top(fh, orc, crowd, spread):
    """Rows whose top holds `crowd` ids within `spread` of each other gather
    about 100, 80-100 and 400 survivors for a top-k of 40 (the 1/8-octave
    bucket holding the 40th largest p is crowded): up to 256 the kernel
    reduces them to their top 64 in one wave, past that (or when ties reach
    the 64th) it sorts them in LDS.  Every id against the oracle, with top-p on and off, raw logits and
    the GPT-2 bridge; a second set of rows has 80 exactly equal values at the
    top (the tie fallback)."""
    import ferrum_hip

    rows, vocab = 6, 50257
    rng = np.random.default_rng(crowd)
    lg = (rng.standard_normal((rows, vocab)) - 3.0).astype(np.float32)
    for r in range(rows):
        ids = rng.choice(vocab, size=crowd, replace=False)
        lg[r, ids] = 4.0 + rng.uniform(0.0, spread, size=crowd).astype(np.float32)
    for kw in (dict(temperature=1.0, top_k=40), dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
               dict(temperature=1.0, top_k=64, top_p=0.5)):
        recents = [list(rng.integers(0, vocab, size=64)) for _ in range(rows)]
        run_and_compare(fh, orc, lg, kw, recents)
        run_and_compare(fh, orc, lg, kw, recents, kind=ferrum_hip.LOGITS_GPT2_SOFTMAX)
    tie = (rng.standard_normal((rows, vocab)) - 3.0).astype(np.float32)
    for r in range(rows):
        tie[r, rng.choice(vocab, size=80, replace=False)] = 4.0
    run_and_compare(fh, orc, tie, dict(temperature=1.0, top_k=40))
    run_and_compare(fh, orc, tie, dict(temperature=1.0, top_k=40, top_p=0.9))


@pytest.mark.parametrize("vocab", [4096, 50257])
def test_recent_ranges_equal_running_offsets(fh, orc, vocab):
    """FH_RECENT_RANGES (each row's window in its own stretch of a [rows, L]
    buffer, as the batched decode keeps them): the same ids as the running-
    offset form and as the oracle, with an empty window, a window of a whole
    stretch and a reversed pair (reported at the next sync, as decreasing
    running offsets are)."""
    import torch

    import ferrum_hip
    from sampler_margins import exempt

    rows, L = 6, 300
    lg = normal_logits(rows, vocab, 23)
    rng = np.random.default_rng(24)
    buf = rng.integers(0, 400, size=(rows, L)).astype(np.int32)
    lg[:, :400] += 1.5
    lens = [0, 1, 57, 120, 299, 300]
    kw = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    params = ferrum_hip.SamplingParams(**kw)
    draws = rng.integers(0, 2**64, size=rows, dtype=np.uint64)
    pairs = np.array([[r * L, r * L + n] for r, n in enumerate(lens)], np.int32)
    rec = [list(buf[r, :n]) for r, n in enumerate(lens)]
    flat, off = ferrum_hip._recent_lists(rec, rows)
    d_lg = torch.from_numpy(lg).cuda()
    d_draws = torch.from_numpy(draws.view(np.int64)).cuda()
    a = torch.zeros(rows, dtype=torch.int32, device="cuda")
    b = torch.zeros(rows, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, params, torch.from_numpy(buf.ravel()).cuda(),
                                 torch.from_numpy(pairs.ravel()).cuda(), d_draws, a,
                                 ferrum_hip.LOGITS_RAW | ferrum_hip.RECENT_RANGES)
    ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, params, torch.from_numpy(flat.astype(np.int32)).cuda(),
                                 torch.from_numpy(off.astype(np.int32)).cuda(), d_draws, b)
    fh.sync()
    got = a.cpu().numpy().astype(np.uint32)
    assert np.array_equal(got, b.cpu().numpy().astype(np.uint32))
    op = orc.SamplingParams(**kw)
    for r in range(rows):
        want, info = orc.sample(lg[r], op, rec[r], int(draws[r]))
        assert got[r] == want or exempt(info, False), (r, got[r], want)
    # a reversed pair is reported; the blocking form refuses the flag
    bad = torch.tensor([0, 5, 9, 3] + [0, 0] * (rows - 2), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.sample_rows_async(fh, d_lg, rows, vocab, params, torch.from_numpy(buf.ravel()).cuda(), bad, d_draws, a,
                                 ferrum_hip.LOGITS_RAW | ferrum_hip.RECENT_RANGES)
    with pytest.raises(ferrum_hip.FerrumHipError, match="recent_offsets decrease") as e:
        fh.sync()
    assert e.value.code == ferrum_hip.FH_ERR_INVALID
    with pytest.raises(ferrum_hip.FerrumHipError, match="FH_RECENT_RANGES"):
        ferrum_hip.sample_rows(fh, lg, params, rec, draws, ferrum_hip.LOGITS_RAW | ferrum_hip.RECENT_RANGES)
    fh.sync()
