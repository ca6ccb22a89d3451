"""The reference's per-token controls in the device-resident decode loops
(GPT2Device.generate, GPT2Batch.generate), which run their steps on the
device in chunks:

  * EOS: the stream draws the EOS id and stops, without returning it
    (slm/token_stream.rs:134-138); every other row of a batch goes on;
  * cancel: the flag is checked before a token is drawn, and a set flag ends
    the run with what was produced (slm/sampling.rs:20-37,
    slm/token_stream.rs:126-131, llm.rs:719-745);
  * draws: one next_u64 per sampled step and none when greedy, so after a
    run the caller's Rng is in the state ferrum_core's loop leaves it in.

Each run is replayed on the oracle's model, sampler and Rng (the draw of
every returned step and of the EOS step), and compared with the host loop
(gpt2_decode, one token at a time)."""
import numpy as np
import pytest

import gpt2_tiny
from sampler_margins import exempt

pytestmark = pytest.mark.gpu

CONFIG3 = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)


class TripAfter:
    """A cancel flag that reads as set from its n-th check on: a flag another
    thread sets between two tokens."""

    def __init__(self, n):
        self.n, self.calls = n, 0

    def is_set(self):
        self.calls += 1
        return self.calls >= self.n


def advanced(seed, n):
    import ferrum_hip

    r = ferrum_hip.Rng(seed)
    for _ in range(n):
        r.next_u64()
    return r.state


def replay(orc, w, prompt, ids, kw, seed, eos=None):
    """The oracle's stream_next over the device's ids: every returned id is the
    oracle's own (or within the sampler's margins), and with `eos` the step
    after the last returned one samples the EOS id.  Returns the oracle Rng's
    state after the run: the draws of the returned steps plus the EOS step's."""
    import ferrum_hip

    ref = gpt2_tiny.OracleGPT2(orc, w)
    win, rng, op = ferrum_hip.GPT2Window(gpt2_tiny.CTX, prompt), orc.Rng(seed), orc.SamplingParams(**kw)
    greedy = kw["temperature"] <= 0.0
    z = ref.forward(win.ids, True)
    for step, tok in enumerate(list(ids) + ([eos] if eos is not None else [])):
        draw = 0 if greedy else rng.next_u64()
        want, info = orc.sample(orc.ln_bridge(orc.softmax_rows(z)[0]), op, win.ids, draw)
        if want != tok:
            assert exempt(info, greedy), (step, tok, want)
        if step == len(ids):
            break
        reprime = win.push(tok)
        z = ref.forward(win.ids, reprime)
    return int(rng.state.value)


@pytest.fixture(scope="module")
def tiny(fh, orc):
    import ferrum_hip

    w = gpt2_tiny.make_weights(orc, seed=11)
    m = ferrum_hip.GPT2Device.from_weights(fh, w, gpt2_tiny.VOCAB, gpt2_tiny.D, gpt2_tiny.HEADS, gpt2_tiny.LAYERS,
                                           gpt2_tiny.FFN, gpt2_tiny.CTX)
    assert m.stack is not None
    yield w, m
    m.free()


def first_new(ids, lo):
    """The first step j >= lo whose id does not occur before it (a planted EOS there ends the run at j)."""
    for j in range(lo, len(ids)):
        if ids[j] not in ids[:j]:
            return j
    pytest.skip("no id occurs for the first time late enough in the run")


def test_a_planted_eos_ends_the_device_run_after_its_draw(fh, orc, tiny):
    """A 40-step sampled run, then the same run with one of its ids as EOS
    (first seen at step j, inside a chunk of 8): the ids before it, none
    after, and the Rng advanced by j + 1 draws, as the host loop and the
    oracle's loop leave it; with prefill too."""
    import ferrum_hip

    w, m = tiny
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, gpt2_tiny.VOCAB, 16)]
    params = ferrum_hip.SamplingParams(**CONFIG3)
    full = m.generate(prompt, 40, params, ferrum_hip.Rng(5))
    assert len(full) == 40
    j = first_new(full, 19)
    eos = full[j]
    for prefill in (False, True):
        rng = ferrum_hip.Rng(5)
        got = m.generate(prompt, 40, params, rng, eos=eos, prefill=prefill, chunk=8)
        assert got == full[:j], prefill
        assert rng.state == advanced(5, j + 1), prefill
    host_rng = ferrum_hip.Rng(5)
    host = ferrum_hip.gpt2_decode(fh, m.forward, prompt, 40, params, host_rng, gpt2_tiny.CTX, eos=eos)
    assert host == full[:j] and host_rng.state == advanced(5, j + 1)
    assert replay(orc, w, prompt, full[:j], CONFIG3, 5, eos) == advanced(5, j + 1)


def test_cancel_stops_the_device_run_before_the_next_draw(fh, orc, tiny):
    """A flag found set before the third chunk of 8 ends the run after 16
    tokens with 16 draws taken (the host loop, checking before every token,
    stops at the same token when the flag is set there); a flag set before
    the call returns nothing and draws nothing; a greedy run draws nothing."""
    import ferrum_hip

    w, m = tiny
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, gpt2_tiny.VOCAB, 16)]
    params = ferrum_hip.SamplingParams(**CONFIG3)
    full = m.generate(prompt, 40, params, ferrum_hip.Rng(6))
    rng = ferrum_hip.Rng(6)
    got = m.generate(prompt, 40, params, rng, cancel=TripAfter(3), chunk=8)
    assert got == full[:16] and rng.state == advanced(6, 16)
    host_rng = ferrum_hip.Rng(6)
    host = ferrum_hip.gpt2_decode(fh, m.forward, prompt, 40, params, host_rng, gpt2_tiny.CTX, cancel=TripAfter(17))
    assert host == full[:16] and host_rng.state == advanced(6, 16)
    assert replay(orc, w, prompt, got, CONFIG3, 6) == advanced(6, 16)
    rng = ferrum_hip.Rng(6)
    assert m.generate(prompt, 40, params, rng, cancel=TripAfter(1)) == [] and rng.state == advanced(6, 0)
    rng = ferrum_hip.Rng(6)
    greedy = m.generate(prompt, 20, ferrum_hip.SamplingParams(temperature=0.0), rng, chunk=8)
    assert len(greedy) == 20 and rng.state == advanced(6, 0)


def test_batch_rows_stop_at_their_own_eos(fh, orc, tiny):
    """Four rows, 30 sampled steps in chunks of 8: with an id that one row
    samples at step 9 as EOS, each row returns its ids up to its own first
    EOS (rows that never sample it run to the end) and its Rng is advanced by
    its own steps plus its EOS step; every row replays on the oracle.  A
    cancel seen before the second chunk of 5 leaves five ids per row."""
    import ferrum_hip

    w, m = tiny
    prompts = np.random.default_rng(42).integers(0, gpt2_tiny.VOCAB, size=(4, 12))
    seeds = [51, 52, 53, 54]
    params = ferrum_hip.SamplingParams(**CONFIG3)
    batch = ferrum_hip.GPT2Batch(m, 4, 64)
    full = batch.generate(prompts, 30, params, [ferrum_hip.Rng(s) for s in seeds])
    assert all(len(r) == 30 for r in full)
    j = first_new(full[1], 9)
    eos = full[1][j]
    rngs = [ferrum_hip.Rng(s) for s in seeds]
    got = batch.generate(prompts, 30, params, rngs, eos=eos, chunk=8)
    for r in range(4):
        cut = full[r].index(eos) if eos in full[r] else None
        want = full[r] if cut is None else full[r][:cut]
        assert got[r] == want, r
        n_draws = 30 if cut is None else cut + 1
        assert rngs[r].state == advanced(seeds[r], n_draws), r
        assert replay(orc, w, [int(t) for t in prompts[r]], want, CONFIG3, seeds[r],
                      None if cut is None else eos) == advanced(seeds[r], n_draws), r
    rngs = [ferrum_hip.Rng(s) for s in seeds]
    got = batch.generate(prompts, 30, params, rngs, cancel=TripAfter(2), chunk=5)
    for r in range(4):
        assert got[r] == full[r][:5] and rngs[r].state == advanced(seeds[r], 5), r


def test_llama_loop_checks_cancel_before_each_draw(fh, orc):
    """LlamaModel::generate_inner's checks (llm.rs:726-745): a flag set while
    the prompt is fed returns nothing; set before token 6 it returns five,
    with five draws."""
    import llama_tiny

    import ferrum_hip

    cfg = llama_tiny.QWEN
    w = llama_tiny.make_weights(orc, cfg, 29, True, True)
    m = ferrum_hip.LlamaDevice.from_weights(fh, w, cfg, 1)
    kw = dict(temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.05)
    prompt = list(np.random.default_rng(12).integers(0, cfg["vocab"], 6))
    try:
        m.next_pos = 0
        full = ferrum_hip.llama_decode(fh, m.forward_one, prompt, 12, ferrum_hip.SamplingParams(**kw),
                                       ferrum_hip.Rng(4), cfg["context"])
        m.next_pos = 0
        rng = ferrum_hip.Rng(4)
        assert ferrum_hip.llama_decode(fh, m.forward_one, prompt, 12, ferrum_hip.SamplingParams(**kw), rng,
                                       cfg["context"], cancel=TripAfter(3)) == []
        assert rng.state == advanced(4, 0)
        m.next_pos = 0
        rng = ferrum_hip.Rng(4)
        got = ferrum_hip.llama_decode(fh, m.forward_one, prompt, 12, ferrum_hip.SamplingParams(**kw), rng,
                                      cfg["context"], cancel=TripAfter(len(prompt) + 6))
        assert got == full[:5] and rng.state == advanced(4, 5)
    finally:
        m.free()
