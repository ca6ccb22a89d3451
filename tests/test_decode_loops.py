"""Token-level decode loops around the hot path (slm/token_stream.rs:66-190,
llm.rs:706-754): window management on the CPU, and on the GPU a whole decode
run (Q8_0 head GEMV + fused sampler per step) replayed against the oracle."""
import numpy as np
import pytest


def test_gpt2_window_cut_keep_and_reprime():
    import ferrum_hip

    w = ferrum_hip.GPT2Window(5, [10, 11, 12, 13, 14, 15, 16, 17])
    assert w.ids == [13, 14, 15, 16, 17] and w.keep == 2
    assert w.push(18) and w.ids == [17, 18]          # 6 > 5: cut to the last keep = 2
    assert not w.push(19) and w.ids == [17, 18, 19]
    assert ferrum_hip.GPT2Window(3, [], bos=7).ids == [7]
    one = ferrum_hip.GPT2Window(0, [1, 2])          # capacity max(0, 1) = 1, keep 1
    assert one.ids == [2] and one.push(3) and one.ids == [3]


def test_llama_loop_rejects_empty_and_oversized_prompts():
    import ferrum_hip

    p = ferrum_hip.SamplingParams(temperature=0.0)
    with pytest.raises(ferrum_hip.DimMismatch, match="non-empty"):
        ferrum_hip.llama_decode(None, lambda t: None, [], 4, p, ferrum_hip.Rng(1), 8)
    with pytest.raises(ferrum_hip.DimMismatch, match="8-token context window"):
        ferrum_hip.llama_decode(None, lambda t: None, list(range(8)), 4, p, ferrum_hip.Rng(1), 8)


class ToyHead:
    """A stand-in model: the next position's scores are the Q8_0 head applied
    to a fixed embedding of the last id (the rest of the network is the
    caller's).  Scores are recorded so the oracle can replay each step."""

    def __init__(self, fh, orc, vocab, d, seed):
        import ferrum_hip

        self.emb = (np.random.default_rng(seed).standard_normal((vocab, d)) * 0.6).astype(np.float32)
        self.raw = orc.quantize_weight(vocab, d, seed, 0.5)
        self.w = ferrum_hip.Q8_0Weight.upload(fh, self.raw, vocab, d)
        self.fh, self.scores, self.fed = fh, [], []

    def __call__(self, ids, reprime=False):
        import ferrum_hip

        last = ids[-1] if isinstance(ids, list) else ids
        z = ferrum_hip.matmul(self.fh, self.emb[last][None, :], self.w)[0]
        self.scores.append(z)
        self.fed.append(reprime)
        return z


@pytest.mark.gpu
def test_gpt2_decode_run_replays_on_the_oracle(fh, orc):
    import ferrum_hip

    vocab, d, cap = 4096, 128, 12
    model = ToyHead(fh, orc, vocab, d, 5)
    kw = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)
    prompt = list(np.random.default_rng(6).integers(0, vocab, 16))
    got = ferrum_hip.gpt2_decode(fh, model, prompt, 40, ferrum_hip.SamplingParams(**kw), ferrum_hip.Rng(9), cap)
    model.w.free()
    assert len(got) == 40 and sum(model.fed) >= 6      # re-primed at every overflow
    # Replay: the same scores, window and Rng on the oracle's sampler.
    win, rng, op = ferrum_hip.GPT2Window(cap, prompt), orc.Rng(9), orc.SamplingParams(**kw)
    for step, tok in enumerate(got):
        want, info = orc.sample(orc.ln_bridge(orc.softmax_rows(model.scores[step])[0]), op, win.ids,
                                rng.next_u64())
        if want != tok:
            assert info.margin < 1e-5, (step, tok, want, info.margin)
            break                                     # the runs part ways at a tie; nothing after is comparable
        win.push(tok)


@pytest.mark.gpu
def test_llama_decode_run_replays_on_the_oracle(fh, orc):
    import ferrum_hip

    vocab, d = 2048, 96
    model = ToyHead(fh, orc, vocab, d, 8)
    kw = dict(temperature=0.9, top_k=50, top_p=0.9, repetition_penalty=1.05)
    prompt = list(np.random.default_rng(3).integers(0, vocab, 10))
    got = ferrum_hip.llama_decode(fh, model, prompt, 100, ferrum_hip.SamplingParams(**kw), ferrum_hip.Rng(4),
                                  context_len=40)
    model.w.free()
    assert len(got) == 30                              # clipped to context - prompt
    recent, op, state = list(prompt), orc.SamplingParams(**kw), orc.Rng(4)
    for step, tok in enumerate(got):
        z = model.scores[len(prompt) - 1 + step]
        want, info = orc.sample(z, op, recent, state.next_u64())
        if want != tok:
            assert info.margin < 1e-5, (step, tok, want, info.margin)
            break
        recent.append(tok)
