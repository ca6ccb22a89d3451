"""Benchmark of the MI355X Q8_0 decode path (one JSON line on stdout).

Workload (GPT-2-124M shape, batch 1): one whole
decode step on the device at position 255 (mid-run of the configuration's
128-token prompt + 256 steps) — Embedding::embed_one, 12 blocks of
forward_with_cache (LayerNorm, fused Q|K|V Q8_0 linear, KV-cache attention,
out projection, residual, LayerNorm, up + GELU, down, residual), the final
LayerNorm, the tied Q8_0 head (50257 x 768) and the fused sampler (GPT-2
softmax -> ln bridge, temperature 0.8, top-k 40, top-p 0.95, repetition
penalty 1.1 over a 128-id window, one host draw), whose id feeds the next
step's embedding on the device.  The 12 blocks run as one launch
(k_gpt2_stack), then the LayerNorm-prologue head GEMV and the sampler: three
launches per token.  Random-init N(0, 0.02) weights, Q8_0-encoded on the GPU.

Residency: three model replicas (3 x 131 MB of Q8_0 + their caches, above the
256 MB MALL) are used in rotation, so every step streams its weights from HBM
("hbm-forced").  The step is captured once per replica into a HIP graph
(torch.cuda.CUDAGraph) and replayed; K timed steps are bracketed by
synchronisations and HIP events.

roofline: the step's dominant kernel, k_gpt2_stack (all 12 blocks), timed
alone (a graph of 12 launches taking the replicas in turn, so each streams
its blocks from HBM; HIP events on its stream);
algorithmic bytes per launch = the 48 layer weights' Q8_0 bytes + the K and V
cache rows it reads (2 x 12 x 256 x 768 x 4 at position 255).  The kernel is
bound by its 60 dependent exchanges between workgroups, not by HBM; the
fraction says how far from the HBM roofline that leaves it.  The lm_head GEMV
roofline (41.2 MB per launch, the largest HBM stream of the step) is reported
beside it.

cpu_baseline: the CPU oracle (oracle/, ferrum_core's arithmetic restated in C,
"port") on one host core — ferrum_core runs the m=1 linear serially at any
thread count (parallel.rs:90-92) — running the same whole decode step over
f32-expanded weights as the reference's loader builds them, at position 255
of a randomly filled KV cache, for a bounded number of steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ferrum-cpu_amd"))

D, L, FFN, V, N_RECENT = 768, 12, 3072, 50257, 128
LAYER_SHAPES = [(3 * D, D), (D, D), (FFN, D), (D, FFN)]  # (n_rows, k): QKV, attn-out, up, down
HBM_PEAK_GBS = 8000.0
SAMPLER = dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1)


B32 = 32
# GPT-2-medium: 24 layers, d 1024, MLP 4096; prefill
# of 32 prompts x 512 tokens = 16,384 activation rows per linear.
MED_D, MED_L, MED_FFN, MED_M = 1024, 24, 4096, 32 * 512
MED_SHAPES = [(3 * MED_D, MED_D), (MED_D, MED_D), (MED_FFN, MED_D), (MED_D, MED_FFN)]
F16_DENSE_TFLOPS, I8_DENSE_TOPS = 2500.0, 5000.0
HEADS, CTX, FULL_POS = 12, 1024, 255  # GPT-2-124M attention; the whole-step leg's position

COPY_BYTES = 256 << 20
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemv_q8_0_lm_head_pmc.json")
STACK_PMC = os.path.join(ROOT, "profiles", "gpt2_stack_124m_pmc.json")
B32_UP_PMC = os.path.join(ROOT, "profiles", "skinny_gemm_b32_up_pmc.json")
QWEN_GU_PMC = os.path.join(ROOT, "profiles", "skinny_gemm_qwen_gate_up_pmc.json")


def q8_bytes(n, k):
    return n * k // 32 * 34


def measured_traffic(path):
    """HBM bytes per launch of a kernel from its committed counter runs
    (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy of known size); None when
    that summary is absent."""
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def make_weight(ctx, fh, torch, n, k, gen):
    """N(0, 0.02) weight [n, k] -> GGUF Q8_0 bytes (GPU encoder) -> device weight."""
    w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    raw = torch.empty(q8_bytes(n, k), dtype=torch.uint8, device="cuda")
    fh.q8_0_encode_async(ctx, w, n * k, raw)
    wt = fh.Q8_0Weight.upload_device(ctx, raw, n, k)
    ctx.sync()
    del w, raw
    return wt


def launch_roofline(ctx, torch, calls, bytes_per_launch, launches=240):
    """A kernel's roofline line: one HIP graph of `launches` back-to-back
    launches cycling over `calls` (one per weight replica, so the weights
    stream from HBM), timed with HIP events on the stream the graph replays
    on; achieved = algorithmic bytes per launch / average launch time."""
    for c in calls:
        c()
    ctx.sync()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        for i in range(launches):
            calls[i % len(calls)]()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    del g
    gbps = bytes_per_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBS, 4), "traffic": None, "avg_launch_us": round(us, 3),
            "bytes_per_launch": bytes_per_launch}


def copy_for_counters(torch, dev):
    """A plain device copy of known size (COPY_BYTES), five times, for scaling
    the PMC byte counters (FETCH_SIZE / WRITE_SIZE) of the same run."""
    src = torch.empty(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()


class Replica:
    def __init__(self, ctx, fh, torch, gen):
        self.layers = [[make_weight(ctx, fh, torch, n, k, gen) for (n, k) in LAYER_SHAPES] for _ in range(L)]
        self.head = make_weight(ctx, fh, torch, V, D, gen)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--replicas", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--leg", choices=["all", "stack", "head", "prefill", "qwen", "qlinear", "dropin", "b32"],
                    default="all",
                    help="'stack': only the whole decode step and its one-launch block stack (for profiles and "
                         "counter runs); 'b32': only the batch-32 step; 'head': only the lm_head GEMV roofline leg; "
                         "'prefill': only the "
                         "GPT-2-medium prefill GEMMs; 'qwen': only the Qwen2-shaped batch-64 step; 'qlinear': only "
                         "the per-row int8 and int4 qlinear steps; 'dropin': the blocking per-call linear and the "
                         "exact mode")
    ap.add_argument("--prefill-steps", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the Q8_0 decode path is sized for one MI355X and has no multi-GPU leg.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import ferrum_hip as fh

    torch.cuda.init()
    dev = torch.device("cuda:0")
    ctx = fh.Context(0)
    stream = torch.cuda.Stream()  # every launch and event of the run goes on this stream
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    x_d = torch.randn((1, D), generator=gen, device=dev)
    x_f = torch.randn((1, FFN), generator=gen, device=dev)
    y_big = torch.empty((1, max(3 * D, FFN)), device=dev)
    # the head's scores as the hot path produces them: N(0,1) activations
    # through N(0, 0.02) weights give scores of spread 0.02 * sqrt(768)
    logits = torch.randn((1, V), generator=gen, device=dev) * (0.02 * D ** 0.5)
    biases = {n: torch.randn(n, generator=gen, device=dev) * 0.1 for n in {s[0] for s in LAYER_SHAPES}}
    rec = torch.from_numpy(np.random.default_rng(3).integers(0, V, size=N_RECENT).astype(np.uint32)).to(dev)
    rec_off = torch.tensor([0, N_RECENT], dtype=torch.int32, device=dev)
    draws = torch.tensor([0x1234_5678_9ABC_DEF1], dtype=torch.int64, device=dev)  # u64 bit pattern
    out_id = torch.zeros(1, dtype=torch.int32, device=dev)
    params = fh.SamplingParams(**SAMPLER)

    def head_gemv(rep):
        fh.linear_forward_async(ctx, rep.head, x_d, 1, D, None, 0, logits)

    def step(rep):
        for li in range(L):
            for (n, k), w in zip(LAYER_SHAPES, rep.layers[li]):
                fh.linear_forward_async(ctx, w, x_d if k == D else x_f, 1, k, biases[n], n, y_big)
        head_gemv(rep)
        fh.sample_rows_async(ctx, logits, 1, V, params, rec, rec_off, draws, out_id, fh.LOGITS_GPT2_SOFTMAX)

    result = {}

    def timed(gs, steps, warmup):
        for i in range(warmup):
            gs[i % len(gs)].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for i in range(steps):
            gs[i % len(gs)].replay()
        e1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        return e0.elapsed_time(e1) / steps, wall / steps

    def capture(fn, items):
        """One HIP graph per item: fn(item) run once eagerly (grows the
        context's areas outside capture), then captured."""
        for it in items:
            fn(it)
        torch.cuda.synchronize()
        ctx.sync()
        graphs = []
        for it in items:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                ctx.set_stream(torch.cuda.current_stream().cuda_stream)
                fn(it)
            ctx.set_stream(stream.cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        return graphs

    if args.leg in ("all", "stack"):
        # ---- the whole decode step (the headline) ----------------------------------
        models = [fh.GPT2Device.random(ctx, V, D, HEADS, L, FFN, CTX, gen) for _ in range(args.replicas)]
        assert all(m.stack is not None for m in models), "the one-launch block stack is not available"

        def full_step(mdl):
            mdl.feed_async(mdl.token, FULL_POS)
            fh.sample_rows_async(ctx, mdl.z, 1, V, params, rec, rec_off, draws, mdl.token, fh.LOGITS_GPT2_SOFTMAX)

        graphs_f = capture(full_step, models)
        ms_full, wall_full = timed(graphs_f, args.steps, args.warmup)
        ms_full_mall, _ = timed(graphs_f[:1], args.steps, args.warmup)
        del graphs_f
        ctx.sync()  # raises if any exchange of the timed steps gave up
        # The same steps with one graph holding a step per replica (three
        # consecutive steps): what a decode loop that keeps its token on the
        # device gets by capturing several steps at once (no host launch and
        # graph boundary between them).
        graphs_3 = capture(lambda _: [full_step(mdl) for mdl in models], [None])
        ms_g3, _ = timed(graphs_3, max(args.steps // len(models), 1), max(args.warmup // len(models), 1))
        ms_full_multi = ms_g3 / len(models)
        del graphs_3
        ctx.sync()

        # Config 3 as a run: a 128-token random prompt fed position by
        # position, then 256 steps sampled on the device (the sampler's id
        # feeds the next step's embedding; GPT2Device.generate), one model
        # (131 MB: it stays in the 256 MB MALL across steps, as a real run's
        # would).  Prime time from a 1-step run; EOS is not special here.
        m3 = models[0]
        prompt = [int(t) for t in np.random.default_rng(128).integers(0, V, 128)]
        m3.generate(prompt, 8, params, fh.Rng(1))  # warm-up (areas, code)
        t0 = time.perf_counter()
        m3.generate(prompt, 1, params, fh.Rng(2))
        t_prime = time.perf_counter() - t0
        # (the wall clock at the end of the prime and of each 32-step chunk is
        # recorded, and the run is repeated: some processes have run it at
        # about half speed, so the record shows where such a run loses time)
        chunks, chunks2 = [], []
        t0 = time.perf_counter()
        run_ids = m3.generate(prompt, 256, params, fh.Rng(3), timings=chunks)
        t_run = time.perf_counter() - t0
        t0 = time.perf_counter()
        m3.generate(prompt, 256, params, fh.Rng(3), timings=chunks2)
        t_run2 = time.perf_counter() - t0
        # the same run with the prompt primed in one pass (prefill=True: its
        # 127 positions as rows of GEMMs and one attention launch per block)
        m3.generate(prompt, 8, params, fh.Rng(1), prefill=True)
        t0 = time.perf_counter()
        m3.generate(prompt, 1, params, fh.Rng(2), prefill=True)
        t_prime_pf = time.perf_counter() - t0
        t0 = time.perf_counter()
        run_ids_pf = m3.generate(prompt, 256, params, fh.Rng(3), prefill=True)
        t_run_pf = time.perf_counter() - t0
        result["config3_run"] = {
            "prompt": 128, "steps": len(run_ids), "run_ms": round(t_run * 1e3, 2), "prime_ms": round(t_prime * 1e3, 2),
            "run_marks_ms": chunks, "repeat_run_ms": round(t_run2 * 1e3, 2), "repeat_marks_ms": chunks2,
            "decode_tok_s": round(255 / max(t_run - t_prime, 1e-9), 1), "run_tok_s": round(len(run_ids) / t_run, 1),
            "prefill": {"run_ms": round(t_run_pf * 1e3, 2), "prime_ms": round(t_prime_pf * 1e3, 2),
                        "run_tok_s": round(len(run_ids_pf) / t_run_pf, 1),
                        "same_ids": run_ids_pf == run_ids},
            "residency": "one model (131 MB, MALL-resident)", "sampler": SAMPLER,
            "what": "GPT2Device.generate: prompt fed position by position (prefill: in one pass), then stack + "
                    "head + sampler per step, wall clock around the whole run (host launches included)"}

        # the dominant kernel alone: k_gpt2_stack, 12 launches per graph taking
        # the replicas in turn, so every launch streams its blocks from HBM as
        # in the timed step (one replica's 131 MB would stay in the MALL)
        n_stack = 4 * len(models)

        def stack_only(_):
            for i in range(n_stack):
                mdl = models[i % len(models)]
                ctx.check(fh.lib().fh_gpt2_stack_forward_async(ctx.h, mdl.stack, mdl.token.data_ptr(), FULL_POS,
                                                               mdl.x.data_ptr()))

        graphs_s = capture(stack_only, [None])
        ms_stack, _ = timed(graphs_s, max(args.steps // n_stack, 5), max(args.warmup // n_stack, 2))
        stack_us = ms_stack / n_stack * 1e3
        del graphs_s
        ctx.sync()

        # the same step one launch per op (64 launches), for comparison
        for mdl in models:
            mdl.fused = False
        graphs_p = capture(full_step, models)
        ms_perop, _ = timed(graphs_p, max(args.steps // 4, 10), args.warmup)
        del graphs_p
        for mdl in models:
            mdl.fused = True

        # Sampler alone: one 50257-wide row (GPT-2 bridge, config-3 params),
        # 50 launches captured in one graph so the host's launch rate is not
        # what is timed.
        ns, nrep = 50, 20
        gs = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gs):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            for _ in range(ns):
                fh.sample_rows_async(ctx, logits, 1, V, params, rec, rec_off, draws, out_id, fh.LOGITS_GPT2_SOFTMAX)
        ctx.set_stream(stream.cuda_stream)
        gs.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(nrep):
            gs.replay()
        e1.record()
        torch.cuda.synchronize()
        sampler_us = e0.elapsed_time(e1) / (ns * nrep) * 1e3
        del gs
        for mdl in models:
            mdl.free()
        del models
        torch.cuda.synchronize()

        layer_bytes = sum(q8_bytes(n, k) for (n, k) in LAYER_SHAPES) * L
        kv_bytes = 2 * L * (FULL_POS + 1) * D * 4
        head_bytes_ln = q8_bytes(V, D) + 4 * D + 4 * V
        step_bytes = layer_bytes + kv_bytes + head_bytes_ln + 4 * V  # + the sampler's logits read
        stack_bytes = layer_bytes + kv_bytes
        stack_gbps = stack_bytes / (stack_us * 1e-6) / 1e9
        result.update(ms_full=ms_full, wall_full=wall_full, ms_full_mall=ms_full_mall, ms_perop=ms_perop,
                      ms_full_multi=ms_full_multi,
                      stack_us=stack_us, stack_bytes=stack_bytes, stack_gbps=stack_gbps, step_bytes=step_bytes,
                      sampler_us=sampler_us, kv_bytes=kv_bytes)
        if args.leg == "stack":
            # A plain device copy of known size, for scaling the PMC byte
            # counters (FETCH_SIZE / WRITE_SIZE) of the same run.
            src = torch.empty(COPY_BYTES // 4, device=dev)
            dst = torch.empty_like(src)
            for _ in range(5):
                dst.copy_(src)
            torch.cuda.synchronize()
            print(json.dumps({"leg": "stack", "stack_us": round(stack_us, 3), "stack_bytes": stack_bytes,
                              "stack_GBps": round(stack_gbps, 1), "ms_per_step": round(ms_full, 5),
                              "per_op_ms_per_step": round(ms_perop, 5), "copy_bytes_per_launch": COPY_BYTES,
                              "multi_step_graph_ms_per_step": round(ms_full_multi, 5),
                              "config3_run": result["config3_run"]}))
            return

    if args.leg in ("all", "b32"):
        reps = [Replica(ctx, fh, torch, gen) for _ in range(args.replicas)]
    if args.leg == "all":
        # ---- the hot path alone, unchained: the 49 Q8_0 linears on fixed
        # inputs + the sampler (no dependence between the linears) -------------
        graphs = capture(step, reps)
        ms_step, _ = timed(graphs, args.steps, args.warmup)
        del graphs
        result["hot_unchained"] = ms_step
        torch.cuda.synchronize()
    if args.leg in ("all", "b32"):

        # ---- batch 32: the same hot path for 32 sequences (BASELINE's b32 decode) ----
        B = B32
        xb_d = torch.randn((B, D), generator=gen, device=dev)
        xb_f = torch.randn((B, FFN), generator=gen, device=dev)
        yb = torch.empty((B, max(3 * D, FFN)), device=dev)
        logits_b = torch.empty((B, V), device=dev)
        rec_b = torch.from_numpy(np.random.default_rng(4).integers(0, V, size=B * N_RECENT).astype(np.uint32)).to(dev)
        off_b = torch.arange(0, (B + 1) * N_RECENT, N_RECENT, dtype=torch.int32, device=dev)
        draws_b = torch.from_numpy(np.random.default_rng(5).integers(0, 2**63, size=B, dtype=np.int64)).to(dev)
        out_b = torch.zeros(B, dtype=torch.int32, device=dev)

        def step_b(rep):
            for li in range(L):
                for (n, k), w in zip(LAYER_SHAPES, rep.layers[li]):
                    fh.linear_forward_async(ctx, w, xb_d if k == D else xb_f, B, k, biases[n], n, yb)
            fh.linear_forward_async(ctx, rep.head, xb_d, B, D, None, 0, logits_b)
            fh.sample_rows_async(ctx, logits_b, B, V, params, rec_b, off_b, draws_b, out_b, fh.LOGITS_GPT2_SOFTMAX)

        graphs_b = capture(step_b, reps)
        ms_b, _ = timed(graphs_b, max(args.steps // 4, 10), args.warmup)
        b32_bytes = L * sum(q8_bytes(n, k) for (n, k) in LAYER_SHAPES) + q8_bytes(V, D)
        result["b32_unchained"] = {
            "tok_s": round(B * 1000.0 / ms_b, 1), "ms_per_step": round(ms_b, 5), "batch": B,
            "sampler_rows": B, "residency": f"hbm-forced ({args.replicas} weight replicas)",
            "weight_bytes": b32_bytes, "weight_GBps": round(b32_bytes / (ms_b * 1e-3) / 1e9, 1),
            "what": "48 Q8_0 skinny GEMMs at m = 32 (k_gemm_skinny) + the 50257 x 768 head "
                    "(k_gemm_wide) + 32 sampler rows, unchained inputs"}
        del graphs_b, reps
        torch.cuda.synchronize()

        # ---- batch 32, the whole step: 32 GPT-2-124M sequences at position
        # 255 (GPT2Batch: embedding, 12 blocks with each row's attention over
        # its own 256 cached positions, final LayerNorm, head, 32 sampler rows
        # over each row's 256-id window); the sampled ids feed the next step
        bmodels = [fh.GPT2Device.random(ctx, V, D, HEADS, L, FFN, CTX, gen) for _ in range(args.replicas)]
        P1 = FULL_POS + 1
        batches = [fh.GPT2Batch(mdl, B, P1) for mdl in bmodels]
        tok_b = torch.from_numpy(np.random.default_rng(6).integers(0, V, size=B).astype(np.int32)).to(dev)
        pos_b = torch.full((B,), FULL_POS, dtype=torch.int32, device=dev)
        hist_b = torch.from_numpy(np.random.default_rng(7).integers(0, V, size=(B, P1)).astype(np.int32)).to(dev)
        rng_b = torch.tensor([[r * P1, (r + 1) * P1] for r in range(B)], dtype=torch.int32, device=dev)

        def full_b(bt):
            bt.feed_async(tok_b, pos_b, FULL_POS, hist_b, P1)
            fh.sample_rows_async(ctx, bt.z, B, V, params, hist_b, rng_b, draws_b, tok_b,
                                 fh.LOGITS_GPT2_SOFTMAX | fh.RECENT_RANGES)

        graphs_fb = capture(full_b, batches)
        ms_fb, wall_fb = timed(graphs_fb, max(args.steps // 4, 10), args.warmup)
        del graphs_fb
        ctx.sync()
        kv_bytes = B * L * 2 * P1 * D * 4
        fb_bytes = b32_bytes + kv_bytes
        result["b32"] = {
            "tok_s": round(B * 1000.0 / ms_fb, 1), "ms_per_step": round(ms_fb, 5), "wall_ms_per_step": round(wall_fb, 5),
            "batch": B, "position": FULL_POS, "sampler": SAMPLER, "launches_per_step": batches[0].launches_per_step() + 1,
            "residency": f"hbm-forced ({len(batches)} model replicas, each with its own 32 KV caches)",
            "weight_bytes": b32_bytes, "kv_cache_bytes_read": kv_bytes,
            "GBps": round(fb_bytes / (ms_fb * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(fb_bytes / (ms_fb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "what": "GPT2Batch: the whole decode step of 32 sequences (embedding, 12 blocks with per-row "
                    "attention, final LayerNorm, head, fused sampler; ids fed back on the device)"}
        del batches
        for mdl in bmodels:
            mdl.free()
        del bmodels
        torch.cuda.synchronize()

        # ---- the step's dominant kernel family, the LayerNorm-in skinny GEMMs
        # (24 of the 65 launches): the MLP up projection, 3072 x 768 at m = 32
        # with GELU out, alone over 128 weight replicas (320 MB, HBM-forced)
        ups = [make_weight(ctx, fh, torch, FFN, D, gen) for _ in range(128)]
        xu = torch.randn((B, D), generator=gen, device=dev)
        stu = torch.rand((B, D // 32, 2), generator=gen, device=dev)
        gu, bu, biu = torch.ones(D, device=dev), torch.zeros(D, device=dev), torch.zeros(FFN, device=dev)
        yu = torch.empty((B, FFN), device=dev)
        calls = [(lambda w=w: fh.linear_normed_async(ctx, w, xu, B, D, stu, gu, bu, 1e-5, False, biu, FFN, yu,
                                                     fh.ACT_GELU)) for w in ups]
        up_bytes = q8_bytes(FFN, D) + 4 * B * D + 8 * B * (D // 32) + 8 * D + 4 * FFN + 4 * B * FFN
        roof = launch_roofline(ctx, torch, calls, up_bytes)
        roof["kernel"] = ("k_gemm_skinny<1,1,3,LayerNorm in> (MLP up 3072 x 768 at m = 32, GELU out; the step's "
                          "24 LayerNorm-in GEMMs are its largest kernel family)")
        roof["traffic"] = measured_traffic(B32_UP_PMC)
        roof["bytes_note"] = "Q8_0 weight + x + row statistics + gamma/beta + bias + y"
        result["b32"]["roofline"] = roof
        for w in ups:
            w.free()
        del ups, calls
        torch.cuda.synchronize()
        if args.leg == "b32":
            copy_for_counters(torch, dev)
            print(json.dumps({"leg": "b32", "b32": result["b32"], "b32_unchained": result["b32_unchained"],
                              "copy_bytes_per_launch": COPY_BYTES}))
            return

    if args.leg in ("all", "dropin"):
        result["dropin"] = dropin_leg(ctx, fh, torch, gen, dev)
    if args.leg == "dropin":
        print(json.dumps({"leg": "dropin", "dropin": result["dropin"]}))
        return

    if args.leg in ("all", "prefill"):
        result["prefill"] = prefill_leg(ctx, fh, torch, gen, dev, args.prefill_steps)

    if args.leg == "prefill":
        print(json.dumps({"leg": "prefill", "prefill": result["prefill"]}))
        return

    if args.leg in ("all", "qlinear"):
        result["qlinear_gpu"] = qlinear_gpu_leg(ctx, fh, torch, dev, max(args.steps // 10, 10), args.replicas, fh.QINT8)
        result["qlinear4_gpu"] = qlinear_gpu_leg(ctx, fh, torch, dev, max(args.steps // 10, 10), args.replicas, fh.QINT4)
    if args.leg == "qlinear":
        print(json.dumps({"leg": "qlinear", "qlinear_int8_gpu": result["qlinear_gpu"],
                          "qlinear_int4_gpu": result["qlinear4_gpu"]}))
        return

    if args.leg in ("all", "qwen"):
        result["qwen2_b64"] = qwen_leg(ctx, fh, torch, gen, dev, max(args.steps // 20, 10), args.warmup)
    if args.leg == "qwen":
        copy_for_counters(torch, dev)
        print(json.dumps({"leg": "qwen", "qwen2_b64": result["qwen2_b64"], "copy_bytes_per_launch": COPY_BYTES}))
        return

    # ---- roofline leg: lm_head GEMV, back-to-back, HBM-forced ----------------------
    n_head_rep = 32  # 32 x 41 MB = 1.3 GB, five times the MALL
    heads = [make_weight(ctx, fh, torch, V, D, gen) for _ in range(n_head_rep)]
    hr = [type("H", (), {"head": h})() for h in heads]
    for i in range(3 * n_head_rep):
        head_gemv(hr[i % n_head_rep])
    torch.cuda.synchronize()
    launches = 400 if args.leg == "all" else 200
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(launches):
        head_gemv(hr[i % n_head_rep])
    e1.record()
    torch.cuda.synchronize()
    head_us = e0.elapsed_time(e1) / launches * 1e3
    head_bytes = q8_bytes(V, D) + 4 * D + 4 * V
    achieved = head_bytes / (head_us * 1e-6) / 1e9
    head_roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(PMC_SUMMARY),
                "kernel": "k_gemv_w8a32<16,3,1,4,false,false> (lm_head 50257x768, Q8_0, m=1)",
                "avg_launch_us": round(head_us, 3), "bytes_per_launch": head_bytes}
    copy_GBps = None
    if args.leg == "all":  # (kept out of the counter runs: their copy calibration must see one size)
        # One GPU's share of a vocabulary-sharded head (50257 / 8 rows), the unit
        # the multi-GPU design would run per rank; HBM-forced over 64 replicas.
        shard_rows = (V + 7) // 8
        shards = [make_weight(ctx, fh, torch, shard_rows, D, gen) for _ in range(64)]
        shard_out = torch.empty((1, shard_rows), device=dev)
        for i in range(64):
            fh.linear_forward_async(ctx, shards[i], x_d, 1, D, None, 0, shard_out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(400):
            fh.linear_forward_async(ctx, shards[i % 64], x_d, 1, D, None, 0, shard_out)
        e1.record()
        torch.cuda.synchronize()
        shard_us = e0.elapsed_time(e1) / 400 * 1e3
        shard_bytes = q8_bytes(shard_rows, D) + 4 * D + 4 * shard_rows
        result["shard_head"] = {"rows": shard_rows, "k": D, "us": round(shard_us, 3),
                                "GBps": round(shard_bytes / (shard_us * 1e-6) / 1e9, 1)}
        for w in shards:
            w.free()
        del shards

        # Measured device copy bandwidth (1 GiB buffers, read + write counted), beside the 8 TB/s spec.
        cbytes = 1 << 30
        csrc = torch.empty(cbytes // 4, device=dev)
        cdst = torch.empty_like(csrc)
        for _ in range(3):
            cdst.copy_(csrc)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            cdst.copy_(csrc)
        e1.record()
        torch.cuda.synchronize()
        copy_GBps = 2 * cbytes * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
        del csrc, cdst

    if args.leg == "head":
        # A plain device copy of known size, for scaling the PMC byte counters
        # (FETCH_SIZE / WRITE_SIZE) of the same run.
        src = torch.empty(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"leg": "head", "roofline": head_roofline, "copy_bytes_per_launch": COPY_BYTES}))
        return

    # ---- CPU baseline: the oracle on this host, one core ----------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)

    ms = result["ms_full"]
    line = {
        "metric": "decode tok/s GPT-2-124M Q8_0 b1 (whole step: embedding, 12 blocks, head, fused sampler)",
        "value": round(1000.0 / ms, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init N(0,0.02) Q8_0 weights, random token history)",
        "config": {"workload": "gpt2-124m-q8_0-decode-step", "batch": 1, "layers": L, "d_model": D, "heads": HEADS,
                   "ffn": FFN, "vocab": V, "position": FULL_POS, "numerics": "W8A32 (ferrum_core)",
                   "sampler": SAMPLER, "launches_per_step": 3,
                   "residency": f"hbm-forced ({args.replicas} model replicas, "
                                f"{args.replicas * result['step_bytes'] / 1e6:.0f} MB > 256 MB MALL)"},
        "roofline": {"bound": "hbm", "achieved": round(result["stack_gbps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(result["stack_gbps"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(STACK_PMC),
                     "kernel": "k_gpt2_stack<768,64,48> (12 GPT-2 blocks, one launch, 48 workgroups + 24 that "
                               "warm each next block's weights in the memory-side cache)",
                     "avg_launch_us": round(result["stack_us"], 3), "bytes_per_launch": result["stack_bytes"],
                     "note": "bound by 60 dependent phases between workgroups (an exchange of ~2 us plus each "
                             "phase's serial LDS/barrier/VALU work), not by HBM"},
        "step_roofline": {"bytes_per_step": result["step_bytes"],
                          "achieved_GBps": round(result["step_bytes"] / (ms * 1e-3) / 1e9, 1),
                          "frac": round(result["step_bytes"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline_lm_head": head_roofline,
        "cpu_baseline": cpu,
        "mall_resident_tok_s": round(1000.0 / result["ms_full_mall"], 1),
        "multi_step_graph": {"tok_s": round(1000.0 / result["ms_full_multi"], 1),
                             "ms_per_step": round(result["ms_full_multi"], 5),
                             "what": "the same HBM-forced steps, three consecutive steps (one per replica) per graph"},
        "per_op_launches_tok_s": round(1000.0 / result["ms_perop"], 1),
        "hot_path_unchained": {"tok_s": round(1000.0 / result["hot_unchained"], 1),
                               "ms_per_step": round(result["hot_unchained"], 5),
                               "what": "the 49 Q8_0 linears on fixed inputs (no dependence between them) + sampler"},
        "config3_run": result["config3_run"],
        "sampler_us_per_row": round(result["sampler_us"], 2),
        "wall_ms_per_step": round(result["wall_full"], 5),
        "b32": result["b32"],
        "b32_unchained": result["b32_unchained"],
        "prefill": result["prefill"],
        "qwen2_b64": result.get("qwen2_b64"),
        "dropin_linear": result.get("dropin"),
        "qlinear_int8_gpu": result.get("qlinear_gpu"),
        "qlinear_int4_gpu": result.get("qlinear4_gpu"),
        "hbm_copy_GBps": round(copy_GBps, 1) if copy_GBps else None,
        "shard_head_gemv": result["shard_head"],
    }
    print(json.dumps(line))


def dropin_leg(ctx, fh, torch, gen, dev, calls=200):
    """The drop-in boundary as ferrum_core's Linear would call it: the blocking
    fh_q8_0_linear (host x and bias in, host y out; it allocates device
    buffers, copies in, runs, copies out and synchronises per call), timed on
    the host per call at m = 1 for the GPT-2-124M shapes, beside the device
    form's kernel time (HIP events, one weight: MALL-resident) and the opt-in
    bit-exact mode (FH_W8A32_EXACT, device form)."""
    import numpy as np

    out = {}
    for (n, k) in LAYER_SHAPES + [(V, D)]:
        w = make_weight(ctx, fh, torch, n, k, gen)
        x = np.random.default_rng(n + k).standard_normal((1, k), dtype=np.float32)
        b = np.random.default_rng(n).standard_normal(n, dtype=np.float32) if n != V else None
        for _ in range(5):
            fh.linear_forward(ctx, x, w, b)
        t0 = time.perf_counter()
        for _ in range(calls):
            fh.linear_forward(ctx, x, w, b)
        blocking_us = (time.perf_counter() - t0) / calls * 1e6
        dx = torch.from_numpy(x).to(dev)
        db = None if b is None else torch.from_numpy(b).to(dev)
        dy = torch.empty((1, n), device=dev)
        row = {"blocking_us": round(blocking_us, 2)}
        for name, mode in (("async_us", fh.W8A32), ("exact_async_us", fh.W8A32_EXACT)):
            for _ in range(5):
                fh.linear_forward_async(ctx, w, dx, 1, k, db, 0 if b is None else n, dy, mode)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(calls):
                fh.linear_forward_async(ctx, w, dx, 1, k, db, 0 if b is None else n, dy, mode)
            e1.record()
            torch.cuda.synchronize()
            row[name] = round(e0.elapsed_time(e1) / calls * 1e3, 3)
        ctx.sync()
        w.free()
        out[f"{n}x{k}"] = row
    out["what"] = ("m = 1, one weight per shape (MALL-resident); blocking = host wall clock per fh_q8_0_linear call "
                   "(host arrays), async = the device form's time per launch (HIP events, back to back)")
    return out


def prefill_leg(ctx, fh, torch, gen, dev, steps):
    """GPT-2-medium prefill linears: 24 x [QKV, attn-out, up, down] at m = 16,384
    (32 prompts x 512 tokens), W8A32 on the f16 matrix cores, then the same in
    W8A8 (bit-exact, then the fast mode).  One step = the 96 GEMMs (bias added),
    captured into one graph; FLOPs = 2 m n k per GEMM."""
    import numpy as np

    layers = [[make_weight(ctx, fh, torch, n, k, gen) for (n, k) in MED_SHAPES] for _ in range(MED_L)]
    biases = {n: torch.randn(n, generator=gen, device=dev) * 0.1 for n in {s[0] for s in MED_SHAPES}}
    x = {k: torch.randn((MED_M, k), generator=gen, device=dev) for k in {s[1] for s in MED_SHAPES}}
    y = torch.empty((MED_M, max(s[0] for s in MED_SHAPES)), device=dev)

    def step(numerics):
        for li in range(MED_L):
            for (n, k), w in zip(MED_SHAPES, layers[li]):
                fh.linear_forward_async(ctx, w, x[k], MED_M, k, biases[n], n, y, numerics)

    def timed_graph(numerics):
        step(numerics)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            step(numerics)
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / steps, e0, e1

    flops = sum(2.0 * MED_M * n * k for (n, k) in MED_SHAPES) * MED_L
    ms, e0, e1 = timed_graph(fh.W8A32)
    tflops = flops / (ms * 1e-3) / 1e12
    ms8, _, _ = timed_graph(fh.W8A8)
    tops8 = flops / (ms8 * 1e-3) / 1e12
    ms8f, _, _ = timed_graph(fh.W8A8_FAST)
    tops8f = flops / (ms8f * 1e-3) / 1e12
    # Config 4's decode: the same model's linears at batch 32 (96 Q8_0 GEMMs at
    # m = 32 + the 50257 x 1024 head) and the greedy sampler on the 32 rows;
    # 357 MB of Q8_0 per step, more than the MALL holds, so it streams from HBM.
    head = make_weight(ctx, fh, torch, V, MED_D, gen)
    xb = {k: torch.randn((B32, k), generator=gen, device=dev) for k in {s_[1] for s_ in MED_SHAPES}}
    yb = torch.empty((B32, max(s_[0] for s_ in MED_SHAPES)), device=dev)
    lb = torch.empty((B32, V), device=dev)
    ob = torch.zeros(B32, dtype=torch.int32, device=dev)
    greedy = fh.SamplingParams(temperature=0.0)

    def dstep():
        for li in range(MED_L):
            for (n, k), w in zip(MED_SHAPES, layers[li]):
                fh.linear_forward_async(ctx, w, xb[k], B32, k, biases[n], n, yb)
        fh.linear_forward_async(ctx, head, xb[MED_D], B32, MED_D, None, 0, lb)
        fh.sample_rows_async(ctx, lb, B32, V, greedy, None, None, None, ob)

    dstep()
    torch.cuda.synchronize()
    gd = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gd):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        dstep()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    gd.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(20):
        gd.replay()
    e1.record()
    torch.cuda.synchronize()
    dms = e0.elapsed_time(e1) / 20
    dbytes = MED_L * sum(q8_bytes(n, k) for (n, k) in MED_SHAPES) + q8_bytes(V, MED_D)
    del gd
    head.free()
    for lw in layers:
        for w in lw:
            w.free()
    del x, y, xb, yb, lb
    # Config 4's prompt attention alone: per block one launch for the 32
    # prompts (fh_attention_prefill_seqs_async: 511 positions each, 16 heads of
    # 64, fp32 matrix cores), 24 launches in a graph.  Useful flops: per
    # (sequence, head) sum over rows r of (r + 1) keys x 64 dims x 2 products
    # (q.k and p.v) x 2 flops.
    pa_rows, pa_cap = 511, 576
    pa_qkv = torch.randn((B32 * pa_rows, 3 * MED_D), generator=gen, device=dev)
    pa_k = torch.zeros((B32, pa_cap, MED_D), device=dev)
    pa_v = torch.zeros((B32, pa_cap, MED_D), device=dev)
    pa_out = torch.empty((B32 * pa_rows, MED_D), device=dev)

    def pa_step():
        for _ in range(MED_L):
            fh.attention_prefill_seqs_async(ctx, pa_qkv, pa_k, pa_v, pa_cap * MED_D, pa_cap, MED_D, 16, 0, pa_rows,
                                            B32, pa_out)

    pa_step()
    torch.cuda.synchronize()
    ga = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ga):
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        pa_step()
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    ga.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        ga.replay()
    e1.record()
    torch.cuda.synchronize()
    pa_ms = e0.elapsed_time(e1) / 5
    pa_flops = MED_L * B32 * 16 * (pa_rows * (pa_rows + 1) / 2) * 64 * 4
    pa_tflops = pa_flops / (pa_ms * 1e-3) / 1e12
    prompt_attention = {"ms": round(pa_ms, 3), "tflops": round(pa_tflops, 1),
                        "mfma_f16_tflops": round(3 * pa_tflops, 1),
                        "mfma_frac_f16_dense_peak": round(3 * pa_tflops / F16_DENSE_TFLOPS, 4),
                        "what": "configs[3]'s prompt attention: 24 blocks x 32 prompts x 511 positions x 16 heads of "
                                "64, causal, one launch per block (flash attention on the f16 matrix cores, each "
                                "f32 operand as two f16 terms: three f16 products per product; the block's k / v rows "
                                "read from q|k|v and written into the caches by the same launch); useful flops of "
                                "the causal triangle"}
    del ga, pa_qkv, pa_k, pa_v, pa_out
    # Config 4 as a run: GPT-2-medium (N(0, 0.02) Q8_0 weights), 32 prompts
    # of 512 random ids primed in one pass (GPT2Batch.prefill_async: the
    # linears at m = 32 x 511, one attention launch per block for all prompts),
    # then 64 greedy steps at batch 32 (every row's attention over its own
    # cache; the sampler's ids feed the next step on the device).  Wall clock
    # around the whole run; the prime from a one-step run.
    mm = fh.GPT2Device.random(ctx, V, MED_D, 16, MED_L, 4 * MED_D, 576, gen)
    cb = fh.GPT2Batch(mm, B32, 576)
    prompts = np.random.default_rng(512).integers(0, V, size=(B32, 512))
    cb.generate(prompts, 2, greedy, [])  # warm-up (areas, code)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cb.generate(prompts, 1, greedy, [])
    t_prime = time.perf_counter() - t0
    t0 = time.perf_counter()
    run = cb.generate(prompts, 64, greedy, [])
    t_run = time.perf_counter() - t0
    config4 = {"prompts": B32, "prompt_len": 512, "steps": 64, "run_ms": round(t_run * 1e3, 2),
               "prime_ms": round(t_prime * 1e3, 2),
               "decode_tok_s": round(B32 * 63 / max(t_run - t_prime, 1e-9), 1),
               "run_tok_s": round(B32 * 64 / t_run, 1), "ids_per_row": len(run[0]),
               "what": "GPT2Batch.generate on GPT-2-medium: one-pass prefill of 32 x 512 ids, then 64 greedy steps "
                       "at batch 32 on the device; wall clock incl. host launches"}
    del cb
    mm.free()
    # The library's route to the same accuracy (torch -> hipBLASLt, f16 GEMM):
    # without the per-block scale step, an f32-accurate product of an f32
    # activation and a Q8_0 weight (d * q: 19 significant bits) takes three
    # f16 products per pair (x_h w_h + x_h w_l + x_l w_h), one GEMM of depth
    # 3k.  The block-scaled kernel needs two (x_h q + x_l q, the scale applied
    # per block), so its own matrix-core work is a GEMM of depth 2k.
    lib_ms = 0.0
    for (n, k) in MED_SHAPES:
        a = torch.randn((MED_M, 3 * k), generator=gen, device=dev).half()
        b = torch.randn((3 * k, n), generator=gen, device=dev).half()
        for _ in range(2):
            torch.matmul(a, b)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(5):
            torch.matmul(a, b)
        e1.record()
        torch.cuda.synchronize()
        lib_ms += e0.elapsed_time(e1) / 5 * MED_L
        del a, b
    return {"workload": "gpt2-medium prefill linears, 32 x 512 tokens (m = 16384), W8A32 f16-MFMA",
            "ms": round(ms, 3), "tflops": round(tflops, 1),
            "frac_f16_dense_peak": round(tflops / F16_DENSE_TFLOPS, 4),
            "frac_i8_dense_peak": round(tflops / I8_DENSE_TOPS, 4),
            "mfma_f16_tflops": round(2 * tflops, 1), "mfma_frac_f16_dense_peak": round(2 * tflops / F16_DENSE_TFLOPS, 4),
            "library_f16_same_accuracy_ms": round(lib_ms, 3), "vs_library": round(lib_ms / ms, 3),
            "roofline": {"bound": "mfma", "achieved": round(2 * tflops, 1), "peak": F16_DENSE_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(2 * tflops / F16_DENSE_TFLOPS, 4), "traffic": None,
                         "kernel": "k_gemm_bscale (+ k_row_scales): f16 MFMA work of two f16 products per "
                                   "activation-weight pair (the h and l terms against the quants), per step of "
                                   "the 96 linears",
                         "note": "the per-block FMA step bounds it with the MFMA work: MFMA busy 34 % "
                                 "(profiles/prefill_gemm_gpt2_medium_kernels.md)"},
            "config4_run": config4, "prompt_attention": prompt_attention,
            "decode_b32": {"ms_per_step": round(dms, 4), "tok_s": round(B32 * 1000.0 / dms, 1),
                           "weight_bytes": dbytes, "weight_GBps": round(dbytes / (dms * 1e-3) / 1e9, 1),
                           "what": "gpt2-medium linears of a batch-32 step: 96 Q8_0 GEMMs + head + greedy sampler, "
                                   "unchained inputs"},
            "w8a8_int8_mfma": {"ms": round(ms8, 3), "tops": round(tops8, 1),
                               "frac_i8_dense_peak": round(tops8 / I8_DENSE_TOPS, 4),
                               "numerics": "W8A8 (activations re-quantised to Q8_0), bit-exact with the reference",
                               "roofline": {"bound": "mfma", "achieved": round(tops8, 1), "peak": I8_DENSE_TOPS,
                                            "unit": "TOP/s", "frac": round(tops8 / I8_DENSE_TOPS, 4), "traffic": None,
                                            "kernel": "k_gemm_w8a8_lds (+ fh_k_encode_panel): 2 m n k ops of "
                                                      "the int8 product per step of the 96 linears",
                                            "note": "bound by the reference's per-block rounding (a product and "
                                                    "a sum per output and block on the VALU): MFMA busy 29 %"}},
            "w8a8_fast": {"ms": round(ms8f, 3), "tops": round(tops8f, 1),
                          "frac_i8_dense_peak": round(tops8f / I8_DENSE_TOPS, 4),
                          "numerics": "FH_W8A8_FAST: W8A8's exact block dots, each block term fused into the sum "
                                      "(one FMA); within 1e-5 of W8A8"}}


def qlinear_gpu_leg(ctx, fh, torch, dev, steps, replicas, kind):
    """The reference's per-row int8 / int4 path on the GPU: the 49 ops::qlinear
    calls of a GPT-2-124M decode step (m = 1, bias-first ascending-p sums, the
    reference's bits), random levels and scales, `replicas` weight sets (HBM-
    forced), one graph per set.  int4 is the reference's default
    `run-gguf --quant`."""
    import numpy as np

    rng = np.random.default_rng(77)
    int4 = kind == fh.QINT4

    def qw(k, n):
        levels = (rng.integers(0, 256, size=k * ((n + 1) // 2), dtype=np.uint8) if int4
                  else rng.integers(-127, 128, size=k * n, dtype=np.int8).view(np.uint8))
        return fh.QWeight(ctx, np.abs(rng.standard_normal(k)).astype(np.float32) * 1e-3, levels, k, n, kind)

    shapes = [(k, n) for (n, k) in LAYER_SHAPES]  # QWeight: k input rows x n outputs
    sets = [([[qw(k, n) for (k, n) in shapes] for _ in range(L)], qw(D, V)) for _ in range(replicas)]
    bias = {n: torch.randn(n, device=dev) * 0.1 for n in {n for (_, n) in shapes} | {V}}
    xs = {k: torch.randn(k, device=dev) for k in (D, FFN)}
    y = torch.empty(V, device=dev)

    def step(ws, head):
        for layer in ws:
            for w in layer:
                fh.qlinear_async(ctx, w, xs[w.k], 1, w.k, bias[w.n], w.n, y)
        fh.qlinear_async(ctx, head, xs[D], 1, D, bias[V], V, y)

    graphs = []
    for ws, head in sets:
        step(ws, head)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            step(ws, head)
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        graphs.append(g)
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    rb = (lambda n: (n + 1) // 2) if int4 else (lambda n: n)  # level bytes per row
    qbytes = L * sum(k * rb(n) + 4 * k for (k, n) in shapes) + D * rb(V) + 4 * D
    for ws, head in sets:
        head.free()
        for layer in ws:
            for w in layer:
                w.free()
    del graphs
    torch.cuda.synchronize()
    return {"ms_per_step": round(ms, 4), "tok_s": round(1000.0 / ms, 1), "weight_bytes": qbytes,
            "weight_GBps": round(qbytes / (ms * 1e-3) / 1e9, 1), "residency": f"hbm-forced ({replicas} weight sets)",
            "what": f"49 ops::qlinear (per-row {'int4' if int4 else 'int8'}) of a GPT-2-124M step at m = 1, "
                    "bit-exact numerics"}


QWEN05 = dict(vocab=151936, d=896, n_heads=14, n_kv=2, head_dim=64, layers=24, ffn=4864, context=512,
              rope_type=1, rope_base=1e6, eps=1e-6)
QWEN_B, QWEN_POS, QWEN_HIST = 64, 255, 1024


def qwen_leg(ctx, fh, torch, gen, dev, steps, warmup):
    """Config 5: a Qwen2-0.5B-shaped decode step for 64 sequences on the
    device (embed, 24 x [RmsNorm, q|k|v Q8_0 linear, RoPE NEOX, GQA attention
    at position 255, output projection, residual + RmsNorm, gate|up Q8_0
    linear, SwiGLU, down], final RmsNorm, tied 151936 x 896 head) and the fused
    sampler on its [64 x 151936] scores (top-k 50, top-p 0.9, repetition
    penalty 1.05 over a 1024-token history per row); and the sampler alone on
    the configuration's logits, N(0, 3) plus 5 planted peaks (+12)."""
    import numpy as np

    B, V = QWEN_B, QWEN05["vocab"]
    rng = np.random.default_rng(55)
    peaks = rng.choice(V, 5, replace=False)
    # histories: 1024 ids per row, repeats included (multiplicity matters)
    hist = np.concatenate([rng.integers(0, V, QWEN_HIST - 24), np.repeat(peaks[:3], 8)])
    rec = torch.from_numpy(np.concatenate([rng.permutation(hist) for _ in range(B)]).astype(np.uint32)).to(dev)
    off = torch.arange(0, (B + 1) * QWEN_HIST, QWEN_HIST, dtype=torch.int32, device=dev)
    draws = torch.from_numpy(rng.integers(0, 2**63, size=B, dtype=np.int64)).to(dev)
    out = torch.zeros(B, dtype=torch.int32, device=dev)
    params = fh.SamplingParams(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.05)

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            fn()
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        for _ in range(max(warmup // 10, 2)):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / n

    logits = torch.randn((B, V), generator=gen, device=dev) * 3.0
    logits[:, torch.from_numpy(peaks).to(dev)] += 12.0
    sampler_ms = timed(lambda: fh.sample_rows_async(ctx, logits, B, V, params, rec, off, draws, out), steps * 4)
    del logits

    m = fh.LlamaDevice.random(ctx, QWEN05, B, gen)
    m.tokens.copy_(torch.from_numpy(rng.integers(0, V, B).astype(np.int32)).to(dev))
    m.pos.fill_(QWEN_POS)

    def step():
        m.feed_async(QWEN_POS)
        fh.sample_rows_async(ctx, m.z, B, V, params, rec, off, draws, m.tokens)

    ms = timed(step, steps)
    c = QWEN05
    qkv = c["n_heads"] * c["head_dim"] + 2 * c["n_kv"] * c["head_dim"]
    per_layer = [(qkv, c["d"]), (c["d"], c["n_heads"] * c["head_dim"]), (2 * c["ffn"], c["d"]), (c["d"], c["ffn"])]
    wbytes = sum(q8_bytes(n, k) for n, k in per_layer) * c["layers"] + q8_bytes(V, c["d"])
    flops = 2.0 * B * (sum(n * k for n, k in per_layer) * c["layers"] + V * c["d"])
    kv_bytes = 2 * c["layers"] * B * (QWEN_POS + 1) * c["n_kv"] * c["head_dim"] * 4
    launches = m.launches_per_step() + 1
    m.free()
    del m
    torch.cuda.synchronize()
    # the step's dominant kernel: the gate|up GEMM (9728 x 896 at m = 64,
    # RmsNorm in, SwiGLU out), alone over 36 weight replicas (333 MB)
    d, f2 = c["d"], 2 * c["ffn"]
    gus = [make_weight(ctx, fh, torch, f2, d, gen) for _ in range(36)]
    xg = torch.randn((B, d), generator=gen, device=dev)
    stg = torch.rand((B, d // 32, 2), generator=gen, device=dev)
    gg = torch.ones(d, device=dev)
    yg = torch.empty((B, c["ffn"]), device=dev)
    calls = [(lambda w=w: fh.linear_normed_async(ctx, w, xg, B, d, stg, gg, None, 1e-6, True, None, 0, yg,
                                                 fh.ACT_SWIGLU32)) for w in gus]
    gu_bytes = q8_bytes(f2, d) + 4 * B * d + 8 * B * (d // 32) + 4 * d + 4 * B * c["ffn"]
    roof = launch_roofline(ctx, torch, calls, gu_bytes)
    roof["kernel"] = ("k_gemm_skinny<2,2,1,RmsNorm in + SwiGLU out> (gate|up 9728 x 896 at m = 64; the step's "
                      "largest kernel)")
    roof["bytes_note"] = "Q8_0 weight + x + row statistics + gamma + y"
    roof["traffic"] = measured_traffic(QWEN_GU_PMC)
    for w in gus:
        w.free()
    del gus, calls
    torch.cuda.synchronize()
    gbps = (wbytes + kv_bytes) / (ms * 1e-3) / 1e9
    return {"workload": "qwen2-0.5b-shaped Q8_0 decode step, batch 64, position 255, tied head, fused sampler",
            "tok_s": round(B * 1000.0 / ms, 1), "ms_per_step": round(ms, 4), "launches_per_step": launches,
            "weight_bytes": wbytes, "kv_cache_bytes_read": kv_bytes, "gemm_gflop": round(flops / 1e9, 1),
            "hbm_GBps": round(gbps, 1), "frac_hbm_peak": round(gbps / HBM_PEAK_GBS, 4), "roofline": roof,
            "sampler_only": {"rows": B, "vocab": V, "us_per_step": round(sampler_ms * 1e3, 2),
                             "us_per_row": round(sampler_ms * 1e3 / B, 3),
                             "logits": "N(0,3) + 5 planted peaks (+12)", "history": QWEN_HIST,
                             "params": {"temperature": 0.8, "top_k": 50, "top_p": 0.9, "repetition_penalty": 1.05}},
            "data": "synthetic (random-init N(0,0.02) Q8_0 weights generated on the GPU)"}


def cpu_baseline(budget_s):
    """ferrum_core's whole decode step on the host CPU (the oracle, one core):
    CachedTransformer::feed at position 255 (embed_one, 12 x forward_with_cache,
    final LayerNorm, the tied head over the f32-expanded weights as the
    reference's loader builds them) + the softmax/ln bridge and the sampler."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    t_setup = time.perf_counter()
    rng = np.random.default_rng(7)
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
    layers = []
    for li in range(L):
        ws = []
        for (n, k) in LAYER_SHAPES:
            raw = oracle.quantize_weight(n, k, seed=li * 10 + n + k)
            ws.append((oracle.q8_0_to_ferrum_weight(raw, n, k), f32(rng.standard_normal(n) * 0.02)))
        ln = [f32(1.0 + rng.standard_normal(D) * 0.02), f32(rng.standard_normal(D) * 0.02),
              f32(1.0 + rng.standard_normal(D) * 0.02), f32(rng.standard_normal(D) * 0.02)]
        # the KV cache of positions 0 .. 254 (random rows: the step's work does not depend on them)
        kc = f32(rng.standard_normal((CTX, D)))
        vc = f32(rng.standard_normal((CTX, D)))
        layers.append((ws, ln, kc, vc))
    head_raw = oracle.quantize_weight(V, D, seed=99)
    head = oracle.q8_0_to_ferrum_weight(head_raw, V, D)          # [D, V], the tied head's f32 expansion
    tok_w = np.ascontiguousarray(head.T)                        # [V, D], the token table
    pos_w = f32(rng.standard_normal((CTX, D)) * 0.02)
    lnf = (f32(1.0 + rng.standard_normal(D) * 0.02), f32(rng.standard_normal(D) * 0.02))
    recent = list(rng.integers(0, V, size=N_RECENT))
    params = oracle.SamplingParams(**SAMPLER)
    orng = oracle.Rng(7)
    setup = time.perf_counter() - t_setup
    token = [int(recent[-1])]

    def one_step():
        x = oracle.embed_one(tok_w, pos_w, token[0], FULL_POS)[None, :]
        for (ws, ln, kc, vc) in layers:
            (wq, bq), (wo, bo), (wu, bu), (wd, bd) = ws
            h = oracle.layernorm(x, ln[0], ln[1])
            qkv = oracle.linear_forward(h, wq, bq, threads=1)[0]
            att = oracle.attention_decode(qkv, kc, vc, HEADS, FULL_POS)
            x = (x + oracle.linear_forward(att[None, :], wo, bo, threads=1)).astype(np.float32)
            h = oracle.layernorm(x, ln[2], ln[3])
            up = oracle.gelu(oracle.linear_forward(h, wu, bu, threads=1))
            x = (x + oracle.linear_forward(up, wd, bd, threads=1)).astype(np.float32)
        z = oracle.linear_forward(oracle.layernorm(x, *lnf), head, None, threads=1)
        l = oracle.ln_bridge(oracle.softmax_rows(z)[0])
        token[0] = oracle.sample_with_params(l, params, recent, orng)

    one_step()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        one_step()
        times.append(time.perf_counter() - t0)
    best, med = min(times), float(np.median(times))
    out = {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": 1, "kind": "port",
           "sample": f"{len(times)} whole GPT-2-124M decode steps at position {FULL_POS} (embed_one, 12 blocks with "
                     f"attention over a randomly filled KV cache, final LayerNorm, tied head; f32-expanded weights, "
                     f"serial m=1 as ferrum_core runs them; softmax/ln bridge + sampler) in {sum(times):.1f} s; "
                     f"median {med * 1e3:.1f} ms/step, best {best * 1e3:.1f} ms; setup {setup:.1f} s",
           "best_tok_s": round(1.0 / best, 3)}
    layers_w = [ws for (ws, _, _, _) in layers]
    x_d = f32(rng.standard_normal((1, D)))
    x_f = f32(rng.standard_normal((1, FFN)))

    # Second figure: the reference's only multi-core m = 1 decode, ops::qlinear
    # on per-row int8 QWeights (column split over T threads, min chunk 64).
    # Not the GPU path's numerics (those are GGUF Q8_0); a CPU bandwidth figure.
    nproc = os.cpu_count() or 1
    threads = max(1, min(nproc, 16))  # a one-GPU box's CPU share is 16 cores whatever nproc shows
    qlayers = [[(oracle.QWeight(w_kn, w_kn.shape[0], w_kn.shape[1], oracle.INT8), b) for (w_kn, b) in ws]
               for ws in layers_w]
    qhead = oracle.QWeight(head, head.shape[0], head.shape[1], oracle.INT8)
    zero_v = np.zeros(V, np.float32)

    def one_qstep():
        for ws in qlayers:
            for (qw, b), (n, k) in zip(ws, LAYER_SHAPES):
                oracle.qlinear(x_d if k == D else x_f, qw, b, threads=threads)
        z = oracle.qlinear(x_d, qhead, zero_v, threads=threads)
        l = oracle.ln_bridge(oracle.softmax_rows(z)[0])
        oracle.sample_with_params(l, params, recent, orng)

    one_qstep()
    qt = []
    t_end = time.perf_counter() + budget_s / 2
    while time.perf_counter() < t_end or len(qt) < 3:
        t0 = time.perf_counter()
        one_qstep()
        qt.append(time.perf_counter() - t0)
    qmed = float(np.median(qt))
    qbytes = sum(qw.q.size + qw.scales.size * 4 for ws in qlayers for (qw, _) in ws) + qhead.q.size + qhead.scales.size * 4
    out["host_nproc"] = nproc
    out["qlinear_int8"] = {"value": round(1.0 / qmed, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                           "weight_GBps": round(qbytes / qmed / 1e9, 2),
                           "sample": f"{len(qt)} GPT-2-124M hot-path steps (the 49 linears + head through ops::qlinear, per-row int8, "
                                     f"{qbytes / 1e6:.0f} MB/token, m = 1 column split over {threads} threads); "
                                     f"median {qmed * 1e3:.1f} ms/step"}
    return out


if __name__ == "__main__":
    main()
