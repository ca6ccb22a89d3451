"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference (ferrum_core, Rust) cannot be built in this image (no cargo or
rustc), so the fixtures are the oracle's outputs on seeded inputs, the oracle
itself being pinned by the reference's known-answer tests (tests/test_oracle_*).
Each fixture is data only (.npz without pickles) plus a sha256 manifest;
tests/test_golden.py re-derives every file from the oracle and checks it bit
for bit, tests/test_gpu_golden.py checks the HIP path against the files.

    python tests/golden/make_golden.py          # rewrite the fixtures
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

# (m, n, k, bias?) -- m = 1 and 2 take the GEMV, 3..64 the skinny GEMM, the rest the tiled GEMM
LINEAR_CASES = [(1, 64, 96, True), (2, 33, 256, False), (3, 67, 96, True), (8, 130, 256, True),
                (32, 65, 768, True), (33, 40, 160, False), (70, 96, 128, True), (5, 9, 4864, True)]
SAMPLER_PARAMS = [dict(temperature=0.0), dict(temperature=0.0, repetition_penalty=1.3),
                  dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.1),
                  dict(temperature=1.0), dict(temperature=0.7, top_k=1), dict(temperature=0.9, top_p=0.5),
                  dict(temperature=1.3, top_k=200, repetition_penalty=0.9)]


def codec_fixture(orc):
    rng = np.random.default_rng(101)
    blocks = [np.array([127, 0.5, 1.5, -0.5, -2.5, 2.4999, -126.5, 0.49] + [0] * 24, np.float32),  # quant.rs:357-365
              np.zeros(32, np.float32), np.full(32, 1e-30, np.float32), np.full(32, 1e-41, np.float32),
              np.array([np.nan] + [1.0] * 31, np.float32), np.array([-np.inf, 2.0] + [0.25] * 30, np.float32),
              np.full(32, 8.3e6, np.float32)]
    blocks.append((rng.standard_normal(32 * 64) * rng.choice([1e-3, 1.0, 1e3], 32 * 64)).astype(np.float32))
    x = np.concatenate(blocks).astype(np.float32)
    raw = orc.q8_0_encode(x)
    return dict(x=x, gguf=raw, dequant=orc.q8_0_dequant(raw, x.size))


def linear_fixture(orc):
    """Both numerics on the same inputs: y (W8A32, ops::linear_forward on the f32
    expansion), y8 (W8A8, llama.cpp order), the activation quants and, for the
    small cases, the exact int32 block dots."""
    out = {}
    for c, (m, n, k, has_bias) in enumerate(LINEAR_CASES):
        seed = 1000 * c + m + n + k
        raw = orc.quantize_weight(n, k, seed, 0.05)
        x = np.random.default_rng(seed + 1).standard_normal((m, k), dtype=np.float32)
        b = (np.random.default_rng(seed + 2).standard_normal(n, dtype=np.float32) * np.float32(0.1)
             if has_bias else np.zeros(0, np.float32))
        bias = b if has_bias else None
        w = np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
        _, qx = orc.q8_0_quantize_rows(x)
        out.update({f"c{c}_shape": np.array([m, n, k], np.int64), f"c{c}_gguf": raw, f"c{c}_x": x,
                    f"c{c}_bias": b, f"c{c}_y": orc.q8_0_linear(x, raw, n, bias),
                    f"c{c}_y8": orc.q8_0_linear_w8a8(x, raw, n, bias),
                    f"c{c}_mass": (np.abs(x.astype(np.float64)) @ w).astype(np.float32), f"c{c}_qx": qx})
        if m * n * (k // 32) <= 20000:
            out[f"c{c}_dots"] = orc.q8_0_block_dots(qx, raw, n)
    out["cases"] = np.array(len(LINEAR_CASES), np.int64)
    return out


def sampler_fixture(orc):
    """Rows x parameter sets; each row has its recent-id window and one draw.
    kind 0 = raw logits, 1 = GPT-2 softmax -> ln bridge in front."""
    rng = np.random.default_rng(7)
    out = {}
    rows = []
    for vocab, count, scale in [(4096, 6, 3.0), (50257, 1, 0.55), (7, 3, 1.0)]:
        for _ in range(count):
            rows.append((rng.standard_normal(vocab) * scale).astype(np.float32))
    for i, z in enumerate(rows):
        rec = rng.integers(0, z.size, size=min(128, z.size * 2)).astype(np.uint32)
        out[f"r{i}_logits"] = z
        out[f"r{i}_recent"] = rec
    out["rows"] = np.array(len(rows), np.int64)
    draws = rng.integers(0, 2**64, size=(len(SAMPLER_PARAMS), 2, len(rows)), dtype=np.uint64)
    ids = np.zeros((len(SAMPLER_PARAMS), 2, len(rows)), np.int64)
    margins = np.zeros((len(SAMPLER_PARAMS), 2, len(rows)), np.float64)
    for pi, kw in enumerate(SAMPLER_PARAMS):
        op = orc.SamplingParams(**kw)
        for kind in (0, 1):
            for i, z in enumerate(rows):
                row = orc.ln_bridge(orc.softmax_rows(z)[0]) if kind == 1 else z
                tok, info = orc.sample(row, op, out[f"r{i}_recent"], int(draws[pi, kind, i]))
                ids[pi, kind, i] = tok
                margins[pi, kind, i] = info.margin
    out.update(draws=draws, ids=ids, margins=margins,
               params=np.array([[kw.get("temperature", 1.0), kw.get("top_k", 0), kw.get("top_p", 1.0),
                                 kw.get("repetition_penalty", 1.0)] for kw in SAMPLER_PARAMS], np.float64))
    return out


def build_all(orc):
    return {"q8_0_codec.npz": codec_fixture(orc), "linear.npz": linear_fixture(orc), "sampler.npz": sampler_fixture(orc)}


def digest(arrays: dict) -> str:
    h = hashlib.sha256()
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        h.update(name.encode())
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def main():
    import oracle

    oracle.build()
    manifest = {}
    for name, arrays in build_all(oracle).items():
        np.savez_compressed(os.path.join(HERE, name), **arrays)
        manifest[name] = digest(arrays)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
