"""Pins for the oracle's IEEE-half and Q8_0 codecs (CPU only).

Each check either re-encodes one of the reference's known-answer tests (cited)
or compares against an independent library routine (numpy's IEEE float16 cast,
numpy's float32 multiply + a float64 half-away rounding) over many inputs.
"""
import numpy as np
import pytest


def f(v):
    return np.float32(v)


# ---- f16 codec -------------------------------------------------------------

def test_f16_roundtrip_every_non_nan_pattern(orc):
    # gguf_write/blocks.rs:226-239
    h = np.arange(0x10000, dtype=np.uint16)
    keep = ~(((h >> 10) & 0x1F == 0x1F) & (h & 0x3FF != 0))
    h = h[keep]
    back = orc.f32_to_f16_array(orc.f16_to_f32_array(h))
    assert np.array_equal(back, h)


def test_f16_decode_equals_numpy_for_all_patterns(orc):
    # library pin: numpy's binary16 -> binary32 conversion is exact
    h = np.arange(0x10000, dtype=np.uint16)
    got = orc.f16_to_f32_array(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_equals_numpy_rne_on_random_and_edge_bits(orc):
    # library pin: numpy's float32 -> float16 cast is IEEE round-to-nearest-even
    rng = np.random.default_rng(1234)
    bits = rng.integers(0, 2**32, size=1 << 21, dtype=np.uint64).astype(np.uint32)
    # every f32 exponent that lands in or near the f16 range, with tie/near-tie mantissas
    exps = np.arange(96, 160, dtype=np.uint32)
    mants = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x2000, 0x3000, 0x7FFFFF, 0x7FE000,
                      0x7FF000, 0x400000, 0x401000, 0x400FFF], dtype=np.uint32)
    edge = (exps[:, None] << 23 | mants[None, :]).ravel()
    bits = np.concatenate([bits, edge, edge | 0x80000000])
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    got = orc.f32_to_f16_array(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_spot_values(orc):
    # gguf_write/blocks.rs:242-250, 353-370
    e = orc.f32_to_f16
    assert e(0.0) == 0x0000 and e(-0.0) == 0x8000 and e(1.0) == 0x3C00 and e(-2.0) == 0xC000
    assert e(65504.0) == 0x7BFF and e(1e5) == 0x7C00 and e(float("inf")) == 0x7C00
    assert e(float("nan")) == 0x7E00 and e(-float("nan")) == 0xFE00
    assert e(float("-inf")) == 0xFC00 and e(65520.0) == 0x7C00 and e(1.0e9) == 0x7C00
    assert e(1.5 * 2.0**-24) == 2
    assert e(2.0**-26) == 0 and e(-(2.0**-26)) == 0x8000
    assert e(float(np.uint32(0x3F801001).view(np.float32))) == 0x3C01


def test_f16_decode_special_values(orc):
    # gguf/dequant.rs:528-538
    d = orc.f16_to_f32
    assert d(0x0000) == 0.0 and d(0x8000) == 0.0 and d(0x3C00) == 1.0
    assert d(0x7C00) == float("inf") and d(0xFC00) == float("-inf")
    assert np.isnan(d(0x7E00))
    assert d(0x0001) == 2.0**-24


# ---- Q8_0 block ------------------------------------------------------------

def half_away(v64):
    return np.sign(v64) * np.floor(np.abs(v64) + 0.5)


def closed_form_q8_0(x):
    """numpy restatement used as a library pin: IEEE f32 ops + half-away rounding."""
    x = x.astype(np.float32)
    amax = np.float32(0.0)
    for v in np.abs(x):
        if not np.isnan(v):
            amax = max(amax, v)
    d = np.float32(amax / np.float32(127.0))
    idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
    with np.errstate(invalid="ignore"):
        q = half_away((x * idv).astype(np.float32).astype(np.float64))
    q = np.where(np.isnan(q), 0, np.clip(q, -128, 127)).astype(np.int8)
    return int(np.float16(d).view(np.uint16)), q


def test_q8_0_block_matches_llama_cpp_reference(orc):
    # quant.rs:332-343
    x = ((np.arange(32, dtype=np.float32) - f(15.5)) * f(0.37)).astype(np.float32)
    d16, q = orc.q8_0_block(x)
    amax = np.float32(np.abs(x).max())
    d = np.float32(amax / np.float32(127.0))
    assert d16 == orc.f32_to_f16(float(d))
    assert np.array_equal(q.astype(np.float64), half_away((x * (np.float32(1.0) / d)).astype(np.float64)))
    assert np.array_equal(orc.q8_0_block(np.zeros(32, np.float32))[1], np.zeros(32, np.int8))


def test_q8_0_block_rounds_half_away_and_pins_amax(orc):
    # quant.rs:357-365
    x = np.zeros(32, np.float32)
    x[:8] = [127.0, 0.5, 1.5, -0.5, -2.5, 2.4999, -126.5, 0.49]
    d16, q = orc.q8_0_block(x)
    assert orc.f16_to_f32(d16) == 1.0
    assert list(q[:8]) == [127, 1, 2, -1, -3, 2, -127, 0]
    assert not q[8:].any()


def test_q8_0_block_negative_extreme_and_outlier(orc):
    # quant.rs:368-388
    neg = np.full(32, -0.01, np.float32)
    neg[7] = -3.0
    d16, q = orc.q8_0_block(neg)
    assert q[7] == -127 and (q <= 0).all()
    d = orc.f16_to_f32(d16)
    assert abs(d - 3.0 / 127.0) < 3.0 / 127.0 * 1e-3
    assert q[0] == int(half_away(np.float64(np.float32(-0.01) * (np.float32(1.0) / np.float32(np.float32(3.0) / np.float32(127.0))))))
    pos = np.zeros(32, np.float32)
    pos[31] = 5.0
    _, q = orc.q8_0_block(pos)
    assert q[31] == 127 and not q[:31].any()


def test_q8_0_zero_and_tiny_blocks(orc):
    # quant.rs:391-401
    d16, q = orc.q8_0_block(np.zeros(32, np.float32))
    assert d16 == 0 and not q.any()
    w = orc.fake_quantize_q8_0_rows(np.zeros(64, np.float32), 32)
    assert (w == 0).all()
    tiny = orc.fake_quantize_q8_0_rows(np.full(32, 1e-30, np.float32), 32)
    assert np.isfinite(tiny).all()


def test_q8_0_snap_blocks_are_independent(orc):
    # quant.rs:404-422
    w = np.concatenate([(np.arange(32, dtype=np.float32) - 16) * f(0.001),
                        (np.arange(32, dtype=np.float32) - 16) * f(100.0)]).astype(np.float32)
    snapped = orc.fake_quantize_q8_0_rows(w, 64)
    for b in range(2):
        src = w[b * 32:(b + 1) * 32]
        d16, q = orc.q8_0_block(src)
        d = np.float32(orc.f16_to_f32(d16))
        assert np.array_equal(snapped[b * 32:(b + 1) * 32], (q.astype(np.float32) * d).astype(np.float32))
        amax = np.abs(src).max()
        assert (np.abs(snapped[b * 32:(b + 1) * 32] - src) <= amax / 127.0 * 0.51 + amax * 1e-3).all()


def test_q8_0_cols_run_down_columns(orc):
    # quant.rs:425-443
    rows, cols = 64, 5
    i = np.arange(rows * cols)
    orig = (((i * 29 % 97).astype(np.float32) - 48.0) * (1.0 + (i % cols))).astype(np.float32)
    w = orc.fake_quantize_q8_0_cols(orig, rows, cols).reshape(rows, cols)
    t = orc.fake_quantize_q8_0_rows(orig.reshape(rows, cols).T.copy().ravel(), rows).reshape(cols, rows)
    assert np.array_equal(w, t.T)


def test_q8_0_degenerate_shapes_are_noops(orc):
    # quant.rs:446-456
    orig = np.full(64, 1.5, np.float32)
    assert np.array_equal(orc.fake_quantize_q8_0_rows(orig, 0), orig)
    assert np.array_equal(orc.fake_quantize_q8_0_cols(orig, 0, 4), orig)
    assert np.array_equal(orc.fake_quantize_q8_0_cols(orig, 63, 1), orig)


def test_q8_0_snap_is_a_fixed_point(orc):
    # quant.rs:346-354
    i = np.arange(96 * 40)
    w = (((i * 37 % 101).astype(np.float32) - 50.0) / 61.0).astype(np.float32)
    once = orc.fake_quantize_q8_0_cols(w, 96, 40)
    assert np.array_equal(orc.fake_quantize_q8_0_cols(once, 96, 40), once)


def test_q8_0_block_equals_closed_form_on_random_blocks(orc):
    rng = np.random.default_rng(7)
    blocks = [rng.standard_normal(32).astype(np.float32) * np.float32(s)
              for s in (1e-6, 1e-3, 0.02, 1.0, 300.0, 6e4) for _ in range(200)]
    # exact half-way products: amax = 127 makes id = 1
    for _ in range(100):
        b = (rng.integers(-254, 255, 32) / 2.0).astype(np.float32)
        b[0] = 127.0
        blocks.append(b)
    with_nan = rng.standard_normal(32).astype(np.float32)
    with_nan[3] = np.nan
    blocks.append(with_nan)
    with_inf = rng.standard_normal(32).astype(np.float32)
    with_inf[5] = np.inf
    blocks.append(with_inf)
    for b in blocks:
        d16, q = orc.q8_0_block(b)
        wd, wq = closed_form_q8_0(b)
        assert d16 == wd
        assert np.array_equal(q, wq)


# ---- GGUF Q8_0 layout and decode -----------------------------------------

def test_enc_q8_0_layout_and_reader_decode_equal_snap(orc):
    # gguf_write/blocks.rs:279-310
    i = np.arange(32 * 4)
    x = (((i * 37 % 101).astype(np.float32) - 50.0) / 7.0).astype(np.float32)
    x[32:64] = 0.0
    x[64:96] = -np.abs(x[64:96])
    x[100] = 900.0
    raw = orc.q8_0_encode(x)
    assert raw.size == 4 * 34
    for b in range(4):
        d16, q = orc.q8_0_block(x[b * 32:(b + 1) * 32])
        blk = raw[b * 34:(b + 1) * 34]
        assert int(blk[0]) | int(blk[1]) << 8 == d16
        assert np.array_equal(blk[2:].view(np.int8), q)
    assert list(raw[34:36]) == [0, 0]
    assert np.array_equal(orc.q8_0_dequant(raw, 128), orc.fake_quantize_q8_0_rows(x, 128))


def test_enc_q8_0_rejects_ragged(orc):
    # gguf_write/blocks.rs:313-318
    with pytest.raises(ValueError):
        orc.q8_0_encode(np.zeros(20, np.float32))


def test_dequant_synth_gguf_vectors(orc):
    # gguf/test_support.rs:52-73 (d = 0.5, q = i - 16) and gguf/tensors.rs:127-130
    raw = np.zeros(34, np.uint8)
    d16 = orc.f32_to_f16(0.5)
    raw[0], raw[1] = d16 & 0xFF, d16 >> 8
    raw[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    got = orc.q8_0_dequant(raw, 32)
    assert np.array_equal(got, (0.5 * (np.arange(32) - 16)).astype(np.float32))
    with pytest.raises(ValueError):
        orc.q8_0_dequant(raw[:33], 32)


def test_dequant_equals_numpy_closed_form(orc):
    raw = orc.quantize_weight(37, 96, seed=3)
    got = orc.q8_0_dequant(raw.ravel(), 37 * 96).reshape(37, 96)
    blocks = raw.reshape(37, 3, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float32)  # [37, 3, 1]
    q = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    want = (d * q).reshape(37, 96).astype(np.float32)
    assert np.array_equal(got, want)
    w_kn = orc.q8_0_to_ferrum_weight(raw, 37, 96)
    assert np.array_equal(w_kn, want.T)
