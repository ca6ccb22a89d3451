"""Q8_0 linear, codec and weight upload on the GPU, checked against the CPU
oracle (oracle/ferrum_oracle.c, a restatement of ferrum_core's arithmetic).

Tolerances:
  * Q8_0 block encode, dequant, weight round trip, int32 block dots: bit-exact.
  * f32 outputs within 1e-5 relative, componentwise:
        |gpu - ref| <= 1e-5 * max(|ref|, sum_p |x_p * w_p|)
    i.e. relative to the size of the terms the output sums.  A pointwise
    |gpu - ref| <= 1e-5 |ref| is not attainable by any summation order but the
    reference's own: its sequential f32 sum is itself off the exact result by
    ~sqrt(k) * eps * |partial sums| (1.5e-5 of |y| in the 4-sigma tail of a
    50257-output GEMV at k = 3072), so outputs that cancel to near zero differ
    between any two orders by more than 1e-5 of their size.  A dropped or
    mis-scaled term moves an output by >= 1e-3 of sum |x w| and fails clearly.
  * and the GPU is at least as accurate as the reference: against the exact
    (float64) product of the same Q8_0 weights its mean absolute error is at
    most 1.5x the reference's (plus 2^-23 of the mean |y|, for cases of a few
    outputs where the reference's own error may be zero), and on the large
    cases its largest error at most 2x the reference's largest.  This is the
    sharp check: the term-mass bound grows like k while rounding error grows
    like sqrt(k), so a lost low-order term (an f16 split that keeps one term,
    a dropped block) passes the first bound at k = 4096 but not this one.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def term_mass(orc, x, raw, n, k):
    """sum_p |x_p * w_jp| per output, in float64 (dequantisation is exact)."""
    w = np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
    return np.abs(np.asarray(x, np.float64)) @ w


def assert_close(got, want, mass, rtol=RTOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.maximum(np.abs(want), mass)
    err = np.abs(got - want)
    bad = err > rtol * scale
    assert not bad.any(), (f"{bad.sum()} of {bad.size} outside tolerance; worst componentwise rel "
                           f"{(err / np.maximum(scale, 1e-30)).max():.3e}, worst pointwise rel "
                           f"{(err / np.maximum(np.abs(want), 1e-30)).max():.3e}")


def assert_as_accurate(got, ref, exact, factor=1.5, max_factor=None):
    exact = np.asarray(exact, np.float64)
    d_gpu = np.abs(np.asarray(got, np.float64) - exact)
    d_ref = np.abs(np.asarray(ref, np.float64) - exact)
    floor = 2.0**-23 * np.abs(exact).mean()
    e_gpu, e_ref = d_gpu.mean(), d_ref.mean()
    print(f"accuracy vs float64: gpu mean {e_gpu:.3e} max {d_gpu.max():.3e}; "
          f"reference mean {e_ref:.3e} max {d_ref.max():.3e} ({d_gpu.size} outputs)")
    assert e_gpu <= factor * e_ref + floor, f"gpu mean abs error {e_gpu:.3e} vs reference {e_ref:.3e}"
    if max_factor is not None:
        assert d_gpu.max() <= max_factor * d_ref.max() + floor, \
            f"gpu max abs error {d_gpu.max():.3e} vs reference {d_ref.max():.3e}"


def sample_rows(m, count, seed):
    """A seeded sample of row indices, always with the first and last row and
    both sides of the 256-row tile boundaries it crosses first."""
    rng = np.random.default_rng(seed)
    fixed = [r for r in (0, 1, 255, 256, 257, m - 257, m - 256, m - 2, m - 1) if 0 <= r < m]
    pick = rng.choice(m, size=min(count, m), replace=False)
    return np.unique(np.r_[fixed, pick]).astype(np.int64)


def exact_linear(orc, x, raw, n, k, bias=None):
    """float64 product of the same Q8_0 weights (dequantisation is exact)."""
    w = orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64)
    y = np.asarray(x, np.float64) @ w
    return y if bias is None else y + np.asarray(bias, np.float64)


def weight(orc, n, k, seed, std=0.02):
    return orc.quantize_weight(n, k, seed, std)


def acts(m, k, seed):
    return np.random.default_rng(seed + 7).standard_normal((m, k), dtype=np.float32)


def bias_for(n, seed):
    return (np.random.default_rng(seed + 11).standard_normal(n, dtype=np.float32) * np.float32(0.1))


# ---- upload / download --------------------------------------------------------

@pytest.mark.parametrize("n,k", [(1, 32), (3, 64), (768, 768), (50257, 768)])
def test_weight_round_trip_is_bit_exact(fh, n, k):
    import ferrum_hip

    raw = np.random.default_rng(n + k).integers(0, 256, size=n * (k // 32) * 34, dtype=np.uint8)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    assert w.dims() == (n, k)
    assert np.array_equal(w.download(), raw)
    w.free()


def test_upload_rejects_a_row_length_off_the_block_grid(fh):
    import ferrum_hip

    with pytest.raises(ferrum_hip.FerrumHipError, match="multiple of the Q8_0 block size"):
        ferrum_hip.Q8_0Weight.upload(fh, np.zeros(34, np.uint8), 1, 48)


# ---- W8A32 (ferrum_core semantics) ------------------------------------------------

CONFIG2 = [(n, k) for n in (768, 2304, 3072, 50257) for k in (768, 3072)]


@pytest.mark.parametrize("n,k", CONFIG2)
def test_gemv_m1_config2_matches_oracle(fh, orc, n, k):
    import ferrum_hip

    seed = n * 31 + k
    raw = weight(orc, n, k, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(1, k, seed), bias_for(n, seed)
    got, ref = ferrum_hip.linear_forward(fh, x, w, b), orc.q8_0_linear(x, raw, n, b)
    w.free()
    assert_close(got, ref, term_mass(orc, x, raw, n, k))
    assert_as_accurate(got, ref, exact_linear(orc, x, raw, n, k, b))
    x2 = acts(1, k, seed + 1)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.matmul(fh, x2, w)
    w.free()
    assert_close(got, orc.q8_0_linear(x2, raw, n, None), term_mass(orc, x2, raw, n, k))


@pytest.mark.parametrize("m,n,k", [(2, 768, 768), (2, 3072, 3072), (3, 2304, 768), (8, 3072, 768),
                                   (8, 768, 3072), (32, 2304, 768), (32, 768, 3072), (32, 50257, 768),
                                   (64, 896, 896), (65, 130, 4864)])
def test_batched_linear_matches_oracle(fh, orc, m, n, k):
    import ferrum_hip

    seed = m * 7 + n * 3 + k
    raw = weight(orc, n, k, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, seed), bias_for(n, seed)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    ref = orc.q8_0_linear(x, raw, n, b)
    assert_close(got, ref, term_mass(orc, x, raw, n, k))
    assert_as_accurate(got, ref, exact_linear(orc, x, raw, n, k, b))


@pytest.mark.parametrize("m", [8, 32])
@pytest.mark.parametrize("n,k", CONFIG2)
def test_config2_batched_sweep(fh, orc, m, n, k):
    """BASELINE configs[1] at M = 8 and 32 over every (N, K): the skinny
    matrix-core GEMM's tile and K-split choices at each shape."""
    import ferrum_hip

    seed = 1000 * m + n * 31 + k
    raw = weight(orc, n, k, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, seed), bias_for(n, seed)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    ref = orc.q8_0_linear(x, raw, n, b)
    assert_close(got, ref, term_mass(orc, x, raw, n, k))
    assert_as_accurate(got, ref, exact_linear(orc, x, raw, n, k, b), max_factor=2.0 if got.size >= 20000 else None)


@pytest.mark.parametrize("n,k", [(1152, 896), (896, 896), (9728, 896), (896, 4864), (151936, 896)])
def test_config5_qwen_layers_at_batch_64(fh, orc, n, k):
    """BASELINE configs[4]'s Qwen2-0.5B layer set at the batch-64 decode step:
    stacked q|k|v (896 + 2 x 128 rows), o, stacked gate|up (2 x 4864), down and
    the tied 151936-row head, against the oracle (16 sampled rows for the
    head) and the float64 product."""
    import ferrum_hip

    m, seed = 64, n + 3 * k
    raw = weight(orc, n, k, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = acts(m, k, seed)
    b = bias_for(n, seed) if n == 1152 else None  # Qwen2 has q/k/v biases only
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    rows = np.arange(m) if n < 100000 else sample_rows(m, 12, seed)
    ref = orc.q8_0_linear(x[rows], raw, n, b)
    assert_close(got[rows], ref, term_mass(orc, x[rows], raw, n, k))
    assert_as_accurate(got[rows], ref, exact_linear(orc, x[rows], raw, n, k, b), max_factor=2.0)


@pytest.mark.parametrize("m", [1, 2, 5])
@pytest.mark.parametrize("n,k", [(1, 32), (3, 64), (67, 96), (5, 128), (33, 256), (17, 512), (9, 896),
                                 (11, 1024), (7, 4096), (5, 4864), (3, 8192), (2, 9216)])
def test_ragged_shapes_match_oracle(fh, orc, m, n, k):
    import ferrum_hip

    seed = m + n * 13 + k
    raw = weight(orc, n, k, seed, std=0.5)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, seed), bias_for(n, seed)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    ref = orc.q8_0_linear(x, raw, n, b)
    assert_close(got, ref, term_mass(orc, x, raw, n, k))
    assert_as_accurate(got, ref, exact_linear(orc, x, raw, n, k, b))


# ---- m >= 3: the matrix-core GEMM ---------------------------------------------------
# Tile edges of all three tilings (32 x 32 with the waves splitting K, 64 x 64,
# 128 x 128), K-block counts that do not fill the last K step, and m, n one off
# a tile boundary.

@pytest.mark.parametrize("m,n,k", [(3, 33, 32), (31, 65, 96), (33, 31, 160), (95, 130, 64), (129, 257, 224),
                                   (257, 97, 1024), (64, 1024, 768), (600, 1000, 128)])
def test_gemm_tile_edges_match_oracle(fh, orc, m, n, k):
    import ferrum_hip

    seed = 3 * m + 5 * n + k
    raw = weight(orc, n, k, seed, std=0.3)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, seed), bias_for(n, seed)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    got_nb = ferrum_hip.matmul(fh, x, w)
    w.free()
    mass = term_mass(orc, x, raw, n, k)
    assert_close(got, orc.q8_0_linear(x, raw, n, b), mass)
    assert_close(got_nb, orc.q8_0_linear(x, raw, n, None), mass)
    assert_as_accurate(got, orc.q8_0_linear(x, raw, n, b), exact_linear(orc, x, raw, n, k, b))


def test_gemm_large_tiles_against_exact_product(fh, orc):
    """A shape that takes the 128 x 128 tiling on 256 CUs (>= 512 tiles),
    against the float64 product of the same weights at the same tolerance."""
    import ferrum_hip

    m, n, k = 2048, 4096, 256
    raw = weight(orc, n, k, 41)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, 41), bias_for(n, 41)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    exact = exact_linear(orc, x, raw, n, k, b)
    assert_close(got, exact, term_mass(orc, x, raw, n, k))
    rows = sample_rows(m, 128, 41)
    ref = orc.q8_0_linear(x[rows], raw, n, b)
    assert_close(got[rows], ref, term_mass(orc, x[rows], raw, n, k))
    assert_as_accurate(got[rows], ref, exact[rows], max_factor=2.0)


def test_gemm_rows_of_any_magnitude(fh, orc):
    """Each row carries its own power-of-two scale: rows near the f32 range
    ends, a row with one large outlier, and an all-zero row."""
    import ferrum_hip

    n, k = 70, 256
    raw = weight(orc, n, k, 8)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((8, k)).astype(np.float32)
    x[0] *= np.float32(1e-30)
    x[1] *= np.float32(1e30)
    x[2] *= np.float32(1e-40)           # subnormal activations
    x[3, 17] = np.float32(3e4)          # one outlier next to O(1) values
    x[4] = 0.0
    x[5] *= np.float32(65504.0 * 4)     # beyond the f16 range
    x[6] *= np.float32(1e-6)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, None)
    w.free()
    ref = orc.q8_0_linear(x, raw, n, None)
    mass = term_mass(orc, x, raw, n, k)
    ok = np.ones(8, bool)
    ok[2] = False                       # checked separately below
    assert_close(got[ok], ref[ok], mass[ok])
    # Subnormal inputs: f16 terms lose the bits below 2^-149 * 2^126; the
    # error stays below 1e-5 of the row's own term mass plus one f32 subnormal step.
    assert np.all(np.abs(got[2].astype(np.float64) - ref[2]) <= 1e-5 * mass[2] + 1.5e-45 * k)
    assert np.all(got[4] == 0.0)


@pytest.mark.parametrize("m,n,k", [(3, 32805, 768), (17, 40000, 896), (32, 50257, 1024), (8, 151936, 896), (45, 33000, 768), (64, 50257, 1024)])
def test_wide_outputs_at_small_batch(fh, orc, m, n, k):
    """Outputs of at least 1024 32-column tiles at m <= 64 (vocabulary heads
    in a batched decode step) take the kernel that splits the activations once
    per workgroup, 32 rows per launch: a ragged last tile, more tiles than
    eight per CU (151936), a second launch of 13 or 32 rows, rows of any
    magnitude, inf/NaN activations, non-finite block scales and the bias,
    against the oracle and the float64 product."""
    import ferrum_hip

    seed = m + n + k
    raw = orc.quantize_weight(n, k, seed, 0.02).reshape(n, k // 32, 34).copy()
    bad_cols = [2, 7, n - 1]
    raw[2, 0, :2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)       # +inf scale
    raw[7, -1, :2] = np.frombuffer(np.uint16(0xFC00).tobytes(), np.uint8)      # -inf scale
    raw[n - 1, 1, :2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)   # NaN scale
    raw = raw.ravel()
    x = acts(m, k, seed)
    x[0] *= np.float32(1e-30)
    if m > 3:
        x[1] *= np.float32(1e30)
        x[2, 17] = np.float32(3e4)      # one outlier next to O(1) values
    if m > 5:
        x[3] = 0.0
        x[4, 5] = np.inf
        x[5, 100] = np.nan
    special = [r for r in (0, 1, 2, 3, 4, 5) if r < m and (r == 0 or m > 3) and (r < 3 or m > 5)]
    if m > 40:                          # the same kinds of row in the second launch
        x[33] *= np.float32(1e-30)
        x[34, 17] = np.float32(3e4)
        x[40, 3] = np.nan
        special += [33, 34, 40]
    b = bias_for(n, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    cols = np.unique(np.r_[bad_cols, 0, 1, 31, 32, n - 33, n - 32, n - 2,
                           np.random.default_rng(seed).choice(n, size=min(n, 6000), replace=False)])
    # every output column depends on its own weight row only: check the
    # sampled columns against the oracle on those rows
    sub = raw.reshape(n, -1)[cols].ravel()
    ref = orc.q8_0_linear(x, sub, cols.size, b[cols])
    g = got[:, cols]
    assert np.array_equal(np.isnan(g), np.isnan(ref))
    assert np.array_equal(np.isposinf(g), np.isposinf(ref)) and np.array_equal(np.isneginf(g), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert_close(g[fin], ref[fin], term_mass(orc, x, sub, cols.size, k)[fin])
    clean_rows = np.setdiff1d(np.arange(m), special)
    clean_cols = ~np.isin(cols, bad_cols)
    exact = exact_linear(orc, x[clean_rows], sub, cols.size, k, b[cols])[:, clean_cols]
    assert_as_accurate(g[clean_rows][:, clean_cols], ref[clean_rows][:, clean_cols], exact, max_factor=2.0)


def test_gemm_propagates_inf_and_nan_like_the_reference(fh, orc):
    import ferrum_hip

    n, k = 40, 128
    raw = weight(orc, n, k, 12)
    x = acts(5, k, 12)
    x[0, 3] = np.inf
    x[1, 100] = -np.inf
    x[2, 5] = np.nan
    x[3, 0], x[3, 64] = np.inf, -np.inf
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, bias_for(n, 12))
    w.free()
    ref = orc.q8_0_linear(x, raw, n, bias_for(n, 12))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)) and np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert_close(got[fin], ref[fin], term_mass(orc, x, raw, n, k)[fin])


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 64), (4100, 4095, 96), (4096, 4352, 128), (4000, 4100, 256),
                                   (4352, 4096, 192)])
def test_gemm_weight_split_tiles_match(fh, orc, m, n, k):
    """Shapes with >= 256 tiles of 256 x 256 take the block-scaled kernel
    (quants as the f16 weight operand, the activation as two f16 terms, one
    FMA per output and block for the block scale; 2 to 8 Q8_0 blocks per row,
    ragged m and n); against the float64 product of the same weights
    (finite rows) and against the oracle on rows with special values.  Weight
    rows of very different scale share tiles."""
    import ferrum_hip

    rng = np.random.default_rng(m + n + k)
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
    w[1::7] *= np.float32(1e-5)          # rows whose block scales are tiny
    w[3::11, :32] *= np.float32(1e3)      # rows with one dominant block
    w[5, :] = 0.0                         # an all-zero row (scales 0)
    raw = orc.q8_0_encode(w.ravel())
    x = acts(m, k, m + k)
    special = [0, 1, 2, 3, 4, 5, 6, m - 1]
    x[0, 3] = np.inf
    x[1, 10] = np.nan
    x[2] *= np.float32(1e-30)
    x[3] *= np.float32(1e30)
    x[4, :] = 0.0
    x[6, 1], x[6, k - 1] = np.inf, -np.inf
    b = bias_for(n, k)
    wt = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, wt, b)
    wt.free()
    plain = np.setdiff1d(np.arange(m), special)
    mass = np.abs(x[plain].astype(np.float64)) @ np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
    exact = exact_linear(orc, x[plain], raw, n, k, b)
    assert_close(got[plain], exact, mass)
    sel = np.setdiff1d(sample_rows(m, 96, m + n), special)
    at = np.searchsorted(plain, sel)
    ref = orc.q8_0_linear(x[sel], raw, n, b)
    assert_close(got[sel], ref, mass[at])
    assert_as_accurate(got[sel], ref, exact[at])
    ref = orc.q8_0_linear(x[special], raw, n, b)
    g = got[special]
    assert np.array_equal(np.isnan(g), np.isnan(ref))
    assert np.array_equal(np.isposinf(g), np.isposinf(ref)) and np.array_equal(np.isneginf(g), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert_close(g[fin], ref[fin], term_mass(orc, x[special], raw, n, k)[fin])


@pytest.mark.parametrize("n,k", [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)])
def test_config4_prefill_at_its_own_depth(fh, orc, n, k):
    """GPT-2-medium prefill of 32 prompts x 512 tokens,
    m = 16,384 activation rows through each layer shape (QKV 3072 x 1024, out
    1024 x 1024, up 4096 x 1024, down 1024 x 4096; ops.rs:233-256 reached
    through layer/transformer.rs:352-354 at m = B * ctx).  These run the
    block-scaled 256 x 256 MFMA kernel over 32 and 128 Q8_0 blocks of K, its
    whole double-buffered K loop and epilogue.  N(0, 0.02) weights and N(0, 1)
    activations as the config draws them; a seeded sample of 265 rows against
    the oracle and against the float64 product."""
    import ferrum_hip

    m, seed = 32 * 512, n * 5 + k
    raw = weight(orc, n, k, seed)
    x, b = acts(m, k, seed), bias_for(n, seed)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b)
    w.free()
    rows = sample_rows(m, 256, seed)
    ref = orc.q8_0_linear(x[rows], raw, n, b)
    assert np.isfinite(got).all()
    assert_close(got[rows], ref, term_mass(orc, x[rows], raw, n, k))
    assert_as_accurate(got[rows], ref, exact_linear(orc, x[rows], raw, n, k, b), max_factor=2.0)


@pytest.mark.parametrize("m,n,k", [(1, 96, 64), (5, 96, 64), (100, 300, 96), (4096, 4096, 64)])
def test_non_finite_block_scales_match_the_reference(fh, orc, m, n, k):
    """GGUF block scales of inf or NaN (f16 0x7C00 / 0x7E00), with zero and
    non-zero quants in the block: inf * 0 = NaN and inf * q = +-inf per weight,
    as the reference's f32 expansion has it.  Every path (GEMV, skinny, tiled,
    block-scaled) must reproduce the inf/NaN pattern and the finite values."""
    import ferrum_hip

    raw = orc.quantize_weight(n, k, 77 + m, 0.05).reshape(n, k // 32, 34).copy()
    bad_rows = [2, 7, n - 1]
    raw[2, 0, :2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)       # +inf scale
    raw[7, -1, :2] = np.frombuffer(np.uint16(0xFC00).tobytes(), np.uint8)      # -inf scale
    raw[7, -1, 2:6] = 0                                                       # ... with zero quants
    raw[n - 1, 1, :2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)   # NaN scale
    raw = raw.ravel()
    x = acts(m, k, 5 + m)
    if m > 3:
        x[3, 0] = 0.0                                                         # 0 * inf = NaN
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, None)
    w.free()
    rows = np.unique(np.r_[0:min(m, 8), m - 1])
    ref = orc.q8_0_linear(x[rows], raw, n, None)
    g = got[rows]
    assert np.array_equal(np.isnan(g), np.isnan(ref))
    assert np.array_equal(np.isposinf(g), np.isposinf(ref)) and np.array_equal(np.isneginf(g), np.isneginf(ref))
    assert not np.isfinite(ref[:, bad_rows]).any()
    fin = np.isfinite(ref)
    assert_close(g[fin], ref[fin], term_mass(orc, x[rows], raw, n, k)[fin])


def test_expanded_weight_path_agrees(fh, orc):
    """The GPU result against ops::linear_forward on the f32 expansion the
    reference's loader builds (dequant + transpose), not only the row form."""
    import ferrum_hip

    n, k = 2304, 768
    raw = weight(orc, n, k, 5)
    w_kn = orc.q8_0_to_ferrum_weight(raw, n, k)
    x, b = acts(3, k, 5), bias_for(n, 5)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    assert_close(ferrum_hip.linear_forward(fh, x, w, b), orc.linear_forward(x, w_kn, b, threads=4),
                 np.abs(x.astype(np.float64)) @ np.abs(w_kn.astype(np.float64)))
    w.free()


def test_empty_batch_and_dim_errors(fh, orc):
    import ferrum_hip

    raw = weight(orc, 8, 64, 1)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, 8, 64)
    assert ferrum_hip.linear_forward(fh, np.zeros((0, 64), np.float32), w).shape == (0, 8)
    with pytest.raises(ferrum_hip.DimMismatch, match="input width 32"):
        ferrum_hip.linear_forward(fh, np.zeros((1, 32), np.float32), w)
    with pytest.raises(ferrum_hip.DimMismatch, match="bias length 7"):
        ferrum_hip.linear_forward(fh, np.zeros((1, 64), np.float32), w, np.zeros(7, np.float32))
    with pytest.raises(ferrum_hip.FerrumHipError, match="unknown numerics"):
        ferrum_hip.linear_forward(fh, np.zeros((1, 64), np.float32), w, None, numerics=9)
    w.free()


def test_async_path_on_torch_buffers(fh, orc):
    import torch

    import ferrum_hip

    n, k, m = 3072, 768, 1
    raw = weight(orc, n, k, 9)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, 9), bias_for(n, 9)
    dx, db = torch.from_numpy(x).cuda(), torch.from_numpy(b).cuda()
    dy = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    fh.set_stream(torch.cuda.current_stream().cuda_stream)
    try:
        ferrum_hip.linear_forward_async(fh, w, dx, m, k, db, n, dy)
        torch.cuda.synchronize()
    finally:
        fh.set_stream(None)
    assert_close(dy.cpu().numpy(), orc.q8_0_linear(x, raw, n, b), term_mass(orc, x, raw, n, k))
    w.free()


# ---- W8A8 (llama.cpp semantics) and the codec -------------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 768, 768), (1, 3072, 3072), (4, 2304, 768), (32, 768, 3072),
                                   (3, 7, 32), (2, 5, 4864)])
def test_w8a8_matches_oracle(fh, orc, m, n, k):
    import ferrum_hip

    raw = weight(orc, n, k, m + n + k)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x, b = acts(m, k, n), bias_for(n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b, numerics=ferrum_hip.W8A8)
    assert_close(got, orc.q8_0_linear_w8a8(x, raw, n, b), term_mass(orc, x, raw, n, k))
    w.free()


@pytest.mark.parametrize("m,n,k,has_bias", [(32, 6144, 32, True), (40, 6200, 96, False), (64, 6144, 64, True),
                                            (100, 3100, 768, True), (257, 2304, 768, False), (1000, 1024, 1024, True),
                                            (1030, 700, 96, True), (2048, 512, 1024, False), (1024, 384, 32, True)])
def test_w8a8_matrix_cores_are_bit_exact(fh, orc, m, n, k, has_bias):
    """With >= 96 output tiles of (32 or 64) x 64, W8A8 runs on the int8
    matrix cores (one v_mfma_i32_32x32x32_i8 per Q8_0 block of a 32 x 32
    tile) and adds the scaled block dots in the reference's order without FMA:
    equal to the reference bit for bit, non-finite rows, ragged shapes and
    odd block counts included.  From m = 1024 the operands go through LDS
    (256 x 256 workgroup tiles) as f16, the block dot is two f16 MFMAs (an
    exact integer in f32) and d_w * d_x one f32 outer-product MFMA: rows and
    columns past a tile edge, one block and an odd number of blocks."""
    import ferrum_hip

    raw = weight(orc, n, k, 7 * m + n + k)
    x = acts(m, k, m + 3)
    x[1, 5] = np.inf                 # amax inf: d = inf, quants 0 -> 0 * inf = NaN
    x[2, :] = 0.0                    # d = 0
    x[3] *= np.float32(1e-30)        # subnormal-range scales
    x[4] *= np.float32(1e20)
    x[m - 1, k - 1] = np.nan
    b = bias_for(n, k) if has_bias else None
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b, numerics=ferrum_hip.W8A8)
    w.free()
    ref = orc.q8_0_linear_w8a8(x, raw, n, b)
    assert np.array_equal(got, ref, equal_nan=True)
    assert np.isnan(got[1]).all() and np.isfinite(got[5:m - 1]).all()


@pytest.mark.parametrize("m,n,k", [(64, 6144, 64), (1030, 700, 96)])
def test_w8a8_takes_rows_at_a_4_byte_offset(fh, orc, m, n, k):
    """x need only be 4-byte aligned: from a torch view one float into its
    buffer the panel encoder reads it with 4-byte loads, and the outputs still
    equal the reference bit for bit (the matrix-core path and the staged one)."""
    import torch

    import ferrum_hip

    raw = weight(orc, n, k, m + n)
    x = acts(m, k, m + n)
    x[2, 7] = np.nan
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    buf = torch.zeros(m * k + 1, device="cuda")
    dx = buf[1:]
    dx.copy_(torch.from_numpy(x.ravel()))
    assert dx.data_ptr() % 16 == 4
    dy = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.linear_forward_async(fh, w, dx, m, k, None, 0, dy, numerics=ferrum_hip.W8A8)
    fh.sync()
    w.free()
    assert np.array_equal(dy.cpu().numpy(), orc.q8_0_linear_w8a8(x, raw, n, None), equal_nan=True)


@pytest.mark.parametrize("m,n,k,has_bias", [(64, 6144, 64, True), (257, 2304, 768, False), (1030, 700, 96, True),
                                            (2048, 512, 1024, False), (40, 300, 96, True)])
def test_w8a8_fast_is_within_the_rule_of_w8a8(fh, orc, m, n, k, has_bias):
    """FH_W8A8_FAST: FH_W8A8's quantisation and exact block dots with each
    block's term fused into the sum (one FMA): within 1e-5 of the reference's
    W8A8 outputs relative to the magnitudes of the block terms summed, the same
    inf/NaN pattern, and at least as accurate as W8A8 against the float64 sum
    of the same terms.  The matrix-core kernel (from 96 output tiles), the
    staged one (m >= 1024) and the block-parallel kernel (below 96 tiles)."""
    import ferrum_hip

    raw = weight(orc, n, k, 5 * m + n + k)
    x = acts(m, k, m + 5)
    x[1, 5] = np.inf
    x[2, :] = 0.0
    x[m - 1, k - 1] = np.nan
    b = bias_for(n, k) if has_bias else None
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b, numerics=ferrum_hip.W8A8_FAST)
    w.free()
    ref = orc.q8_0_linear_w8a8(x, raw, n, b)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)) and np.array_equal(np.isneginf(got), np.isneginf(ref))
    d16, q = orc.q8_0_quantize_rows(x)
    xq = (q.astype(np.float64).reshape(m, k // 32, 32)
          * d16.view(np.float16).astype(np.float64)[:, :, None]).reshape(m, k)
    wf = orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64)
    fin = np.isfinite(ref).all(axis=1)
    mass = np.abs(xq[fin]) @ np.abs(wf)
    assert_close(got[fin], ref[fin], mass)
    exact = xq[fin] @ wf + (0.0 if b is None else b.astype(np.float64))
    assert_as_accurate(got[fin], ref[fin], exact)


def test_int32_block_dots_are_bit_exact(fh, orc):
    import torch

    import ferrum_hip

    m, n, k = 3, 257, 768
    raw = weight(orc, n, k, 3)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    x = acts(m, k, 3) * np.float32(5.0)
    _, qx = orc.q8_0_quantize_rows(x)
    dq = torch.from_numpy(qx).cuda()
    dots = torch.empty((m, n, k // 32), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.q8_0_block_dots_async(fh, w, dq, m, dots)
    fh.sync()
    assert np.array_equal(dots.cpu().numpy(), orc.q8_0_block_dots(qx, raw, n))
    w.free()


def encode_cases():
    rng = np.random.default_rng(77)
    blocks = [
        np.array([127, 0.5, 1.5, -0.5, -2.5, 2.4999, -126.5, 0.49] + [0] * 24, np.float32),  # quant.rs:357-365
        np.zeros(32, np.float32),
        np.full(32, 1e-30, np.float32),
        np.full(32, -1e-38, np.float32),
        np.full(32, 1e-41, np.float32),
        (rng.standard_normal(32) * 1e-37).astype(np.float32),
        np.full(32, 8.3e6, np.float32),
        np.array([65504.0 * 127] + [1.0] * 31, np.float32),
        np.array([np.nan] + [1.0] * 31, np.float32),
        np.array([np.inf] + [1.0] * 31, np.float32),
        np.array([-np.inf, np.nan] + [0.25] * 30, np.float32),
        np.arange(32, dtype=np.float32) - 16,
    ]
    blocks.append((rng.standard_normal(32 * 4096) * rng.choice([1e-3, 1, 1e3], 32 * 4096)).astype(np.float32))
    # ties of x * (1/d) at .5 for many scales
    ties = (np.arange(-63, 64, dtype=np.float32)[:, None] + 0.5) * np.float32(1 / 127)
    blocks.append(np.concatenate([np.concatenate([[1.0], t.repeat(31)]) for t in ties.ravel()]).astype(np.float32))
    return np.concatenate(blocks).astype(np.float32)


def test_q8_0_encode_is_bit_exact(fh, orc):
    import ferrum_hip

    x = encode_cases()
    assert np.array_equal(ferrum_hip.q8_0_encode(fh, x), orc.q8_0_encode(x))


def test_q8_0_encode_length_error(fh):
    import ferrum_hip

    with pytest.raises(ferrum_hip.FerrumHipError, match="not a multiple of block size 32"):
        ferrum_hip.q8_0_encode(fh, np.zeros(33, np.float32))


def test_q8_0_dequant_is_bit_exact(fh, orc):
    import torch

    import ferrum_hip

    raw = np.random.default_rng(4).integers(0, 256, size=34 * 5000, dtype=np.uint8)
    # finite scales only: NaN payloads are compared separately
    raw16 = raw.view(np.uint16).reshape(-1, 17)
    raw16[:, 0] &= 0x7BFF
    dr = torch.from_numpy(raw).cuda()
    out = torch.empty(32 * 5000, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.q8_0_dequant_async(fh, dr, 32 * 5000, out)
    fh.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.q8_0_dequant(raw, 32 * 5000).view(np.uint32))
