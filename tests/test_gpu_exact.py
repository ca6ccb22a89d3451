"""FH_W8A32_EXACT: the Q8_0 linear bit for bit as ferrum_core computes it.

The reference expands Q8_0 weights to f32 at load and runs ops::linear_forward
(ops.rs:233-256): every output is the products x[p] * w[p][j] added to 0.0 in
ascending p, each product and add rounded, then + bias.  The oracle restates
that (fo_linear_forward over fo_q8_0_to_ferrum_weight; the oracle's own tests
pin it against a numpy sequential sum), and the exact mode must match it in
every bit, including -0.0, infinities and NaN propagation.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits_equal(got, want):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    assert got.shape == want.shape
    same = got.view(np.uint32) == want.view(np.uint32)
    both_nan = np.isnan(got) & np.isnan(want)
    bad = ~(same | both_nan)
    assert not bad.any(), (f"{bad.sum()} of {bad.size} outputs differ in their bits; first at "
                           f"{np.argwhere(bad)[0].tolist()}: {got[bad][0]!r} vs {want[bad][0]!r}")


def reference(orc, x, raw, n, k, bias):
    return orc.linear_forward(x, orc.q8_0_to_ferrum_weight(raw, n, k), bias)


@pytest.mark.parametrize("m,n,k,with_bias", [
    (1, 768, 768, True), (1, 2304, 768, True), (1, 3072, 768, True), (1, 768, 3072, True),
    (1, 50257, 768, False), (1, 130, 4864, True), (1, 1, 32, True), (1, 65, 224, False),
    (2, 768, 768, True), (3, 100, 416, True), (8, 3072, 768, True), (32, 768, 3072, False),
    (64, 896, 896, True), (2, 20000, 224, True), (1, 16384, 4864, False)])
def test_exact_matches_the_reference_bit_for_bit(fh, orc, m, n, k, with_bias):
    import ferrum_hip

    seed = m * 1009 + n * 31 + k
    raw = orc.quantize_weight(n, k, seed, 0.02)
    x = np.random.default_rng(seed).standard_normal((m, k), dtype=np.float32)
    b = (np.random.default_rng(seed + 1).standard_normal(n, dtype=np.float32) * np.float32(0.1)
         if with_bias else None)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, b, numerics=ferrum_hip.W8A32_EXACT)
    w.free()
    want = reference(orc, x, raw, n, k, b)
    bits_equal(got, want)
    # the restatement straight from GGUF rows agrees too (the same sums)
    bits_equal(got, orc.q8_0_linear(x, raw, n, b))


def test_exact_keeps_signed_zeros_and_specials(fh, orc):
    """0 + (-0) is +0 in the reference's sum; inf and NaN propagate as f32
    arithmetic says (inf - inf is NaN)."""
    import ferrum_hip

    n, k = 70, 96
    raw = orc.quantize_weight(n, k, 5, 0.05)
    x = np.zeros((4, k), np.float32)
    x[0] = -0.0                      # products of -0 and +-w: signed zeros
    x[1, 5] = np.inf                 # one infinite activation
    x[2, 3] = np.nan
    x[3, ::2] = np.float32(3.0e38)   # sums that overflow to +-inf
    x[3, 1::2] = np.float32(-3.0e38)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    got = ferrum_hip.linear_forward(fh, x, w, None, numerics=ferrum_hip.W8A32_EXACT)
    w.free()
    want = reference(orc, x, raw, n, k, None)
    assert np.signbit(want[0]).sum() == 0, "the reference's sums start at +0"
    bits_equal(got, want)


def test_exact_device_form_and_blocking_form_agree(fh, orc):
    import torch

    import ferrum_hip

    m, n, k = 5, 2304, 768
    raw = orc.quantize_weight(n, k, 77, 0.02)
    x = np.random.default_rng(3).standard_normal((m, k), dtype=np.float32)
    b = np.random.default_rng(4).standard_normal(n, dtype=np.float32)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    host = ferrum_hip.linear_forward(fh, x, w, b, numerics=ferrum_hip.W8A32_EXACT)
    dx, db = torch.from_numpy(x).cuda(), torch.from_numpy(b).cuda()
    dy = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.linear_forward_async(fh, w, dx, m, k, db, n, dy, numerics=ferrum_hip.W8A32_EXACT)
    fh.sync()
    w.free()
    bits_equal(dy.cpu().numpy(), host)
    bits_equal(host, reference(orc, x, raw, n, k, b))


def test_exact_and_fast_modes_agree_to_the_rounding_rule(fh, orc):
    """The fast W8A32 mode stays within 1e-5 of the term mass of the exact one."""
    import ferrum_hip

    n, k = 3072, 3072
    raw = orc.quantize_weight(n, k, 9, 0.02)
    x = np.random.default_rng(9).standard_normal((1, k), dtype=np.float32)
    w = ferrum_hip.Q8_0Weight.upload(fh, raw, n, k)
    exact = ferrum_hip.linear_forward(fh, x, w, None, numerics=ferrum_hip.W8A32_EXACT)
    fast = ferrum_hip.linear_forward(fh, x, w, None, numerics=ferrum_hip.W8A32)
    w.free()
    mass = np.abs(x.astype(np.float64)) @ np.abs(orc.q8_0_to_ferrum_weight(raw, n, k).astype(np.float64))
    assert (np.abs(fast.astype(np.float64) - exact) <= 1e-5 * np.maximum(np.abs(exact), mass)).all()
