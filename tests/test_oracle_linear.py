"""Pins for the oracle's linear layer, W8A8 mode, softmax/ln bridge and RNG (CPU).

The W8A32 linear is pinned bit-for-bit by numpy: float32 products (IEEE
multiply) followed by ``np.cumsum`` in float32, which is a strictly sequential
accumulation, then the bias.  That fixes the ascending-K order, the absence of
FMA and the bias-last epilogue (ops.rs:19-28, 132-148, 233-256).
"""
import ctypes
import ctypes.util

import numpy as np
import pytest


def seq_linear(x, w_kn, bias=None):
    """numpy library pin: sequential float32 sum of float32 products."""
    prods = (x[:, :, None] * w_kn[None, :, :]).astype(np.float32)  # [m, k, n]
    y = np.cumsum(prods, axis=1, dtype=np.float32)[:, -1, :] if x.shape[1] else np.zeros((x.shape[0], w_kn.shape[1]), np.float32)
    if bias is not None:
        y = (y + bias[None, :]).astype(np.float32)
    return y


def det_data(n, seed):
    """ops.rs:803-813"""
    x = (seed | 1) & 0xFFFFFFFFFFFFFFFF
    out = np.empty(n, np.float32)
    M = 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        x ^= (x << 13) & M
        x ^= x >> 7
        x ^= (x << 17) & M
        out[i] = np.float32((x >> 40) / float(1 << 23) - 1.0)
    return out


def test_matmul_known_answers(orc):
    # ops.rs:582-597
    assert orc.linear_forward(np.array([[1, 2, 3]], np.float32), np.array([[1], [0], [-1]], np.float32))[0, 0] == -2.0
    y = orc.linear_forward(np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32))
    assert y.ravel().tolist() == [19.0, 22.0, 43.0, 50.0]
    with pytest.raises(ValueError):
        orc.linear_forward(np.zeros((2, 3), np.float32), np.zeros((2, 2), np.float32))
    with pytest.raises(ValueError):
        orc.linear_forward(np.zeros((2, 2), np.float32), np.zeros((2, 2), np.float32), np.zeros(3, np.float32))


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (1, 7, 5), (2, 3, 9), (3, 5, 7), (5, 1, 13), (7, 33, 3),
                                   (17, 33, 9), (31, 64, 47), (130, 67, 45), (257, 9, 130),
                                   (6, 300, 270), (3, 513, 11)])
def test_linear_equals_sequential_numpy_at_every_thread_count(orc, m, k, n):
    # ops.rs:730-799 shapes; panels KC=NC=256 crossed by the last two
    rng = np.random.default_rng(m * 1000 + k * 10 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((k, n)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    for bias in (None, b):
        want = seq_linear(x, w, bias)
        for threads in (1, 2, 3, 8):
            got = orc.linear_forward(x, w, bias, threads=threads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, threads)


def test_linear_det_data_reference_shape(orc):
    # ops.rs:816-834: fused bias equals add_bias(matmul) bit for bit
    m, k, n = 40, 70, 130
    x = det_data(m * k, 1).reshape(m, k)
    w = det_data(k * n, 2).reshape(k, n)
    b = det_data(n, 3)
    fused = orc.linear_forward(x, w, b, threads=4)
    unfused = (orc.linear_forward(x, w, None) + b[None, :]).astype(np.float32)
    assert np.array_equal(fused, unfused)
    assert np.array_equal(fused, seq_linear(x, w, b))


def test_fma_would_be_caught(orc):
    """A fused multiply-add changes the bits: the pin above is sensitive to it."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 768)).astype(np.float32)
    w = rng.standard_normal((768, 64)).astype(np.float32)
    seq = seq_linear(x, w)
    fma = np.zeros(64, np.float64)
    acc = np.zeros(64, np.float32)
    for p in range(768):  # round(acc + x*w) with the product unrounded
        acc = (acc.astype(np.float64) + x[0, p].astype(np.float64) * w[p].astype(np.float64)).astype(np.float32)
    assert not np.array_equal(acc, seq[0])
    assert np.array_equal(orc.linear_forward(x, w), seq)


@pytest.mark.parametrize("n,k,m", [(96, 64, 1), (33, 96, 3), (768, 768, 1), (64, 3072, 2)])
def test_q8_0_linear_rows_equals_expanded_linear(orc, n, k, m):
    # loader/decode.rs:97-100 expands Q8_0 to f32 then runs linear_forward;
    # the direct-from-rows form must be bit-identical.
    raw = orc.quantize_weight(n, k, seed=n + k)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    w_kn = orc.q8_0_to_ferrum_weight(raw, n, k)
    want = orc.linear_forward(x, w_kn, b)
    assert np.array_equal(orc.q8_0_linear(x, raw, n, b), want)
    assert np.array_equal(want, seq_linear(x, w_kn, b))
    # and close to the float64 product
    ref64 = x.astype(np.float64) @ w_kn.astype(np.float64) + b
    assert np.abs(want - ref64).max() <= 1e-5 * max(1.0, np.abs(ref64).max())


# ---- W8A8 ------------------------------------------------------------------

def test_w8a8_block_dots_equal_integer_matmul(orc):
    n, k, m = 40, 128, 3
    raw = orc.quantize_weight(n, k, seed=11)
    x = np.random.default_rng(2).standard_normal((m, k)).astype(np.float32)
    dx, qx = orc.q8_0_quantize_rows(x)
    dots = orc.q8_0_block_dots(qx, raw, n)
    qw = raw.reshape(n, k // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    qxx = qx.reshape(m, k // 32, 32).astype(np.int64)
    want = np.einsum("mbt,nbt->mnb", qxx, qw)
    assert np.array_equal(dots.astype(np.int64), want)
    # activation blocks are the q8_0_block encode
    for i in range(m):
        for b in range(k // 32):
            d16, q = orc.q8_0_block(x[i, b * 32:(b + 1) * 32])
            assert d16 == dx[i, b] and np.array_equal(q, qx[i, b * 32:(b + 1) * 32])


def test_w8a8_epilogue_sequential_over_blocks(orc):
    n, k, m = 17, 256, 2
    raw = orc.quantize_weight(n, k, seed=12)
    x = np.random.default_rng(3).standard_normal((m, k)).astype(np.float32)
    b = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    dx, qx = orc.q8_0_quantize_rows(x)
    dots = orc.q8_0_block_dots(qx, raw, n).astype(np.float32)  # [m, n, kb]
    dw = raw.reshape(n, k // 32, 34)[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    dxf = dx.view(np.float16).astype(np.float32)
    scale = (dw[None, :, :] * dxf[:, None, :]).astype(np.float32)
    terms = (dots * scale).astype(np.float32)
    want = (np.cumsum(terms, axis=2, dtype=np.float32)[:, :, -1] + b).astype(np.float32)
    got = orc.q8_0_linear_w8a8(x, raw, n, b)
    assert np.array_equal(got, want)


# ---- softmax + ln bridge (libm) -------------------------------------------

@pytest.fixture(scope="module")
def libm():
    m = ctypes.CDLL(ctypes.util.find_library("m"))
    m.expf.argtypes = [ctypes.c_float]
    m.expf.restype = ctypes.c_float
    m.logf.argtypes = [ctypes.c_float]
    m.logf.restype = ctypes.c_float
    return m


def test_softmax_rows_is_libm_exp_with_sequential_sum(orc, libm):
    # ops.rs:478-502; the platform expf is the library routine the reference calls
    z = np.random.default_rng(9).standard_normal((2, 300)).astype(np.float32) * 4
    got = orc.softmax_rows(z)
    for r in range(2):
        mx = z[r].max()
        e = np.array([libm.expf(float(np.float32(v - mx))) for v in z[r]], np.float32)
        s = np.cumsum(e, dtype=np.float32)[-1]
        assert np.array_equal(got[r], (e / s).astype(np.float32))
    assert np.allclose(got.sum(1), 1.0, atol=1e-5)


def test_ln_bridge_is_libm_log_of_clamped(orc, libm):
    # slm/token_stream.rs:134
    p = np.array([0.0, 1e-13, 1e-12, 0.5, 1.0, 3e-5], np.float32)
    got = orc.ln_bridge(p)
    want = np.array([libm.logf(float(max(v, np.float32(1e-12)))) for v in p], np.float32)
    assert np.array_equal(got, want)
    assert got[0] == got[1] == got[2]


# ---- RNG ---------------------------------------------------------------------

def xorshift_star(state, n):
    M = (1 << 64) - 1
    out = []
    for _ in range(n):
        x = state
        x ^= (x << 13) & M
        x ^= x >> 7
        x ^= (x << 17) & M
        state = x
        out.append((x * 0x2545F4914F6CDD1D) & M)
    return out


def test_rng_closed_form_and_properties(orc):
    # rng.rs:10-41 (closed-form integer arithmetic in Python big ints) and 67-98
    for seed in (1, 7, 42, 2**63 + 5):
        r = orc.Rng(seed)
        assert [r.next_u64() for _ in range(64)] == xorshift_star(seed, 64)
    r0 = orc.Rng(0)
    assert [r0.next_u64() for _ in range(4)] == xorshift_star(0x9E3779B97F4A7C15, 4)
    r = orc.Rng(7)
    xs = [r.next_f32() for _ in range(10000)]
    assert all(0.0 <= x < 1.0 for x in xs)
    assert all(x * (1 << 24) == int(x * (1 << 24)) for x in xs)
    d = xorshift_star(42, 3)
    assert [orc.draw_to_f32(v) for v in d] == [(v >> 40) / float(1 << 24) for v in d]
