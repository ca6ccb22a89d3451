"""Pins for the oracle's packed per-row int8/int4 path (QWeight and
ops::qlinear, quant.rs:130-263, ops.rs:268-377), CPU only: the reference's own
tests re-run on the restatement, plus closed forms that a dropped scale, a
swapped nibble lane or a bias added last would fail."""
import numpy as np
import pytest

from test_oracle_linear import det_data


def sinf_data(n, step, amp):
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(step)) * np.float32(amp)).astype(np.float32)


def test_qweight_int8_round_trip_within_half_a_step(orc):
    # quant.rs:598-614
    rows, cols = 5, 40
    data = sinf_data(rows * cols, 0.017, 1.3).reshape(rows, cols)
    qw = orc.QWeight(data, rows, cols, orc.INT8)
    assert qw.q.size + qw.scales.size * 4 == rows * cols + rows * 4
    back = qw.to_f32()
    for r in range(rows):
        scale = np.float32(np.abs(data[r]).max()) / np.float32(127.0)
        assert np.all(np.abs(data[r] - back[r]) <= scale * 0.5 + 1e-6)


def test_qweight_int4_round_trip_within_half_a_step(orc):
    # quant.rs:617-637 (odd cols: per-row nibble padding)
    rows, cols = 4, 31
    data = np.cos(np.arange(rows * cols, dtype=np.float32) * np.float32(0.07)).astype(np.float32).reshape(rows, cols)
    qw = orc.QWeight(data, rows, cols, orc.INT4)
    assert qw.q.size == rows * 16
    back = qw.to_f32()
    for r in range(rows):
        step = np.float32(np.abs(data[r]).max()) / np.float32(7.0)
        assert np.all(np.abs(data[r] - back[r]) <= step * 0.5 + 1e-6)


def test_qweight_sizes_and_row_bytes(orc):
    # quant.rs:640-648 and 681-686
    assert orc.QWeight(np.full(64 * 64, 0.5, np.float32), 64, 64, orc.INT4).q.size == 64 * 64 // 2
    w = np.full(3 * 5, 0.5, np.float32)
    assert orc.QWeight(w, 3, 5, orc.INT8).row_bytes() == 5
    assert orc.QWeight(w, 3, 5, orc.INT4).row_bytes() == 3


def test_nibble_sign_extension_and_split_half_layout(orc):
    # quant.rs:651-656: 0x0 -> 0, 0x7 -> 7, 0xF -> -1, 0x9 -> -7; low nibbles hold
    # columns [0, half), high nibbles [half, cols)
    q = np.array([0x70, 0xF9, 0x00], np.uint8)  # cols 5, half 3: c0=0, c1=9, c2=0 | c3=7, c4=F
    out = np.zeros((1, 5), np.float32)
    orc.lib().fo_qweight_to_f32(np.ones(1, np.float32), q, 1, 5, orc.INT4, out)
    assert out.tolist() == [[0.0, -7.0, 0.0, 7.0, -1.0]]


def test_qweight_levels_are_round_half_away_and_saturate(orc):
    row = np.array([127.0, 63.5, -63.5, 0.49, -0.5, np.nan, 1e-30, -127.0], np.float32)
    qw = orc.QWeight(row, 1, row.size, orc.INT8)
    assert qw.scales[0] == np.float32(1.0)
    assert qw.q.view(np.int8).tolist() == [127, 64, -64, 0, -1, 0, 0, -127]


def levels_of(qw):
    """The stored integer levels, decoded from the packed bytes."""
    rb = qw.row_bytes()
    q = qw.q.reshape(qw.rows, rb)
    if qw.kind == 0:
        return q.view(np.int8).astype(np.float32)
    half = (qw.cols + 1) // 2
    nib = np.concatenate([q & 0x0F, q >> 4], axis=1)[:, :qw.cols].astype(np.int8)
    cols = np.r_[np.arange(half), half + np.arange(qw.cols - half)]
    return np.where(nib[:, cols] > 7, nib[:, cols] - 16, nib[:, cols]).astype(np.float32)


def sequential_qlinear(x, qw, bias):
    """bias + sum_p (x[p] * scale[p]) * level(p, :), in float32, p ascending."""
    levels = levels_of(qw)
    y = np.tile(np.asarray(bias, np.float32), (x.shape[0], 1))
    a = (x * qw.scales[None, :]).astype(np.float32)
    for p in range(x.shape[1]):
        y = (y + (a[:, p:p + 1] * levels[p][None, :]).astype(np.float32)).astype(np.float32)
    return y


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("m,k,n,threads", [(1, 64, 2048, 8), (1, 8, 8, 4), (4, 64, 300, 3), (3, 33, 17, 1)])
def test_qlinear_equals_the_sequential_form_at_any_thread_count(orc, kind, m, k, n, threads):
    w = det_data(k * n, 5 + m + kind).reshape(k, n)
    qw = orc.QWeight(w, k, n, kind)
    x, b = det_data(m * k, 6).reshape(m, k), det_data(n, 7)
    want = sequential_qlinear(x, qw, b)
    for t in (1, threads):
        assert np.array_equal(orc.qlinear(x, qw, b, threads=t), want)


def test_qlinear_int8_close_to_f32_linear(orc):
    # ops.rs:837-852
    k, n = 96, 200
    w = det_data(k * n, 7).reshape(k, n)
    b, x = det_data(n, 8), det_data(k, 9).reshape(1, k)
    ref = orc.linear_forward(x, w, b)
    got = orc.qlinear(x, orc.QWeight(w, k, n, orc.INT8), b)
    assert got.shape == (1, n) and np.all(np.abs(ref - got) < 0.05)


def test_qlinear_int4_tracks_f32_linear(orc):
    # ops.rs:855-875
    k, n = 96, 200
    w = det_data(k * n, 11).reshape(k, n)
    b, x = det_data(n, 12), det_data(k, 13).reshape(1, k)
    ref = orc.linear_forward(x, w, b)
    got = orc.qlinear(x, orc.QWeight(w, k, n, orc.INT4), b)
    assert np.abs(ref - got).mean() < 0.5


def test_qlinear_decode_gemv_equals_serial_dequant_reference(orc):
    # ops.rs:878-900 (m = 1 crosses the column-split threshold)
    k, n = 64, 2048
    qw = orc.QWeight(det_data(k * n, 21).reshape(k, n), k, n, orc.INT8)
    b, x = det_data(n, 22), det_data(k, 23).reshape(1, k)
    got = orc.qlinear(x, qw, b, threads=8)
    wf = qw.to_f32()
    want = b.copy()
    for p in range(k):
        want = (want + x[0, p] * wf[p]).astype(np.float32)
    assert np.all(np.abs(want - got[0]) < 1e-3)


def test_qlinear_prefill_matches_f32_int8_and_int4(orc):
    # ops.rs:904-929
    m, k, n = 4, 64, 300
    w = det_data(k * n, 31).reshape(k, n)
    b, x = det_data(n, 32), det_data(m * k, 33).reshape(m, k)
    ref = orc.linear_forward(x, w, b)
    assert np.all(np.abs(ref - orc.qlinear(x, orc.QWeight(w, k, n, orc.INT8), b, threads=4)) < 0.06)
    assert np.abs(ref - orc.qlinear(x, orc.QWeight(w, k, n, orc.INT4), b, threads=4)).mean() < 0.6


def test_qlinear_rejects_bad_shapes(orc):
    # ops.rs:952-960
    qw = orc.QWeight(det_data(3 * 4, 1).reshape(3, 4), 3, 4, orc.INT8)
    with pytest.raises(ValueError, match="input width 5"):
        orc.qlinear(np.zeros((1, 5), np.float32), qw, np.zeros(4, np.float32))
    with pytest.raises(ValueError, match="bias length 2"):
        orc.qlinear(np.zeros((1, 3), np.float32), qw, np.zeros(2, np.float32))


def test_a_bias_added_last_would_be_caught(orc):
    """The bias enters first: with a large bias and small products the two
    orders round differently, and the oracle must match bias-first."""
    k, n = 16, 64
    qw = orc.QWeight(det_data(k * n, 3).reshape(k, n) * np.float32(1e-3), k, n, orc.INT8)
    x = det_data(k, 4).reshape(1, k)
    b = np.full(n, 1000.0, np.float32)
    got = orc.qlinear(x, qw, b)
    last = (sequential_qlinear(x, qw, np.zeros(n, np.float32)) + b).astype(np.float32)
    assert np.array_equal(got, sequential_qlinear(x, qw, b)) and not np.array_equal(got, last)
