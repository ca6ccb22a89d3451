"""ops::qlinear on the GPU (packed per-row int8 / int4 QWeight): every output
bit-equal to the oracle's restatement of qaccum_cols (bias first, p
ascending, no FMA), across int8 / int4, odd widths (the split-half nibble
layout's last column), several rows of x, K beyond one LDS chunk, the
one-row kernel's chunk and 4-row-group tails (K = 1, 2, 7, 389) and its
16-, 32- and 64-byte column tiles (chosen by the output width; int4 takes
the 64-byte tile, where a lane owns two nibble columns, only above 16,384
outputs, so two such cases end on partial chunks and row groups), and the
reference's dimension errors (ops.rs:316-330)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(fh, t):
    import torch

    fh.sync()
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("m,k,n,bias", [(1, 768, 768, True), (1, 768, 50257, False), (3, 1100, 333, True),
                                        (5, 64, 7, True), (8, 3072, 768, True), (1, 513, 1, True),
                                        (1, 3072, 2304, True), (1, 389, 129, True), (1, 7, 130, False),
                                        (1, 1, 5, True), (1, 2, 64, True), (1, 777, 5000, True),
                                        (1, 1000, 10000, False), (1, 1001, 9000, True),
                                        (1, 1001, 20001, True), (1, 389, 50257, False)])
def test_qlinear_is_bit_exact(fh, orc, kind, m, k, n, bias):
    import torch

    import ferrum_hip

    rng = np.random.default_rng(k * 7 + n + kind)
    wf = (rng.standard_normal((k, n)) * 0.05).astype(np.float32)
    ow = orc.QWeight(wf, k, n, kind)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32) if bias else np.zeros(n, np.float32)
    want = orc.qlinear(x, ow, b, threads=1)
    w = ferrum_hip.QWeight(fh, ow.scales, ow.q, k, n, kind)
    y = torch.full((m, n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.qlinear_async(fh, w, dev(x), m, k, dev(b) if bias else None, n if bias else 0, y)
    got = host(fh, y)
    w.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_qlinear_errors(fh, orc):
    import torch

    import ferrum_hip

    ow = orc.QWeight(np.ones((64, 10), np.float32), 64, 10, 0)
    w = ferrum_hip.QWeight(fh, ow.scales, ow.q, 64, 10, 0)
    x, y = dev(np.ones((1, 64), np.float32)), torch.empty(10, device="cuda")
    with pytest.raises(ferrum_hip.DimMismatch, match="input width 63"):
        ferrum_hip.qlinear_async(fh, w, x, 1, 63, None, 0, y)
    with pytest.raises(ferrum_hip.DimMismatch, match="bias length 9"):
        ferrum_hip.qlinear_async(fh, w, x, 1, 64, dev(np.zeros(9, np.float32)), 9, y)
    with pytest.raises(ferrum_hip.FerrumHipError, match="unknown kind"):
        ferrum_hip.QWeight(fh, ow.scales, ow.q, 64, 10, 2)
    w.free()
