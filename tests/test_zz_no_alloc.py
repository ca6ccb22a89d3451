"""fh_q8_0_linear_noalloc_async (the Q8_0 linear for callers that cannot
allocate) against fh_q8_0_linear_async, through the C ABI: the same kernels run,
so the outputs must be bit-identical, on two calls in a row with the second on a
smaller input (the shared scratch keeps the first call's contents), for the
GEMV (m <= 2), the skinny GEMM without a K split and with one (partials and
counters in the fixed scratch), and the documented refusals."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def noalloc(fh, w, x, m, k, bias, y, numerics=0):
    import ferrum_hip

    L = ferrum_hip.lib()
    return L.fh_q8_0_linear_noalloc_async(fh.h, w.h, ferrum_hip._ptr(x), m, k, ferrum_hip._ptr(bias),
                                          0 if bias is None else w.n, ferrum_hip._ptr(y), numerics)


class W:
    def __init__(self, fh, orc, n, k, seed):
        import ferrum_hip

        self.raw = orc.quantize_weight(n, k, seed, 0.02)
        self.q = ferrum_hip.Q8_0Weight.upload(fh, self.raw, n, k)
        self.h, self.n, self.k = self.q.h, n, k


def run_pair(fh, w, m, seed, with_bias):
    import torch

    import ferrum_hip

    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((m, w.k)).astype(np.float32)).cuda()
    b = torch.from_numpy((rng.standard_normal(w.n) * 0.1).astype(np.float32)).cuda() if with_bias else None
    y_ref = torch.full((m, w.n), float("nan"), device="cuda")
    y_new = torch.full((m, w.n), float("nan"), device="cuda")
    torch.cuda.synchronize()
    ferrum_hip.linear_forward_async(fh, w.q, x, m, w.k, b, 0 if b is None else w.n, y_ref)
    fh.sync()
    fh.check(noalloc(fh, w, x, m, w.k, b, y_new))
    fh.sync()
    a, c = y_ref.cpu().numpy(), y_new.cpu().numpy()
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), (m, w.n, w.k)


# (n, k, m first, m second): GEMV, unsplit skinny tiles, and K-split skinny
# GEMMs (few output tiles) at m <= 32 and 32 < m <= 64.
CASES = [(3072, 768, 2, 1), (50257, 768, 1, 1), (768, 3072, 32, 8), (896, 4864, 64, 40), (2304, 768, 17, 3),
         (4096, 1024, 64, 33), (9728, 896, 64, 5), (1024, 12288, 2, 1), (2304, 768, 64, 40),
         (3072, 3072, 32, 8)]


@pytest.mark.parametrize("n,k,m1,m2", CASES)
def test_noalloc_linear_matches_the_allocating_call(fh, orc, n, k, m1, m2):
    w = W(fh, orc, n, k, n + k)
    try:
        run_pair(fh, w, m1, 1, True)
        run_pair(fh, w, m2, 2, False)
    finally:
        w.q.free()


def test_noalloc_refusals(fh, orc):
    import torch

    import ferrum_hip

    w = W(fh, orc, 64, 128, 3)
    x = torch.zeros((65, 128), device="cuda")
    y = torch.zeros((65, 64), device="cuda")
    torch.cuda.synchronize()
    try:
        assert noalloc(fh, w, x, 65, 128, None, y) == ferrum_hip.FH_ERR_LIMIT
        assert "above 64" in ferrum_hip.lib().fh_last_error(fh.h).decode()
        assert noalloc(fh, w, x, 4, 128, None, y, numerics=1) == ferrum_hip.FH_ERR_LIMIT
        assert noalloc(fh, w, x, 4, 96, None, y) == ferrum_hip.FH_ERR_DIM
        assert noalloc(fh, w, x, 0, 128, None, y) == ferrum_hip.FH_OK
    finally:
        w.q.free()
