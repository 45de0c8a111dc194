"""smoe_qmv_argmax (the LM head with the greedy pick, io/gpu_lm_head.rs:
130-193) called many times in a row and replayed from a HIP graph with new
inputs between replays, as a decode loop uses it (the per-wave partials
and the merge launch reuse the handle's scratch on every call), and on
row counts up to 300,001. The pick is the reference's scan (first maximal
index), here with a three-way tie of equal rows."""
import numpy as np
import pytest

from helpers import gen_quant_matrix
from test_gpu_decode import dev, host, qweights

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _first_max(y):
    best = 0
    for i in range(1, len(y)):
        if y[i] > y[best]:
            best = i
    return best


@pytest.fixture(scope="module")
def lm(kernels):
    V, H = 151936, 2048
    rng = np.random.default_rng(0x1A)
    codes, s, b = gen_quant_matrix(rng, V, H, 64, 4)
    # Rows 5000, 90000 and 140000: every code 15, scale 1, bias 0, so their
    # sums are equal (15 * sum x) and, for a positive x, the maximum, tied
    # three ways (the first index wins).
    for r in (5000, 90000, 140000):
        codes[r], s[r], b[r] = 0xFF, 0x3F80, 0
    return dict(V=V, H=H, w=qweights(codes, s, b, 64, 4), rng=rng)


def test_many_calls_in_a_row(kernels, lm):
    torch = _torch()
    V, H = lm["V"], lm["H"]
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    for call in range(40):
        x = lm["rng"].standard_normal(H).astype(np.float32)
        assert kernels.qmv_argmax(lm["w"], dev(x), y, V, H, out) == 0
        kernels.sync()
        got_y = host(y)
        assert int(host(out)[0]) == int(np.argmax(got_y)) == _first_max(got_y), call


def test_graph_replays(kernels, lm):
    """One captured call replayed with new x between replays: every replay
    (a new tag each time) picks its own y's first maximum."""
    import streamoe_amd as sa

    torch = _torch()
    V, H = lm["V"], lm["H"]
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    x.copy_(torch.from_numpy(lm["rng"].standard_normal(H).astype(np.float32)))

    def step():
        sa.check(kernels.qmv_argmax(lm["w"], x, y, V, H, out), "smoe_qmv_argmax")

    g = sa.capture_graph(kernels, step)
    for rep in range(12):
        xv = lm["rng"].standard_normal(H).astype(np.float32)
        if rep % 3 == 2:
            # x > 0: rows 5000 / 90000 / 140000 (equal sums) are the maximum
            xv = np.abs(xv) + np.float32(1.0)
        x.copy_(torch.from_numpy(xv))
        g.replay()
        torch.cuda.synchronize()
        got_y = host(y)
        assert int(host(out)[0]) == _first_max(got_y), rep
        if rep % 3 == 2:
            assert int(host(out)[0]) == 5000
    kernels.sync()


@pytest.mark.parametrize("rows,in_dim", [(262143, 256), (300001, 512)])
def test_large_row_counts(kernels, rows, in_dim):
    """The maximum planted in the last row."""
    torch = _torch()
    rng = np.random.default_rng(rows)
    codes, s, b = gen_quant_matrix(rng, rows, in_dim, 64, 4)
    codes[rows - 1] = 0xFF  # every code 15
    s[rows - 1] = 0x3F80    # scale 1.0
    b[rows - 1] = 0x3F80    # bias 1.0
    x = np.abs(rng.standard_normal(in_dim)).astype(np.float32)
    w = qweights(codes, s, b, 64, 4)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv_argmax(w, dev(x), y, rows, in_dim, out) == 0
    kernels.sync()
    got_y = host(y)
    assert int(host(out)[0]) == _first_max(got_y) == rows - 1
