"""GPU parity of the noaux_tc router (smoe_noaux_tc_topk) against the CPU
oracle's noaux_tc_router (moe_router.rs:211-330), through the C ABI.

Bars: top-k indices in the reference's slot order equal the oracle's;
weights within 1e-6 of the scaled weights. The device sigmoid uses the
device expf and the oracle the C library's, which differ by an ULP on some
inputs; every later step is compare-and-add arithmetic in the reference's
order. So on a token whose sigmoid scores agree bit for bit the indices
must match unconditionally, and on any other token they must match unless
a selection margin (group scores or masked biased scores) is below 1e-5,
which is reported.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def _run(kernels, L, bias, n_group, topk_group, k, scale, in_place=False):
    torch = _torch()
    T, E = L.shape
    lg = dev(L)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    so = lg if in_place else torch.empty((T, E), dtype=torch.float32, device="cuda")
    rc = kernels.noaux_tc_topk(lg, dev(bias), T, E, n_group, topk_group, k, scale, idx, w, so)
    assert rc == 0
    return host(idx), host(w), host(so)


def _margins(L, bias, n_group, topk_group, k):
    """Smallest gap at the two selection boundaries (group scores, masked
    biased scores), in float64 from the oracle's float32 scores."""
    s = 1.0 / (1.0 + np.exp(-L.astype(np.float64)))
    b = s + bias.astype(np.float64)
    g = np.sort(b.reshape(n_group, -1), axis=1)[:, -2:].sum(axis=1)
    gs = np.sort(g)[::-1]
    gm = gs[topk_group - 1] - gs[topk_group] if topk_group < n_group else np.inf
    keep = np.argsort(-g, kind="stable")[:topk_group]
    m = np.full_like(b, -np.inf)
    size = b.size // n_group
    for gi in keep:
        m[gi * size:(gi + 1) * size] = b[gi * size:(gi + 1) * size]
    ms = np.sort(m)[::-1]
    em = ms[k - 1] - ms[k] if k < b.size and np.isfinite(ms[k]) else np.inf
    return min(gm, em)


def _check(L, bias, n_group, topk_group, k, scale, gi, gw, gs):
    exact = 0
    for t in range(L.shape[0]):
        rc, widx, ww, ws = oracle.noaux_tc_router(L[t], bias, n_group, topk_group, k, scale)
        assert rc == 0
        same_scores = np.array_equal(gs[t].view(np.uint32), ws.view(np.uint32))
        exact += same_scores
        if same_scores:
            assert np.array_equal(gi[t], widx), (t, gi[t], widx)
        elif not np.array_equal(gi[t], widx):
            margin = _margins(L[t], bias, n_group, topk_group, k)
            assert margin < 1e-5, (t, gi[t], widx, margin)
            print(f"noaux t={t}: near tie (margin {margin:.2e}), indices differ")
            continue
        else:
            assert np.max(np.abs(gs[t] - ws)) <= 2e-7
        assert np.max(np.abs(gw[t] - ww)) <= 1e-6 * max(1.0, abs(scale)), t
    return exact


def test_noaux_hand_reference(kernels):
    """moe_router.rs:528-580: idx {5, 7}, weights 1.1822 / 1.3178."""
    L = np.array([[3.0, -2.0, 1.0, -1.0, -3.0, 2.0, 0.0, 4.0]], np.float32)
    bias = np.array([0.1, 0.2, -0.3, 0.0, 0.0, 0.4, -0.1, 0.05], np.float32)
    gi, gw, gs = _run(kernels, L, bias, 2, 1, 2, 2.5)
    pairs = sorted(zip(gi[0].tolist(), gw[0].tolist()))
    assert [i for i, _ in pairs] == [5, 7]
    assert abs(pairs[0][1] - 1.1822) < 1e-3 and abs(pairs[1][1] - 1.3178) < 1e-3
    _check(L, bias, 2, 1, 2, 2.5, gi, gw, gs)


def test_noaux_cogito_fixture(kernels):
    """moe_router.rs:585-640 inputs (256 experts, 8 groups, top-4 groups,
    k 8, scaling 2.5): same indices and weights as the oracle."""
    i = np.arange(256, dtype=np.float32)
    L = (np.sin(i * np.float32(0.137)) * 2).astype(np.float32)[None, :]
    bias = (np.cos(i * np.float32(0.241)) * np.float32(0.5)).astype(np.float32)
    gi, gw, gs = _run(kernels, L, bias, 8, 4, 8, 2.5)
    assert abs(float(gw.sum()) - 2.5) < 1e-3
    assert len({int(j) // 32 for j in gi[0]}) <= 4 and len(set(gi[0].tolist())) == 8
    _check(L, bias, 8, 4, 8, 2.5, gi, gw, gs)


@pytest.mark.parametrize("T,E,n_group,topk_group,k", [
    (1, 256, 8, 4, 8), (64, 256, 8, 4, 8), (16, 64, 4, 2, 6), (8, 512, 16, 3, 10),
    (4, 1024, 64, 8, 16), (6, 128, 1, 1, 8), (5, 96, 3, 3, 4), (9, 8, 2, 1, 2), (3, 160, 32, 32, 16),
    # every power-of-two group size (1 .. 64 experts per group: the lane
    # path) and two that are not (the scan path)
    (4, 64, 64, 16, 8), (4, 128, 64, 9, 8), (4, 256, 64, 7, 8), (4, 256, 32, 5, 8), (4, 256, 16, 3, 8),
    (4, 256, 4, 2, 8), (4, 192, 16, 5, 8), (4, 240, 5, 2, 8),
])
def test_noaux_random_vs_oracle(kernels, T, E, n_group, topk_group, k):
    rng = np.random.default_rng(E * 7 + T + k)
    L = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    gi, gw, gs = _run(kernels, L, bias, n_group, topk_group, k, 2.5)
    exact = _check(L, bias, n_group, topk_group, k, 2.5, gi, gw, gs)
    print(f"noaux E={E} groups={n_group}/{topk_group} k={k}: {exact}/{T} tokens with identical sigmoid scores")


def test_noaux_ties_nan_and_start_slots(kernels):
    """Cases the reference's compares decide: equal scores everywhere (the
    first groups and experts keep their slots), NaN logits (never win a
    compare), a group whose bias is -inf, and k above the kept experts (the
    start slots keep index 0)."""
    E = 64
    cases = []
    cases.append((np.zeros(E, np.float32), np.zeros(E, np.float32), 4, 2, 8))
    L = np.random.default_rng(5).standard_normal(E).astype(np.float32)
    L[[3, 17, 40]] = np.nan
    cases.append((L, np.zeros(E, np.float32), 4, 2, 8))
    b = np.zeros(E, np.float32)
    b[16:32] = -np.inf
    cases.append((np.random.default_rng(6).standard_normal(E).astype(np.float32), b, 4, 3, 8))
    cases.append((np.random.default_rng(7).standard_normal(E).astype(np.float32), np.zeros(E, np.float32), 16, 1,
                  8))  # 4 kept experts, k 8
    L = np.full(E, 1.0, np.float32)
    L[::2] = 0.5
    cases.append((L, np.zeros(E, np.float32), 8, 3, 5))
    for L, bias, ng, tg, k in cases:
        gi, gw, gs = _run(kernels, L[None, :], bias, ng, tg, k, 1.0)
        rc, widx, ww, ws = oracle.noaux_tc_router(L, bias, ng, tg, k, 1.0)
        assert rc == 0
        assert np.array_equal(gi[0], widx), (ng, tg, k, gi[0], widx)
        assert np.array_equal(np.isnan(gs[0]), np.isnan(ws))
        assert np.allclose(gw[0], ww, rtol=0, atol=1e-6, equal_nan=True), (gw[0], ww)


def test_noaux_in_place_scores(kernels):
    """scores_out == logits: the logits are replaced by the sigmoid scores
    (the reference mutates its logits in place) and the routing is
    unchanged."""
    rng = np.random.default_rng(21)
    L = rng.standard_normal((8, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.2).astype(np.float32)
    gi0, gw0, gs0 = _run(kernels, L, bias, 8, 4, 8, 2.5)
    gi1, gw1, gs1 = _run(kernels, L, bias, 8, 4, 8, 2.5, in_place=True)
    assert np.array_equal(gi0, gi1) and np.array_equal(gw0, gw1) and np.array_equal(gs0, gs1)


def test_noaux_argument_errors(kernels):
    """moe_router.rs:221-255 order (EmptyScores, then BadK), plus this
    build's limits; nothing is launched."""
    torch = _torch()
    lg = torch.zeros(2048, dtype=torch.float32, device="cuda")
    b = torch.zeros(2048, dtype=torch.float32, device="cuda")
    idx = torch.empty(16, dtype=torch.int32, device="cuda")
    w = torch.empty(16, dtype=torch.float32, device="cuda")

    def call(E, ng, tg, k, T=1):
        return kernels.noaux_tc_topk(lg, b, T, E, ng, tg, k, 1.0, idx, w)

    assert call(0, 1, 1, 1) == 1
    assert call(8, 1, 1, 1, T=0) == 1
    assert call(8, 0, 1, 1) == 2
    assert call(8, 3, 1, 1) == 2
    assert call(8, 2, 0, 1) == 2
    assert call(8, 2, 3, 1) == 2
    assert call(8, 2, 1, 0) == 2
    assert call(8, 2, 1, 9) == 2
    assert call(64, 2, 1, 17) == 2
    assert call(2048, 8, 4, 8) == 6
    assert call(1024, 128, 4, 8) == 6
    assert kernels.noaux_tc_topk(None, b, 1, 8, 2, 1, 2, 1.0, idx, w) == 1
