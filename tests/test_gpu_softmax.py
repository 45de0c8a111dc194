"""The router softmax on the device, bit for bit against the CPU oracle
(moe_router.rs:52-72: max, expf(v - max), a sum in index order, 1 / sum,
multiply), and the top-k indices it decides in the zone where near-equal
probabilities make the reference's rules (strict `>` against the running
minimum, earlier index wins a tie, moe_router.rs:83-124) depend on the
last bit of every probability.

* The exponential: smoe_expf against the host libm's expf (what the
  oracle and the reference's f32::exp call) on every float in
  [-0x1.9fe368p6, 0] and the special inputs.
* Whole rows: smoe_softmax against oracle.softmax_rows on random logits of
  several widths and spreads (including -inf, repeated values and NaN).
* Sum-order-sensitive boundaries: 256-logit vectors whose k-th and
  (k+1)-th experts have adjacent exp values, chosen (on the CPU, with the
  oracle's expf) so that they tie in probability under the reference's
  sequential sum and do not under a pairwise (tree) sum, or the other way
  round, and so that this changes the reference's top-k output (which
  expert is routed, or the slot order). Plus logits 0, 1 and 2 ulps apart at the
  boundary and near-equal pairs inside the top-k (which decide the slot
  order), over 100+ seeds each. Run through smoe_softmax_topk, both decode
  paths of smoe_moe_decode_layer and smoe_moe_decode_tokens: idx and the
  routing weights equal the oracle's bit for bit.

Router rows carry the planted logits in column 0 and x[0] = 1 (all other
router columns zero), so every logit is exact on both sides whatever the
summation order of the router matvec.
"""
import numpy as np
import pytest

import oracle
from helpers import rel_err

pytestmark = pytest.mark.gpu

H = 2048
TOL = 1e-3
EXP_LO = 0xC2CFF1B4  # -0x1.9fe368p6: below it expf underflows to 0


def _torch():
    import torch

    return torch


def _dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def _same_bits(a, b):
    """Bit equality, any NaN equal to any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]) and np.array_equal(
        np.isnan(a), np.isnan(b))


# ---------------------------------------------------------------------------
# The exponential.
# ---------------------------------------------------------------------------
def test_expf_equals_oracle_on_every_softmax_input(kernels):
    torch = _torch()
    chunk = 1 << 26
    lo, hi = 0x80000000, EXP_LO
    xd = torch.empty(chunk, dtype=torch.float32, device="cuda")
    yd = torch.empty(chunk, dtype=torch.float32, device="cuda")
    total = bad = 0
    for start in range(lo, hi + 1, chunk):
        n = min(chunk, hi + 1 - start)
        x = np.arange(start, start + n, dtype=np.uint64).astype(np.uint32).view(np.float32)
        xd[:n].copy_(torch.from_numpy(x))
        assert kernels.expf(xd, yd, n) == 0
        got = yd[:n].cpu().numpy()
        want = oracle.expf_many(x)
        diff = got.view(np.uint32) != want.view(np.uint32)
        if diff.any():
            i = np.flatnonzero(diff)[:3]
            print("mismatch x", x[i], "gpu", got[i], "cpu", want[i])
        bad += int(diff.sum())
        total += n
    edge = np.float32(float.fromhex("-0x1.9fe368p6"))
    special = np.array([edge, np.nextafter(edge, np.float32(-np.inf)), -104.0,
                        -1e4, -np.inf, np.inf, np.nan, 0.0, -0.0, 1e-30, 1.0, 10.0, 88.0, 88.72, 89.0],
                       np.float32)
    sd = _dev(special)
    sy = torch.empty_like(sd)
    assert kernels.expf(sd, sy, special.size) == 0
    assert _same_bits(_host(sy), oracle.expf_many(special))
    print(f"expf: {total} inputs, {bad} mismatches")
    assert total == 1120924085 and bad == 0


# ---------------------------------------------------------------------------
# Whole softmax rows.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 2, 64, 128, 256, 300, 512, 1024])
def test_softmax_rows_bit_exact(kernels, n):
    torch = _torch()
    rng = np.random.default_rng(4000 + n)
    rows = []
    for sig in (0.02, 0.9, 5.0, 40.0):
        rows.append((rng.standard_normal((32, n)) * sig).astype(np.float32))
    r = (rng.standard_normal((8, n))).astype(np.float32)
    r[:, ::7] = -np.inf                          # masked experts
    rows.append(r)
    r = np.repeat((rng.standard_normal((8, 1))).astype(np.float32), n, axis=1)  # all equal
    rows.append(r)
    r = np.round(rng.standard_normal((8, n)) * 4).astype(np.float32) / 4       # many repeats
    rows.append(r)
    if n > 1:
        r = rng.standard_normal((2, n)).astype(np.float32)
        r[0, n // 2] = np.nan
        r[1, 0] = np.nan
        rows.append(r)
    x = np.concatenate(rows)
    p = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    assert kernels.softmax(_dev(x), x.shape[0], n, p) == 0
    got, want = _host(p), oracle.softmax_rows(x)
    bad = [i for i in range(x.shape[0]) if not _same_bits(got[i], want[i])]
    assert not bad, (bad[:5], got[bad[0]][:8], want[bad[0]][:8])


# ---------------------------------------------------------------------------
# Boundary cases.
# ---------------------------------------------------------------------------
def _probs_pairwise(e):
    """Probabilities with the sum taken as a pairwise tree (what a wave
    reduction computes), float32 throughout."""
    s = e.astype(np.float32).copy()
    while s.size > 1:
        if s.size % 2:
            s = np.append(s, np.float32(0))
        s = (s[0::2] + s[1::2]).astype(np.float32)
    inv = np.float32(1.0) / s[0]
    return (e * inv).astype(np.float32)


def _with_boundary(rng, E, k, a, b_idx, a_idx, d_ulps):
    """E logits: k - 1 clear winners, expert a_idx = a (the k-th), expert
    b_idx (< a_idx) d_ulps below it (the (k+1)-th), the rest lower."""
    lg = np.empty(E, np.float32)
    others = [e for e in rng.permutation(E) if e not in (a_idx, b_idx)]
    top, rest = others[:k - 1], others[k - 1:]
    lg[top] = (a + 0.05 + rng.uniform(0, 1.0, k - 1)).astype(np.float32)
    lg[rest] = (a - 0.05 - rng.uniform(0, 3.0, len(rest))).astype(np.float32)
    lg[a_idx] = a
    b = np.float32(a)
    for _ in range(d_ulps):
        b = np.nextafter(b, np.float32(-np.inf))
    lg[b_idx] = b
    return lg


def order_sensitive_cases(E=256, k=8, want=24, seed=0x5EED):
    """Vectors whose boundary tie status differs between the sequential sum
    (the reference) and a pairwise sum, and for which that changes the
    reference's top-k output (indices in slot order): computed with the
    pairwise sum's probabilities, the running-minimum scan routes a
    different expert or fills the slots in a different order."""
    rng = np.random.default_rng(seed)
    out = []
    tries = 0
    while len(out) < want and tries < 200000:
        tries += 1
        a_idx = int(rng.integers(1, E))
        b_idx = int(rng.integers(0, a_idx))
        a = np.float32(rng.uniform(-1.0, 1.0))
        for d in (1, 2, 3):
            lg = _with_boundary(rng, E, k, a, b_idx, a_idx, d)
            e = oracle.expf_many(lg - lg.max())
            if e[a_idx] == e[b_idx] or np.nextafter(e[b_idx], np.float32(1)) != e[a_idx]:
                continue  # want adjacent exp values
            p_seq = oracle.softmax(lg)
            p_tree = _probs_pairwise(e)
            if (p_seq[a_idx] == p_seq[b_idx]) != (p_tree[a_idx] == p_tree[b_idx]):
                if not np.array_equal(oracle.topk(p_seq, k)[1], oracle.topk(p_tree, k)[1]):
                    out.append((lg, a_idx, b_idx))
            break
    assert len(out) == want, (len(out), tries)
    return out


def ulp_cases(E, k, n_seeds, seed):
    """Boundary pairs 0, 1 and 2 ulps apart (the lower-index expert below),
    and, for the slot order, near-equal pairs inside the top-k."""
    rng = np.random.default_rng(seed)
    out = []
    for s in range(n_seeds):
        a_idx = int(rng.integers(1, E))
        b_idx = int(rng.integers(0, a_idx))
        lg = _with_boundary(rng, E, k, np.float32(rng.uniform(-2, 2)), b_idx, a_idx, s % 3)
        if s % 2:
            # two of the k - 1 winners 1 ulp apart (they decide the slot order)
            top = np.argsort(-lg.astype(np.float64), kind="stable")[:k - 1]
            i, j = top[0], top[1]
            lg[j] = np.nextafter(lg[i], np.float32(-np.inf))
        out.append(lg)
    return out


def _check_router(kernels, logits, k, normalize):
    torch = _torch()
    T, E = logits.shape
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    assert kernels.softmax_topk(_dev(logits), T, E, k, normalize, idx, w) == 0
    gi, gw = _host(idx), _host(w)
    for t in range(T):
        rc, widx, ww = oracle.router(logits[t], k, normalize)
        assert rc == 0
        assert np.array_equal(gi[t], widx), (t, list(gi[t]), list(widx))
        assert _same_bits(gw[t], ww), (t, gw[t], ww)


@pytest.mark.parametrize("normalize", [True, False], ids=["renorm", "raw"])
def test_router_order_sensitive_boundary(kernels, normalize):
    cases = order_sensitive_cases()
    _check_router(kernels, np.stack([c[0] for c in cases]), 8, normalize)


@pytest.mark.parametrize("E,k", [(256, 8), (64, 8), (512, 10), (128, 4)])
def test_router_ulp_boundary(kernels, E, k):
    _check_router(kernels, np.stack(ulp_cases(E, k, 120, 700 + E + k)), k, True)


@pytest.fixture(scope="module")
def layer_env(kernels):
    """One 256-expert C2-shape arena (4-bit) with a shared expert; routers
    are planted per case."""
    import streamoe_amd as sa

    torch = _torch()
    E = 256
    lay = sa.ExpertLayout(H, 512, 4, 64)
    arena = torch.empty(E * lay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, lay.expert_size, lay, 77) == 0
    sh = torch.empty(lay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(sh, 1, lay.expert_size, lay, 78) == 0
    gate = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(gate, 79, 0.02) == 0
    return dict(lay=lay, arena=arena, arena_h=_host(arena), sh=sh, sh_h=_host(sh), gate=gate,
                gate_h=_host(gate), E=E)


def _planted_router(env, cols):
    router = np.zeros((env["E"], H), np.float32)
    for t, lg in enumerate(cols):
        router[:, t] = lg
    return router


def _decode_case(kernels, env, logits_list, path, rng):
    torch = _torch()
    E, k = env["E"], 8
    lay = env["lay"]
    router = _planted_router(env, [logits_list])
    L = kernels.layer(lay, env["arena"], lay.expert_size, E, k, True, _dev(router), env["sh"], env["gate"])
    x = rng.standard_normal(H).astype(np.float32)
    x[0] = 1.0
    h_mid = rng.standard_normal(H).astype(np.float32)
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    w = torch.empty(k, dtype=torch.float32, device="cuda")
    kernels.set_decode_path(path)
    try:
        assert kernels.moe_decode_layer(L, _dev(x), _dev(h_mid), out, idx, w) == 0
        kernels.sync()
    finally:
        kernels.set_decode_path(0)
    want, widx, ww, wlog = oracle.moe_decode_layer(env["arena_h"], lay.expert_size, H, 512, E, k, 64, 4, True,
                                                   router, x, h_mid, env["sh_h"], env["gate_h"])
    assert np.array_equal(wlog.view(np.uint32), logits_list.view(np.uint32))
    gi, gw, got = _host(idx), _host(w), _host(out)
    assert np.array_equal(gi, widx), (list(gi), list(widx))
    assert _same_bits(gw, ww), (gw, ww)
    assert rel_err(got, want) <= TOL


@pytest.mark.parametrize("path", [1, 3], ids=["per-phase", "three-kernel"])
def test_decode_layer_order_sensitive_boundary(kernels, layer_env, path):
    rng = np.random.default_rng(31 + path)
    for lg, _, _ in order_sensitive_cases(want=12, seed=0xB0 + path):
        _decode_case(kernels, layer_env, lg, path, rng)


@pytest.mark.parametrize("path", [1, 3], ids=["per-phase", "three-kernel"])
def test_decode_layer_ulp_boundary(kernels, layer_env, path):
    rng = np.random.default_rng(41 + path)
    for lg in ulp_cases(256, 8, 12, 900 + path):
        _decode_case(kernels, layer_env, lg, path, rng)


def test_decode_tokens_ulp_boundary(kernels, layer_env):
    """smoe_moe_decode_tokens, four tokens, each on its own planted router
    column (x_t = e_t), boundary pairs 0-2 ulps apart and one
    order-sensitive vector."""
    torch = _torch()
    env = layer_env
    E, k, T = env["E"], 8, 4
    lay = env["lay"]
    cols = ulp_cases(E, k, 3, 555) + [order_sensitive_cases(want=1, seed=0xC0)[0][0]]
    router = _planted_router(env, cols)
    L = kernels.layer(lay, env["arena"], lay.expert_size, E, k, True, _dev(router), env["sh"], env["gate"])
    rng = np.random.default_rng(5)
    x = np.zeros((T, H), np.float32)
    for t in range(T):
        x[t, t] = 1.0
    xd = _dev(x)
    resid = xd.clone()
    work = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_tokens([L], None, 1e-6, T, xd, resid, work, idx, w) == 0
    kernels.sync()
    gi, gw, got = _host(idx), _host(w), _host(resid)
    for t in range(T):
        want, widx, ww, wlog = oracle.moe_decode_layer(env["arena_h"], lay.expert_size, H, 512, E, k, 64, 4, True,
                                                       router, x[t], x[t], env["sh_h"], env["gate_h"])
        assert np.array_equal(wlog.view(np.uint32), cols[t].view(np.uint32))
        assert np.array_equal(gi[t], widx), (t, list(gi[t]), list(widx))
        assert _same_bits(gw[t], ww)
        assert rel_err(got[t], want) <= TOL
    del rng
