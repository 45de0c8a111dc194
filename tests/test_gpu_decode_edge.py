"""Routing edge cases and activation outliers on the decode hot path,
through the C ABI, against the CPU oracle.

Routing: the router rows carry one non-zero (column 0) and x[0] = 1, so
every logit is an exact multiple of 2^-23 on the GPU and in the oracle
alike, whatever the summation order. The k-th / (k+1)-th boundary then
holds an exact tie, a tie of three, or a margin of 2^-22 (inside the zone
where the decode kernels' fast top-k set refuses and the exact
running-minimum scan runs), or one logit is NaN. The reference's rules
(crates/streammoe/src/riir/moe/moe_router.rs:52-141): strict `>` against
the running minimum, so of equal values the earlier index wins and the
slot order is the replacement order; a NaN logit makes every probability
NaN, so no score beats the -1e30 start and all k slots stay (index 0,
value -1e30), which the guarded renormalisation leaves as they are.

Outliers: x = N(0, 1) with a few +-100 channels and one 32-value chunk
spanning 2^20 between its largest and smallest magnitude (the decode
matvecs hold x as 24-bit block floating point per chunk).
"""
import numpy as np
import pytest

import oracle
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3
H = 2048
UNIT = 2.0 ** -23


def _torch():
    import torch

    return torch


def _dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def boundary_logits(E, k, kind, first, second, rng):
    """E exact logits (multiples of 2^-23): k - 1 clear winners in [0.4, 0.5),
    the rest below 0.25, and at the k-th / (k+1)-th boundary experts
    `first` and `second` as `kind` says: "tie" equal, "tie3" equal with a
    third expert (the next index after `second`), "margin" second larger
    by 2^-22, "nan" first is NaN."""
    taken = {first, second}
    if kind == "tie3":
        third = next(e for e in range(second + 1, E) if e not in taken)
        taken.add(third)
    others = [e for e in rng.permutation(E) if e not in taken]
    lg = np.empty(E, np.float64)
    top = others[:k - 1] if kind != "tie3" else others[:k - 2]
    for i, e in enumerate(top):
        lg[e] = 0.4 + 0.01 * i
    for e in others[len(top):]:
        lg[e] = rng.uniform(-2.0, 0.25)
    lg = np.round(lg / UNIT) * UNIT
    b = np.round(0.3 / UNIT) * UNIT
    lg[first] = b
    lg[second] = b + (2 * UNIT if kind == "margin" else 0.0)
    if kind == "tie3":
        lg[third] = b
    out = lg.astype(np.float32)
    assert np.all(out.astype(np.float64) == lg)
    if kind == "nan":
        out[first] = np.nan
    return out


def _layer(kernels, logits, k, normalize, shared, seed, inter=512, bits=4, hid=H):
    import streamoe_amd as sa

    torch = _torch()
    H = hid
    E = logits.size
    lay = sa.ExpertLayout(H, inter, bits, 64)
    arena = torch.empty(E * lay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, lay.expert_size, lay, seed) == 0
    router = np.zeros((E, H), np.float32)
    router[:, 0] = logits
    sh = gate = None
    if shared:
        slay = sa.ExpertLayout(H, inter, 4, 64)
        sh = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(sh, 1, slay.expert_size, slay, seed + 1) == 0
        gate = torch.empty(H, dtype=torch.float32, device="cuda")
        assert kernels.synth_normal_f32(gate, seed + 2, 0.02) == 0
    r_dev = _dev(router)
    L = kernels.layer(lay, arena, lay.expert_size, E, k, normalize, r_dev, sh, gate)
    return dict(L=L, arena=arena, router=router, r_dev=r_dev, sh=sh, gate=gate, lay=lay, E=E, k=k,
                normalize=normalize, bits=bits, inter=inter, H=H)


def _oracle(c, x, h_mid):
    return oracle.moe_decode_layer(_host(c["arena"]), c["lay"].expert_size, c["H"], c["inter"], c["E"], c["k"], 64,
                                   c["bits"], c["normalize"], c["router"], x, h_mid,
                                   None if c["sh"] is None else _host(c["sh"]),
                                   None if c["gate"] is None else _host(c["gate"]))


CASES = [
    # kind, E, k, first, second
    ("tie", 256, 8, 37, 200),      # earlier index wins
    ("tie", 256, 8, 201, 12),      # the later expert in index order loses although listed first
    ("tie3", 256, 8, 9, 140),      # three equal values for two slots
    ("margin", 256, 8, 50, 51),    # the larger wins by 2^-22
    ("margin", 256, 8, 180, 3),
    ("tie", 64, 8, 5, 6),          # OLMoE-size router
    ("tie", 128, 10, 100, 90),     # the reference's other supported top-k
    ("nan", 256, 8, 77, 78),
]
CASE_IDS = [f"{c[0]}-E{c[1]}-k{c[2]}-{c[3]}-{c[4]}" for c in CASES]


CASES_4096 = [
    # hidden 4096, the Qwen3.5-397B-A17B router width (512 experts, top-10)
    ("tie", 512, 10, 300, 17),
    ("tie3", 512, 10, 8, 400),
    ("margin", 512, 10, 250, 251),
    ("nan", 512, 10, 5, 6),
]


@pytest.mark.parametrize("path", [1, 3], ids=["per-phase", "three-kernel"])
@pytest.mark.parametrize("kind,E,k,first,second,hid",
                         [c + (2048,) for c in CASES] + [c + (4096,) for c in CASES_4096],
                         ids=CASE_IDS + [f"h4096-{c[0]}-E{c[1]}-k{c[2]}-{c[3]}-{c[4]}" for c in CASES_4096])
def test_decode_layer_routing_boundary(kernels, path, kind, E, k, first, second, hid):
    torch = _torch()
    H = hid
    rng = np.random.default_rng(E * 1000 + first * 7 + second)
    logits = boundary_logits(E, k, kind, first, second, rng)
    c = _layer(kernels, logits, k, True, True, seed=first * 31 + second, hid=H)
    x = rng.standard_normal(H).astype(np.float32)
    x[0] = 1.0
    h_mid = rng.standard_normal(H).astype(np.float32)
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    w = torch.empty(k, dtype=torch.float32, device="cuda")
    kernels.set_decode_path(path)
    try:
        assert kernels.moe_decode_layer(c["L"], _dev(x), _dev(h_mid), out, idx, w) == 0
        kernels.sync()
    finally:
        kernels.set_decode_path(0)
    want, widx, ww, wlog = _oracle(c, x, h_mid)
    assert np.array_equal(wlog.view(np.uint32), logits.view(np.uint32))  # the oracle saw the planted logits
    gi, gw, got = _host(idx), _host(w), _host(out)
    print(f"{kind} path={path}: idx gpu={list(gi)} cpu={list(widx)}")
    assert np.array_equal(gi, widx)
    if kind == "nan":
        assert np.all(widx == 0) and np.all(ww == np.float32(-1e30))
        assert np.array_equal(gw.view(np.uint32), ww.view(np.uint32))
        assert np.array_equal(np.isfinite(got), np.isfinite(want))
        fin = np.isfinite(want)
        if fin.any():
            assert rel_err(got[fin], want[fin]) <= TOL
        return
    assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
    err = rel_err(got, want)
    print(f"  rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("kind,first,second", [("tie", 37, 200), ("margin", 50, 51), ("tie3", 9, 140)])
def test_decode_tokens_routing_boundary(kernels, kind, first, second):
    """smoe_moe_decode_tokens: two tokens, both at the planted boundary;
    the last layer's idx / w come back in the reference's slot order."""
    torch = _torch()
    E, k, T = 256, 8, 2
    rng = np.random.default_rng(first + second)
    logits = boundary_logits(E, k, kind, first, second, rng)
    c = _layer(kernels, logits, k, True, True, seed=first + 3 * second)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[:, 0] = 1.0
    xd = _dev(x)
    resid = xd.clone()
    work = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_tokens([c["L"]], None, 1e-6, T, xd, resid, work, idx, w) == 0
    kernels.sync()
    gi, gw, got = _host(idx), _host(w), _host(resid)
    for t in range(T):
        want, widx, ww, _ = _oracle(c, x[t], x[t])
        assert np.array_equal(gi[t], widx), (t, list(gi[t]), list(widx))
        assert np.max(np.abs(gw[t] - ww)) <= 1e-5 * np.max(np.abs(ww))
        assert rel_err(got[t], want) <= TOL


def outlier_x(rng, n):
    """N(0, 1) with a few +-100 channels and, in chunk 5, magnitudes spread
    over 2^20 (max / min = 2^20)."""
    x = rng.standard_normal(n).astype(np.float32)
    hot = rng.choice(n, 6, replace=False)
    x[hot] = np.float32(100.0) * np.sign(rng.standard_normal(6)).astype(np.float32)
    ch = np.arange(5 * 32, 6 * 32)
    mags = 2.0 ** (-np.linspace(0, 20, 32))
    x[ch] = (mags * np.sign(rng.standard_normal(32))).astype(np.float32)
    return x


@pytest.mark.parametrize("path", [1, 3], ids=["per-phase", "three-kernel"])
@pytest.mark.parametrize("bits,H", [(4, 2048), (3, 2048), (4, 4096)], ids=["4bit", "3bit", "4bit-h4096"])
def test_decode_layer_outlier_activations(kernels, path, bits, H):
    """C2 layer (256 experts, top-8, shared expert) on outlier activations;
    the same at hidden 4096 (two 32-value chunks per lane)."""
    import streamoe_amd as sa

    torch = _torch()
    E, k = 256, 8
    rng = np.random.default_rng(900 + bits + H)
    lay = sa.ExpertLayout(H, 512, bits, 64)
    slay = sa.ExpertLayout(H, 512, 4, 64)
    arena = torch.empty(E * lay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, lay.expert_size, lay, 901) == 0
    sh = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(sh, 1, slay.expert_size, slay, 902) == 0
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    gate = (rng.standard_normal(H) * 0.02).astype(np.float32)
    x = outlier_x(rng, H)
    h_mid = rng.standard_normal(H).astype(np.float32)
    rd, gd = _dev(router), _dev(gate)
    L = kernels.layer(lay, arena, lay.expert_size, E, k, True, rd, sh, gd)
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    kernels.set_decode_path(path)
    try:
        assert kernels.moe_decode_layer(L, _dev(x), _dev(h_mid), out, idx) == 0
        kernels.sync()
    finally:
        kernels.set_decode_path(0)
    want, widx, _, wlog = oracle.moe_decode_layer(_host(arena), lay.expert_size, H, 512, E, k, 64, bits, True,
                                                  router, x, h_mid, _host(sh), gate)
    p = np.sort(oracle.softmax(wlog))[::-1]
    got = _host(out)
    err = rel_err(got, want)
    moe_err = rel_err(got - h_mid, want - h_mid)
    print(f"outliers bits={bits} path={path}: rel_err={err:.3e} (MoE part alone {moe_err:.3e}), "
          f"top-k gap={p[k - 1] - p[k]:.3e}")
    assert np.array_equal(_host(idx), widx)
    assert err <= TOL and moe_err <= TOL


def test_lm_head_outlier_activations(kernels):
    """C1 LM head (151,936 x 2048, 4-bit g64) on outlier activations:
    rel err within 1e-3 and the argmax bit-exact when certified."""
    import streamoe_amd as sa
    from helpers import gen_quant_matrix
    from test_gpu_decode import oracle_matvec, qweights

    torch = _torch()
    V = 151936
    rng = np.random.default_rng(0xC10)
    codes, s, b = gen_quant_matrix(rng, V, H, 64, 4)
    x = outlier_x(rng, H)
    w = qweights(codes, s, b, 64, 4)
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv_argmax(w, _dev(x), y, V, H, am) == 0
    want, _ = oracle_matvec(codes, s, b, H, V, 64, 4, x)
    got = _host(y)
    err = rel_err(got, want)
    top2 = np.sort(want)[-2:]
    dmax = float(np.max(np.abs(got - want)))
    print(f"lm_head outliers: rel_err={err:.3e} max|d|={dmax:.3e} top-2 gap={top2[1] - top2[0]:.3e}")
    assert err <= TOL
    if top2[1] - top2[0] > 2 * dmax:
        assert int(_host(am)[0]) == oracle.argmax(want)
    del sa
