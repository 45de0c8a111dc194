"""8-bit affine router and shared gate on the GPU, through the C ABI.

The reference's A3B models keep `mlp.gate.weight` and
`mlp.shared_expert_gate.weight` in 8-bit affine form
(linear_attn_forward.rs:1300-1301; dequant_matvec_8bit_gs_cpu,
cpu_matvec.rs:205-283; GPU kernel dequant_matvec_8bit_v3,
shaders.metal:619-677). Checked here: smoe_qmv / smoe_qmv_argmax /
smoe_qmm with bits 8 against the oracle; decode layers with an 8-bit router
and gate (per-phase and three-kernel paths, hidden 2048 and 4096, several
tokens at once, the no-allocation chain) against the oracle within the
decode bars (top-k indices exact, output within 1e-3), and bit for bit
against the f32 router holding the same weights when every dequantized
weight is exact; argument errors."""
import ctypes as C

import numpy as np
import pytest

import oracle
from helpers import bf16, gen_quant_matrix, rel_err
from test_gpu_decode import dev, host, qweights

pytestmark = pytest.mark.gpu

TOL = 1e-3
PATHS = [1, 3]
PATH_IDS = ["per-phase", "three-kernel"]


def _torch():
    import torch

    return torch


def _q8(rng, rows, H, G=64):
    """A generic 8-bit matrix with router-like weights (|w| ~ 0.02)."""
    return gen_quant_matrix(rng, rows, H, G, 8, ssig=2e-4, bsig=0.02)


def _exact_q8(rng, rows, H, G=64):
    """8-bit rows whose weights fma(q, s, b) = (q - k) 2^-10 are exact in
    f32; returns (codes, scales, biases) and the f32 weights."""
    q = rng.integers(0, 256, (rows, H), dtype=np.uint8)
    s = np.full((rows, H // G), bf16(2.0 ** -10), np.uint16)
    kb = rng.integers(100, 156, (rows, H // G))
    b = bf16(-kb * 2.0 ** -10)
    w = ((q.astype(np.float64) - np.repeat(kb, G, 1)) * 2.0 ** -10).astype(np.float32)
    return (q, s, b), w


def _dequant_f64(q, s, b, G):
    return (q.astype(np.float64) * np.repeat(oracle.bf16_to_f32(s).astype(np.float64), G, 1) +
            np.repeat(oracle.bf16_to_f32(b).astype(np.float64), G, 1))


# --- matvec ------------------------------------------------------------------------

@pytest.mark.parametrize("out_dim,in_dim,group", [
    (256, 2048, 64), (1, 2048, 64), (512, 4096, 64), (100, 1024, 32), (77, 8192, 128), (3, 64, 32),
    (5000, 2048, 64),
])
def test_qmv8_matches_oracle(kernels, out_dim, in_dim, group):
    rng = np.random.default_rng(out_dim + 3 * in_dim + group)
    q, s, b = _q8(rng, out_dim, in_dim, group)
    x = rng.standard_normal(in_dim).astype(np.float32)
    torch = _torch()
    y = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    assert kernels.qmv(qweights(q, s, b, group, 8), dev(x), y, out_dim, in_dim) == 0
    rc, want = oracle.dequant_matvec_8bit_gs(q, s, b, in_dim, out_dim, group, x)
    assert rc == 0
    got = host(y)
    # Both are f32 FMA chains over the same weights fma(q, s, b), summed in
    # different orders: within 2 in_dim 2^-24 sum |w x| of each other.
    W = _dequant_f64(q, s, b, group)
    bound = 2 * in_dim * 2.0 ** -24 * (np.abs(W) @ np.abs(x.astype(np.float64)))
    print(f"qmv8 {out_dim}x{in_dim} g{group}: rel_err={rel_err(got, want):.3e}")
    assert np.all(np.abs(got - want) <= bound)


def test_qmv8_argmax_and_qmm(kernels):
    """smoe_qmv_argmax gives smoe_qmv's y and its first maximum; smoe_qmm
    gives each token row as smoe_qmv does (bit for bit)."""
    torch = _torch()
    rng = np.random.default_rng(81)
    O, I, G, T = 2000, 2048, 64, 3
    q, s, b = _q8(rng, O, I, G)
    w = qweights(q, s, b, G, 8)
    xs = rng.standard_normal((T, I)).astype(np.float32)
    xd = dev(xs)
    ys = []
    for t in range(T):
        y = torch.empty(O, dtype=torch.float32, device="cuda")
        assert kernels.qmv(w, xd[t], y, O, I) == 0
        ys.append(host(y))
    y2 = torch.empty(O, dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv_argmax(w, xd[0], y2, O, I, out) == 0
    assert np.array_equal(host(y2).view(np.uint32), ys[0].view(np.uint32))
    assert int(host(out)[0]) == int(np.argmax(ys[0]))
    ws = torch.empty(max(1, kernels.qmm_workspace_size(I, G, T)), dtype=torch.uint8, device="cuda")
    ym = torch.empty((T, O), dtype=torch.float32, device="cuda")
    assert kernels.qmm(w, xd, ym, O, I, T, ws) == 0
    assert np.array_equal(host(ym).view(np.uint32), np.stack(ys).view(np.uint32))


@pytest.mark.parametrize("rows,in_dim,group,row0", [
    (7, 2048, 64, 2), (1, 2048, 64, 0), (64, 1024, 32, 5), (3, 8192, 128, 1), (1, 32, 32, 0),
])
def test_dequant8_bit_exact(kernels, rows, in_dim, group, row0):
    """smoe_dequant on 8-bit rows (the load-time f32 form of an 8-bit
    shared-expert gate): every weight fma(q, s, b) bit for bit against the
    oracle, from row row0 on."""
    rng = np.random.default_rng(rows * 7 + in_dim + group)
    q, s, b = _q8(rng, rows + row0, in_dim, group)
    torch = _torch()
    out = torch.empty((rows, in_dim), dtype=torch.float32, device="cuda")
    assert kernels.dequant(qweights(q, s, b, group, 8), in_dim, row0, rows, out) == 0
    want = oracle.dequant_8bit(q, s, b, in_dim, rows + row0, group)[row0:]
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


def test_qmv8_argument_errors(kernels):
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(16384, dtype=torch.float32, device="cuda")
    y = torch.zeros(16, dtype=torch.float32, device="cuda")
    w = sa.QuantWeights(buf, 0, 1 << 18, 1 << 19, 64, 8)
    assert kernels.qmv(w, x, y, 2, 16384) == _abi.CODES["SMOE_ERR_UNSUPPORTED_SHAPE"]
    assert kernels.dequant(w, 2048 + 16, 0, 1, x) == _abi.CODES["SMOE_ERR_IN_DIM_NOT_MULTIPLE"]
    w = sa.QuantWeights(buf, 4, 1 << 18, 1 << 19, 64, 8)
    assert kernels.qmv(w, x, y, 2, 2048) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    w = sa.QuantWeights(buf, 0, 1 << 18, 1 << 19, 64, 8)
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv_argmax(w, x, y[1:], 2, 2048, out) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    torch.cuda.synchronize()


# --- decode layers -----------------------------------------------------------------

def _layer(kernels, H, I, E, k, seed, router="q8", gate="q8", exact=False):
    """A layer with the router / shared gate in 8-bit ("q8") or f32 form
    (gate None: no gate; "none": no shared expert). Returns (layer, host
    data for the oracle, device tensors kept alive)."""
    import streamoe_amd as sa

    torch = _torch()
    rng = np.random.default_rng(seed)
    lay = sa.ExpertLayout(H, I, 4, 64)
    stride = lay.expert_size
    arena = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, stride, lay, seed) == 0
    keep = [arena]
    d = dict(H=H, I=I, E=E, k=k, stride=stride, arena=arena, router_w=None, router_q8=None, gate_w=None,
             gate_q8=None, shared=None)

    def rows(n):
        if exact:
            (q, s, b), wf = _exact_q8(rng, n, H)
        else:
            q, s, b = _q8(rng, n, H)
            wf = _dequant_f64(q, s, b, 64).astype(np.float32)
        return (q, s, b, 64), wf

    rq = gq = rw = gw = None
    if router == "q8":
        d["router_q8"], d["router_f32"] = rows(E)
        rq = qweights(*d["router_q8"][:3], 64, 8)
        keep.append(rq.buffer)
    else:
        d["router_w"] = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        rw = dev(d["router_w"])
        keep.append(rw)
    sh = None
    if gate != "none":
        slay = sa.ExpertLayout(H, I, 4, 64)
        sh = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(sh, 1, slay.expert_size, slay, seed + 4) == 0
        keep.append(sh)
        d["shared"] = sh
        if gate == "q8":
            d["gate_q8"], d["gate_f32"] = rows(1)
            gq = qweights(*d["gate_q8"][:3], 64, 8)
            keep.append(gq.buffer)
        elif gate == "f32":
            d["gate_w"] = (rng.standard_normal(H) * 0.02).astype(np.float32)
            gw = dev(d["gate_w"])
            keep.append(gw)
    L = kernels.layer(lay, arena, stride, E, k, True, rw, sh, gw, router_q=rq, shared_gate_q=gq)
    return L, d, keep


def _run(kernels, L, H, k, x, h_mid):
    torch = _torch()
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    w = torch.empty(k, dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_layer(L, x, h_mid, out, idx, w) == 0
    kernels.sync()
    return host(out), host(idx), host(w)


def _inputs(kernels, H, seed):
    torch = _torch()
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(x, seed + 2, 1.0) == 0
    h_mid = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(h_mid, seed + 3, 1.0) == 0
    return x, h_mid


@pytest.mark.parametrize("path", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("H,I,E,k", [(2048, 512, 256, 8), (4096, 1024, 512, 10)])
def test_q8_layer_equals_f32_layer_of_its_weights(kernels, path, H, I, E, k):
    """Every dequantized weight exact: the 8-bit router and gate give the
    f32 router and gate layer's output, indices and weights bit for bit
    (the same values enter the same FMA chains)."""
    kernels.set_decode_path(path)
    try:
        seed = 900 + H + path
        Lq, d, keep = _layer(kernels, H, I, E, k, seed, exact=True)
        x, h_mid = _inputs(kernels, H, seed)
        rw, gw = dev(d["router_f32"]), dev(d["gate_f32"][0])
        import streamoe_amd as sa

        lay = sa.ExpertLayout(H, I, 4, 64)
        Lf = kernels.layer(lay, d["arena"], d["stride"], E, k, True, rw, d["shared"], gw)
        a = _run(kernels, Lq, H, k, x, h_mid)
        b = _run(kernels, Lf, H, k, x, h_mid)
        for u, v in zip(a, b):
            assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
    finally:
        kernels.set_decode_path(0)


Q8_CASES = [
    # name, H, I, E, k, router, gate
    ("a3b-q8", 2048, 512, 256, 8, "q8", "q8"),
    ("a3b-q8-router-f32-gate", 2048, 512, 256, 8, "q8", "f32"),
    ("a3b-f32-router-q8-gate", 2048, 512, 256, 8, "f32", "q8"),
    ("a3b-q8-ungated", 2048, 512, 256, 8, "q8", None),
    ("a3b-q8-noshared", 2048, 512, 256, 8, "q8", "none"),
    ("q397b-q8", 4096, 1024, 512, 10, "q8", "q8"),
    ("olmoe-q8", 2048, 1024, 64, 8, "q8", "none"),
]


@pytest.mark.parametrize("path", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("name,H,I,E,k,router,gate", Q8_CASES, ids=[c[0] for c in Q8_CASES])
def test_q8_layer_matches_oracle(kernels, path, name, H, I, E, k, router, gate):
    kernels.set_decode_path(path)
    try:
        seed = sum(map(ord, name)) * 5 + path
        L, d, keep = _layer(kernels, H, I, E, k, seed, router, gate)
        x, h_mid = _inputs(kernels, H, seed)
        got, gi, gw = _run(kernels, L, H, k, x, h_mid)
        want, wi, ww, logits = oracle.moe_decode_layer(
            host(d["arena"]), d["stride"], H, I, E, k, 64, 4, True, d["router_w"], host(x), host(h_mid),
            None if d["shared"] is None else host(d["shared"]), d["gate_w"], router_q8=d["router_q8"],
            gate_q8=d["gate_q8"])
        p = np.sort(oracle.softmax(logits))[::-1]
        err = rel_err(got, want)
        print(f"q8 layer {name} path={path}: idx gpu={list(gi)} cpu={list(wi)} gap={p[k - 1] - p[k]:.3e} "
              f"rel_err={err:.3e}")
        assert np.array_equal(gi, wi)
        assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
        assert err <= TOL
    finally:
        kernels.set_decode_path(0)


@pytest.mark.parametrize("name,H,I,E,k", [("flash-next-q8", 2560, 640, 512, 10), ("tiny-q8", 256, 64, 8, 3)])
def test_q8_layer_other_shapes_per_phase(kernels, name, H, I, E, k):
    """Shapes without a three-kernel instance (the default path takes the
    per-phase kernels for them): the 8-bit router and gate against the
    oracle."""
    seed = sum(map(ord, name)) * 3
    L, d, keep = _layer(kernels, H, I, E, k, seed)
    x, h_mid = _inputs(kernels, H, seed)
    got, gi, gw = _run(kernels, L, H, k, x, h_mid)
    want, wi, ww, logits = oracle.moe_decode_layer(
        host(d["arena"]), d["stride"], H, I, E, k, 64, 4, True, None, host(x), host(h_mid), host(d["shared"]), None,
        router_q8=d["router_q8"], gate_q8=d["gate_q8"])
    err = rel_err(got, want)
    print(f"q8 layer {name}: idx gpu={list(gi)} cpu={list(wi)} rel_err={err:.3e}")
    assert np.array_equal(gi, wi)
    assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
    assert err <= TOL


def _q8_chain(kernels, NL, H, I, E, k, seed):
    """NL layers with 8-bit routers and gates, bf16 RMSNorm weights."""
    torch = _torch()
    rng = np.random.default_rng(seed)
    layers, norms, keep = [], [], []
    for l in range(NL):
        L, d, kp = _layer(kernels, H, I, E, k, seed + 100 * l)
        layers.append(L)
        keep += kp
        nw = bf16(1.0 + 0.1 * rng.standard_normal(H)).view(np.int16)
        norms.append(torch.from_numpy(nw.copy()).cuda())
    return layers, norms, keep


@pytest.mark.parametrize("T", [2, 3, 4])
def test_q8_tokens_match_single_token_decode(kernels, T):
    """Several tokens at once through 8-bit-routed layers: each token equals
    its own single-token chain bit for bit (K_A's multi-token instances)."""
    torch = _torch()
    H = 2048
    layers, norms, keep = _q8_chain(kernels, 2, H, 512, 256, 8, 5300 + T)
    xs = torch.empty((T, H), dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(xs, 5400 + T, 1.0) == 0
    resid = xs.clone()
    work = torch.empty_like(xs)
    assert kernels.moe_decode_tokens(layers, norms, 1e-6, T, xs, resid, work) == 0
    kernels.sync()
    got = host(resid)
    for t in range(T):
        r1 = xs[t].clone()
        w1 = torch.empty(H, dtype=torch.float32, device="cuda")
        assert kernels.moe_decode_layers(layers, norms, 1e-6, xs[t].contiguous(), r1, w1) == 0
        kernels.sync()
        assert np.array_equal(got[t].view(np.uint32), host(r1).view(np.uint32)), f"token {t}"


def test_q8_noalloc_chain_matches_handle_chain(kernels):
    import streamoe_amd as sa

    torch = _torch()
    H = 2048
    layers, norms, keep = _q8_chain(kernels, 3, H, 512, 256, 8, 5500)
    x0 = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(x0, 5501, 1.0) == 0
    r_h, w_h = x0.clone(), torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_layers(layers, norms, 1e-6, x0, r_h, w_h) == 0
    kernels.sync()
    r_n = x0.clone()
    n = len(layers)
    arr = (sa._abi.Layer * n)(*layers)
    nw = (C.c_void_p * n)(*[t.data_ptr() for t in norms])
    stream = torch.cuda.current_stream().cuda_stream
    rc = sa._lib.smoe_moe_decode_layers_noalloc(C.c_void_p(stream), arr, n, nw, C.c_float(1e-6),
                                                C.c_void_p(x0.data_ptr()), C.c_void_p(r_n.data_ptr()))
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(host(r_n).view(np.uint32), host(r_h).view(np.uint32))


def test_q8_layer_argument_errors(kernels):
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    H, I, E, k = 2048, 512, 64, 4
    L, d, keep = _layer(kernels, H, I, E, k, 77)
    x, h_mid = _inputs(kernels, H, 77)
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    lay = sa.ExpertLayout(H, I, 4, 64)
    rq = qweights(*d["router_q8"][:3], 64, 8)
    rw = torch.zeros((E, H), dtype=torch.float32, device="cuda")
    g = torch.zeros(H, dtype=torch.float32, device="cuda")
    gq = qweights(*d["gate_q8"][:3], 64, 8)
    both = kernels.layer(lay, d["arena"], d["stride"], E, k, True, rw, d["shared"], None, router_q=rq)
    assert kernels.moe_decode_layer(both, x, h_mid, out) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    neither = kernels.layer(lay, d["arena"], d["stride"], E, k, True, None, d["shared"], None)
    assert kernels.moe_decode_layer(neither, x, h_mid, out) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    two_gates = kernels.layer(lay, d["arena"], d["stride"], E, k, True, None, d["shared"], g, router_q=rq,
                              shared_gate_q=gq)
    assert kernels.moe_decode_layer(two_gates, x, h_mid, out) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    r4 = sa.QuantWeights(rq.buffer, rq.packed_offset, rq.scales_offset, rq.biases_offset, 64, 4)
    bad_bits = kernels.layer(lay, d["arena"], d["stride"], E, k, True, None, d["shared"], None, router_q=r4)
    assert kernels.moe_decode_layer(bad_bits, x, h_mid, out) == _abi.CODES["SMOE_ERR_UNSUPPORTED_BITS"]
    r_mis = sa.QuantWeights(rq.buffer, rq.packed_offset + 4, rq.scales_offset, rq.biases_offset, 64, 8)
    mis = kernels.layer(lay, d["arena"], d["stride"], E, k, True, None, d["shared"], None, router_q=r_mis)
    assert kernels.moe_decode_layer(mis, x, h_mid, out) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    torch.cuda.synchronize()
