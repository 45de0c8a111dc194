"""The oracle's 8-bit affine matvec (dequant_matvec_8bit_gs_cpu,
cpu_matvec.rs:205-283) and the 8-bit router / shared gate of its decode
layer (the A3B `mlp.gate.weight` / `mlp.shared_expert_gate.weight`,
linear_attn_forward.rs:1300-1301), pinned on the CPU by one-hot byte-order
checks, closed forms, a float64 brute force and the exact equivalence with
the f32 router when every dequantized weight is exact."""
import numpy as np
import pytest

import oracle
from helpers import bf16, expert_f64, gen_expert_blob, gen_quant_matrix, rel_err


def _dequant_f64(q, s, b, group):
    return (q.astype(np.float64) * np.repeat(oracle.bf16_to_f32(s).astype(np.float64), group, 1) +
            np.repeat(oracle.bf16_to_f32(b).astype(np.float64), group, 1))


def test_q8_byte_order_one_hot():
    """Code byte n of u32 word i weights input 4 i + n: a single code 1 at
    (row r, input j) with scale 1 and bias 0 returns x[j] in row r only (a
    reversed or word-transposed byte order picks another input)."""
    O, I, G = 3, 128, 64
    x = np.arange(1, I + 1, dtype=np.float32)
    s = np.full((O, I // G), bf16(1.0), np.uint16)
    b = np.zeros((O, I // G), np.uint16)
    for r, j in ((0, 0), (1, 5), (2, 127), (1, 66)):
        q = np.zeros((O, I), np.uint8)
        q[r, j] = 1
        rc, y = oracle.dequant_matvec_8bit_gs(q, s, b, I, O, G, x)
        assert rc == 0
        want = np.zeros(O, np.float32)
        want[r] = x[j]
        assert np.array_equal(y, want), (r, j, y)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_q8_dequant_rows(group):
    """orc_dequant_8bit: each weight fma(q, s, b) with one rounding. Pinned
    two ways: column j equals the matvec against the unit vector e_j (whose
    byte order the one-hot test fixes), and every weight equals q s + b
    formed exactly in float64 (q s has at most 16 significant bits and the
    exponents here are close, so the sum is exact) rounded once to f32."""
    O, I = 5, 256
    rng = np.random.default_rng(group)
    q, s, b = gen_quant_matrix(rng, O, I, group, 8)
    w = oracle.dequant_8bit(q, s, b, I, O, group)
    assert w.shape == (O, I) and w.dtype == np.float32
    assert np.array_equal(w, _dequant_f64(q, s, b, group).astype(np.float32))
    for j in (0, 3, 4, group - 1, group, I - 1):
        e = np.zeros(I, np.float32)
        e[j] = 1.0
        rc, y = oracle.dequant_matvec_8bit_gs(q, s, b, I, O, group, e)
        assert rc == 0
        assert np.array_equal(y.view(np.uint32), np.ascontiguousarray(w[:, j]).view(np.uint32)), j


def test_q8_closed_form_constant_codes():
    """Codes c everywhere, per-group scale s_g and bias b_g: row = sum_g
    (c s_g + b_g) sum_{j in g} x_j, exact with small integers and powers of
    two (every product and partial sum is representable)."""
    O, I, G = 2, 256, 32
    rng = np.random.default_rng(3)
    x = rng.integers(-8, 9, I).astype(np.float32)
    sv = 2.0 ** rng.integers(-4, 2, (O, I // G))
    bv = rng.integers(-3, 4, (O, I // G)).astype(np.float64)
    for c in (0, 1, 200, 255):
        q = np.full((O, I), c, np.uint8)
        rc, y = oracle.dequant_matvec_8bit_gs(q, bf16(sv), bf16(bv), I, O, G, x)
        assert rc == 0
        xs = x.astype(np.float64).reshape(I // G, G).sum(1)
        want = ((c * sv + bv) * xs[None, :]).sum(1)
        assert np.array_equal(y.astype(np.float64), want), (c, y, want)


def test_q8_bias_only_and_zero_input():
    O, I, G = 4, 192, 64
    rng = np.random.default_rng(4)
    q, s, b = gen_quant_matrix(rng, O, I, G, 8)
    rc, y = oracle.dequant_matvec_8bit_gs(q, s, b, I, O, G, np.zeros(I, np.float32))
    assert rc == 0 and np.all(y == 0)
    x = np.ones(I, np.float32)
    rc, y = oracle.dequant_matvec_8bit_gs(np.zeros_like(q), s, b, I, O, G, x)
    want = oracle.bf16_to_f32(b).astype(np.float64).sum(1) * G
    assert rel_err(y, want) < 1e-6


@pytest.mark.parametrize("O,I,G", [(8, 2048, 64), (5, 4096, 64), (7, 512, 32), (3, 1024, 128)])
def test_q8_matvec_vs_f64(O, I, G):
    rng = np.random.default_rng(O * I + G)
    q, s, b = gen_quant_matrix(rng, O, I, G, 8, ssig=2e-4, bsig=0.02)
    x = rng.standard_normal(I).astype(np.float32)
    rc, y = oracle.dequant_matvec_8bit_gs(q, s, b, I, O, G, x)
    assert rc == 0
    W = _dequant_f64(q, s, b, G)
    want = W @ x.astype(np.float64)
    # Sequential f32 fma chains: error well under in_dim * 2^-24 * sum |w x|.
    bound = I * 2.0 ** -24 * (np.abs(W) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - want) <= bound), np.max(np.abs(y - want) / bound)


def test_q8_sequential_order():
    """The row sum is one fma chain in input order: inputs that cancel
    only in that order (1e8, 1, -1e8 ...) give what the chain gives."""
    I, G = 64, 64
    q = np.zeros((1, I), np.uint8)
    q[0, :4] = 1
    x = np.zeros(I, np.float32)
    x[:4] = [1e8, 1.0, -1e8, 1.0]
    rc, y = oracle.dequant_matvec_8bit_gs(q, np.full((1, 1), bf16(1.0), np.uint16), np.zeros((1, 1), np.uint16),
                                          I, 1, G, x)
    acc = np.float32(0)
    for v in x[:4]:
        acc = np.float32(acc + v)
    assert y[0] == acc == 1.0


@pytest.mark.parametrize("group,in_dim", [(0, 64), (6, 96), (64, 96)])
def test_q8_group_errors(group, in_dim):
    rc, _ = oracle.dequant_matvec_8bit_gs(np.zeros((1, 96), np.uint8), np.zeros(96, np.uint16),
                                          np.zeros(96, np.uint16), in_dim, 1, group, np.zeros(96, np.float32))
    assert rc != 0


def _exact_q8(rng, rows, H, G):
    """8-bit rows whose dequantized weights are exact in f32: scale 2^-10,
    bias -k 2^-10 (k a small integer), so fma(q, s, b) = (q - k) 2^-10."""
    q = rng.integers(0, 256, (rows, H), dtype=np.uint8)
    s = np.full((rows, H // G), bf16(2.0 ** -10), np.uint16)
    kb = rng.integers(100, 156, (rows, H // G))
    b = bf16(-kb * 2.0 ** -10)
    w = ((q.astype(np.float64) - np.repeat(kb, G, 1)) * 2.0 ** -10).astype(np.float32)
    return (q, s, b, G), w


def test_decode_layer_q8_router_equals_f32_router_of_its_weights():
    """With every dequantized weight exact, the 8-bit router and shared gate
    give bit for bit the layer of the f32 router and gate holding those
    weights (the same fma chain in the same order): the 8-bit rows are
    wired into the layer with the right row stride and group indexing."""
    rng = np.random.default_rng(22)
    H, I, E, k, G = 256, 64, 16, 4, 64
    blobs = [gen_expert_blob(rng, H, I, G, 4) for _ in range(E)]
    stride = blobs[0].size
    experts = np.concatenate(blobs)
    shared = gen_expert_blob(rng, H, I, G, 4)
    rq, rw = _exact_q8(rng, E, H, G)
    gq, gw = _exact_q8(rng, 1, H, G)
    x = (rng.standard_normal(H) * 0.5).astype(np.float32)
    h_mid = rng.standard_normal(H).astype(np.float32)
    a = oracle.moe_decode_layer(experts, stride, H, I, E, k, G, 4, True, None, x, h_mid, shared, None,
                                router_q8=rq, gate_q8=gq)
    b = oracle.moe_decode_layer(experts, stride, H, I, E, k, G, 4, True, rw, x, h_mid, shared, gw[0])
    for u, v in zip(a, b):
        assert np.array_equal(u, v)


def test_decode_layer_q8_router_vs_f64():
    """A generic 8-bit router (A3B-like scales): logits within the fma-chain
    bound of the float64 dequantized router, and the layer within 1e-4 of a
    float64 brute force with the same picks."""
    import math

    rng = np.random.default_rng(23)
    H, I, E, k, G = 512, 64, 32, 4, 64
    blobs = [gen_expert_blob(rng, H, I, G, 4) for _ in range(E)]
    stride = blobs[0].size
    experts = np.concatenate(blobs)
    shared = gen_expert_blob(rng, H, I, G, 4)
    rq = gen_quant_matrix(rng, E, H, G, 8, ssig=2e-4, bsig=0.02) + (G,)
    gq = gen_quant_matrix(rng, 1, H, G, 8, ssig=2e-4, bsig=0.02) + (G,)
    x = rng.standard_normal(H).astype(np.float32)
    h_mid = rng.standard_normal(H).astype(np.float32)
    out, idx, w, logits = oracle.moe_decode_layer(experts, stride, H, I, E, k, G, 4, True, None, x, h_mid,
                                                  shared, None, router_q8=rq, gate_q8=gq)
    W = _dequant_f64(rq[0], rq[1], rq[2], G)
    want_lg = W @ x.astype(np.float64)
    assert np.all(np.abs(logits - want_lg) <= H * 2.0 ** -24 * (np.abs(W) @ np.abs(x.astype(np.float64))))
    _, idx2, w2 = oracle.router(logits, k, True)
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    want = h_mid.astype(np.float64)
    for s_, e in enumerate(idx):
        want = want + float(w[s_]) * expert_f64(blobs[e], H, I, G, x)
    g = float(_dequant_f64(gq[0], gq[1], gq[2], G)[0] @ x.astype(np.float64))
    want = want + expert_f64(shared, H, I, G, x) / (1.0 + math.exp(-g))
    assert rel_err(out, want) < 1e-4
