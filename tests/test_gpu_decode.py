"""GPU parity of the decode path against the CPU oracle, through the C ABI.

Bars: dequantized values and top-k indices
bit-exact; matvec / expert outputs within max relative error 1e-3 under
fp32 accumulation, measured as max|got - want| / max|want| (the
reference's metric, crates/streammoe/tests/group32_kernels.rs:141-150).
"""
import numpy as np
import pytest

import oracle
from helpers import bf16, expert_pair, gen_expert_blob, gen_quant_matrix, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max relative error, fp32 accumulation


def _torch():
    import torch

    return torch


def dev(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy()


def pack_matrix(codes, scales, biases):
    """One device buffer [codes | scales | biases] with 256-byte aligned regions."""
    def pad(n):
        return (n + 255) // 256 * 256

    c = codes.ravel().view(np.uint8)
    s = scales.ravel().view(np.uint8)
    b = biases.ravel().view(np.uint8)
    so = pad(c.size)
    bo = so + pad(s.size)
    buf = np.zeros(bo + pad(b.size), np.uint8)
    buf[:c.size] = c
    buf[so:so + s.size] = s
    buf[bo:bo + b.size] = b
    return dev(buf), 0, so, bo


def qweights(codes, scales, biases, group, bits):
    import streamoe_amd as sa

    buf, po, so, bo = pack_matrix(codes, scales, biases)
    return sa.QuantWeights(buf, po, so, bo, group, bits)


def oracle_matvec(codes, scales, biases, in_dim, out_dim, group, bits, x):
    if bits == 3:
        words = np.zeros(out_dim * in_dim // 8, np.uint32)
        c3 = codes.reshape(-1, 3).astype(np.uint32)
        p = c3[:, 0] | (c3[:, 1] << 8) | (c3[:, 2] << 16)
        for i in range(8):
            words |= ((p >> np.uint32(3 * i)) & np.uint32(7)) << np.uint32(4 * i)
        packed = words
    else:
        packed = codes.view(np.uint32)
    rc, y = oracle.dequant_matvec_4bit_gs(packed, scales, biases, in_dim, out_dim, group, x)
    assert rc == 0
    return y, packed


# --- qmv --------------------------------------------------------------------------

@pytest.mark.parametrize("out_dim,in_dim,group,bits", [
    (512, 2048, 64, 4), (2048, 512, 64, 4), (1000, 1024, 32, 4), (77, 4096, 128, 4),
    (512, 2048, 64, 3), (2048, 512, 64, 3), (333, 8192, 64, 4), (5, 2048, 64, 4),
    # Input widths that are not a power of two times 32 (padded instances):
    # the reference variants' 2560, 640 and 7168, a 256-wide test model,
    # three chunks.
    (1000, 2560, 64, 4), (300, 640, 32, 3), (513, 7168, 64, 4), (129, 7168, 128, 3), (77, 256, 64, 4),
    (64, 96, 32, 4),
])
def test_qmv_matches_oracle(kernels, out_dim, in_dim, group, bits):
    rng = np.random.default_rng(out_dim * 7 + in_dim + bits)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, group, bits)
    x = rng.standard_normal(in_dim).astype(np.float32)
    w = qweights(codes, s, b, group, bits)
    torch = _torch()
    y = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    assert kernels.qmv(w, dev(x), y, out_dim, in_dim) == 0
    want, _ = oracle_matvec(codes, s, b, in_dim, out_dim, group, bits, x)
    err = rel_err(host(y), want)
    print(f"qmv {out_dim}x{in_dim} g{group} {bits}-bit rel_err={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("out_dim,in_dim,group,bits", [
    (40000, 2048, 64, 4), (30001, 2048, 32, 3), (16391, 4096, 128, 4), (20000, 4096, 64, 3),
    (50003, 2048, 128, 4), (16384, 2048, 64, 4),
])
def test_qmv_large_ragged_row_slices(kernels, out_dim, in_dim, group, bits):
    """Large matrices with ragged row counts (the persistent grid's last
    steps clamp their rows): within 1e-3 of the oracle, and every row's
    result independent of the launch that computes it: the same rows as
    slices of at most 8000 rows (other grids, other wave-to-row mappings)
    give the same bits."""
    import streamoe_amd as sa

    rng = np.random.default_rng(out_dim + in_dim + group + bits)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, group, bits)
    x = rng.standard_normal(in_dim).astype(np.float32)
    w = qweights(codes, s, b, group, bits)
    torch = _torch()
    xd = dev(x)
    y = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    assert kernels.qmv(w, xd, y, out_dim, in_dim) == 0
    want, _ = oracle_matvec(codes, s, b, in_dim, out_dim, group, bits, x)
    got = host(y)
    err = rel_err(got, want)
    print(f"qmv {out_dim}x{in_dim} g{group} {bits}-bit rel_err={err:.3e}")
    assert err <= TOL
    rb, sb = in_dim * bits // 8, in_dim // group * 2
    ys = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    for r0 in range(0, out_dim, 8000):
        n = min(8000, out_dim - r0)
        ws = sa.QuantWeights(w.buffer, w.packed_offset + r0 * rb, w.scales_offset + r0 * sb,
                             w.biases_offset + r0 * sb, group, bits)
        assert kernels.qmv(ws, xd, ys[r0:r0 + n], n, in_dim) == 0
    assert np.array_equal(host(ys).view(np.uint32), got.view(np.uint32))


def test_lm_head_qwen3_shape_and_argmax(kernels):
    """Config 1: 151,936 x 2048 4-bit g64 LM head; greedy argmax bit-exact."""
    V, H, G = 151936, 2048, 64
    rng = np.random.default_rng(0xC1)
    codes, s, b = gen_quant_matrix(rng, V, H, G, 4)
    x = rng.standard_normal(H).astype(np.float32)
    w = qweights(codes, s, b, G, 4)
    torch = _torch()
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv(w, dev(x), y, V, H) == 0
    assert kernels.argmax(y, V, am) == 0
    want, _ = oracle_matvec(codes, s, b, H, V, G, 4, x)
    got = host(y)
    err = rel_err(got, want)
    top2 = np.sort(want)[-2:]
    print(f"lm_head rel_err={err:.3e} argmax gpu={int(host(am)[0])} cpu={oracle.argmax(want)} "
          f"gap={top2[1] - top2[0]:.3e} max|d|={np.max(np.abs(got - want)):.3e}")
    assert err <= TOL
    # The gap between the top two logits exceeds twice the largest deviation,
    # so the argmax cannot flip: the certified comparison is exact equality.
    assert top2[1] - top2[0] > 2 * np.max(np.abs(got - want))
    assert int(host(am)[0]) == oracle.argmax(want)


@pytest.mark.parametrize("n", [1, 3, 4, 255, 1023, 4097, 151936, 151939])
def test_argmax_first_index_on_ties(kernels, n):
    """Argmax equals numpy's (first maximal index) with the maximum planted
    several times, including in the ragged tail and across slice borders."""
    torch = _torch()
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    peak = np.float32(10.0)
    for pos in sorted({n - 1, n // 2, (n * 3) // 4, min(n - 1, 600)}, reverse=True):
        v[pos] = peak
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.argmax(dev(v), n, out) == 0
    assert int(host(out)[0]) == int(np.argmax(v)) == oracle.argmax(v)


def _ref_argmax(v):
    """The reference's greedy pick (engine_tests.rs:105-107): fold from
    index 0, replace only when strictly greater."""
    best = 0
    for i in range(1, len(v)):
        if v[i] > v[best]:
            best = i
    return best


@pytest.mark.parametrize("case", ["nan-first", "nan-inside", "all-nan", "nan-first-of-one"])
def test_argmax_nan_like_the_reference(kernels, case):
    """NaN never wins, and a NaN at index 0 is never replaced (the
    reference's scan keeps index 0): smoe_argmax over 4097 values (slice
    borders included) and the oracle agree with the restated scan."""
    torch = _torch()
    rng = np.random.default_rng(77)
    n = 1 if case == "nan-first-of-one" else 4097
    v = rng.standard_normal(n).astype(np.float32)
    if case in ("nan-first", "nan-first-of-one"):
        v[0] = np.nan
    elif case == "nan-inside":
        v[[5, 1000, 2100, 4096]] = np.nan
        v[3000] = 9.0
    else:
        v[:] = np.nan
    want = _ref_argmax(v)
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.argmax(dev(v), n, out) == 0
    assert int(host(out)[0]) == want == oracle.argmax(v)


@pytest.mark.parametrize("out_dim", [9000, 20000])
def test_qmv_argmax_nan_first_row(kernels, out_dim):
    """smoe_qmv_argmax when row 0's scales are NaN (y[0] = NaN): index 0, as
    the reference's scan over the logits gives."""
    torch = _torch()
    in_dim = 2048
    rng = np.random.default_rng(9)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, 64, 4)
    s[0, :] = 0x7FC0  # bf16 NaN
    x = rng.standard_normal(in_dim).astype(np.float32)
    w = qweights(codes, s, b, 64, 4)
    y = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    i = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv_argmax(w, dev(x), y, out_dim, in_dim, i) == 0
    got = host(y)
    assert np.isnan(got[0]) and np.all(np.isfinite(got[1:]))
    assert int(host(i)[0]) == 0 == _ref_argmax(got) == oracle.argmax(got)


@pytest.mark.parametrize("out_dim,in_dim,bits", [(151936, 2048, 4), (50000, 1024, 4), (9000, 2048, 3),
                                                 (77, 512, 4), (40000, 2048, 3), (20000, 4096, 4)])
def test_qmv_argmax_fused(kernels, out_dim, in_dim, bits):
    """smoe_qmv_argmax: y identical to smoe_qmv, index = numpy's first
    maximal index of y, with the maximum planted on several rows (identical
    weight rows give bit-identical sums) across waves and steps."""
    torch = _torch()
    rng = np.random.default_rng(out_dim + bits)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, 64, bits)
    # Plant one large row and copy it over later rows: equal maxima.
    s[:, :] = s // 2  # keep ordinary rows small
    big = out_dim // 3
    s[big] = (np.abs(s[big].view(np.int16)).astype(np.uint16) | 0x3F00).astype(np.uint16) & 0x7FFF
    for r in sorted({big, out_dim - 1, (2 * out_dim) // 3, min(out_dim - 1, big + 5)}):
        codes[r], s[r], b[r] = codes[big], s[big], b[big]
    x = np.abs(rng.standard_normal(in_dim)).astype(np.float32)
    w = qweights(codes, s, b, 64, bits)
    y1 = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    y2 = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    i1 = torch.empty(1, dtype=torch.int32, device="cuda")
    i2 = torch.empty(1, dtype=torch.int32, device="cuda")
    assert kernels.qmv(w, dev(x), y1, out_dim, in_dim) == 0
    assert kernels.argmax(y1, out_dim, i1) == 0
    assert kernels.qmv_argmax(w, dev(x), y2, out_dim, in_dim, i2) == 0
    got = host(y2)
    assert np.array_equal(got.view(np.uint32), host(y1).view(np.uint32))
    assert int(host(i2)[0]) == int(host(i1)[0]) == int(np.argmax(got))
    assert int(np.argmax(got)) == min(big, out_dim - 1)


def test_qmv_argmax_back_to_back(kernels):
    """Calls of different grid sizes in a row (full LM-head grid, a
    one-block grid, a mid-size 3-bit grid, the full grid again) each give
    numpy's first maximal index of their own y: no partial left by a larger
    earlier call enters a later call's merge."""
    torch = _torch()
    cases = [(151936, 2048, 4), (77, 512, 4), (9000, 2048, 3), (151936, 2048, 4), (300, 1024, 3)]
    mats = {}
    for n, (out_dim, in_dim, bits) in enumerate(cases):
        rng = np.random.default_rng(0xA0 + n)
        if (out_dim, in_dim, bits) not in mats:
            codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, 64, bits)
            mats[(out_dim, in_dim, bits)] = qweights(codes, s, b, 64, bits)
        w = mats[(out_dim, in_dim, bits)]
        x = rng.standard_normal(in_dim).astype(np.float32)
        y = torch.empty(out_dim, dtype=torch.float32, device="cuda")
        i = torch.full((1,), -7, dtype=torch.int32, device="cuda")
        assert kernels.qmv_argmax(w, dev(x), y, out_dim, in_dim, i) == 0
        got = host(y)
        assert int(host(i)[0]) == int(np.argmax(got)), (n, out_dim, in_dim, bits)


# --- dequant (bit-exact) --------------------------------------------------------------

@pytest.mark.parametrize("bits,group", [(4, 64), (3, 64), (4, 32), (3, 128)])
def test_dequant_bit_exact(kernels, bits, group):
    rng = np.random.default_rng(bits * 100 + group)
    out_dim, in_dim = 64, 1024
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, group, bits)
    w = qweights(codes, s, b, group, bits)
    torch = _torch()
    out = torch.empty((out_dim - 3, in_dim), dtype=torch.float32, device="cuda")
    assert kernels.dequant(w, in_dim, 3, out_dim - 3, out) == 0
    _, packed = oracle_matvec(codes, s, b, in_dim, out_dim, group, bits, np.zeros(in_dim, np.float32))
    want = oracle.dequant_4bit(packed, s, b, in_dim, out_dim, group)[3:]
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


# --- router -----------------------------------------------------------------------------

def test_topk_bit_exact_on_identical_scores(kernels):
    """Given the same scores the device top-k reproduces the reference's
    slot order and values bit for bit, including ties."""
    torch = _torch()
    cases = [
        ([0.1, 0.5, 0.3, 0.9, 0.2], 3),
        ([1.0, 1.0, 1.0, 1.0], 2),
        ([2.0, 1.0, 1.0, 3.0], 2),
        ([1.0, 1.0, 2.0], 2),
        ([5.0, 4.0, 3.0, 2.0, 1.0], 5),
        (list(np.arange(300, dtype=np.float32)), 16),        # every index is an event
        (list(np.arange(300, dtype=np.float32)[::-1]), 16),  # no events after the first k
        ([-1e31, -2e31, 5.0, -1e31], 2),                     # scores below the -1e30 start
    ]
    rng = np.random.default_rng(3)
    for n in (64, 256, 1024):
        v = rng.standard_normal(n).astype(np.float32)
        v[rng.integers(0, n, n // 4)] = 0.25  # many exact ties
        cases.append((list(v), 8))
    for scores, k in cases:
        sc = np.array(scores, np.float32)
        idx = torch.empty(k, dtype=torch.int32, device="cuda")
        val = torch.empty(k, dtype=torch.float32, device="cuda")
        assert kernels.topk(dev(sc), 1, sc.size, k, idx, val) == 0
        rc, widx, wval = oracle.topk(sc, k)
        assert rc == 0
        assert np.array_equal(host(idx), widx), (scores[:8], k)
        assert np.array_equal(host(val).view(np.uint32), wval.view(np.uint32))


@pytest.mark.parametrize("n_tokens,E,k,normalize", [(1, 256, 8, True), (8, 256, 8, True), (64, 64, 8, False),
                                                      (32, 512, 10, True), (4, 1024, 16, True)])
def test_router_matches_oracle(kernels, n_tokens, E, k, normalize):
    """f32 router GEMV + softmax + top-k (+ renorm) per token. Index sets
    and slot order equal the oracle whenever the k-th / (k+1)-th probability
    gap exceeds the logit deviation (reported); weights within 1e-5."""
    torch = _torch()
    H = 2048
    rng = np.random.default_rng(E * 31 + n_tokens)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    X = rng.standard_normal((n_tokens, H)).astype(np.float32)
    idx = torch.empty((n_tokens, k), dtype=torch.int32, device="cuda")
    w = torch.empty((n_tokens, k), dtype=torch.float32, device="cuda")
    logits = torch.empty((n_tokens, E), dtype=torch.float32, device="cuda")
    assert kernels.router(dev(W), dev(X), n_tokens, E, H, k, normalize, idx, w, logits) == 0
    gi, gw, gl = host(idx), host(w), host(logits)
    for t in range(n_tokens):
        lg = oracle.f32_matvec(W, X[t])
        assert rel_err(gl[t], lg) < 1e-5
        probs = oracle.softmax(lg)
        srt = np.sort(probs)[::-1]
        gap = srt[k - 1] - srt[k]
        _, widx, ww = oracle.router(lg, k, normalize)
        if gap > 1e-5 * srt[0]:
            assert np.array_equal(gi[t], widx), (t, gap)
            assert np.max(np.abs(gw[t] - ww)) <= 1e-5 * np.max(np.abs(ww))
        print(f"router t={t} gap={gap:.3e} match={np.array_equal(gi[t], widx)}")


def test_softmax_topk_from_oracle_logits(kernels):
    """Same logits on both sides: the device softmax differs from libm's
    by ULPs only, so indices match and weights agree to 1e-6."""
    torch = _torch()
    rng = np.random.default_rng(17)
    E, k, T = 256, 8, 16
    L = rng.standard_normal((T, E)).astype(np.float32)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    assert kernels.softmax_topk(dev(L), T, E, k, True, idx, w) == 0
    gi, gw = host(idx), host(w)
    for t in range(T):
        _, widx, ww = oracle.router(L[t], k, True)
        assert np.array_equal(gi[t], widx)
        assert np.max(np.abs(gw[t] - ww)) <= 1e-6


# --- K-expert decode (bindings API) ----------------------------------------------------

def _experts_case(kernels, H, I, k, bits, with_shared, seed):
    torch = _torch()
    rng = np.random.default_rng(seed)
    blobs = [gen_expert_blob(rng, H, I, 64, bits) for _ in range(k)]
    arena = dev(np.concatenate(blobs))
    import streamoe_amd as sa

    lay = sa.ExpertLayout(H, I, bits, 64)
    x = rng.standard_normal(H).astype(np.float32)
    h_mid = rng.standard_normal(H).astype(np.float32)
    shared = (0.1 * rng.standard_normal(H)).astype(np.float32) if with_shared else None
    wts = (rng.random(k) + 0.1).astype(np.float32)
    score = 0.3
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    rc = kernels.experts_decode(lay, [(arena, s * lay.expert_size) for s in range(k)], list(wts), dev(x),
                                dev(h_mid), None if shared is None else dev(shared), score, out)
    assert rc == 0
    outs = np.stack([oracle.expert_swiglu(b, bits, H, I, 64, x) for b in blobs])
    want = oracle.combine(outs, wts, h_mid, shared, score if with_shared else float("nan"))
    return host(out), want, h_mid


@pytest.mark.parametrize("H,I,k,bits,shared", [
    (2048, 512, 8, 4, True),    # Qwen3.6-A3B
    (2048, 1024, 8, 4, False),  # OLMoE
    (2048, 512, 8, 3, True),    # packed 3-bit
    (2048, 512, 16, 4, True),   # MAX_K
    (2048, 512, 1, 4, False),
    (4096, 1024, 10, 4, True),
    (1024, 256, 4, 3, False),
    # The other reference variants (variants.rs): Qwen3.8-Flash-Next
    # (2560 x 640, top-10), Cogito-V2 (7168 x 2048), the tiny test models.
    (2560, 640, 10, 4, True),
    (2560, 640, 10, 3, True),
    (7168, 2048, 8, 4, True),
    (256, 64, 3, 4, True),
    (512, 128, 10, 3, True),
])
def test_experts_decode_matches_oracle(kernels, H, I, k, bits, shared):
    if H > 4096:
        kernels.reserve(H, max(I, 2048), 1024)
    got, want, h_mid = _experts_case(kernels, H, I, k, bits, shared, seed=H + I + k + bits)
    # The expert outputs are small next to h_mid: the MoE part (output -
    # h_mid) is compared on its own as well.
    err = rel_err(got, want)
    moe_err = rel_err(got - h_mid, want - h_mid)
    print(f"experts H={H} I={I} k={k} {bits}-bit rel_err={err:.3e} MoE part {moe_err:.3e}")
    assert err <= TOL and moe_err <= TOL


def test_packed_3bit_bit_identical_to_nibbles(kernels):
    """tests/packed_3bit.rs:65-106: the K-expert decode on packed 3-bit
    equals the same codes stored as 4-bit nibbles, bit for bit (seed
    0x3B17_DEC0_0001, A3B shapes, k = 8)."""
    import streamoe_amd as sa

    rng = oracle.XorShift64s(0x3B17DEC00001)
    k = 8
    nib, packed = [], []
    for _ in range(k):
        a, b = expert_pair(rng)
        nib.append(a)
        packed.append(b)
    h_post = rng.unit(2048)
    h_mid = rng.unit(2048)
    shared_out = (np.float32(0.1) * rng.unit(2048)).astype(np.float32)
    weights = [np.float32(1.0) / np.float32(i + 2) for i in range(k)]
    payload = sa.ExpertPayload(h_post, h_mid, shared_out, weights, 0.3)
    a = sa.gpu_batched_experts_forward(kernels, sa.ExpertLayout(2048, 512, 4, 64), k, np.concatenate(nib), payload)
    b = sa.gpu_batched_experts_forward(kernels, sa.ExpertLayout(2048, 512, 3, 64), k, np.concatenate(packed), payload)
    assert np.any(a != 0) and np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # And both match the CPU path.
    outs = np.stack([oracle.expert_swiglu(n, 4, 2048, 512, 64, h_post) for n in nib])
    want = oracle.combine(outs, np.array(weights, np.float32), h_mid, shared_out, 0.3)
    assert rel_err(a, want) <= TOL


def test_experts_decode_argument_errors(kernels):
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    buf = torch.zeros(4 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(2048, dtype=torch.float32, device="cuda")
    lay = sa.ExpertLayout(2048, 512, 4, 64)
    ok = [(buf, 0)]
    assert kernels.experts_decode(lay, [], [], x, x, None, 0.0, x) == _abi.CODES["SMOE_ERR_BAD_K"]
    assert kernels.experts_decode(lay, ok * 17, [1.0] * 17, x, x, None, 0.0, x) == _abi.CODES["SMOE_ERR_BAD_K"]
    assert kernels.experts_decode(lay, [(buf, 8)], [1.0], x, x, None, 0.0, x) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    assert kernels.experts_decode(sa.ExpertLayout(2048, 512, 5, 64), ok, [1.0], x, x, None, 0.0, x) == \
        _abi.CODES["SMOE_ERR_UNSUPPORTED_BITS"]
    assert kernels.experts_decode(sa.ExpertLayout(2048, 512, 4, 48), ok, [1.0], x, x, None, 0.0, x) == \
        _abi.CODES["SMOE_ERR_UNSUPPORTED_GROUP"]
    assert kernels.experts_decode(sa.ExpertLayout(2048, 500, 4, 64), ok, [1.0], x, x, None, 0.0, x) == \
        _abi.CODES["SMOE_ERR_IN_DIM_NOT_MULTIPLE"]
    w = sa.QuantWeights(buf, 0, 4096, 8192, 64, 4)
    assert kernels.qmv(w, x, x, 10, 2000) == _abi.CODES["SMOE_ERR_IN_DIM_NOT_MULTIPLE"]
    w = sa.QuantWeights(buf, 4, 4096, 8192, 64, 4)
    assert kernels.qmv(w, x, x, 10, 2048) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    idx = torch.zeros(32, dtype=torch.int32, device="cuda")
    assert kernels.topk(x, 1, 8, 9, idx, x) == _abi.CODES["SMOE_ERR_BAD_K"]
    torch.cuda.synchronize()


# --- one resident layer with device routing ---------------------------------------------

def _layer_case(kernels, H, I, E, k, bits, normalize, shared, seed):
    """Returns (gpu hidden, gpu idx, gpu w, oracle hidden, oracle idx, oracle w, gap)."""
    import streamoe_amd as sa

    torch = _torch()
    lay = sa.ExpertLayout(H, I, bits, 64)
    stride = lay.expert_size
    arena = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, stride, lay, seed) == 0
    router_w = torch.empty((E, H), dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(router_w, seed + 1, 0.02) == 0
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(x, seed + 2, 1.0) == 0
    h_mid = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(h_mid, seed + 3, 1.0) == 0
    sh_blob = sh_gate = None
    if shared:
        slay = sa.ExpertLayout(H, I, 4, 64)
        sh_blob = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(sh_blob, 1, slay.expert_size, slay, seed + 4) == 0
        if shared != "ungated":
            sh_gate = torch.empty(H, dtype=torch.float32, device="cuda")
            assert kernels.synth_normal_f32(sh_gate, seed + 5, 0.02) == 0
    L = kernels.layer(lay, arena, stride, E, k, normalize, router_w, sh_blob, sh_gate)
    out = torch.empty(H, dtype=torch.float32, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    w = torch.empty(k, dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_layer(L, x, h_mid, out, idx, w) == 0
    experts_h = host(arena)
    oh, oi, ow, logits = oracle.moe_decode_layer(experts_h, stride, H, I, E, k, 64, bits, normalize, host(router_w),
                                                 host(x), host(h_mid), None if sh_blob is None else host(sh_blob),
                                                 None if sh_gate is None else host(sh_gate))
    p = np.sort(oracle.softmax(logits))[::-1]
    return host(out), host(idx), host(w), oh, oi, ow, p[k - 1] - p[k]


LAYER_CASES = [
    ("olmoe", 2048, 1024, 64, 8, 4, False, False),   # config 0
    ("a3b", 2048, 512, 256, 8, 4, True, True),       # config 2
    ("a3b-3bit", 2048, 512, 256, 8, 3, True, True),  # config 3
    ("a3b-noshared", 2048, 512, 256, 8, 4, True, False),
    ("k4-e128", 2048, 512, 128, 4, 4, False, True),
    ("k16", 2048, 512, 128, 16, 4, True, True),      # beyond the persistent kernel
    ("a3b-ungated", 2048, 512, 256, 8, 4, True, "ungated"),  # shared expert added unscaled
    ("olmoe-3bit-e32", 2048, 1024, 32, 2, 3, True, False),
    ("k16-i1024", 2048, 1024, 64, 16, 4, True, True),  # down kernel: 8 rows per lane, > 64 KB LDS
    ("k10", 2048, 512, 128, 10, 4, True, True),      # the reference's other supported top-k
    ("e512-k10", 2048, 512, 512, 10, 4, True, True),  # 512 experts, top-10, shared expert
    ("e300-k8", 2048, 512, 300, 8, 4, True, False),   # 8 logits per lane, ragged last lanes
    # Hidden 4096: two 32-value chunks per lane in every wave.
    ("q397b", 4096, 1024, 512, 10, 4, True, True),    # the reference's Qwen3.5-397B-A17B layer
    ("h4096-3bit", 4096, 512, 128, 8, 3, True, "ungated"),
    ("h4096-k16-i1024", 4096, 1024, 64, 16, 4, False, True),  # down kernel: one row part, > 64 KB LDS
]

PATHS = [1, 3]
PATH_IDS = ["per-phase", "three-kernel"]


@pytest.mark.parametrize("path", PATHS, ids=PATH_IDS)
@pytest.mark.parametrize("name,H,I,E,k,bits,normalize,shared", LAYER_CASES)
def test_moe_decode_layer_matches_oracle(kernels, path, name, H, I, E, k, bits, normalize, shared):
    kernels.set_decode_path(path)
    try:
        seed = sum(map(ord, name)) * 7 + 1
        got, gi, gw, want, wi, ww, gap = _layer_case(kernels, H, I, E, k, bits, normalize, shared, seed=seed)
        kernels.sync()
        err = rel_err(got, want)
        print(f"layer {name} path={path}: idx gpu={list(gi)} cpu={list(wi)} gap={gap:.3e} rel_err={err:.3e}")
        assert np.array_equal(gi, wi)
        assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
        assert err <= TOL
    finally:
        kernels.set_decode_path(0)


OTHER_SHAPES = [
    ("flash-next", 2560, 640, 512, 10, 4, True, True),    # Qwen3.8-Flash-Next-4bit
    ("flash-next-3bit", 2560, 640, 512, 10, 3, True, True),
    ("cogito-v2", 7168, 2048, 256, 8, 4, True, True),     # DeepSeek-V3 width (routed by softmax top-k here)
    ("flash-next-tiny", 256, 64, 8, 3, 4, True, True),
    ("qwen3-next-tiny", 512, 128, 32, 10, 4, True, True),
    ("h3072", 3072, 768, 128, 8, 4, False, False),
]


@pytest.mark.parametrize("name,H,I,E,k,bits,normalize,shared", OTHER_SHAPES)
def test_decode_layer_other_shapes(kernels, name, H, I, E, k, bits, normalize, shared):
    """Shapes without a three-kernel instance take the per-phase kernels on
    the default path (padded instances for widths that are not a power of
    two times 32); forcing the three-kernel path reports them unsupported."""
    from streamoe_amd import _abi

    if H > 4096:
        kernels.reserve(H, max(I, 2048), 1024)
    kernels.set_decode_path(0)
    seed = sum(map(ord, name)) * 5 + 3
    got, gi, gw, want, wi, ww, gap = _layer_case(kernels, H, I, E, k, bits, normalize, shared, seed=seed)
    kernels.sync()
    err = rel_err(got, want)
    print(f"layer {name}: idx gpu={list(gi)} cpu={list(wi)} gap={gap:.3e} rel_err={err:.3e}")
    assert np.array_equal(gi, wi)
    assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
    assert err <= TOL
    kernels.set_decode_path(3)
    try:
        import streamoe_amd as sa

        torch = _torch()
        lay = sa.ExpertLayout(H, I, bits, 64)
        a = torch.zeros(E * lay.expert_size, dtype=torch.uint8, device="cuda")
        r = torch.zeros((E, H), dtype=torch.float32, device="cuda")
        L = kernels.layer(lay, a, lay.expert_size, E, k, normalize, r)
        x = torch.zeros(H, dtype=torch.float32, device="cuda")
        assert kernels.moe_decode_layer(L, x, x, x.clone()) == _abi.CODES["SMOE_ERR_UNSUPPORTED_SHAPE"]
    finally:
        kernels.set_decode_path(0)


def test_decode_layer_hidden_4096_default_is_three_kernel(kernels):
    """The reference's Qwen3.5-397B-A17B shape (hidden 4096, 512 experts,
    top-10, inter 1024, gated shared expert): the default path takes the
    three-kernel decode (same bits as forcing it) and agrees with the
    oracle."""
    res = {}
    try:
        for path in (0, 3):
            kernels.set_decode_path(path)
            res[path] = _layer_case(kernels, 4096, 1024, 512, 10, 4, True, True, seed=4096)
            kernels.sync()
    finally:
        kernels.set_decode_path(0)
    got, gi, gw, want, wi, ww, gap = res[0]
    assert np.array_equal(got.view(np.uint32), res[3][0].view(np.uint32))
    err = rel_err(got, want)
    print(f"hidden 4096 E=512 k=10: idx gpu={list(gi)} cpu={list(wi)} gap={gap:.3e} rel_err={err:.3e}")
    assert np.array_equal(gi, wi)
    assert np.max(np.abs(gw - ww)) <= 1e-5 * np.max(np.abs(ww))
    assert err <= TOL


def _chain(kernels, NL, E, k, bits, seed, norm_sigma=0.0, I=512, H=2048):
    """NL resident config-2-style layers (routed `bits`, 4-bit shared expert
    with gate) and per-layer bf16 RMSNorm weights 1 + N(0, norm_sigma)."""
    import streamoe_amd as sa

    torch = _torch()
    lay = sa.ExpertLayout(H, I, bits, 64)
    slay = sa.ExpertLayout(H, I, 4, 64)
    stride = lay.expert_size
    rng = np.random.default_rng(seed)
    c = dict(H=H, I=I, E=E, k=k, bits=bits, stride=stride, sstride=slay.expert_size, arenas=[], routers=[],
             shareds=[], gates=[], norms=[], layers=[])
    for l in range(NL):
        a = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(a, E, stride, lay, seed + 100 * l + 1) == 0
        r = torch.empty((E, H), dtype=torch.float32, device="cuda")
        assert kernels.synth_normal_f32(r, seed + 100 * l + 2, 0.02) == 0
        s_ = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(s_, 1, slay.expert_size, slay, seed + 100 * l + 3) == 0
        g = torch.empty(H, dtype=torch.float32, device="cuda")
        assert kernels.synth_normal_f32(g, seed + 100 * l + 4, 0.02) == 0
        nw = bf16(1.0 + norm_sigma * rng.standard_normal(H)).view(np.int16)
        c["arenas"].append(a), c["routers"].append(r), c["shareds"].append(s_), c["gates"].append(g)
        c["norms"].append(torch.from_numpy(nw.copy()).cuda())
        c["layers"].append(kernels.layer(lay, a, stride, E, k, True, r, s_, g))
    x0 = torch.empty(H, dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(x0, seed + 99, 1.0) == 0
    c["x0"] = x0
    return c


def _chain_oracle(c, eps):
    """The CPU chain: the oracle router, only the chosen experts' FFNs, the
    combine; x_{l+1} = RMSNorm(r_{l+1}) * w_{l+1}. Returns (residual, min
    k-th/(k+1)-th probability gap)."""
    H, I, k, stride, bits = c["H"], c["I"], c["k"], c["stride"], c["bits"]
    r = host(c["x0"]).copy()
    x = r.copy()
    min_gap = 1.0
    for l in range(len(c["layers"])):
        if l > 0:
            x = oracle.rms_norm_bf16(r, host(c["norms"][l]).view(np.uint16), eps)
        logits = oracle.f32_matvec(host(c["routers"][l]), x)
        p = np.sort(oracle.softmax(logits))[::-1]
        min_gap = min(min_gap, float(p[k - 1] - p[k]))
        _, idx, w = oracle.router(logits, k, True)
        arena = c["arenas"][l]
        outs = np.stack([oracle.expert_swiglu(host(arena[int(e) * stride:(int(e) + 1) * stride]), bits, H, I, 64, x)
                         for e in idx])
        sh = oracle.expert_swiglu(host(c["shareds"][l]), 4, H, I, 64, x)
        score = oracle.f32_matvec(host(c["gates"][l])[None, :], x)[0]
        r = oracle.combine(outs, w, r, sh, score)
    return r, min_gap


@pytest.mark.parametrize("bits", [4, 3])
@pytest.mark.parametrize("path", PATHS, ids=PATH_IDS)
def test_decode_chain_with_norm_weights(kernels, path, bits):
    """Four layers with non-unit RMSNorm weights between them (the norm is
    computed inside the router kernel on the three-kernel path)."""
    torch = _torch()
    c = _chain(kernels, 4, 256, 8, bits, seed=4242 + bits, norm_sigma=0.1)
    resid = c["x0"].clone()
    work = torch.empty(c["H"], dtype=torch.float32, device="cuda")
    kernels.set_decode_path(path)
    try:
        assert kernels.moe_decode_layers(c["layers"], c["norms"], 1e-6, c["x0"], resid, work) == 0
        kernels.sync()
    finally:
        kernels.set_decode_path(0)
    want, gap = _chain_oracle(c, 1e-6)
    err = rel_err(host(resid), want)
    print(f"norm chain path={path} bits={bits}: rel_err={err:.3e} min gap={gap:.3e}")
    assert err <= TOL


def test_three_kernel_decode_graph_replays_match_eager(kernels):
    """The three-kernel decode allocates nothing and sets no memory, so it
    can live in a HIP graph. Every replay, with eager work (the residual
    reset) and a synchronisation between replays, gives the eager result
    bit for bit."""
    import streamoe_amd as sa

    torch = _torch()
    c = _chain(kernels, 4, 256, 8, 4, seed=777, norm_sigma=0.1)
    resid = torch.empty_like(c["x0"])
    work = torch.empty(c["H"], dtype=torch.float32, device="cuda")

    def step():
        assert kernels.moe_decode_layers(c["layers"], c["norms"], 1e-6, c["x0"], resid, work) == 0

    kernels.set_decode_path(3)
    try:
        resid.copy_(c["x0"])
        step()
        kernels.sync()
        ref = host(resid).view(np.uint32).copy()
        resid.copy_(c["x0"])
        graph = sa.capture_graph(kernels, step)
        for i in range(4):
            resid.copy_(c["x0"])
            graph.replay()
            torch.cuda.synchronize()
            got = host(resid).view(np.uint32)
            assert np.array_equal(got, ref), f"replay {i} differs from the eager result"
        kernels.sync()
    finally:
        kernels.set_decode_path(0)


@pytest.mark.parametrize("bits", [4, 3], ids=["c2-4bit", "c3-3bit"])
@pytest.mark.parametrize("path", PATHS, ids=PATH_IDS)
def test_decode_40_layers_matches_oracle_chain(kernels, path, bits):
    """Configs 2 and 3 at full size: 40 resident layers (256 experts each,
    18 GB at 4-bit, 14 GB with packed 3-bit routed experts), one token;
    between layers x = RMSNorm(residual) with unit bf16 weights. The CPU
    chain fetches only the experts its router picks. The final residual
    must agree within 1e-3 (the smallest k-th/(k+1)-th probability gap over
    the layers is reported)."""
    torch = _torch()
    c = _chain(kernels, 40, 256, 8, bits, seed=5000 + bits)
    resid = c["x0"].clone()
    work = torch.empty(c["H"], dtype=torch.float32, device="cuda")
    kernels.set_decode_path(path)
    try:
        assert kernels.moe_decode_layers(c["layers"], c["norms"], 1e-6, c["x0"], resid, work) == 0
        kernels.sync()
    finally:
        kernels.set_decode_path(0)
    got = host(resid)
    want, min_gap = _chain_oracle(c, 1e-6)
    err = rel_err(got, want)
    print(f"40-layer chain path={path} bits={bits}: rel_err={err:.3e} min top-k gap={min_gap:.3e}")
    assert np.all(np.isfinite(got))
    assert err <= TOL
    del c
    torch.cuda.empty_cache()
