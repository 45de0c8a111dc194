"""Error bound of the decode matvecs' integer-limb dot product, on the CPU.

The decode kernels hold x as 24-bit block floating point per 32-input
chunk: f = 22 - e with e the frexp exponent of the chunk's largest |x|
(so 2^(e-1) <= max|x| < 2^e), m_j = rint(x_j * 2^f) with |m_j| <= 2^22,
split exactly into three signed bytes m = d0 + 2^8 d1 + 2^16 d2. The codes
q_j (0..15) meet the bytes in exact int32 sums S_L = sum_j q_j d_Lj, and
the chunk's sum_j q_j x_j is t * 2^-f with t = fma(S2, 2^16, fma(S1, 2^8,
S0)) rounded once in f32. Hence, per chunk,

    |t * 2^-f - sum_j q_j x_j| <= 2^-22 * max|x| * sum_j q_j
                                  + 2^-24 * sum_j q_j |x_j| + 2^-150,

the first term from rounding x to the grid 2^-f (half a step, at most
2^-23 * 2^e <= 2^-22 * max|x|), the second from the one f32 rounding of t,
the last from t * 2^-f landing below the normal f32 range (tiny chunks).
When the chunk's largest |x| is below 2^-128 (f >= 150), the scale 2^-f
itself underflows to 0 in f32 and the chunk contributes 0: the error is
then sum_j q_j |x_j| < 480 * 2^-128 in absolute terms, and the bound's
last term is that sum instead.
This test restates that arithmetic in numpy (integer parts exact in int64,
the f32 steps as float32) and checks the bound on random and adversarial
chunks: N(0, 1), +-100 outliers, magnitudes spread over 2^20, signed
zeros, values near the bottom of the normal range, all-subnormal chunks,
and all-zero chunks. It also reports the
worst error relative to sum_j q_j |x_j| (the scale of the f32 sequential
sum's own error)."""
import numpy as np


def limb_dot(q, x):
    """The kernel's chunk dot (common.h make_limbs / chunk_dot_i) on one
    chunk: q uint codes [32], x float32 [32]."""
    x = np.asarray(x, np.float32)
    amax = np.max(np.abs(x))
    if amax > 0:
        _, e = np.frexp(amax)
        f = 22 - int(e)
    else:
        f = 0
    m = np.rint(np.ldexp(x.astype(np.float64), f)).astype(np.int64)
    assert np.all(np.abs(m) <= 2 ** 22)
    d0 = ((m & 0xFF) ^ 0x80) - 0x80
    m1 = (m - d0) >> 8
    d1 = ((m1 & 0xFF) ^ 0x80) - 0x80
    d2 = (m1 - d1) >> 8
    assert np.all(d0 + 256 * d1 + 65536 * d2 == m)
    assert np.all(np.abs(np.stack([d0, d1, d2])) <= 128)
    q = np.asarray(q, np.int64)
    s0, s1, s2 = (int(np.sum(q * d)) for d in (d0, d1, d2))
    # t = fma(S2, 65536, fma(S1, 256, S0)) in f32 (the inner fma is exact).
    inner = np.float32(s1 * 256 + s0)
    assert float(inner) == s1 * 256 + s0
    t = np.float32(s2 * 65536 + float(inner))  # one rounding (exact product, f32 sum)
    # t * 2^-f in f32, as the kernel forms it before the scale: exact unless
    # the product falls below the normal range (then one more rounding,
    # absolute error <= 2^-150).
    return float(np.float32(t) * np.float32(2.0 ** (-f)))


def chunks(rng):
    yield rng.standard_normal(32)
    x = rng.standard_normal(32)
    x[rng.integers(0, 32, 2)] = 100.0
    yield x
    yield np.sign(rng.standard_normal(32)) * 2.0 ** (-np.linspace(0, 20, 32))
    yield np.sign(rng.standard_normal(32)) * 2.0 ** rng.uniform(-30, 10, 32)
    x = rng.standard_normal(32) * 1e-38  # near the bottom of the normal range
    yield x
    yield rng.standard_normal(32) * 1e-40  # all subnormal: the scale underflows
    x = np.zeros(32)
    x[::3] = -0.0
    yield x
    yield np.full(32, -3.0) * 2.0 ** rng.integers(-60, 60)


def test_limb_dot_error_within_bound():
    rng = np.random.default_rng(20261202)
    worst, worst_normal = 0.0, 0.0
    n = 0
    for _ in range(400):
        for kind, x in enumerate(chunks(rng)):
            x = np.asarray(x, np.float32)
            q = rng.integers(0, 16, 32)
            got = limb_dot(q, x)
            exact = float(np.sum(q.astype(np.float64) * x.astype(np.float64)))
            mag = float(np.sum(q * np.abs(x.astype(np.float64))))
            amax = float(np.max(np.abs(x)))
            f = 22 - int(np.frexp(np.float32(amax))[1]) if amax > 0 else 0
            bound = 2.0 ** -22 * amax * float(np.sum(q)) + 2.0 ** -24 * mag + (mag if f >= 150 else 2.0 ** -150)
            err = abs(got - exact)
            assert err <= bound * (1 + 1e-12), (x, q, err, bound)
            if mag > 0 and f < 150:
                worst = max(worst, err / mag)
                if kind == 0:
                    worst_normal = max(worst_normal, err / mag)
            n += 1
    print(f"{n} chunks: worst |error| / sum q|x| = {worst:.3e} (N(0, 1) chunks: {worst_normal:.3e})")
    # Relative to sum_j q_j |x_j| the error is at most about 2^-22 * sum_j q_j
    # / max q_j times that sum (one dominant value, every other value off by
    # up to half a grid step): < 2^-16 even for chunks whose values span
    # 2^30; for N(0, 1) chunks it stays near f32 resolution.
    assert worst < 2.0 ** -16
    assert worst_normal < 2.0 ** -20


def test_limb_dot_exact_on_grid_values():
    """Values already on the chunk's 24-bit grid are represented exactly:
    the only error is the final f32 rounding of t, zero for small sums."""
    rng = np.random.default_rng(5)
    for _ in range(200):
        m = rng.integers(-2 ** 10, 2 ** 10, 32)
        x = (m * 2.0 ** -10).astype(np.float32)
        q = rng.integers(0, 16, 32)
        assert limb_dot(q, x) == float(np.sum(q * x.astype(np.float64)))
