"""Multi-token decode (1..4 tokens through the same layers at once,
decode_multi.rs moe_dispatch_multi): every token equals its own
single-token decode bit for bit, and the oracle within 1e-3, with the
last layer's slot order bit-exact."""
import numpy as np
import pytest

import oracle
from helpers import rel_err
from test_gpu_decode import _chain, _chain_oracle, host

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _tokens(kernels, c, T, seed):
    import torch

    xs = torch.empty((T, c["H"]), dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(xs, seed, 1.0) == 0
    return xs


def _match_single_token(kernels, c, T, bits, seed):
    import torch

    k = c["k"]
    xs = _tokens(kernels, c, T, seed)
    resid = xs.clone()
    work = torch.empty_like(xs)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_tokens(c["layers"], c["norms"], 1e-6, T, xs, resid, work, idx, w) == 0
    kernels.sync()
    got = host(resid)
    for t in range(T):
        r1 = xs[t].clone()
        w1 = torch.empty(c["H"], dtype=torch.float32, device="cuda")
        assert kernels.moe_decode_layers(c["layers"], c["norms"], 1e-6, xs[t].contiguous(), r1, w1) == 0
        kernels.sync()
        assert np.array_equal(got[t].view(np.uint32), host(r1).view(np.uint32)), f"token {t}"
        ct = dict(c, x0=xs[t].contiguous())
        want, gap = _chain_oracle(ct, 1e-6)
        err = rel_err(got[t], want)
        print(f"H={c['H']} T={T} bits={bits} token {t}: rel_err={err:.3e} gap={gap:.2e}")
        assert err <= TOL


@pytest.mark.parametrize("T", [1, 2, 3, 4])
@pytest.mark.parametrize("bits", [4, 3])
def test_tokens_match_single_token_decode(kernels, T, bits):
    c = _chain(kernels, 3, 256, 8, bits, seed=7100 + 10 * T + bits, norm_sigma=0.1)
    _match_single_token(kernels, c, T, bits, 7200 + T)


@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_tokens_hidden_4096(kernels, T):
    """Hidden 4096: two Qwen3.5-397B-A17B-shaped layers (512 experts,
    top-10, inter 1024, gated shared expert); 3 and 4 tokens run the router
    kernel as two launches."""
    import torch

    c = _chain(kernels, 2, 512, 10, 4, seed=7500 + T, norm_sigma=0.1, I=1024, H=4096)
    _match_single_token(kernels, c, T, 4, 7600 + T)
    del c
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 3])
def test_tokens_other_shapes_take_per_token_chain(kernels, T):
    """Shapes without a three-kernel instance (Qwen3.8-Flash-Next 2560 x 640,
    top-10): each token through the per-phase chain, bit for bit its own
    smoe_moe_decode_layers, within 1e-3 of the oracle."""
    c = _chain(kernels, 2, 64, 10, 4, seed=7700 + T, norm_sigma=0.1, I=640, H=2560)
    _match_single_token(kernels, c, T, 4, 7800 + T)


def test_tokens_slot_order_of_last_layer(kernels):
    """idx_out / w_out of the last layer: the reference's exact slot order
    per token (moe_router.rs:83-141)."""
    import torch

    c = _chain(kernels, 2, 256, 8, 4, seed=7300, norm_sigma=0.0)
    T = 4
    xs = _tokens(kernels, c, T, 7301)
    resid = xs.clone()
    work = torch.empty_like(xs)
    idx = torch.empty((T, 8), dtype=torch.int32, device="cuda")
    w = torch.empty((T, 8), dtype=torch.float32, device="cuda")
    assert kernels.moe_decode_tokens(c["layers"], None, 1e-6, T, xs, resid, work, idx, w) == 0
    kernels.sync()
    for t in range(T):
        # The last layer's input: layer 0 on token t (no norm weights).
        r = host(xs[t]).copy()
        arena0 = c["arenas"][0]
        logits = oracle.f32_matvec(host(c["routers"][0]), r)
        _, i0, w0 = oracle.router(logits, 8, True)
        outs = np.stack([oracle.expert_swiglu(host(arena0[int(e) * c["stride"]:(int(e) + 1) * c["stride"]]), 4,
                                              c["H"], c["I"], 64, r) for e in i0])
        sh = oracle.expert_swiglu(host(c["shareds"][0]), 4, c["H"], c["I"], 64, r)
        score = oracle.f32_matvec(host(c["gates"][0])[None, :], r)[0]
        r1 = oracle.combine(outs, w0, r, sh, score)
        logits1 = oracle.f32_matvec(host(c["routers"][1]), r1)
        _, i1, w1 = oracle.router(logits1, 8, True)
        assert np.array_equal(host(idx[t]), i1), t
        assert np.max(np.abs(host(w[t]) - w1)) <= 1e-5


def test_tokens_argument_errors(kernels):
    import torch

    import streamoe_amd as sa
    from streamoe_amd import _abi

    c = _chain(kernels, 1, 64, 4, 4, seed=7400)
    xs = _tokens(kernels, c, 4, 7401)
    resid, work = xs.clone(), torch.empty_like(xs)
    codes = _abi.CODES
    assert kernels.moe_decode_tokens(c["layers"], None, 1e-6, 0, xs, resid, work) == codes["SMOE_ERR_INVALID_ARG"]
    assert kernels.moe_decode_tokens(c["layers"], None, 1e-6, 5, xs, resid, work) == codes["SMOE_ERR_INVALID_ARG"]
    # No three-kernel instance for hidden 1024: unsupported when only the
    # three-kernel path is allowed, else each token through the per-phase chain.
    lay = sa.ExpertLayout(1024, 512, 4, 64)
    a = torch.zeros(8 * lay.expert_size, dtype=torch.uint8, device="cuda")
    r = torch.zeros((8, 1024), dtype=torch.float32, device="cuda")
    L = kernels.layer(lay, a, lay.expert_size, 8, 2, True, r)
    x4 = torch.zeros((2, 1024), dtype=torch.float32, device="cuda")
    kernels.set_decode_path(3)
    try:
        assert kernels.moe_decode_tokens([L], None, 1e-6, 2, x4, x4.clone(), x4.clone()) == \
            codes["SMOE_ERR_UNSUPPORTED_SHAPE"]
    finally:
        kernels.set_decode_path(0)
    assert kernels.moe_decode_tokens([L], None, 1e-6, 2, x4, x4.clone(), x4.clone()) == 0
    kernels.sync()
