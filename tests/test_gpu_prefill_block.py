"""The prefill MoE block of one layer on the GPU (smoe_moe_prefill_block:
routed experts, the shared expert over all tokens with its sigmoid gate,
and the residual), against the oracle's moe_prefill_block:
build_expert_buckets + moe_permute_fuse (moe_router.rs:374-436,
moe_cpu.rs:282-339), run_packed_expert_swiglu per token for the shared
expert, gate . x_t, and moe_combine_residual_n_tokens_cpu (backend/cpu/
mod.rs:657-695). Bar: max|d| / max|ref| <= 1e-3 on the block output and on
its MoE part (output - h_mid) alone."""
import numpy as np
import pytest

import oracle
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _torch():
    import torch

    return torch


def host(t):
    return t.detach().cpu().numpy()


def _block(kernels, n, H, I, E, k, bits, group, x_bf16, seed, shared=True, gated=True, routing="zipf",
           in_place=False):
    import streamoe_amd as sa

    torch = _torch()
    lay = sa.ExpertLayout(H, I, bits, group)
    slay = sa.ExpertLayout(H, I, 4, group)
    stride = lay.expert_size
    arena = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, stride, lay, seed) == 0
    sh = gate = None
    if shared:
        sh = torch.empty(slay.expert_size, dtype=torch.uint8, device="cuda")
        assert kernels.synth_experts(sh, 1, slay.expert_size, slay, seed + 7) == 0
        if gated:
            gate = torch.empty(H, dtype=torch.float32, device="cuda")
            assert kernels.synth_normal_f32(gate, seed + 8, 0.02) == 0
    if routing == "zipf":
        idx, w = sa.zipf_routing(n, E, k, 1.1, seed=seed)
    else:  # every token picks expert 0 plus k - 1 others
        rng = np.random.default_rng(seed)
        idx = np.stack([np.concatenate([[0], rng.choice(np.arange(1, E), k - 1, replace=False)])
                        for _ in range(n)]).astype(np.int32)
        w = rng.random((n, k)).astype(np.float32)
    if x_bf16:
        xd = torch.empty((n, H), dtype=torch.int16, device="cuda")
        assert kernels.synth_normal_bf16(xd, seed + 1, 1.0) == 0
        x_host = oracle.bf16_to_f32(host(xd).view(np.uint16)).reshape(n, H)
    else:
        xd = torch.empty((n, H), dtype=torch.float32, device="cuda")
        assert kernels.synth_normal_f32(xd, seed + 1, 1.0) == 0
        x_host = host(xd)
    h_mid = torch.empty((n, H), dtype=torch.float32, device="cuda")
    assert kernels.synth_normal_f32(h_mid, seed + 2, 1.0) == 0
    h_host = host(h_mid)
    out = h_mid if in_place else torch.empty((n, H), dtype=torch.float32, device="cuda")
    need = kernels.moe_prefill_block_workspace_size(lay, n, E, k, shared)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    idx_d, w_d = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
    rc = kernels.moe_prefill_block(lay, arena, stride, E, idx_d, w_d, xd, x_bf16, n, k, sh, gate, h_mid, out, ws)
    assert rc == 0, rc
    kernels.sync()
    want, moe, so, sg = oracle.moe_prefill_block(host(arena), stride, bits, H, I, group, E, x_host, idx, w,
                                                 h_host, None if sh is None else host(sh),
                                                 None if gate is None else host(gate))
    st = (lay, arena, stride, E, idx_d, w_d, xd, sh, gate, h_mid, ws)
    return host(out), want, h_host, st


CASES = [
    # name, n, H, I, E, k, bits, group, x_bf16, shared, gated, routing
    ("c4-a3b-shared", 512, 2048, 512, 256, 8, 4, 64, True, True, True, "zipf"),   # config 4 with the tail
    ("c4-a3b-3bit-shared", 512, 2048, 512, 256, 8, 3, 64, True, True, True, "zipf"),  # 4-bit shared beside 3-bit
    ("c4-noshared", 512, 2048, 512, 256, 8, 4, 64, True, False, False, "zipf"),
    ("c4-ungated", 256, 2048, 512, 256, 8, 4, 64, True, True, False, "zipf"),
    ("f32-x", 96, 2048, 512, 64, 8, 4, 64, False, True, True, "zipf"),
    ("one-token", 1, 2048, 512, 256, 8, 4, 64, True, True, True, "zipf"),
    ("ragged-33", 33, 2048, 512, 128, 8, 4, 64, True, True, True, "zipf"),
    ("hot-expert", 200, 2048, 512, 64, 8, 4, 64, True, True, True, "hot"),
    ("g32", 40, 1024, 512, 32, 4, 4, 32, True, True, True, "zipf"),
    ("g128-act-sums", 72, 1024, 512, 32, 4, 4, 128, False, True, True, "zipf"),
    ("g128-3bit", 40, 1024, 512, 32, 4, 3, 128, True, True, True, "zipf"),
    ("k10", 48, 1024, 512, 64, 10, 4, 32, True, True, True, "zipf"),
    ("max-n1024-k16", 1024, 2048, 512, 256, 16, 4, 64, True, True, True, "zipf"),
    ("olmoe-noshared", 64, 2048, 1024, 64, 8, 4, 64, True, False, False, "zipf"),
    ("h4096", 64, 4096, 1024, 512, 10, 4, 64, True, True, True, "zipf"),
]


@pytest.mark.parametrize("name,n,H,I,E,k,bits,group,x_bf16,shared,gated,routing", CASES, ids=[c[0] for c in CASES])
def test_prefill_block_matches_oracle(kernels, name, n, H, I, E, k, bits, group, x_bf16, shared, gated, routing):
    got, want, h, _ = _block(kernels, n, H, I, E, k, bits, group, x_bf16, sum(map(ord, name)), shared, gated,
                             routing)
    err = rel_err(got, want)
    moe_err = rel_err(got - h, want - h)
    print(f"prefill block {name}: rel_err={err:.3e} MoE part {moe_err:.3e}")
    assert np.all(np.isfinite(got))
    assert err <= TOL and moe_err <= TOL


DOWN_TILE_CASES = ["c4-a3b-shared", "c4-a3b-3bit-shared", "f32-x", "max-n1024-k16", "h4096"]


@pytest.mark.parametrize("name", DOWN_TILE_CASES)
def test_prefill_block_down_tile_option(kernels, name):
    """SMOE_OPT_PREFILL_GEMM = 2 (the down GEMM on k_pf_mm's 16 x 16 tiles
    instead of the default 32 x 32 ones, for the 4-bit group-64 experts:
    routed, or the 4-bit shared expert's own list beside 3-bit routed ones)
    meets the same bar as the default."""
    c = next(c for c in CASES if c[0] == name)
    kernels.set_prefill_gemm(2)
    try:
        got, want, h, _ = _block(kernels, *c[1:9], sum(map(ord, name)), *c[9:])
    finally:
        kernels.set_prefill_gemm(0)
    err, moe_err = rel_err(got, want), rel_err(got - h, want - h)
    print(f"prefill block {name} (16 x 16 down): rel_err={err:.3e} MoE part {moe_err:.3e}")
    assert np.all(np.isfinite(got))
    assert err <= TOL and moe_err <= TOL


def test_prefill_block_in_place_and_deterministic(kernels):
    """hidden_out may alias h_mid; two runs give the same bits."""
    got, want, h, st = _block(kernels, 128, 2048, 512, 64, 8, 4, 64, True, 21, in_place=True)
    assert rel_err(got, want) <= TOL
    torch = _torch()
    lay, arena, stride, E, idx_d, w_d, xd, sh, gate, h_mid, ws = st
    h2 = torch.from_numpy(h).cuda()
    assert kernels.moe_prefill_block(lay, arena, stride, E, idx_d, w_d, xd, True, 128, 8, sh, gate, h2, h2, ws) == 0
    kernels.sync()
    assert np.array_equal(host(h2).view(np.uint32), got.view(np.uint32))


def test_prefill_block_without_shared_equals_prefill_plus_residual(kernels):
    """No shared expert: hidden = h_mid + out_sum with out_sum from
    smoe_moe_prefill, bit for bit."""
    torch = _torch()
    got, _, h, st = _block(kernels, 96, 2048, 512, 64, 8, 4, 64, True, 31, shared=False)
    lay, arena, stride, E, idx_d, w_d, xd, _, _, _, _ = st
    out = torch.empty((96, 2048), dtype=torch.float32, device="cuda")
    ws = torch.empty(kernels.moe_prefill_workspace_size(lay, 96, E, 8), dtype=torch.uint8, device="cuda")
    assert kernels.moe_prefill(lay, arena, stride, E, idx_d, w_d, xd, True, 96, 8, out, ws) == 0
    kernels.sync()
    assert np.array_equal((h + host(out)).view(np.uint32), got.view(np.uint32))


def test_prefill_block_argument_errors(kernels):
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    lay = sa.ExpertLayout(2048, 512, 4, 64)
    t = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    f = torch.zeros(4096, dtype=torch.float32, device="cuda")
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    # a gate without a shared expert
    rc = kernels.moe_prefill_block(lay, t, lay.expert_size, 8, i, f, f, True, 1, 8, None, f, f, f, t)
    assert rc == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    # no h_mid
    rc = kernels.moe_prefill_block(lay, t, lay.expert_size, 8, i, f, f, True, 1, 8, None, None, None, f, t)
    assert rc == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    # a shape without grouped-GEMM tiles
    lay2 = sa.ExpertLayout(2560, 640, 4, 64)
    assert kernels.moe_prefill_block_workspace_size(lay2, 4, 8, 2, True) == 0
    rc = kernels.moe_prefill_block(lay2, t, lay2.expert_size, 8, i, f, f, True, 1, 2, None, None, f, f, t)
    assert rc == _abi.CODES["SMOE_ERR_UNSUPPORTED_SHAPE"]
    # workspace too small
    rc = kernels.moe_prefill_block(lay, t, lay.expert_size, 8, i, f, f, True, 1, 8, None, None, f, f, t[:256])
    assert rc == _abi.CODES["SMOE_ERR_WORKSPACE_TOO_SMALL"]
