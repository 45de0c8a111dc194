"""Prefill (many tokens through one layer's routed experts) on the GPU vs the
oracle's build_expert_buckets + moe_permute_fuse (moe_router.rs:374-436,
moe_cpu.rs:282-339). Bar: max|d| / max|ref| <= 1e-3."""
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


def _case(kernels, n_tokens, H, I, E, k, bits, group, x_bf16, seed, routing="zipf"):
    import streamoe_amd as sa

    torch = _torch()
    lay = sa.ExpertLayout(H, I, bits, group)
    stride = lay.expert_size
    arena = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, stride, lay, seed) == 0
    if routing == "zipf":
        idx, w = sa.zipf_routing(n_tokens, E, k, 1.1, seed=seed)
    elif routing == "hot":  # every token picks expert 0 plus k-1 others
        rng = np.random.default_rng(seed)
        idx = np.stack([np.concatenate([[0], rng.choice(np.arange(1, E), k - 1, replace=False)])
                        for _ in range(n_tokens)]).astype(np.int32)
        w = rng.random((n_tokens, k)).astype(np.float32)
    else:
        raise ValueError(routing)
    if x_bf16:
        xb = torch.empty((n_tokens, H), dtype=torch.int16, device="cuda")
        assert kernels.synth_normal_bf16(xb, seed + 1, 1.0) == 0
        x_host = oracle.bf16_to_f32(host(xb).view(np.uint16)).reshape(n_tokens, H)
        x_dev = xb
    else:
        x_dev = torch.empty((n_tokens, H), dtype=torch.float32, device="cuda")
        assert kernels.synth_normal_f32(x_dev, seed + 1, 1.0) == 0
        x_host = host(x_dev)
    idx_d = torch.from_numpy(idx).cuda()
    w_d = torch.from_numpy(w).cuda()
    out = torch.empty((n_tokens, H), dtype=torch.float32, device="cuda")
    need = kernels.moe_prefill_workspace_size(lay, n_tokens, E, k)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    rc = kernels.moe_prefill(lay, arena, stride, E, idx_d, w_d, x_dev, x_bf16, n_tokens, k, out, ws)
    assert rc == 0, rc
    kernels.sync()
    buckets = oracle.build_expert_buckets(idx, w, n_tokens, k, E)
    assert buckets[0] == 0
    want = oracle.moe_permute_fuse(host(arena), stride, bits, H, I, group, x_host, buckets, n_tokens)
    return host(out), want, (arena, idx_d, w_d, x_dev, out, ws, lay, stride)


@pytest.mark.parametrize("name,n,H,I,E,k,bits,group,x_bf16,routing", [
    ("c4-a3b", 512, 2048, 512, 256, 8, 4, 64, True, "zipf"),          # config 4
    ("c4-a3b-3bit", 512, 2048, 512, 256, 8, 3, 64, True, "zipf"),
    ("f32-x", 96, 2048, 512, 64, 8, 4, 64, False, "zipf"),
    ("olmoe-shape", 64, 2048, 1024, 64, 8, 4, 64, True, "zipf"),
    ("g32", 40, 1024, 512, 32, 4, 4, 32, True, "zipf"),
    ("g128", 72, 2048, 512, 64, 8, 4, 128, True, "zipf"),
    ("g128-hot", 300, 1024, 1024, 32, 4, 4, 128, True, "hot"),
    ("g128-3bit", 40, 1024, 512, 32, 4, 3, 128, False, "zipf"),
    ("hot-expert", 200, 2048, 512, 64, 8, 4, 64, True, "hot"),
    ("one-token", 1, 2048, 512, 256, 8, 4, 64, True, "zipf"),
    ("k1", 33, 1024, 256 * 2, 16, 1, 4, 64, True, "zipf"),
    ("k10-g32", 48, 1024, 512, 64, 10, 4, 32, True, "zipf"),  # the reference's other supported top-k
    ("max-n1024-k16", 1024, 2048, 512, 256, 16, 4, 64, True, "zipf"),  # largest tokens x k (16384 entries)
    ("e512-k10", 256, 2048, 512, 512, 10, 4, 64, True, "zipf"),  # 512 experts, top-10
    ("max-e512-n1024", 1024, 2048, 512, 512, 10, 4, 64, True, "zipf"),  # largest bucketing bitmaps
    ("e512-f32-x", 64, 1024, 512, 512, 10, 3, 32, False, "zipf"),
    ("h4096-q397b", 64, 4096, 1024, 512, 10, 4, 64, True, "zipf"),  # Qwen3.5-397B-A17B layer shape
    # Shapes without grouped-GEMM tiles (hidden or inter not a multiple of
    # 256, hidden below 1024, more than 512 experts): one token at a time
    # through the per-phase decode kernels.
    ("flash-next", 40, 2560, 640, 512, 10, 4, 64, True, "zipf"),   # Qwen3.8-Flash-Next-4bit
    ("flash-next-3bit-f32", 24, 2560, 640, 128, 10, 3, 64, False, "zipf"),
    ("flash-next-tiny", 50, 256, 64, 8, 3, 4, 64, True, "zipf"),
    ("qwen3-next-tiny", 30, 512, 128, 32, 10, 4, 32, True, "hot"),
    ("e600", 20, 2048, 512, 600, 8, 4, 64, True, "zipf"),
])
def test_prefill_matches_oracle(kernels, name, n, H, I, E, k, bits, group, x_bf16, routing):
    got, want, _ = _case(kernels, n, H, I, E, k, bits, group, x_bf16, seed=sum(map(ord, name)), routing=routing)
    err = rel_err(got, want)
    print(f"prefill {name}: rel_err={err:.3e} max|ref|={np.max(np.abs(want)):.3e}")
    assert np.all(np.isfinite(got))
    assert err <= TOL


@pytest.mark.parametrize("name,n,H,I,E,k,routing", [
    ("c4-a3b", 512, 2048, 512, 256, 8, "zipf"),
    ("hot-expert", 200, 2048, 512, 64, 8, "hot"),
    ("olmoe-inter1024", 64, 2048, 1024, 64, 8, "zipf"),
    ("h1024-k4", 40, 1024, 512, 32, 4, "zipf"),
    ("inter768", 48, 2048, 768, 32, 8, "zipf"),  # down on k_pf_mm under every option
])
def test_prefill_gate_up_tiles_agree(kernels, name, n, H, I, E, k, routing):
    """The GEMM tile choices of SMOE_OPT_PREFILL_GEMM on the same inputs:
    0 (gate/up and down on 32 x 32 tiles, units of <= 16 rows on 16 x 16
    ones: the default for 4-bit group-64 experts over bf16 x), 1 (k_pf_mm's
    16 x 16 tiles only) and 2 (down on k_pf_mm) each meet the oracle bar and
    agree with each other to fp32 rounding-order differences (and the fp16
    rounding of the activations they feed)."""
    seed = sum(map(ord, name)) + 3
    got = {}
    try:
        for path in (0, 1, 2):
            kernels.set_prefill_gemm(path)
            got[path], want_p, _ = _case(kernels, n, H, I, E, k, 4, 64, True, seed=seed, routing=routing)
            if path == 0:
                want = want_p
            assert np.array_equal(want, want_p)
    finally:
        kernels.set_prefill_gemm(0)
    errs = {p: rel_err(g, want) for p, g in got.items()}
    between = {p: rel_err(got[p], got[0]) for p in (1, 2)}
    print(f"prefill {name}: vs oracle {errs}, vs path 0 {between}")
    assert all(e <= TOL for e in errs.values())
    assert all(e <= 2e-4 for e in between.values())


def test_prefill_gemm_option_values(kernels):
    import streamoe_amd as sa

    for bad in (3, -1):
        with pytest.raises(sa.SmoeError):
            kernels.set_prefill_gemm(bad)
    for ok in (2, 1, 0):
        kernels.set_prefill_gemm(ok)


def test_prefill_is_deterministic(kernels):
    """Fixed-order reductions and no atomics in the arithmetic: two runs give
    the same bits."""
    import streamoe_amd as sa

    torch = _torch()
    got, _, st = _case(kernels, 128, 2048, 512, 64, 8, 4, 64, True, seed=11)
    arena, idx_d, w_d, x_dev, out, ws, lay, stride = st
    out2 = torch.empty_like(out)
    assert kernels.moe_prefill(lay, arena, stride, 64, idx_d, w_d, x_dev, True, 128, 8, out2, ws) == 0
    kernels.sync()
    assert np.array_equal(host(out2).view(np.uint32), got.view(np.uint32))


def test_prefill_argument_errors(kernels):
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    lay = sa.ExpertLayout(2048, 512, 4, 64)
    arena = torch.zeros(4 * lay.expert_size, dtype=torch.uint8, device="cuda")
    idx = torch.zeros((4, 2), dtype=torch.int32, device="cuda")
    w = torch.zeros((4, 2), dtype=torch.float32, device="cuda")
    x = torch.zeros((4, 2048), dtype=torch.int16, device="cuda")
    out = torch.zeros((4, 2048), dtype=torch.float32, device="cuda")
    need = kernels.moe_prefill_workspace_size(lay, 4, 4, 2)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    small = torch.empty(need // 2, dtype=torch.uint8, device="cuda")
    c = _abi.CODES
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, idx, w, x, True, 4, 2, out, small) == \
        c["SMOE_ERR_WORKSPACE_TOO_SMALL"]
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, idx, w, x, True, 4, 5, out, ws) == c["SMOE_ERR_BAD_K"]
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, idx, w, x, True, 4, 0, out, ws) == c["SMOE_ERR_BAD_K"]
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, idx, w, x, True, 2000, 2, out, ws) == \
        c["SMOE_ERR_UNSUPPORTED_SHAPE"]
    # Hidden sizes above 8192 have no kernel instance (checked before any launch).
    big_h = sa.ExpertLayout(8256, 512, 4, 64)
    assert kernels.moe_prefill(big_h, arena, big_h.expert_size, 4, idx, w, x, True, 4, 2, out, ws) == \
        c["SMOE_ERR_UNSUPPORTED_SHAPE"]
    # Invalid routing is caught on the device and reported by smoe_sync.
    bad = torch.tensor([[0, 1], [2, 9], [3, 0], [1, 2]], dtype=torch.int32, device="cuda")
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, bad, w, x, True, 4, 2, out, ws) == 0
    with pytest.raises(sa.SmoeError) as ei:
        kernels.sync()
    assert ei.value.status == c["SMOE_ERR_INVALID_ARG"]
    dup = torch.tensor([[0, 1], [2, 2], [3, 0], [1, 2]], dtype=torch.int32, device="cuda")
    assert kernels.moe_prefill(lay, arena, lay.expert_size, 4, dup, w, x, True, 4, 2, out, ws) == 0
    with pytest.raises(sa.SmoeError):
        kernels.sync()
    kernels.sync()  # the error word was cleared


def test_prefill_per_token_path_errors_and_workspace(kernels):
    """The per-token path (hidden 768: no grouped-GEMM tiles) reports invalid
    routing through smoe_sync like the grouped path, needs its own
    workspace size, and leaves the error word clear after a good call."""
    import streamoe_amd as sa
    from streamoe_amd import _abi

    torch = _torch()
    c = _abi.CODES
    lay = sa.ExpertLayout(768, 256, 4, 64)
    E, n, k = 4, 4, 2
    arena = torch.empty(E * lay.expert_size, dtype=torch.uint8, device="cuda")
    assert kernels.synth_experts(arena, E, lay.expert_size, lay, 5) == 0
    w = torch.full((n, k), 0.5, dtype=torch.float32, device="cuda")
    x = torch.zeros((n, 768), dtype=torch.int16, device="cuda")
    out = torch.zeros((n, 768), dtype=torch.float32, device="cuda")
    need = kernels.moe_prefill_workspace_size(lay, n, E, k)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    small = torch.empty(need // 4, dtype=torch.uint8, device="cuda")
    good = torch.tensor([[0, 1], [2, 3], [3, 0], [1, 2]], dtype=torch.int32, device="cuda")
    assert kernels.moe_prefill(lay, arena, lay.expert_size, E, good, w, x, True, n, k, out, small) == \
        c["SMOE_ERR_WORKSPACE_TOO_SMALL"]
    assert kernels.moe_prefill(lay, arena, lay.expert_size, E, good, w, x, True, n, k, out, ws) == 0
    kernels.sync()
    for bad in ([[0, 1], [2, 9], [3, 0], [1, 2]], [[0, 1], [2, 2], [3, 0], [1, 2]], [[0, -1], [2, 3], [3, 0], [1, 2]]):
        b = torch.tensor(bad, dtype=torch.int32, device="cuda")
        assert kernels.moe_prefill(lay, arena, lay.expert_size, E, b, w, x, True, n, k, out, ws) == 0
        with pytest.raises(sa.SmoeError) as ei:
            kernels.sync()
        assert ei.value.status == c["SMOE_ERR_INVALID_ARG"]
    kernels.sync()
