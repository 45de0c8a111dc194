"""smoe_moe_decode_layers_noalloc: the decode chain with no handle and no
allocation (fixed device scratch) gives smoe_moe_decode_layers' result bit
for bit, on two calls in a row, the second with a smaller input; captured
in a HIP graph after a first call and replayed (with eager work between the
replays), every replay equals the handle path's result bit for bit.

Inside a test run a handle already exists (smoe_create looks up the
scratch address), so the entry point's own first-call lookup is covered by
running the two-call check once more in a fresh process that creates no
handle before its first no-allocation call
(test_noalloc_first_call_in_a_fresh_process)."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _layers(torch, sa, n_layers, E, k, inter, seed, H=2048):
    """n_layers resident layers generated with torch on the device: 4-bit
    codes uniform, bf16 scales |N(0, .02)| and biases N(0, .01), f32 router
    N(0, .02), a 4-bit shared expert with an f32 gate, bf16 norm weights."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    lay = sa.ExpertLayout(H, inter, 4, 64)
    stride = lay.expert_size
    keep, layers, norms = [], [], []

    def blobs(n):
        a = torch.randint(0, 256, (n, stride), dtype=torch.uint8, device="cuda", generator=g)
        for blk in range(3):
            _, so, bo = lay.offsets(blk)
            nb = bo - so
            for off, sig, absval in ((so, 0.02, True), (bo, 0.01, False)):
                v = torch.randn((n, nb // 2), device="cuda", generator=g) * sig
                v = v.abs() if absval else v
                a[:, off:off + nb] = v.to(torch.bfloat16).view(torch.uint8).view(n, nb)
        return a

    for _ in range(n_layers):
        arena = blobs(E)
        router = torch.randn((E, H), device="cuda", generator=g) * 0.02
        shared = blobs(1)
        gate = torch.randn(H, device="cuda", generator=g) * 0.02
        nw = (1.0 + 0.1 * torch.randn(H, device="cuda", generator=g)).to(torch.bfloat16).view(torch.int16)
        keep += [arena, router, shared, gate]
        norms.append(nw)
        layers.append(sa.Kernels.layer(lay, arena, stride, E, k, True, router, shared, gate))
    x0 = torch.randn(H, device="cuda", generator=g)
    return layers, norms, x0, keep


def _noalloc(sa, torch, layers, norms, x0, resid):
    n = len(layers)
    arr = (sa._abi.Layer * n)(*layers)
    nw = (C.c_void_p * n)(*[t.data_ptr() for t in norms])
    stream = torch.cuda.current_stream().cuda_stream
    return sa._lib.smoe_moe_decode_layers_noalloc(C.c_void_p(stream), arr, n, nw, C.c_float(1e-6),
                                                  C.c_void_p(x0.data_ptr()), C.c_void_p(resid.data_ptr()))


def test_noalloc_decode_matches_handle_decode_twice():
    _two_calls_then_handle()


def _two_calls_then_handle():
    import torch

    import streamoe_amd as sa

    cases = [(4, 256, 8, 512, 11), (2, 64, 4, 512, 12)]  # second call: fewer layers, experts and slots
    data = [_layers(torch, sa, *c) for c in cases]
    torch.cuda.synchronize()
    got = []
    for layers, norms, x0, _ in data:  # both no-allocation calls first, back to back
        resid = x0.clone()
        print(f"noalloc call: {len(layers)} layers", flush=True)
        assert _noalloc(sa, torch, layers, norms, x0, resid) == 0
        got.append(resid)
    torch.cuda.synchronize()
    kern = sa.Kernels(0)
    try:
        for (layers, norms, x0, _), g_resid, case in zip(data, got, cases):
            resid = x0.clone()
            work = torch.empty_like(x0)
            assert kern.moe_decode_layers(layers, norms, 1e-6, x0, resid, work) == 0
            kern.sync()
            a = g_resid.cpu().numpy()
            b = resid.cpu().numpy()
            assert np.all(np.isfinite(a)) and np.any(a != x0.cpu().numpy())
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"case {case} differs"
            print(f"case {case}: bit-identical, max|resid| {np.max(np.abs(a)):.3f}")
    finally:
        kern.close()


def test_noalloc_decode_hidden_4096():
    """Two Qwen3.5-397B-A17B-shaped layers (hidden 4096, 512 experts, top-10,
    inter 1024): the fixed scratch holds them, and the result equals the
    handle path's bit for bit."""
    import torch

    import streamoe_amd as sa

    layers, norms, x0, keep = _layers(torch, sa, 2, 512, 10, 1024, 13, H=4096)
    resid = x0.clone()
    print("noalloc call: hidden 4096", flush=True)
    assert _noalloc(sa, torch, layers, norms, x0, resid) == 0
    torch.cuda.synchronize()
    kern = sa.Kernels(0)
    try:
        r2 = x0.clone()
        assert kern.moe_decode_layers(layers, norms, 1e-6, x0, r2, torch.empty_like(x0)) == 0
        kern.sync()
        a, b = resid.cpu().numpy(), r2.cpu().numpy()
        assert np.all(np.isfinite(a)) and np.any(a != x0.cpu().numpy())
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        kern.close()
    del keep


def test_noalloc_decode_argument_errors():
    import torch

    import streamoe_amd as sa
    from streamoe_amd import _abi

    lay = sa.ExpertLayout(2048, 512, 4, 64)
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    r = torch.zeros((8, 2048), dtype=torch.float32, device="cuda")
    x = torch.zeros(2048, dtype=torch.float32, device="cuda")
    nw = torch.zeros(2048, dtype=torch.int16, device="cuda")
    ok = sa.Kernels.layer(lay, buf, lay.expert_size, 8, 2, True, r)
    # Hidden 1024 has no three-kernel instance: rejected before any launch
    # (the buffers below would be too small for a launch at that shape).
    lay1k = sa.ExpertLayout(1024, 512, 4, 64)
    r1k = torch.zeros((8, 1024), dtype=torch.float32, device="cuda")
    small = sa.Kernels.layer(lay1k, buf, lay1k.expert_size, 8, 2, True, r1k)
    assert _noalloc(sa, torch, [small], [nw], x, x) == _abi.CODES["SMOE_ERR_UNSUPPORTED_SHAPE"]
    assert _noalloc(sa, torch, [ok], [nw], x[1:], x) == _abi.CODES["SMOE_ERR_MISALIGNED"]
    assert sa._lib.smoe_moe_decode_layers_noalloc(None, None, 0, None, C.c_float(0), None, None) == \
        _abi.CODES["SMOE_ERR_INVALID_ARG"]
    torch.cuda.synchronize()


def test_noalloc_graph_capture_and_replay():
    """A first call outside capture (the per-device set-up), then the chain
    captured into a HIP graph and replayed three times, the residual reset
    by eager work between replays: every replay equals the handle path."""
    import torch

    import streamoe_amd as sa

    layers, norms, x0, keep = _layers(torch, sa, 3, 256, 8, 512, 21)
    resid = x0.clone()
    assert _noalloc(sa, torch, layers, norms, x0, resid) == 0  # outside capture
    torch.cuda.synchronize()
    kern = sa.Kernels(0)
    try:
        want = x0.clone()
        assert kern.moe_decode_layers(layers, norms, 1e-6, x0, want, torch.empty_like(x0)) == 0
        kern.sync()
        want = want.cpu().numpy()
    finally:
        kern.close()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        resid.copy_(x0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            assert _noalloc(sa, torch, layers, norms, x0, resid) == 0
    torch.cuda.synchronize()
    for rep in range(3):
        resid.copy_(x0)          # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = resid.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
    del keep


def test_noalloc_first_call_in_a_fresh_process():
    """The two-call check in a new Python process that creates no handle
    before its first no-allocation call, so that call does the per-device
    scratch lookup itself."""
    env = dict(os.environ)
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "--fresh"], capture_output=True,
                       text=True, timeout=600, env=env)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "fresh process: ok" in r.stdout


if __name__ == "__main__" and "--fresh" in sys.argv:
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    _two_calls_then_handle()
    print("fresh process: ok", flush=True)
