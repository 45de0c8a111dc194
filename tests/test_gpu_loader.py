"""Expert arena loader on the GPU: layer files -> device arenas, byte for
byte, and a decode layer on a loaded arena == the same layer on the
arena the file was written from."""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def host(t):
    return t.detach().cpu().numpy()


def test_load_file_bytes_offsets_and_errors(kernels, tmp_path):
    import torch

    import streamoe_amd as sa
    from streamoe_amd import _abi

    # 80 MiB + 123 bytes: more than two staging buffers, ragged last chunk.
    n = (80 << 20) + 123
    data = np.random.default_rng(7).integers(0, 256, n, dtype=np.uint8)
    path = str(tmp_path / "blob.bin")
    data.tofile(path)
    dst = torch.zeros(n, dtype=torch.uint8, device="cuda")
    assert kernels.load_file(path, dst) == n
    assert np.array_equal(host(dst), data)
    part = torch.zeros(1000, dtype=torch.uint8, device="cuda")
    assert kernels.load_file(path, part, offset=(32 << 20) - 7, nbytes=1000) == 1000
    assert np.array_equal(host(part), data[(32 << 20) - 7:(32 << 20) + 993])
    c = _abi.CODES
    with pytest.raises(sa.SmoeError) as ei:
        kernels.load_file(str(tmp_path / "missing.bin"), part)
    assert ei.value.status == c["SMOE_ERR_IO"]
    with pytest.raises(sa.SmoeError) as ei:
        kernels.load_file(path, part, offset=n - 10, nbytes=20)  # past the end
    assert ei.value.status == c["SMOE_ERR_IO"]
    with pytest.raises(sa.SmoeError) as ei:
        kernels.load_file(path, part)  # destination too small
    assert ei.value.status == c["SMOE_ERR_INVALID_ARG"]


def _write_layers(kernels, root, shape, n_experts, layers, seed):
    import torch

    import streamoe_amd as sa

    H, I, G, bits = shape
    lay = sa.ExpertLayout(H, I, bits, G)
    d = os.path.join(root, "packed_experts")
    os.makedirs(d, exist_ok=True)
    arenas = {}
    for l in layers:
        a = torch.empty(n_experts * lay.expert_size, dtype=torch.uint8, device="cuda")
        sa.check(kernels.synth_experts(a, n_experts, lay.expert_size, lay, seed + l), "synth")
        host(a).tofile(os.path.join(d, f"layer_{l:02d}.bin"))
        arenas[l] = a
    return lay, arenas


def test_expert_files_load_resident_layers(kernels, tmp_path):
    import streamoe_amd as sa

    E = 16
    lay, src = _write_layers(kernels, str(tmp_path), (2048, 512, 64, 4), E, [0, 2], seed=40)
    files = sa.ExpertFiles(kernels, str(tmp_path), 3, E, 2048, 512, 64)
    assert files.layout.bits == 4 and files.stride == lay.expert_size
    assert files.arena(1) is None  # missing layer file
    for l in (0, 2):
        assert np.array_equal(host(files.arena(l)), host(src[l]))
    arena, off = files.binding(2, 5)
    assert off == 5 * lay.expert_size


def test_expert_files_reject_mixed_layouts(kernels, tmp_path):
    import streamoe_amd as sa

    _write_layers(kernels, str(tmp_path), (2048, 512, 64, 4), 4, [0], seed=50)
    _write_layers(kernels, str(tmp_path), (2048, 512, 64, 3), 4, [1], seed=51)
    with pytest.raises(sa.ExpertIoError, match="MixedLayouts"):
        sa.ExpertFiles(kernels, str(tmp_path), 2, 4, 2048, 512, 64)


@pytest.mark.parametrize("bits", [4, 3])
def test_decode_layer_on_loaded_arena_matches_source(kernels, tmp_path, bits):
    """The loaded arena is the written one: a full decode layer (router,
    top-k, experts, combine) gives bit-identical outputs and indices, and
    matches the oracle."""
    import torch

    import streamoe_amd as sa

    H, I, E, k = 2048, 512, 32, 8
    lay, src = _write_layers(kernels, str(tmp_path), (H, I, 64, bits), E, [0], seed=60 + bits)
    files = sa.ExpertFiles(kernels, str(tmp_path), 1, E, H, I, 64)
    assert files.layout.bits == bits
    router = torch.empty((E, H), dtype=torch.float32, device="cuda")
    sa.check(kernels.synth_normal_f32(router, 61, 0.02), "synth")
    x = torch.empty(H, dtype=torch.float32, device="cuda")
    sa.check(kernels.synth_normal_f32(x, 62, 1.0), "synth")
    h_mid = torch.zeros(H, dtype=torch.float32, device="cuda")
    outs = []
    for arena in (src[0], files.arena(0)):
        L = kernels.layer(lay, arena, lay.expert_size, E, k, True, router, None, None)
        out = torch.empty(H, dtype=torch.float32, device="cuda")
        idx = torch.empty(k, dtype=torch.int32, device="cuda")
        w = torch.empty(k, dtype=torch.float32, device="cuda")
        sa.check(kernels.moe_decode_layer(L, x, h_mid, out, idx, w), "decode")
        kernels.sync()
        outs.append((host(out), host(idx), host(w)))
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.array_equal(outs[0][1], outs[1][1])
    ref, ref_idx, _, _ = oracle.moe_decode_layer(host(files.arena(0)), lay.expert_size, H, I, E, k, 64, bits,
                                                 True, host(router), host(x), host(h_mid))
    assert np.array_equal(outs[1][1], ref_idx)
    err = np.max(np.abs(outs[1][0] - ref)) / np.max(np.abs(ref))
    assert err <= 1e-3, err
