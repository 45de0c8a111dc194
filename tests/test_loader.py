"""Layer-file layout detection (io/expert_io.rs:229-267) and the loader's
host-side argument checks; CPU only."""
import ctypes as C
import json
import os

import pytest

import oracle

H, I, G = 2048, 512, 64


def test_layout_and_stride_honours_declared_padding():
    """expert_io.rs:1108-1118: a padded stride is honoured only when the
    file is exactly n_experts strides long; otherwise the dense layout."""
    import streamoe_amd as sa

    n = 256
    size = oracle.expert_bytes(H, I, 4, G)
    stride = (size + 4095) // 4096 * 4096 + 4096
    lay, st = sa.layout_and_stride(n * stride, n, H, I, G, (size, stride))
    assert (lay.bits, st) == (4, stride)
    lay, st = sa.layout_and_stride(n * size, n, H, I, G, None)
    assert (lay.bits, st) == (4, size)
    lay, st = sa.layout_and_stride(n * size, n, H, I, G, (size, stride))
    assert (lay.bits, st) == (4, size)


def test_layout_of_len_detects_3bit_and_falls_back_to_4bit():
    """layout_of_len (expert_io.rs:229-237) + from_expert_size
    (variants.rs:442-450)."""
    import streamoe_amd as sa

    n = 256
    s3 = oracle.expert_bytes(H, I, 3, G)
    s4 = oracle.expert_bytes(H, I, 4, G)
    assert s3 == 1_376_256 and s4 == 1_769_472
    lay, st = sa.layout_and_stride(n * s3, n, H, I, G)
    assert (lay.bits, st) == (3, s3)
    # Not a whole number of known blobs: the legacy 4-bit assumption.
    for length in (n * s3 + 1, 12345, n * s4 - 256):
        lay, st = sa.layout_and_stride(length, n, H, I, G)
        assert (lay.bits, st) == (4, s4)
    # A declared size that is no known layout is ignored.
    lay, st = sa.layout_and_stride(n * 2_000_000, n, H, I, G, (1_999_999, 2_000_000))
    assert (lay.bits, st) == (4, s4)
    # A declared padded 3-bit layout.
    pad = s3 + 4096
    lay, st = sa.layout_and_stride(n * pad, n, H, I, G, (s3, pad))
    assert (lay.bits, st) == (3, pad)


def test_declared_stride_reads_layout_json(tmp_path):
    import streamoe_amd as sa

    d = tmp_path / "packed_experts"
    d.mkdir()
    assert sa.declared_stride(str(d)) is None  # no file
    (d / "layout.json").write_text(json.dumps({"expert_size": 100, "expert_stride": 4096}))
    assert sa.declared_stride(str(d)) == (100, 4096)
    (d / "layout.json").write_text(json.dumps({"expert_size": 4096, "expert_stride": 4096}))
    assert sa.declared_stride(str(d)) is None  # no padding
    (d / "layout.json").write_text("{not json")
    assert sa.declared_stride(str(d)) is None


def test_layout_and_load_argument_errors():
    from streamoe_amd import _abi

    lib = _abi.load()
    c = _abi.CODES
    out = _abi.FileLayout()
    assert lib.smoe_layer_file_layout(100, 0, H, I, G, 0, 0, C.byref(out)) == c["SMOE_ERR_INVALID_ARG"]
    assert lib.smoe_layer_file_layout(100, 4, H, I, 48, 0, 0, C.byref(out)) == c["SMOE_ERR_INVALID_ARG"]
    assert lib.smoe_layer_file_layout(100, 4, H, I, G, 0, 0, None) == c["SMOE_ERR_INVALID_ARG"]
    got = C.c_uint64(7)
    assert lib.smoe_load_file(None, b"/nonexistent", 0, 0, None, 0, C.byref(got)) == c["SMOE_ERR_INVALID_ARG"]
    assert got.value == 0
