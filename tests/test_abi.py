"""The C ABI library (CPU side): it loads, exports every entry point that
include/smoe.h declares, and its host-only functions behave. No GPU
compute is called here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "smoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from streamoe_amd import _abi

    lib = _abi.load()
    names = _declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The ctypes prototypes cover exactly the declared set.
    assert sorted(_abi.PROTOTYPES) == names


def test_strerror_and_version():
    from streamoe_amd import _abi

    lib = _abi.load()
    texts = [lib.smoe_strerror(c).decode() for c in range(14)]
    assert texts[0] == "ok" and len(set(texts)) == 14
    assert lib.smoe_strerror(99).decode() == "unknown status"
    assert lib.smoe_abi_version() >= 1


@pytest.mark.parametrize("h,i,bits,g", [(2048, 1024, 4, 64), (2048, 512, 4, 64), (2048, 512, 3, 64),
                                        (4096, 1024, 4, 32), (1024, 256, 3, 128)])
def test_expert_bytes_matches_oracle(h, i, bits, g):
    from streamoe_amd import _abi

    lib = _abi.load()
    shape = _abi.ExpertShape(h, i, g, bits)
    assert lib.smoe_expert_bytes(C.byref(shape)) == oracle.expert_bytes(h, i, bits, g)


def test_layout_mirror_matches_oracle():
    import streamoe_amd as sa

    for bits in (4, 3):
        lay = sa.ExpertLayout(2048, 512, bits, 64)
        assert lay.expert_size == oracle.expert_bytes(2048, 512, bits, 64)
        for blk in range(3):
            assert lay.offsets(blk) == oracle.expert_offsets(2048, 512, bits, 64, blk)
        assert sa.ExpertLayout.from_expert_size(lay.expert_size, 2048, 512) == lay
    assert sa.ExpertLayout.from_expert_size(12345, 2048, 512) is None


def test_create_destroy_argument_errors():
    from streamoe_amd import _abi

    lib = _abi.load()
    assert lib.smoe_create(0, None, None) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    assert lib.smoe_destroy(None) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    assert lib.smoe_sync(None) == _abi.CODES["SMOE_ERR_INVALID_ARG"]
    assert lib.smoe_expert_bytes(None) == 0


def test_noalloc_decode_argument_errors_without_gpu():
    """The no-allocation decode validates its arguments on the host before
    any HIP call."""
    from streamoe_amd import _abi

    lib = _abi.load()
    assert lib.smoe_moe_decode_layers_noalloc(None, None, 0, None, C.c_float(0), None, None) == \
        _abi.CODES["SMOE_ERR_INVALID_ARG"]
    lay = _abi.Layer()
    arr = (_abi.Layer * 1)(lay)
    assert lib.smoe_moe_decode_layers_noalloc(None, arr, 1, None, C.c_float(0), C.c_void_p(16),
                                              C.c_void_p(16)) == _abi.CODES["SMOE_ERR_INVALID_ARG"]


def test_create_without_gpu_reports_no_device():
    import torch
    from streamoe_amd import _abi

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = _abi.load()
    h = C.c_void_p()
    assert lib.smoe_create(0, None, C.byref(h)) == _abi.CODES["SMOE_ERR_NO_DEVICE"]
