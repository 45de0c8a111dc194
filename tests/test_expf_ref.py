"""The router softmax's exponential (streamoe_amd/csrc/expf_ref.h) against
the host libm's expf, which is what the reference's CPU softmax calls
(moe_router.rs:64, `(*v - max_val).exp()`): every float in
[-0x1.9fe368p6, 0] (1,120,924,085 values; below that both give 0) plus the
special inputs, bit for bit. The same header runs on the GPU; the GPU side
is checked against the oracle in tests/test_gpu_softmax.py."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wno-unknown-pragmas", "-pthread", "-o", exe,
                    os.path.join(HERE, "native", "expf_check.cpp"), "-lm"], check=True)
    return exe


def test_expf_ref_equals_libm_on_every_softmax_input(checker):
    r = subprocess.run([checker], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "n=1120924100 mismatches=0" in r.stdout, r.stdout


def test_expf_check_detects_a_wrong_table_entry(tmp_path):
    """The check is sensitive: one wrong hex digit in one table entry is caught (a 1-ulp change of a double entry almost never changes the float result, so it is not the planted case)."""
    src = open(os.path.join(HERE, "native", "expf_check.cpp")).read()
    src = src.replace("return smoe::kExpTab[i];", "return smoe::kExpTab[i] ^ (i == 7 ? 1ull << 32 : 0ull);")
    path = tmp_path / "bad.cpp"
    path.write_text(src.replace('"../../streamoe_amd', '"' + os.path.join(HERE, "..", "streamoe_amd")))
    exe = str(tmp_path / "bad")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wno-unknown-pragmas", "-pthread", "-o", exe, str(path), "-lm"],
                   check=True)
    r = subprocess.run([exe, "97"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 1 and "mismatches=0" not in r.stdout, r.stdout
