"""Build libsmoe.so (HIP, gfx950) in-tree.

    python streamoe_amd/build.py

(Run it as a script: importing the streamoe_amd package loads the built
library, which a build must not depend on.)

Each translation unit is compiled separately (in parallel) with hipcc for
gfx950 only, then linked into streamoe_amd/libsmoe.so. Packed-FP32 VALU
instructions are disabled for all device code.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsmoe.so")
SOURCES = ["api.hip", "decode.hip", "fused.hip", "loader.hip", "prefill.hip", "router.hip", "synth.hip"]
HEADERS = ["common.h", "handle.h", "kernels.h", os.path.join("..", "..", "include", "smoe.h")]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    return os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _compile(src, build_dir=BUILD, defines=()):
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *FLAGS, *[f"-D{d}" for d in defines], "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(verbose=False, out=LIB, defines=()):
    """Compile every HIP source for gfx950 and link libsmoe.so (or `out`,
    with extra preprocessor `defines` such as the kernel tunables)."""
    build_dir = BUILD if out == LIB else out + ".objs"
    os.makedirs(build_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(lambda src: _compile(src, build_dir, defines), SOURCES))
    objs = [o for o, _ in results]
    for _, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    tmp = out + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
