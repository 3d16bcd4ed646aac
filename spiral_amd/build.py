"""Build libspiral_quants.so for gfx950 with hipcc (no CMake).

    python -m spiral_amd.build          # compile every source, link in-tree

Each HIP source is compiled for gfx950 only, with packed-fp32 instructions
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops); host C++ sources
go through hipcc's host compiler. Objects land in spiral_amd/_build/ and the
library in spiral_amd/libspiral_quants.so, next to this file, so it ships with
the source tree.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libspiral_quants.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src):
    obj = BUILD / (src.name + ".o")
    inc = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    if src.suffix == ".hip":
        cmd = [hipcc(), *HIP_FLAGS, *inc, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *CXX_FLAGS, *inc, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # that line is expected and dropped.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n" + "\n".join(msgs))
    return obj, msgs


def build(verbose=False):
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, srcs))
    for obj, msgs in results:
        if verbose and msgs:
            print("\n".join(msgs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    """Build the CPU oracle (test infrastructure) with its Makefile."""
    res = subprocess.run(["make", "-C", str(ROOT / "oracle"), "-j4"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}{res.stderr}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
