"""Build libgemma4_attn.so for gfx950 with hipcc (no torch build machinery).

Usage: python gemma4-fa4-kernels_amd/build.py [--verbose]
"""

from __future__ import annotations

import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(HERE, "gemma4_fa4_amd", "_lib")
LIB = os.path.join(LIB_DIR, "libgemma4_attn.so")
SOURCES = ["g4_api.hip", "g4_meta.hip", "g4_fwd.hip", "g4_bwd.hip", "g4_bwd_roles.hip",
           "g4_kvprep.hip"]
ARCH = "gfx950"
FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    # packed-fp32 VALU forms are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fgpu-flush-denormals-to-zero",
    "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def build(verbose: bool = False, extra: list[str] | None = None) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = [hipcc(), *FLAGS, *(extra or []), f"-I{INCLUDE}", f"-I{CSRC}",
           *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    os.replace(tmp, LIB)
    if verbose:
        print(out)
        print(f"built {LIB} in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    build(verbose="--verbose" in sys.argv)
