"""In-tree build of libswamla_mi355x.so for gfx950 (hipcc, no cmake).

The library is compiled next to this file so it travels with the source tree;
``_abi.lib()`` loads it from there.  ``build_library()`` always recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [
    os.path.join(HERE, "csrc", "mla_kernels.hip"),
    os.path.join(HERE, "csrc", "mla_prefill.hip"),
    os.path.join(HERE, "csrc", "mla_linear.hip"),
    os.path.join(HERE, "csrc", "mla_abi.cpp"),
]
OUTPUT = os.path.join(HERE, "libswamla_mi355x.so")
ARCH = os.environ.get("SWAMLA_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build)")


def compile_command(output: str = OUTPUT) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # packed fp32 VALU ops are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
        *SOURCES,
        "-o", output,
    ]


def build_library(verbose: bool = False) -> str:
    tmp = OUTPUT + ".tmp"
    cmd = compile_command(tmp)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose and res.stderr:
        print(res.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose=True))
