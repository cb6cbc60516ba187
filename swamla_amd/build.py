"""In-tree build of libswamla_mi355x.so for gfx950 (hipcc, no cmake).

The library is compiled next to this file so it travels with the source tree;
``_abi.lib()`` loads it from there.  ``build_library()`` always recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [
    os.path.join(HERE, "csrc", "mla_kernels.hip"),
    os.path.join(HERE, "csrc", "mla_decode.hip"),
    os.path.join(HERE, "csrc", "mla_prefill.hip"),
    os.path.join(HERE, "csrc", "mla_linear.hip"),
    os.path.join(HERE, "csrc", "mla_absorb.hip"),
    os.path.join(HERE, "csrc", "mla_scratch.hip"),
    os.path.join(HERE, "csrc", "mla_probe.hip"),
    os.path.join(HERE, "csrc", "mla_abi.cpp"),
]
OUTPUT = os.path.join(HERE, "libswamla_mi355x.so")
ARCH = os.environ.get("SWAMLA_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build)")


# Per-source options.  The decode kernel keeps its MFMA accumulators in
# ordinary VGPRs (its softmax rescales them on the VALU every sub-tile, and
# AGPR accumulators would be copied back and forth each time).
EXTRA = {
    "mla_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}
BUILD_DIR = os.path.join(HERE, "_build")


def base_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # packed fp32 VALU ops are kept out of the generated code (without
        # this the device compiler emits thousands of v_pk_{add,mul,fma}_f32
        # in the attention kernels; tests/test_codegen.py checks the built
        # code objects).  The host pass does not know the feature and warns
        # that it ignores it; -Xarch_device cannot forward -Xclang options.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"),
    ]


def compile_commands(output: str = OUTPUT) -> tuple[list[list[str]], list[str]]:
    """(one compile command per source, the link command)."""
    objs, cmds = [], []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
        cmds.append([hipcc(), *base_flags(), *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj])
        objs.append(obj)
    # -z defs: an unresolved symbol (for example a kernel stub the host pass
    # did not emit) fails the link instead of the first load
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *objs, "-o", output]
    return cmds, link


def build_library(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = OUTPUT + ".tmp"
    cmds, link = compile_commands(tmp)
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1, 8)) as ex:
        results = list(ex.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds))
    for cmd, res in zip(cmds, results):
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}) on {cmd[-3]}:\n{res.stderr[-4000:]}")
        if verbose and res.stderr:
            print(res.stderr)
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose=True))
