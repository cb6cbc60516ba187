"""Checks on the machine code this repository builds (the gfx950 code objects
inside swamla_amd/libswamla_mi355x.so, disassembled with ROCm's own tools):

  * no packed fp32 VALU arithmetic (v_pk_add_f32 / v_pk_mul_f32 /
    v_pk_fma_f32): swamla_amd/build.py turns the feature off for the device
    pass; without that flag the compiler emits thousands of them in the
    attention kernels;
  * no writes through the scalar data cache (scalar memory stores and
    atomics, its write-back and discard): every store is a vector store;
  * the MFMA kernels are there (the disassembly is of the real code);
  * the decode step's kernels keep everything in registers (no scratch
    loads or stores: a spill inside the products' load phase doubled their
    time), and the prompt-pass attention at most its few per-item spills.

CPU only; skipped when the library or the ROCm tools are absent.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "swamla_amd", "libswamla_mi355x.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _disassembly(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    tools = [shutil.which("objcopy"), os.path.join(LLVM, "clang-offload-bundler"), os.path.join(LLVM, "llvm-objdump")]
    if not all(t and os.path.exists(t) for t in tools):
        pytest.skip("ROCm disassembly tools not available")
    objcopy, bundler, objdump = tools
    fat = tmp_path / "fatbin.bin"
    subprocess.run([objcopy, "-O", "binary", "--only-section=.hip_fatbin", LIB, str(fat)], check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundles in the library"
    texts = []
    for k, s in enumerate(starts):
        e = starts[k + 1] if k + 1 < len(starts) else len(data)
        b, co = tmp_path / f"b{k}.bin", tmp_path / f"b{k}.co"
        b.write_bytes(data[s:e])
        subprocess.run([bundler, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={b}",
                        f"--output={co}", "--unbundle"], check=True, capture_output=True)
        texts.append(subprocess.run([objdump, "-d", "--mcpu=gfx950", str(co)], check=True, capture_output=True,
                                    text=True).stdout)
    return "\n".join(texts)


def test_device_code_has_no_packed_fp32_or_scalar_stores(tmp_path):
    dis = _disassembly(tmp_path)
    assert dis.count("v_mfma") > 1000
    packed = re.findall(r"\bv_pk_(?:add|mul|fma)_f32\b", dis)
    assert not packed, f"{len(packed)} packed fp32 instructions in the device code"
    scalar_writes = re.findall(
        r"\b(?:s_store_\w+|s_buffer_store_\w+|s_scratch_store_\w+|s_atomic_\w+|s_buffer_atomic_\w+|s_dcache_wb\w*"
        r"|s_dcache_discard\w*)\b", dis)
    assert not scalar_writes, f"scalar-cache writes in the device code: {sorted(set(scalar_writes))}"


# kernel name fragment -> scratch instructions allowed in each instance
SCRATCH_BUDGET = {
    "mla_linear_packed_kernel": 0,
    "mla_decode_dma": 0,
    "mla_decode_wide": 0,
    "mla_merge_project_kernel": 0,
    "mla_merge_kernel": 0,
    "mla_append_g16_kernel": 0,
    "mla_prefill_m32": 8,  # the persistent item loop re-loads a few values once per query group
}


def test_hot_kernels_do_not_spill(tmp_path):
    dis = _disassembly(tmp_path)
    seen = {k: 0 for k in SCRATCH_BUDGET}
    over = []
    for body in re.split(r"\n(?=[0-9a-f]+ <[^>]+>:)", dis):
        m = re.match(r"[0-9a-f]+ <([^>]+)>:", body)
        if not m:
            continue
        for frag, budget in SCRATCH_BUDGET.items():
            if frag in m.group(1):
                seen[frag] += 1
                n = len(re.findall(r"\bscratch_(?:load|store)_\w+", body))
                if n > budget:
                    over.append((m.group(1), n))
    assert all(seen.values()), f"kernels missing from the disassembly: {[k for k, v in seen.items() if not v]}"
    assert not over, f"scratch spills above budget: {over}"
