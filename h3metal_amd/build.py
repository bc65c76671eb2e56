"""Builds libh3hip.so (the C ABI of include/h3hip.h) for gfx950 with hipcc.

    python -m h3metal_amd.build

Each source compiles to an object in h3metal_amd/_build/ in parallel, then one
shared library is linked next to this file, where gpu.py loads it. Flags:
  * --offload-arch=gfx950 only (CDNA4; no other targets),
  * packed fp32 instructions disabled (-target-feature -packed-fp32-ops),
  * the row kernels (pre-pass, rot_q8) and the GEMM epilogue without FMA contraction, so their
    float32 steps are the separately rounded operations a CPU restatement
    reproduces bit for bit.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libh3hip.so")

COMMON = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# H3_DEFINES (space-separated -D flags) builds a variant, e.g. the attention kernels' timing-only instrumentation
COMMON += [f for f in os.environ.get("H3_DEFINES", "").split() if f.startswith("-D")]
PER_FILE = {
    "qk_prepass.hip": ["-ffp-contract=off"],
    "rot_q8.hip": ["-ffp-contract=off"],
    "gemm.hip": ["-ffp-contract=off"],
    # score MFMAs with VGPR results (the softmax reads them), P V accumulators in AGPRs (inline assembly)
    "attention_wave.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "attention_pair.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "attention_pp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}
# sources whose inline assembly (MFMAs, DPP fmacs) is checked for hazards in the generated code (isa_check.py)
ISA_CHECKED = ["attention_wave.hip", "attention_pair.hip", "attention_pp.hip", "qk_prepass.hip", "rot_q8.hip"]
# Kernels with two waves per SIMD (amdgpu-waves-per-eu "2,2") get 256 registers per lane, which the backend splits
# into equal VGPR and AGPR halves by default. These sources have their device code generated from patched IR
# instead, with the AGPR share given here (the kernels keep 96 accumulation registers: O and Q), so that the
# VGPRs of the softmax and the operands get the rest.
AGPR_ALLOC = {"attention_pair.hip": 96, "attention_pp.hip": 96}
SOURCES = ["attention_wave.hip", "attention_pair.hip", "attention_pp.hip", "attention.hip", "capi.hip", "qk_prepass.hip", "rot_q8.hip",
           "gemm.hip"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC", ""), "/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if c and os.path.exists(c):
            return c
    raise FileNotFoundError("hipcc not found (ROCm is required to build the gfx950 kernels)")


def _run(cmd: list, what: str) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's driver has returned 0 after a front-end error: its message counts as a failure too
    if r.returncode or " error: " in r.stderr or "failed to execute" in r.stderr:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")


def _llvm(tool: str) -> str:
    root = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    for c in (os.path.join(root, "llvm", "bin", tool), os.path.join(root, "lib", "llvm", "bin", tool)):
        if os.path.exists(c):
            return c
    raise FileNotFoundError(f"{tool} not found next to hipcc")


def _compile_patched(src: str, agprs: int) -> str:
    """hipcc's own steps for one source, with the device IR patched between the front end and code generation:
    device IR -> add "amdgpu-agpr-alloc" to the two-waves-per-SIMD kernels -> gfx950 code object -> offload bundle
    -> host object that embeds it (hipcc's -fcuda-include-gpubinary step)."""
    base = os.path.join(OUT_DIR, src.replace(".hip", ""))
    flags = [*COMMON, *PER_FILE.get(src, [])]
    mllvm = [f for i, f in enumerate(PER_FILE.get(src, [])) if f == "-mllvm" or (i and PER_FILE[src][i - 1] == "-mllvm")]
    _run([hipcc(), *flags, "--cuda-device-only", "-emit-llvm", "-S", os.path.join(CSRC, src), "-o", base + ".dev.ll"],
         f"compiling {src} to IR")
    with open(base + ".dev.ll") as f:
        ir = f.read()
    key = '"amdgpu-waves-per-eu"="2,2"'
    if key not in ir:
        raise RuntimeError(f"{src}: no kernel with amdgpu-waves-per-eu 2,2 to patch")
    with open(base + ".dev.ll", "w") as f:
        f.write(ir.replace(key, f'{key} "amdgpu-agpr-alloc"="{agprs}"'))
    dev = ["-target", "amdgcn-amd-amdhsa", "-mcpu=gfx950", "-O3", *mllvm]
    _run([_llvm("clang"), *dev, "-c", base + ".dev.ll", "-o", base + ".dev.o"], f"code generation of {src}")
    _run([_llvm("ld.lld"), "-flavor", "gnu", "-m", "elf64_amdgpu", "--no-undefined", "-shared", base + ".dev.o", "-o",
          base + ".co"], f"linking the code object of {src}")
    _run([_llvm("clang-offload-bundler"), "-type=o", "-bundle-align=4096",
          "-targets=host-x86_64-unknown-linux-gnu,hipv4-amdgcn-amd-amdhsa--gfx950", "-input=/dev/null",
          "-input=" + base + ".co", "-output=" + base + ".hipfb"], f"bundling {src}")
    obj = base + ".o"
    _run([hipcc(), *flags, "--cuda-host-only", "-Xclang", "-fcuda-include-gpubinary", "-Xclang", base + ".hipfb", "-c",
          os.path.join(CSRC, src), "-o", obj], f"compiling the host side of {src}")
    if src in ISA_CHECKED:
        _run([_llvm("clang"), *dev, "-S", base + ".dev.ll", "-o", base + ".s"], f"code generation of {src} (assembly)")
        _isa_scan(src, base + ".s")
    return obj


def _isa_scan(src: str, asm: str) -> None:
    from .isa_check import scan
    with open(asm) as f:
        bad = scan(f.read(), asm)
    if bad:
        raise RuntimeError(f"{src}: MFMA hazards in the generated code:\n" + "\n".join(bad[:20]))


def _compile(src: str) -> str:
    if src in AGPR_ALLOC:
        return _compile_patched(src, AGPR_ALLOC[src])
    obj = os.path.join(OUT_DIR, src.replace(".hip", ".o"))
    cmd = [hipcc(), *COMMON, *PER_FILE.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"compiling {src} failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    if src in ISA_CHECKED:
        asm = os.path.join(OUT_DIR, src.replace(".hip", ".s"))
        cmd = [hipcc(), *COMMON, *PER_FILE.get(src, []), "--cuda-device-only", "-S", os.path.join(CSRC, src),
               "-o", asm]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"compiling {src} to assembly failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
        _isa_scan(src, asm)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    try:
        build()
    except Exception as e:  # noqa: BLE001
        print(e, file=sys.stderr)
        sys.exit(1)
