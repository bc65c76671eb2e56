"""Builds libh3hip.so (the C ABI of include/h3hip.h) for gfx950 with hipcc.

    python -m h3metal_amd.build

Each source compiles to an object in h3metal_amd/_build/ in parallel, then one
shared library is linked next to this file, where gpu.py loads it. Flags:
  * --offload-arch=gfx950 only (CDNA4; no other targets),
  * packed fp32 instructions disabled (-target-feature -packed-fp32-ops),
  * the row kernels (pre-pass, rot_q8) and the GEMM epilogue without FMA contraction, so their
    float32 steps are the separately rounded operations a CPU restatement
    reproduces bit for bit.
H3_DEFINES in the environment (space-separated -D flags) adds defines to every source: build variants such as the
attention kernels' timing-only instrumentation.
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
COMMON += [f for f in os.environ.get("H3_DEFINES", "").split() if f.startswith("-D")]
PER_FILE = {
    "qk_prepass.hip": ["-ffp-contract=off"],
    "rot_q8.hip": ["-ffp-contract=off"],
    "gemm.hip": ["-ffp-contract=off"],
    # score MFMAs with VGPR results (the softmax reads them), P V accumulators in AGPRs (inline assembly)
    "attention_wave.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}
# sources whose inline assembly (MFMAs, DPP fmacs) is checked for hazards in the generated code (isa_check.py)
ISA_CHECKED = ["attention_wave.hip", "qk_prepass.hip", "rot_q8.hip"]
SOURCES = ["attention_wave.hip", "attention.hip", "capi.hip", "qk_prepass.hip", "rot_q8.hip",
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


def _isa_scan(src: str, asm: str) -> None:
    from .isa_check import scan
    with open(asm) as f:
        bad = scan(f.read(), asm)
    if bad:
        raise RuntimeError(f"{src}: MFMA hazards in the generated code:\n" + "\n".join(bad[:20]))


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, src.replace(".hip", ".o"))
    _run([hipcc(), *COMMON, *PER_FILE.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj], f"compiling {src}")
    if src in ISA_CHECKED:
        asm = os.path.join(OUT_DIR, src.replace(".hip", ".s"))
        _run([hipcc(), *COMMON, *PER_FILE.get(src, []), "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o",
              asm], f"compiling {src} to assembly")
        _isa_scan(src, asm)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], "linking")
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
