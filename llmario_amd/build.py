"""Build the HIP backend library in-tree: ``llmario_amd/libllmario_hip.so`` for gfx950.

Every source compiles with hipcc (host.cpp too: it includes the device structures; the scheduler
and SHA-256 sources as plain host C++), objects in parallel, then one shared-library link. Packed FP32 instructions are disabled for all device
code (``-target-feature -packed-fp32-ops``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libllmario_hip.so")
SOURCES = ["host.cpp", "plan.cpp", "sched.cpp", "sha256.cpp", "kv_kernels.hip", "decode.hip", "prefill.hip"]
# host-only sources (no device code): compiled as plain C++ by the same compiler
HOST_ONLY = {"plan.cpp", "sched.cpp", "sha256.cpp"}
ARCH = os.environ.get("LMH_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]
# build(verify=True): the backend also checks every machine instruction it emits, so an illegal
# operand (which the object path would otherwise encode silently) fails the build. The check does
# not change the code; it roughly quadruples the compile time.
VERIFY = ["-mllvm", "-verify-machineinstrs"]


# Per-source extras. prefill.hip: its scores come from matrix products and masks (-inf), never
# NaN payloads the kernel must preserve, so max/min need no sNaN-quieting canonicalisation; its
# LDS-DMA statements set M0 themselves and nothing else in that file uses M0, so the warning about
# clobbering a reserved register is silenced there.
EXTRA = {"prefill.hip": ["-fno-honor-nans", "-Wno-inline-asm"]}


def _compile(src: str, verify: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src in HOST_ONLY:
        cmd = [HIPCC, "-O3", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(HERE, "..", "include"),
               "-x", "c++", "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [HIPCC, *FLAGS, *(VERIFY if verify else []), *EXTRA.get(src, []), "-x", "hip", "-c",
               os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False, verify: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 7)) as ex:
        objs = list(ex.map(lambda src: _compile(src, verify), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
