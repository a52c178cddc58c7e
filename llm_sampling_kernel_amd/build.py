"""Compile the HIP sources into llm_sampling_kernel_amd/libfsamp.so for gfx950.

Plain hipcc, no torch extension machinery: the library exports the C ABI of include/fsamp.h
and depends only on the HIP runtime.  Objects go to llm_sampling_kernel_amd/_build/.
Run as ``python -m llm_sampling_kernel_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libfsamp.so")
# (source, object, extra flags): the sampler kernel is compiled in eight parts plus its table
# (fsamp_kernel.hip, FSAMP_PART), so that the instantiations build in parallel
SOURCES = ([("fsamp_kernel.hip", f"fsamp_kernel_part{n}.o", [f"-DFSAMP_PART={n}"]) for n in range(8)]
           + [("fsamp_kernel.hip", "fsamp_kernel_table.o", []),
              ("fsamp_api.hip", "fsamp_api.o", []), ("fsamp_probes.hip", "fsamp_probes.o", []),
              ("fsamp_selftest.hip", "fsamp_selftest.o", [])])

# -ffp-contract=off: the sampling tail's fp32 operations are evaluated exactly as written (the
# CPU oracle mirrors them bit for bit).  Packed fp32 ops are disabled for device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build libfsamp.so")
    return path


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src, oname, extra in SOURCES:
        obj = os.path.join(BUILD, oname)
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((oname, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        msg = "\n".join(f"--- {s}\n{t}" for s, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB + ".tmp"
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
