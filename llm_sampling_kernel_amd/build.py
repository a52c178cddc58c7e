"""Compile the HIP sources into llm_sampling_kernel_amd/libfsamp.so for gfx950, then the torch
extension module llm_sampling_kernel_amd/_fsamp_torch.so on top of it.

Plain hipcc for the library: it exports the C ABI of include/fsamp.h and depends only on the
HIP runtime.  The torch module is one C++ file built with g++ against torch's HIP headers.
Objects go to llm_sampling_kernel_amd/_build/.
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


TORCH_OP = os.path.join(PKG, "_fsamp_torch.so")


TORCH_OP_OBJ = os.path.join(BUILD, "fsamp_torch.o")


def _torch_lib_dir() -> str:
    import torch

    return os.path.join(os.path.dirname(torch.__file__), "lib")


def torch_op_compile_command(obj: str) -> list:
    """g++ line compiling the torch extension module (csrc/fsamp_torch.cpp) against torch's HIP
    headers directly (no hipify)."""
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ce

    abi = "1" if torch.compiled_with_cxx11_abi() else "0"
    inc = [f"-I{d}" for d in ce.include_paths(device_type="cuda")]
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-w", "-c",
            "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_API_INCLUDE_EXTENSION_H",
            "-DTORCH_EXTENSION_NAME=_fsamp_torch", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            *inc, f"-I{sysconfig.get_paths()['include']}", f"-I{os.path.join(ROOT, 'include')}",
            os.path.join(CSRC, "fsamp_torch.cpp"), "-o", obj]


def torch_op_link_command(obj: str, out: str) -> list:
    """Link line of the module: libtorch, the HIP runtime and libfsamp.so (found beside the
    module through its rpath)."""
    tlib = _torch_lib_dir()
    return ["g++", "-shared", "-fPIC", obj, "-o", out,
            f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
            "-ltorch_python", "-L/opt/rocm/lib", "-lamdhip64", f"-L{PKG}", "-lfsamp",
            "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}", "-Wl,-rpath,/opt/rocm/lib"]


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
    cmd = torch_op_compile_command(TORCH_OP_OBJ)
    if verbose:
        print(" ".join(cmd), flush=True)
    procs.append(("fsamp_torch.cpp", subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                      stderr=subprocess.STDOUT, text=True)))
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
    # the torch module links against the library just built
    tmp_op = TORCH_OP + ".tmp"
    cmd = torch_op_link_command(TORCH_OP_OBJ, tmp_op)
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp_op, TORCH_OP)
    return LIB


def build_torch_op(verbose: bool = False) -> str:
    """Rebuild only the torch module against the libfsamp.so already built."""
    os.makedirs(BUILD, exist_ok=True)
    for cmd in (torch_op_compile_command(TORCH_OP_OBJ),
                torch_op_link_command(TORCH_OP_OBJ, TORCH_OP + ".tmp")):
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"torch extension build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(TORCH_OP + ".tmp", TORCH_OP)
    return TORCH_OP


if __name__ == "__main__":
    if "--torch-only" in sys.argv:
        print(build_torch_op(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
