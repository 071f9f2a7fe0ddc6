"""Compile the in-tree libraries with hipcc.

* ``libfsctep_hip.so``: the gfx950 HIP kernels behind the C ABI of ``include/fsctep.h``.
* ``libfsctep_torch.so``: the ``torch.ops.fsctep.*`` registration (schemas, device, Meta and
  autograd kernels) over that C ABI; loadable by LibTorch processes without Python.
* ``tests/cpp/core_run``: a LibTorch program with no Python that runs an exported core.pt the way the
  LAMMPS engine does (used by the GPU tests of the TorchScript core).

    python -m fsctep_amd.build
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libfsctep_hip.so")
TORCH_LIB = os.path.join(PKG, "libfsctep_torch.so")
CORE_RUN_SRC = os.path.join(ROOT, "tests", "cpp", "core_run.cpp")
CORE_RUN = os.path.join(ROOT, "tests", "cpp", "core_run")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 (v_pk_*_f32) code generation disabled for every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", "-Wl,-soname,libfsctep_hip.so",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _torch_dirs() -> tuple[str, str]:
    import torch
    base = os.path.dirname(torch.__file__)
    return os.path.join(base, "include"), os.path.join(base, "lib")


def _check(res: subprocess.CompletedProcess | None, proc, what: str) -> str:
    out, err = proc.communicate()
    if proc.returncode != 0:
        sys.stderr.write(out + err)
        raise RuntimeError(f"hipcc failed building {what}")
    return "\n".join(ln for ln in (out + err).splitlines()
                     if ln.strip() and "packed-fp32-ops" not in ln and "not a recognized feature" not in ln)


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    tmp = LIB + ".tmp"
    hip_cmd = [hipcc, *HIP_FLAGS, *inc, *sources(), "-o", tmp]
    tinc, tlib = _torch_dirs()
    torch_srcs = ["torch_ops.cpp", "torch_bucket_ops.cpp"]
    objs = [os.path.join(PKG, src.replace(".cpp", ".o.tmp")) for src in torch_srcs]
    torch_ccs = [[hipcc, "-std=c++17", "-O2", "-fPIC", "-c", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
                  "-D_GLIBCXX_USE_CXX11_ABI=1", "-I", tinc, "-I", os.path.join(tinc, "torch", "csrc", "api", "include"),
                  "-I", "/opt/rocm/include", *inc, os.path.join(CSRC, src), "-o", obj]
                 for src, obj in zip(torch_srcs, objs)]
    crun_tmp = CORE_RUN + ".tmp"
    core_cc = ["g++", "-std=c++17", "-O1", "-D_GLIBCXX_USE_CXX11_ABI=1", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
               "-I", tinc, "-I", os.path.join(tinc, "torch", "csrc", "api", "include"), "-I", "/opt/rocm/include",
               CORE_RUN_SRC, "-o", crun_tmp,
               "-L", tlib, "-Wl,--no-as-needed", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip",
               f"-Wl,-rpath,{tlib}", "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-ldl"]
    if verbose:
        print(" ".join(hip_cmd), "\n", "\n ".join(" ".join(c) for c in torch_ccs), "\n", " ".join(core_cc),
              flush=True)
    procs = [subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
             for c in (hip_cmd, *torch_ccs, core_cc)]
    notes = [_check(None, procs[0], "libfsctep_hip.so")]
    notes += [_check(None, pr, src) for pr, src in zip(procs[1:-1], torch_srcs)]
    notes.append(_check(None, procs[-1], "tests/cpp/core_run"))
    os.replace(crun_tmp, CORE_RUN)
    os.replace(tmp, LIB)
    ttmp = TORCH_LIB + ".tmp"
    link = [hipcc, "-shared", "-fPIC", *objs, "-o", ttmp, "-L", PKG, "-lfsctep_hip", "-L", tlib, "-ltorch",
            "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}"]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("linking libfsctep_torch.so failed")
    for obj in objs:
        os.remove(obj)
    os.replace(ttmp, TORCH_LIB)
    if verbose and any(notes):
        print("\n".join(n for n in notes if n))
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
