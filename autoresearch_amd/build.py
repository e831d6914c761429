"""Build the gfx950 engine (libfgpt.so) and the Fortran host layer in-tree.

hipcc compiles every .hip source for gfx950 only; amdflang builds the
iso_c_binding module, the drop-in gpt_forward/gpt_step module and the
ids-in/ids-out harness against the library. Outputs stay inside the package
directory, next to the sources, so a copy of the repository carries them.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
FSRC = os.path.join(PKG, "fortran")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libfgpt.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLANG = os.environ.get("FC_AMD", "/opt/rocm/bin/amdflang")

HIP_SOURCES = ["fgpt_engine.hip", "fgpt_weights.hip", "fgpt_spec.hip", "kern_core.hip",
               "kern_gemm.hip", "kern_attn.hip", "kern_sample.hip", "kern_fused.hip",
               "kern_fused_gqa.hip"]
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-Wno-unused-result"]
F_SOURCES = ["fgpt_c.f90", "fgpt_drop_in.f90", "fgpt_util.f90"]
F_PROGRAMS = ["fgpt_run.f90"]
# check programs of the drop-in (test code, built next to their sources)
F_CHECKS = [os.path.join(ROOT, "tests", "fortran", "dropin_checks.f90")]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")
    return r


def build_hip(jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs, procs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    failed = []
    for cmd, p in procs:
        out, err = p.communicate()
        if p.returncode != 0:
            failed.append((cmd, out + err))
    if failed:
        for cmd, msg in failed:
            sys.stderr.write(" ".join(cmd) + "\n" + msg)
        raise RuntimeError("hipcc failed")
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_fortran() -> str:
    """Compile the Fortran binding + drop-in modules and the harness."""
    os.makedirs(BUILD, exist_ok=True)
    mod = os.path.join(BUILD, "fmod")
    os.makedirs(mod, exist_ok=True)
    objs = []
    for src in F_SOURCES:
        obj = os.path.join(BUILD, src.replace(".f90", ".o"))
        _run([FLANG, "-O2", "-fPIC", "-module-dir", mod, "-c", os.path.join(FSRC, src), "-o", obj])
        objs.append(obj)
    exe = os.path.join(PKG, "fgpt_run")
    for prog in F_PROGRAMS:
        _run([FLANG, "-O2", "-I", mod, os.path.join(FSRC, prog), *objs, "-L", PKG, "-lfgpt",
              "-Wl,-rpath,$ORIGIN", "-o", exe + ".tmp"])
        os.replace(exe + ".tmp", exe)
    for src in F_CHECKS:
        out = src[:-len(".f90")]
        rpath = os.path.relpath(PKG, os.path.dirname(src))
        _run([FLANG, "-O2", "-I", mod, src, *objs, "-L", PKG, "-lfgpt",
              f"-Wl,-rpath,$ORIGIN/{rpath}", "-o", out + ".tmp"])
        os.replace(out + ".tmp", out)
    return exe


def build_seedgen() -> str:
    out = os.path.join(PKG, "libfgpt_seed.so")
    _run(["gcc", "-O2", "-fPIC", "-fopenmp", "-shared", "-o", out + ".tmp",
          os.path.join(CSRC, "seedgen.c"), "-lm"])
    os.replace(out + ".tmp", out)
    return out


def build(fortran: bool = True) -> None:
    build_seedgen()
    build_hip()
    if fortran and os.path.exists(os.path.join(FSRC, F_PROGRAMS[0])):
        build_fortran()


if __name__ == "__main__":
    build()
    print(LIB)
