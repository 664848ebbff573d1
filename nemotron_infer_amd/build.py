"""Build recipe for the in-tree native code (gfx950 only).

    python -m nemotron_infer_amd.build          # or __graft_entry__.build()

Produces
  nemotron_infer_amd/lib/libnmi.so                 HIP kernels + C ABI (include/nmi_fp8_linear.h)
  nemotron_infer_amd/csrc/binding<EXT_SUFFIX>      pybind11 module `binding` over the C ABI

Every HIP translation unit is compiled with ``--offload-arch=gfx950`` and with packed-fp32
code generation disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).  The build
always recompiles (it is also the "does it build" check) and replaces outputs atomically.
CMakeLists.txt at the repository root builds the same two artefacts with the same flags
(``cmake -S . -B build -G Ninja && cmake --build build``; tests/test_cmake_build.py checks that
both builds export the same symbols).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_SOURCES = ["gemv_stream.hip", "gemv_fp8.hip", "skinny4_fp8.hip", "skinny16_fp8.hip", "gemm_fp8.hip", "gemm_short.hip", "decode_fp8.hip", "rmsnorm.hip", "noalloc.hip", "sdpa_decode.hip",
               "mamba_decode.hip", "sdpa_prefill.hip", "mamba_prefill.hip"]
HOST_SOURCES = ["capi.cpp", "allocator.cpp", "block.cpp", "attention.cpp", "mamba.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}"]


def _run(cmd):
    # one compile or link step takes well under a minute; a step that runs for 15 minutes is stuck
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n  " + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


def _compile(src, obj, extra=()):
    flags = HIP_FLAGS if src.endswith(".hip") else HOST_FLAGS
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    _run([HIPCC, *lang, *flags, *extra, "-c", os.path.join(CSRC, src), "-o", obj])


def _atomic_copy(src, dst):
    tmp = dst + ".tmp"
    shutil.copyfile(src, tmp)
    os.chmod(tmp, 0o755)
    os.replace(tmp, dst)


def build_lib(verbose=False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    out = os.path.join(LIBDIR, "libnmi.so")
    with tempfile.TemporaryDirectory(prefix="nmi_build_") as tmp:
        jobs = []
        for src in HIP_SOURCES + HOST_SOURCES:
            jobs.append((src, os.path.join(tmp, os.path.basename(src) + ".o")))
        with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
            list(ex.map(lambda j: _compile(*j), jobs))
        so = os.path.join(tmp, "libnmi.so")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", so,
              *[o for _, o in jobs], "-Wl,-soname,libnmi.so"])
        _atomic_copy(so, out)
    if verbose:
        print("built", out)
    return out


def build_binding(verbose=False) -> str:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(CSRC, "binding" + suffix)
    with tempfile.TemporaryDirectory(prefix="nmi_bind_") as tmp:
        so = os.path.join(tmp, "binding" + suffix)
        _run(["g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall",
              f"-I{sysconfig.get_paths()['include']}", f"-I{pybind11.get_include()}", f"-I{INCLUDE}",
              os.path.join(CSRC, "binding.cpp"), "-o", so,
              f"-L{LIBDIR}", "-lnmi", "-Wl,-rpath,$ORIGIN/../lib"])
        _atomic_copy(so, out)
    if verbose:
        print("built", out)
    return out


def build(verbose=False):
    lib = build_lib(verbose)
    bnd = build_binding(verbose)
    return lib, bnd


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
