"""The CMake build (CMakeLists.txt) produces the same artefacts as nemotron_infer_amd/build.py:
libnmi.so exporting exactly the same nmi_* symbols (every one include/*.h declares), built for
gfx950 only, and the pybind module `binding` over it.  Runs on the CPU (hipcc cross-compiles);
the build takes about a minute and a half on 8 cores."""
import os
import shutil
import subprocess

import pytest

from tests.conftest import ROOT
from tests.test_capi_cpu import _declared_symbols

pytestmark = pytest.mark.skipif(shutil.which("cmake") is None or shutil.which("ninja") is None,
                                reason="cmake and ninja are needed")


def _exports(so):
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()[-1].startswith("nmi_")}


def test_cmake_build_matches_build_py(tmp_path):
    bdir = tmp_path / "build"
    env = dict(os.environ, CMAKE_BUILD_PARALLEL_LEVEL=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run(["cmake", "-S", ROOT, "-B", str(bdir), "-G", "Ninja"], capture_output=True, text=True,
                       env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run(["cmake", "--build", str(bdir)], capture_output=True, text=True, env=env, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    so = bdir / "libnmi.so"
    assert so.exists()
    cm = _exports(str(so))
    py = _exports(os.path.join(ROOT, "nemotron_infer_amd", "lib", "libnmi.so"))
    assert cm == py
    assert cm == _declared_symbols()
    # gfx950 code objects only: the offload bundle names its targets
    import re
    data = so.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[a-z]*-(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets
    mods = [f for f in os.listdir(bdir) if f.startswith("binding") and f.endswith(".so")]
    assert mods, os.listdir(bdir)


def test_cmake_rejects_other_architectures(tmp_path):
    r = subprocess.run(["cmake", "-S", ROOT, "-B", str(tmp_path / "b"), "-G", "Ninja",
                        "-DCMAKE_HIP_ARCHITECTURES=gfx942"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "gfx950" in (r.stdout + r.stderr)
