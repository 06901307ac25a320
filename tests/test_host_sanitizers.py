"""The C ABI's host code (csrc/gdn2_api.cpp and the host side of every .hip
source: shape validation, workspace sizing, dispatch and every rejection made
before a launch) built with AddressSanitizer and UndefinedBehaviorSanitizer on
the host side only, and driven by tests/host_checks.cpp over about two million
shape combinations, the extremes of int included.  CPU only: no call reaches
a kernel launch or needs a GPU (the device code is compiled, as the objects
register it with the HIP runtime at load, but never run)."""
import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "gdn2-jax-kernel_amd" / "csrc"
SOURCES = ["gdn2_api.cpp", "gdn2_fwd.hip", "gdn2_bwd.hip", "gdn2_decode.hip", "gdn2_noalloc.hip",
           "gdn2_stage.hip"]


def _tool(name):
    for cand in (shutil.which(name), f"/opt/rocm/bin/{name}", f"/opt/rocm/llvm/bin/{name}"):
        if cand and Path(cand).exists():
            return cand
    return None


def test_host_code_under_asan_and_ubsan(tmp_path):
    hipcc, clangxx = _tool("hipcc"), _tool("clang++")
    if hipcc is None or clangxx is None or not Path("/opt/rocm/llvm/bin/clang++").exists():
        pytest.skip("ROCm toolchain not available")
    clangxx = "/opt/rocm/llvm/bin/clang++"
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=all"]

    def compile_one(src):
        obj = tmp_path / (Path(src).stem + ".o")
        cmd = [hipcc, "-x", "hip", "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *san,
               f"-I{CSRC}", f"-I{ROOT / 'include'}", "-c", str(CSRC / src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-2000:]
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(5, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    harness = tmp_path / "host_checks.o"
    subprocess.run([clangxx, "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined",
                    f"-I{ROOT / 'include'}", "-c", str(ROOT / "tests" / "host_checks.cpp"),
                    "-o", str(harness)], check=True)
    exe = tmp_path / "host_checks"
    subprocess.run([hipcc, "--offload-arch=gfx950", *san, str(harness), *map(str, objs),
                    "-o", str(exe)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert res.returncode == 0 and "0 failures" in res.stdout, res.stdout + res.stderr[-4000:]
