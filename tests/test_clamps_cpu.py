"""The chunk-table clamps the kernels read variable-length tables through
(chunk_rows, seq_chunks in csrc/gdn2_layout.h), pinned on the CPU: the header
is compiled with g++ into tests/clamp_check.cpp, which feeds random and
adversarial tables (negative, past-the-end, INT_MIN/INT_MAX entries) and checks
that every touched token row and chunk range stays inside its buffer; and
xcd_split (same header), the workgroup-to-(chunk, part) map of fwd_out and
gram_bwd, for being a bijection that keeps a chunk's parts on one XCD.  The
GPU test test_varlen_bad_tables_stay_in_bounds exercises the clamps on the
device."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_chunk_table_clamps_stay_in_bounds(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "clamp_check"
    # under AddressSanitizer and UndefinedBehaviorSanitizer: an out-of-range index
    # or an overflowing clamp computation aborts the run
    subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-Wall", "-Werror",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    f"-I{ROOT / 'gdn2-jax-kernel_amd' / 'csrc'}",
                    str(ROOT / "tests" / "clamp_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.startswith("ok"), res.stdout + res.stderr
