"""The persistent GEMMs run on mxk::balanced_grid(tiles, resident blocks)
blocks (mx_kernels.hpp): the fewest, in whole XCD multiples, that walk the
tiles in as many rounds as one block per CU would. The check is compiled from
the library's own header as host code and run over every tile count up to
20,000 (tests/cpu_checks/balanced_grid.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc for the HIP headers")
def test_balanced_grid_keeps_the_rounds_with_the_fewest_blocks(tmp_path):
    exe = tmp_path / "balanced_grid"
    subprocess.run([HIPCC, "-O1", "-std=c++17",
                    "-I", os.path.join(ROOT, "npu-embeddings-xdna1_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"),
                    "-o", str(exe), os.path.join(HERE, "cpu_checks", "balanced_grid.cpp")],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.split()[0] == "ok" and int(r.stdout.split()[1]) == 4 * 20000
