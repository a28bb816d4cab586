"""The drop-in runner builds inside the reference tree.

hip_runner.cpp (make_hip_runner, the ModelRunner over include/mp_hip.h) is
copied with its one extension header (staged_runner.h) into an empty
directory and compiled against the reference's own headers
(miniprefix/include/miniprefix/model.h, where ModelWeights holds
tinyinfer::Tensor), as a maintainer would add it next to the CPU and CUDA
runners. Only the reference's ModelRunner, KVManager and ModelWeights
interfaces may be used."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "tinyinfer_amd" / "csrc" / "host"
REFERENCE = Path("/root/reference")
GXX = shutil.which("g++")


@pytest.mark.skipif(GXX is None, reason="g++ not available")
@pytest.mark.skipif(not (REFERENCE / "miniprefix").exists(), reason="reference tree not present")
def test_hip_runner_compiles_against_reference_headers(tmp_path):
    for name in ("hip_runner.cpp", "staged_runner.h"):
        shutil.copy(HOST / name, tmp_path / name)
    assert not (tmp_path / "miniprefix").exists()
    proc = subprocess.run([GXX, "-std=c++17", "-Wall", "-Wextra", "-Werror", "-c", "hip_runner.cpp", "-o", "hip_runner.o",
                           f"-I{tmp_path}", f"-I{REFERENCE / 'miniprefix' / 'include'}", f"-I{REFERENCE / 'include'}",
                           f"-I{ROOT / 'include'}"], cwd=tmp_path, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    symbols = subprocess.run(["nm", "-C", "hip_runner.o"], cwd=tmp_path, capture_output=True, text=True).stdout
    assert "miniprefix::make_hip_runner" in symbols
    # Its KV bookkeeping is the reference's own KVManager.
    assert "miniprefix::KVManager::prepare_append" in symbols
