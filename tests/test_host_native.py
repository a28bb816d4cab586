"""Host runtime (KV pool, KV manager, prefix cache, scheduler, engine):
tests/native/host_tests.cpp compiled against this repository's restatement
and, where the reference tree exists, against the reference's own sources;
both builds must pass the same assertions."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "tinyinfer_amd" / "csrc" / "host"
TEST = ROOT / "tests" / "native" / "host_tests.cpp"
REFERENCE = Path("/root/reference")
GXX = shutil.which("g++")

pytestmark = pytest.mark.skipif(GXX is None, reason="g++ not available")


def _build_and_run(tmp_path, name, includes, sources):
    exe = tmp_path / name
    cmd = [GXX, "-std=c++17", "-O1", "-w", *[f"-I{i}" for i in includes], str(TEST), *map(str, sources), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert "host tests passed" in out.stdout


def test_host_runtime_restatement(tmp_path):
    sources = [HOST / f for f in ("paged_kv.cpp", "prefix_cache.cpp", "kv_manager.cpp", "scheduler.cpp",
                                  "engine.cpp", "model.cpp")]
    _build_and_run(tmp_path, "host_tests_restated", [HOST], sources)


@pytest.mark.skipif(not (REFERENCE / "miniprefix").exists(), reason="reference tree not present")
def test_same_assertions_hold_on_reference_sources(tmp_path):
    m = REFERENCE / "miniprefix"
    sources = sorted((m / "src" / "kv").glob("*.cpp")) + [m / "src" / "scheduler" / "scheduler.cpp",
                                                         m / "src" / "engine" / "engine.cpp"]
    _build_and_run(tmp_path, "host_tests_reference", [m / "include", REFERENCE / "include"], sources)
