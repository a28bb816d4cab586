"""The protocol-v3 worker (tinyinfer_amd/csrc/worker, built into
tinyinfer_amd/lib/miniprefix_worker) against the reference worker.

CPU:
- tests/native/worker_tests.cpp (parse errors in validation order, exact
  response lines, a session transcript over a recording runner, end of input,
  a failed engine) on this repository's protocol and host runtime and, where
  the reference tree exists, on the reference's own protocol sources
  (miniprefix/apps/protocol/*.cpp) and runtime: both must pass; also on this
  repository's protocol and runtime built with AddressSanitizer and
  UndefinedBehaviorSanitizer;
- the reference's own miniprefix/tests/worker_protocol_test.cpp compiled
  against this repository's protocol and runtime, with the same output as
  when built on the reference's;
- the executable's start-up errors (usage, unreadable model, unknown backend).
GPU: the worker over the HIP runner (backends `hip` and `hip-fast`) on an
MPFX0001 checkpoint, driven through its stdin/stdout: every STEP line (tokens
and finish reasons) equals the reference Engine over the reference CpuRunner
on the same file, and for `hip` the FORWARD line (logits printed with nine
significant digits) equals the reference CpuRunner's bit for bit."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tinyinfer_amd.host import Engine, Runner, Weights

from .helpers import reference_library, smollm_config
from .test_host_native import GXX, MINE_SOURCES, REFERENCE, REF_OUT, SANITIZE, _archive, _build, _run, \
    needs_reference, reference_includes, reference_sources
from .test_mpfx_loader import source_tensors, write_mpfx

ROOT = Path(__file__).resolve().parent.parent
WORKER_SRC = ROOT / "tinyinfer_amd" / "csrc" / "worker"
HOST = ROOT / "tinyinfer_amd" / "csrc" / "host"
WORKER = ROOT / "tinyinfer_amd" / "lib" / "miniprefix_worker"
NATIVE = ROOT / "tests" / "native"

pytestmark = pytest.mark.skipif(GXX is None, reason="g++ not available")


@pytest.fixture(scope="module")
def mine_protocol(tmp_path_factory):
    out = tmp_path_factory.mktemp("worker_mine")
    return out, [HOST, WORKER_SRC], _archive(out, "mine_worker", [HOST, WORKER_SRC],
                                             MINE_SOURCES + [WORKER_SRC / "protocol.cpp"])


@pytest.fixture(scope="module")
def reference_protocol():
    if not (REFERENCE / "miniprefix").exists():
        pytest.skip("reference tree not present")
    apps = REFERENCE / "miniprefix" / "apps"
    includes = reference_includes() + [apps]
    sources = reference_sources() + sorted((apps / "protocol").glob("*.cpp"))
    return REF_OUT, includes, _archive(REF_OUT, "reference_worker", includes, sources)


def test_protocol_restatement(mine_protocol):
    out, includes, archive = mine_protocol
    proc = _run(_build(out, "worker_tests", NATIVE / "worker_tests.cpp", includes, archive))
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "passed" in proc.stdout


def test_protocol_restatement_under_sanitizers(tmp_path):
    """The same restatement on the protocol and runtime built with
    AddressSanitizer and UndefinedBehaviorSanitizer (host code only)."""
    probe = subprocess.run([GXX, *SANITIZE, "-x", "c++", "-", "-o", str(tmp_path / "probe")], input="int main(){}",
                           capture_output=True, text=True, timeout=120)
    if probe.returncode != 0:
        pytest.skip("the sanitizer runtimes are not available")
    includes = [HOST, WORKER_SRC]
    archive = _archive(tmp_path, "mine_worker", includes, MINE_SOURCES + [WORKER_SRC / "protocol.cpp"], SANITIZE)
    exe = _build(tmp_path, "worker_tests", NATIVE / "worker_tests.cpp", includes, archive, SANITIZE)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "passed" in proc.stdout
    assert "runtime error" not in proc.stderr and "AddressSanitizer" not in proc.stderr


@needs_reference
def test_restatement_holds_on_reference_protocol(reference_protocol):
    out, includes, archive = reference_protocol
    proc = _run(_build(out, "worker_tests_on_reference", NATIVE / "worker_tests.cpp", includes, archive))
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "passed" in proc.stdout


@needs_reference
def test_reference_protocol_test_file(mine_protocol, reference_protocol):
    source = REFERENCE / "miniprefix" / "tests" / "worker_protocol_test.cpp"
    _, inc_m, lib_m = mine_protocol
    _, inc_r, lib_r = reference_protocol
    on_mine = _run(_build(REF_OUT, "worker_protocol_test_on_mine", source, inc_m, lib_m))
    on_ref = _run(_build(REF_OUT, "worker_protocol_test_on_reference", source, inc_r, lib_r))
    assert on_ref.returncode == 0, on_ref.stderr[-2000:]
    assert on_mine.returncode == 0, on_mine.stderr[-2000:]
    assert on_mine.stdout == on_ref.stdout


def needs_worker():
    if not WORKER.exists():
        pytest.skip("worker not built (tinyinfer_amd.build.build())")


def model_file(tmp_path, vocabulary=4096):
    cfg = dict(smollm_config(layers=2, context=512, vocabulary=vocabulary))
    path = tmp_path / "model.mpfx"
    write_mpfx(path, cfg, source_tensors(cfg, seed=17))
    return cfg, path


def test_worker_startup_errors(tmp_path):
    needs_worker()
    usage = subprocess.run([str(WORKER)], capture_output=True, text=True, timeout=60)
    assert usage.returncode == 1 and usage.stderr.startswith("usage: miniprefix_worker MODEL hip|hip-fast CONTEXT")
    missing = subprocess.run([str(WORKER), str(tmp_path / "none.mpfx"), "hip", "64"], capture_output=True, text=True,
                             timeout=60)
    assert missing.returncode == 1 and "cannot open model" in missing.stderr
    _, path = model_file(tmp_path, vocabulary=64)
    cpu = subprocess.run([str(WORKER), str(path), "cpu", "64"], capture_output=True, text=True, timeout=60)
    assert cpu.returncode == 1 and cpu.stderr.strip() == "backend unavailable in this build"


SUBMITS = [(1, 6, [5, 900, 17, 3, 3000, 41, 7]), (2, 4, [2048, 11, 12]), (3, 5, list(range(100, 140)))]
ENGINE = dict(max_batch_size=2, token_budget=48, prefill_chunk=16, context=512)
KV = dict(block_tokens=16, max_blocks=64, prefix_cache_blocks=0)
FORWARD = [9, 4095, 77, 1]


FINISH = {"eos": 0, "length": 1, "cancelled": 2, "error": 3}  # FinishReason's wire integers


def event_line(events):
    return "OK " + " ".join([str(len(events))] + [
        f"{e['id']} {e['token'] if e['token'] is not None else -1} {FINISH[e['finish']] if e['finish'] else -1}"
        for e in events])


def reference_transcript(path, cfg):
    """The STEP and FORWARD lines the reference worker prints for the same
    commands: reference Engine and CpuRunner (oracle/_ref) on the same file."""
    ref = reference_library()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    w = Weights.load(str(path), library=ref)
    runner = Runner(w, context=cfg["context"], kind=0, **KV)
    engine = Engine(runner, **ENGINE)
    for rid, limit, prompt in SUBMITS:
        engine.submit(str(rid), prompt, max_new_tokens=limit, eos_token_id=None)
    steps = []
    while not engine.idle():
        engine.step()
        steps.append(event_line(engine.poll_events()))
    engine.shutdown()
    probe = Runner(w, context=cfg["context"], kind=0, **KV)
    probe.create("reference/9")
    logits = probe.append("reference/9", FORWARD)
    return steps, "OK" + "".join(" %.9g" % float(v) for v in np.asarray(logits, dtype=np.float32))


def drive(path, backend, steps):
    lines = [f"SUBMIT {rid} {limit} -1 {len(p)} " + " ".join(map(str, p)) for rid, limit, p in SUBMITS]
    lines += ["STEP"] * steps
    lines += [f"FORWARD 9 {len(FORWARD)} " + " ".join(map(str, FORWARD)), "STEP_STATS", "STATS", "COST_STATS",
              "QUIT"]
    args = [str(WORKER), str(path), backend, "512", str(ENGINE["max_batch_size"]), str(ENGINE["token_budget"]),
            str(ENGINE["prefill_chunk"]), str(KV["block_tokens"]), str(KV["max_blocks"]), str(KV["prefix_cache_blocks"])]
    proc = subprocess.run(args, input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return proc.stdout.splitlines()


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["hip", "hip-fast"])
def test_worker_serves_the_hip_runner(torch_cuda, tmp_path, backend):
    needs_worker()
    cfg, path = model_file(tmp_path)
    want_steps, want_forward = reference_transcript(path, cfg)
    out = drive(path, backend, len(want_steps))
    assert out[0] == f"READY MINIPREFIX 3 {cfg['vocabulary']} {cfg['eos']} 512 {backend}"
    assert out[1:1 + len(SUBMITS)] == ["OK"] * len(SUBMITS)
    got_steps = out[1 + len(SUBMITS):1 + len(SUBMITS) + len(want_steps)]
    assert got_steps == want_steps
    forward, step_stats, stats, cost, quit_line = out[1 + len(SUBMITS) + len(want_steps):]
    if backend == "hip":
        assert forward == want_forward
    else:
        got = np.array([float(v) for v in forward.split()[1:]], dtype=np.float32)
        want = np.array([float(v) for v in want_forward.split()[1:]], dtype=np.float32)
        assert float(np.max(np.abs(got - want)) / np.max(np.abs(want))) <= 1e-3
    assert step_stats.startswith("OK ") and len(step_stats.split()) == 4
    fields = stats.split()
    assert fields[0] == "OK" and len(fields) == 26 and fields[1] == "1"  # the FORWARD sequence is still live
    assert cost.split()[0] == "OK" and len(cost.split()) == 9
    assert quit_line == "OK"
