"""The shipped C++ page bookkeeping under AddressSanitizer + UndefinedBehavior-
Sanitizer: every reference trace replays with no sanitizer report and with the
same per-op results and final state the reference recorded.  Host code only
(g++, no device code)."""
import os
import shutil
import subprocess

import pytest

from oracle import paged_memory as pm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "nitrorag_amd", "csrc")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("asan") / "host_driver")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", f"-I{CSRC}",
           os.path.join(ROOT, "tests", "host_driver.cpp"), os.path.join(CSRC, "paged_memory.cpp"),
           "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def script(trace):
    lines = [f"{trace['total_blocks']} {trace['max_seqs']} {len(trace['ops'])}"]
    for op in trace["ops"]:
        toks = op.get("toks", [])
        lines.append(" ".join(str(x) for x in [op["op"], op.get("a", 0), op.get("b", 0),
                                               op.get("h", 0), len(toks), *toks]))
    return "\n".join(lines) + "\n"


def test_traces_replay_clean_under_asan_ubsan(driver, golden_traces):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    for trace in golden_traces:
        r = subprocess.run([driver], input=script(trace), capture_output=True, text=True, env=env,
                           timeout=120)
        assert r.returncode == 0 and "runtime error" not in r.stderr, (trace["name"], r.stderr[-3000:])
        out = r.stdout.strip().splitlines()
        steps = [list(map(int, ln.split())) for ln in out[:-1]]
        assert steps == [s[:2] for s in trace["steps"]], trace["name"]
        words = [int(x) for x in out[-1].split()[1:]]
        state = pm.decode_snapshot(words, trace["total_blocks"], trace["max_seqs"])
        assert state == trace["final"], trace["name"]
