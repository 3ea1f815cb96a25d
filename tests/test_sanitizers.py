"""CPU builds of the host code under the sanitizers (no GPU).

* The oracle (oracle/attn_oracle.c: the reference's attention, Pool, linear layers, layer norm and
  GELU restated in C) with AddressSanitizer + UndefinedBehaviorSanitizer, and again with
  ThreadSanitizer for its spin-then-futex Pool: tests/cpp/test_oracle_sanitize.c runs attention
  against a double-precision triple loop and every pooled op on 1 and 4 threads, bit for bit.
* The host planner (zwhisper_amd/csrc/attn_plan.hpp: shape rules, work units, key splits, the
  workspace layout) with AddressSanitizer + UndefinedBehaviorSanitizer:
  tests/cpp/test_plan_sanitize.cpp checks tens of thousands of random plans against the
  invariants the kernels and the merge pass rely on.

Any sanitizer report fails the run (-fno-sanitize-recover for undefined behaviour; ASan and TSan
exit non-zero on a report).
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
CSRC = os.path.join(ROOT, "zwhisper_amd", "csrc")
INCLUDE = os.path.join(ROOT, "include")
ORACLE = os.path.join(ROOT, "oracle", "attn_oracle.c")

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None, reason="no gcc/g++")


def build_and_run(cmd: list[str], exe: str, timeout: int = 300) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, "build failed:\n" + r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", TSAN_OPTIONS="halt_on_error=1")
    run = subprocess.run([exe], capture_output=True, text=True, timeout=timeout, env=env)
    out = run.stdout + run.stderr
    print(out[-2000:])
    assert run.returncode == 0, out[-4000:]
    assert "ok" in run.stdout.split()
    return out


@pytest.mark.parametrize("sanitizer", ["address,undefined", "thread"])
def test_oracle_under_sanitizers(tmp_path, sanitizer):
    exe = str(tmp_path / f"oracle_{sanitizer.replace(',', '_')}")
    cmd = ["gcc", "-std=gnu11", "-O1", "-g", f"-fsanitize={sanitizer}", "-pthread", "-march=x86-64-v3", "-Wno-psabi",
           ORACLE, os.path.join(CPP, "test_oracle_sanitize.c"), "-o", exe, "-lm"]
    if "undefined" in sanitizer:
        cmd.insert(4, "-fno-sanitize-recover=undefined")
    out = build_and_run(cmd, exe)
    assert "WARNING: ThreadSanitizer" not in out


def test_planner_under_sanitizers(tmp_path):
    exe = str(tmp_path / "planner_asan")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           f"-I{INCLUDE}", f"-I{CSRC}", os.path.join(CPP, "test_plan_sanitize.cpp"), "-o", exe]
    build_and_run(cmd, exe)
