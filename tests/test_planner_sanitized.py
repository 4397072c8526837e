"""The decode planner's host code under AddressSanitizer and
UndefinedBehaviorSanitizer: ``tests/native/planner_fuzz.cpp`` drives
``pg_decode_plan_host`` with random and malformed batches and checks every
accepted plan against the work-item contract of ``include/pagegauge_hip.h``
(exact tiling of each page table, item bounds, closed-form items, the
workspace size).  The planner is plain C++ (``pg_plan.cpp``), so it is built
here with the host compiler; no GPU is involved."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "pagegauge_amd" / "csrc"


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not available")
    exe = tmp_path_factory.mktemp("planner") / "planner_fuzz"
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           f"-I{ROOT / 'include'}", f"-I{CSRC}", str(ROOT / "tests" / "native" / "planner_fuzz.cpp"),
           str(CSRC / "pg_plan.cpp"), str(CSRC / "pg_error.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=240)
    return exe


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_planner_fuzz_under_sanitizers(fuzzer, seed):
    run = subprocess.run([str(fuzzer), str(seed), "3000"], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    words = run.stdout.split()
    assert words[0] == "ok", run.stdout
    plans, rejected, closed = map(int, words[1:4])
    assert plans > 1000 and rejected > 100 and closed > 50     # every branch is exercised
