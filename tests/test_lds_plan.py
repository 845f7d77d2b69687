"""The LDS-staged GEMM's planner (bus-fill_amd/csrc/bf_lds_plan.h, plain C++)
checked on the CPU: tests/lds_plan_check.cpp compiles it with g++ and runs a
model of the kernel's loader and compute waves on every plan it makes for a
grid of shapes (bounds, no deadlock, no slot reused early, every partial parked
once), on a fifth of them again with a producer that never delivers (bounded
waits give up, and every sub-tile computed from data that had not landed is
stored as NaN), then on plans with planted mistakes, each of which must be
caught."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("lds_plan") / "lds_plan_check")
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(ROOT, "bus-fill_amd", "csrc"),
                    os.path.join(ROOT, "tests", "lds_plan_check.cpp"), "-o", exe], check=True)
    return exe


def test_every_plan_passes_the_protocol_model(checker):
    r = subprocess.run([checker], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    # "ok: P plans (R with a step ring, A with windows / activation ring), X model runs"
    words = r.stdout.split()
    plans, rings, arings = int(words[1]), int(words[3].lstrip("(")), int(words[8])
    assert plans > 2000 and rings > 100 and arings > 100, r.stdout
    # "..., D with missing producers"
    assert int(words[-4]) > 400, r.stdout


def test_planted_mistakes_are_caught(checker):
    r = subprocess.run([checker, "--self-test"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "5 of 5 planted mistakes caught" in r.stdout
