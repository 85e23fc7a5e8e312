"""The optimizer update plan on the CPU (plast_amd/csrc/opt_plan.hpp, built with g++ into a small
checker): tensors split into pieces a grid can hold, workgroup numbering, launches of the
kernel-argument path (every entry once, in order, within the group size and the grid), and the
device-table cache (an equal table reused without a wait or an upload, other tables uploaded after
the wait, the table grown only when too small, and a failed wait, allocation or upload leaving
the next call to try again)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_opt_plan_rules(tmp_path):
    exe = tmp_path / "opt_plan_check"
    # host code only: the address and undefined-behaviour sanitizers watch the cache's tables
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    f"-I{ROOT / 'plast_amd' / 'csrc'}", str(ROOT / "tests" / "opt_plan_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
