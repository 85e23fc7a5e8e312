"""The workspace ledger's rules on the CPU (plast_amd/csrc/ws_ledger.hpp, built with g++ into a
small checker): an outgrown workspace is freed at once with no graph alive, retired while any graph
the library made is alive (replays keep their recorded addresses), and freed with the last of them;
an unknown or already destroyed graph changes nothing."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_ledger_rules(tmp_path):
    exe = tmp_path / "ledger_check"
    # host code only: the address and undefined-behaviour sanitizers watch the ledger's frees
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    f"-I{ROOT / 'plast_amd' / 'csrc'}", str(ROOT / "tests" / "ledger_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
