"""Shared pytest setup: the `gpu` marker, and building missing artifacts in a container that has the
toolchain (the GPU box receives them prebuilt)."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # Build what is missing, when this machine can (hipcc/make present); never rebuild here.
    if shutil.which("make") and not (ROOT / "oracle" / "liboracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "all"], check=False)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if Path(hipcc).exists() and not (ROOT / "plast_amd" / "libplast_hip.so").exists():
        subprocess.run([sys.executable, "-m", "plast_amd.build"], cwd=str(ROOT), check=False)
