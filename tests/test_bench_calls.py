"""bench_calls.c, the bench's C call loop, on the CPU: built with gcc into a temporary folder, it
makes every call of every round in order with the inputs, output and parameters it was given,
calls sync once at the end, returns the loop's wall time, and returns -1 when sync fails or the
error count is non-zero. Python callbacks stand in for the entry points."""
from __future__ import annotations

import ctypes as C
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from plast_amd.abi import KernelParams  # noqa: E402

ENTRY = C.CFUNCTYPE(None, C.c_void_p, C.c_void_p, KernelParams)
NOARG = C.CFUNCTYPE(C.c_int)


class BenchCall(C.Structure):
    _fields_ = [("fn", ENTRY), ("inputs", C.c_void_p), ("output", C.c_void_p),
                ("params", KernelParams)]


@pytest.fixture(scope="module")
def loop(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    so = tmp_path_factory.mktemp("bench_calls") / "bench_calls.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Werror",
                    f"-I{ROOT / 'include'}", str(ROOT / "bench_calls.c"), "-o", str(so)],
                   check=True)
    h = C.CDLL(str(so))
    f = h.bench_call_loop
    f.argtypes = [C.POINTER(BenchCall), C.c_int, C.c_int, NOARG, NOARG]
    f.restype = C.c_double
    return f


def _calls(log):
    def entry(tag):
        return ENTRY(lambda ins, out, p: log.append((tag, ins, out, p.dim, p.keepdim, p.fval)))
    fns = [entry("a"), entry("b")]
    arr = (BenchCall * 2)(BenchCall(fns[0], 0x100, 0x200, KernelParams(7, 1, 0.5)),
                          BenchCall(fns[1], 0x300, 0x400, KernelParams(9, 0, -2.0)))
    return arr, fns


def test_every_call_in_order_then_one_sync(loop):
    log, syncs = [], []
    arr, keep = _calls(log)
    sync = NOARG(lambda: syncs.append(len(log)) or 0)
    errors = NOARG(lambda: 0)
    us = loop(arr, 2, 3, sync, errors)
    assert us >= 0.0
    assert log == [("a", 0x100, 0x200, 7, 1, 0.5), ("b", 0x300, 0x400, 9, 0, -2.0)] * 3
    assert syncs == [6]  # once, after the last call


def test_failure_is_reported(loop):
    log = []
    arr, keep = _calls(log)
    ok, bad = NOARG(lambda: 0), NOARG(lambda: 1)
    assert loop(arr, 2, 1, bad, ok) == -1.0   # sync failed
    assert loop(arr, 2, 1, ok, bad) == -1.0   # an entry point reported an error
    assert loop(arr, 2, 0, ok, ok) >= 0.0     # no rounds: nothing called
    assert len(log) == 4
