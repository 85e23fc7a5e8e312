"""CPU checks of oracle/_ref/libplast_ref_hip.so, the reference built with the
drop-in's scheduler edit applied (its fusion_optimize calls this library's elementwise-chain pass): it links and
resolves plast_hip_fuse_elementwise_chains from libplast_hip.so, and its scheduler
(src/scheduler/scheduler.c:16-52) in JIT mode runs config 2's chain on CPU tensors (which the pass
leaves alone: it fuses GPU tensors only) through a cache miss and then a hit, with the reference's
own CPU kernels, matching the oracle bit for bit on both calls. No GPU is touched."""
from __future__ import annotations

import ctypes as C
import subprocess

import numpy as np
import pytest

from cases import assert_bits
from hostlib import REF_HIP_PATH, HostTensor, oracle_forward
from plast_amd import abi
from plast_amd.abi import KernelParams, TensorP, TensorPP
from ref_executor import CHAIN, FORWARD, _ref_executor

pytestmark = pytest.mark.skipif(not REF_HIP_PATH.exists(),
                                reason="oracle/_ref/libplast_ref_hip.so absent")


def test_patched_reference_calls_the_chain_pass():
    syms = subprocess.run(["nm", "-D", str(REF_HIP_PATH)], capture_output=True, text=True).stdout
    assert " U plast_hip_fuse_elementwise_chains" in syms
    for name in ("schedule", "jit_lookup", "jit_insert", "fusion_optimize"):
        assert f" T {name}" in syms, name
    deps = subprocess.run(["ldd", str(REF_HIP_PATH)], capture_output=True, text=True).stdout
    assert "libplast_hip.so" in deps and "not found" not in deps, deps


def test_jit_schedule_on_cpu_tensors_miss_then_hit():
    R = _ref_executor(REF_HIP_PATH)
    R.get_op_impl.argtypes, R.get_op_impl.restype = [C.c_int], abi.Op
    arena = R.arena_create(1 << 20, 0)
    sched = R.init_scheduler(R.jit_create(16))
    R.set_jit_mode(sched, True)
    keep = []
    try:
        n = 1003
        rng = np.random.RandomState(31)
        vals = [rng.randn(n).astype(np.float32) for _ in range(3)]
        leaves = [HostTensor(v) for v in vals]
        ts, root = {}, None
        for i, (op, srcs) in enumerate(CHAIN):
            ins = [leaves[s] if isinstance(s, int) else ts[s] for s in srcs]
            out = HostTensor(np.zeros(n, np.float32))
            arr = (TensorP * len(ins))(*[C.pointer(t.t) for t in ins])
            keep += [arr, out]
            code = abi.OP[op.upper()]
            root = R.arena_node_alloc(C.byref(arena), C.cast(arr, TensorPP), len(ins),
                                      C.pointer(out.t), R.get_op_impl(code), code,
                                      KernelParams(0, 0, 0.0))
            ts[f"t{i}"] = out
        for call in range(2):
            if call:
                for t in leaves:
                    t.buf[:] = rng.randn(n).astype(np.float32)
            R.schedule(sched, root, FORWARD, C.byref(arena))
            jit = sched.contents.jit.contents
            assert jit.count == 1, f"call {call}: {jit.count} cached DAGs"
            h = [HostTensor(t.numpy()) for t in leaves]
            hts = {}
            for i, (op, srcs) in enumerate(CHAIN):
                ins = [h[s] if isinstance(s, int) else hts[s] for s in srcs]
                o = HostTensor(np.zeros(n, np.float32))
                oracle_forward(op, ins, o, KernelParams(0, 0, 0.0))
                hts[f"t{i}"] = o
            assert_bits(ts["t4"].numpy(), hts["t4"].numpy(), f"call {call}")
    finally:
        R.scheduler_release(sched)
        R.arena_release(C.byref(arena))
