"""The elementwise-chain pass on a DAG that the compiled reference built (no GPU needed: the pass
only rewrites structs). Config 2's five nodes come from the reference's arena_node_alloc
(src/core/node.c:3-20) over device-1 tensors, are ordered by its build_dag (src/core/graph.c:30-55)
and pass through its fusion_optimize (src/scheduler/fusion.c:209-224), which finds no pattern;
plast_hip_fuse_elementwise_chains, allocating through the reference's arena_alloc, then leaves one
FUSED_ELEMENTWISE node over the three leaves whose tape is the chain, with the library's GPU slots.
The same harness, given the reference's own CPU slots, runs its dag_forward on host tensors and
matches the chain's closed form, which pins the harness itself."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from hostlib import REF_PATH, HostTensor
from plast_amd import abi
from plast_amd.abi import KernelParams
from plast_amd.runtime import LIB_PATH
from ref_executor import CHAIN, RefGraph

pytestmark = pytest.mark.skipif(not REF_PATH.exists() or not LIB_PATH.exists(),
                                reason="needs oracle/_ref/libplast_ref.so and libplast_hip.so")


class _Struct:
    """A device-1 `Tensor` struct over a host buffer the pass never reads."""

    def __init__(self, n):
        self.buf = np.zeros(n, np.float32)
        self.t = abi.make_tensor(self.buf.ctypes.data, (n,), None, abi.FLOAT32, abi.GPU, False,
                                 None)


def _hip_lib():
    L = C.CDLL(str(LIB_PATH))   # loading initialises no device
    L.plast_hip_get_op_impl.argtypes = [C.c_int]
    L.plast_hip_get_op_impl.restype = abi.Op
    L.plast_hip_fuse_elementwise_chains.argtypes = [C.POINTER(abi.DAG), abi.ArenaAllocFn]
    L.plast_hip_fuse_elementwise_chains.restype = C.c_uint32
    L.check = lambda what="": None
    return L


class _RefCpuSlots:
    """get_op_impl of the reference itself, in the library's place (its CPU slots run)."""

    def __init__(self, R):
        R.get_op_impl.argtypes = [C.c_int]
        R.get_op_impl.restype = abi.Op
        self.plast_hip_get_op_impl = R.get_op_impl
        self.plast_hip_fuse_elementwise_chains = _hip_lib().plast_hip_fuse_elementwise_chains
        self.check = lambda what="": None


def test_chain_pass_fuses_a_dag_the_reference_built():
    L = _hip_lib()
    g = RefGraph(L)
    n = 4096
    leaves = [_Struct(n) for _ in range(3)]
    ts = {}
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [leaves[s] if isinstance(s, int) else ts[s] for s in srcs]
        ts[f"t{i}"] = g.node(op, ins, _Struct(n), KernelParams(0, 0, 0.0))
    try:
        assert g.build(fuse=False) == 0 and g.op_types() == ["MUL", "ADD", "LEAKY_RELU", "NEG",
                                                             "EXP"]
        g.R.dag_release(g.dag)
        g.dag = None
        assert g.build(fuse=True) == 1
        assert g.op_types() == ["FUSED_ELEMENTWISE"]
        node = g.dag.contents.nodes[0].contents
        assert node.num_inputs == 3
        assert [C.addressof(node.inputs[i].contents) for i in range(3)] == \
            [C.addressof(t.t) for t in leaves]
        assert C.addressof(node.output.contents) == C.addressof(ts["t4"].t)
        slots = L.plast_hip_get_op_impl(abi.OP["FUSED_ELEMENTWISE"])
        assert (node.op.gpu_forward, node.op.gpu_backward) == (slots.gpu_forward, slots.gpu_backward)
        assert node.op.gpu_forward
        tape = C.cast(C.c_void_p(node.params.dim), C.POINTER(abi.FusedTape)).contents
        ops = [abi.TAPE_OPS[tape.ins[i].op] for i in range(tape.num_ins)]
        assert tape.num_inputs == 3 and ops == ["LOAD", "MUL", "ADD", "LEAKY_RELU", "NEG", "EXP"]
    finally:
        g.close()


def test_harness_runs_the_reference_cpu_slots():
    g = RefGraph(_RefCpuSlots(C.CDLL(str(REF_PATH))))
    n = 1000
    rng = np.random.RandomState(1)
    a, b, c = (rng.randn(n).astype(np.float32) for _ in range(3))
    leaves = [HostTensor(v) for v in (a, b, c)]
    ts = {}
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [leaves[s] if isinstance(s, int) else ts[s] for s in srcs]
        ts[f"t{i}"] = g.node(op, ins, HostTensor(np.zeros(n, np.float32)), KernelParams(0, 0, 0.0))
    try:
        assert g.build(fuse=True) == 0           # host tensors: nothing for the chain pass
        g.forward()
        got = ts["t4"].numpy().astype(np.float64)
    finally:
        g.close()
    want = np.exp(-np.maximum(a.astype(np.float64) * b + c, 0.0))
    assert np.max(np.abs(got - want) / want) < 1e-6
