"""The compiled reference's executor (oracle/_ref/libplast_ref.so) over this library's GPU op
slots: nodes from arena_node_alloc (src/core/node.c:3-20) in a CPU arena of the reference, ordered
by build_dag (src/core/graph.c:30-55), rewritten by fusion_optimize (src/scheduler/fusion.c:209-224)
and the elementwise-chain pass the integration adds there, run by dag_forward / dag_backward
(graph.c:57-65). With oracle/_ref/libplast_ref_hip.so (the reference built with the
drop-in's scheduler edit applied) its own fusion_optimize runs the pass, and its scheduler (schedule, JIT cache:
src/scheduler/scheduler.c:16-52, jit.c:30-114) drives the DAG. Test infrastructure."""
from __future__ import annotations

import ctypes as C

from hostlib import REF_HIP_PATH, REF_PATH
from plast_amd import abi
from plast_amd.abi import KernelParams, TensorP, TensorPP

# config 2's chain exp(-leaky_relu(a * b + c, 0)): (op, sources), a source being a leaf index or an
# earlier node's output t<i>
CHAIN = [("mul", (0, 1)), ("add", ("t0", 2)), ("leaky_relu", ("t1",)), ("neg", ("t2",)),
         ("exp", ("t3",))]

CPU_DEVICE = 0
FORWARD, BACKWARD = 0, 1   # PASS (include/scheduler/scheduler.h)


class JITEntry(C.Structure):
    """include/scheduler/jit.h: JITEntry."""
    _fields_ = [("fingerprint", C.c_uint64), ("dag", C.POINTER(abi.DAG)), ("occupied", C.c_bool)]


class JIT(C.Structure):
    """include/scheduler/jit.h: JIT."""
    _fields_ = [("entries", C.POINTER(JITEntry)), ("cap", C.c_uint32), ("count", C.c_uint32)]


class Scheduler(C.Structure):
    """include/scheduler/scheduler.h: Scheduler."""
    _fields_ = [("jit", C.POINTER(JIT)), ("jit_mode", C.c_bool)]


_LIBS: dict = {}


def _ref_executor(path=REF_PATH):
    if str(path) in _LIBS:
        return _LIBS[str(path)]
    R = C.CDLL(str(path))
    sig = {
        "arena_create": ([C.c_uint64, C.c_int], abi.Arena),
        "arena_release": ([C.POINTER(abi.Arena)], None),
        "arena_node_alloc": ([C.POINTER(abi.Arena), TensorPP, C.c_int, TensorP, abi.Op, C.c_int,
                              KernelParams], C.POINTER(abi.Node)),
        "alloc_dag": ([C.c_uint32], C.POINTER(abi.DAG)),
        "build_dag": ([C.POINTER(abi.DAG), C.POINTER(abi.Node)], None),
        "fusion_optimize": ([C.POINTER(abi.DAG)], C.c_uint32),
        "dag_forward": ([C.POINTER(abi.DAG)], None),
        "dag_backward": ([C.POINTER(abi.DAG)], None),
        "dag_release": ([C.POINTER(abi.DAG)], None),
        "jit_create": ([C.c_uint32], C.POINTER(JIT)),
        "jit_fingerprint": ([C.POINTER(abi.Node)], C.c_uint64),
        "init_scheduler": ([C.POINTER(JIT)], C.POINTER(Scheduler)),
        "set_jit_mode": ([C.POINTER(Scheduler), C.c_bool], None),
        "schedule": ([C.POINTER(Scheduler), C.POINTER(abi.Node), C.c_int, C.POINTER(abi.Arena)],
                     None),
        "scheduler_release": ([C.POINTER(Scheduler)], None),
    }
    for name, (args, res) in sig.items():
        f = getattr(R, name)
        f.argtypes, f.restype = args, res
    _LIBS[str(path)] = R
    return R


class RefGraph:
    """Nodes in a CPU arena of the reference, over device tensors."""

    def __init__(self, lib=None, ref_path=REF_PATH):
        if lib is None:
            from plast_amd.runtime import lib as runtime_lib
            lib = runtime_lib()
        self.R = _ref_executor(ref_path)
        self.L = lib
        self.arena = self.R.arena_create(1 << 20, CPU_DEVICE)
        self.keep = []
        self.root = None

    def node(self, op, inputs, output, p=None):
        """A node over objects holding a `Tensor` struct in `.t` (device tensors, or stand-ins)."""
        arr = (TensorP * len(inputs))(*[C.pointer(t.t) for t in inputs])
        self.keep += [arr, *inputs, output]
        code = abi.OP[op.upper()]
        n = self.R.arena_node_alloc(C.byref(self.arena), C.cast(arr, TensorPP), len(inputs),
                                    C.pointer(output.t), self.L.plast_hip_get_op_impl(code), code,
                                    p or KernelParams(0, 0, 0.0))
        assert n and output.t.creator == C.addressof(n.contents)
        self.root = n
        return output

    def build(self, fuse):
        """build_dag from the last node; with fuse, the reference's pass then the chain pass (the
        chain pass called here, as the unpatched reference's fusion_optimize does not)."""
        dag = self.R.alloc_dag(1)
        dag.contents.arena = C.pointer(self.arena)
        self.R.build_dag(dag, self.root)
        applied = 0
        if fuse:
            assert self.R.fusion_optimize(dag) == 0
            alloc = C.cast(self.R.arena_alloc, abi.ArenaAllocFn)
            applied = self.L.plast_hip_fuse_elementwise_chains(dag, alloc)
            self.L.check("plast_hip_fuse_elementwise_chains")
        self.dag = dag
        return applied

    def op_types(self):
        d = self.dag.contents
        return [abi.OP_NAMES[d.nodes[i].contents.op_type] for i in range(d.count)]

    def forward(self):
        self.R.dag_forward(self.dag)
        self.L.check("reference dag_forward")

    def backward(self):
        self.R.dag_backward(self.dag)
        self.L.check("reference dag_backward")

    def close(self):
        if getattr(self, "dag", None):
            self.R.dag_release(self.dag)
            self.dag = None
        self.R.arena_release(C.byref(self.arena))


