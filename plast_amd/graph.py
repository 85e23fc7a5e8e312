"""Build and run op DAGs over device tensors through the library's `Op` table.

Standalone stand-in for the reference's L1 executor (src/core/node.c:3-32, src/core/graph.c:30-65)
and for its scheduler's fusion hook (src/scheduler/scheduler.c:16-52, fusion.c:209-224): nodes are
`Node` structs with GPU slots from plast_hip_get_op_impl, ordered by the same depth-first
topological sort, optionally rewritten by plast_hip_fuse_elementwise_chains, then executed by
calling each node's gpu_forward slot.
"""
from __future__ import annotations

import ctypes as C

from . import abi
from .abi import KernelParams
from .runtime import DeviceTensor, lib


class Graph:
    def __init__(self):
        self.nodes: list[abi.Node] = []
        self._keep = []       # ctypes objects the C side points into
        self._arena_bufs = []
        self._alloc_cb = abi.ArenaAllocFn(self._alloc)
        self.dag = None

    # --- construction
    def node(self, op: str, inputs, output: DeviceTensor, p: KernelParams | None = None) -> DeviceTensor:
        L = lib()
        n = abi.Node()
        arr = (abi.TensorP * len(inputs))(*[C.pointer(t.t) for t in inputs])
        self._keep.append(arr)
        # the nodes point into these tensors' structs and device memory: keep the owners alive
        # as long as the graph (a collected DeviceTensor frees its buffer)
        self._keep.extend(inputs)
        self._keep.append(output)
        n.inputs = C.cast(arr, abi.TensorPP)
        n.output = C.pointer(output.t)
        n.op = L.plast_hip_get_op_impl(abi.OP[op.upper()])
        n.op_type = abi.OP[op.upper()]
        n.num_inputs = len(inputs)
        n.params = p or KernelParams(0, 0, 0.0)
        self.nodes.append(n)
        output.t.creator = C.addressof(n)
        return output

    # --- the fusion pass allocates its nodes and tapes through this callback
    def _alloc(self, arena, size, align):
        buf = C.create_string_buffer(int(size) + int(align))
        self._arena_bufs.append(buf)
        addr = C.addressof(buf)
        return (addr + align - 1) // align * align

    def build(self, root: DeviceTensor, fuse: bool = False) -> int:
        """Topologically order the nodes reachable from root's creator (graph.c:30-39); with
        fuse=True run the elementwise-chain pass. Returns the number of chains fused."""
        by_addr = {C.addressof(n): n for n in self.nodes}
        order: list[abi.Node] = []
        seen: set[int] = set()

        def visit(addr):
            seen.add(addr)
            n = by_addr[addr]
            for i in range(n.num_inputs):
                cr = n.inputs[i].contents.creator
                if cr and cr not in seen and cr in by_addr:
                    visit(cr)
            order.append(n)

        visit(root.t.creator)
        ptrs = (C.POINTER(abi.Node) * len(order))(*[C.pointer(n) for n in order])
        self._keep.append(ptrs)
        dag = abi.DAG()
        dag.nodes = ptrs
        dag.count = len(order)
        dag.capacity = len(order)
        dag.arena = None
        self.dag = dag
        fused = 0
        if fuse:
            fused = lib().plast_hip_fuse_elementwise_chains(C.byref(dag), self._alloc_cb)
            lib().check("plast_hip_fuse_elementwise_chains")
        return int(fused)

    def op_types(self) -> list[str]:
        return [abi.OP_NAMES[self.dag.nodes[i].contents.op_type] for i in range(self.dag.count)]

    def forward(self) -> None:
        """dag_forward (graph.c:57-60): each node's GPU forward slot in order."""
        L = lib()
        for i in range(self.dag.count):
            n = self.dag.nodes[i].contents
            f = C.cast(n.op.gpu_forward, abi.ForwardKernel)
            f(n.inputs, n.output, n.params)
        L.check("dag forward")

    def backward(self) -> None:
        """dag_backward (graph.c:62-65): GPU backward slots in reverse order."""
        L = lib()
        for i in range(self.dag.count - 1, -1, -1):
            n = self.dag.nodes[i].contents
            f = C.cast(n.op.gpu_backward, abi.BackwardKernel)
            f(n.inputs, n.output, n.params)
        L.check("dag backward")
