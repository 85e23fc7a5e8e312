"""CPU checks of the drop-in boundary: struct layouts equal the reference's, the library loads and
exports every entry point include/*.h declares, and the host-side fusion pass and op table behave
(metadata only, no GPU call)."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from plast_amd import abi

ROOT = Path(__file__).resolve().parent.parent
REF_INC = Path("/root/reference/include")
LIB = ROOT / "plast_amd" / "libplast_hip.so"

LAYOUT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m))
#define S(T) printf(#T " %zu\n", sizeof(T))
int main(void) {
  S(Tensor); F(Tensor, grad); F(Tensor, creator); F(Tensor, data); F(Tensor, shape);
  F(Tensor, strides); F(Tensor, ndim); F(Tensor, dtype); F(Tensor, device); F(Tensor, requires_grad);
  S(KernelParams); F(KernelParams, dim); F(KernelParams, keepdim); F(KernelParams, fval);
  S(Arena); F(Arena, current); F(Arena, device);
  S(ArenaBlock); F(ArenaBlock, prev); F(ArenaBlock, capacity); F(ArenaBlock, offset); F(ArenaBlock, buffer);
  S(Op); S(Node); F(Node, inputs); F(Node, output); F(Node, op); F(Node, op_type); F(Node, num_inputs);
  F(Node, visited); F(Node, on_stack); F(Node, params);
  S(DAG); F(DAG, nodes); F(DAG, count); F(DAG, capacity); F(DAG, changed); F(DAG, arena);
  printf("ADD %d SUB %d MEAN %d SUM %d CONV_RELU %d FLOAT32 %d INT32 %d CPU %d\n",
         (int)ADD, (int)SUB, (int)MEAN, (int)SUM, (int)CONV_RELU, (int)FLOAT32, (int)INT32, (int)CPU);
  return 0;
}
"""


def _probe(tmp_path, includes: str, flags: list[str]) -> str:
    src = tmp_path / "probe.c"
    src.write_text(includes + LAYOUT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-o", str(exe), str(src), *flags], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


@pytest.mark.skipif(not REF_INC.exists(), reason="reference headers absent")
def test_struct_layouts_match_reference(tmp_path):
    ours = _probe(tmp_path, '#include "plast_abi.h"\n', [f"-I{ROOT / 'include'}"])
    theirs = _probe(tmp_path, '#include "core/graph.h"\n#include "core/arena.h"\n',
                    [f"-I{REF_INC}"])
    assert ours == theirs


def test_ctypes_mirror_matches_header(tmp_path):
    out = _probe(tmp_path, '#include "plast_abi.h"\n', [f"-I{ROOT / 'include'}"])
    vals = dict(line.rsplit(" ", 1) for line in out.splitlines() if "." in line or line.count(" ") == 1)
    assert int(vals["Tensor"]) == C.sizeof(abi.Tensor)
    assert int(vals["Node"]) == C.sizeof(abi.Node)
    assert int(vals["DAG"]) == C.sizeof(abi.DAG)
    assert int(vals["Node.params"]) == abi.Node.params.offset
    assert int(vals["Tensor.requires_grad"]) == abi.Tensor.requires_grad.offset


def _declared_functions() -> list[str]:
    names = []
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^PLAST_HIP_KERNEL_PAIR\((\w+)\)", text, flags=re.M):
            names += [f"{m.group(1)}_hip_forward", f"{m.group(1)}_hip_backward"]
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M):
            if m.group(1) not in ("PLAST_HIP_KERNEL_PAIR",) and not m.group(0).startswith("typedef"):
                names.append(m.group(1))
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "run `python -m plast_amd.build`"
    names = _declared_functions()
    assert len(names) > 60
    lib = C.CDLL(str(LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_op_table_fills_gpu_slots():
    from plast_amd.runtime import Library
    L = Library()
    for name in ["ADD", "SUB", "MUL", "DIV", "EXP", "LOG", "NEG", "ABS", "LEAKY_RELU", "SUM",
                 "MEAN", "MAX", "MIN", "ARGMAX", "TRANSPOSE", "FUSED_ELEMENTWISE",
                 "SOFTMAX_CROSS_ENTROPY", "SOFTMAX", "LOG_SOFTMAX"]:
        op = L.plast_hip_get_op_impl(abi.OP[name])
        assert op.gpu_forward and op.gpu_backward and not op.cpu_forward, name
    op = L.plast_hip_get_op_impl(abi.OP["MATMUL"])
    assert not op.gpu_forward


# ------------------------------------------------------------------------------- fusion pass
class _MetaGraph:
    """Nodes over metadata-only tensors (data = NULL): exercises the pass without a GPU."""

    def __init__(self, L):
        self.L = L
        self.keep = []
        self.nodes = []
        self.bufs = []
        self.cb = abi.ArenaAllocFn(self._alloc)

    def _alloc(self, arena, size, align):
        b = C.create_string_buffer(size + align)
        self.bufs.append(b)
        return (C.addressof(b) + align - 1) // align * align

    def t(self, shape, grad=False):
        x = abi.make_tensor(0, shape, None, abi.FLOAT32, abi.GPU, grad)
        self.keep.append(x)
        return x

    def node(self, op, ins, out, fval=0.0):
        n = abi.Node()
        arr = (abi.TensorP * len(ins))(*[C.pointer(i) for i in ins])
        self.keep.append(arr)
        n.inputs = C.cast(arr, abi.TensorPP)
        n.output = C.pointer(out)
        n.op = self.L.plast_hip_get_op_impl(abi.OP[op])
        n.op_type = abi.OP[op]
        n.num_inputs = len(ins)
        n.params = abi.KernelParams(0, 0, fval)
        out.creator = C.addressof(n)
        self.nodes.append(n)
        return out

    def run(self):
        ptrs = (C.POINTER(abi.Node) * len(self.nodes))(*[C.pointer(n) for n in self.nodes])
        self.keep.append(ptrs)
        dag = abi.DAG()
        dag.nodes = ptrs
        dag.count = dag.capacity = len(self.nodes)
        k = self.L.plast_hip_fuse_elementwise_chains(C.byref(dag), self.cb)
        return k, dag, [dag.nodes[i].contents for i in range(dag.count)]


def _tape(node) -> abi.FusedTape:
    return C.cast(C.c_void_p(node.params.dim), C.POINTER(abi.FusedTape)).contents


def test_fusion_pass_config2_chain():
    from plast_amd.runtime import Library
    g = _MetaGraph(Library())
    a, b, c = g.t((64,)), g.t((64,)), g.t((64,))
    m = g.node("MUL", [a, b], g.t((64,)))
    s = g.node("ADD", [m, c], g.t((64,)))
    r = g.node("LEAKY_RELU", [s], g.t((64,)))
    ng = g.node("NEG", [r], g.t((64,)))
    y = g.node("EXP", [ng], g.t((64,)))
    k, dag, nodes = g.run()
    assert k == 1 and dag.count == 1 and nodes[0].op_type == abi.OP["FUSED_ELEMENTWISE"]
    f = nodes[0]
    assert f.num_inputs == 3 and C.addressof(f.output.contents) == C.addressof(y)
    assert y.creator == C.addressof(f)
    tp = _tape(f)
    ops = [abi.TAPE_OPS[tp.ins[i].op] for i in range(tp.num_ins)]
    assert ops == ["LOAD", "MUL", "ADD", "LEAKY_RELU", "NEG", "EXP"]
    assert [tp.ins[i].idx for i in range(3)] == [0, 1, 2]


def test_fusion_pass_respects_consumers_grads_and_shapes():
    from plast_amd.runtime import Library
    L = Library()
    # an intermediate with a second consumer ends the chain
    g = _MetaGraph(L)
    a, b = g.t((8,)), g.t((8,))
    m = g.node("MUL", [a, b], g.t((8,)))
    e = g.node("EXP", [m], g.t((8,)))
    g.node("ADD", [e, m], g.t((8,)))
    k, dag, nodes = g.run()
    assert k == 1 and [n.op_type for n in nodes] == [abi.OP["MUL"], abi.OP["FUSED_ELEMENTWISE"]]
    tp = _tape(nodes[1])
    # EXP then ADD with the MUL output as external input: acc = exp(m); acc = acc + m
    assert [abi.TAPE_OPS[tp.ins[i].op] for i in range(tp.num_ins)] == ["LOAD", "EXP", "ADD"]
    # requires_grad blocks fusion
    g = _MetaGraph(L)
    a = g.t((8,), grad=True)
    g.node("NEG", [g.node("EXP", [a], g.t((8,), grad=True))], g.t((8,), grad=True))
    assert g.run()[0] == 0
    # a broadcasting intermediate (shape change) ends the chain
    g = _MetaGraph(L)
    x, row = g.t((4, 8)), g.t((8,))
    e = g.node("EXP", [row], g.t((8,)))
    g.node("ADD", [x, e], g.t((4, 8)))
    assert g.run()[0] == 0
    # sub with the accumulator on the right keeps operand order
    g = _MetaGraph(L)
    a, b = g.t((8,)), g.t((8,))
    e = g.node("EXP", [a], g.t((8,)))
    g.node("SUB", [b, e], g.t((8,)))
    k, dag, nodes = g.run()
    tp = _tape(nodes[0])
    assert k == 1 and tp.ins[2].acc_rhs == 1 and tp.ins[2].idx == 1
