"""Benchmark of the MI355X elementwise / broadcast / reduction path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c2,c4r,...] [--no-cpu]
    python bench.py --only KEYS --compare LIB1.so,LIB2.so   (builds timed against each other)
    python bench.py --placement adam|epilogue               (a kernel's arrays at set offsets)

Prints ONE JSON line. `value` is config 5 (the largest single-GPU
config): a whole softmax-cross-entropy training step over [32768, 32000] fp32 logits - the forward's
row max, log-sum-exp and loss, the backward (softmax - onehot)/N and the bias gradient (the sum over
rows of that gradient) - as achieved HBM GB/s (algorithmic bytes / time) through the one-pass step
entry point. Inputs are resident in HBM before timing. Every other config (and config 5 as three
separate passes) is measured in `detail` with its own GB/s, fraction of the 8 TB/s peak and
elements/s. The CPU baselines are the reference's own CPU kernels (oracle/_ref/libplast_ref.so,
compiled from the reference's sources; OpenMP on this host's online cores, whose count is reported)
on bounded samples of the same workloads.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from plast_amd import abi  # noqa: E402
from plast_amd.abi import DIM_ALL, FLOAT32, INT32, INT64, KernelParams  # noqa: E402
from plast_amd.graph import Graph  # noqa: E402
from plast_amd.runtime import DeviceTensor, forward, backward, lib  # noqa: E402

PEAK_GBS = 8000.0
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"] if (ROOT / "BASELINE.json").exists() else \
    "achieved HBM GB/s (% of MI355X peak) + elems/s for elementwise/broadcast/reduce"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def timed(fn, steps: int, warmup: int, warm_ms: float = 0.0) -> float:
    """Average device milliseconds per call of fn, from HIP events on the library stream, after
    `warmup` untimed calls, continued (for the detail rows) until `warm_ms` of wall time have
    passed: an MI355X idle for a while runs the first few milliseconds of work about 2% slower
    (the headline measured 1.434 ms per step right after its setup or a 2 s pause, 1.407-1.408
    once warm, in one process)."""
    L = lib()
    for _ in range(warmup):
        fn()
    if warm_ms > 0:
        L.plast_hip_synchronize()
        t0 = time.perf_counter()
        n = 0
        while (time.perf_counter() - t0) * 1e3 < warm_ms and n < 10000:
            fn()
            n += 1
            if n % 8 == 0:
                L.plast_hip_synchronize()
    L.plast_hip_synchronize()
    L.plast_hip_timer_begin()
    for _ in range(steps):
        fn()
    ms = L.plast_hip_timer_end()
    L.check("timed region")
    return ms / steps


class BenchCall(C.Structure):
    """One entry-point call for bench_calls.c's bench_call_loop (same field layout)."""
    _fields_ = [("fn", C.c_void_p), ("inputs", C.c_void_p), ("output", C.c_void_p),
                ("params", KernelParams)]


_HELPER: list = []


def bench_helper():
    """bench_calls.so (built by plast_amd/build.py:build_bench_helper), or None when absent."""
    if not _HELPER:
        p = ROOT / "bench_calls.so"
        h = C.CDLL(str(p)) if p.exists() else None
        if h is not None:
            h.bench_call_loop.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
            h.bench_call_loop.restype = C.c_double
        _HELPER.append(h)
    return _HELPER[0]


# ----------------------------------------------------------------------------- workloads
class Workload:
    name = ""
    desc = ""
    bytes_per_call = 0
    elems = 0
    min_steps = 0  # a floor on the timed calls (warm-up: a tenth of it)

    def setup(self):
        ...

    def step(self):
        ...

    def rebind(self):
        """Take the current build's entry points where setup() stored some (a graph's op slots);
        the buffers stay."""

    def cpu(self):
        return None

    def free(self):
        for v in list(vars(self).values()):
            if isinstance(v, DeviceTensor):
                v.free()


class C2Fused(Workload):
    """Config 2: out = relu(a*b + c); y = exp(-out) over flat [67108864], a, b, c ~ N(0,1)."""
    name = "config2_fused_chain_64M"
    N = 1 << 26

    def __init__(self, fused=True):
        self.fused = fused
        if not fused:
            self.name = "config2_unfused_5_launches"
        self.elems = self.N
        # fused: 3 reads + 1 write; unfused: 3+3+2+2+2 tensor passes
        self.bytes_per_call = (4 if fused else 12) * 4 * self.N

    def setup(self):
        n = self.N
        self.a = DeviceTensor((n,), zero=False).fill_("normal", 42, 0.0, 1.0)
        self.b = DeviceTensor((n,), zero=False).fill_("normal", 43, 0.0, 1.0)
        self.c = DeviceTensor((n,), zero=False).fill_("normal", 44, 0.0, 1.0)
        self.t = [DeviceTensor((n,), zero=False) for _ in range(4)]
        self.y = DeviceTensor((n,), zero=False)
        self.rebind()

    def rebind(self):
        g = Graph()
        m = g.node("mul", [self.a, self.b], self.t[0])
        s = g.node("add", [m, self.c], self.t[1])
        r = g.node("leaky_relu", [s], self.t[2], KernelParams(0, 0, 0.0))
        ng = g.node("neg", [r], self.t[3])
        g.node("exp", [ng], self.y)
        self.nfused = g.build(self.y, fuse=self.fused)
        self.g = g
        self.kinds = g.op_types()

    def step(self):
        self.g.forward()

    def check(self, k=1 << 20):
        """Max ulp distance of the first k outputs from the oracle (bench-side sanity check; the
        chain's only inexact op is exp, allowed 2 ulp)."""
        sys.path.insert(0, str(ROOT / "tests"))
        from hostlib import fused_chain2
        a = self.a.numpy()[:k]
        b = self.b.numpy()[:k]
        c = self.c.numpy()[:k]
        want = fused_chain2(a, b, c)
        got = self.y.numpy()[:k]
        ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        return int(ulp.max())

    def cpu_from(self, head_inputs=None, budget_s=6.0):
        """The CPU baseline of config 2 for the detail block: its own inputs, generated here."""
        self.setup()
        try:
            return self.cpu(budget_s=budget_s, min_reps=2)
        finally:
            self.free()

    def cpu(self, budget_s=10.0, min_reps=3):
        """The reference's unfused chain (MUL, ADD, LEAKY_RELU, NEG, EXP) through its CPU kernels,
        repeated for about `budget_s` seconds of CPU work (at least `min_reps` times)."""
        sys.path.insert(0, str(ROOT / "tests"))
        from hostlib import HostTensor, ref_available, ref_forward, oracle_forward
        n = self.N
        a, b, c = self.a.numpy(), self.b.numpy(), self.c.numpy()
        kind = "reference" if ref_available() else "port"
        fwd = ref_forward if ref_available() else oracle_forward
        A, B, Cc = HostTensor(a), HostTensor(b), HostTensor(c)
        T = [HostTensor(np.empty(n, np.float32)) for _ in range(5)]
        times = []
        t_start = time.perf_counter()
        while len(times) < min_reps or time.perf_counter() - t_start < budget_s:
            t0 = time.perf_counter()
            fwd("mul", [A, B], T[0])
            fwd("add", [T[0], Cc], T[1])
            fwd("leaky_relu", [T[1]], T[2], KernelParams(0, 0, 0.0))
            fwd("neg", [T[2]], T[3])
            fwd("exp", [T[3]], T[4])
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        gbs = 4 * 4 * n / med / 1e9
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": kind,
                "sample": f"full config-2 workload (64M fp32), unfused reference chain MUL, ADD, "
                          f"LEAKY_RELU, NEG, EXP through the reference's own CPU kernels "
                          f"(oracle/_ref, compiled from its sources), {len(times)} repetitions in "
                          f"{time.perf_counter() - t_start:.1f} s, median; its contiguous elementwise "
                          f"kernels carry no OpenMP pragma, so one core runs them; GB/s counts the "
                          f"fused algorithmic bytes (16 B/element)",
                "ms": round(med * 1e3, 2), "best_ms": round(min(times) * 1e3, 2),
                "elems_per_s": round(n / med, 1)}


class C1(Workload):
    """Config 1: Y = relu(X + b), X [1024,256], b [256] ~ U(-1,1); grad_b = sum_0 grad_Y. "big":
    the same fused chain over [16384, 4096] (a layer of realistic width, through the tape
    interpreter's rows form). "dag" / "dagbig": the training step as the executor runs it - an
    ADD and a LEAKY_RELU node with X and b requiring grad, fused by the elementwise-chain pass into
    one node, then the graph's forward (Y) and backward (dX += 0 + dY * (Y > 0), grad_b += its
    column sum, one pass) - at config 1's shape and at [16384, 4096]."""

    def __init__(self, part):
        self.part = part
        self.name = {"fwd": "config1_bias_relu_fwd_fused", "bwd": "config1_grad_b_sum_axis0",
                     "graph": "config1_step_fwd_bwd_graph",
                     "big": "bias_relu_fused_16384x4096",
                     "dag": "config1_step_dag_fused_fwd_bwd",
                     "dagbig": "bias_relu_step_dag_16384x4096"}[part]
        self.dag = part in ("dag", "dagbig")
        self.rows, self.cols = (16384, 4096) if part in ("big", "dagbig") else (1024, 256)
        # calls of a few microseconds: enough of them that the timed region is not a handful of
        # host round trips
        self.min_steps = 0 if part in ("big", "dagbig") else 500
        self.elems = self.rows * self.cols
        n, c = self.elems, self.cols
        fwd, bwd = n * 8 + c * 4, n * 4 + c * 4
        # the DAG's backward: dY and Y read, dX read and written, grad_b read and written
        dag_bwd = n * 16 + c * 8
        self.bytes_per_call = {"fwd": fwd, "bwd": bwd, "graph": fwd + bwd, "big": fwd,
                               "dag": fwd + dag_bwd, "dagbig": fwd + dag_bwd}[part]

    def setup(self):
        R, Cn = self.rows, self.cols
        g = self.dag
        self.X = DeviceTensor((R, Cn), requires_grad=g, zero=False).fill_("uniform", 42, -1.0, 1.0)
        self.b = DeviceTensor((Cn,), requires_grad=g, zero=False).fill_("uniform", 43, -1.0, 1.0)
        self.gy = DeviceTensor((R, Cn), zero=False).fill_("uniform", 44, -1.0, 1.0)
        self.Y = DeviceTensor((R, Cn), requires_grad=g, zero=False)
        self.gb = DeviceTensor((Cn,), zero=False)
        if self.dag:
            self.S = DeviceTensor((R, Cn), requires_grad=True, zero=False)
            self.Y.grad.fill_("uniform", 44, -1.0, 1.0)
        from plast_amd.ops import make_tape
        self.tape = make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", abi.SRC_INPUT, 1, 0, 0.0),
                               ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)

        self.graph = None
        self.g = None
        self.rebind()

    def rebind(self):
        if self.dag:
            # the executor's graph over this build's op slots, fused by this build's pass
            self.g = Graph()
            self.g.node("add", [self.X, self.b], self.S)
            self.g.node("leaky_relu", [self.S], self.Y, KernelParams(0, 0, 0.0))
            if self.g.build(self.Y, fuse=True) != 1 or self.g.op_types() != ["FUSED_ELEMENTWISE"]:
                raise SystemExit(f"bench.py: the pass did not fuse config 1's step: "
                                 f"{self.g.op_types()}")
            return
        if self.part != "graph":
            return
        if self.graph:
            self.graph_lib.plast_hip_graph_destroy(self.graph)
            self.graph = None
        # the forward and backward ops recorded once and replayed as one graph launch
        import gc
        self.eager_step()
        gc.collect()
        L = self.graph_lib = lib()
        if L.plast_hip_capture_begin() != 0:
            raise SystemExit("bench.py: graph capture failed")
        try:
            self.eager_step()
        finally:
            self.graph = L.plast_hip_capture_end()
        L.check("capture")

    def eager_step(self):
        forward("fused_elementwise", [self.X, self.b], self.Y,
                KernelParams(C.addressof(self.tape), 0, 0.0))
        forward("sum", [self.gy], self.gb, KernelParams(0, 0, 0.0))

    def call(self):
        """(op, inputs, output, params) of the one entry-point call a step of fwd, big or bwd is."""
        if self.part in ("fwd", "big"):
            return ("fused_elementwise", [self.X, self.b], self.Y,
                    KernelParams(C.addressof(self.tape), 0, 0.0))
        return "sum", [self.gy], self.gb, KernelParams(0, 0, 0.0)

    def step(self):
        if self.dag:
            self.g.forward()
            self.g.backward()
        elif self.part == "graph":
            if lib().plast_hip_graph_launch(self.graph) != 0:
                raise SystemExit("bench.py: graph launch failed")
        else:
            forward(*self.call())

    def c_us(self, calls: int = 5000, reps: int = 3):
        """Wall microseconds per call when a C loop (bench_calls.c) makes the calls back to back,
        the library asynchronous and its stream drained at the end: what a C caller such as the
        reference's executor pays per call, without Python's cost. Best of `reps` loops; None for
        the graph and big workloads or without bench_calls.so."""
        h = bench_helper()
        if h is None or self.part not in ("fwd", "bwd"):
            return None
        L = lib()
        name, ins, out, p = self.call()
        arr = (abi.TensorP * len(ins))(*[x.p for x in ins])
        bc = BenchCall(C.cast(L.entry["forward", name], C.c_void_p).value, C.addressof(arr),
                       C.addressof(out.t), p)
        sync = C.cast(L._L.plast_hip_synchronize, C.c_void_p).value
        errors = C.cast(L._L.plast_hip_error_count, C.c_void_p).value
        L.plast_hip_synchronize()
        best = None
        for i in range(reps + 1):  # the first loop warms up
            n = calls // 10 if i == 0 else calls
            us = h.bench_call_loop(C.byref(bc), 1, n, sync, errors)
            if us < 0:
                L.check("bench_call_loop")
                raise SystemExit("bench.py: the C call loop failed")
            if i:
                best = us / n if best is None else min(best, us / n)
        return round(best, 2)

    def kernel_us(self, calls: int = 100, reps: int = 5):
        """Device microseconds per call without the host's per-call cost: `calls` back-to-back
        calls captured as one graph, replayed `reps` times (the graph launch is spread over the
        calls). None for the graph workload itself."""
        if self.part not in ("fwd", "bwd", "dag"):
            return None
        import gc
        L = lib()
        self.step()  # sizes the workspaces outside the capture
        gc.collect()  # no tensor of an earlier workload is freed inside the capture
        if L.plast_hip_capture_begin() != 0:
            raise SystemExit("bench.py: graph capture failed")
        try:
            for _ in range(calls):
                self.step()
        finally:
            g = L.plast_hip_capture_end()
        L.check("capture")
        try:
            ms = timed(lambda: L.plast_hip_graph_launch(g), reps, 2)
        finally:
            L.plast_hip_graph_destroy(g)
        return round(ms * 1e3 / calls, 2)

    def free(self):
        if getattr(self, "graph", None):
            self.graph_lib.plast_hip_graph_destroy(self.graph)
            self.graph = None
        super().free()


class C3(Workload):
    """Config 3: (permute(A,(0,2,1)) + B) * C, A [256,512,512] ~ N(0,1), B [1,512,1], C [256,1,512]."""

    def __init__(self, part):
        self.part = part
        self.name = {"fused": "config3_permuted_bcast_fused", "add": "config3_add_permuted",
                     "mul": "config3_mul_bcast"}[part]
        n = 256 * 512 * 512
        self.elems = n
        self.bytes_per_call = {"fused": 4 * n * 2 + 2048 + 524288,
                               "add": 4 * n * 2 + 2048, "mul": 4 * n * 2 + 524288}[part]

    def setup(self):
        from plast_amd.ops import make_tape
        self.Ab = DeviceTensor((256, 512, 512), zero=False).fill_("normal", 42, 0.0, 1.0)
        self.Av = DeviceTensor((256, 512, 512), base=self.Ab, strides=(262144, 1, 512), zero=False)
        self.B = DeviceTensor((1, 512, 1), zero=False).fill_("uniform", 43, 0.5, 1.5)
        self.Cm = DeviceTensor((256, 1, 512), zero=False).fill_("uniform", 44, 0.5, 1.5)
        self.T = DeviceTensor((256, 512, 512), zero=False)
        self.O = DeviceTensor((256, 512, 512), zero=False)
        self.tape = make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", abi.SRC_INPUT, 1, 0, 0.0),
                               ("MUL", abi.SRC_INPUT, 2, 0, 0.0)], 3)
        if self.part == "mul":
            forward("add", [self.Av, self.B], self.T)

    def step(self):
        if self.part == "fused":
            forward("fused_elementwise", [self.Av, self.B, self.Cm], self.O,
                    KernelParams(C.addressof(self.tape), 0, 0.0))
        elif self.part == "add":
            forward("add", [self.Av, self.B], self.T)
        else:
            forward("mul", [self.T, self.Cm], self.O)


class C4(Workload):
    """Config 4: X [65536,4096] row sum/mean/max/argmax; X^T-shaped [4096,65536] axis-0 sum/max."""

    def __init__(self, op, axis):
        """axis 1: per row, 0: over the leading axis, None: the whole tensor (dim == 9)."""
        self.op, self.axis = op, axis
        self.name = f"config4_{op}_{ {1: 'rows', 0: 'axis0', None: 'all'}[axis] }"
        n = 65536 * 4096
        nout = 1 if axis is None else 65536
        self.elems = n
        self.bytes_per_call = 4 * n + nout * (8 if op == "argmax" else 4)

    def setup(self):
        shape = (65536, 4096) if self.axis != 0 else (4096, 65536)
        self.X = DeviceTensor(shape, zero=False).fill_("normal", 42, 0.0, 1.0)
        nout = 1 if self.axis is None else 65536
        self.out = DeviceTensor((nout,), INT64 if self.op == "argmax" else FLOAT32, zero=False)
        self.p = KernelParams(DIM_ALL if self.axis is None else self.axis, 0, 0.0)

    def step(self):
        forward(self.op, [self.X], self.out, self.p)


class C5(Workload):
    """Config 5: logits [32768,32000] ~ N(0,2), labels U{0..31999}: CE fwd, bwd, bias-grad sum; and
    softmax over the same logits (one read, one write: 8 B/element) and its backward (y, dy and
    the accumulated dx read, dx written: 16 B/element); and the reference chain's individual ops
    on the logits: MAX and SUM over dim 1 with keepdim (4 B/element + 4 B/row), EXP (8 B/element)."""

    def __init__(self, part):
        self.part = part
        self.name = {"fwd": "config5_softmax_ce_fwd", "bwd": "config5_ce_bwd_accumulate",
                     "bwd_w": "config5_ce_bwd_overwrite", "bias": "config5_bias_grad_sum_axis0",
                     "softmax": "softmax_last_axis_32768x32000",
                     "softmax_bwd": "softmax_backward_last_axis_32768x32000",
                     "op_max": "config5_op_max_dim1", "op_exp": "config5_op_exp",
                     "op_sum": "config5_op_sum_dim1"}[part]
        N, Cn = 32768, 32000
        self.elems = N * Cn
        x = 4 * N * Cn
        self.bytes_per_call = {"fwd": x + 3 * 4 * N, "bwd": 3 * x + 3 * 4 * N,
                               "bwd_w": 2 * x + 3 * 4 * N, "bias": x + 4 * Cn,
                               "softmax": 2 * x, "softmax_bwd": 4 * x,
                               "op_max": x + 4 * N, "op_exp": 2 * x, "op_sum": x + 4 * N}[part]

    def setup(self):
        N, Cn = 32768, 32000
        self.X = DeviceTensor((N, Cn), FLOAT32,
                              requires_grad=self.part in ("bwd", "bwd_w", "softmax_bwd"),
                              zero=False).fill_("normal", 42, 0.0, 2.0)
        self.lab = DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
        self.st = DeviceTensor((N, 2), zero=False)
        self.loss = DeviceTensor((N,), requires_grad=True, zero=False)
        if self.part in ("bwd", "bwd_w"):
            forward("softmax_cross_entropy", [self.X, self.lab, self.st], self.loss)
            self.loss.grad.fill_("uniform", 7, 1.0 / N, 1.0 / N)
        if self.part == "bias":
            self.G = DeviceTensor((N, Cn), zero=False).fill_("normal", 46, 0.0, 1e-4)
            self.gb = DeviceTensor((Cn,), zero=False)
        if self.part in ("softmax", "softmax_bwd"):
            self.Y = DeviceTensor((N, Cn), requires_grad=self.part == "softmax_bwd", zero=False)
        if self.part == "softmax_bwd":
            forward("softmax", [self.X], self.Y, KernelParams(1, 0, 0.0))
            self.Y.grad.fill_("normal", 47, 0.0, 1.0)
        if self.part in ("op_max", "op_sum"):
            self.R = DeviceTensor((N, 1), zero=False)
        if self.part == "op_exp":
            self.Y = DeviceTensor((N, Cn), zero=False)

    def step(self):
        if self.part == "fwd":
            forward("softmax_cross_entropy", [self.X, self.lab, self.st], self.loss)
        elif self.part == "bwd":
            backward("softmax_cross_entropy", [self.X, self.lab, self.st], self.loss)
        elif self.part == "bwd_w":
            backward("softmax_cross_entropy", [self.X, self.lab, self.st], self.loss,
                     KernelParams(0, 1, 0.0))
        elif self.part == "bias":
            forward("sum", [self.G], self.gb, KernelParams(0, 0, 0.0))
        elif self.part == "softmax":
            forward("softmax", [self.X], self.Y, KernelParams(1, 0, 0.0))
        elif self.part in ("op_max", "op_sum"):
            forward(self.part[3:], [self.X], self.R, KernelParams(1, 1, 0.0))
        elif self.part == "op_exp":
            forward("exp", [self.X], self.Y)
        else:
            backward("softmax", [self.X], self.Y, KernelParams(1, 0, 0.0))


class C5Step(Workload):
    """Config 5's whole training step in one pass (softmax_cross_entropy_step_hip): logits
    [32768, 32000] ~ N(0, 2), labels U{0..31999}, dloss = 1/N (the mean's gradient); writes the
    row statistics and loss, dlogits = dloss * (softmax - onehot), dbias = sum_rows dlogits and
    the mean loss (the chain's MEAN, the scalar the reference's loss returns).
    Algorithmic bytes: the logits read once and dlogits written once (8 B/element), labels, dloss,
    loss (4 B/row each), stats (8 B/row), dbias (4 B/column), the loss read again for its mean
    (4 B/row) and the mean (4 B); the workgroups' column-sum partials (256 x 32000 x 4 B written
    and read) are workspace, not counted."""
    name = "config5_ce_step_one_pass"

    def __init__(self):
        self.N, self.C = 32768, 32000
        self.elems = self.N * self.C
        self.bytes_per_call = (8 * self.elems + 4 * self.N * 3 + 8 * self.N + 4 * self.C +
                               4 * self.N + 4)

    def setup(self):
        N, Cn = self.N, self.C
        self.X = DeviceTensor((N, Cn), zero=False).fill_("normal", 42, 0.0, 2.0)
        self.lab = DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
        self.g = DeviceTensor((N,), zero=False).fill_("uniform", 7, 1.0 / N, 1.0 / N)
        self.st = DeviceTensor((N, 2), zero=False)
        self.loss = DeviceTensor((N,), zero=False)
        self.dx = DeviceTensor((N, Cn), zero=False)
        self.db = DeviceTensor((Cn,), zero=False)
        self.mean = DeviceTensor((1,), zero=False)

    def step(self):
        lib().softmax_cross_entropy_step_hip(self.X.ptr, self.lab.ptr, self.g.ptr, self.st.ptr,
                                             self.loss.ptr, self.dx.ptr, self.db.ptr,
                                             self.mean.ptr, self.N, self.C)


class Optim(Workload):
    """Optimizer row: one step of SGD / Adam / AdamW over `count` fp32 parameters totalling 64M
    elements (gradients ~ N(0, 0.1)), or zero_grad of a 64M gradient. Bytes per element: SGD reads
    p, g and writes p (12 B); Adam/AdamW read p, g, m, v and write p, m, v (28 B); zero_grad writes
    4 B."""

    def __init__(self, kind, count=1):
        self.kind, self.count = kind, count
        # zero_grad writes only: a 1 GiB gradient, larger than the 256 MB last-level cache
        self.elems = 1 << 28 if kind == "zero_grad" else 1 << 26
        self.name = (f"optim_{kind}_{self.elems >> 20}M" if count == 1 else
                     f"optim_{kind}_{count}x{self.elems // count}")
        self.bytes_per_call = self.elems * {"sgd": 12, "adam": 28, "adamw": 28, "zero_grad": 4}[kind]

    def setup(self):
        n = self.elems // self.count
        self.params = [DeviceTensor((n,), requires_grad=True, zero=False).fill_("normal", 50 + i, 0.0, 1.0)
                       for i in range(self.count)]
        for i, t in enumerate(self.params):
            t.grad.fill_("normal", 900 + i, 0.0, 0.1)
        self.ptrs, self._keep = abi.tensor_array(*[t.t for t in self.params])
        if self.kind == "sgd":
            self.opt = abi.SGD(1e-3)
        elif self.kind == "adam":
            self.opt = abi.Adam(1e-3, 0.9, 0.999, 1e-8, 0, None, None, None, None)
        elif self.kind == "adamw":
            self.opt = abi.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01, 0, None, None, None, None)
        if self.kind in ("adam", "adamw"):
            # zero moments owned by the bench (the library uses caller-set m and v as given), so
            # that builds timed against each other in one process update the same buffers
            self.moments = [[DeviceTensor((n,)) for _ in range(self.count)] for _ in range(2)]
            self._marr = [(abi.TensorP * self.count)(*[C.pointer(t.t) for t in ms])
                          for ms in self.moments]
            self.opt.m = C.cast(self._marr[0], abi.TensorPP)
            self.opt.v = C.cast(self._marr[1], abi.TensorPP)

    def step(self):
        L = lib()
        if self.kind == "zero_grad":
            for t in self.params:
                L.zero_grad_hip(C.byref(t.t))
        else:
            getattr(L, f"{self.kind}_step_hip")(C.byref(self.opt), self.ptrs, self.count)

    def free(self):
        for t in self.params + [t for ms in getattr(self, "moments", []) for t in ms]:
            t.free()


class Pack(Workload):
    """Pack row: config 3's permuted view, A_base [256,512,512] as permute (0,2,1), gathered into a
    contiguous buffer (hip_tensor_pack_init; 256 MiB read + 256 MiB written), or copied to pinned
    host memory in row-major order (plast_hip_tensor_to_host: pack, then a device-to-host copy of
    256 MiB over the host link; its GB/s counts the 256 MiB delivered)."""

    def __init__(self, part):
        self.part = part
        self.name = {"pack": "pack_permuted_256x512x512", "host": "to_host_permuted_256x512x512"}[part]
        self.elems = 256 * 512 * 512
        self.bytes_per_call = self.elems * (8 if part == "pack" else 4)

    def setup(self):
        self.Ab = DeviceTensor((256, 512, 512), zero=False).fill_("normal", 42, 0.0, 1.0)
        self.Av = DeviceTensor((256, 512, 512), base=self.Ab, strides=(262144, 1, 512), zero=False)
        self.host = lib().plast_hip_host_alloc(self.elems * 4) if self.part == "host" else None

    def step(self):
        L = lib()
        if self.part == "pack":
            # the released buffer returns to the library's pack pool, so each call reuses it
            p = abi.HipTensorPack()
            L.hip_tensor_pack_init(C.byref(p), C.byref(self.Av.t))
            L.hip_tensor_pack_release(C.byref(p))
        else:
            L.plast_hip_tensor_to_host(C.byref(self.Av.t), self.host)

    def plain_copy(self, steps: int, warmup: int) -> dict:
        """The host link's ceiling for this row: a plain device-to-host copy of the same 256 MiB
        from a contiguous device buffer into the same page-locked host buffer (one
        hipMemcpyAsync on the library's stream, then a synchronize)."""
        L = lib()
        n = self.elems * 4
        ms = timed(lambda: (L.arena_memcpy_d2h_hip(self.host, self.Ab.ptr, n),
                            L.plast_hip_synchronize()), steps, warmup)
        return {"ms": round(ms, 4), "GB_s": round(n / (ms * 1e-3) / 1e9, 2)}

    def free(self):
        if self.host:
            lib().plast_hip_host_free(self.host)
            self.host = None
        lib().plast_hip_pack_trim()
        super().free()


class Epilogue(Workload):
    """Matmul-epilogue row on a [16384, 4096] output: the leaky-relu gradient modulation
    dc = dout * (out > 0 ? 1 : alpha) (reads dout, out; writes dc: 12 B/element), the bias
    gradient column sum of dc into [4096] (4 B/element + 16 KiB), and both in one pass
    (12 B/element + 16 KiB: dc is not read back)."""

    def __init__(self, part):
        self.part = part
        self.name = {"mod": "epilogue_relu_grad_modulate_16384x4096",
                     "bias": "epilogue_bias_grad_16384x4096",
                     "fused": "epilogue_modulate_and_bias_grad_one_pass_16384x4096"}[part]
        self.M, self.N = 16384, 4096
        self.elems = self.M * self.N
        self.bytes_per_call = {"mod": self.elems * 12, "bias": self.elems * 4 + self.N * 4,
                               "fused": self.elems * 12 + self.N * 4}[part]

    def setup(self):
        M, N = self.M, self.N
        self.dout = DeviceTensor((M, N), zero=False).fill_("normal", 60, 0.0, 1.0)
        self.out = DeviceTensor((M, N), zero=False).fill_("normal", 61, 0.0, 1.0)
        self.dc = DeviceTensor((M, N), zero=False).fill_("normal", 62, 0.0, 1.0)
        self.db = DeviceTensor((N,), zero=False)

    def step(self):
        L = lib()
        if self.part == "mod":
            L.launch_relu_grad_modulate_hip(self.dout.ptr, self.out.ptr, self.dc.ptr, self.elems,
                                            0.01, 0, 0)
        elif self.part == "bias":
            L.bias_grad_reduce_hip(self.dc.ptr, self.db.ptr, self.elems, self.N)
        else:
            L.relu_grad_modulate_bias_grad_hip(self.dout.ptr, self.out.ptr, self.dc.ptr,
                                               self.db.ptr, self.elems, self.N, 0.01)


class Copy(Workload):
    """float4 device copy of 256 MiB: the measured bandwidth ceiling."""
    name = "copy_256MiB"

    def __init__(self):
        self.elems = 1 << 26
        self.bytes_per_call = 8 * self.elems

    def setup(self):
        self.src = DeviceTensor((self.elems,), zero=False).fill_("uniform", 1, 0, 1)
        self.dst = DeviceTensor((self.elems,), zero=False)

    def step(self):
        lib().plast_hip_copy(self.dst.ptr, self.src.ptr, self.elems)


# ----------------------------------------------------------------------------- CPU baselines
def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _cpu_lib():
    """(kind, forward, backward, HostTensor) for the reference's compiled CPU kernels, or the
    oracle's restatement where the reference was not built."""
    sys.path.insert(0, str(ROOT / "tests"))
    import hostlib
    if hostlib.ref_available():
        return "reference", hostlib.ref_forward, hostlib.ref_backward, hostlib.HostTensor
    return "port", hostlib.oracle_forward, hostlib.oracle_backward, hostlib.HostTensor


def _repeat(fn, budget_s, min_reps=2):
    """Median seconds of fn over repetitions filling about budget_s (at least min_reps)."""
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times), time.perf_counter() - t_start


def cpu_config5(X, lab, budget_s=12.0, rows=256):
    """The reference's cross-entropy step on the host: the op chain of src/api/loss.c:97-169 (MAX,
    SUB, EXP, SUM, LOG, SUB, MUL one-hot, SUM, NEG, MEAN), its backward in reverse node order, and
    the bias gradient through its ADD backward (kernel_macros.h:283-299, omp atomics into [C]),
    over row chunks of the same logits (a full [32768, 32000] chain needs ~10 x 4 GiB of
    intermediates)."""
    kind, fwd, bwd, HT = _cpu_lib()
    sys.path.insert(0, str(ROOT / "tests"))
    import hostlib
    N, Cn = X.shape
    chunks = []
    for k in range(4):          # four row chunks spread over the logits, read back once
        r0 = (k * N // 4) // rows * rows
        chunks.append((X.rows_numpy(r0, rows), lab.numpy()[r0:r0 + rows]))
    which = "ref" if kind == "reference" else "oracle"
    state = {"i": 0}

    def one():
        x, y = chunks[state["i"] % len(chunks)]
        state["i"] += 1
        *_, dx = hostlib.ref_ce_chain(x, y, which, backward=True)
        z = HT(x)
        b = HT(np.zeros(Cn, np.float32), requires_grad=True)
        out = HT(np.zeros((rows, Cn), np.float32), requires_grad=True)
        out.grad.buf[:] = dx.reshape(-1)
        bwd("add", [z, b], out)

    med, reps, spent = _repeat(one, budget_s)
    per_row = med / rows
    bytes_per_row = 8 * Cn + 24  # the step's bytes per row, its mean loss's read included
    return {"value": round(bytes_per_row / per_row / 1e9, 3), "unit": "GB/s", "kind": kind,
            "ms_full_step": round(per_row * N * 1e3, 1), "rows_per_s": round(1 / per_row, 1),
            "sample": f"{reps} chunks of {rows} rows x {Cn} of the same logits in {spent:.1f} s, "
                      f"median; GB/s counts the one-pass step's algorithmic bytes per row "
                      f"({bytes_per_row} B); ms_full_step extrapolates to {N} rows; the "
                      f"reference's CPU sources built by oracle/Makefile with -O3 -mavx2 -fopenmp "
                      f"-ffp-contract=off (its own Makefile:7 has -O3 -march=native -fopenmp)"}


def cpu_config1(budget_s=3.0):
    """relu(X + b) (ADD's broadcast path: omp; LEAKY_RELU: one thread) and grad_b = SUM over axis
    0 (the dim reduction: omp over outputs) on the full [1024, 256] config."""
    kind, fwd, bwd, HT = _cpu_lib()
    rng = np.random.RandomState(42)
    X = HT(rng.uniform(-1, 1, (1024, 256)).astype(np.float32))
    b = HT(rng.uniform(-1, 1, 256).astype(np.float32))
    gy = HT(rng.uniform(-1, 1, (1024, 256)).astype(np.float32))
    S, Y, gb = (HT(np.zeros(s, np.float32)) for s in ((1024, 256), (1024, 256), (256,)))
    f_ms, _, _ = _repeat(lambda: (fwd("add", [X, b], S),
                                  fwd("leaky_relu", [S], Y, KernelParams(0, 0, 0.0))), budget_s / 2, 20)
    b_ms, _, _ = _repeat(lambda: fwd("sum", [gy], gb, KernelParams(0, 0, 0.0)), budget_s / 2, 20)
    return {"fwd_us": round(f_ms * 1e6, 1), "grad_b_us": round(b_ms * 1e6, 1), "kind": kind,
            "sample": "full config-1 shapes, median of repeated calls"}


def cpu_config3(budget_s=4.0, batches=32):
    """(permute(A, (0,2,1)) + B) * C through the reference's broadcast binary path (omp over
    output elements with per-element index math) on the first `batches` of the 256 batches."""
    kind, fwd, bwd, HT = _cpu_lib()
    rng = np.random.RandomState(42)
    base = HT(rng.randn(batches, 512, 512).astype(np.float32))
    A = HT(base=base, shape=(batches, 512, 512), strides=(262144, 1, 512))
    B = HT(rng.uniform(0.5, 1.5, (1, 512, 1)).astype(np.float32))
    Cm = HT(rng.uniform(0.5, 1.5, (batches, 1, 512)).astype(np.float32))
    T, O = HT(np.zeros((batches, 512, 512), np.float32)), HT(np.zeros((batches, 512, 512), np.float32))
    med, reps, spent = _repeat(lambda: (fwd("add", [A, B], T), fwd("mul", [T, Cm], O)), budget_s)
    n = batches * 512 * 512
    return {"value": round(8 * n / med / 1e9, 3), "unit": "GB/s (fused algorithmic bytes)",
            "kind": kind, "ms_full": round(med * 256 / batches * 1e3, 1),
            "sample": f"{batches} of 256 batches, add then mul, {reps} repetitions in {spent:.1f} s"}


def cpu_config4(budget_s=4.0, rows=8192, cols0=16384):
    """SUM and MAX over the last axis of [rows, 4096] (the dim reduction: omp over rows) and over
    axis 0 of [4096, cols0] (each output walks 4096 rows at a stride of cols0 floats)."""
    kind, fwd, bwd, HT = _cpu_lib()
    rng = np.random.RandomState(42)
    X = HT(rng.randn(rows, 4096).astype(np.float32))
    XT = HT(rng.randn(4096, cols0).astype(np.float32))
    r_out, c_out = HT(np.zeros(rows, np.float32)), HT(np.zeros(cols0, np.float32))
    res = {"kind": kind}
    for op in ("sum", "max"):
        med, _, _ = _repeat(lambda: fwd(op, [X], r_out, KernelParams(1, 0, 0.0)), budget_s / 4)
        res[f"{op}_rows_GB_s"] = round(4 * rows * 4096 / med / 1e9, 3)
        med, _, _ = _repeat(lambda: fwd(op, [XT], c_out, KernelParams(0, 0, 0.0)), budget_s / 4)
        res[f"{op}_axis0_GB_s"] = round(4 * 4096 * cols0 / med / 1e9, 3)
    res["sample"] = f"rows: [{rows}, 4096] of [65536, 4096]; axis 0: [4096, {cols0}] of [4096, 65536]"
    return res


def detail_workloads():
    return {
        "copy": Copy(),
        "c1f": C1("fwd"), "c1b": C1("bwd"), "c1g": C1("graph"), "c1big": C1("big"),
        "c1dag": C1("dag"), "c1dagbig": C1("dagbig"),
        "c2f": C2Fused(True), "c2u": C2Fused(False),
        "c3f": C3("fused"), "c3a": C3("add"), "c3m": C3("mul"),
        "c4sum": C4("sum", 1), "c4mean": C4("mean", 1), "c4max": C4("max", 1),
        "c4argmax": C4("argmax", 1), "c4csum": C4("sum", 0), "c4cmax": C4("max", 0),
        "c4asum": C4("sum", None), "c4amax": C4("max", None),
        "c5f": C5("fwd"), "c5b": C5("bwd"), "c5bw": C5("bwd_w"), "c5bias": C5("bias"),
        "c5softmax": C5("softmax"), "c5softmaxb": C5("softmax_bwd"),
        "c5max": C5("op_max"), "c5exp": C5("op_exp"), "c5sum": C5("op_sum"),
        "c5step": C5Step(),
        "optsgd": Optim("sgd"), "optadam": Optim("adam"), "optadamw": Optim("adamw"),
        "optadam512": Optim("adam", 512), "zerograd": Optim("zero_grad"),
        "pack": Pack("pack"), "tohost": Pack("host"),
        "epimod": Epilogue("mod"), "epibias": Epilogue("bias"),
        "epifused": Epilogue("fused"),
    }


# --no-graphs: eager launches only (no graph capture or replay, no C call loop), for runs under a
# tracer
NO_GRAPHS = False


def measure(w: Workload, steps: int, warmup: int) -> dict:
    w.setup()
    steps, warmup = max(steps, w.min_steps), max(warmup, w.min_steps // 10)
    ms = timed(w.step, steps, warmup, warm_ms=50.0)
    gbs = w.bytes_per_call / (ms * 1e-3) / 1e9
    r = {"ms": round(ms, 4), "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
         "elems_per_s": round(w.elems / (ms * 1e-3), 1), "algorithmic_bytes": w.bytes_per_call}
    if isinstance(w, Pack) and w.part == "host":
        # the same bytes through a plain copy of a contiguous buffer: the link's ceiling
        c = w.plain_copy(steps, warmup)
        r["plain_d2h_copy"] = c
        r["frac_of_plain_d2h_copy"] = round(c["ms"] / ms, 4)
    if isinstance(w, C1) and w.part not in ("big", "dagbig"):
        # latency-bound: microseconds per call as a Python caller and a C caller see them, and on
        # the device alone
        r["us_per_call"] = round(ms * 1e3, 2)
        if NO_GRAPHS:
            return r
        k = w.kernel_us()
        if k is not None:
            r["kernel_us_per_call"] = k
        c = w.c_us()
        if c is not None:
            r["c_caller_us_per_call"] = c
    return r


def check_step(w: "C5Step", rows=64) -> dict:
    """Bench-side parity of the headline: `rows` sampled rows against the oracle's cross-entropy
    (row max bit-exact; log-sum-exp, loss and dlogits at 1e-5 relative), the step's bias
    gradient against the library's own leading-axis sum of its dlogits (a separate kernel) at
    1e-5 of sum |dlogits| per column, and the mean loss against the float64 mean of the step's
    per-row losses at 1e-5 of mean |loss|."""
    sys.path.insert(0, str(ROOT / "tests"))
    from hostlib import HostTensor, oracle_backward, oracle_forward
    N, Cn = w.N, w.C
    idx = np.random.RandomState(5).choice(N, rows, replace=False)
    worst = {"stats_max_bits": 0, "lse": 0.0, "loss": 0.0, "dlogits": 0.0, "dbias": 0.0}
    st, lo, g = w.st.numpy(), w.loss.numpy(), w.g.numpy()
    lab = w.lab.numpy()
    for r in idx:
        x = w.X.rows_numpy(int(r), 1)
        hx, hl = HostTensor(x, requires_grad=True), HostTensor(lab[r:r + 1])
        hs, ho = HostTensor(np.zeros((1, 2), np.float32)), HostTensor(np.zeros(1, np.float32), requires_grad=True)
        oracle_forward("softmax_cross_entropy", [hx, hl, hs], ho)
        ho.grad.buf[:] = g[r]
        oracle_backward("softmax_cross_entropy", [hx, hl, hs], ho)
        ws = hs.numpy().reshape(2)
        worst["stats_max_bits"] += int(np.float32(st[r, 0]).view(np.uint32) != np.float32(ws[0]).view(np.uint32))
        worst["lse"] = max(worst["lse"], abs(float(st[r, 1]) - float(ws[1])) / (abs(float(ws[1])) + 1e-6))
        worst["loss"] = max(worst["loss"], abs(float(lo[r]) - float(ho.numpy()[0])) /
                            (abs(float(ho.numpy()[0])) + abs(float(ws[1])) + 1e-6))
        d = w.dx.rows_numpy(int(r), 1).astype(np.float64)
        wd = hx.grad.numpy().astype(np.float64)
        worst["dlogits"] = max(worst["dlogits"], float(np.max(np.abs(d - wd) / (np.abs(wd) + 1e-2 / N))))
    L = lib()
    ref_bias = DeviceTensor((Cn,), zero=False)
    L.bias_grad_reduce_hip(w.dx.ptr, ref_bias.ptr, N * Cn, Cn)
    L.check("bias sum")
    db, rb = w.db.numpy().astype(np.float64), ref_bias.numpy().astype(np.float64)
    ref_bias.free()
    # sum over rows of |dlogits| per column: with dlogits = g (softmax - onehot) and g = 1/N it is at
    # most |dbias| + 2 count / N (count: the rows labelled with that column)
    count = np.bincount(lab, minlength=Cn).astype(np.float64)
    scale = np.abs(db) + 2.0 * count * float(g.max()) + 1e-30
    worst["dbias"] = float(np.max(np.abs(db - rb) / scale))
    # the mean loss against the float64 mean of the step's own per-row losses
    mean, want = float(w.mean.numpy()[0]), float(lo.astype(np.float64).mean())
    worst["mean_loss"] = abs(mean - want) / (float(np.abs(lo).astype(np.float64).mean()) + 1e-30)
    worst["ok"] = (worst["stats_max_bits"] == 0 and worst["lse"] <= 1e-5 and worst["loss"] <= 1e-5
                   and worst["dlogits"] <= 1e-5 and worst["dbias"] <= 1e-5
                   and worst["mean_loss"] <= 1e-5)
    return worst


def compare_builds(a) -> int:
    """Library builds timed against each other in ONE process: the same box, the same process
    state and the same input buffers (rates of one kernel differ by a few percent from one process
    or box to the next, which a comparison across processes would mistake for the variants').
    Seven passes over one set of buffers; in each, every build times every --only workload in
    turn. Prints one JSON line: per build and workload, the GB/s of each pass and their median."""
    from plast_amd.runtime import load_library, use_library
    keys = [k for k in a.only.split(",") if k]
    if not keys:
        raise SystemExit("bench.py: --compare needs --only")
    base = lib()
    base.plast_hip_set_sync(0)
    builds = []
    for p in a.compare.split(","):
        L = load_library(Path(p))
        L.plast_hip_set_sync(0)
        builds.append((Path(p).name, L))
    # one set of buffers for every build: where the buffers land moves a kernel's rate by a few
    # percent, so fresh allocations per build would mix that into the comparison
    work = [detail_workloads()[k] for k in keys]
    for w in work:
        w.setup()
    res = {tag: {w.name: [] for w in work} for tag, _ in builds}
    try:
        for _ in range(7):
            for tag, L in builds:
                use_library(L)
                for w in work:
                    w.rebind()
                    steps = max(a.steps, w.min_steps)
                    # calls of a few microseconds: device time per call (calls replayed from a
                    # graph), which the host's per-call cost would otherwise hide
                    k = w.kernel_us() if isinstance(w, C1) else None
                    ms = k * 1e-3 if k is not None else timed(w.step, steps, max(a.warmup, 2))
                    res[tag][w.name].append(round(w.bytes_per_call / (ms * 1e-3) / 1e9, 1))
                    log(f"{tag} {w.name}: {res[tag][w.name][-1]} GB/s")
    finally:
        use_library(base)
        for w in work:
            w.rebind()
            w.free()
    print(json.dumps({"compare": {tag: {n: {"GB_s": v, "median": float(np.median(v))}
                                        for n, v in r.items()} for tag, r in res.items()}}),
          flush=True)
    return 0


def placement_probe(kind: str) -> int:
    """The relative placement of a kernel's arrays as the variable: Adam over 64M parameters (p,
    g, m, v) or the one-pass epilogue over [16384, 4096] (dout, out, dc), with the arrays carved
    from one allocation 2^26 floats plus 16 MiB of slack apart and array k shifted by k times a
    skew (1 KiB to 4 MiB; for the epilogue also dc first, then out, then dout). Two passes in one
    process; prints one JSON line of GB/s (algorithmic bytes / HIP-event time) per placement."""
    L = lib()
    L.plast_hip_set_sync(0)
    n, pad = 1 << 26, 1 << 22
    arrays = {"adam": 4, "epilogue": 3}[kind]
    big = DeviceTensor((arrays * (n + pad),), zero=False).fill_("normal", 7, 0.0, 1.0)
    keep = []
    if kind == "adam":
        def call(ptr):
            g = abi.make_tensor(ptr[1], (n,))
            prm = abi.make_tensor(ptr[0], (n,), requires_grad=True, grad=g)
            m, v = abi.make_tensor(ptr[2], (n,)), abi.make_tensor(ptr[3], (n,))
            marr, varr = (abi.TensorP * 1)(C.pointer(m)), (abi.TensorP * 1)(C.pointer(v))
            opt = abi.Adam(1e-3, 0.9, 0.999, 1e-8, 0, None, None, None, None)
            opt.m, opt.v = C.cast(marr, abi.TensorPP), C.cast(varr, abi.TensorPP)
            parr = (abi.TensorP * 1)(C.pointer(prm))
            keep[:] = [g, prm, m, v, marr, varr, opt, parr]
            pp = C.cast(parr, abi.TensorPP)
            return lambda: L.adam_step_hip(C.byref(opt), pp, 1)
        bytes_per = 28
    else:
        db = DeviceTensor((4096,), zero=False)
        keep.append(db)

        def call(ptr):
            return lambda: L.relu_grad_modulate_bias_grad_hip(ptr[0], ptr[1], ptr[2], db.ptr, n,
                                                              4096, 0.01)
        bytes_per = 12
    cases = {"aligned": [0] * arrays}
    for kb in (1, 2, 4, 8, 16, 64, 256, 1024, 4096):
        cases[f"{kb}K skew"] = [k * kb * 256 for k in range(arrays)]
    if kind == "epilogue":
        cases["dc first"] = [2 * (n + pad), -(n + pad), -(n + pad)]
    res = {name: [] for name in cases}
    for _ in range(2):
        for name, skews in cases.items():
            ptr = [big.ptr + 4 * (k * (n + pad) + sk) for k, sk in enumerate(skews)]
            ms = timed(call(ptr), 20, 5, warm_ms=30.0)
            res[name].append(round(bytes_per * n / (ms * 1e-3) / 1e9, 1))
            log(f"{kind} {name}: {res[name][-1]} GB/s")
    big.free()
    print(json.dumps({"placement": kind, "GB_s": res}), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 50 steps of the headline are ~70 ms of GPU work: enough for an idle GPU to reach its
    # steady clocks before the timed region (see timed())
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--only", default="", help="comma list of detail keys (default: all)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-graphs", action="store_true",
                    help="eager launches only: skip the graph-replayed and C-loop timings and the "
                         "graph workload (for runs under a kernel tracer)")
    ap.add_argument("--placement", default="", choices=["", "adam", "epilogue"],
                    help="time one kernel with its arrays at chosen relative offsets in one "
                         "allocation (a placement probe) and print its JSON line")
    ap.add_argument("--compare", default="",
                    help="comma list of library builds (plast_amd.build --out): time the --only "
                         "workloads with each in turn in this process and print their medians")
    a = ap.parse_args(argv)
    global NO_GRAPHS
    NO_GRAPHS = a.no_graphs
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (no collective or multi-GPU path is "
              "built); run with --gpus 1", file=sys.stderr)
        return 2
    if a.placement:
        return placement_probe(a.placement)
    if a.compare:
        return compare_builds(a)
    cores = host_cores()
    # the reference's CPU kernels use OpenMP: every online core of this host, stated in the line
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))

    L = lib()
    L.plast_hip_set_sync(0)  # order on the library stream; timing brackets synchronise

    # ---- headline: config 5's whole training step, one pass
    head = C5Step()
    head.setup()
    ms = timed(head.step, a.steps, a.warmup)
    gbs = head.bytes_per_call / (ms * 1e-3) / 1e9
    L.plast_hip_synchronize()
    log(f"config5 step: {ms:.4f} ms/step, {gbs:.1f} GB/s")

    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get(head.name)
        except Exception:
            traffic = None

    cpu, cpu_detail, parity = None, {}, None
    if not a.no_cpu:
        # the CPU leg: the oracle checks sampled rows of the timed step's outputs, then is timed
        parity = check_step(head)
        log(f"config5 step parity: {parity}")
        if not parity["ok"]:
            raise SystemExit(f"bench.py: config 5 step differs from the oracle: {parity}")
        cpu = cpu_config5(head.X, head.lab)
        cpu["cores"] = int(os.environ["OMP_NUM_THREADS"])
        log(f"cpu baseline (config 5): {cpu}")
        for name, fn in (("config1", cpu_config1), ("config3", cpu_config3),
                         ("config4", cpu_config4)):
            try:
                cpu_detail[name] = fn()
            except Exception as e:  # report, keep going
                cpu_detail[name] = {"error": str(e)}
            log(f"cpu baseline ({name}): {cpu_detail[name]}")
        cpu_detail["config2"] = C2Fused(True).cpu_from(head_inputs=None)
    head.free()

    detail = {}
    if not a.no_detail:
        keys = [k for k in a.only.split(",") if k] or [k for k in detail_workloads() if k != "c5step"]
        if a.no_graphs:
            keys = [k for k in keys if k != "c1g"]
        for k in keys:
            w = detail_workloads()[k]
            try:
                detail[w.name] = measure(w, max(3, a.steps // 2), 2)
                log(f"{w.name}: {detail[w.name]}")
            except Exception as e:  # report, keep measuring the rest
                detail[w.name] = {"error": str(e)}
                log(f"{w.name}: ERROR {e}")
            finally:
                w.free()
        three = [detail.get(n, {}).get("ms") for n in ("config5_softmax_ce_fwd",
                                                       "config5_ce_bwd_overwrite",
                                                       "config5_bias_grad_sum_axis0")]
        if all(isinstance(t, float) for t in three):
            detail["config5_step_as_three_passes"] = {
                "ms": round(sum(three), 4), "passes": ["forward", "backward (overwrite)",
                                                       "bias gradient sum"],
                "speedup_of_one_pass": round(sum(three) / ms, 3)}
    head_detail = {"ms": round(ms, 4), "GB_s": round(gbs, 1), "parity": parity,
                   "launches_per_step": 2,
                   "kernels": ["ce_step_kernel", "ce_step_tail"]}

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: on-device counter-based PRNG, logits ~ N(0, 2) seed 42, labels "
                "U{0..31999} seed 45, dloss = 1/N",
        "config": {"workload": "config5: softmax cross-entropy training step over [32768, 32000] "
                               "fp32 logits - row max, log-sum-exp, loss, dlogits = (softmax - "
                               "onehot)/N and the [32000] bias gradient - in one pass "
                               "(softmax_cross_entropy_step_hip)",
                   "rows": head.N, "classes": head.C,
                   "algorithmic_bytes_per_step": head.bytes_per_call},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "elems_per_s": round(head.elems / (ms * 1e-3), 1),
        "detail": {"config5_step_one_pass": head_detail,
                   "traffic_source": "profiles/traffic.json (FETCH_SIZE + WRITE_SIZE of the "
                                     "dominant kernel per launch, calibrated on the copy kernel)",
                   "cpu_baselines": cpu_detail, **detail},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
