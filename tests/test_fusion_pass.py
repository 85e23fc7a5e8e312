"""The elementwise-chain fusion pass (plast_hip_fuse_elementwise_chains, plast_amd/csrc/ops.cpp) on
the host, under the address and undefined-behaviour sanitizers: tests/fusion_fuzz.cpp builds
thousands of random DAGs (chains, fan-out, broadcast inputs, x*x, nodes the pass must leave alone),
checks the rewritten DAG's structure and that every tensor it still produces keeps its values bit
for bit (fused nodes evaluated by a restatement of the tape's semantics). The pass is linked
against no-op stand-ins for the kernel entry points its op table names: it only rewrites structs
(no device code is built or run)."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _build(tmp_path, ops_src: str, tag: str) -> Path:
    names = sorted(set(re.findall(r"SLOT\(\w+, (\w+)\)", ops_src)))
    assert "add" in names and "fused_elementwise" in names
    stubs = ['#include "plast_hip.h"', 'extern "C" {']
    for n in names:
        stubs.append(f"void {n}_hip_forward(const Tensor **, Tensor *, KernelParams) {{}}")
        stubs.append(f"void {n}_hip_backward(Tensor **, const Tensor *, KernelParams) {{}}")
    stubs.append("}")
    (tmp_path / "stubs.cpp").write_text("\n".join(stubs) + "\n")
    ops = tmp_path / f"ops_{tag}.cpp"
    ops.write_text(ops_src)
    exe = tmp_path / f"fusion_fuzz_{tag}"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Werror",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                    f"-I{ROOT / 'include'}", str(ops), str(tmp_path / "stubs.cpp"),
                    str(ROOT / "tests" / "fusion_fuzz.cpp"), "-o", str(exe)], check=True)
    return exe


def _ops_src() -> str:
    # the pass as committed; its include is made absolute so a copy elsewhere builds the same
    return (ROOT / "plast_amd" / "csrc" / "ops.cpp").read_text().replace(
        '"../../include/plast_hip.h"', '"plast_hip.h"').replace(
        '"fused_grad.hpp"', f'"{ROOT / "plast_amd" / "csrc" / "fused_grad.hpp"}"')


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fusion_pass_fuzz(tmp_path):
    exe = _build(tmp_path, _ops_src(), "committed")
    r = subprocess.run([str(exe), "3000"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
    trials, fused, grad_pairs = map(int, r.stdout.split()[1:4])
    assert fused > trials // 4, f"only {fused} chains fused over {trials} DAGs: the DAGs rarely chain"
    assert grad_pairs > 20, f"only {grad_pairs} leaky_relu(x + bias) pairs with gradients fused"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fusion_fuzz_catches_a_swapped_operand(tmp_path):
    """A copy of the pass that never marks the accumulator as the right operand (so b - acc
    would be taped as acc - b) must fail the harness."""
    src = _ops_src()
    planted = src.replace("u8(lhs ? 0 : 1)", "u8(0)")
    assert planted != src
    exe = _build(tmp_path, planted, "planted")
    r = subprocess.run([str(exe), "3000"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "differs after fusion" in r.stdout, r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fusion_fuzz_catches_a_negative_slope_pair(tmp_path):
    """A copy of the pass that fuses leaky_relu(x + bias) with gradients for any slope (whose
    backward could not read its mask from the output when the slope is negative) must fail the
    harness."""
    src = _ops_src()
    planted = src.replace("!plast::fused_grad::alpha_ok(nodes[l]->params.fval) ||", "")
    assert planted != src
    exe = _build(tmp_path, planted, "slope")
    r = subprocess.run([str(exe), "3000"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "not leaky_relu(x + bias)" in r.stdout, r.stdout
