"""Build plast_amd/libplast_hip.so for gfx950 with hipcc (and the oracle with make).

    python -m plast_amd.build            # library only
    python -m plast_amd.build --oracle   # also oracle/liboracle.so and oracle/_ref (test checker)
    python -m plast_amd.build -D PLAST_ADAM_BLOCK=256 --out /tmp/adam256.so   # a tuning variant

Objects go to plast_amd/_build/; the shared library is written in-tree so it travels with the
repository snapshot to the GPU box. A variant (launch-shape knobs of csrc/common.hpp set with -D)
is built in its own object folder into --out, and is loaded instead of the in-tree library by
setting PLAST_HIP_LIB to its path.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libplast_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("PLAST_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: every reference operation is separately rounded (no a*b+c -> FMA).
# -packed-fp32-ops off: keep fp32 math on scalar VALU forms.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-pragmas",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l and "ignoring feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_library(jobs: int | None = None, defines: list[str] | None = None,
                  out: Path | None = None) -> Path:
    defines = list(defines or [])
    lib = Path(out).resolve() if out else LIB
    build = BUILD
    if defines or out:
        build = PKG / ("_build_" + lib.stem)
    build.mkdir(exist_ok=True)
    flags = HIP_FLAGS + [f"-D{d}" for d in defines]
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    cmds = []
    objs = []
    for src in sources:
        obj = build / (src.stem + ".o")
        objs.append(obj)
        if src.suffix == ".hip":
            cmds.append([HIPCC, *flags, "-c", str(src), "-o", str(obj)])
        else:
            cmds.append(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{ROOT / 'include'}",
                         "-c", str(src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, lib)
    return lib


def build_bench_helper() -> Path:
    """bench_calls.so: bench.py's C loop that times entry-point calls without Python (gcc; it links
    nothing and runs no GPU code of its own)."""
    out = ROOT / "bench_calls.so"
    tmp = out.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", f"-I{ROOT / 'include'}",
          str(ROOT / "bench_calls.c"), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_oracle() -> None:
    """Test infrastructure: the C restatement and, when /root/reference exists, the reference."""
    make = shutil.which("make") or "make"
    subprocess.run([make, "-s", "-C", str(ROOT / "oracle"), "all"], check=True)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--oracle", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-D", dest="defines", action="append", default=[],
                    help="NAME=VALUE for a launch-shape knob (a variant; needs --out)")
    ap.add_argument("--out", type=Path, default=None, help="variant library path")
    a = ap.parse_args(argv)
    if a.defines and not a.out:
        ap.error("-D builds a variant: give it --out so the in-tree library stays the default")
    print(build_library(a.j, a.defines, a.out))
    if not a.out:
        print(build_bench_helper())
    if a.oracle:
        build_oracle()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
