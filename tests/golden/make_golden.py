"""Write tests/golden/reference_cases.npz: inputs and outputs of every case in tests/cases.py, as
computed by the reference's own CPU library (oracle/_ref/libplast_ref.so, compiled from
/root/reference's C sources by oracle/Makefile). Cases for argmax (no reference op) are omitted.

    python tests/golden/make_golden.py

The fixture is data only (arrays); it lets the oracle be checked where the reference tree is absent.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

from cases import CASES, materialize, run_case  # noqa: E402
from hostlib import HostBackend, ref_available  # noqa: E402

OUT = HERE / "reference_cases.npz"


def key(case_id: str) -> str:
    return re.sub(r"[^A-Za-z0-9_.-]+", "_", case_id)


def main() -> int:
    if not ref_available():
        print("oracle/_ref/libplast_ref.so is not built (needs /root/reference)", file=sys.stderr)
        return 1
    arrays = {}
    for c in CASES:
        if c.op == "argmax":
            continue
        k = key(c.id)
        for i, a in enumerate(c.inputs):
            arrays[f"{k}@in{i}"] = a.base_array()
        for name, v in run_case(HostBackend("ref"), c).items():
            arrays[f"{k}@{name}"] = v
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
