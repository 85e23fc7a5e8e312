"""Write tests/golden/optimizer_cases.npz: parameters and moments after three SGD / Adam / AdamW
steps computed by the reference's own CPU optimizers (oracle/_ref/libplast_ref.so, compiled from
/root/reference's src/optimizers/cpu sources by oracle/Makefile), for the parameter sets of
tests/optim_cases.py. Inputs are regenerated from the same seeds, so the fixture holds outputs only.

    python tests/golden/make_golden_optim.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

from hostlib import ref_available  # noqa: E402
from optim_cases import MANY, SIZES  # noqa: E402
from test_optim import run_host  # noqa: E402

OUT = HERE / "optimizer_cases.npz"


def main() -> int:
    if not ref_available():
        print("oracle/_ref/libplast_ref.so is not built (needs /root/reference)", file=sys.stderr)
        return 1
    arrays = {}
    for set_name, sizes in (("shapes", SIZES), ("many", MANY)):
        with_grad = [i % 5 != 3 for i in range(len(sizes))]
        for kind in ("sgd", "adam", "adamw"):
            ps, mv, _ = run_host("ref", kind, sizes, 11, 3, with_grad)
            for i, p in enumerate(ps):
                arrays[f"{set_name}@{kind}@p{i}"] = p
                if mv is not None:
                    arrays[f"{set_name}@{kind}@m{i}"] = mv[i][0]
                    arrays[f"{set_name}@{kind}@v{i}"] = mv[i][1]
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
