"""Test infrastructure: applies the drop-in's scheduler edit to a temporary copy of the
reference's src/scheduler/fusion.c, so that its fusion_optimize (fusion.c:209-224) runs this
library's elementwise-chain pass after its own patterns when built with -DPLAST_HIP. The copy is
written to OUT (a temporary directory the Makefile removes); nothing of the reference is kept.

    python3 hip_fusion_hook.py REF/src/scheduler/fusion.c OUT/fusion.c

The edit adds a declaration of plast_hip_fuse_elementwise_chains in the reference's own types
(include/plast_hip.h declares the same function over the layout-identical plast_abi.h types;
the reference's headers are already in scope in fusion.c) and one call before fusion_optimize
returns, passing the reference's arena_alloc (include/core/arena.h:37) as the allocator for the
fused node and its tape."""
import re
import sys

DECL = """#ifdef PLAST_HIP
/* libplast_hip.so (include/plast_hip.h): fuses GPU elementwise chains of the DAG into
 * FUSED_ELEMENTWISE nodes allocated from dag->arena; returns the number of chains fused. */
u32 plast_hip_fuse_elementwise_chains(DAG *dag, void *(*alloc)(Arena *, u64, u64));
#endif

"""
CALL = """#ifdef PLAST_HIP
  applied += plast_hip_fuse_elementwise_chains(dag, arena_alloc);
#endif
"""


def main(src: str, out: str) -> int:
    text = open(src).read()
    head = re.search(r"^u32 fusion_optimize\(DAG \*dag\) \{$", text, re.M)
    if not head:
        raise SystemExit(f"{src}: fusion_optimize's definition not found")
    body_end = text.find("\n}\n", head.end())
    ret = text.rfind("return applied;", head.end(), body_end)
    if body_end < 0 or ret < 0:
        raise SystemExit(f"{src}: fusion_optimize's final return not found")
    line = text.rfind("\n", 0, ret) + 1
    text = text[:line] + CALL + text[line:]
    text = text[:head.start()] + DECL + text[head.start():]
    with open(out, "w") as f:
        f.write(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1], sys.argv[2]))
