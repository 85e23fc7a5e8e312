"""Tapes that exercise every case of the fused-chain interpreter (shared by the GPU parity tests):
each op, each operand source, both operand orders of SUB/DIV, broadcast scalar inputs, the longest
tape, and config 2's chain."""
from __future__ import annotations

from plast_amd.abi import SRC_ACC, SRC_IMM, SRC_INPUT, SRC_NONE

# (name, num_inputs, broadcast mask, instructions (op, src, idx, acc_rhs, imm))
TAPES = [
    ("config2", 3, 0, [("LOAD", 0, 0, 0, 0.0), ("MUL", SRC_INPUT, 1, 0, 0.0),
                       ("ADD", SRC_INPUT, 2, 0, 0.0), ("LEAKY_RELU", SRC_NONE, 0, 0, 0.0),
                       ("NEG", SRC_NONE, 0, 0, 0.0), ("EXP", SRC_NONE, 0, 0, 0.0)]),
    ("sub_div_both_orders", 2, 0, [("LOAD", 0, 1, 0, 0.0), ("SUB", SRC_INPUT, 0, 1, 0.0),
                                   ("DIV", SRC_INPUT, 1, 0, 0.0), ("SUB", SRC_IMM, 0, 0, 0.75),
                                   ("DIV", SRC_IMM, 0, 1, -2.5), ("ADD", SRC_ACC, 0, 0, 0.0)]),
    ("unary_run", 1, 0, [("LOAD", 0, 0, 0, 0.0), ("ABS", SRC_NONE, 0, 0, 0.0),
                         ("LOG", SRC_NONE, 0, 0, 0.0), ("LEAKY_RELU", SRC_NONE, 0, 0, 0.01),
                         ("NEG", SRC_NONE, 0, 0, 0.0), ("EXP", SRC_NONE, 0, 0, 0.0),
                         ("MUL", SRC_ACC, 0, 0, 0.0)]),
    ("trig", 2, 0, [("LOAD", 0, 0, 0, 0.0), ("SIN", SRC_NONE, 0, 0, 0.0),
                    ("ADD", SRC_INPUT, 1, 0, 0.0), ("COS", SRC_NONE, 0, 0, 0.0),
                    ("MUL", SRC_IMM, 0, 0, 0.3), ("TAN", SRC_NONE, 0, 0, 0.0)]),
    ("broadcast_scalars", 4, 0b1010, [("LOAD", 0, 0, 0, 0.0), ("MUL", SRC_INPUT, 1, 0, 0.0),
                                      ("ADD", SRC_INPUT, 2, 0, 0.0), ("DIV", SRC_INPUT, 3, 1, 0.0),
                                      ("NEG", SRC_NONE, 0, 0, 0.0)]),
    ("sixteen", 2, 0, [("LOAD", 0, 0, 0, 0.0)] +
     [("ADD", SRC_INPUT, 1, 0, 0.0), ("MUL", SRC_IMM, 0, 0, 0.5), ("NEG", SRC_NONE, 0, 0, 0.0)] * 5),
]
