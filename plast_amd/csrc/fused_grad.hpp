// fused_grad.hpp — the fused chain that carries a gradient: leaky_relu(x + bias, alpha) over a
// row-major x and a row-major bias row, alpha >= 0 (host code, plain C++, shared by the fusion
// pass in ops.cpp and the fused node's backward in epilogue.hip). For alpha >= 0 the chain's
// output y is > 0 exactly where x + bias is, so the backward takes its mask from y and the
// intermediate x + bias is never written.
#pragma once

#include "../../include/plast_hip.h"

namespace plast {
namespace fused_grad {

inline bool row_major(const Tensor *t) {
  u64 want = 1;
  for (u64 d = t->ndim; d-- > 0;) {
    if (t->shape[d] != 1 && t->strides[d] != want) return false;
    want *= t->shape[d];
  }
  return true;
}

inline bool gpu_f32(const Tensor *t) { return t && t->device == GPU && t->dtype == FLOAT32; }

inline bool same_extents(const Tensor *a, const Tensor *b) {
  if (a->ndim != b->ndim) return false;
  for (u64 d = 0; d < a->ndim; ++d)
    if (a->shape[d] != b->shape[d]) return false;
  return true;
}

// A bias row for y: y's last extent, 1 on every other axis, no more axes than y.
inline bool bias_row(const Tensor *b, const Tensor *y) {
  if (y->ndim == 0 || b->ndim == 0 || b->ndim > y->ndim) return false;
  if (b->shape[b->ndim - 1] != y->shape[y->ndim - 1]) return false;
  for (u64 d = 0; d + 1 < b->ndim; ++d)
    if (b->shape[d] != 1) return false;
  return true;
}

// Which of the ADD's two operands (0 or 1) is x for output y, the other being the bias; -1 when
// the pair is not (x, bias) or (bias, x) with every tensor fp32 on the GPU and row-major.
inline int x_operand(const Tensor *p, const Tensor *q, const Tensor *y) {
  if (!gpu_f32(p) || !gpu_f32(q) || !gpu_f32(y) || !row_major(y)) return -1;
  for (int k = 0; k < 2; ++k) {
    const Tensor *x = k == 0 ? p : q, *b = k == 0 ? q : p;
    if (same_extents(x, y) && row_major(x) && bias_row(b, y) && row_major(b) && x != b) return k;
  }
  return -1;
}

inline bool alpha_ok(float alpha) { return alpha >= 0.0f; }  // false for NaN as well

// The tape the pass writes for the chain: LOAD in[i]; ADD in[j]; LEAKY_RELU alpha. Gives the
// input slots of the two operands in ADD order (i, j) and alpha.
inline bool is_leaky_bias_tape(const PlastFusedTape &t, u32 *i, u32 *j, float *alpha) {
  if (t.num_inputs != 2 || t.num_ins != 3) return false;
  const PlastTapeIns &l = t.ins[0], &a = t.ins[1], &r = t.ins[2];
  if (l.op != TAPE_LOAD || l.idx >= 2) return false;
  if (a.op != TAPE_ADD || a.src != TAPE_SRC_INPUT || a.idx >= 2 || a.idx == l.idx) return false;
  if (r.op != TAPE_LEAKY_RELU || !alpha_ok(r.imm)) return false;
  *i = l.idx;
  *j = a.idx;
  *alpha = r.imm;
  return true;
}

}  // namespace fused_grad
}  // namespace plast
