// ops.cpp — the GPU op table and the elementwise-chain fusion pass (host code only).
#include <cstring>
#include <vector>

#include "../../include/plast_hip.h"
#include "fused_grad.hpp"

namespace {

// Fills the GPU slots as the reference's X-macro does for its CUDA slots (src/core/op.c:9-49,
// include/core/ops.def:1-28). View ops run their metadata forward on the host for either device,
// as the reference's OP_CPU entries do.
Op make_op(OP_TYPE t) {
  Op op;
  memset(&op, 0, sizeof op);
  switch (t) {
#define SLOT(ENUM, name)                                                                           \
  case ENUM:                                                                                       \
    op.gpu_forward = name##_hip_forward;                                                           \
    op.gpu_backward = name##_hip_backward;                                                         \
    break;
    SLOT(ADD, add)
    SLOT(SUB, sub)
    SLOT(MUL, mul)
    SLOT(DIV, div)
    SLOT(LEAKY_RELU, leaky_relu)
    SLOT(LOG, log)
    SLOT(EXP, exp)
    SLOT(ABS, abs)
    SLOT(NEG, neg)
    SLOT(SIN, sin)
    SLOT(COS, cos)
    SLOT(TAN, tan)
    SLOT(VIEW, view)
    SLOT(TRANSPOSE, transpose)
    SLOT(UNSQUEEZE, unsqueeze)
    SLOT(SQUEEZE, squeeze)
    SLOT(EXPAND, expand)
    SLOT(FLATTEN, flatten)
    SLOT(BROADCAST, broadcast)
    SLOT(MEAN, mean)
    SLOT(MIN, min)
    SLOT(MAX, max)
    SLOT(SUM, sum)
    SLOT(ARGMAX, argmax)
    SLOT(FUSED_ELEMENTWISE, fused_elementwise)
    SLOT(SOFTMAX_CROSS_ENTROPY, softmax_cross_entropy)
    SLOT(SOFTMAX, softmax)
    SLOT(LOG_SOFTMAX, log_softmax)
#undef SLOT
  default:
    break;  // MATMUL, CONV2D and their fused epilogues have no GPU slot here
  }
  return op;
}

bool is_binary(OP_TYPE t) { return t == ADD || t == SUB || t == MUL || t == DIV; }
bool is_unary(OP_TYPE t) {
  return t == LEAKY_RELU || t == EXP || t == LOG || t == NEG || t == ABS || t == SIN || t == COS ||
         t == TAN;
}

u8 tape_op(OP_TYPE t) {
  switch (t) {
  case ADD: return TAPE_ADD;
  case SUB: return TAPE_SUB;
  case MUL: return TAPE_MUL;
  case DIV: return TAPE_DIV;
  case LEAKY_RELU: return TAPE_LEAKY_RELU;
  case EXP: return TAPE_EXP;
  case LOG: return TAPE_LOG;
  case NEG: return TAPE_NEG;
  case ABS: return TAPE_ABS;
  case SIN: return TAPE_SIN;
  case COS: return TAPE_COS;
  default: return TAPE_TAN;
  }
}

bool same_shape(const Tensor *a, const Tensor *b) {
  if (a->ndim != b->ndim) return false;
  for (u64 d = 0; d < a->ndim; ++d)
    if (a->shape[d] != b->shape[d]) return false;
  return true;
}

// A node the pass may place in a chain: a GPU fp32 elementwise op with nothing requiring grad
// (the only fused chain with a backward is the leaky_relu(x + bias) pair below).
bool fusable(const Node *n) {
  if (!is_binary(n->op_type) && !is_unary(n->op_type)) return false;
  if (n->num_inputs != (is_binary(n->op_type) ? 2 : 1)) return false;
  const Tensor *o = n->output;
  if (!o || o->device != GPU || o->dtype != FLOAT32 || o->requires_grad) return false;
  for (int i = 0; i < n->num_inputs; ++i) {
    const Tensor *t = n->inputs[i];
    if (!t || t->device != GPU || t->dtype != FLOAT32 || t->requires_grad) return false;
  }
  return true;
}

// A member of the fused leaky_relu(x + bias) pair: fp32 GPU tensors, gradients allowed.
bool grad_pair_member(const Node *n) {
  if (!plast::fused_grad::gpu_f32(n->output)) return false;
  for (int i = 0; i < n->num_inputs; ++i)
    if (!plast::fused_grad::gpu_f32(n->inputs[i])) return false;
  return true;
}

struct Chain {
  std::vector<u32> idx;  // positions in dag->nodes, increasing
  std::vector<Tensor *> ext;
  PlastFusedTape tape;
};

int ext_slot(Chain &c, Tensor *t) {
  for (size_t k = 0; k < c.ext.size(); ++k)
    if (c.ext[k] == t) return int(k);
  if (c.ext.size() >= PLAST_TAPE_MAX_INPUTS) return -1;
  c.ext.push_back(t);
  return int(c.ext.size() - 1);
}

// Append node n to the chain's tape given that `acc` (may be null for the first node) holds the
// previous node's output. Returns false if the chain would exceed its limits.
bool append(Chain &c, const Node *n, const Tensor *acc) {
  PlastFusedTape &tp = c.tape;
  if (tp.num_ins + 2 > PLAST_TAPE_MAX_INS) return false;
  Chain saved = c;
  if (!acc) {
    int k = ext_slot(c, n->inputs[0]);
    if (k < 0) return false;
    tp.ins[tp.num_ins++] = PlastTapeIns{TAPE_LOAD, TAPE_SRC_NONE, u8(k), 0, 0.0f};
    if (is_unary(n->op_type)) {
      tp.ins[tp.num_ins++] = PlastTapeIns{tape_op(n->op_type), TAPE_SRC_NONE, 0, 0, n->params.fval};
    } else {
      int k2 = ext_slot(c, n->inputs[1]);
      if (k2 < 0) {
        c = saved;
        return false;
      }
      tp.ins[tp.num_ins++] = PlastTapeIns{tape_op(n->op_type), TAPE_SRC_INPUT, u8(k2), 0, 0.0f};
    }
    return true;
  }
  if (is_unary(n->op_type)) {
    tp.ins[tp.num_ins++] = PlastTapeIns{tape_op(n->op_type), TAPE_SRC_NONE, 0, 0, n->params.fval};
    return true;
  }
  const bool lhs = n->inputs[0] == acc, rhs = n->inputs[1] == acc;
  if (lhs && rhs) {
    tp.ins[tp.num_ins++] = PlastTapeIns{tape_op(n->op_type), TAPE_SRC_ACC, 0, 0, 0.0f};
    return true;
  }
  Tensor *other = lhs ? n->inputs[1] : n->inputs[0];
  int k = ext_slot(c, other);
  if (k < 0) return false;
  tp.ins[tp.num_ins++] =
      PlastTapeIns{tape_op(n->op_type), TAPE_SRC_INPUT, u8(k), u8(lhs ? 0 : 1), 0.0f};
  return true;
}

}  // namespace

extern "C" {

Op plast_hip_get_op_impl(OP_TYPE op_type) { return make_op(op_type); }

u32 plast_hip_fuse_elementwise_chains(DAG *dag, PlastArenaAllocFn alloc) {
  if (!dag || !alloc || dag->count < 2) return 0;
  const u32 n = dag->count;
  Node **nodes = dag->nodes;
  const Tensor *root_out = nodes[n - 1]->output;

  // consumers of each tensor inside the DAG
  auto uses = [&](const Tensor *t) {
    u32 c = 0;
    for (u32 i = 0; i < n; ++i)
      for (int j = 0; j < nodes[i]->num_inputs; ++j)
        if (nodes[i]->inputs[j] == t) ++c;
    return c;
  };
  // position of the (unique) consumer of t, or n
  auto consumer = [&](const Tensor *t, u32 from) {
    for (u32 i = from; i < n; ++i)
      for (int j = 0; j < nodes[i]->num_inputs; ++j)
        if (nodes[i]->inputs[j] == t) return i;
    return n;
  };

  std::vector<bool> taken(n, false);
  std::vector<Chain> chains;
  // leaky_relu(x + bias, alpha >= 0) with gradients: its backward reads the mask from the output,
  // so the intermediate x + bias must feed the leaky node alone (it is never written)
  for (u32 i = 0; i < n; ++i) {
    const Node *a = nodes[i];
    if (a->op_type != ADD || a->num_inputs != 2 || !grad_pair_member(a)) continue;
    const Tensor *t = a->output;
    if (t == root_out) continue;
    const u32 l = consumer(t, i + 1);
    if (l >= n || nodes[l]->op_type != LEAKY_RELU || nodes[l]->num_inputs != 1 ||
        !grad_pair_member(nodes[l]) || uses(t) != 1)
      continue;
    const Tensor *y = nodes[l]->output;
    if (!plast::fused_grad::alpha_ok(nodes[l]->params.fval) || !plast::fused_grad::same_extents(t, y) ||
        plast::fused_grad::x_operand(a->inputs[0], a->inputs[1], y) < 0)
      continue;
    const bool grads = a->inputs[0]->requires_grad || a->inputs[1]->requires_grad;
    if (!grads) continue;  // no gradients: the chain loop below takes it (and may extend it)
    Chain c;
    memset(&c.tape, 0, sizeof c.tape);
    if (!append(c, a, nullptr) || !append(c, nodes[l], t)) continue;
    c.idx = {i, l};
    c.tape.num_inputs = u32(c.ext.size());
    taken[i] = taken[l] = true;
    chains.push_back(c);
  }
  for (u32 i = 0; i < n; ++i) {
    if (taken[i] || !fusable(nodes[i])) continue;
    Chain c;
    memset(&c.tape, 0, sizeof c.tape);
    if (!append(c, nodes[i], nullptr)) continue;
    c.idx.push_back(i);
    u32 cur = i;
    for (;;) {
      const Tensor *out = nodes[cur]->output;
      if (out == root_out) break;
      const u32 nxt = consumer(out, cur + 1);
      if (nxt >= n || taken[nxt] || !fusable(nodes[nxt])) break;
      // the intermediate must feed only this next node, and keep the chain's shape
      u32 in_next = 0;
      for (int j = 0; j < nodes[nxt]->num_inputs; ++j) in_next += nodes[nxt]->inputs[j] == out;
      if (uses(out) != in_next) break;
      if (!same_shape(out, nodes[nxt]->output)) break;
      if (!append(c, nodes[nxt], out)) break;
      c.idx.push_back(nxt);
      cur = nxt;
    }
    if (c.idx.size() < 2) continue;
    // every external input must broadcast to the chain's output shape
    const Tensor *fo = nodes[c.idx.back()]->output;
    bool ok = true;
    for (Tensor *t : c.ext) {
      if (t->ndim > fo->ndim) ok = false;
      for (u64 d = 0; ok && d < t->ndim; ++d) {
        const u64 e = t->shape[t->ndim - 1 - d], f = fo->shape[fo->ndim - 1 - d];
        if (e != f && e != 1) ok = false;
      }
    }
    if (!ok) continue;
    c.tape.num_inputs = u32(c.ext.size());
    for (u32 k : c.idx) taken[k] = true;
    chains.push_back(c);
  }
  if (chains.empty()) return 0;

  // Splice: the fused node takes the slot of the chain's last node (all of the chain's external
  // inputs are produced before it in topological order); the other members are removed.
  std::vector<Node *> replacement(n, nullptr);
  for (const Chain &c : chains) {
    Node *f = static_cast<Node *>(alloc(dag->arena, sizeof(Node), 8));
    Tensor **ins = static_cast<Tensor **>(alloc(dag->arena, sizeof(Tensor *) * c.ext.size(), 8));
    PlastFusedTape *tape = static_cast<PlastFusedTape *>(alloc(dag->arena, sizeof(PlastFusedTape), 8));
    if (!f || !ins || !tape) return 0;
    memset(f, 0, sizeof(Node));
    for (size_t k = 0; k < c.ext.size(); ++k) ins[k] = c.ext[k];
    *tape = c.tape;
    f->inputs = ins;
    f->num_inputs = int(c.ext.size());
    f->output = nodes[c.idx.back()]->output;
    f->op = make_op(FUSED_ELEMENTWISE);
    f->op_type = FUSED_ELEMENTWISE;
    f->params.dim = u64(reinterpret_cast<uintptr_t>(tape));
    f->output->creator = f;
    replacement[c.idx.back()] = f;
  }
  std::vector<bool> drop(n, false);
  for (const Chain &c : chains)
    for (size_t k = 0; k + 1 < c.idx.size(); ++k) drop[c.idx[k]] = true;
  u32 w = 0;
  for (u32 i = 0; i < n; ++i) {
    if (drop[i]) continue;
    nodes[w++] = replacement[i] ? replacement[i] : nodes[i];
  }
  dag->count = w;
  dag->changed = true;
  return u32(chains.size());
}

}  // extern "C"
