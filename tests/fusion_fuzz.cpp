// Randomised host check of the elementwise-chain fusion pass (plast_hip_fuse_elementwise_chains,
// plast_amd/csrc/ops.cpp), built with the address and undefined-behaviour sanitizers by
// tests/test_fusion_pass.py against no-op kernel stubs (the pass only rewrites structs).
//
// Each trial builds a random DAG in topological order: unary and binary elementwise nodes over
// GPU fp32 tensors of broadcast-compatible shapes, with random fan-out, leaky slopes of either
// sign, gradients required by some leaves (and by every tensor computed from one), and nodes the
// pass must leave alone (an input on the CPU, a non-elementwise op). It
// evaluates the DAG node by node on the host, runs the pass, evaluates the rewritten DAG (fused
// nodes through a restatement of the tape's semantics, include/plast_hip.h: PlastTapeOp) and
// requires:
//   - every tensor the rewritten DAG produces to equal the first evaluation bit for bit (the tape
//     must keep each operand's side of sub and div, and each input's broadcast);
//   - the rewritten DAG to be in topological order, each fused node to have 2..MAX_INS
//     instructions and at most MAX_INPUTS inputs, and the node count to drop by the fused chains'
//     lengths minus one;
//   - no fused node to hold an op the pass must not touch, and a fused node with a gradient to be
//     exactly leaky_relu(x + bias, slope >= 0): x of the output's shape, the bias a row of its
//     last extent (the only chain whose backward the library has).
// Prints "ok <trials> <fused chains> <of them with gradients>" or the first failures, and exits
// non-zero on failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <random>
#include <vector>

#include "plast_hip.h"

namespace {

std::vector<void *> g_arena;  // the pass's allocations, freed after each trial

void *arena_alloc_cb(Arena *, u64 size, u64 align) {
  const size_t a = align < 16 ? 16 : size_t(align);
  void *p = std::aligned_alloc(a, (size_t(size) + a - 1) / a * a);
  g_arena.push_back(p);
  return p;
}

struct T {  // a tensor: its struct, host values and shape as (rows, cols)
  Tensor t;
  std::vector<float> v;
  int rows = 1, cols = 1;
};

int fails = 0;
#define CHECK(cond, ...)                                                                           \
  do {                                                                                             \
    if (!(cond) && fails++ < 5) {                                                                  \
      std::printf("trial %d: ", trial);                                                            \
      std::printf(__VA_ARGS__);                                                                    \
      std::printf("\n");                                                                           \
    }                                                                                              \
  } while (0)

void make(T &x, int rows, int cols, int ndim) {
  memset(&x.t, 0, sizeof x.t);
  x.rows = rows, x.cols = cols;
  x.v.assign(size_t(rows) * cols, 0.0f);
  x.t.data = x.v.data();
  x.t.ndim = u64(ndim);
  if (ndim == 1) {
    x.t.shape[0] = u64(cols), x.t.strides[0] = 1;
  } else {
    x.t.shape[0] = u64(rows), x.t.shape[1] = u64(cols);
    x.t.strides[0] = u64(cols), x.t.strides[1] = 1;
  }
  x.t.dtype = FLOAT32;
  x.t.device = GPU;
}

float at(const T &x, int i, int j) { return x.v[size_t(x.rows == 1 ? 0 : i) * x.cols + (x.cols == 1 ? 0 : j)]; }

float unary(OP_TYPE op, float a, float slope) {
  switch (op) {
  case LEAKY_RELU: return a > 0.0f ? a : a * slope;
  case EXP: return expf(a);
  case LOG: return logf(a);
  case NEG: return -a;
  case ABS: return fabsf(a);
  case SIN: return sinf(a);
  case COS: return cosf(a);
  default: return tanf(a);
  }
}

float binary(OP_TYPE op, float a, float b) {
  switch (op) {
  case ADD: return a + b;
  case SUB: return a - b;
  case MUL: return a * b;
  default: return a / b;
  }
}

OP_TYPE unary_of_tape(u8 op) {
  switch (op) {
  case TAPE_LEAKY_RELU: return LEAKY_RELU;
  case TAPE_EXP: return EXP;
  case TAPE_LOG: return LOG;
  case TAPE_NEG: return NEG;
  case TAPE_ABS: return ABS;
  case TAPE_SIN: return SIN;
  case TAPE_COS: return COS;
  default: return TAN;
  }
}

OP_TYPE binary_of_tape(u8 op) {
  switch (op) {
  case TAPE_ADD: return ADD;
  case TAPE_SUB: return SUB;
  case TAPE_MUL: return MUL;
  default: return DIV;
  }
}

bool is_tape_binary(u8 op) { return op == TAPE_ADD || op == TAPE_SUB || op == TAPE_MUL || op == TAPE_DIV; }

bool same_extents(const Tensor *a, const Tensor *b) {
  if (a->ndim != b->ndim) return false;
  for (u64 d = 0; d < a->ndim; ++d)
    if (a->shape[d] != b->shape[d]) return false;
  return true;
}

// The one fused chain allowed to carry a gradient: LOAD, ADD of the other input, LEAKY_RELU with
// a slope >= 0, over x (the output's extents) and a bias row (the output's last extent, 1 before).
bool leaky_bias_node(const Node *n) {
  const PlastFusedTape *tp = reinterpret_cast<const PlastFusedTape *>(uintptr_t(n->params.dim));
  if (n->num_inputs != 2 || tp->num_ins != 3 || tp->ins[0].op != TAPE_LOAD ||
      tp->ins[1].op != TAPE_ADD || tp->ins[1].src != TAPE_SRC_INPUT ||
      tp->ins[2].op != TAPE_LEAKY_RELU || !(tp->ins[2].imm >= 0.0f))
    return false;
  const Tensor *y = n->output;
  for (int k = 0; k < 2; ++k) {
    const Tensor *x = n->inputs[k], *b = n->inputs[1 - k];
    bool row = b->ndim >= 1 && b->ndim <= y->ndim && b->shape[b->ndim - 1] == y->shape[y->ndim - 1];
    for (u64 d = 0; row && d + 1 < b->ndim; ++d) row = b->shape[d] == 1;
    if (same_extents(x, y) && row) return true;
  }
  return false;
}

// A node of the harness: its struct, and an opaque op the pass may not fuse (evaluated as a copy
// of its input) when `opaque`.
struct N {
  Node n;
  std::vector<Tensor *> ins;
  bool opaque = false;
};

T *owner_of(std::vector<std::unique_ptr<T>> &ts, const Tensor *t) {
  for (auto &x : ts)
    if (&x->t == t) return x.get();
  return nullptr;
}

void eval_node(std::vector<std::unique_ptr<T>> &ts, const Node *n, bool opaque) {
  T *o = owner_of(ts, n->output);
  T *a = owner_of(ts, n->inputs[0]);
  if (n->op_type == FUSED_ELEMENTWISE) {
    const PlastFusedTape *tp = reinterpret_cast<const PlastFusedTape *>(uintptr_t(n->params.dim));
    std::vector<T *> in;
    for (int k = 0; k < n->num_inputs; ++k) in.push_back(owner_of(ts, n->inputs[k]));
    for (int i = 0; i < o->rows; ++i)
      for (int j = 0; j < o->cols; ++j) {
        float acc = 0.0f;
        for (u32 s = 0; s < tp->num_ins; ++s) {
          const PlastTapeIns &ins = tp->ins[s];
          if (ins.op == TAPE_LOAD) {
            acc = at(*in[ins.idx], i, j);
          } else if (is_tape_binary(ins.op)) {
            const float other = ins.src == TAPE_SRC_INPUT ? at(*in[ins.idx], i, j)
                                : ins.src == TAPE_SRC_IMM ? ins.imm
                                                          : acc;
            acc = ins.acc_rhs ? binary(binary_of_tape(ins.op), other, acc)
                              : binary(binary_of_tape(ins.op), acc, other);
          } else {
            acc = unary(unary_of_tape(ins.op), acc, ins.imm);
          }
        }
        o->v[size_t(i) * o->cols + j] = acc;
      }
    return;
  }
  for (int i = 0; i < o->rows; ++i)
    for (int j = 0; j < o->cols; ++j) {
      float r;
      if (opaque) r = at(*a, i, j);
      else if (n->num_inputs == 2) r = binary(n->op_type, at(*a, i, j), at(*owner_of(ts, n->inputs[1]), i, j));
      else r = unary(n->op_type, at(*a, i, j), n->params.fval);
      o->v[size_t(i) * o->cols + j] = r;
    }
}

}  // namespace

int main(int argc, char **argv) {
  const int trials = argc > 1 ? atoi(argv[1]) : 3000;
  std::mt19937 rng(12345);
  auto pick = [&](int n) { return int(rng() % unsigned(n)); };
  const OP_TYPE un[] = {LEAKY_RELU, EXP, LOG, NEG, ABS, SIN, COS, TAN};
  const OP_TYPE bin[] = {ADD, SUB, MUL, DIV};
  long total_fused = 0, grad_pairs = 0;
  for (int trial = 0; trial < trials; ++trial) {
    std::vector<std::unique_ptr<T>> ts;
    std::vector<std::unique_ptr<N>> ns;
    const int R = 1 + pick(4), C = 1 + pick(6);
    // leaves: full, a row, a column, a 1-D row, a scalar; some on the CPU
    const int nleaves = 2 + pick(4);
    std::vector<Tensor *> avail;
    for (int k = 0; k < nleaves; ++k) {
      auto x = std::make_unique<T>();
      const int kind = pick(5);
      if (kind == 0 || kind == 1) make(*x, R, C, 2);
      else if (kind == 2) make(*x, 1, C, 2);
      else if (kind == 3) make(*x, R, 1, 2);
      else make(*x, 1, C, 1);
      for (float &f : x->v) f = float(int(rng() % 2001) - 1000) / 250.0f + (pick(7) == 0 ? 0.0f : 0.5f);
      if (pick(12) == 0) x->t.device = CPU;
      if (pick(5) == 0) x->t.requires_grad = true;
      avail.push_back(&x->t);
      ts.push_back(std::move(x));
    }
    // in some trials an explicit leaky_relu(x + bias) pair first (either operand order, a slope of
    // either sign), which random DAGs rarely hold
    if (pick(3) == 0) {
      Tensor *x = nullptr, *b = nullptr;
      for (Tensor *t : avail) {
        const T *o = owner_of(ts, t);
        if (!x && o->rows == R && o->cols == C && t->ndim == 2) x = t;
        else if (!b && o->rows == 1 && o->cols == C) b = t;
      }
      if (x && b) {
        Tensor *prev = nullptr;
        for (int k = 0; k < 2; ++k) {
          auto nd = std::make_unique<N>();
          memset(&nd->n, 0, sizeof nd->n);
          auto o = std::make_unique<T>();
          make(*o, R, C, 2);
          if (k == 0) {
            nd->n.op_type = ADD;
            nd->ins = pick(2) ? std::vector<Tensor *>{x, b} : std::vector<Tensor *>{b, x};
          } else {
            nd->n.op_type = LEAKY_RELU;
            nd->n.params.fval = 0.01f * float(pick(50) - 10);
            nd->ins = {prev};
          }
          for (Tensor *in : nd->ins) o->t.requires_grad = o->t.requires_grad || in->requires_grad;
          nd->n.inputs = nd->ins.data();
          nd->n.num_inputs = int(nd->ins.size());
          nd->n.output = &o->t;
          nd->n.op = plast_hip_get_op_impl(nd->n.op_type);
          o->t.creator = &nd->n;
          prev = &o->t;
          avail.push_back(&o->t);
          ts.push_back(std::move(o));
          ns.push_back(std::move(nd));
        }
      }
    }
    const int nnodes = 2 + pick(14);
    for (int q = 0; q < nnodes; ++q) {
      auto nd = std::make_unique<N>();
      memset(&nd->n, 0, sizeof nd->n);
      const int kind = pick(10);
      // the latest outputs are likelier operands, so chains form
      auto operand = [&]() {
        const int s = int(avail.size());
        return avail[pick(3) ? s - 1 - pick(s < 3 ? s : 3) : pick(s)];
      };
      Tensor *a = operand();
      T *ta = owner_of(ts, a);
      auto o = std::make_unique<T>();
      if (kind < 4) {  // binary
        Tensor *b = pick(8) == 0 ? a : operand();
        T *tb = owner_of(ts, b);
        const int rows = ta->rows > tb->rows ? ta->rows : tb->rows;
        const int cols = ta->cols > tb->cols ? ta->cols : tb->cols;
        if ((ta->rows != rows && ta->rows != 1) || (tb->rows != rows && tb->rows != 1) ||
            (ta->cols != cols && ta->cols != 1) || (tb->cols != cols && tb->cols != 1)) {
          --q;
          continue;
        }
        make(*o, rows, cols, 2);
        nd->n.op_type = bin[pick(4)];
        nd->ins = {a, b};
      } else {
        make(*o, ta->rows, ta->cols, 2);
        nd->n.op_type = un[pick(8)];
        nd->n.params.fval = 0.01f * float(pick(50) - 10);
        nd->ins = {a};
        if (kind == 9) {  // an op the pass must not fuse (a reduction slot, evaluated as a copy)
          nd->n.op_type = SUM;
          nd->opaque = true;
        }
      }
      for (Tensor *in : nd->ins) o->t.requires_grad = o->t.requires_grad || in->requires_grad;
      nd->n.inputs = nd->ins.data();
      nd->n.num_inputs = int(nd->ins.size());
      nd->n.output = &o->t;
      nd->n.op = plast_hip_get_op_impl(nd->n.op_type);
      o->t.creator = &nd->n;
      avail.push_back(&o->t);
      ts.push_back(std::move(o));
      ns.push_back(std::move(nd));
    }
    // evaluate unfused, keep every output's values
    std::vector<Node *> order;
    for (auto &nd : ns) order.push_back(&nd->n);
    for (auto &nd : ns) eval_node(ts, &nd->n, nd->opaque);
    std::vector<std::vector<float>> first;
    for (auto &x : ts) first.push_back(x->v);
    for (auto &x : ts)
      if (x->t.creator) std::fill(x->v.begin(), x->v.end(), std::nanf("7"));
    // the pass
    Arena arena;
    memset(&arena, 0, sizeof arena);
    DAG dag;
    memset(&dag, 0, sizeof dag);
    dag.nodes = order.data();
    dag.count = u32(order.size());
    dag.capacity = dag.count;
    dag.arena = &arena;
    const u32 before = dag.count;
    const u32 fused = plast_hip_fuse_elementwise_chains(&dag, arena_alloc_cb);
    total_fused += fused;
    // structure
    u32 dropped = 0;
    std::vector<const Tensor *> made;
    for (u32 i = 0; i < dag.count; ++i) {
      const Node *n = dag.nodes[i];
      for (int k = 0; k < n->num_inputs; ++k) {
        const Tensor *in = n->inputs[k];
        bool ok = in->creator == nullptr;
        for (const Tensor *m : made) ok = ok || m == in;
        CHECK(ok, "node %u reads a tensor no earlier node produces", i);
      }
      made.push_back(n->output);
      if (n->op_type == FUSED_ELEMENTWISE) {
        const PlastFusedTape *tp = reinterpret_cast<const PlastFusedTape *>(uintptr_t(n->params.dim));
        CHECK(tp->num_ins >= 2 && tp->num_ins <= PLAST_TAPE_MAX_INS, "tape of %u instructions", tp->num_ins);
        CHECK(n->num_inputs >= 1 && n->num_inputs <= PLAST_TAPE_MAX_INPUTS && tp->num_inputs == u32(n->num_inputs),
              "fused node with %d inputs (tape says %u)", n->num_inputs, tp->num_inputs);
        CHECK(tp->ins[0].op == TAPE_LOAD, "tape does not start with a load");
        u32 members = 0;
        for (u32 s = 0; s < tp->num_ins; ++s) {
          const u8 op = tp->ins[s].op;
          members += op != TAPE_LOAD;
          if (tp->ins[s].src == TAPE_SRC_INPUT || op == TAPE_LOAD)
            CHECK(tp->ins[s].idx < u32(n->num_inputs), "tape reads input %u of %d", tp->ins[s].idx, n->num_inputs);
        }
        dropped += members - 1;
        CHECK(n->output->creator == n, "fused output's creator is not the fused node");
        bool grads = n->output->requires_grad;
        for (int k = 0; k < n->num_inputs; ++k) {
          CHECK(n->inputs[k]->device == GPU, "fused a CPU input");
          grads = grads || n->inputs[k]->requires_grad;
        }
        if (grads) {
          CHECK(leaky_bias_node(n), "fused a chain with gradients that is not leaky_relu(x + bias)");
          ++grad_pairs;
        }
      } else {
        for (auto &nd : ns)
          if (&nd->n == n && nd->opaque) CHECK(n->op_type == SUM, "opaque node changed");
      }
    }
    CHECK(before - dag.count == dropped, "%u nodes before, %u after, %u members dropped", before, dag.count, dropped);
    // values
    for (u32 i = 0; i < dag.count; ++i) {
      const Node *n = dag.nodes[i];
      bool opaque = false;
      for (auto &nd : ns)
        if (&nd->n == n) opaque = nd->opaque;
      eval_node(ts, n, opaque);
    }
    for (size_t k = 0; k < ts.size(); ++k) {
      bool produced = ts[k]->t.creator == nullptr;
      for (const Tensor *m : made) produced = produced || m == &ts[k]->t;
      if (!produced) continue;
      CHECK(memcmp(ts[k]->v.data(), first[k].data(), first[k].size() * sizeof(float)) == 0,
            "tensor %zu differs after fusion", k);
    }
    for (void *p : g_arena) std::free(p);
    g_arena.clear();
  }
  if (fails) {
    std::printf("FAILED %d checks\n", fails);
    return 1;
  }
  std::printf("ok %d %ld %ld\n", trials, total_fused, grad_pairs);
  return 0;
}
