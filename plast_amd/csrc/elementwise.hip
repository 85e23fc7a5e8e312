// elementwise.hip — binary and unary ops (forward and backward), the view ops' metadata forwards
// and GPU backwards, and the fused elementwise-chain op.
#include "ew_impl.hpp"
#include "red_impl.hpp"

namespace plast {
namespace {

bool check_f32(const Tensor *t, const char *where) {
  if (t->dtype != FLOAT32) {
    report_error(where, "unsupported dtype %d", int(t->dtype));
    return false;
  }
  return true;
}

// Fill the first `rank` axes of operand k from tensor t aligned to `shape` (broadcast rule).
void set_operand(Space &s, int k, const Tensor *t) {
  bcast_strides(t, s.shape, s.rank, s.st[k]);
}

// Operand k follows tensor t's own strides over an identical shape.
void set_own(Space &s, int k, const Tensor *t) {
  for (int d = 0; d < s.rank; ++d) s.st[k][d] = t->shape[d] == 1 ? 0 : int64_t(t->strides[d]);
}

void init_space(Space &s, const uint64_t *shape, int rank) {
  s.rank = rank;
  for (int d = 0; d < rank; ++d) s.shape[d] = shape[d];
}

// ------------------------------------------------------------------------- binary

template <Bin OP>
void binary_forward(const Tensor **in, Tensor *out, const char *where) {
  if (!ensure_init()) return;
  const Tensor *a = in[0], *b = in[1];
  if (!check_f32(a, where) || !check_f32(b, where) || !check_f32(out, where)) return;
  uint64_t bshape[kMaxRank];
  int brank;
  if (!broadcast_shape(a, b, bshape, &brank)) {
    report_error(where, "shapes are not broadcastable");
    return;
  }
  if (brank > int(out->ndim) || numel(out) != [&] {
        uint64_t n = 1;
        for (int d = 0; d < brank; ++d) n *= bshape[d];
        return n;
      }()) {
    report_error(where, "output shape does not match the broadcast shape");
    return;
  }
  Space s;
  init_space(s, out->shape, int(out->ndim));
  set_operand(s, 0, a);
  set_operand(s, 1, b);
  set_own(s, 2, out);
  const void *ins[2] = {a->data, b->data};
  launch_elementwise(BinBody<OP>{}, ins, out->data, s, where);
  finish(where);
}

// Does tensor t cover every element of `shape` exactly once (no broadcast axis)?
bool covers(const Tensor *t, const uint64_t *shape, int rank) {
  if (int(t->ndim) > rank) return false;
  int lead = rank - int(t->ndim);
  for (int d = 0; d < rank; ++d) {
    uint64_t e = d < lead ? 1 : t->shape[d - lead];
    if (e != shape[d]) return false;
  }
  return true;
}

// One past the largest element offset that shape and strides address (0 for an empty shape).
uint64_t extent(const uint64_t *shape, const uint64_t *strides, uint64_t ndim) {
  uint64_t hi = 0;
  for (uint64_t d = 0; d < ndim; ++d) {
    if (shape[d] == 0) return 0;
    hi += (shape[d] - 1) * strides[d];
  }
  return hi + 1;
}

// Accumulate one operand's gradient. The reference's broadcast backward addresses the gradient
// buffer with the operand's *data* strides (kernel_macros.h:314-317 passes a->strides as
// da_strides; its contiguous path indexes da flat, the same offsets for a contiguous operand). A
// view's grad keeps the layout it was allocated with (tensor.c:66-78) while the view's forward
// rewrote its data strides (shape_ops.c:59-80), so on a transposed view the two layouts differ, and
// this follows the reference. Elementwise when those offsets are distinct, otherwise a
// deterministic reduction over the axes that repeat an offset (broadcast or expanded axes; the
// reference uses `omp atomic` here: kernel_macros.h:283-299). Offsets past the gradient's own
// extent (the reference would write out of bounds) are refused.
template <class Elem, class Term>
void grad_into(const Tensor *x, const Tensor *out, const Tensor *a, const Tensor *b,
               const Elem &elem, const Term &term, const char *where) {
  const Tensor *g = out->grad;
  const int rank = int(g->ndim);
  int64_t tst[kMaxRank];
  bcast_strides(x, g->shape, rank, tst);
  const uint64_t need = extent(x->shape, x->strides, x->ndim);
  const uint64_t have = extent(x->grad->shape, x->grad->strides, x->grad->ndim);
  if (need > have) {
    report_error(where, "the operand's strides address %llu gradient elements, its gradient holds "
                 "%llu", (unsigned long long)need, (unsigned long long)have);
    return;
  }
  bool repeats = false;
  for (int d = 0; d < rank; ++d) repeats = repeats || (tst[d] == 0 && g->shape[d] > 1);
  Space s;
  init_space(s, g->shape, rank);
  if (!repeats) {
    for (int d = 0; d < rank; ++d) s.st[0][d] = s.st[4][d] = tst[d];
    set_own(s, 1, g);
    set_operand(s, 2, a);
    set_operand(s, 3, b);
    const void *ins[4] = {x->grad->data, g->data, a->data, b->data};
    launch_elementwise(elem, ins, x->grad->data, s, where);
  } else {
    set_own(s, 0, g);
    set_operand(s, 1, a);
    set_operand(s, 2, b);
    for (int d = 0; d < rank; ++d) s.st[3][d] = tst[d];
    const void *ins[3] = {g->data, a->data, b->data};
    reduce_accumulate(term, ins, static_cast<float *>(x->grad->data), s, where);
  }
}

// Gradient term of one operand from (g, a, b), for the reduction path.
template <Bin OP, bool B>
struct BinTerm {
  static constexpr int NIN = 3;
  __device__ __forceinline__ float eval(const float *v) const {
    if constexpr (B) return grad_b<OP>(v[0], v[1], v[2], false);
    else return grad_a<OP>(v[0], v[1], v[2]);
  }
};

template <Bin OP>
void binary_backward(Tensor **in, const Tensor *out, const char *where) {
  if (!ensure_init()) return;
  const Tensor *a = in[0], *b = in[1];
  if (!check_f32(a, where) || !check_f32(b, where)) return;
  if (!out->grad) {
    report_error(where, "output has no gradient");
    return;
  }
  const bool da = a->requires_grad && a->grad, db = b->requires_grad && b->grad;
  const Tensor *g = out->grad;
  const uint64_t n = numel(out);
  // The reference's contiguous same-shape path (kernel_macros.h:306-311) rounds the B-gradient of
  // sub/div from 0 - g inside its SIMD blocks.
  const bool ref_contig = contiguous(a) && contiguous(b) && contiguous(out) && same_shape(a, b);
  if (da) grad_into(a, out, a, b, BinGradABody<OP>{}, BinTerm<OP, false>{}, where);
  if (db) {
    BinGradBBody<OP> body;
    body.simd_end = ref_contig ? simd_end(n) : 0;
    grad_into(b, out, a, b, body, BinTerm<OP, true>{}, where);
  }
  (void)g;
  finish(where);
}

// ------------------------------------------------------------------------- unary

template <Un OP>
void unary_forward(const Tensor **in, Tensor *out, KernelParams p, const char *where) {
  if (!ensure_init()) return;
  const Tensor *a = in[0];
  if (!check_f32(a, where) || !check_f32(out, where)) return;
  if (numel(out) != numel(a)) {
    report_error(where, "output has %llu elements, input %llu", (unsigned long long)numel(out),
                 (unsigned long long)numel(a));
    return;
  }
  const uint64_t n = numel(a);
  UnBody<OP> body;
  body.alpha = p.fval;
  body.simd_end = (contiguous(a) && contiguous(out)) ? simd_end(n) : 0;
  Space s;
  init_space(s, a->shape, int(a->ndim));
  set_own(s, 0, a);
  // the reference indexes the output with its own strides over the input's shape
  for (int d = 0; d < s.rank; ++d) s.st[1][d] = a->shape[d] == 1 ? 0 : int64_t(out->strides[d]);
  const void *ins[1] = {a->data};
  launch_elementwise(body, ins, out->data, s, where);
  finish(where);
}

template <Un OP>
void unary_backward(Tensor **in, const Tensor *out, KernelParams p, const char *where) {
  if (!ensure_init()) return;
  const Tensor *a = in[0];
  if (!a->requires_grad || !a->grad) return;
  if (!check_f32(a, where)) return;
  if (!out->grad) {
    report_error(where, "output has no gradient");
    return;
  }
  UnGradBody<OP> body;
  body.alpha = p.fval;
  body.contig = contiguous(a) && contiguous(out);
  Space s;
  init_space(s, a->shape, int(a->ndim));
  set_own(s, 0, a->grad);
  for (int d = 0; d < s.rank; ++d)
    s.st[1][d] = a->shape[d] == 1 ? 0 : int64_t(out->grad->strides[d]);
  set_own(s, 2, a);
  set_own(s, 3, a->grad);
  const void *ins[3] = {a->grad->data, out->grad->data, a->data};
  launch_elementwise(body, ins, a->grad->data, s, where);
  finish(where);
}

// ------------------------------------------------------------------------- view ops

// Backward of a view that kept numel: da[i] += dout[i] over contiguous buffers
// (shape_ops.c:14-26).
void reshape_accumulate(float *da, const float *dout, uint64_t n, const char *where) {
  Space s;
  s.rank = 1;
  s.shape[0] = n;
  s.st[0][0] = s.st[1][0] = s.st[2][0] = 1;
  const void *ins[2] = {da, dout};
  launch_elementwise(AccumBody{}, ins, da, s, where);
}

void alias_meta(const Tensor *a, Tensor *out) {
  out->data = a->data;
  out->dtype = a->dtype;
  out->device = a->device;
  out->requires_grad = a->requires_grad;
}

// Row-major strides of the caller-provided output shape (cpu_utils.c:19-26).
void row_major(Tensor *out) {
  uint64_t s = 1;
  for (uint64_t d = out->ndim; d-- > 0;) {
    out->strides[d] = s;
    s *= out->shape[d];
  }
}

void view_like_forward(const Tensor **in, Tensor *out) {
  alias_meta(in[0], out);
  row_major(out);
}

void view_like_backward(Tensor **in, const Tensor *out, const char *where) {
  if (!ensure_init()) return;
  Tensor *a = in[0];
  if (!a->requires_grad || !out->grad || !a->grad) return;
  reshape_accumulate(static_cast<float *>(a->grad->data),
                     static_cast<const float *>(out->grad->data), numel(a), where);
  finish(where);
}

// expand / broadcast forward (shape_ops.c:54-57 with cpu_utils.c:59-119): stride 0 on new and on
// expanded size-1 axes. The output shares the input's grad, so their backward is a no-op
// (kernel_macros.h:141-153).
void expand_like_forward(const Tensor **in, Tensor *out) {
  const Tensor *a = in[0];
  alias_meta(a, out);
  out->grad = a->grad;
  const uint64_t lead = out->ndim - a->ndim;
  for (uint64_t d = 0; d < out->ndim; ++d) {
    if (d < lead) {
      out->strides[d] = 0;
    } else {
      const uint64_t s = d - lead;
      out->strides[d] = (a->shape[s] == 1 && out->shape[d] > 1) ? 0 : a->strides[s];
    }
  }
}

// A fused chain on the interpreter instantiated for op set OPS and its input count.
template <uint32_t OPS>
void launch_tape(const PlastFusedTape &t, uint64_t se, uint32_t neg_simd, int nin,
                 const void *const *ins, void *out, const Space &s, const char *where) {
  switch (nin) {
  case 1: launch_elementwise(TapeBody<1, OPS>{t, se, neg_simd}, ins, out, s, where); break;
  case 2: launch_elementwise(TapeBody<2, OPS>{t, se, neg_simd}, ins, out, s, where); break;
  case 3: launch_elementwise(TapeBody<3, OPS>{t, se, neg_simd}, ins, out, s, where); break;
  default: launch_elementwise(TapeBody<4, OPS>{t, se, neg_simd}, ins, out, s, where); break;
  }
}

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

#define BINARY_ENTRY(name, OPV)                                                                    \
  void name##_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {            \
    (void)params;                                                                                  \
    binary_forward<OPV>(inputs, output, #name "_hip_forward");                                     \
  }                                                                                                \
  void name##_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {           \
    (void)params;                                                                                  \
    binary_backward<OPV>(inputs, output, #name "_hip_backward");                                   \
  }
BINARY_ENTRY(add, Bin::Add)
BINARY_ENTRY(sub, Bin::Sub)
BINARY_ENTRY(mul, Bin::Mul)
BINARY_ENTRY(div, Bin::Div)
#undef BINARY_ENTRY

#define UNARY_ENTRY(name, OPV)                                                                     \
  void name##_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {            \
    unary_forward<OPV>(inputs, output, params, #name "_hip_forward");                              \
  }                                                                                                \
  void name##_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {           \
    unary_backward<OPV>(inputs, output, params, #name "_hip_backward");                            \
  }
UNARY_ENTRY(exp, Un::Exp)
UNARY_ENTRY(log, Un::Log)
UNARY_ENTRY(neg, Un::Neg)
UNARY_ENTRY(abs, Un::Abs)
UNARY_ENTRY(sin, Un::Sin)
UNARY_ENTRY(cos, Un::Cos)
UNARY_ENTRY(tan, Un::Tan)
UNARY_ENTRY(leaky_relu, Un::Leaky)
#undef UNARY_ENTRY

#define VIEW_ENTRY(name)                                                                           \
  void name##_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {            \
    (void)params;                                                                                  \
    view_like_forward(inputs, output);                                                             \
  }                                                                                                \
  void name##_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {           \
    (void)params;                                                                                  \
    view_like_backward(inputs, output, #name "_hip_backward");                                     \
  }
VIEW_ENTRY(view)
VIEW_ENTRY(flatten)
VIEW_ENTRY(squeeze)
VIEW_ENTRY(unsqueeze)
#undef VIEW_ENTRY

void expand_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  (void)params;
  expand_like_forward(inputs, output);
}
void expand_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  (void)inputs;
  (void)output;
  (void)params;
}
void broadcast_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  (void)params;
  expand_like_forward(inputs, output);
}
void broadcast_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  (void)inputs;
  (void)output;
  (void)params;
}

// shape_ops.c:59-80
void transpose_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  const Tensor *a = inputs[0];
  const uint64_t x = params.dim, y = params.keepdim;
  if (x >= a->ndim || y >= a->ndim) {
    report_error("transpose_hip_forward", "axes (%llu, %llu) out of range for rank %llu",
                 (unsigned long long)x, (unsigned long long)y, (unsigned long long)a->ndim);
    return;
  }
  alias_meta(a, output);
  output->ndim = a->ndim;
  for (uint64_t d = 0; d < a->ndim; ++d) {
    output->shape[d] = a->shape[d];
    output->strides[d] = a->strides[d];
  }
  std::swap(output->shape[x], output->shape[y]);
  std::swap(output->strides[x], output->strides[y]);
}

// shape_ops.c:82-120: da[c] += dout[c with axes swapped].
void transpose_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  Tensor *a = inputs[0];
  if (!a->requires_grad || !output->grad || !a->grad) return;
  transpose_backward_hip(static_cast<float *>(a->grad->data),
                         static_cast<const float *>(output->grad->data), a->shape,
                         a->grad->strides, output->grad->strides, a->ndim, params.dim,
                         params.keepdim, numel(a));
}

void reshape_backward_hip(float *da, const float *dout, u64 num_elements) {
  if (!ensure_init()) return;
  reshape_accumulate(da, dout, num_elements, "reshape_backward_hip");
  finish("reshape_backward_hip");
}

void transpose_backward_hip(float *da, const float *dout, const u64 *a_shape, const u64 *da_strides,
                            const u64 *dout_strides, u64 ndim, u64 axis1, u64 axis2,
                            u64 num_elements) {
  if (!ensure_init()) return;
  if (ndim > uint64_t(kMaxRank) || axis1 >= ndim || axis2 >= ndim) {
    report_error("transpose_backward_hip", "bad rank/axes");
    return;
  }
  (void)num_elements;
  Space s;
  s.rank = int(ndim);
  for (uint64_t d = 0; d < ndim; ++d) s.shape[d] = a_shape[d];
  for (uint64_t d = 0; d < ndim; ++d) {
    s.st[0][d] = a_shape[d] == 1 ? 0 : int64_t(da_strides[d]);
    // coordinate d of `a` is coordinate swap(d) of the transposed gradient
    const uint64_t td = d == axis1 ? axis2 : (d == axis2 ? axis1 : d);
    s.st[1][d] = a_shape[d] == 1 ? 0 : int64_t(dout_strides[td]);
    s.st[2][d] = s.st[0][d];
  }
  const void *ins[2] = {da, dout};
  launch_elementwise(AccumBody{}, ins, da, s, "transpose_backward_hip");
  finish("transpose_backward_hip");
}

// ---- fused elementwise chain

void fused_elementwise_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  const char *where = "fused_elementwise_hip_forward";
  if (!ensure_init()) return;
  const PlastFusedTape *tape = reinterpret_cast<const PlastFusedTape *>(uintptr_t(params.dim));
  if (!tape || tape->num_inputs == 0 || tape->num_inputs > PLAST_TAPE_MAX_INPUTS ||
      tape->num_ins == 0 || tape->num_ins > PLAST_TAPE_MAX_INS || tape->ins[0].op != TAPE_LOAD) {
    report_error(where, "malformed tape");
    return;
  }
  for (uint32_t i = 0; i < tape->num_ins; ++i) {
    const PlastTapeIns &t = tape->ins[i];
    if (t.op >= TAPE_NUM_OPS || ((t.src == TAPE_SRC_INPUT || t.op == TAPE_LOAD) &&
                                 t.idx >= tape->num_inputs)) {
      report_error(where, "tape instruction %u is invalid", i);
      return;
    }
  }
  if (!check_f32(output, where)) return;
  for (uint32_t k = 0; k < tape->num_inputs; ++k)
    if (!check_f32(inputs[k], where)) return;
  const uint64_t n = numel(output);
  Space s;
  init_space(s, output->shape, int(output->ndim));
  const void *ins[PLAST_TAPE_MAX_INPUTS];
  bool all_contig = contiguous(output);
  for (uint32_t k = 0; k < tape->num_inputs; ++k) {
    if (!covers(inputs[k], output->shape, int(output->ndim))) {
      // broadcast inputs are fine; shapes that do not broadcast are not
      uint64_t bs[kMaxRank];
      int br;
      if (!broadcast_shape(inputs[k], output, bs, &br) || br != int(output->ndim)) {
        report_error(where, "input %u does not broadcast to the output", k);
        return;
      }
      all_contig = false;
    }
    all_contig = all_contig && contiguous(inputs[k]);
    set_operand(s, int(k), inputs[k]);
    ins[k] = inputs[k]->data;
  }
  const int nin = int(tape->num_inputs);
  set_own(s, nin, output);
  // The reference's neg takes its 8-wide SIMD path (0 - x below simd_end) only when its input and
  // its output are both contiguous (DEFINE_UNARY_CPU_FORWARD, kernel_macros.h:19-31), and -x
  // otherwise. Every intermediate of the unfused chain is a fresh contiguous tensor, so only a NEG
  // reading the loaded input directly or writing the chain's output can meet a strided tensor.
  uint32_t neg_simd = 0;
  for (uint32_t i = 1; i < tape->num_ins; ++i) {
    if (tape->ins[i].op != TAPE_NEG) continue;
    const bool in_ok = i > 1 || contiguous(inputs[tape->ins[0].idx]);
    const bool out_ok = i + 1 < tape->num_ins || contiguous(output);
    if (in_ok && out_ok) neg_simd |= 1u << i;
  }
  const uint64_t se = simd_end(n);
  (void)all_contig;
  switch (tape_ops_class(*tape)) {
  case kTapeArith: launch_tape<kTapeArith>(*tape, se, neg_simd, nin, ins, output->data, s, where); break;
  case kTapeExp: launch_tape<kTapeExp>(*tape, se, neg_simd, nin, ins, output->data, s, where); break;
  case kTapeExp | kTapeLog:
    launch_tape<kTapeExp | kTapeLog>(*tape, se, neg_simd, nin, ins, output->data, s, where);
    break;
  default:
    launch_tape<kTapeExp | kTapeLog | kTapeTrig>(*tape, se, neg_simd, nin, ins, output->data, s, where);
    break;
  }
  finish(where);
}

// fused_elementwise_hip_backward (the one chain that carries a gradient) is in epilogue.hip, beside
// the bias-gradient kernels it shares.

}  // extern "C"
