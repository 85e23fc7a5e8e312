// epilogue.hip — the elementwise pieces of the fused matmul epilogues' backward: the leaky-relu
// gradient modulation and the bias-gradient column sum (src/kernels/cuda/matmul_relu.cu:138-151,
// matmul_bias_relu.cu:143-151; CPU: src/kernels/cpu/fused_ops.c:105-111, 294-304). The GEMMs
// around them are not part of this library. Also the backward of the fused leaky_relu(x + bias)
// node, which is the same modulation and column sum without a GEMM.
#include "ew_impl.hpp"
#include "fused_grad.hpp"
#include "red_impl.hpp"

using namespace plast;

namespace {

void modulate(const float *dout, const float *out_data, float *dc, u64 num_elements, float alpha,
              const char *where) {
  Space s;
  s.rank = 1;
  s.shape[0] = num_elements;
  s.st[0][0] = s.st[1][0] = s.st[2][0] = 1;
  ReluGradBody body;
  body.alpha = alpha;
  const void *ins[2] = {dout, out_data};
  launch_elementwise(body, ins, dc, s, where);
}

// [rows, cols] row-major, every operand with the same strides; the target (index nin) is reduced
// over rows.
Space column_space(u64 num_elements, u64 cols, int nin) {
  Space s;
  s.rank = 2;
  s.shape[0] = num_elements / cols;
  s.shape[1] = cols;
  for (int k = 0; k < nin; ++k) {
    s.st[k][0] = int64_t(cols);
    s.st[k][1] = 1;
  }
  s.st[nin][0] = 0;
  s.st[nin][1] = 1;
  return s;
}

void bias_sum(const float *dc_mod, float *dbias, u64 num_elements, u64 cols, const char *where) {
  // overwritten, as the reference's memset then accumulate: the deterministic leading-axis
  // reduction
  const void *ins[1] = {dc_mod};
  launch_reduction<Load1, SumComb>(Load1{}, ins, dbias, column_space(num_elements, cols, 1),
                                   Post::Write, 1.0f, where);
}

bool overlaps(const float *a, u64 na, const float *b, u64 nb) {
  return a < b + nb && b < a + na;
}

// The gradient buffer of t if it requires one: row-major over t's extents, else an error (null).
float *grad_of(const Tensor *t, const char *where, bool *bad) {
  if (!t->requires_grad) return nullptr;
  const Tensor *g = t->grad;
  if (!g || !g->data || g->dtype != FLOAT32 || !fused_grad::same_extents(g, t) ||
      !fused_grad::row_major(g)) {
    report_error(where, "an input's gradient is missing or not row-major fp32");
    *bad = true;
    return nullptr;
  }
  return static_cast<float *>(g->data);
}

bool whole_rows(const char *where, u64 num_elements, u64 cols) {
  if (cols != 0 && num_elements % cols == 0) return true;
  report_error(where, "need %llu elements in whole rows of %llu columns",
               (unsigned long long)num_elements, (unsigned long long)cols);
  return false;
}

}  // namespace

extern "C" {

void launch_relu_grad_modulate_hip(const float *dout, const float *out_data, float *dc,
                                   u64 num_elements, float alpha, int grid_size, int block_size) {
  const char *where = "launch_relu_grad_modulate_hip";
  (void)grid_size;   // the launch shape is this library's own (the reference caller passes
  (void)block_size;  // ceil(n / 256) x 256)
  if (!ensure_init() || num_elements == 0) return;
  if (!dout || !out_data || !dc) {
    report_error(where, "null buffer");
    return;
  }
  modulate(dout, out_data, dc, num_elements, alpha, where);
  finish(where);
}

void bias_grad_reduce_hip(const float *dc_mod, float *dbias, u64 num_elements, u64 cols) {
  const char *where = "bias_grad_reduce_hip";
  if (!ensure_init()) return;
  if (!dc_mod || !dbias) {
    report_error(where, "null buffer");
    return;
  }
  if (!whole_rows(where, num_elements, cols)) return;
  bias_sum(dc_mod, dbias, num_elements, cols, where);
  finish(where);
}

// One pass where the leading-axis kernel applies (dout and out_data read once, dc written as it
// is summed); elsewhere the two steps above, which give the same bits: the one-pass kernel is the
// bias sum's own kernel and launch shape with the modulation as its producer.
void relu_grad_modulate_bias_grad_hip(const float *dout, const float *out_data, float *dc,
                                      float *dbias, u64 num_elements, u64 cols, float alpha) {
  const char *where = "relu_grad_modulate_bias_grad_hip";
  if (!ensure_init()) return;
  if (!dout || !out_data || !dc || !dbias) {
    report_error(where, "null buffer");
    return;
  }
  if (!whole_rows(where, num_elements, cols)) return;
  // the float4 form stores dc at the inputs' float4 offsets, so all three share their alignment
  const bool fits = num_elements > 0 && aligned16(dout) == aligned16(dc) &&
                    aligned16(out_data) == aligned16(dc);
  const int errors = plast_hip_error_count();
  if (fits) {
    const void *ins[2] = {dout, out_data};
    ReluGradStore prod;
    prod.alpha = alpha;
    prod.dst = dc;
    if (launch_reduction<ReluGradStore, SumComb>(prod, ins, dbias,
                                                 column_space(num_elements, cols, 2),
                                                 Post::Write, 1.0f, where)) {
      finish(where);
      return;
    }
    if (plast_hip_error_count() != errors) return;  // reported (a workspace allocation failed)
  }
  if (num_elements > 0) modulate(dout, out_data, dc, num_elements, alpha, where);
  bias_sum(dc, dbias, num_elements, cols, where);
  finish(where);
}

// The backward of the one fused chain that carries a gradient, leaky_relu(x + bias, alpha) with
// alpha >= 0 (the fusion pass forms it for that pattern only; fused_grad.hpp). The unfused nodes'
// backwards, the leaky one into the intermediate's zeroed gradient (unary_ops.c:236-258) and then
// the ADD's (kernel_macros.h:283-299), come to dx += 0 + dy * m and dbias += the same terms summed
// over rows, m = (y > 0 ? 1 : alpha) read from the node's output. With both gradients wanted, one
// pass: the leading-axis column sum of the terms with dx + term stored as each is summed (dx bit
// for bit the unfused one; the bias's sum in this library's order, where the reference's omp
// atomics leave it unspecified). Otherwise the one that is wanted.
void fused_elementwise_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  const char *where = "fused_elementwise_hip_backward";
  const PlastFusedTape *tape = reinterpret_cast<const PlastFusedTape *>(uintptr_t(params.dim));
  if (!tape || tape->num_inputs == 0 || tape->num_inputs > PLAST_TAPE_MAX_INPUTS) {
    report_error(where, "malformed tape");
    return;
  }
  bool wanted = false;
  for (u32 k = 0; k < tape->num_inputs; ++k) wanted = wanted || inputs[k]->requires_grad;
  if (!wanted) return;  // a chain formed without gradients
  u32 i = 0, j = 0;
  float alpha = 0.0f;
  if (!fused_grad::is_leaky_bias_tape(*tape, &i, &j, &alpha)) {
    report_error(where, "only a fused leaky_relu(x + bias) chain with alpha >= 0 has a gradient");
    return;
  }
  const int xo = fused_grad::x_operand(inputs[i], inputs[j], output);
  if (xo < 0) {
    report_error(where, "the chain's operands are not (x, bias) for its output");
    return;
  }
  const Tensor *x = xo == 0 ? inputs[i] : inputs[j];
  const Tensor *b = xo == 0 ? inputs[j] : inputs[i];
  if (!ensure_init()) return;
  const Tensor *gy = output->grad;
  if (!gy || !gy->data || gy->dtype != FLOAT32 || !fused_grad::same_extents(gy, output) ||
      !fused_grad::row_major(gy)) {
    report_error(where, "the output's gradient is missing or not row-major fp32");
    return;
  }
  bool bad = false;
  float *gx = grad_of(x, where, &bad);
  float *gb = grad_of(b, where, &bad);
  if (bad) return;
  const u64 n = numel(output), cols = output->shape[output->ndim - 1];
  if (n == 0 || (!gx && !gb)) return;
  const float *dy = static_cast<const float *>(gy->data);
  const float *y = static_cast<const float *>(output->data);
  if ((gx && (overlaps(gx, n, dy, n) || overlaps(gx, n, y, n))) ||
      (gb && (overlaps(gb, cols, dy, n) || overlaps(gb, cols, y, n) ||
              (gx && overlaps(gb, cols, gx, n))))) {
    report_error(where, "a gradient buffer overlaps the output or its gradient");
    return;
  }
  const int errors = plast_hip_error_count();
  if (gx && gb) {
    LeakyAddGradStore prod;
    prod.alpha = alpha;
    prod.dst = gx;
    const void *ins[3] = {dy, y, gx};
    if (launch_reduction<LeakyAddGradStore, SumComb>(prod, ins, gb, column_space(n, cols, 3),
                                                     Post::Accum, 1.0f, where)) {
      finish(where);
      return;
    }
    if (plast_hip_error_count() != errors) return;  // reported (a workspace allocation failed)
  }
  // one at a time (a single row, say): the bias's sum reads dy and y only, so it goes first
  if (gb) {
    LeakyAddGrad prod;
    prod.alpha = alpha;
    const void *ins[2] = {dy, y};
    if (!launch_reduction<LeakyAddGrad, SumComb>(prod, ins, gb, column_space(n, cols, 2),
                                                 Post::Accum, 1.0f, where)) {
      if (plast_hip_error_count() == errors) report_error(where, "bias sum not launched");
      return;
    }
  }
  if (gx) {
    Space s;
    s.rank = 1;
    s.shape[0] = n;
    s.st[0][0] = s.st[1][0] = s.st[2][0] = s.st[3][0] = 1;
    LeakyAddGradAccumBody body;
    body.alpha = alpha;
    const void *ins[3] = {dy, y, gx};
    launch_elementwise(body, ins, gx, s, where);
  }
  finish(where);
}

}  // extern "C"
