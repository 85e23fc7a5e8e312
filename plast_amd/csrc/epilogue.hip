// epilogue.hip — the elementwise pieces of the fused matmul epilogues' backward: the leaky-relu
// gradient modulation and the bias-gradient column sum (src/kernels/cuda/matmul_relu.cu:138-151,
// matmul_bias_relu.cu:143-151; CPU: src/kernels/cpu/fused_ops.c:105-111, 294-304). The GEMMs
// around them are not part of this library.
#include "ew_impl.hpp"
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

}  // extern "C"
