// epilogue.hip — the elementwise pieces of the fused matmul epilogues' backward: the leaky-relu
// gradient modulation and the bias-gradient column sum (src/kernels/cuda/matmul_relu.cu:138-151,
// matmul_bias_relu.cu:143-151; CPU: src/kernels/cpu/fused_ops.c:105-111, 294-304). The GEMMs
// around them are not part of this library.
#include "ew_impl.hpp"
#include "red_impl.hpp"

using namespace plast;

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
  Space s;
  s.rank = 1;
  s.shape[0] = num_elements;
  s.st[0][0] = s.st[1][0] = s.st[2][0] = 1;
  ReluGradBody body;
  body.alpha = alpha;
  const void *ins[2] = {dout, out_data};
  launch_elementwise(body, ins, dc, s, where);
  finish(where);
}

void bias_grad_reduce_hip(const float *dc_mod, float *dbias, u64 num_elements, u64 cols) {
  const char *where = "bias_grad_reduce_hip";
  if (!ensure_init()) return;
  if (!dc_mod || !dbias || cols == 0 || num_elements % cols != 0) {
    report_error(where, "need %llu elements in whole rows of %llu columns",
                 (unsigned long long)num_elements, (unsigned long long)cols);
    return;
  }
  // [rows, cols] row-major, reduced over rows into dbias (overwritten, as the reference's memset
  // then accumulate): the deterministic leading-axis reduction
  Space s;
  s.rank = 2;
  s.shape[0] = num_elements / cols;
  s.shape[1] = cols;
  s.st[0][0] = int64_t(cols);
  s.st[0][1] = 1;
  s.st[1][0] = 0;
  s.st[1][1] = 1;
  const void *ins[1] = {dc_mod};
  launch_reduction<Load1, SumComb>(Load1{}, ins, dbias, s, Post::Write, 1.0f, where);
  finish(where);
}

}  // extern "C"
