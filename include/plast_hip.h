/*
 * plast_hip.h — C-ABI of the MI355X (gfx950) backend for plast's elementwise / broadcast /
 * reduction hot path. Built as plast_amd/libplast_hip.so.
 *
 * Drop-in contract:
 *  - every <op>_hip_forward / <op>_hip_backward has the reference's ForwardKernel / BackwardKernel
 *    signature (include/core/op.h:5-6) and fills the GPU slots of `Op` (op.h:39-44) where the
 *    reference binds <op>_cuda_forward / <op>_cuda_backward (src/core/op.c:11-17);
 *  - tensor metadata (shape, strides, ndim) is host memory and is read by the host side of each
 *    entry point, then passed to the kernels by value; `data` / `grad->data` are device pointers;
 *  - forward kernels overwrite the output; backward kernels accumulate (+=) into input->grad and
 *    skip inputs with requires_grad == false (include/kernels/kernel_macros.h:40, 310-311);
 *  - reductions rewrite output->shape/ndim/strides like the reference CPU path
 *    (src/kernels/cpu/reduce_ops.c:80-81);
 *  - every entry point returns after its GPU work has completed (the reference synchronises after
 *    every op: src/kernels/cuda/binary_ops.cu:113), unless the caller switched the library to
 *    asynchronous mode with plast_hip_set_sync(0), in which case work is ordered on the library's
 *    stream and plast_hip_synchronize() waits for it;
 *  - errors never cross the ABI as exceptions: a message goes to stderr, as in the reference
 *    (include/kernels/cuda/cuda_check.h:6-14), and is also kept for plast_hip_last_error().
 */
#ifndef PLAST_HIP_H
#define PLAST_HIP_H

#include "plast_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PLAST_HIP_KERNEL_PAIR(name)                                                                \
  void name##_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params);             \
  void name##_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params);

/* Binary ops: replace {add,sub,mul,div}_cuda_forward/backward (include/kernels/ops/binary.h:21-24).
 * inputs[0], inputs[1] broadcast against each other numpy-style (right-aligned, size-1 axes read
 * coordinate 0: include/kernels/kernel_macros.h:156-168); output has the broadcast shape. */
PLAST_HIP_KERNEL_PAIR(add)
PLAST_HIP_KERNEL_PAIR(sub)
PLAST_HIP_KERNEL_PAIR(mul)
PLAST_HIP_KERNEL_PAIR(div)

/* Unary ops: replace {abs,cos,sin,tan,exp,log,neg,leaky_relu}_cuda_forward/backward
 * (include/kernels/ops/unary.h:25-28). leaky_relu's slope is params.fval (unary_ops.c:323). */
PLAST_HIP_KERNEL_PAIR(exp)
PLAST_HIP_KERNEL_PAIR(log)
PLAST_HIP_KERNEL_PAIR(neg)
PLAST_HIP_KERNEL_PAIR(abs)
PLAST_HIP_KERNEL_PAIR(sin)
PLAST_HIP_KERNEL_PAIR(cos)
PLAST_HIP_KERNEL_PAIR(tan)
PLAST_HIP_KERNEL_PAIR(leaky_relu)

/* Reductions: replace {sum,mean,max,min}_cuda_forward/backward (include/kernels/ops/reduce.h:21-24).
 * params.dim = axis, or PLAST_DIM_ALL for all elements; params.keepdim = 0/1. */
PLAST_HIP_KERNEL_PAIR(sum)
PLAST_HIP_KERNEL_PAIR(mean)
PLAST_HIP_KERNEL_PAIR(max)
PLAST_HIP_KERNEL_PAIR(min)

/* argmax: no reference counterpart (OP_TYPE has none: include/core/op.h:8-37). First index of the
 * maximum along params.dim (a NaN counts as the maximum), int64 output (dtype INT64); backward is a
 * no-op. */
PLAST_HIP_KERNEL_PAIR(argmax)

/* View ops: metadata-only forwards that alias data and rewrite shape/strides on the host, as the
 * reference's CPU functions do when bound to the GPU slot (src/core/op.c:28-35, ops.def:14-19,24,
 * src/kernels/cpu/shape_ops.c:28-80); backwards accumulate on the GPU. */
PLAST_HIP_KERNEL_PAIR(view)
PLAST_HIP_KERNEL_PAIR(flatten)
PLAST_HIP_KERNEL_PAIR(squeeze)
PLAST_HIP_KERNEL_PAIR(unsqueeze)
PLAST_HIP_KERNEL_PAIR(expand)
PLAST_HIP_KERNEL_PAIR(broadcast)
PLAST_HIP_KERNEL_PAIR(transpose)

/* Fused elementwise chain: no reference counterpart (the reference fuses only matmul/conv
 * epilogues: src/scheduler/fusion.c:28-90). params.dim holds a `const PlastFusedTape *` (host
 * memory); inputs are the chain's external tensors in tape order. One kernel launch. The forward
 * writes only the chain's output. The backward is a no-op for a chain formed without gradients;
 * the one chain formed with them, leaky_relu(x + bias, alpha >= 0) over row-major x and a bias row,
 * adds 0 + dy * (y > 0 ? 1 : alpha) into x->grad (bit for bit the unfused nodes' backwards,
 * unary_ops.c:236-258 then kernel_macros.h:283-299) and the same terms summed over rows into
 * bias->grad (summation order: the library's, as the reference's omp atomics leave it open), in
 * one launch when both require grad. */
PLAST_HIP_KERNEL_PAIR(fused_elementwise)

/* Softmax cross-entropy: no reference op; replaces the op chain of src/api/loss.c:97-169 up to NEG.
 * inputs: [0] logits [N,C] fp32, [1] labels [N] int32, [2] stats [N,2] fp32 (written by forward:
 * row max and log of the row's exp-sum; read by backward). output: [N] fp32 per-row loss. Backward:
 * logits->grad += dloss[i] * (softmax - onehot). */
PLAST_HIP_KERNEL_PAIR(softmax_cross_entropy)

/* Softmax / log-softmax over the last axis: no reference op; each replaces the op chain of
 * plast/nn/functional.py:75-97 (MAX(dim, keepdim) -> SUB -> EXP -> SUM(dim, keepdim) -> DIV, or
 * -> LOG -> SUB). inputs: [0] x, contiguous fp32; output: y, contiguous fp32 of x's shape;
 * params.dim: the last axis (x->ndim - 1), any other is an error. Backward reads y and y's grad:
 * x->grad += y * (dy - sum(dy * y)) (softmax) or dy - exp(y) * sum(dy) (log-softmax), per row. */
PLAST_HIP_KERNEL_PAIR(softmax)
PLAST_HIP_KERNEL_PAIR(log_softmax)

#undef PLAST_HIP_KERNEL_PAIR

/* ------------------------------------------------------------------ fused-chain tape --------- */

/* A fused chain is a straight-line program over one accumulator: the first instruction loads an
 * external input, every later instruction combines the accumulator with an external input, an
 * immediate or itself. This covers every chain the fusion pass forms (each fused node consumes the
 * previous node's output plus at most one external tensor). */
typedef enum PlastTapeOp {
  TAPE_LOAD = 0, /* acc = in[src] */
  TAPE_ADD,
  TAPE_SUB,
  TAPE_MUL,
  TAPE_DIV,      /* binary: acc = acc OP operand, or operand OP acc when acc_rhs */
  TAPE_LEAKY_RELU, /* acc = acc > 0 ? acc : acc * imm */
  TAPE_EXP,
  TAPE_LOG,
  TAPE_NEG,      /* the reference's neg: 0 - acc inside its 8-wide SIMD blocks, -acc in the tail */
  TAPE_ABS,
  TAPE_SIN,
  TAPE_COS,
  TAPE_TAN,
  TAPE_NUM_OPS
} PlastTapeOp;

typedef enum PlastTapeSrc { TAPE_SRC_NONE = 0, TAPE_SRC_INPUT, TAPE_SRC_ACC, TAPE_SRC_IMM } PlastTapeSrc;

#define PLAST_TAPE_MAX_INS 16
#define PLAST_TAPE_MAX_INPUTS 4

typedef struct PlastTapeIns {
  u8 op;      /* PlastTapeOp */
  u8 src;     /* PlastTapeSrc of the second operand (binary ops) */
  u8 idx;     /* input index when src == TAPE_SRC_INPUT */
  u8 acc_rhs; /* 1: operand OP acc (order matters for SUB and DIV) */
  float imm;  /* leaky slope, or the operand when src == TAPE_SRC_IMM */
} PlastTapeIns;

typedef struct PlastFusedTape {
  u32 num_inputs;
  u32 num_ins;
  PlastTapeIns ins[PLAST_TAPE_MAX_INS];
} PlastFusedTape;

/* ------------------------------------------------------------------ optimizers --------------- */

/* Parameter updates over `num_parameters` tensors (parameters[i]->data += f(grad, state)),
 * replacing sgd_step_cuda / adam_step_cuda / adamw_step_cuda / zero_grad_cuda
 * (include/optimizers/sgd.h:13, adam.h:24, adamw.h:25, zero_grad.h:11; the reference's CUDA Adam
 * and AdamW are empty: src/optimizers/cuda/adam.cu:72-73, adamw.cu:20-21). Per element they apply
 * the reference CPU update in its operation order (src/optimizers/cpu/sgd.c:16-28,
 * adam.c:21-68, adamw.c:19-69); parameters that are NULL or have no grad are skipped; data and
 * grad are read as flat arrays of numel(param) floats, as the reference does. All parameters of one
 * call are updated by one kernel launch. With more than 64 tensors their table is kept in device
 * memory, and uploaded (waiting for the library stream) only when it differs from the previous
 * call's; while a graph is captured such a call is recorded as one launch per 64 tensors.
 * Adam/AdamW: `t` is incremented first and the bias-corrected step
 * lr_t = lr * sqrt(1 - beta2^t) / (1 - beta1^t) is evaluated on the host exactly as the reference
 * evaluates it (double sqrt, float powf). On the first call, when optimizer->m is NULL, the moment
 * tensors are allocated by this library (device memory zero-filled, Tensor structs on the host
 * heap) and stay owned by it until plast_hip_adam_release / plast_hip_adamw_release; a caller
 * that sets m and v beforehand (for instance from its own device arenas) keeps ownership of them. */
void sgd_step_hip(SGD *optimizer, Tensor **parameters, int num_parameters);
void adam_step_hip(Adam *optimizer, Tensor **parameters, int num_parameters);
void adamw_step_hip(AdamW *optimizer, Tensor **parameters, int num_parameters);
/* grad[0 .. numel(t->grad)) = 0 (src/optimizers/cpu/zero_grad.c:4-11). */
void zero_grad_hip(Tensor *t);
/* Free moment tensors allocated by the first adam_step_hip / adamw_step_hip and reset m, v to
 * NULL (no effect on caller-provided ones, which the library never owns). */
void plast_hip_adam_release(Adam *optimizer, int num_parameters);
void plast_hip_adamw_release(AdamW *optimizer, int num_parameters);

/* ------------------------------------------------------------------ matmul epilogue pieces ---- */

/* dc[i] = dout[i] * (out_data[i] > 0 ? 1 : alpha) over num_elements contiguous floats: replaces
 * launch_relu_grad_modulate_cuda (include/kernels/matmul.h:43, src/kernels/cuda/
 * matmul_relu.cu:138-151; CPU fused_ops.c:105-111). grid_size and block_size are accepted for
 * signature compatibility and ignored. */
void launch_relu_grad_modulate_hip(const float *dout, const float *out_data, float *dc,
                                   u64 num_elements, float alpha, int grid_size, int block_size);
/* dbias[c] = sum over rows of dc_mod[row * cols + c] (dbias overwritten), num_elements a multiple
 * of cols: the bias-gradient column sum of matmul_bias_relu's backward (src/kernels/cuda/
 * matmul_bias_relu.cu:143-151, 215-220; CPU fused_ops.c:294-304), deterministic (no atomics). */
void bias_grad_reduce_hip(const float *dc_mod, float *dbias, u64 num_elements, u64 cols);
/* Both of the above in one call: dc as launch_relu_grad_modulate_hip writes it and dbias as
 * bias_grad_reduce_hip(dc, ...) writes it, bit for bit, with dout and out_data read once and dc
 * not read back. Replaces the pair in matmul_bias_relu_cuda_backward (src/kernels/cuda/
 * matmul_bias_relu.cu:181-186 then 215-220), which writes dc_mod and then re-reads it for the
 * bias gradient; the reference has no single call for the pair. */
void relu_grad_modulate_bias_grad_hip(const float *dout, const float *out_data, float *dc,
                                      float *dbias, u64 num_elements, u64 cols, float alpha);

/* ------------------------------------------------------------------ cross-entropy step ------- */

/* One pass of a cross-entropy training step over row-major [N, C] fp32 logits with int32 labels
 * [N]: the forward of softmax_cross_entropy_hip_forward (stats [N, 2] = row max and log of the
 * exp-sum, loss [N] per row), its backward dlogits = dloss[i] * (softmax - onehot) written (not
 * accumulated), and, when dbias is not NULL, dbias[c] = sum over rows of dlogits[., c] written:
 * the gradient of a bias broadcast-added to the logits (the reference's ADD backward into a [C]
 * operand, kernel_macros.h:283-299). dloss [N] is the upstream gradient of each row's loss (1/N
 * for a mean), known before the step. Each logit is read once and each gradient written once
 * (16-byte aligned rows of whole float4 up to 32768 floats; other rows run the three passes).
 * stats, loss and dlogits are the same bits on every call; dbias, a sum over rows, is split over
 * the GPU's workgroups by the rows each one took, which varies from call to call (its last bits
 * may too) unless plast_hip_set_deterministic(1) fixes the split. No counterpart in the
 * reference, which runs the op chain of src/api/loss.c:97-169, its backward and the bias's ADD
 * backward as separate passes (its ADD backward accumulates the bias gradient with omp atomics,
 * kernel_macros.h:292-297, in no fixed order either); for callers that train with a
 * cross-entropy loss. When mean_loss is not NULL, mean_loss[0] = the mean of loss over the rows:
 * the chain's last node, MEAN (src/api/loss.c:161-163), the scalar the reference's loss returns
 * (summed in a fixed order, within the sum tolerance of the reference's serial sum; an overflowing
 * sum is summed again in row order). All pointers are device memory; returns after the work
 * completes (or is queued, in asynchronous mode). */
void softmax_cross_entropy_step_hip(const float *logits, const i32 *labels, const float *dloss,
                                    float *stats, float *loss, float *dlogits, float *dbias,
                                    float *mean_loss, u64 N, u64 C);

/* softmax_cross_entropy_step_hip without allocating: same arguments and results, with its
 * per-workgroup column sums in a fixed 32 MiB device array of the library (each GPU holds its own
 * until the process ends) rather than in workspace. It calls no hipMalloc or other allocating
 * routine, so it serves callers that cannot allocate: code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation. Only one-pass rows are taken: C a multiple of 4 up to
 * 32768, logits and dlogits 16-byte aligned, N below 2^31; anything else is reported as an error
 * (the three-pass form allocates). The results are softmax_cross_entropy_step_hip's (the same
 * kernels over the same grid; bit-identical in deterministic mode). Calls that overlap on one GPU
 * (other streams, other threads) share the array and race. No counterpart in the reference. */
void softmax_cross_entropy_step_noalloc_hip(const float *logits, const i32 *labels,
                                            const float *dloss, float *stats, float *loss,
                                            float *dlogits, float *dbias, float *mean_loss, u64 N,
                                            u64 C);

/* ------------------------------------------------------------------ pack / host transfer ----- */

/* A contiguous image of a possibly strided tensor, layout-identical to CudaTensorPack
 * (include/kernels/pack.h:17-20). */
typedef struct HipTensorPack {
  void *data;   /* t->data when t is contiguous, else the packed device buffer */
  void *_d_buf; /* owned device buffer, or NULL */
} HipTensorPack;

/* Replace cuda_tensor_pack_init / cuda_tensor_pack_release (include/kernels/pack.h:22-23,
 * src/kernels/cuda/cuda_pack.cu:28-96): alias a contiguous tensor, otherwise allocate
 * numel * element-size bytes and gather the view into them in row-major order (any dtype, copied
 * bit for bit). On failure data is NULL. Contiguity checks every stride (the reference's
 * is_contiguous ignores strides[0]: src/core/tensor.c:32-42). */
void hip_tensor_pack_init(HipTensorPack *p, const Tensor *t);
/* Returns an owned buffer to a library pool (at most 8 GiB kept) for the next pack of a similar
 * size, without waiting: work that reads the pack must be ordered before its release, as work on
 * the library stream is. */
void hip_tensor_pack_release(HipTensorPack *p);
/* Frees every pooled pack buffer (waits for the library stream first). */
void plast_hip_pack_trim(void);

/* Host transfers of a possibly strided device tensor, the data movement of the bindings' numpy()
 * and copy_from_numpy (src/python/bindings.cpp:81-151): to_host writes numel(t) elements in
 * row-major order to `dst` (packing through a library staging buffer when t is strided);
 * from_host reads numel(t) row-major elements from `src` into t's view (scattering when t is
 * strided; a destination with a broadcast axis is rejected). Both return 0 on success, -1 on
 * error, and return after the copy has completed. */
int plast_hip_tensor_to_host(const Tensor *t, void *dst);
int plast_hip_tensor_from_host(Tensor *t, const void *src);
/* Page-locked host memory (hipHostMalloc) for transfer staging: transfers from and to it run at
 * the host link's rate without an internal bounce. */
void *plast_hip_host_alloc(u64 bytes);
void plast_hip_host_free(void *p);

/* ------------------------------------------------------------------ op table ----------------- */

/* GPU slots for every OP_TYPE this backend implements (CPU slots left NULL): the table the
 * reference's get_op_impl builds from include/core/ops.def (src/core/op.c:37-49). Unimplemented
 * ops (MATMUL, CONV2D and their fused forms) get NULL GPU slots. */
Op plast_hip_get_op_impl(OP_TYPE op_type);

/* ------------------------------------------------------------------ scheduler pass ----------- */

/* Allocator used by the pass for fused Nodes, input arrays and tapes; pass the reference's
 * arena_alloc (include/core/arena.h:37) with dag->arena, as fusion_apply does
 * (src/scheduler/fusion.c:106). */
typedef void *(*PlastArenaAllocFn)(Arena *arena, u64 size, u64 align);

/* Elementwise-chain fusion over a topologically sorted DAG (the output of build_dag,
 * src/core/graph.c:52-55): every maximal run of GPU elementwise nodes in which each intermediate
 * tensor feeds only the next node, nothing in the run requires grad, and the chain has at most
 * PLAST_TAPE_MAX_INPUTS external inputs is replaced by one FUSED_ELEMENTWISE node writing the last
 * node's output, spliced into the node array the way fusion_apply does (fusion.c:155-206). So is
 * an ADD(x, bias) feeding only a LEAKY_RELU with alpha >= 0 when x or the bias requires grad
 * (x row-major fp32 of the output's shape, the bias a row-major row of its last extent): the fused
 * node's backward writes both gradients, and the intermediate x + bias (and its gradient) is
 * never written.
 * Returns the number of chains fused. Called from fusion_optimize (fusion.c:209-224). */
u32 plast_hip_fuse_elementwise_chains(DAG *dag, PlastArenaAllocFn alloc);

/* ------------------------------------------------------------------ L0/L1 hooks -------------- */

/* Arena device hooks: replace arena_*_cuda (include/core/arena_cuda.h:9-14), called from
 * src/core/arena.c:20-24, 83-87, 98-102 and 108-127. Allocation failure prints and exits, as the
 * reference does (src/core/arena_cuda.cu:5-11). */
void *arena_alloc_hip(u64 size);
/* arena_free_hip during a graph capture (a garbage-collected tensor, say) is deferred: the captured
 * kernels may use the buffer, so it is freed when the last graph the library made is destroyed
 * (at once if the capture made no graph). A buffer freed outside a capture is freed at once: the
 * caller keeps every buffer a live graph uses until that graph is destroyed. */
void arena_free_hip(void *ptr);
void arena_memset_hip(void *ptr, int value, u64 size);
void arena_memcpy_h2d_hip(void *dest, const void *src, u64 size);
void arena_memcpy_d2h_hip(void *dest, const void *src, u64 size);
void arena_memcpy_d2d_hip(void *dest, const void *src, u64 size);

/* Tensor fill hooks: replace zeros_cuda / ones_cuda / set_ones_grad_cuda
 * (include/kernels/cuda/cuda_tensor_init.h:9-11), called from src/core/tensor.c:86-89, 105-120,
 * 147-151. */
void zeros_hip(Tensor *t, u64 num_elements);
void ones_hip(Tensor *t, u64 num_elements);
void set_ones_grad_hip(Tensor *t);

/* Shape-op backward hooks: replace reshape_backward_cuda / transpose_backward_cuda
 * (src/kernels/cpu/shape_ops.c:7-12). Shape and strides are host arrays. */
void reshape_backward_hip(float *da, const float *dout, u64 num_elements);
void transpose_backward_hip(float *da, const float *dout, const u64 *a_shape, const u64 *da_strides,
                            const u64 *dout_strides, u64 ndim, u64 axis1, u64 axis2,
                            u64 num_elements);

/* ------------------------------------------------------------------ runtime control ---------- */

/* Select the device (once per process, before any other call; default device 0). Returns 0 on
 * success. */
int plast_hip_init(int device);
/* 1 (default): every entry point waits for its GPU work before returning. 0: asynchronous. */
void plast_hip_set_sync(int sync);
/* 1: results that are sums over many rows are the same bits on every call (the one-pass
 * cross-entropy step's bias gradient: its rows are split over workgroups statically, about 10%
 * slower on MI355X). 0 (default): workgroups take rows in order as they become free, so the
 * split, and the last bits of such sums, vary between calls. No counterpart in the reference,
 * whose CPU bias gradient accumulates with omp atomics (kernel_macros.h:292-297). */
void plast_hip_set_deterministic(int on);
int plast_hip_deterministic(void);
/* Wait for all work queued on the library stream. Returns 0 on success. */
int plast_hip_synchronize(void);
/* Graph capture of launch-bound work. Between plast_hip_capture_begin() and
 * plast_hip_capture_end(), every kernel the library's entry points launch is recorded on its
 * stream instead of run (no host waits happen in between), and capture_end returns an
 * instantiated graph (a hipGraphExec_t) that plast_hip_graph_launch() replays with the same
 * pointers and shapes, reading whatever the buffers hold at replay time; plast_hip_graph_destroy()
 * frees it. Only device work can be captured: run each op once before capturing so that the
 * library's workspaces are already sized (a capture that would grow one fails with an error), and
 * keep host transfers and allocation outside. The library records fills as kernels, never as
 * memset nodes. A workspace that eager work outgrows while a graph is alive is kept (retired)
 * until the last graph the library made is destroyed, so a replay never reaches freed memory.
 * Returns 0 / a non-null graph on success. No counterpart in the reference, which launches and
 * synchronises op by op. */
int plast_hip_capture_begin(void);
void *plast_hip_capture_end(void);
int plast_hip_graph_launch(void *graph);
void plast_hip_graph_destroy(void *graph);
/* Grow workspace slot 0, 1 or 2 to at least `bytes` now (for instance before a capture; slot 0
 * holds reduction and cross-entropy partial sums, 1 max/min backward tie counts, 2 pack staging),
 * and the bytes a slot holds. Returns 0 on success. */
int plast_hip_workspace_reserve(int slot, u64 bytes);
u64 plast_hip_workspace_bytes(int slot);
/* The graphs made by plast_hip_capture_end() and not yet destroyed, and the workspace buffers
 * retired while they live (freed with the last of them). */
int plast_hip_graphs_alive(void);
int plast_hip_workspace_retired(void);
/* The library's stream (a hipStream_t), for callers that order their own work against it. */
void *plast_hip_stream(void);
/* Number of errors since the last plast_hip_clear_error(), and the most recent message. */
int plast_hip_error_count(void);
const char *plast_hip_last_error(void);
void plast_hip_clear_error(void);

/* Device time between two marks recorded on the library stream, in milliseconds. */
int plast_hip_timer_begin(void);
float plast_hip_timer_end(void);

/* Deterministic device-side input generation for tests and benchmarks: element i depends only on
 * (seed, i) (a counter-based hash), so any sub-range can be regenerated independently.
 * uniform in [lo, hi); normal(mean, std) by Box-Muller; int32 uniform in [lo, hi). */
void plast_hip_fill_uniform(float *dst, u64 n, u64 seed, float lo, float hi);
void plast_hip_fill_normal(float *dst, u64 n, u64 seed, float mean, float std);
void plast_hip_fill_randint(i32 *dst, u64 n, u64 seed, i32 lo, i32 hi);

/* Plain device copy of n floats with the library's streaming load/store path: the measured
 * bandwidth ceiling the elementwise kernels are compared against. */
void plast_hip_copy(float *dst, const float *src, u64 n);

#ifdef __cplusplus
}
#endif

#endif /* PLAST_HIP_H */
