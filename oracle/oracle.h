/*
 * oracle.h — CPU restatement of plast's reference CPU path for the elementwise / broadcast /
 * reduction hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (plast_amd/) links, loads or calls this.
 * It is used by tests/ as the parity checker, by __graft_entry__.smoke() as the checker, and by
 * bench.py's cpu_baseline leg when the compiled reference (oracle/_ref) is absent.
 *
 * Every entry point has the reference's ForwardKernel / BackwardKernel signature
 * (include/core/op.h:5-6) and operates on host-memory tensors. The arithmetic of each output element
 * is the reference's: same IEEE operation sequence, same serial accumulation order inside each
 * reduction, same select semantics (`x > 0 ? x : x*alpha`, `acc > x ? acc : x`).
 *
 * Pinning (how each function is checked by something other than itself):
 *  - every forward/backward op: bit-exact against the compiled reference library (oracle/_ref) on
 *    seeded cases, and against the committed golden vectors made from it (tests/golden);
 *  - exp/log: glibc expf/logf (the same library routine the reference calls);
 *  - sum/mean: fp64 brute force within the fp32 serial-summation error bound;
 *  - argmax (no reference op): numpy.argmax (first index of the maximum, first NaN wins);
 *  - softmax cross-entropy: bit-exact against the reference op chain (src/api/loss.c:97-169) run
 *    through oracle/_ref, plus the invariants that softmax rows sum to 1 and gradient rows sum to 0;
 *  - the broadcast backward (reference uses `omp atomic`, so its order is not fixed): fp64 brute
 *    force within the summation bound;
 *  - optimizers: bit-exact against the reference's own src/optimizers/cpu sources compiled into
 *    oracle/_ref, over several steps, plus a float64 restatement of the update within 1e-6.
 * Deliberate deviation: the reference's is_contiguous never inspects strides[0]
 * (src/core/tensor.c:32-42), so a tensor whose leading stride is 0 or padded is read linearly past
 * its storage. The oracle always honours the real strides.
 */
#ifndef PLAST_ORACLE_H
#define PLAST_ORACLE_H

#include "../include/plast_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_OP(name)                                                                            \
  void oracle_##name##_forward(const Tensor **inputs, Tensor *output, KernelParams params);         \
  void oracle_##name##_backward(Tensor **inputs, const Tensor *output, KernelParams params);

ORACLE_OP(add)
ORACLE_OP(sub)
ORACLE_OP(mul)
ORACLE_OP(div)
ORACLE_OP(exp)
ORACLE_OP(log)
ORACLE_OP(neg)
ORACLE_OP(abs)
ORACLE_OP(sin)
ORACLE_OP(cos)
ORACLE_OP(tan)
ORACLE_OP(leaky_relu)
ORACLE_OP(sum)
ORACLE_OP(mean)
ORACLE_OP(max)
ORACLE_OP(min)
ORACLE_OP(argmax)
ORACLE_OP(transpose)
ORACLE_OP(softmax_cross_entropy)
#undef ORACLE_OP

/* Metadata-only view ops: alias data, rewrite shape/strides (src/kernels/cpu/shape_ops.c:28-80). */
void oracle_expand_forward(const Tensor **inputs, Tensor *output, KernelParams params);

/* y = exp(-relu(a*b + c)), evaluated as five separately rounded reference ops (MUL, ADD,
 * LEAKY_RELU(0), NEG, EXP), contiguous fp32 of n elements. Config 2's op chain. */
void oracle_fused_chain2(const float *a, const float *b, const float *c, float *out, u64 n);

/* Optimizers (src/optimizers/cpu/{sgd,adam,adamw,zero_grad}.c): the same per-element statements
 * in the same order; Adam/AdamW allocate zero-filled host moment tensors on the first step, freed
 * by oracle_optimizer_release. Pinned bit-exact against the compiled reference (oracle/_ref). */
void oracle_sgd_step(SGD *o, Tensor **params, int n);
void oracle_adam_step(Adam *o, Tensor **params, int n);
void oracle_adamw_step(AdamW *o, Tensor **params, int n);
void oracle_zero_grad(Tensor *t);
void oracle_optimizer_release(Tensor **m, Tensor **v, int n);

/* The matmul epilogues' elementwise pieces (src/kernels/cpu/fused_ops.c:105-111, 294-304), pinned
 * through the reference's exported matmul_bias_relu_cpu_backward with an identity weight. */
void oracle_relu_grad_modulate(const float *dout, const float *out, float *dc, u64 n, float alpha);
void oracle_bias_grad_reduce(const float *dc, float *dbias, u64 n, u64 cols);

#ifdef __cplusplus
}
#endif

#endif
