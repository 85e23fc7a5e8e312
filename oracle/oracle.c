/*
 * oracle.c — CPU restatement of plast's reference CPU path (elementwise, broadcast, reductions).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for tests/, smoke() and bench.py's cpu_baseline leg.
 * The product (plast_amd/) never links or calls it. Pinning of each function is listed in oracle.h.
 *
 * Built with -ffp-contract=off so that every `x op y` below is one IEEE round-to-nearest-even
 * operation, exactly as the reference's separate kernels round.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- index helpers ---------------- */

static u64 o_numel(const Tensor *t) {
  u64 n = 1;
  for (u64 d = 0; d < t->ndim; ++d) n *= t->shape[d];
  return n;
}

/* Row-major contiguity with every stride checked (see the strides[0] note in oracle.h). */
static int o_contig(const Tensor *t) {
  u64 want = 1;
  for (u64 d = t->ndim; d-- > 0;) {
    if (t->shape[d] != 1 && t->strides[d] != want) return 0;
    want *= t->shape[d];
  }
  return 1;
}

/* Linear index -> coordinates, last dimension fastest (cpu_utils.c:12-17). */
static void o_coords(u64 idx, const u64 *shape, u64 ndim, u64 *coords) {
  for (u64 d = ndim; d-- > 0;) {
    coords[d] = idx % shape[d];
    idx /= shape[d];
  }
}

static u64 o_offset(const u64 *coords, const u64 *strides, u64 ndim) {
  u64 off = 0;
  for (u64 d = 0; d < ndim; ++d) off += coords[d] * strides[d];
  return off;
}

/* Right-aligned numpy broadcasting: a size-1 dimension always reads coordinate 0
 * (kernel_macros.h:156-168). */
static u64 o_bcast_offset(const u64 *coords, u64 cnd, const u64 *strides, const u64 *shape,
                          u64 nd) {
  u64 off = 0;
  u64 shift = cnd - nd;
  for (u64 d = 0; d < nd; ++d) {
    u64 c = shape[d] == 1 ? 0 : coords[d + shift];
    off += c * strides[d];
  }
  return off;
}

static int o_same_shape(const Tensor *a, const Tensor *b) {
  if (a->ndim != b->ndim) return 0;
  for (u64 d = 0; d < a->ndim; ++d)
    if (a->shape[d] != b->shape[d]) return 0;
  return 1;
}

/* Width of the reference's AVX2 blocks: contiguous loops run 8-wide SIMD over the first
 * n - n%8 elements and a scalar tail after (kernel_macros.h:192-204). Only neg and the sub/div
 * B-gradients round differently in the two halves (0-x versus -x on a signed zero). */
#define O_SIMD 8
static u64 o_simd_end(u64 n) { return n - n % O_SIMD; }

/* ---------------------------------------------------------------- binary ops ------------------- */

typedef enum { O_ADD, O_SUB, O_MUL, O_DIV } OBin;

static inline float o_bin(OBin op, float x, float y) {
  switch (op) {
  case O_ADD: return x + y;
  case O_SUB: return x - y;
  case O_MUL: return x * y;
  default: return x / y;
  }
}

/* binary_ops.c:17-60 via DEFINE_BINARY_CPU_FORWARD (kernel_macros.h:191-242). Both of the
 * reference's paths compute c = a op b with one rounding; only the index math differs. */
static void o_binary_forward(OBin op, const Tensor **in, Tensor *out) {
  const Tensor *a = in[0], *b = in[1];
  const float *pa = (const float *)a->data, *pb = (const float *)b->data;
  float *pc = (float *)out->data;
  u64 n = o_numel(out);
  if (o_contig(a) && o_contig(b) && o_contig(out) && o_same_shape(a, b)) {
#pragma omp parallel for
    for (u64 i = 0; i < n; ++i) pc[i] = o_bin(op, pa[i], pb[i]);
    return;
  }
#pragma omp parallel for
  for (u64 i = 0; i < n; ++i) {
    u64 c[PLAST_MAX_NDIM];
    o_coords(i, out->shape, out->ndim, c);
    u64 oa = o_bcast_offset(c, out->ndim, a->strides, a->shape, a->ndim);
    u64 ob = o_bcast_offset(c, out->ndim, b->strides, b->shape, b->ndim);
    pc[o_offset(c, out->strides, out->ndim)] = o_bin(op, pa[oa], pb[ob]);
  }
}

/* Gradient expressions (binary_ops.c:18-57). `simd` selects the reference's AVX2 form, which for
 * sub and div starts the B-gradient from (0 - g) instead of -(g). */
static inline float o_grad_a(OBin op, float g, float x, float y) {
  switch (op) {
  case O_ADD:
  case O_SUB: return g;
  case O_MUL: return g * y;
  default: return g / y;
  }
}
static inline float o_grad_b(OBin op, float g, float x, float y, int simd) {
  float ng = simd ? 0.0f - g : -g;
  switch (op) {
  case O_ADD: return g;
  case O_SUB: return ng;
  case O_MUL: return g * x;
  default: return ng * x / (y * y);
  }
}

/* DEFINE_BINARY_CPU_BACKWARD (kernel_macros.h:244-325). The reference's broadcast path adds into
 * the smaller operand with `omp atomic`, so its summation order is unspecified; the oracle adds
 * serially in dout index order. */
static void o_binary_backward(OBin op, Tensor **in, const Tensor *out) {
  const Tensor *a = in[0], *b = in[1];
  const float *pa = (const float *)a->data, *pb = (const float *)b->data;
  const float *g = (const float *)out->grad->data;
  float *da = a->requires_grad ? (float *)a->grad->data : NULL;
  float *db = b->requires_grad ? (float *)b->grad->data : NULL;
  u64 n = o_numel(out);
  if (o_contig(a) && o_contig(b) && o_contig(out) && o_same_shape(a, b)) {
    u64 se = o_simd_end(n);
#pragma omp parallel for
    for (u64 i = 0; i < n; ++i) {
      if (da) da[i] = da[i] + o_grad_a(op, g[i], pa[i], pb[i]);
      if (db) db[i] = db[i] + o_grad_b(op, g[i], pa[i], pb[i], i < se);
    }
    return;
  }
  const Tensor *go = out->grad;
  u64 c[PLAST_MAX_NDIM];
  for (u64 i = 0; i < n; ++i) {
    o_coords(i, go->shape, go->ndim, c);
    float gi = g[o_offset(c, go->strides, go->ndim)];
    u64 oa = o_bcast_offset(c, go->ndim, a->strides, a->shape, a->ndim);
    u64 ob = o_bcast_offset(c, go->ndim, b->strides, b->shape, b->ndim);
    if (da) da[oa] += o_grad_a(op, gi, pa[oa], pb[ob]);
    if (db) db[ob] += o_grad_b(op, gi, pa[oa], pb[ob], 0);
  }
}

#define O_BINARY(name, OPV)                                                                        \
  void oracle_##name##_forward(const Tensor **inputs, Tensor *output, KernelParams params) {        \
    (void)params;                                                                                  \
    o_binary_forward(OPV, inputs, output);                                                         \
  }                                                                                                \
  void oracle_##name##_backward(Tensor **inputs, const Tensor *output, KernelParams params) {       \
    (void)params;                                                                                  \
    o_binary_backward(OPV, inputs, output);                                                        \
  }
O_BINARY(add, O_ADD)
O_BINARY(sub, O_SUB)
O_BINARY(mul, O_MUL)
O_BINARY(div, O_DIV)

/* ---------------------------------------------------------------- unary ops -------------------- */

typedef enum { O_EXP, O_LOG, O_NEG, O_ABS, O_SIN, O_COS, O_TAN, O_LEAKY } OUn;

/* unary_ops.c:68-91 (forward expressions), 196-206 (neg's AVX2 body is 0 - x). */
static inline float o_un(OUn op, float x, float alpha, int simd) {
  switch (op) {
  case O_EXP: return expf(x);
  case O_LOG: return logf(x);
  case O_NEG: return simd ? 0.0f - x : -x;
  case O_ABS: return fabsf(x);
  case O_SIN: return sinf(x);
  case O_COS: return cosf(x);
  case O_TAN: return tanf(x);
  default: return x > 0 ? x : x * alpha;
  }
}

/* Gradient terms added into da (unary_ops.c:68-91 and the contiguous loops 101-319). */
static inline float o_un_grad(OUn op, float g, float x, float alpha, int contig) {
  switch (op) {
  case O_EXP: return g * expf(x);
  case O_LOG: return g * (1.0f / x);
  case O_NEG: return -g;
  case O_ABS:
    if (contig) return g * (x > 0 ? 1.0f : (x < 0 ? -1.0f : 0.0f));
    return x > 0 ? g : (x < 0 ? -g : 0.0f);
  case O_SIN: return g * cosf(x);
  case O_COS: return g * (-sinf(x));
  case O_TAN: {
    float t = tanf(x);
    return g * (1.0f + t * t);
  }
  default:
    if (contig) return g * (x > 0 ? 1.0f : alpha);
    return x > 0 ? g : g * alpha;
  }
}

/* DEFINE_UNARY_CPU_FORWARD / _NONCONTIG_FORWARD (kernel_macros.h:19-31, 84-94). */
static void o_unary_forward(OUn op, const Tensor **in, Tensor *out, float alpha) {
  const Tensor *a = in[0];
  const float *pa = (const float *)a->data;
  float *pc = (float *)out->data;
  u64 n = o_numel(a);
  if (o_contig(a) && o_contig(out)) {
    u64 se = o_simd_end(n);
#pragma omp parallel for
    for (u64 i = 0; i < n; ++i) pc[i] = o_un(op, pa[i], alpha, i < se);
    return;
  }
#pragma omp parallel for
  for (u64 i = 0; i < n; ++i) {
    u64 c[PLAST_MAX_NDIM];
    o_coords(i, a->shape, a->ndim, c);
    pc[o_offset(c, out->strides, a->ndim)] = o_un(op, pa[o_offset(c, a->strides, a->ndim)], alpha, 0);
  }
}

/* DEFINE_UNARY_CPU_BACKWARD / _NONCONTIG_BACKWARD (kernel_macros.h:33-48, 96-110). The reference
 * computes neg's contiguous gradient as da - g, which is the same IEEE operation as da + (-g). */
static void o_unary_backward(OUn op, Tensor **in, const Tensor *out, float alpha) {
  const Tensor *a = in[0];
  if (!a->requires_grad) return;
  const float *pa = (const float *)a->data;
  const float *g = (const float *)out->grad->data;
  float *da = (float *)a->grad->data;
  u64 n = o_numel(a);
  if (o_contig(a) && o_contig(out)) {
#pragma omp parallel for
    for (u64 i = 0; i < n; ++i) da[i] = da[i] + o_un_grad(op, g[i], pa[i], alpha, 1);
    return;
  }
#pragma omp parallel for
  for (u64 i = 0; i < n; ++i) {
    u64 c[PLAST_MAX_NDIM];
    o_coords(i, a->shape, a->ndim, c);
    u64 od = o_offset(c, a->grad->strides, a->ndim);
    float gi = g[o_offset(c, out->grad->strides, a->ndim)];
    da[od] = da[od] + o_un_grad(op, gi, pa[o_offset(c, a->strides, a->ndim)], alpha, 0);
  }
}

#define O_UNARY(name, OPV)                                                                         \
  void oracle_##name##_forward(const Tensor **inputs, Tensor *output, KernelParams params) {        \
    o_unary_forward(OPV, inputs, output, params.fval);                                             \
  }                                                                                                \
  void oracle_##name##_backward(Tensor **inputs, const Tensor *output, KernelParams params) {       \
    o_unary_backward(OPV, inputs, output, params.fval);                                            \
  }
O_UNARY(exp, O_EXP)
O_UNARY(log, O_LOG)
O_UNARY(neg, O_NEG)
O_UNARY(abs, O_ABS)
O_UNARY(sin, O_SIN)
O_UNARY(cos, O_COS)
O_UNARY(tan, O_TAN)
O_UNARY(leaky_relu, O_LEAKY)

/* ---------------------------------------------------------------- reductions ------------------- */

typedef enum { O_SUM, O_MEAN, O_MAX, O_MIN } ORed;

static inline float o_red_init(ORed op) {
  return op == O_MAX ? -FLT_MAX : (op == O_MIN ? FLT_MAX : 0.0f);
}
/* reduce_ops.c:8-10: ties and NaNs follow the literal select, not fmaxf/fminf. */
static inline float o_red_step(ORed op, float acc, float x) {
  switch (op) {
  case O_MAX: return acc > x ? acc : x;
  case O_MIN: return acc < x ? acc : x;
  default: return acc + x;
  }
}
static inline float o_red_post(ORed op, float acc, u64 n) {
  return op == O_MEAN ? acc / (float)n : acc;
}

/* Output shape of a dim-reduction (cpu_utils.c:121-154); the reference rewrites the output's
 * metadata in the forward call, and so does the oracle. */
static void o_reduced_meta(const Tensor *a, u64 dim, int keepdim, Tensor *out) {
  u64 nd = 0;
  for (u64 d = 0; d < a->ndim; ++d) {
    if (d == dim) {
      if (keepdim) out->shape[nd++] = 1;
    } else {
      out->shape[nd++] = a->shape[d];
    }
  }
  if (nd == 0) out->shape[nd++] = 1;
  out->ndim = nd;
  u64 s = 1;
  for (u64 d = nd; d-- > 0;) {
    out->strides[d] = s;
    s *= out->shape[d];
  }
}

/* Input coordinates of the first element reduced into output coordinate `oc`
 * (kernel_macros.h:171-188). */
static void o_out_to_in(const u64 *oc, u64 *ic, u64 and_, u64 dim, int keepdim) {
  for (u64 d = 0; d < and_; ++d) {
    if (d == dim) ic[d] = 0;
    else ic[d] = keepdim ? oc[d] : (d < dim ? oc[d] : oc[d - 1]);
  }
}

/* DEFINE_REDUCE_CPU_FORWARD (reduce_ops.c:24-87): serial fp32 accumulation in index order. */
static void o_reduce_forward(ORed op, const Tensor **in, Tensor *out, KernelParams p) {
  const Tensor *a = in[0];
  const float *pa = (const float *)a->data;
  float *pc = (float *)out->data;
  if (p.dim == PLAST_DIM_ALL) {
    u64 n = o_numel(a);
    float acc = o_red_init(op);
    u64 c[PLAST_MAX_NDIM];
    for (u64 i = 0; i < n; ++i) {
      o_coords(i, a->shape, a->ndim, c);
      acc = o_red_step(op, acc, pa[o_offset(c, a->strides, a->ndim)]);
    }
    pc[0] = o_red_post(op, acc, n);
    return;
  }
  u64 dim = p.dim;
  int keep = p.keepdim != 0;
  o_reduced_meta(a, dim, keep, out);
  u64 nout = o_numel(out);
  u64 len = a->shape[dim];
#pragma omp parallel for
  for (u64 o = 0; o < nout; ++o) {
    u64 oc[PLAST_MAX_NDIM], ic[PLAST_MAX_NDIM];
    o_coords(o, out->shape, out->ndim, oc);
    o_out_to_in(oc, ic, a->ndim, dim, keep);
    float acc = o_red_init(op);
    for (u64 k = 0; k < len; ++k) {
      ic[dim] = k;
      acc = o_red_step(op, acc, pa[o_offset(ic, a->strides, a->ndim)]);
    }
    pc[o] = o_red_post(op, acc, len);
  }
}

/* DEFINE_REDUCE_CPU_BACKWARD_SUM_MEAN (reduce_ops.c:89-154). */
static void o_sum_mean_backward(ORed op, Tensor **in, const Tensor *out, KernelParams p) {
  Tensor *a = in[0];
  if (!a->requires_grad) return;
  const float *dc = (const float *)out->grad->data;
  float *da = (float *)a->grad->data;
  if (p.dim == PLAST_DIM_ALL) {
    u64 n = o_numel(a);
    float g = op == O_MEAN ? dc[0] / (float)n : dc[0];
#pragma omp parallel for
    for (u64 i = 0; i < n; ++i) {
      u64 c[PLAST_MAX_NDIM];
      o_coords(i, a->shape, a->ndim, c);
      u64 od = o_offset(c, a->grad->strides, a->ndim);
      da[od] = da[od] + g;
    }
    return;
  }
  u64 dim = p.dim;
  int keep = p.keepdim != 0;
  u64 nout = o_numel(out);
  u64 len = a->shape[dim];
#pragma omp parallel for
  for (u64 o = 0; o < nout; ++o) {
    u64 oc[PLAST_MAX_NDIM], ic[PLAST_MAX_NDIM];
    o_coords(o, out->shape, out->ndim, oc);
    float g = dc[o_offset(oc, out->strides, out->ndim)];
    if (op == O_MEAN) g = g / (float)len;
    o_out_to_in(oc, ic, a->ndim, dim, keep);
    for (u64 k = 0; k < len; ++k) {
      ic[dim] = k;
      u64 od = o_offset(ic, a->grad->strides, a->ndim);
      da[od] = da[od] + g;
    }
  }
}

/* DEFINE_REDUCE_CPU_BACKWARD_MAX_MIN (reduce_ops.c:156-262): the gradient is split equally over
 * every element equal to the extreme. The full contiguous path recomputes the extreme with a
 * strict compare from the init value; the other paths read it from the forward output. */
static void o_max_min_backward(ORed op, Tensor **in, const Tensor *out, KernelParams p) {
  Tensor *a = in[0];
  if (!a->requires_grad) return;
  const float *pa = (const float *)a->data;
  const float *pc = (const float *)out->data;
  const float *dc = (const float *)out->grad->data;
  float *da = (float *)a->grad->data;
  if (p.dim == PLAST_DIM_ALL) {
    u64 n = o_numel(a);
    float ext;
    if (o_contig(a)) {
      ext = o_red_init(op);
      for (u64 i = 0; i < n; ++i)
        if (op == O_MAX ? pa[i] > ext : pa[i] < ext) ext = pa[i];
    } else {
      ext = pc[0];
    }
    u64 cnt = 0;
    u64 c[PLAST_MAX_NDIM];
    for (u64 i = 0; i < n; ++i) {
      o_coords(i, a->shape, a->ndim, c);
      if (pa[o_offset(c, a->strides, a->ndim)] == ext) cnt++;
    }
    if (cnt == 0) return;
    float g = dc[0] / (float)cnt;
    for (u64 i = 0; i < n; ++i) {
      o_coords(i, a->shape, a->ndim, c);
      if (pa[o_offset(c, a->strides, a->ndim)] == ext) {
        u64 od = o_offset(c, a->grad->strides, a->ndim);
        da[od] = da[od] + g;
      }
    }
    return;
  }
  u64 dim = p.dim;
  int keep = p.keepdim != 0;
  u64 nout = o_numel(out);
  u64 len = a->shape[dim];
#pragma omp parallel for
  for (u64 o = 0; o < nout; ++o) {
    u64 oc[PLAST_MAX_NDIM], ic[PLAST_MAX_NDIM];
    o_coords(o, out->shape, out->ndim, oc);
    u64 oo = o_offset(oc, out->strides, out->ndim);
    float ext = pc[oo];
    float g = dc[oo];
    o_out_to_in(oc, ic, a->ndim, dim, keep);
    u64 cnt = 0;
    for (u64 k = 0; k < len; ++k) {
      ic[dim] = k;
      if (pa[o_offset(ic, a->strides, a->ndim)] == ext) cnt++;
    }
    if (cnt == 0) continue;
    g = g / (float)cnt;
    for (u64 k = 0; k < len; ++k) {
      ic[dim] = k;
      if (pa[o_offset(ic, a->strides, a->ndim)] == ext) {
        u64 od = o_offset(ic, a->grad->strides, a->ndim);
        da[od] = da[od] + g;
      }
    }
  }
}

void oracle_sum_forward(const Tensor **i, Tensor *o, KernelParams p) { o_reduce_forward(O_SUM, i, o, p); }
void oracle_mean_forward(const Tensor **i, Tensor *o, KernelParams p) { o_reduce_forward(O_MEAN, i, o, p); }
void oracle_max_forward(const Tensor **i, Tensor *o, KernelParams p) { o_reduce_forward(O_MAX, i, o, p); }
void oracle_min_forward(const Tensor **i, Tensor *o, KernelParams p) { o_reduce_forward(O_MIN, i, o, p); }
void oracle_sum_backward(Tensor **i, const Tensor *o, KernelParams p) { o_sum_mean_backward(O_SUM, i, o, p); }
void oracle_mean_backward(Tensor **i, const Tensor *o, KernelParams p) { o_sum_mean_backward(O_MEAN, i, o, p); }
void oracle_max_backward(Tensor **i, const Tensor *o, KernelParams p) { o_max_min_backward(O_MAX, i, o, p); }
void oracle_min_backward(Tensor **i, const Tensor *o, KernelParams p) { o_max_min_backward(O_MIN, i, o, p); }

/* ---------------------------------------------------------------- argmax (no reference op) ----- */

/* First index of the maximum along `dim` (or over all elements in row-major order when
 * dim == PLAST_DIM_ALL); a NaN counts as the maximum, so the first NaN wins. This is
 * numpy.argmax, the only argmax the reference's code uses (train_mnist.py:51,107). */
static i64 o_argmax_run(const float *pa, u64 len, const u64 *ic0, u64 dim, const Tensor *a) {
  u64 ic[PLAST_MAX_NDIM];
  memcpy(ic, ic0, sizeof(u64) * a->ndim);
  i64 best = 0;
  float bv = 0.0f;
  for (u64 k = 0; k < len; ++k) {
    ic[dim] = k;
    float x = pa[o_offset(ic, a->strides, a->ndim)];
    if (k == 0) {
      bv = x;
      if (isnan(x)) return 0;
      continue;
    }
    if (isnan(x)) return (i64)k;
    if (x > bv) {
      bv = x;
      best = (i64)k;
    }
  }
  return best;
}

void oracle_argmax_forward(const Tensor **in, Tensor *out, KernelParams p) {
  const Tensor *a = in[0];
  const float *pa = (const float *)a->data;
  i64 *pc = (i64 *)out->data;
  if (p.dim == PLAST_DIM_ALL) {
    /* View the tensor as flat: walk it in logical row-major order. */
    u64 n = o_numel(a);
    i64 best = 0;
    float bv = 0.0f;
    u64 c[PLAST_MAX_NDIM];
    for (u64 i = 0; i < n; ++i) {
      o_coords(i, a->shape, a->ndim, c);
      float x = pa[o_offset(c, a->strides, a->ndim)];
      if (i == 0) {
        bv = x;
        if (isnan(x)) break;
        continue;
      }
      if (isnan(x)) {
        best = (i64)i;
        break;
      }
      if (x > bv) {
        bv = x;
        best = (i64)i;
      }
    }
    pc[0] = best;
    return;
  }
  u64 dim = p.dim;
  int keep = p.keepdim != 0;
  o_reduced_meta(a, dim, keep, out);
  u64 nout = o_numel(out);
#pragma omp parallel for
  for (u64 o = 0; o < nout; ++o) {
    u64 oc[PLAST_MAX_NDIM], ic[PLAST_MAX_NDIM];
    o_coords(o, out->shape, out->ndim, oc);
    o_out_to_in(oc, ic, a->ndim, dim, keep);
    pc[o] = o_argmax_run(pa, a->shape[dim], ic, dim, a);
  }
}

/* An integer index has no gradient. */
void oracle_argmax_backward(Tensor **in, const Tensor *out, KernelParams p) {
  (void)in;
  (void)out;
  (void)p;
}

/* ---------------------------------------------------------------- shape ops -------------------- */

/* shape_ops.c:59-80: alias data, swap shape/strides of axes params.dim and params.keepdim. */
void oracle_transpose_forward(const Tensor **in, Tensor *out, KernelParams p) {
  const Tensor *a = in[0];
  out->data = a->data;
  out->dtype = a->dtype;
  out->device = a->device;
  out->requires_grad = a->requires_grad;
  out->ndim = a->ndim;
  memcpy(out->shape, a->shape, sizeof(u64) * a->ndim);
  memcpy(out->strides, a->strides, sizeof(u64) * a->ndim);
  u64 x = p.dim, y = p.keepdim, t;
  t = out->shape[x]; out->shape[x] = out->shape[y]; out->shape[y] = t;
  t = out->strides[x]; out->strides[x] = out->strides[y]; out->strides[y] = t;
}

/* shape_ops.c:82-120: da[coords] += dout[coords with the two axes swapped]. */
void oracle_transpose_backward(Tensor **in, const Tensor *out, KernelParams p) {
  Tensor *a = in[0];
  if (!a->requires_grad || !out->grad) return;
  float *da = (float *)a->grad->data;
  const float *g = (const float *)out->grad->data;
  u64 n = o_numel(a);
  u64 c[PLAST_MAX_NDIM], ct[PLAST_MAX_NDIM];
  for (u64 i = 0; i < n; ++i) {
    o_coords(i, a->shape, a->ndim, c);
    memcpy(ct, c, sizeof(u64) * a->ndim);
    u64 t = ct[p.dim]; ct[p.dim] = ct[p.keepdim]; ct[p.keepdim] = t;
    u64 od = o_offset(c, a->grad->strides, a->ndim);
    da[od] = da[od] + g[o_offset(ct, out->grad->strides, out->ndim)];
  }
}

/* shape_ops.c:54-57 + cpu_utils.c:59-76: alias data, stride 0 on new or size-1 expanded axes.
 * The caller fills output->shape/ndim with the target shape. */
void oracle_expand_forward(const Tensor **in, Tensor *out, KernelParams p) {
  (void)p;
  const Tensor *a = in[0];
  out->data = a->data;
  out->dtype = a->dtype;
  out->device = a->device;
  out->requires_grad = a->requires_grad;
  out->grad = a->grad;
  u64 lead = out->ndim - a->ndim;
  for (u64 d = 0; d < out->ndim; ++d) {
    if (d < lead) {
      out->strides[d] = 0;
    } else {
      u64 s = d - lead;
      out->strides[d] = (a->shape[s] == 1 && out->shape[d] > 1) ? 0 : a->strides[s];
    }
  }
}

/* ---------------------------------------------------------------- softmax cross-entropy -------- */

/* The reference's cross-entropy op chain (src/api/loss.c:97-169; plast/nn/functional.py:312-333)
 * up to and including NEG, evaluated row by row with each node's rounding:
 *   m = MAX(x, dim=1)            serial `acc > x ? acc : x` from -FLT_MAX
 *   s = SUM(EXP(x - m), dim=1)   serial fp32 sum of expf
 *   l = LOG(s)
 *   t = SUM(onehot * ((x - m) - l), dim=1)   serial, onehot built from the integer label
 *   loss = NEG(t)                0 - t inside the AVX2 blocks, -t in the scalar tail
 * inputs: [0] logits [N,C] fp32 contiguous, [1] labels [N] int32, [2] stats [N,2] fp32 that
 * receives (m, l) per row for the backward. output: [N] fp32 per-row loss. The MEAN over rows is
 * a separate reduction node, as in the reference chain. */
void oracle_softmax_cross_entropy_forward(const Tensor **in, Tensor *out, KernelParams p) {
  (void)p;
  const Tensor *x = in[0];
  const i32 *lab = (const i32 *)in[1]->data;
  float *stats = (float *)in[2]->data;
  float *loss = (float *)out->data;
  u64 N = x->shape[0], C = x->shape[1];
  const float *px = (const float *)x->data;
  u64 se = o_simd_end(N);
#pragma omp parallel for
  for (u64 r = 0; r < N; ++r) {
    const float *row = px + r * C;
    float m = -FLT_MAX;
    for (u64 j = 0; j < C; ++j) m = m > row[j] ? m : row[j];
    float s = 0.0f;
    for (u64 j = 0; j < C; ++j) s = s + expf(row[j] - m);
    float l = logf(s);
    float t = 0.0f;
    for (u64 j = 0; j < C; ++j) {
      float oh = (i64)j == (i64)lab[r] ? 1.0f : 0.0f;
      t = t + oh * ((row[j] - m) - l);
    }
    stats[2 * r] = m;
    stats[2 * r + 1] = l;
    loss[r] = r < se ? 0.0f - t : -t;
  }
}

/* d logits[i,j] += dloss[i] * (softmax[i,j] - onehot[i,j]), softmax = expf((x - m) - l) from the
 * forward's stats. With dloss = 1/N (the MEAN node's backward) this is (softmax - onehot)/N, the
 * closed form of backpropagation through the reference chain (its max path contributes only
 * rounding residue). */
void oracle_softmax_cross_entropy_backward(Tensor **in, const Tensor *out, KernelParams p) {
  (void)p;
  Tensor *x = in[0];
  if (!x->requires_grad) return;
  const i32 *lab = (const i32 *)in[1]->data;
  const float *stats = (const float *)in[2]->data;
  const float *dl = (const float *)out->grad->data;
  float *dx = (float *)x->grad->data;
  const float *px = (const float *)x->data;
  u64 N = x->shape[0], C = x->shape[1];
#pragma omp parallel for
  for (u64 r = 0; r < N; ++r) {
    float m = stats[2 * r], l = stats[2 * r + 1], g = dl[r];
    for (u64 j = 0; j < C; ++j) {
      float sm = expf((px[r * C + j] - m) - l);
      float oh = (i64)j == (i64)lab[r] ? 1.0f : 0.0f;
      dx[r * C + j] = dx[r * C + j] + g * (sm - oh);
    }
  }
}

/* ---------------------------------------------------------------- config-2 chain --------------- */

void oracle_fused_chain2(const float *a, const float *b, const float *c, float *out, u64 n) {
  u64 se = o_simd_end(n);
#pragma omp parallel for
  for (u64 i = 0; i < n; ++i) {
    float t = a[i] * b[i];
    t = t + c[i];
    t = t > 0 ? t : t * 0.0f;
    t = i < se ? 0.0f - t : -t;
    out[i] = expf(t);
  }
}

/* ---------------------------------------------------------------- optimizers -------------------- */

/* src/optimizers/cpu/sgd.c:16-28: data[j] -= lr * grad[j] over numel(param) floats. */
void oracle_sgd_step(SGD *o, Tensor **params, int n) {
  if (!o) return;
  for (int i = 0; i < n; ++i) {
    Tensor *p = params[i];
    if (!p || !p->grad) continue;
    float *d = (float *)p->data;
    const float *g = (const float *)p->grad->data;
    for (u64 j = 0; j < o_numel(p); ++j) d[j] -= o->lr * g[j];
  }
}

/* Zero-filled contiguous host tensors shaped like each parameter (adam.c:29-46 allocates them
 * with init(..., zeros) on the first step). */
static Tensor **o_moments(Tensor **params, int n) {
  Tensor **m = (Tensor **)calloc((size_t)n, sizeof(Tensor *));
  for (int i = 0; m && i < n; ++i) {
    if (!params[i]) continue;
    Tensor *t = (Tensor *)calloc(1, sizeof(Tensor));
    u64 cnt = o_numel(params[i]);
    t->data = calloc(cnt ? cnt : 1, sizeof(float));
    t->ndim = params[i]->ndim;
    u64 s = 1;
    for (u64 d = t->ndim; d-- > 0;) {
      t->shape[d] = params[i]->shape[d];
      t->strides[d] = s;
      s *= t->shape[d];
    }
    t->dtype = FLOAT32;
    t->device = CPU;
    m[i] = t;
  }
  return m;
}

void oracle_optimizer_release(Tensor **m, Tensor **v, int n) {
  Tensor **arrs[2] = {m, v};
  for (int a = 0; a < 2; ++a) {
    if (!arrs[a]) continue;
    for (int i = 0; i < n; ++i)
      if (arrs[a][i]) {
        free(arrs[a][i]->data);
        free(arrs[a][i]);
      }
    free(arrs[a]);
  }
}

/* adam.c:21-68 and adamw.c:19-69 share everything but AdamW's decoupled decay step
 * (adamw.c:130), which runs first in each element's update. */
static void o_adam_like(float lr, float b1, float b2, float eps, float wd, int decoupled, int *t,
                        Tensor ***mp, Tensor ***vp, Tensor **params, int n) {
  (*t)++;
  if (!*mp) {
    *mp = o_moments(params, n);
    *vp = o_moments(params, n);
  }
  /* the reference's expression: float * double sqrt / float, rounded once to float */
  float lr_t = lr * sqrt(1.0f - powf(b2, *t)) / (1.0f - powf(b1, *t));
  for (int i = 0; i < n; ++i) {
    Tensor *p = params[i];
    if (!p || !p->grad) continue;
    float *d = (float *)p->data;
    const float *g = (const float *)p->grad->data;
    float *m = (float *)(*mp)[i]->data;
    float *v = (float *)(*vp)[i]->data;
    for (u64 j = 0; j < o_numel(p); ++j) {
      if (decoupled) d[j] -= lr * wd * d[j];
      m[j] = b1 * m[j] + (1.0f - b1) * g[j];
      v[j] = b2 * v[j] + (1.0f - b2) * g[j] * g[j];
      d[j] -= lr_t * m[j] / (sqrtf(v[j]) + eps);
    }
  }
}

void oracle_adam_step(Adam *o, Tensor **params, int n) {
  if (!o) return;
  o_adam_like(o->lr, o->beta1, o->beta2, o->epsilon, 0.0f, 0, &o->t, &o->m, &o->v, params, n);
}

void oracle_adamw_step(AdamW *o, Tensor **params, int n) {
  if (!o) return;
  o_adam_like(o->lr, o->beta1, o->beta2, o->epsilon, o->weight_decay, 1, &o->t, &o->m, &o->v,
              params, n);
}

/* src/optimizers/cpu/zero_grad.c:4-11 */
void oracle_zero_grad(Tensor *t) {
  if (!t || !t->grad) return;
  float *g = (float *)t->grad->data;
  for (u64 i = 0; i < o_numel(t->grad); ++i) g[i] = 0.0f;
}

/* ---------------------------------------------------------------- matmul epilogue pieces -------- */

/* fused_ops.c:19-21, 105-111: dc[i] = dout[i] * (out[i] > 0 ? 1 : alpha). */
void oracle_relu_grad_modulate(const float *dout, const float *out, float *dc, u64 n, float alpha) {
  for (u64 i = 0; i < n; ++i) dc[i] = dout[i] * (out[i] > 0.0f ? 1.0f : alpha);
}

/* fused_ops.c:294-304: dbias zeroed, then rows added in index order. */
void oracle_bias_grad_reduce(const float *dc, float *dbias, u64 n, u64 cols) {
  for (u64 c = 0; c < cols; ++c) dbias[c] = 0.0f;
  for (u64 i = 0; i < n; ++i) dbias[i % cols] += dc[i];
}
