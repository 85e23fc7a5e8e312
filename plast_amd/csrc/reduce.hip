// reduce.hip — sum / mean / max / min / argmax forward and backward entry points.
#include "ew_impl.hpp"
#include "red_impl.hpp"

namespace plast {
namespace {

// Output metadata of a reduction over `dim` (cpu_utils.c:121-154), written into `out` as the
// reference CPU forward does (reduce_ops.c:80-81).
void reduced_meta(const Tensor *a, uint64_t dim, bool keep, Tensor *out) {
  uint64_t nd = 0;
  for (uint64_t d = 0; d < a->ndim; ++d) {
    if (d == dim) {
      if (keep) out->shape[nd++] = 1;
    } else {
      out->shape[nd++] = a->shape[d];
    }
  }
  if (nd == 0) out->shape[nd++] = 1;
  out->ndim = nd;
  uint64_t s = 1;
  for (uint64_t d = nd; d-- > 0;) {
    out->strides[d] = s;
    s *= out->shape[d];
  }
}

// Stride, inside a's iteration space, of a tensor laid out like the reduction output with
// strides `ost` (axis `dim` of `a` maps to no output axis, or to a size-1 one when keepdim).
void output_strides_in_input_space(const Tensor *a, uint64_t dim, bool keep, const uint64_t *ost,
                                   int64_t *st) {
  for (uint64_t d = 0; d < a->ndim; ++d) {
    if (d == dim || a->shape[d] == 1) {
      st[d] = 0;
    } else {
      const uint64_t od = keep ? d : (d < dim ? d : d - 1);
      st[d] = int64_t(ost[od]);
    }
  }
}

bool dims_ok(const Tensor *a, KernelParams p, const char *where) {
  if (p.dim != PLAST_DIM_ALL && p.dim >= a->ndim) {
    report_error(where, "dim %llu out of range for rank %llu", (unsigned long long)p.dim,
                 (unsigned long long)a->ndim);
    return false;
  }
  if (a->dtype != FLOAT32) {
    report_error(where, "unsupported dtype %d", int(a->dtype));
    return false;
  }
  return true;
}

template <class Comb>
void reduce_forward(const Tensor **in, Tensor *out, KernelParams p, Post post,
                    const char *where) {
  if (!ensure_init()) return;
  const Tensor *a = in[0];
  if (!dims_ok(a, p, where)) return;
  const bool keep = p.keepdim != 0;
  Space s;
  s.rank = int(a->ndim);
  for (int d = 0; d < s.rank; ++d) {
    s.shape[d] = a->shape[d];
    s.st[0][d] = a->shape[d] == 1 ? 0 : int64_t(a->strides[d]);
  }
  float divisor;
  if (p.dim == PLAST_DIM_ALL) {
    for (int d = 0; d < s.rank; ++d) s.st[1][d] = 0;
    divisor = float(numel(a));
  } else {
    reduced_meta(a, p.dim, keep, out);
    output_strides_in_input_space(a, p.dim, keep, out->strides, s.st[1]);
    divisor = float(a->shape[p.dim]);
  }
  const void *ins[1] = {a->data};
  launch_reduction<Load1, Comb>(Load1{}, ins, out->data, s, post, divisor, where);
  finish(where);
}

// da += dc (/ n) broadcast back over the reduced axis (reduce_ops.c:89-154).
void sum_mean_backward(Tensor **in, const Tensor *out, KernelParams p, bool mean,
                       const char *where) {
  if (!ensure_init()) return;
  Tensor *a = in[0];
  if (!a->requires_grad || !a->grad) return;
  if (!dims_ok(a, p, where)) return;
  if (!out->grad) {
    report_error(where, "output has no gradient");
    return;
  }
  const bool keep = p.keepdim != 0;
  Space s;
  s.rank = int(a->ndim);
  for (int d = 0; d < s.rank; ++d) {
    s.shape[d] = a->shape[d];
    s.st[0][d] = a->shape[d] == 1 ? 0 : int64_t(a->grad->strides[d]);
    s.st[2][d] = s.st[0][d];
  }
  uint64_t len;
  if (p.dim == PLAST_DIM_ALL) {
    for (int d = 0; d < s.rank; ++d) s.st[1][d] = 0;
    len = numel(a);
  } else {
    output_strides_in_input_space(a, p.dim, keep, out->strides, s.st[1]);
    len = a->shape[p.dim];
  }
  const void *ins[2] = {a->grad->data, out->grad->data};
  if (mean) {
    AccumDivBody body;
    body.divisor = float(len);
    launch_elementwise(body, ins, a->grad->data, s, where);
  } else {
    launch_elementwise(AccumBody{}, ins, a->grad->data, s, where);
  }
  finish(where);
}

// operands: da, a, extreme, dc, count -> da + dc/count where a == extreme (reduce_ops.c:156-262)
struct ExtGradBody : ScalarBody<ExtGradBody> {
  static constexpr int NIN = 5;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    if (v[4] > 0.0f && v[1] == v[2]) return v[0] + v[3] / v[4];
    return v[0];
  }
};

// NaN-ignoring extreme from the init value with a strict compare: the value the reference's full
// contiguous max/min backward recomputes (reduce_ops.c:159-164). Only compared with ==, so the
// sign of a zero result is immaterial.
template <bool IS_MAX>
struct StrictExtComb {
  using Part = float;
  using Out = float;
  static constexpr bool kExact = false;
  __device__ static Part empty() { return IS_MAX ? -FLT_MAX : FLT_MAX; }
  __device__ static Part merge(Part a, Part b) { return IS_MAX ? fmaxf(a, b) : fminf(a, b); }
  __device__ static void first(Part &p, float x, int64_t) { p = merge(empty(), x); }
  __device__ static void next(Part &p, float x, int64_t) { p = merge(p, x); }
  __device__ static Part shfl(Part p, int m) { return __shfl_xor(p, m); }
};

template <bool IS_MAX>
void ext_backward(Tensor **in, const Tensor *out, KernelParams p, const char *where) {
  if (!ensure_init()) return;
  Tensor *a = in[0];
  if (!a->requires_grad || !a->grad) return;
  if (!dims_ok(a, p, where)) return;
  if (!out->grad) {
    report_error(where, "output has no gradient");
    return;
  }
  const bool keep = p.keepdim != 0;
  const bool all = p.dim == PLAST_DIM_ALL;
  const uint64_t nout = all ? 1 : numel(out);
  // slot-1 temporaries: [count per output][recomputed extreme (full contiguous case)]
  float *tmp = static_cast<float *>(workspace(sizeof(float) * (nout + 1), 1));
  if (!tmp) return;
  float *cnt = tmp;
  const float *ext = static_cast<const float *>(out->data);
  Space s;
  s.rank = int(a->ndim);
  for (int d = 0; d < s.rank; ++d) {
    s.shape[d] = a->shape[d];
    s.st[0][d] = a->shape[d] == 1 ? 0 : int64_t(a->strides[d]);
  }
  int64_t ost[kMaxRank];       // where each point of a's space finds its output element
  int64_t cst[kMaxRank];       // same for the contiguous count buffer
  if (all) {
    for (int d = 0; d < s.rank; ++d) ost[d] = cst[d] = 0;
    if (contiguous(a)) {
      Space e = s;
      for (int d = 0; d < e.rank; ++d) e.st[1][d] = 0;
      float *ext_buf = tmp + nout;
      const void *ins[1] = {a->data};
      launch_reduction<Load1, StrictExtComb<IS_MAX>>(Load1{}, ins, ext_buf, e, Post::Write, 1.0f,
                                                     where);
      ext = ext_buf;
    }
  } else {
    output_strides_in_input_space(a, p.dim, keep, out->strides, ost);
    uint64_t cs[kMaxRank];
    uint64_t c = 1;
    for (uint64_t d = out->ndim; d-- > 0;) {
      cs[d] = c;
      c *= out->shape[d];
    }
    output_strides_in_input_space(a, p.dim, keep, cs, cst);
  }
  // tie count per output
  {
    Space c = s;
    for (int d = 0; d < c.rank; ++d) {
      c.st[1][d] = ost[d];
      c.st[2][d] = cst[d];
    }
    const void *ins[2] = {a->data, ext};
    launch_reduction<EqualCount, SumComb>(EqualCount{}, ins, cnt, c, Post::Write, 1.0f, where);
  }
  // accumulate
  {
    Space g;
    g.rank = s.rank;
    for (int d = 0; d < g.rank; ++d) {
      g.shape[d] = s.shape[d];
      g.st[0][d] = a->shape[d] == 1 ? 0 : int64_t(a->grad->strides[d]);
      g.st[1][d] = s.st[0][d];
      g.st[2][d] = ost[d];
      g.st[3][d] = ost[d];
      g.st[4][d] = cst[d];
      g.st[5][d] = g.st[0][d];
    }
    const void *ins[5] = {a->grad->data, a->data, ext, out->grad->data, cnt};
    launch_elementwise(ExtGradBody{}, ins, a->grad->data, g, where);
  }
  finish(where);
}

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

void sum_hip_forward(const Tensor **i, Tensor *o, KernelParams p) {
  reduce_forward<SumComb>(i, o, p, Post::Write, "sum_hip_forward");
}
void mean_hip_forward(const Tensor **i, Tensor *o, KernelParams p) {
  reduce_forward<SumComb>(i, o, p, Post::Mean, "mean_hip_forward");
}
void max_hip_forward(const Tensor **i, Tensor *o, KernelParams p) {
  reduce_forward<ExtComb<true>>(i, o, p, Post::Write, "max_hip_forward");
}
void min_hip_forward(const Tensor **i, Tensor *o, KernelParams p) {
  reduce_forward<ExtComb<false>>(i, o, p, Post::Write, "min_hip_forward");
}
void argmax_hip_forward(const Tensor **i, Tensor *o, KernelParams p) {
  if (o->dtype != INT64) {
    report_error("argmax_hip_forward", "output dtype must be INT64, got %d", int(o->dtype));
    return;
  }
  reduce_forward<ArgmaxComb>(i, o, p, Post::Write, "argmax_hip_forward");
}

void sum_hip_backward(Tensor **i, const Tensor *o, KernelParams p) {
  sum_mean_backward(i, o, p, false, "sum_hip_backward");
}
void mean_hip_backward(Tensor **i, const Tensor *o, KernelParams p) {
  sum_mean_backward(i, o, p, true, "mean_hip_backward");
}
void max_hip_backward(Tensor **i, const Tensor *o, KernelParams p) {
  ext_backward<true>(i, o, p, "max_hip_backward");
}
void min_hip_backward(Tensor **i, const Tensor *o, KernelParams p) {
  ext_backward<false>(i, o, p, "min_hip_backward");
}
// An integer index carries no gradient.
void argmax_hip_backward(Tensor **i, const Tensor *o, KernelParams p) {
  (void)i;
  (void)o;
  (void)p;
}

}  // extern "C"
