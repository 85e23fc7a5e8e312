// red_impl.hpp — the reduction engine.
//
// A reduction problem is a Space whose last operand is the target: the target has stride 0 on
// every reduced axis. After collapsing, one of three kernel families runs:
//   rows   — the only reduced axis is the innermost and is unit-stride: one wave64 per (row,
//            segment), float4 loads, wave shuffle reduction; long rows split into segments whose
//            partials a finalize pass combines in order;
//   cols   — the innermost axis is kept and unit-stride, one reduced axis: each lane owns four
//            adjacent outputs and walks its chunk of the reduced axis in order; chunks combine in
//            order in a finalize pass (no atomics anywhere, so results are deterministic);
//   generic— any layout: one lane per output, serial walk in index order.
//
// Max/min reproduce the reference's literal fold `acc > x ? acc : x` from -FLT_MAX
// (reduce_ops.c:9, 26-30) bit for bit, including NaN (a NaN resets the fold: the result is the
// fold of what follows the last NaN) and signed zeros (ties keep the later element). Per index
// range the fold is summarised as (r, flags): r is the fold started at the range's first element,
// INDEP set when the range contains a NaN (then the range's result does not depend on what came
// before). Ranges combine in index order.
#pragma once

#include <cfloat>
#include <type_traits>

#include "common.hpp"

namespace plast {

// ------------------------------------------------------------------------- producers
// A producer turns the NIN operand values at one point of the space into the reduced value.

// A producer with kStore = true also writes its values out, at operand 0's offsets from its `dst`
// (the leading-axis kernel only; launch_reduction launches nothing and returns false for any other
// layout). Producers without the member do not store.
template <class P, class = void>
struct StoresValues : std::false_type {};
template <class P>
struct StoresValues<P, std::void_t<decltype(P::kStore)>> : std::bool_constant<P::kStore> {};
template <class P>
constexpr bool kStores = StoresValues<P>::value;

struct Load1 {
  static constexpr int NIN = 1;
  __device__ __forceinline__ float eval(const float *v) const { return v[0]; }
};

// 1 where a == e (e broadcast from the forward output), else 0: tie count of max/min backward.
struct EqualCount {
  static constexpr int NIN = 2;
  __device__ __forceinline__ float eval(const float *v) const { return v[0] == v[1] ? 1.0f : 0.0f; }
};

// dout * (z > 0 ? 1 : alpha), stored to dst as it is summed: the relu-gradient modulation of the
// fused matmul epilogues' backward (matmul_relu.cu:138-144) fused with the bias-gradient sum.
struct ReluGradStore {
  static constexpr int NIN = 2;
  static constexpr bool kStore = true;
  float alpha;
  float *dst;
  __device__ __forceinline__ float eval(const float *v) const {
    return v[0] * (v[1] > 0.0f ? 1.0f : alpha);
  }
};

// The gradient a fused leaky_relu(x + bias) node hands to its ADD, for the operands (dout, y):
// 0 + dout * (y > 0 ? 1 : alpha), the chain's leaky backward (unary_ops.c:236-258) accumulated into
// the intermediate's zeroed gradient, with its mask read from the node's output y (for alpha >= 0,
// y > 0 exactly where x + bias > 0). Summed over rows: the bias's gradient.
struct LeakyAddGrad {
  static constexpr int NIN = 2;
  float alpha;
  __device__ __forceinline__ float eval(const float *v) const {
    return 0.0f + v[0] * (v[1] > 0.0f ? 1.0f : alpha);
  }
};

// The same term for the operands (dout, y, g), summed, with g + term stored to dst (g's own
// buffer): x's gradient from the ADD's backward (kernel_macros.h:283-299) written in the pass that
// sums the bias's. A refold recomputes its terms from dout and y, which the stores leave intact.
struct LeakyAddGradStore {
  static constexpr int NIN = 3;
  static constexpr bool kStore = true;
  static constexpr bool kRefoldInputs = true;
  float alpha;
  float *dst;
  __device__ __forceinline__ float eval(const float *v) const {
    return 0.0f + v[0] * (v[1] > 0.0f ? 1.0f : alpha);
  }
  __device__ __forceinline__ float stored(const float *v, float y) const { return v[2] + y; }
};

// What a storing producer writes for the value y it sums at operands v: y itself, or, for one
// with kRefoldInputs, its own stored(v, y).
template <class P, class = void>
struct StoresOther : std::false_type {};
template <class P>
struct StoresOther<P, std::void_t<decltype(P::kRefoldInputs)>> : std::bool_constant<P::kRefoldInputs> {};
template <class P>
__device__ __forceinline__ float stored_value(const P &prod, const float *v, float y) {
  if constexpr (StoresOther<P>::value) return prod.stored(v, y);
  else return y;
}

// ------------------------------------------------------------------------- combiners

enum class Post : int { Write = 0, Mean = 1, Accum = 2 };

struct SumComb {
  using Part = float;
  using Out = float;
  static constexpr bool kExact = false;
  __device__ static Part empty() { return 0.0f; }
  // the reference's accumulator starts at 0.0f, so a lone -0 sums to +0
  __device__ static void first(Part &p, float x, int64_t) { p = 0.0f + x; }
  __device__ static void next(Part &p, float x, int64_t) { p = p + x; }
  __device__ static Part merge(Part a, Part b) { return a + b; }
  __device__ static Part shfl(Part p, int m) { return __shfl_xor(p, m); }
};

// Exact max (IS_MAX) / min fold summaries.
constexpr uint32_t kIndep = 1, kNonEmpty = 2;
struct ExtPart {
  float r;
  uint32_t flags;
};

template <bool IS_MAX>
struct ExtComb {
  using Part = ExtPart;
  using Out = float;
  static constexpr bool kExact = true;
  __device__ static float pick(float acc, float x) {
    if constexpr (IS_MAX) return acc > x ? acc : x;
    else return acc < x ? acc : x;
  }
  __device__ static float init() { return IS_MAX ? -FLT_MAX : FLT_MAX; }
  __device__ static Part empty() { return Part{0.0f, 0u}; }
  __device__ static void first(Part &p, float x, int64_t) {
    p.r = x;
    p.flags = kNonEmpty | (x != x ? kIndep : 0u);
  }
  __device__ static void next(Part &p, float x, int64_t) {
    p.r = pick(p.r, x);
    if (x != x) p.flags |= kIndep;
  }
  // a covers earlier indices than b
  __device__ static Part merge(Part a, Part b) {
    if (!(b.flags & kNonEmpty)) return a;
    if (!(a.flags & kNonEmpty) || (b.flags & kIndep)) return b;
    return Part{pick(a.r, b.r), a.flags};
  }
  // value of the reference's accumulator after folding the whole summarised range from init
  __device__ static float finish(Part p) {
    if (!(p.flags & kNonEmpty)) return init();
    if (p.flags & kIndep) return p.r;
    return pick(init(), p.r);
  }
};

// numpy argmax: first NaN if any, else first index of the maximum.
struct ArgPart {
  float v;
  int64_t i;
};
struct ArgmaxComb {
  using Part = ArgPart;
  using Out = int64_t;
  static constexpr bool kExact = false;
  __device__ static Part empty() { return Part{-__builtin_huge_valf(), INT64_MAX}; }
  // Order-free: the better of two (value, index) candidates.
  __device__ static Part merge(Part a, Part b) {
    const bool an = a.v != a.v, bn = b.v != b.v;
    if (an || bn) {
      if (an && bn) return a.i < b.i ? a : b;
      return an ? a : b;
    }
    if (a.v > b.v) return a;
    if (b.v > a.v) return b;
    return a.i < b.i ? a : b;
  }
  __device__ static void first(Part &p, float x, int64_t k) { p = Part{x, k}; }
  __device__ static void next(Part &p, float x, int64_t k) { p = merge(p, Part{x, k}); }
  __device__ static Part shfl(Part p, int m) {
    Part q;
    q.v = __shfl_xor(p.v, m);
    q.i = __shfl_xor(p.i, m);
    return q;
  }
};

// ------------------------------------------------------------------------- arguments

template <int NIN>
struct RedArgs {
  const float *in[NIN];
  void *out;
  int64_t ost[NIN][kMaxRank];  // operand strides on the kept (output) axes, innermost excluded
  int64_t tst[kMaxRank];       // target strides on the same axes
  MagicDiv dv[kMaxRank];       // extents of those axes
  int nouter;                  // number of such axes
  int64_t rst[NIN];            // operand strides along the reduced axis
  int64_t kst[NIN];            // operand strides along the kept innermost axis (cols)
  int64_t tkst;                // target stride along the kept innermost axis (cols)
  uint64_t len;                // reduced extent
  uint64_t rows;               // rows (rows kernel) / outer count (cols kernel)
  uint64_t inner;              // kept innermost extent (cols kernel)
  uint32_t segs;               // segments per row / chunks of the reduced axis
  uint64_t seglen;
  uint32_t vec_mask;           // bit k: operand k is streamed with float4 loads (else splat)
  void *part;                  // partial summaries [segs][outputs] when segs > 1
  int post;                    // Post
  float divisor;               // Mean
};

// Outer-axis decode: index -> per-operand base offsets and the target offset.
template <int NIN>
__device__ __forceinline__ void decode_outer(const RedArgs<NIN> &A, uint32_t idx, int64_t *base,
                                             int64_t &tbase) {
#pragma unroll
  for (int k = 0; k < NIN; ++k) base[k] = 0;
  tbase = 0;
  for (int d = A.nouter - 1; d >= 0; --d) {
    const uint32_t nxt = A.dv[d].div(idx);
    const int64_t c = int64_t(idx - nxt * A.dv[d].d);
    idx = nxt;
#pragma unroll
    for (int k = 0; k < NIN; ++k) base[k] += c * A.ost[k][d];
    tbase += c * A.tst[d];
  }
}

template <class Comb>
__device__ __forceinline__ void store_final(void *out, int64_t off, const typename Comb::Part &p,
                                            int post, float divisor) {
  if constexpr (std::is_same<Comb, ArgmaxComb>::value) {
    static_cast<int64_t *>(out)[off] = p.i == INT64_MAX ? 0 : p.i;
  } else if constexpr (Comb::kExact) {
    static_cast<float *>(out)[off] = Comb::finish(p);
  } else {
    float *o = static_cast<float *>(out);
    if (post == int(Post::Accum)) o[off] = o[off] + p;
    else if (post == int(Post::Mean)) o[off] = p / divisor;
    else o[off] = p;
  }
}

// ------------------------------------------------------------------------- rows kernel

// The i-th term of a serial refold. A storing producer's terms are read back from where it stored
// them (only a sum over a leading axis refolds one, after its workgroup or launch has stored every
// term of the column): its inputs may have been overwritten by those stores (dc written over
// dout). One with kRefoldInputs stores something other than its terms, over none of the operands
// its terms read, and recomputes them.
template <class Prod, int NIN>
__device__ __forceinline__ float value_at(const RedArgs<NIN> &A, const Prod &prod,
                                          const int64_t *base, uint64_t i) {
  if constexpr (kStores<Prod> && !StoresOther<Prod>::value) {
    return prod.dst[base[0] + int64_t(i) * A.rst[0]];
  } else {
    float v[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) v[k] = A.in[k][base[k] + int64_t(i) * A.rst[k]];
    return prod.eval(v);
  }
}

template <class T>
__device__ __forceinline__ T wave_max_t(T v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    T o = __shfl_xor(v, m);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ float wave_fmax(float v, bool is_max) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    float o = __shfl_xor(v, m);
    v = is_max ? fmaxf(v, o) : fminf(v, o);
  }
  return v;
}
__device__ __forceinline__ bool wave_any(bool b) { return __any(b); }

// Exact fold summary of [b, e) by one wave, used when the fast path saw a NaN or a zero extreme.
template <bool IS_MAX, class Prod, int NIN>
__device__ ExtPart exact_range(const RedArgs<NIN> &A, const Prod &prod, const int64_t *base,
                               uint64_t b, uint64_t e, int lane) {
  // last NaN
  int64_t last_nan = -1;
  for (uint64_t i = b + lane; i < e; i += 64) {
    const float x = value_at(A, prod, base, i);
    if (x != x) last_nan = int64_t(i);
  }
  last_nan = wave_max_t(last_nan);
  const uint64_t s = last_nan >= 0 ? uint64_t(last_nan) + 1 : b;
  if (s >= e) {
    // the range ends in a NaN: the fold's value is that NaN
    return ExtPart{value_at(A, prod, base, uint64_t(last_nan)), kNonEmpty | kIndep};
  }
  float m = IS_MAX ? -__builtin_huge_valf() : __builtin_huge_valf();
  for (uint64_t i = s + lane; i < e; i += 64) {
    const float x = value_at(A, prod, base, i);
    m = IS_MAX ? fmaxf(m, x) : fminf(m, x);
  }
  m = wave_fmax(m, IS_MAX);
  float r = m;
  if (m == 0.0f) {
    // several zeros may tie: the fold keeps the last one, whose sign decides the bits
    int64_t last_zero = -1;
    for (uint64_t i = s + lane; i < e; i += 64)
      if (value_at(A, prod, base, i) == 0.0f) last_zero = int64_t(i);
    last_zero = wave_max_t(last_zero);
    r = value_at(A, prod, base, uint64_t(last_zero));
  }
  return ExtPart{r, kNonEmpty | (last_nan >= 0 ? kIndep : 0u)};
}

// A parallel-order sum that is not finite (an overflow, or inf - inf) can differ from the
// reference's serial one, whose outcome depends on the order: such an output is summed again in
// the reference's order (index order from 0.0f, one rounding per addition: reduce_ops.c:57-61).
template <class Comb>
constexpr bool kSerialSum = std::is_same<Comb, SumComb>::value;

__device__ __forceinline__ bool finite_sum(float p) { return fabsf(p) <= FLT_MAX; }

// By one lane: the serial sum of elements [0, len) at base.
template <class Prod, int NIN>
__device__ float serial_sum_lane(const RedArgs<NIN> &A, const Prod &prod, const int64_t *base,
                                 uint64_t len) {
  float s = 0.0f;
  for (uint64_t i = 0; i < len; ++i) s = s + value_at(A, prod, base, i);
  return s;
}

// By a wave, for a whole row: a NaN operand makes every order's sum NaN, so the wave first looks
// for one (in parallel) and only a row without one is refolded, by lane 0; every lane returns the
// result.
template <class Prod, int NIN>
__device__ float serial_sum_wave(const RedArgs<NIN> &A, const Prod &prod, const int64_t *base,
                                 uint64_t len, float p, int lane) {
  bool nan = false;
  for (uint64_t i = lane; i < len; i += 64) {
    const float x = value_at(A, prod, base, i);
    nan = nan || (x != x);
  }
  if (__any(nan)) return p;
  float r = 0.0f;
  if (lane == 0) r = serial_sum_lane(A, prod, base, len);
  return __shfl(r, 0);
}

constexpr int kRowUnroll = PLAST_ROW_UNROLL;  // float4 loads in flight per lane per operand

template <class Prod, class Comb, bool VEC>
__global__ __launch_bounds__(kBlock) void red_rows_kernel(RedArgs<Prod::NIN> A, Prod prod) {
  constexpr int NIN = Prod::NIN;
  using Part = typename Comb::Part;
  const int lane = threadIdx.x & 63;
  const uint32_t bx = blockIdx.x;
  const uint64_t task = uint64_t(bx) * (kBlock / 64) + (threadIdx.x >> 6);
  if (task >= A.rows * A.segs) return;  // whole wave exits together
  const uint32_t row = uint32_t(task / A.segs);
  const uint32_t seg = uint32_t(task - uint64_t(row) * A.segs);
  int64_t base[NIN], tbase;
  decode_outer(A, row, base, tbase);
  const uint64_t b = uint64_t(seg) * A.seglen;
  const uint64_t e = b + A.seglen < A.len ? b + A.seglen : A.len;

  Part p;
  if constexpr (Comb::kExact) {
    // fast path: plain extreme ignoring NaN, plus a NaN flag
    constexpr bool IS_MAX = std::is_same<Comb, ExtComb<true>>::value;
    float m = IS_MAX ? -__builtin_huge_valf() : __builtin_huge_valf();
    bool nan = false;
    auto take = [&](float x) {
      m = IS_MAX ? fmaxf(m, x) : fminf(m, x);
      nan = nan || (x != x);
    };
    if constexpr (VEC) {
      for (uint64_t i0 = b + uint64_t(lane) * 4; i0 < e; i0 += 256 * kRowUnroll) {
        f4 x[kRowUnroll][NIN];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const uint64_t i = i0 + uint64_t(u) * 256;
          if (i < e)
#pragma unroll
            for (int k = 0; k < NIN; ++k)
              x[u][k] = (A.vec_mask >> k & 1u)
                            ? __builtin_nontemporal_load(
                                  reinterpret_cast<const f4 *>(A.in[k] + base[k] + int64_t(i)))
                            : f4(A.in[k][base[k]]);
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          if (i0 + uint64_t(u) * 256 >= e) continue;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float v[NIN];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = x[u][k][c];
            take(prod.eval(v));
          }
        }
      }
    } else {
      for (uint64_t i = b + lane; i < e; i += 64) take(value_at(A, prod, base, i));
    }
    m = wave_fmax(m, IS_MAX);
    nan = wave_any(nan);
    if (!nan && m != 0.0f) {
      p = ExtPart{m, e > b ? kNonEmpty : 0u};
    } else if (e > b) {
      p = exact_range<IS_MAX>(A, prod, base, b, e, lane);
    } else {
      p = Comb::empty();
    }
  } else {
    p = Comb::empty();
    Part acc[4] = {Comb::empty(), Comb::empty(), Comb::empty(), Comb::empty()};
    if constexpr (VEC) {
      for (uint64_t i0 = b + uint64_t(lane) * 4; i0 < e; i0 += 256 * kRowUnroll) {
        f4 x[kRowUnroll][NIN];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const uint64_t i = i0 + uint64_t(u) * 256;
          if (i < e)
#pragma unroll
            for (int k = 0; k < NIN; ++k)
              x[u][k] = (A.vec_mask >> k & 1u)
                            ? __builtin_nontemporal_load(
                                  reinterpret_cast<const f4 *>(A.in[k] + base[k] + int64_t(i)))
                            : f4(A.in[k][base[k]]);
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const uint64_t i = i0 + uint64_t(u) * 256;
          if (i >= e) continue;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float v[NIN];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = x[u][k][c];
            Comb::next(acc[c], prod.eval(v), int64_t(i + c));
          }
        }
      }
      p = Comb::merge(Comb::merge(acc[0], acc[1]), Comb::merge(acc[2], acc[3]));
    } else {
      for (uint64_t i = b + lane; i < e; i += 64) {
        Comb::next(p, value_at(A, prod, base, i), int64_t(i));
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) p = Comb::merge(p, Comb::shfl(p, m));
    // every lane holds the row's sum: the check is uniform over the wave
    if constexpr (kSerialSum<Comb>)
      if (A.segs == 1 && !finite_sum(p)) p = serial_sum_wave(A, prod, base, A.len, p, lane);
  }

  if (lane != 0) return;
  if (A.segs == 1) {
    store_final<Comb>(A.out, tbase, p, A.post, A.divisor);
  } else {
    static_cast<Part *>(A.part)[task] = p;
  }
}

// Combine the segments of each row in index order.
// Merge segs partials part[0], part[stride], ... in index order. The loads of a batch are issued
// before its merges: the partials come from L2 or HBM, and a serial load-merge chain would pay
// that latency once per partial (a [16384, 4096] column sum split in 64 chunks spent most of
// its time in that chain).
template <class Comb>
__device__ __forceinline__ typename Comb::Part merge_in_order(const typename Comb::Part *part,
                                                              uint64_t stride, uint32_t segs) {
  using Part = typename Comb::Part;
  constexpr uint32_t kBatch = 16;
  // whole batches of loads, the last one clamped to the final partial (loaded, not merged): a
  // partial batch of one-at-a-time loads would wait out a memory latency per partial
  Part p{};
  for (uint32_t s = 0; s < segs; s += kBatch) {
    Part q[kBatch];
#pragma unroll
    for (uint32_t i = 0; i < kBatch; ++i) {
      const uint32_t k = s + i < segs ? s + i : segs - 1;
      q[i] = part[uint64_t(k) * stride];
    }
#pragma unroll
    for (uint32_t i = 0; i < kBatch; ++i) {
      if (s + i == 0) p = q[0];
      else if (s + i < segs) p = Comb::merge(p, q[i]);
    }
  }
  return p;
}

// Any trivially copyable summary, moved `off` lanes down the wave word by word.
template <class P>
__device__ __forceinline__ P shfl_down_part(const P &p, int off) {
  static_assert(sizeof(P) % 4 == 0, "summaries are whole words");
  P q;
  const int *src = reinterpret_cast<const int *>(&p);
  int *dst = reinterpret_cast<int *>(&q);
#pragma unroll
  for (int w = 0; w < int(sizeof(P) / 4); ++w) dst[w] = __shfl_down(src[w], off);
  return q;
}

// One wave per row: lane l merges the l-th run of consecutive partials in index order, then the
// runs merge pairwise, always earlier run on the left (every combiner's merge is associative over
// ordered ranges; for sums this fixes a different, still deterministic, rounding order than one
// serial pass). A row of 4096 partials took one thread 50 us to merge serially.
template <class Prod, class Comb>
__global__ __launch_bounds__(kBlock) void red_rows_finalize(RedArgs<Prod::NIN> A, Prod prod) {
  using Part = typename Comb::Part;
  constexpr int NIN = Prod::NIN;
  const int lane = threadIdx.x & 63;
  const uint64_t row = uint64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= A.rows) return;  // whole wave
  const Part *part = static_cast<const Part *>(A.part) + row * A.segs;
  const uint32_t run = (A.segs + 63) / 64;
  const uint32_t active = (A.segs + run - 1) / run;  // lanes holding a non-empty run
  const uint32_t s0 = uint32_t(lane) * run;
  Part p = Comb::empty();
  if (uint32_t(lane) < active) {
    const uint32_t n = A.segs - s0 < run ? A.segs - s0 : run;
    p = merge_in_order<Comb>(part + s0, 1, n);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const Part q = shfl_down_part(p, off);
    if ((lane & (2 * off - 1)) == 0 && uint32_t(lane + off) < active) p = Comb::merge(p, q);
  }
  int64_t base[NIN], tbase;
  decode_outer(A, uint32_t(row), base, tbase);
  if constexpr (kSerialSum<Comb>) {
    p = __shfl(p, 0);  // lane 0 holds the row's sum
    if (!finite_sum(p)) p = serial_sum_wave(A, prod, base, A.len, p, lane);
  }
  if (lane != 0) return;
  store_final<Comb>(A.out, tbase, p, A.post, A.divisor);
}

// ------------------------------------------------------------------------- cols kernel

template <class Prod>
constexpr int kColUnroll = Prod::NIN == 1   ? PLAST_COL_UNROLL
                           : Prod::NIN == 2 ? PLAST_COL_UNROLL2
                                            : PLAST_COL_UNROLL3;

template <class Prod>
__device__ __forceinline__ void store_col(f4 *p, f4 v) {
  constexpr bool nt = PLAST_COL_NT_STORE == 1 || (PLAST_COL_NT_STORE == -1 && StoresOther<Prod>::value);
  if constexpr (nt) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <class Prod>
constexpr int kColMinRows = Prod::NIN >= 3 ? PLAST_COL_MIN_ROWS3 : 64;
template <class Prod>
constexpr int kColSmallS4 = Prod::NIN >= 3 ? PLAST_COL_SMALL_S4_3 : PLAST_COL_SMALL_S4;
template <class Prod>
constexpr int kColSmallU = Prod::NIN >= 3 ? PLAST_COL_SMALL_U3 : PLAST_COL_SMALL_U;

// Fast summary of an order-sensitive fold (exact max/min): the plain extreme and a NaN flag.
struct ExtFast {
  float m;
  uint32_t nan;
};

// grid.x: (outer index, slice of 64 lanes x W columns of the kept innermost axis); grid.y: chunk
// of the reduced axis. The workgroup's four waves take interleaved rows of the chunk (wave w reads
// rows k0 + w, k0 + w + 4, ...), so each wave streams its own rows while the workgroup still
// covers one contiguous slice per row; each lane owns W adjacent columns. The four partials of a
// column combine through LDS in wave order (deterministic). Order-free combiners (sum, argmax)
// merge directly. The exact max/min fold keeps a plain extreme and a NaN flag per wave, and a
// column is refolded serially in index order only when its chunk holds a NaN or its extreme is
// zero (the cases where order decides the bits).
// ALLV (with VEC): every operand is streamed with float4 loads, so the loads take no branch on
// the operand mask (a broadcast operand's splat makes the compiler wait for each load in turn).
template <class Prod, class Comb, bool VEC, bool ALLV>
__global__ __launch_bounds__(kBlock) void red_cols_kernel(RedArgs<Prod::NIN> A, Prod prod,
                                                          uint32_t xblocks) {
  constexpr int NIN = Prod::NIN;
  constexpr int W = VEC ? 4 : 1;
  using Part = typename Comb::Part;
  constexpr bool kExt = Comb::kExact;
  constexpr bool IS_MAX = std::is_same<Comb, ExtComb<true>>::value;
  using Fast = typename std::conditional<kExt, ExtFast, Part>::type;
  static_assert(!(kStores<Prod> && kExt), "a storing producer visits each element once");
  __shared__ Fast sh[kBlock / 64][64 * W];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t bx = blockIdx.x, chunk = blockIdx.y;
  const uint32_t o = bx / xblocks;
  const uint64_t j = (uint64_t(bx - o * xblocks) * 64 + lane) * W;
  const bool active = j < A.inner;  // no early return: the workgroup meets at a barrier
  int64_t base[NIN], lbase[NIN], tbase;
  decode_outer(A, o, base, tbase);
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    // an inactive lane loads column 0 (in bounds) and drops it: the loads take no branch
    lbase[k] = base[k];
    base[k] += int64_t(j) * A.kst[k];
    if (active) lbase[k] = base[k];
  }
  const uint64_t k0 = uint64_t(chunk) * A.seglen;
  const uint64_t k1 = k0 + A.seglen < A.len ? k0 + A.seglen : A.len;

  Fast f[W];
#pragma unroll
  for (int c = 0; c < W; ++c) {
    if constexpr (kExt) f[c] = Fast{IS_MAX ? -__builtin_huge_valf() : __builtin_huge_valf(), 0u};
    else f[c] = Comb::empty();
  }
  constexpr int kU = kColUnroll<Prod>;
  for (uint64_t r0 = k0 + wv; r0 < k1; r0 += 4 * kU) {
    float xv[kU][NIN][W];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      // a row past the chunk is clamped to its last row: loaded, not used
      const uint64_t r = r0 + 4 * u < k1 ? r0 + 4 * u : k1 - 1;
#pragma unroll
      for (int k = 0; k < NIN; ++k) {
        const float *src = A.in[k] + lbase[k] + int64_t(r) * A.rst[k];
        if constexpr (VEC) {
          const f4 v = (ALLV || (A.vec_mask >> k & 1u))
                           ? __builtin_nontemporal_load(reinterpret_cast<const f4 *>(src))
                           : f4(src[0]);
#pragma unroll
          for (int c = 0; c < W; ++c) xv[u][k][c] = v[c];
        } else {
          xv[u][k][0] = src[0];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint64_t r = r0 + 4 * u;
      if (!active || r >= k1) continue;
      float yv[W];
#pragma unroll
      for (int c = 0; c < W; ++c) {
        float v[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) v[k] = xv[u][k][c];
        const float y = prod.eval(v);
        yv[c] = stored_value(prod, v, y);
        if constexpr (kExt) {
          f[c].m = IS_MAX ? fmaxf(f[c].m, y) : fminf(f[c].m, y);
          f[c].nan |= y != y ? 1u : 0u;
        } else {
          Comb::next(f[c], y, int64_t(r));
        }
      }
      if constexpr (kStores<Prod>) {
        float *dst = prod.dst + base[0] + int64_t(r) * A.rst[0];
        if constexpr (VEC)
          store_col<Prod>(reinterpret_cast<f4 *>(dst), f4{yv[0], yv[1], yv[2], yv[3]});
        else
          dst[0] = yv[0];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < W; ++c) sh[wv][lane * W + c] = f[c];
  __syncthreads();
  if (wv != 0 || !active) return;

#pragma unroll
  for (int c = 0; c < W; ++c) {
    Part p;
    if constexpr (kExt) {
      float m = sh[0][lane * W + c].m;
      uint32_t nan = sh[0][lane * W + c].nan;
#pragma unroll
      for (int w = 1; w < kBlock / 64; ++w) {
        m = IS_MAX ? fmaxf(m, sh[w][lane * W + c].m) : fminf(m, sh[w][lane * W + c].m);
        nan |= sh[w][lane * W + c].nan;
      }
      if (!nan && m != 0.0f) {
        p = ExtPart{m, kNonEmpty};
      } else {
        // the reference's fold over [k0, k1) in index order
        p = Comb::empty();
        for (uint64_t r = k0; r < k1; ++r) {
          float v[NIN];
#pragma unroll
          for (int k = 0; k < NIN; ++k)
            v[k] = A.in[k][base[k] + int64_t(c) * A.kst[k] + int64_t(r) * A.rst[k]];
          const float y = prod.eval(v);
          if (r == k0) Comb::first(p, y, int64_t(r));
          else Comb::next(p, y, int64_t(r));
        }
      }
    } else {
      p = sh[0][lane * W + c];
#pragma unroll
      for (int w = 1; w < kBlock / 64; ++w) p = Comb::merge(p, sh[w][lane * W + c]);
      if constexpr (kSerialSum<Comb>) {
        if (A.segs == 1 && !finite_sum(p)) {
          int64_t bc[NIN];
#pragma unroll
          for (int k = 0; k < NIN; ++k) bc[k] = base[k] + int64_t(c) * A.kst[k];
          p = serial_sum_lane(A, prod, bc, A.len);
        }
      }
    }
    if (A.segs == 1) {
      store_final<Comb>(A.out, tbase + int64_t(j + c) * A.tkst, p, A.post, A.divisor);
    } else {
      const uint64_t oi = uint64_t(o) * A.inner + j + c;
      static_cast<Part *>(A.part)[uint64_t(chunk) * (A.rows * A.inner) + oi] = p;
    }
  }
}

// Small leading-axis sums in one launch (no partials leave the workgroup, so no finalize), also
// for a storing producer (the one-pass epilogue), which then sums in the same order as the plain
// sum of what it stores. A workgroup owns S4 float4 columns (4 * S4 adjacent outputs) of one outer index and walks every row
// of the reduced axis: lane (g, c) sums the rows g, g + G, g + 2G, ... (G = kBlock / S4 row groups)
// of float4 column c in order. The row groups of a wave then merge with a fixed butterfly, and the
// four waves' partials in wave order: the result is deterministic. A column whose sum is not finite
// is summed again serially in index order (the reference's order decides such sums).
template <class Prod, bool ALLV>
__global__ __launch_bounds__(kBlock) void red_cols_small_kernel(RedArgs<Prod::NIN> A, Prod prod,
                                                                uint32_t xblocks) {
  constexpr int NIN = Prod::NIN;
  constexpr int S4 = kColSmallS4<Prod>, G = kBlock / S4, kU = kColSmallU<Prod>;
  static_assert(64 % S4 == 0, "row groups split evenly over the waves");
  __shared__ f4 sh[kBlock / 64][S4];
  const uint32_t t = threadIdx.x, c4 = t % S4, g = t / S4, lane = t & 63, wv = t >> 6;
  // XCD numbering: the workgroups of one XCD take adjacent column slices, so the slices that share
  // a cache line share that XCD's L2
  const uint32_t b = PLAST_COL_SMALL_XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const uint32_t o = b / xblocks;
  const uint64_t j0 = uint64_t(b - o * xblocks) * (4 * S4);  // the slice's first column
  const uint64_t j = j0 + 4 * c4;
  const bool active = j < A.inner;
  int64_t base0[NIN], base[NIN], lbase[NIN], tbase;
  decode_outer(A, o, base0, tbase);
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    base[k] = base0[k] + int64_t(j) * A.kst[k];
    lbase[k] = active ? base[k] : base0[k];  // an inactive lane loads column 0 and drops it
  }
  f4 f = f4(0.0f);
  for (uint64_t r0 = g; r0 < A.len; r0 += uint64_t(G) * kU) {
    f4 xv[kU][NIN];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      // rows past the end are clamped to the last row: loaded, not used (the loads take no branch)
      const uint64_t r = r0 + uint64_t(u) * G < A.len ? r0 + uint64_t(u) * G : A.len - 1;
#pragma unroll
      for (int k = 0; k < NIN; ++k) {
        const float *src = A.in[k] + lbase[k] + int64_t(r) * A.rst[k];
        xv[u][k] = (ALLV || (A.vec_mask >> k & 1u)) ? *reinterpret_cast<const f4 *>(src)
                                                    : f4(src[0]);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint64_t r = r0 + uint64_t(u) * G;
      if (!active || r >= A.len) continue;
      f4 yv;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float v[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) v[k] = xv[u][k][c];
        const float y = prod.eval(v);
        f[c] = f[c] + y;
        yv[c] = stored_value(prod, v, y);
      }
      if constexpr (kStores<Prod>)  // a storing producer also writes each value it sums
        store_col<Prod>(reinterpret_cast<f4 *>(prod.dst + base[0] + int64_t(r) * A.rst[0]), yv);
    }
  }
  // the wave's row groups (lanes c4, c4 + S4, ...) merge pairwise with a fixed butterfly
#pragma unroll
  for (int m = S4; m < 64; m <<= 1)
#pragma unroll
    for (int c = 0; c < 4; ++c) f[c] = f[c] + __shfl_xor(f[c], m);
  if (lane < uint32_t(S4)) sh[wv][lane] = f;
  __syncthreads();
  if (t >= uint32_t(4 * S4)) return;
  // lane t finishes output column j0 + t: the waves' partials in wave order
  const uint64_t jc = j0 + t;
  if (jc >= A.inner) return;
  float p = sh[0][t / 4][t % 4];
#pragma unroll
  for (int w = 1; w < kBlock / 64; ++w) p = p + sh[w][t / 4][t % 4];
  if (!finite_sum(p)) {
    int64_t bc[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) bc[k] = base0[k] + int64_t(jc) * A.kst[k];
    p = serial_sum_lane(A, prod, bc, A.len);
  }
  store_final<SumComb>(A.out, tbase + int64_t(jc) * A.tkst, p, A.post, A.divisor);
}

template <class Prod, class Comb>
__global__ __launch_bounds__(kBlock) void red_cols_finalize(RedArgs<Prod::NIN> A, Prod prod) {
  using Part = typename Comb::Part;
  constexpr int NIN = Prod::NIN;
  const uint64_t oi = uint64_t(blockIdx.x) * kBlock + threadIdx.x;
  const uint64_t nout = A.rows * A.inner;
  if (oi >= nout) return;
  Part p = merge_in_order<Comb>(static_cast<const Part *>(A.part) + oi, nout, A.segs);
  const uint32_t o = uint32_t(oi / A.inner);
  const uint64_t j = oi - uint64_t(o) * A.inner;
  int64_t base[NIN], tbase;
  decode_outer(A, o, base, tbase);
  if constexpr (kSerialSum<Comb>) {
    if (!finite_sum(p)) {
#pragma unroll
      for (int k = 0; k < NIN; ++k) base[k] += int64_t(j) * A.kst[k];
      p = serial_sum_lane(A, prod, base, A.len);
    }
  }
  store_final<Comb>(A.out, tbase + int64_t(j) * A.tkst, p, A.post, A.divisor);
}

// The same merge with Q lanes per output, for many chunks: lane (q, o) merges the q-th run of
// consecutive chunks of output o in index order (lanes with the same q read consecutive outputs),
// then the runs merge pairwise through shuffles with the earlier run always on the left, as in
// red_rows_finalize. One batch of loads per lane instead of segs / 16 batches in sequence.
template <class Prod, class Comb, int Q>
__global__ __launch_bounds__(kBlock) void red_cols_finalize_q(RedArgs<Prod::NIN> A, Prod prod) {
  using Part = typename Comb::Part;
  constexpr int NIN = Prod::NIN;
  constexpr uint32_t OPW = 64 / Q;  // outputs per wave
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t(blockIdx.x) * kBlock + threadIdx.x) >> 6;
  const uint32_t q = lane / OPW;
  const uint64_t nout = A.rows * A.inner;
  const uint64_t oi = wave * OPW + (lane % OPW);
  const bool valid = oi < nout;
  const uint32_t run = (A.segs + Q - 1) / Q;
  const uint32_t active = (A.segs + run - 1) / run;  // runs holding at least one chunk
  Part p = Comb::empty();
  if (valid && q < active) {
    const uint32_t s0 = q * run;
    const uint32_t n = A.segs - s0 < run ? A.segs - s0 : run;
    p = merge_in_order<Comb>(static_cast<const Part *>(A.part) + uint64_t(s0) * nout + oi, nout,
                             n);
  }
#pragma unroll
  for (uint32_t off = 1; off < uint32_t(Q); off <<= 1) {
    const Part o = shfl_down_part(p, int(off * OPW));
    if ((q & (2 * off - 1)) == 0 && q + off < active) p = Comb::merge(p, o);
  }
  if (q != 0 || !valid) return;
  const uint32_t o = uint32_t(oi / A.inner);
  const uint64_t j = oi - uint64_t(o) * A.inner;
  int64_t base[NIN], tbase;
  decode_outer(A, o, base, tbase);
  if constexpr (kSerialSum<Comb>) {
    if (!finite_sum(p)) {
#pragma unroll
      for (int k = 0; k < NIN; ++k) base[k] += int64_t(j) * A.kst[k];
      p = serial_sum_lane(A, prod, base, A.len);
    }
  }
  store_final<Comb>(A.out, tbase + int64_t(j) * A.tkst, p, A.post, A.divisor);
}

// ------------------------------------------------------------------------- generic kernel

template <int NIN>
struct GenArgs {
  const float *in[NIN];
  void *out;
  int nk, nr;                      // kept / reduced axis counts
  uint64_t kext[kMaxRank], rext[kMaxRank];
  int64_t kst[NIN + 1][kMaxRank];  // strides on kept axes (operand NIN = target)
  int64_t rst[NIN][kMaxRank];      // strides on reduced axes
  uint64_t nout, len;
  int post;
  float divisor;
};

template <class Prod, class Comb>
__global__ __launch_bounds__(kBlock) void red_generic_kernel(GenArgs<Prod::NIN> A, Prod prod) {
  constexpr int NIN = Prod::NIN;
  using Part = typename Comb::Part;
  const uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t o = uint64_t(blockIdx.x) * kBlock + threadIdx.x; o < A.nout; o += stride) {
    int64_t base[NIN] = {};
    int64_t tbase = 0;
    uint64_t rem = o;
    for (int d = A.nk - 1; d >= 0; --d) {
      const int64_t c = int64_t(rem % A.kext[d]);
      rem /= A.kext[d];
#pragma unroll
      for (int k = 0; k < NIN; ++k) base[k] += c * A.kst[k][d];
      tbase += c * A.kst[NIN][d];
    }
    Part p = Comb::empty();
    uint64_t rc[kMaxRank] = {};
    int64_t off[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) off[k] = base[k];
    for (uint64_t r = 0; r < A.len; ++r) {
      float v[NIN];
#pragma unroll
      for (int k = 0; k < NIN; ++k) v[k] = A.in[k][off[k]];
      const float y = prod.eval(v);
      if (r == 0) Comb::first(p, y, int64_t(r));
      else Comb::next(p, y, int64_t(r));
      // odometer step over the reduced axes, innermost fastest
      for (int d = A.nr - 1; d >= 0; --d) {
        if (++rc[d] < A.rext[d]) {
#pragma unroll
          for (int k = 0; k < NIN; ++k) off[k] += A.rst[k][d];
          break;
        }
#pragma unroll
        for (int k = 0; k < NIN; ++k) off[k] -= int64_t(rc[d] - 1) * A.rst[k][d];
        rc[d] = 0;
      }
    }
    store_final<Comb>(A.out, tbase, p, A.post, A.divisor);
  }
}

// ------------------------------------------------------------------------- host dispatch

// Reduce over every axis where operand NIN (the target) has stride 0 and extent > 1.
// `post` and `divisor` describe the epilogue; `out` is float* or int64_t* per Comb::Out.
template <class Prod, class Comb>
bool launch_reduction(const Prod &prod, const void *const *in, void *out, Space s, Post post,
                      float divisor, const char *where) {
  constexpr int NIN = Prod::NIN;
  using Part = typename Comb::Part;
  s.nops = NIN + 1;
  // An empty space: every output holds the fold of nothing (sum 0, mean 0/0, max -FLT_MAX, ...).
  if (s.numel() == 0) {
    if constexpr (kStores<Prod>) return false;
    GenArgs<NIN> G;
    memset(&G, 0, sizeof G);
    G.out = out;
    uint64_t nout = 1;
    for (int d = 0; d < s.rank; ++d) {
      if (s.st[NIN][d] == 0 && s.shape[d] != 1) continue;  // reduced axis
      G.kext[G.nk] = s.shape[d];
      G.kst[NIN][G.nk] = s.st[NIN][d];
      ++G.nk;
      nout *= s.shape[d];
    }
    if (nout == 0) return true;
    G.nout = nout;
    G.len = 0;
    G.post = int(post);
    G.divisor = divisor;
    const uint64_t gb = (nout + kBlock - 1) / kBlock;
    red_generic_kernel<Prod, Comb><<<unsigned(gb < 65536 ? gb : 65536), kBlock, 0, stream()>>>(G, prod);
    return true;
  }
  // collapse() never merges a reduced axis with a kept one: the target's stride is 0 on one and
  // not on the other.
  collapse(s);
  const int r = s.rank;
  int nred = 0, red_ax = -1;
  uint64_t nout = 1;
  for (int d = 0; d < r; ++d) {
    if (s.st[NIN][d] == 0 && s.shape[d] > 1) {
      ++nred;
      red_ax = d;
    } else {
      nout *= s.shape[d];
    }
  }
  const bool empty_space = false;

  const bool small_idx = s.numel() < (uint64_t(1) << 32) && nout < (uint64_t(1) << 32);

  // ---- rows: single reduced axis, innermost, unit stride for streamed operands
  // one wave per row (segment): the grid is rows * segs / 4 workgroups (rows < 2^32 segments
  // are only split when there are fewer than PLAST_ROW_WAVES rows)
  if (!kStores<Prod> && !empty_space && small_idx && nred == 1 && red_ax == r - 1 &&
      nout <= max_blocks(kBlock) * (kBlock / 64)) {
    RedArgs<NIN> A;
    memset(&A, 0, sizeof A);
    for (int k = 0; k < NIN; ++k) A.in[k] = static_cast<const float *>(in[k]);
    A.out = out;
    A.nouter = r - 1;
    bool vec = s.shape[r - 1] % 4 == 0;
    for (int k = 0; k < NIN; ++k) {
      A.rst[k] = s.st[k][r - 1];
      if (A.rst[k] == 1 && aligned16(in[k])) A.vec_mask |= 1u << k;
      else if (A.rst[k] != 0) vec = false;
      if (A.rst[k] == 1 && !aligned16(in[k])) vec = false;
    }
    bool unit = true;
    for (int k = 0; k < NIN; ++k) unit = unit && (A.rst[k] == 0 || A.rst[k] == 1);
    if (unit) {
      for (int d = 0; d < r - 1; ++d) {
        A.dv[d] = MagicDiv::make(uint32_t(s.shape[d]));
        A.tst[d] = s.st[NIN][d];
        for (int k = 0; k < NIN; ++k) {
          A.ost[k][d] = s.st[k][d];
          if ((A.vec_mask >> k & 1u) && s.st[k][d] % 4 != 0) vec = false;
        }
      }
      A.len = s.shape[r - 1];
      A.rows = nout;
      // enough waves to cover the machine: split long rows when there are few of them
      uint32_t segs = 1;
      const uint64_t want_waves = PLAST_ROW_WAVES;
      if (A.rows < want_waves && A.len >= 8192) {
        uint64_t sg = (want_waves + A.rows - 1) / A.rows;
        const uint64_t max_sg = A.len / 4096;
        if (sg > max_sg) sg = max_sg;
        if (sg > 65535) sg = 65535;
        segs = uint32_t(sg < 1 ? 1 : sg);
      }
      uint64_t seglen = (A.len + segs - 1) / segs;
      seglen = (seglen + 255) / 256 * 256;
      segs = uint32_t((A.len + seglen - 1) / seglen);
      A.segs = segs;
      A.seglen = seglen;
      A.post = int(post);
      A.divisor = divisor;
      if (segs > 1) {
        A.part = workspace(sizeof(Part) * A.rows * segs);
        if (!A.part) return false;
      }
      const uint64_t waves = A.rows * segs;
      const unsigned grid = ceil_div(waves, kBlock / 64);
      if (vec) red_rows_kernel<Prod, Comb, true><<<grid, kBlock, 0, stream()>>>(A, prod);
      else red_rows_kernel<Prod, Comb, false><<<grid, kBlock, 0, stream()>>>(A, prod);
      if (segs > 1)  // the finalize reads the partials, and the inputs for a serial refold
        red_rows_finalize<Prod, Comb>
            <<<ceil_div(A.rows, kBlock / 64), kBlock, 0, stream()>>>(A, prod);
      return true;
    }
  }

  // ---- cols: innermost axis kept with unit target stride, exactly one reduced axis
  if (!empty_space && small_idx && nred == 1 && red_ax != r - 1 && s.st[NIN][r - 1] != 0) {
    RedArgs<NIN> A;
    memset(&A, 0, sizeof A);
    for (int k = 0; k < NIN; ++k) A.in[k] = static_cast<const float *>(in[k]);
    A.out = out;
    A.inner = s.shape[r - 1];
    A.tkst = s.st[NIN][r - 1];
    A.len = s.shape[red_ax];
    bool vec = A.inner % 4 == 0 && A.tkst == 1;
    int no = 0;
    for (int d = 0; d < r - 1; ++d) {
      if (d == red_ax) continue;
      A.dv[no] = MagicDiv::make(uint32_t(s.shape[d]));
      A.tst[no] = s.st[NIN][d];
      for (int k = 0; k < NIN; ++k) A.ost[k][no] = s.st[k][d];
      ++no;
    }
    A.nouter = no;
    for (int k = 0; k < NIN; ++k) {
      A.rst[k] = s.st[k][red_ax];
      A.kst[k] = s.st[k][r - 1];
      if (A.kst[k] == 1 && aligned16(in[k])) A.vec_mask |= 1u << k;
      else if (A.kst[k] != 0) vec = false;
      if (A.kst[k] == 1 && !aligned16(in[k])) vec = false;
      if (A.kst[k] == 1) {
        if (A.rst[k] % 4 != 0) vec = false;
        for (int d = 0; d < no; ++d)
          if (A.ost[k][d] % 4 != 0) vec = false;
      }
    }
    A.rows = nout / A.inner;  // outer count
    const bool allv = A.vec_mask == (1u << NIN) - 1;
    const uint32_t W = vec ? 4 : 1;
    const uint32_t xblocks = ceil_div(A.inner, uint64_t(64) * W);
    const uint64_t base_blocks = uint64_t(xblocks) * A.rows;
    // chunk the reduced axis until the grid has ~PLAST_COL_BLOCKS workgroups, keeping at least
    // kColMinRows rows per chunk
    uint64_t chunks = 1;
    constexpr uint64_t min_rows = kColMinRows<Prod>;
    if (base_blocks < PLAST_COL_BLOCKS && A.len >= 2 * min_rows) {
      chunks = (PLAST_COL_BLOCKS + base_blocks - 1) / base_blocks;
      const uint64_t max_c = A.len / min_rows;
      if (chunks > max_c) chunks = max_c;
      if (chunks > 65535) chunks = 65535;
      if (chunks < 1) chunks = 1;
    }
    uint64_t seglen = (A.len + chunks - 1) / chunks;
    chunks = (A.len + seglen - 1) / seglen;
    A.segs = uint32_t(chunks);
    A.seglen = seglen;
    A.post = int(post);
    A.divisor = divisor;
    if constexpr (std::is_same<Comb, SumComb>::value) {
      // small: one launch over narrow column slices instead of chunks plus a finalize
      if (chunks > 1 && vec && A.len * nout <= PLAST_COL_SMALL_MAX &&
          (NIN < 3 || PLAST_COL_SMALL3 != 0)) {
        const uint32_t sblocks = ceil_div(A.inner, uint64_t(4) * kColSmallS4<Prod>);
        const unsigned grid = unsigned(uint64_t(sblocks) * A.rows);
        if (allv) red_cols_small_kernel<Prod, true><<<grid, kBlock, 0, stream()>>>(A, prod, sblocks);
        else red_cols_small_kernel<Prod, false><<<grid, kBlock, 0, stream()>>>(A, prod, sblocks);
        return true;
      }
    }
    if (base_blocks <= max_blocks(kBlock)) {
      if (chunks > 1) {
        A.part = workspace(sizeof(Part) * nout * chunks);
        if (!A.part) return false;
      }
      const dim3 grid{unsigned(base_blocks), unsigned(chunks), 1u};
      if (vec && allv)
        red_cols_kernel<Prod, Comb, true, true><<<grid, kBlock, 0, stream()>>>(A, prod, xblocks);
      else if (vec)
        red_cols_kernel<Prod, Comb, true, false><<<grid, kBlock, 0, stream()>>>(A, prod, xblocks);
      else
        red_cols_kernel<Prod, Comb, false, false><<<grid, kBlock, 0, stream()>>>(A, prod, xblocks);
      if (chunks > 1) {  // the finalize reads the partials, and the inputs for a serial refold
        // chunks > 1 only when base_blocks < PLAST_COL_BLOCKS, so nout * Q lanes (at most
        // PLAST_COL_BLOCKS * 256 * Q) stay far inside one launch
        if (PLAST_COL_FIN_Q > 1 && chunks >= 2 * PLAST_COL_FIN_Q)
          red_cols_finalize_q<Prod, Comb, PLAST_COL_FIN_Q>
              <<<ceil_div(nout * PLAST_COL_FIN_Q, kBlock), kBlock, 0, stream()>>>(A, prod);
        else
          red_cols_finalize<Prod, Comb><<<ceil_div(nout, kBlock), kBlock, 0, stream()>>>(A, prod);
      }
      return true;
    }
  }

  // ---- generic
  if constexpr (kStores<Prod>) return false;
  GenArgs<NIN> G;
  memset(&G, 0, sizeof G);
  for (int k = 0; k < NIN; ++k) G.in[k] = static_cast<const float *>(in[k]);
  G.out = out;
  G.len = 1;
  for (int d = 0; d < r; ++d) {
    const bool red = s.st[NIN][d] == 0 && s.shape[d] > 1;
    if (red) {
      G.rext[G.nr] = s.shape[d];
      for (int k = 0; k < NIN; ++k) G.rst[k][G.nr] = s.st[k][d];
      G.len *= s.shape[d];
      ++G.nr;
    } else {
      G.kext[G.nk] = s.shape[d];
      for (int k = 0; k <= NIN; ++k) G.kst[k][G.nk] = s.st[k][d];
      ++G.nk;
    }
  }
  G.nout = nout;
  G.post = int(post);
  G.divisor = divisor;
  uint64_t blocks = (nout + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) blocks = 1;
  red_generic_kernel<Prod, Comb><<<unsigned(blocks), kBlock, 0, stream()>>>(G, prod);
  (void)where;
  return true;
}

// Accumulating sum into a broadcast target: target[t] += sum over its broadcast axes of prod.
template <class Prod>
bool reduce_accumulate(const Prod &prod, const void *const *in, float *target, Space s,
                       const char *where) {
  return launch_reduction<Prod, SumComb>(prod, in, target, s, Post::Accum, 1.0f, where);
}

}  // namespace plast
