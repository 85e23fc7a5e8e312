// ew.hpp — the elementwise engine: op bodies (fixed ops, gradients, the fused-chain tape) and the
// layout-specialised kernels that stream them over an iteration space.
#pragma once

#include "common.hpp"

namespace plast {

enum class Bin { Add, Sub, Mul, Div };
enum class Un { Exp, Log, Neg, Abs, Sin, Cos, Tan, Leaky };

// ------------------------------------------------------------------------- scalar semantics
// One IEEE fp32 operation per reference operation (the library is compiled with
// -ffp-contract=off, so a*b+c is two roundings, as in the reference's separate kernels).

template <Bin OP>
__device__ __forceinline__ float bin_op(float x, float y) {
  if constexpr (OP == Bin::Add) return x + y;
  else if constexpr (OP == Bin::Sub) return x - y;
  else if constexpr (OP == Bin::Mul) return x * y;
  else return x / y;
}

// `simd` is true for elements the reference computes inside its 8-wide AVX2 blocks; only neg
// differs there (0 - x instead of -x: unary_ops.c:200 versus 204).
template <Un OP>
__device__ __forceinline__ float un_op(float x, float alpha, bool simd) {
  if constexpr (OP == Un::Exp) return expf(x);
  else if constexpr (OP == Un::Log) return logf(x);
  else if constexpr (OP == Un::Neg) return simd ? 0.0f - x : -x;
  else if constexpr (OP == Un::Abs) return fabsf(x);
  else if constexpr (OP == Un::Sin) return sinf(x);
  else if constexpr (OP == Un::Cos) return cosf(x);
  else if constexpr (OP == Un::Tan) return tanf(x);
  else return x > 0.0f ? x : x * alpha;
}

// Gradient term added into da (unary_ops.c:68-91, contiguous loops 101-319). `contig` selects
// the reference's contiguous form where it rounds differently (abs, leaky: g * multiplier).
template <Un OP>
__device__ __forceinline__ float un_grad(float g, float x, float alpha, bool contig) {
  if constexpr (OP == Un::Exp) return g * expf(x);
  else if constexpr (OP == Un::Log) return g * (1.0f / x);
  else if constexpr (OP == Un::Neg) return -g;
  else if constexpr (OP == Un::Abs) {
    if (contig) return g * (x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f));
    return x > 0.0f ? g : (x < 0.0f ? -g : 0.0f);
  } else if constexpr (OP == Un::Sin) return g * cosf(x);
  else if constexpr (OP == Un::Cos) return g * (-sinf(x));
  else if constexpr (OP == Un::Tan) {
    float t = tanf(x);
    return g * (1.0f + t * t);
  } else {
    if (contig) return g * (x > 0.0f ? 1.0f : alpha);
    return x > 0.0f ? g : g * alpha;
  }
}

// Binary gradients (binary_ops.c:18-57). The B-gradient of sub/div starts from 0 - g inside the
// reference's SIMD blocks and from -g elsewhere.
template <Bin OP>
__device__ __forceinline__ float grad_a(float g, float x, float y) {
  if constexpr (OP == Bin::Add || OP == Bin::Sub) return g;
  else if constexpr (OP == Bin::Mul) return g * y;
  else return g / y;
}
template <Bin OP>
__device__ __forceinline__ float grad_b(float g, float x, float y, bool simd) {
  if constexpr (OP == Bin::Add) return g;
  else if constexpr (OP == Bin::Sub) return simd ? 0.0f - g : -g;
  else if constexpr (OP == Bin::Mul) return g * x;
  else return (simd ? 0.0f - g : -g) * x / (y * y);
}

// ------------------------------------------------------------------------- bodies
// A body maps NIN loaded operands to one output value. `eval4` handles four consecutive elements
// of the iteration (one float4); `idx` is the linear index of the first of them.

template <class Derived>
struct ScalarBody {
  __device__ __forceinline__ f4 eval4(const f4 *x, uint64_t idx) const {
    const Derived &d = static_cast<const Derived &>(*this);
    constexpr int N = Derived::NIN;
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v[N];
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = x[k][c];
      r[c] = d.eval(v, idx + c);
    }
    return r;
  }
};

template <Bin OP>
struct BinBody : ScalarBody<BinBody<OP>> {
  static constexpr int NIN = 2;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return bin_op<OP>(v[0], v[1]);
  }
};

template <Un OP>
struct UnBody : ScalarBody<UnBody<OP>> {
  static constexpr int NIN = 1;
  float alpha;
  uint64_t simd_end;  // 0 when the reference would take its non-contiguous path
  __device__ __forceinline__ float eval(const float *v, uint64_t i) const {
    return un_op<OP>(v[0], alpha, i < simd_end);
  }
};

// operands: da, g, a  ->  da + grad
template <Un OP>
struct UnGradBody : ScalarBody<UnGradBody<OP>> {
  static constexpr int NIN = 3;
  float alpha;
  int contig;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return v[0] + un_grad<OP>(v[1], v[2], alpha, contig != 0);
  }
};

// operands: da, g, a, b  ->  da + grad_a
template <Bin OP>
struct BinGradABody : ScalarBody<BinGradABody<OP>> {
  static constexpr int NIN = 4;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return v[0] + grad_a<OP>(v[1], v[2], v[3]);
  }
};

// operands: db, g, a, b  ->  db + grad_b
template <Bin OP>
struct BinGradBBody : ScalarBody<BinGradBBody<OP>> {
  static constexpr int NIN = 4;
  uint64_t simd_end;
  __device__ __forceinline__ float eval(const float *v, uint64_t i) const {
    return v[0] + grad_b<OP>(v[1], v[2], v[3], i < simd_end);
  }
};

// operands: da, g  ->  da + g  (reshape backward, sum backward broadcast, transpose backward)
struct AccumBody : ScalarBody<AccumBody> {
  static constexpr int NIN = 2;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const { return v[0] + v[1]; }
};

// operands: da, g, scale  ->  da + g / scale  (mean backward: SCALE_MEAN, reduce_ops.c:18)
struct AccumDivBody : ScalarBody<AccumDivBody> {
  static constexpr int NIN = 2;
  float divisor;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return v[0] + v[1] / divisor;
  }
};

// Runtime tape interpreter for fused chains. Every branch is on a wave-uniform kernel argument,
// so the interpretation costs scalar instructions only; the vector work is the chain's own math.
template <int N>
struct TapeBody {
  static constexpr int NIN = N;
  PlastFusedTape t;
  uint64_t simd_end;

  __device__ __forceinline__ static f4 pick(const f4 *x, int k) {
    switch (k) {
    case 0: return x[0];
    case 1: return x[N > 1 ? 1 : 0];
    case 2: return x[N > 2 ? 2 : 0];
    default: return x[N > 3 ? 3 : 0];
    }
  }
  template <class F>
  __device__ __forceinline__ static f4 map(f4 a, F f) {
    return f4{f(a[0]), f(a[1]), f(a[2]), f(a[3])};
  }

  __device__ __forceinline__ f4 eval4(const f4 *x, uint64_t idx) const {
    f4 acc = pick(x, t.ins[0].idx);
    const bool simd = idx < simd_end;  // idx is a multiple of 4 and simd_end of 8
    for (uint32_t i = 1; i < t.num_ins; ++i) {
      const PlastTapeIns in = t.ins[i];
      f4 o = acc;
      if (in.src == TAPE_SRC_INPUT) o = pick(x, in.idx);
      else if (in.src == TAPE_SRC_IMM) o = f4(in.imm);
      const f4 l = in.acc_rhs ? o : acc;
      const f4 r = in.acc_rhs ? acc : o;
      switch (in.op) {
      case TAPE_ADD: acc = l + r; break;
      case TAPE_SUB: acc = l - r; break;
      case TAPE_MUL: acc = l * r; break;
      case TAPE_DIV: acc = l / r; break;
      case TAPE_LEAKY_RELU: {
        const float al = in.imm;
        acc = map(acc, [al](float v) { return v > 0.0f ? v : v * al; });
        break;
      }
      case TAPE_EXP: acc = map(acc, [](float v) { return expf(v); }); break;
      case TAPE_LOG: acc = map(acc, [](float v) { return logf(v); }); break;
      case TAPE_NEG:
        acc = simd ? f4(0.0f) - acc : map(acc, [](float v) { return -v; });
        break;
      case TAPE_ABS: acc = map(acc, [](float v) { return fabsf(v); }); break;
      case TAPE_SIN: acc = map(acc, [](float v) { return sinf(v); }); break;
      case TAPE_COS: acc = map(acc, [](float v) { return cosf(v); }); break;
      case TAPE_TAN: acc = map(acc, [](float v) { return tanf(v); }); break;
      default: break;
      }
    }
    return acc;
  }
  __device__ __forceinline__ float eval(const float *v, uint64_t idx) const {
    f4 x[N];
#pragma unroll
    for (int k = 0; k < N; ++k) x[k] = f4(v[k]);
    // The NEG rule is decided per group of four; a scalar element may sit alone in its group.
    TapeBody<N> me = *this;
    me.simd_end = idx < simd_end ? ~uint64_t(0) : 0;
    return me.eval4(x, 0)[0];
  }
};

// ------------------------------------------------------------------------- launch

// Launch `body` over iteration space `s`: operands 0..NIN-1 are inputs, operand NIN is the output.
// `s` need not be collapsed. Returns false (after reporting) when the launch was impossible.
template <class Body>
bool launch_elementwise(const Body &body, const void *const *in, void *out, Space s,
                        const char *where);

}  // namespace plast
