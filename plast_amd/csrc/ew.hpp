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
  static constexpr bool kTape = false;             // selects the vectorised launch shape
  static constexpr bool kTileFixed3 = false;       // fixed-role tile kernels for 3 operands
  static constexpr int kTileRows = 1;              // tile rows per evaluation
  template <int U, int N>
  __device__ __forceinline__ void eval_units(const f4 (&x)[U][N], const uint64_t (&idx)[U],
                                             const bool (&valid)[U], f4 (&acc)[U]) const {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (valid[u]) acc[u] = eval4(x[u], idx[u]);
  }
  // the kernels' common interface with the tape body, which reads per-wave state first
  __device__ __forceinline__ uint32_t load_words() const { return 0; }
  template <int U, int N>
  __device__ __forceinline__ void eval_units_with(uint32_t, const f4 (&x)[U][N],
                                                  const uint64_t (&idx)[U], const bool (&valid)[U],
                                                  f4 (&acc)[U]) const {
    eval_units<U, N>(x, idx, valid, acc);
  }
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

// operands: dout, out  ->  dout * (out > 0 ? 1 : alpha): the leaky-relu gradient modulation of the
// fused matmul epilogues (src/kernels/cpu/fused_ops.c:19-21, 105-111)
struct ReluGradBody : ScalarBody<ReluGradBody> {
  static constexpr int NIN = 2;
  float alpha;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return v[0] * (v[1] > 0.0f ? 1.0f : alpha);
  }
};

// operands: dout, y, dx  ->  dx + (0 + dout * (y > 0 ? 1 : alpha)): x's gradient through a fused
// leaky_relu(x + bias) node, the leaky backward into the intermediate's zeroed gradient
// (unary_ops.c:236-258) then the ADD backward's accumulation (kernel_macros.h:283-299), with the
// mask read from the node's output (the same for alpha >= 0)
struct LeakyAddGradAccumBody : ScalarBody<LeakyAddGradAccumBody> {
  static constexpr int NIN = 3;
  float alpha;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const {
    return v[2] + (0.0f + v[0] * (v[1] > 0.0f ? 1.0f : alpha));
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

// Op classes a fused chain's kernel is compiled for (a bit set: the OPS parameter of TapeBody).
// The arithmetic ops (add, sub, mul, div, leaky relu, neg, abs) are always in; each class below
// adds the ocml routine it needs. A tape runs on the smallest instantiated set that holds its ops
// (tape_ops_class), so a chain without exp or log carries none of their code or registers.
enum TapeOps : uint32_t { kTapeArith = 0, kTapeExp = 1, kTapeLog = 2, kTapeTrig = 4 };

// The instantiated sets: arithmetic only, + exp, + exp and log, everything.
inline uint32_t tape_ops_class(const PlastFusedTape &t) {
  uint32_t m = 0;
  for (uint32_t i = 0; i < t.num_ins; ++i) {
    const uint8_t op = t.ins[i].op;
    if (op == TAPE_EXP) m |= kTapeExp;
    else if (op == TAPE_LOG) m |= kTapeLog;
    else if (op == TAPE_SIN || op == TAPE_COS || op == TAPE_TAN) m |= kTapeTrig;
  }
  if (m & kTapeTrig) return kTapeExp | kTapeLog | kTapeTrig;
  if (m & kTapeLog) return kTapeExp | kTapeLog;
  return m;
}

// Tape interpreter for fused chains. Every field read is a scalar load of the kernel argument and
// every branch is on an SGPR value, so the interpretation costs scalar instructions only. The tape
// loop is the outer loop, so each dispatch is paid once per U float4 units. OPS (TapeOps bits):
// the op classes compiled in; a tape must hold no op outside them (the host picks OPS with
// tape_ops_class).
template <int N, uint32_t OPS>
struct TapeBody {
  static constexpr int NIN = N;
  static constexpr bool kTape = true;
  static constexpr bool kTileFixed3 = true;
  static constexpr int kTileRows = PLAST_TAPE_TILE_ROWS;
  static constexpr bool kExp = (OPS & kTapeExp) != 0;
  static constexpr bool kLog = (OPS & kTapeLog) != 0;
  static constexpr bool kTrig = (OPS & kTapeTrig) != 0;
  PlastFusedTape t;
  uint64_t simd_end;
  // bit i: the NEG at instruction i follows the reference's contiguous path (0 - x below simd_end,
  // -x in the tail); a NEG whose bit is clear takes its strided path (-x everywhere)
  uint32_t neg_simd;

  template <class F>
  __device__ __forceinline__ static f4 map(f4 a, F f) {
    return f4{f(a[0]), f(a[1]), f(a[2]), f(a[3])};
  }

  // acc[u] = tape(x[u]); idx[u] is the linear index of unit u's first element (a multiple of 4,
  // while simd_end is a multiple of 8, so a unit never straddles the NEG rule's boundary).
  // Invalid units compute on whatever their registers hold; only their stores are skipped.
  template <int U>
  __device__ __forceinline__ void eval_units(const f4 (&x)[U][N], const uint64_t (&idx)[U],
                                             const bool (&valid)[U], f4 (&acc)[U]) const {
    eval_units_with<U>(load_words(), x, idx, valid, acc);
  }

  // The tape's 2 * PLAST_TAPE_MAX_INS dwords, one per lane (lane 2i: op/src/idx/acc_rhs bytes of
  // instruction i; lane 2i+1: its immediate), read back with v_readlane. A scalar load per
  // instruction would need a wait on the shared scalar/LDS counter, which also drains a tile
  // kernel's outstanding LDS reads. Every lane of the wave must execute this load (v_readlane
  // reads lanes the caller's branch may have switched off), and a kernel that prefetches operands
  // loads the words once up front: waiting for a load issued after a prefetch waits for the
  // prefetch too.
  __device__ __forceinline__ uint32_t load_words() const {
    static_assert(sizeof(PlastTapeIns) == 8, "tape instruction is two dwords");
    return reinterpret_cast<const uint32_t *>(t.ins)[__lane_id() & (2 * PLAST_TAPE_MAX_INS - 1)];
  }

  template <int U>
  __device__ __forceinline__ void eval_units_with(uint32_t words, const f4 (&x)[U][N],
                                                  const uint64_t (&idx)[U], const bool (&valid)[U],
                                                  f4 (&acc)[U]) const {
    (void)valid;
    const uint32_t w0x = uint32_t(__builtin_amdgcn_readlane(int(words), 0));
    select_input(x, int((w0x >> 16) & 0xffu), acc);
    // not unrolled: the loop sits outside any lane-divergent branch, so i stays uniform
    for (uint32_t i = 1; i < t.num_ins; ++i) {
      const uint32_t wx = uint32_t(__builtin_amdgcn_readlane(int(words), int(2 * i)));
      const uint32_t wy = uint32_t(__builtin_amdgcn_readlane(int(words), int(2 * i + 1)));
      const int op = int(wx & 0xffu), src = int((wx >> 8) & 0xffu), k = int((wx >> 16) & 0xffu);
      const bool rhs = (wx >> 24) != 0u;
      const float imm = __uint_as_float(wy);
      f4 o[U];
      if (src == TAPE_SRC_INPUT) {
        select_input(x, k, o);
      } else if (src == TAPE_SRC_IMM) {
#pragma unroll
        for (int u = 0; u < U; ++u) o[u] = f4(imm);
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) o[u] = acc[u];
      }
      switch (op) {
      case TAPE_ADD:
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = acc[u] + o[u];  // commutative
        break;
      case TAPE_MUL:
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = acc[u] * o[u];  // commutative
        break;
      case TAPE_SUB:
        if (rhs) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = o[u] - acc[u];
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = acc[u] - o[u];
        }
        break;
      case TAPE_DIV:
        if (rhs) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = o[u] / acc[u];
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = acc[u] / o[u];
        }
        break;
      case TAPE_LEAKY_RELU:
#pragma unroll
        for (int u = 0; u < U; ++u)
          acc[u] = map(acc[u], [imm](float v) { return v > 0.0f ? v : v * imm; });
        break;
      case TAPE_EXP:
        if constexpr (kExp) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return expf(v); });
        }
        break;
      case TAPE_LOG:
        if constexpr (kLog) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return logf(v); });
        }
        break;
      case TAPE_NEG: {
        const bool contig = (neg_simd >> i & 1u) != 0u;
#pragma unroll
        for (int u = 0; u < U; ++u)
          acc[u] = contig && idx[u] < simd_end ? f4(0.0f) - acc[u]
                                               : map(acc[u], [](float v) { return -v; });
        break;
      }
      case TAPE_ABS:
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return fabsf(v); });
        break;
      case TAPE_SIN:
        if constexpr (kTrig) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return sinf(v); });
        }
        break;
      case TAPE_COS:
        if constexpr (kTrig) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return cosf(v); });
        }
        break;
      case TAPE_TAN:
        if constexpr (kTrig) {
#pragma unroll
          for (int u = 0; u < U; ++u) acc[u] = map(acc[u], [](float v) { return tanf(v); });
        }
        break;
      default:
        break;
      }
    }
  }

  // dst[u] = x[u][k] for a uniform k, one branch for all units
  template <int U>
  __device__ __forceinline__ static void select_input(const f4 (&x)[U][N], int k, f4 (&dst)[U]) {
    switch (k) {
    case 0:
#pragma unroll
      for (int u = 0; u < U; ++u) dst[u] = x[u][0];
      break;
    case 1:
#pragma unroll
      for (int u = 0; u < U; ++u) dst[u] = x[u][N > 1 ? 1 : 0];
      break;
    case 2:
#pragma unroll
      for (int u = 0; u < U; ++u) dst[u] = x[u][N > 2 ? 2 : 0];
      break;
    default:
#pragma unroll
      for (int u = 0; u < U; ++u) dst[u] = x[u][N > 3 ? 3 : 0];
      break;
    }
  }

  __device__ __forceinline__ float eval(const float *v, uint64_t idx) const {
    f4 x[1][N];
#pragma unroll
    for (int k = 0; k < N; ++k) x[0][k] = f4(v[k]);
    // a lone element decides the NEG rule for itself
    TapeBody<N, OPS> me = *this;
    me.simd_end = idx < simd_end ? ~uint64_t(0) : 0;
    const uint64_t i0[1] = {0};
    const bool ok[1] = {true};
    f4 r[1];
    me.template eval_units<1>(x, i0, ok, r);
    return r[0][0];
  }
};

// ------------------------------------------------------------------------- launch

// Launch `body` over iteration space `s`: operands 0..NIN-1 are inputs, operand NIN is the output.
// `s` need not be collapsed. Returns false (after reporting) when the launch was impossible.
template <class Body>
bool launch_elementwise(const Body &body, const void *const *in, void *out, Space s,
                        const char *where);

}  // namespace plast
