// ew_impl.hpp — kernels and host dispatch of the elementwise engine (included by the translation
// units that instantiate it).
#pragma once

#include "ew.hpp"

namespace plast {

// Kernel arguments: operand base pointers and per-axis element strides of a collapsed space.
// Passed by value, so shapes, strides and magic divisors live in SGPRs.
template <int NIN>
struct EwArgs {
  const float *in[NIN];
  float *out;
  int64_t ist[NIN][kMaxRank];
  int64_t ost[kMaxRank];
  MagicDiv dv[kMaxRank];  // divisors for the outer axes (vec kernel) or every axis (generic)
  int rank;
  uint32_t bcast_inner;   // bit k: input k has stride 0 on the innermost axis
  uint64_t n;             // elements in the space
  uint64_t units;         // float4 units (vec kernel)
  MagicDiv dinner4;       // innermost extent / 4 (vec kernel)
  uint64_t shape64[kMaxRank];  // extents, for the 64-bit generic kernel
};

constexpr int kEwUnroll = 4;  // float4 units per lane per launch tile

template <int NIN>
__device__ __forceinline__ f4 load4(const EwArgs<NIN> &A, int k, int64_t off) {
  if (A.bcast_inner & (1u << k)) return f4(A.in[k][off]);
  return __builtin_nontemporal_load(reinterpret_cast<const f4 *>(A.in[k] + off));
}

// Vectorised kernel: innermost axis has stride 1 (output, streamed inputs) or 0 (broadcast
// inputs) and a multiple-of-4 extent; the other ORANK axes (ORANK < 0: runtime count) are decoded
// from the unit index with magic division. A workgroup owns kBlock * kEwUnroll consecutive units,
// so each wave reads and writes whole contiguous 1 KiB runs per operand.
template <class Body, int ORANK>
__global__ __launch_bounds__(kBlock) void ew_vec_kernel(EwArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  const uint64_t base = uint64_t(blockIdx.x) * (kBlock * kEwUnroll) + threadIdx.x;
  f4 x[kEwUnroll][NIN];
  int64_t oo[kEwUnroll];
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    const uint64_t q = base + uint64_t(u) * kBlock;
    if (q >= A.units) continue;
    int64_t off[NIN];
    int64_t ooff;
    if constexpr (ORANK == 0) {
      const int64_t e = int64_t(q) * 4;
#pragma unroll
      for (int k = 0; k < NIN; ++k) off[k] = (A.bcast_inner & (1u << k)) ? 0 : e;
      ooff = e;
    } else {
      const uint32_t q32 = uint32_t(q);
      uint32_t row = A.dinner4.div(q32);
      const int64_t c = int64_t(q32 - row * A.dinner4.d) * 4;
#pragma unroll
      for (int k = 0; k < NIN; ++k) off[k] = (A.bcast_inner & (1u << k)) ? 0 : c;
      ooff = c;
      const int nouter = ORANK > 0 ? ORANK : A.rank - 1;
#pragma unroll
      for (int j = 0; j < (ORANK > 0 ? ORANK : kMaxRank - 1); ++j) {
        if (ORANK < 0 && j >= nouter) break;
        const int d = nouter - 1 - j;
        uint32_t nxt = A.dv[d].div(row);
        const int64_t cd = int64_t(row - nxt * A.dv[d].d);
        row = nxt;
#pragma unroll
        for (int k = 0; k < NIN; ++k) off[k] += cd * A.ist[k][d];
        ooff += cd * A.ost[d];
      }
    }
#pragma unroll
    for (int k = 0; k < NIN; ++k) x[u][k] = load4(A, k, off[k]);
    oo[u] = ooff;
  }
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    const uint64_t q = base + uint64_t(u) * kBlock;
    if (q >= A.units) continue;
    const f4 r = body.eval4(x[u], q * 4);
    __builtin_nontemporal_store(r, reinterpret_cast<f4 *>(A.out + oo[u]));
  }
}

// Generic kernel: any strides, one element per lane per step. IDX64 selects 64-bit division for
// spaces of 2^32 elements or more.
template <class Body, bool IDX64>
__global__ __launch_bounds__(kBlock) void ew_generic_kernel(EwArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  const uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t e = uint64_t(blockIdx.x) * kBlock + threadIdx.x; e < A.n; e += stride) {
    int64_t off[NIN] = {};
    int64_t ooff = 0;
    if constexpr (IDX64) {
      uint64_t rem = e;
      for (int d = A.rank - 1; d >= 0; --d) {
        const uint64_t ext = A.shape64[d];
        const int64_t cd = int64_t(rem % ext);
        rem /= ext;
#pragma unroll
        for (int k = 0; k < NIN; ++k) off[k] += cd * A.ist[k][d];
        ooff += cd * A.ost[d];
      }
    } else {
      uint32_t rem = uint32_t(e);
      for (int d = A.rank - 1; d >= 0; --d) {
        const uint32_t nxt = A.dv[d].div(rem);
        const int64_t cd = int64_t(rem - nxt * A.dv[d].d);
        rem = nxt;
#pragma unroll
        for (int k = 0; k < NIN; ++k) off[k] += cd * A.ist[k][d];
        ooff += cd * A.ost[d];
      }
    }
    float v[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) v[k] = A.in[k][off[k]];
    A.out[ooff] = body.eval(v, e);
  }
}

// ------------------------------------------------------------------------- host dispatch

template <class Body>
bool launch_elementwise(const Body &body, const void *const *in, void *out, Space s,
                        const char *where) {
  constexpr int NIN = Body::NIN;
  s.nops = NIN + 1;
  collapse(s);
  const uint64_t n = s.numel();
  if (n == 0) return true;

  EwArgs<NIN> A;
  memset(&A, 0, sizeof A);
  for (int k = 0; k < NIN; ++k) A.in[k] = static_cast<const float *>(in[k]);
  A.out = static_cast<float *>(out);
  A.rank = s.rank;
  A.n = n;
  for (int d = 0; d < s.rank; ++d) {
    for (int k = 0; k < NIN; ++k) A.ist[k][d] = s.st[k][d];
    A.ost[d] = s.st[NIN][d];
  }
  const int in_ax = s.rank - 1;
  const uint64_t inner = s.shape[in_ax];

  // --- vectorised path
  bool vec = (n < (uint64_t(1) << 32) || in_ax == 0) && inner % 4 == 0 && s.st[NIN][in_ax] == 1 && aligned16(out);
  for (int k = 0; k < NIN && vec; ++k) {
    const int64_t si = s.st[k][in_ax];
    if (si == 0) {
      A.bcast_inner |= 1u << k;
    } else {
      vec = si == 1 && aligned16(in[k]);
    }
  }
  for (int d = 0; d < in_ax && vec; ++d)
    for (int k = 0; k <= NIN && vec; ++k)
      if ((k == NIN || !(A.bcast_inner & (1u << k))) && s.st[k][d] % 4 != 0) vec = false;
  if (vec) {
    A.units = n / 4;
    A.dinner4 = MagicDiv::make(uint32_t(inner / 4));
    for (int d = 0; d < in_ax; ++d) A.dv[d] = MagicDiv::make(uint32_t(s.shape[d]));
    const unsigned grid = ceil_div(A.units, uint64_t(kBlock) * kEwUnroll);
    switch (in_ax) {
    case 0: ew_vec_kernel<Body, 0><<<grid, kBlock, 0, stream()>>>(A, body); break;
    case 1: ew_vec_kernel<Body, 1><<<grid, kBlock, 0, stream()>>>(A, body); break;
    case 2: ew_vec_kernel<Body, 2><<<grid, kBlock, 0, stream()>>>(A, body); break;
    default: ew_vec_kernel<Body, -1><<<grid, kBlock, 0, stream()>>>(A, body); break;
    }
    return true;
  }

  // --- generic path
  uint64_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > 262144) blocks = 262144;
  if (n < (uint64_t(1) << 32)) {
    for (int d = 0; d < s.rank; ++d) A.dv[d] = MagicDiv::make(uint32_t(s.shape[d]));
    ew_generic_kernel<Body, false><<<unsigned(blocks), kBlock, 0, stream()>>>(A, body);
    return true;
  }
  for (int d = 0; d < s.rank; ++d) A.shape64[d] = s.shape[d];
  ew_generic_kernel<Body, true><<<unsigned(blocks), kBlock, 0, stream()>>>(A, body);
  (void)where;
  return true;
}

}  // namespace plast
