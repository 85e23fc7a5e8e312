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
  uint32_t reused;        // bit k: input k has stride 0 on some axis (re-read: cached loads)
  uint64_t n;             // elements in the space
  uint64_t units;         // float4 units (vec kernel)
  MagicDiv dinner4;       // innermost extent / 4 (vec kernel)
  uint64_t shape64[kMaxRank];  // extents, for the 64-bit generic kernel
};


// Load policy is a compile-time choice per launch (a run-time select between a nontemporal and an
// ordinary load of the same address is folded into one ordinary load by the compiler). Launches
// whose operands are all read once stream them with nontemporal loads; launches with an operand
// re-read along a broadcast axis use ordinary loads, so the reuse hits in the caches.
template <bool REUSE>
__device__ __forceinline__ f4 load_operand(const float *p) {
  if constexpr (REUSE) return *reinterpret_cast<const f4 *>(p);
  else return __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
}

template <bool REUSE, int NIN>
__device__ __forceinline__ f4 load4(const EwArgs<NIN> &A, int k, int64_t off) {
  if (A.bcast_inner & (1u << k)) return f4(A.in[k][off]);
  return load_operand<REUSE>(A.in[k] + off);
}

// Vectorised kernel: innermost axis has stride 1 (output, streamed inputs) or 0 (broadcast
// inputs) and a multiple-of-4 extent; the other ORANK axes (ORANK < 0: runtime count) are decoded
// from the unit index with magic division. A workgroup owns kBlock * kEwUnroll consecutive units,
// so each wave reads and writes whole contiguous 1 KiB runs per operand.
template <class Body, int ORANK, bool REUSE>
__global__ __launch_bounds__(kBlock) void ew_vec_kernel(EwArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  constexpr int kEwUnroll = Body::kUnroll;
  // measured: ordinary stores when every operand streams once, nontemporal stores when an operand
  // is re-read from cache (config 2 chain 6.2 -> 6.6 TB/s; config 3 multiply 5.4 -> 6.9 TB/s)
  constexpr bool kNtStore = PLAST_EW_NT_STORE < 0 ? REUSE : PLAST_EW_NT_STORE != 0;
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
    for (int k = 0; k < NIN; ++k) x[u][k] = load4<REUSE>(A, k, off[k]);
    oo[u] = ooff;
  }
  uint64_t idx[kEwUnroll];
  bool valid[kEwUnroll];
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    idx[u] = (base + uint64_t(u) * kBlock) * 4;
    valid[u] = base + uint64_t(u) * kBlock < A.units;
  }
  f4 r[kEwUnroll];
  body.template eval_units<kEwUnroll>(x, idx, valid, r);
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u)
    if (valid[u]) store_stream<kNtStore>(r[u], reinterpret_cast<f4 *>(A.out + oo[u]));
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

// Transposed-operand kernel. Some input is unit-stride along axis q while the output is
// unit-stride along the innermost axis p. Each workgroup owns a 64x64 (q, p) tile of one batch
// index: transposed inputs are read coalesced along q (float4) into LDS, then every output row is
// produced coalesced along p (float4) with the other inputs read directly (float4 along p, or a
// broadcast scalar). Requires extents of q and p divisible by 4 and 16-byte aligned rows.
constexpr int kTile = 64;
constexpr int kTilePad = 1;

template <int NIN>
struct TileArgs {
  const float *in[NIN];
  float *out;
  int64_t bst[NIN + 1][kMaxRank];  // batch-axis strides (output last)
  MagicDiv bdv[kMaxRank];
  int nbatch;
  int64_t qst[NIN + 1], pst[NIN + 1];
  uint32_t eq, ep;                 // extents of q and p
  uint32_t tq, tp;                 // tiles along q and p
  uint32_t lds_mask;               // bit k: input k is staged through LDS
  uint32_t lds_slot[NIN];
  uint64_t row_stride_p_index;     // elements per unit of the output's q coordinate in idx terms
};

template <class Body>
__global__ __launch_bounds__(kBlock) void ew_tile_kernel(TileArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  extern __shared__ float lds[];
  uint32_t bid = blockIdx.x;
  const uint32_t tpi = bid % A.tp;
  bid /= A.tp;
  const uint32_t tqi = bid % A.tq;
  uint32_t bi = bid / A.tq;
  int64_t base[NIN + 1] = {};
  for (int d = A.nbatch - 1; d >= 0; --d) {
    const uint32_t nxt = A.bdv[d].div(bi);
    const int64_t c = int64_t(bi - nxt * A.bdv[d].d);
    bi = nxt;
#pragma unroll
    for (int k = 0; k <= NIN; ++k) base[k] += c * A.bst[k][d];
  }
  const uint32_t q0 = tqi * kTile, p0 = tpi * kTile;
  const int t = threadIdx.x;
  // stage: thread t loads float4 (along q) of rows b = t/16 + 16r of the tile
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    if (!(A.lds_mask >> k & 1u)) continue;
    float *tile = lds + A.lds_slot[k] * (kTile * (kTile + kTilePad));
    const uint32_t a4 = (t & 15) * 4;
    f4 v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t b = (t >> 4) + 16 * r;
      if (q0 + a4 < A.eq && p0 + b < A.ep)
        v[r] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(
            A.in[k] + base[k] + int64_t(q0 + a4) * A.qst[k] + int64_t(p0 + b) * A.pst[k]));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t b = (t >> 4) + 16 * r;
#pragma unroll
      for (int c = 0; c < 4; ++c) tile[b * (kTile + kTilePad) + a4 + c] = v[r][c];
    }
  }
  // an unstaged operand constant along q (stride 0 there) has the same float4 on every output row
  // of the thread: load it once
  const uint32_t b4 = (t & 15) * 4;
  f4 rowfree[NIN];
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    rowfree[k] = f4(0.0f);
    if (!(A.lds_mask >> k & 1u) && A.qst[k] == 0 && A.pst[k] != 0 && p0 + b4 < A.ep)
      rowfree[k] = load_operand<true>(A.in[k] + base[k] + int64_t(p0 + b4) * A.pst[k]);
  }
  __syncthreads();
  // produce: thread t writes float4 (along p) of output rows a = t/16 + 16r, one row per body
  // evaluation (measured best: fewer live registers)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t a = (t >> 4) + 16 * r;
    f4 x[1][NIN];
    const uint64_t idx[1] = {0};  // the NEG rule never applies to a strided chain
    const bool valid[1] = {q0 + a < A.eq && p0 + b4 < A.ep};
    if (valid[0]) {
#pragma unroll
      for (int k = 0; k < NIN; ++k) {
        if (A.lds_mask >> k & 1u) {
          const float *tile = lds + A.lds_slot[k] * (kTile * (kTile + kTilePad));
#pragma unroll
          for (int c = 0; c < 4; ++c) x[0][k][c] = tile[(b4 + c) * (kTile + kTilePad) + a];
        } else {
          const float *src =
              A.in[k] + base[k] + int64_t(q0 + a) * A.qst[k] + int64_t(p0 + b4) * A.pst[k];
          // operands not staged through LDS are broadcast along q or p (re-read), or direct
          if (A.pst[k] == 0) x[0][k] = f4(src[0]);
          else if (A.qst[k] == 0) x[0][k] = rowfree[k];
          else x[0][k] = load_operand<true>(src);
        }
      }
    }
    f4 res[1];
    body.template eval_units<1>(x, idx, valid, res);
    if (valid[0])
      store_stream<PLAST_TILE_NT_STORE>(res[0], reinterpret_cast<f4 *>(A.out + base[NIN] +
                                                   int64_t(q0 + a) * A.qst[NIN] + int64_t(p0 + b4)));
  }
}

// Bit k set when input k of collapsed space `s` has stride 0 on an axis of extent > 1.
template <int NIN>
uint32_t reused_mask(const Space &s) {
  uint32_t m = 0;
  for (int k = 0; k < NIN; ++k)
    for (int d = 0; d < s.rank; ++d)
      if (s.st[k][d] == 0 && s.shape[d] > 1) m |= 1u << k;
  return m;
}

// Try the transposed-operand kernel on collapsed space `s`; false when the layout does not fit.
template <class Body>
bool try_tile(const Body &body, const void *const *in, void *out, const Space &s) {
  constexpr int NIN = Body::NIN;
  const int r = s.rank;
  if (r < 2 || !aligned16(out) || s.st[NIN][r - 1] != 1) return false;
  const int p = r - 1;
  int q = -1;
  for (int k = 0; k < NIN; ++k) {
    const int64_t sp = s.st[k][p];
    if (sp == 0 || sp == 1) continue;
    int qk = -1;
    for (int d = 0; d < p; ++d)
      if (s.st[k][d] == 1) qk = d;
    if (qk < 0 || (q >= 0 && qk != q)) return false;
    q = qk;
  }
  if (q < 0) return false;
  if (s.shape[p] % 4 || s.shape[q] % 4 || s.shape[p] >= (1u << 31) || s.shape[q] >= (1u << 31))
    return false;
  TileArgs<NIN> A;
  memset(&A, 0, sizeof A);
  uint32_t slots = 0;
  for (int k = 0; k <= NIN; ++k) {
    A.qst[k] = s.st[k][q];
    A.pst[k] = s.st[k][p];
    if (k < NIN) {
      A.in[k] = static_cast<const float *>(in[k]);
      const bool staged = A.pst[k] != 0 && A.pst[k] != 1;
      const bool vec_ok = staged ? (A.pst[k] % 4 == 0 && aligned16(in[k]))
                                 : (A.pst[k] == 0 || aligned16(in[k]));
      if (!vec_ok) return false;
      if (staged) {
        A.lds_mask |= 1u << k;
        A.lds_slot[k] = slots++;
      } else if (A.pst[k] == 1 && A.qst[k] % 4 != 0) {
        return false;
      }
    } else if (A.qst[k] % 4 != 0) {
      return false;
    }
  }
  uint64_t batch = 1;
  int nb = 0;
  for (int d = 0; d < p; ++d) {
    if (d == q) continue;
    for (int k = 0; k <= NIN; ++k) {
      A.bst[k][nb] = s.st[k][d];
      const bool f4_operand = k == NIN || !((A.lds_mask >> k & 1u) == 0 && A.pst[k] == 0);
      if (f4_operand && s.st[k][d] % 4 != 0) return false;
    }
    A.bdv[nb] = MagicDiv::make(uint32_t(s.shape[d]));
    batch *= s.shape[d];
    ++nb;
  }
  A.nbatch = nb;
  A.out = static_cast<float *>(out);
  A.eq = uint32_t(s.shape[q]);
  A.ep = uint32_t(s.shape[p]);
  A.tq = ceil_div(A.eq, kTile);
  A.tp = ceil_div(A.ep, kTile);
  const uint64_t blocks = batch * A.tq * A.tp;
  if (blocks >= (uint64_t(1) << 31)) return false;
  const size_t lds_bytes = size_t(slots) * kTile * (kTile + kTilePad) * sizeof(float);
  ew_tile_kernel<Body><<<unsigned(blocks), kBlock, lds_bytes, stream()>>>(A, body);
  return true;
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
  A.reused = reused_mask<NIN>(s);

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
    const unsigned grid = ceil_div(A.units, uint64_t(kBlock) * Body::kUnroll);
    // a broadcast-inner operand is a scalar load; only float4-streamed operands decide the policy
    const bool reuse = (A.reused & ~A.bcast_inner) != 0;
    if (reuse) {
      switch (in_ax) {
      case 0: ew_vec_kernel<Body, 0, true><<<grid, kBlock, 0, stream()>>>(A, body); break;
      case 1: ew_vec_kernel<Body, 1, true><<<grid, kBlock, 0, stream()>>>(A, body); break;
      case 2: ew_vec_kernel<Body, 2, true><<<grid, kBlock, 0, stream()>>>(A, body); break;
      default: ew_vec_kernel<Body, -1, true><<<grid, kBlock, 0, stream()>>>(A, body); break;
      }
    } else {
      switch (in_ax) {
      case 0: ew_vec_kernel<Body, 0, false><<<grid, kBlock, 0, stream()>>>(A, body); break;
      case 1: ew_vec_kernel<Body, 1, false><<<grid, kBlock, 0, stream()>>>(A, body); break;
      case 2: ew_vec_kernel<Body, 2, false><<<grid, kBlock, 0, stream()>>>(A, body); break;
      default: ew_vec_kernel<Body, -1, false><<<grid, kBlock, 0, stream()>>>(A, body); break;
      }
    }
    return true;
  }

  // --- transposed-operand path
  if (n < (uint64_t(1) << 32) && try_tile(body, in, out, s)) return true;

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
