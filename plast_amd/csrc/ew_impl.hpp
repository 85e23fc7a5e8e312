// ew_impl.hpp — kernels and host dispatch of the elementwise engine (included by the translation
// units that instantiate it).
#pragma once

#include <type_traits>
#include <utility>

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
// from the unit index with magic division. A workgroup owns kEwBlock * kEwUnroll consecutive units,
// so each wave reads and writes whole contiguous 1 KiB runs per operand.
template <class Body, bool REUSE>
struct VecLaunch {
  static constexpr int block = Body::kTape ? (REUSE ? PLAST_TAPE_REUSE_BLOCK : PLAST_TAPE_BLOCK)
                                           : REUSE ? PLAST_EWR_BLOCK : PLAST_EW_BLOCK;
  static constexpr int unroll = Body::kTape ? PLAST_TAPE_UNROLL : REUSE ? PLAST_EWR_UNROLL : PLAST_EW_UNROLL;
  static constexpr bool xcd = (Body::kTape ? PLAST_TAPE_XCD : REUSE ? PLAST_EWR_XCD : PLAST_EW_XCD) != 0;
};

template <class Body, int ORANK, bool REUSE>
__global__ __launch_bounds__((VecLaunch<Body, REUSE>::block)) void ew_vec_kernel(EwArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  constexpr int kEwBlock = VecLaunch<Body, REUSE>::block;
  constexpr int kEwUnroll = VecLaunch<Body, REUSE>::unroll;
  // measured: ordinary stores when every operand streams once, nontemporal stores when an operand
  // is re-read from cache (config 2 chain 6.2 -> 6.6 TB/s; config 3 multiply 5.4 -> 6.9 TB/s)
  constexpr bool kNtStore = PLAST_EW_NT_STORE < 0 ? REUSE : PLAST_EW_NT_STORE != 0;
  const uint32_t bid = VecLaunch<Body, REUSE>::xcd ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const uint64_t base = uint64_t(bid) * (kEwBlock * kEwUnroll) + threadIdx.x;
  const uint32_t words = body.load_words();
  f4 x[kEwUnroll][NIN];
  int64_t oo[kEwUnroll];
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u) {
    const uint64_t q = base + uint64_t(u) * kEwBlock;
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
    idx[u] = (base + uint64_t(u) * kEwBlock) * 4;
    valid[u] = base + uint64_t(u) * kEwBlock < A.units;
  }
  f4 r[kEwUnroll];
  body.template eval_units_with<kEwUnroll>(words, x, idx, valid, r);
#pragma unroll
  for (int u = 0; u < kEwUnroll; ++u)
    if (valid[u]) store_stream<kNtStore>(r[u], reinterpret_cast<f4 *>(A.out + oo[u]));
}

// Generic kernel: any strides, one element per lane per step. IDX64 selects 64-bit division for
// spaces of 2^32 elements or more. The loop runs per workgroup, not per lane, so every lane is
// active when the body is evaluated (the tape interpreter reads its instruction words across the
// wave's lanes); lanes past the end only skip their loads and their store.
template <class Body, bool IDX64>
__global__ __launch_bounds__(kBlock) void ew_generic_kernel(EwArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  const uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t e0 = uint64_t(blockIdx.x) * kBlock; e0 < A.n; e0 += stride) {
    const uint64_t e = e0 + threadIdx.x;
    const bool in_range = e < A.n;
    int64_t off[NIN] = {};
    int64_t ooff = 0;
    if (!in_range) {
      // nothing to address: the loads and the store below are skipped
    } else if constexpr (IDX64) {
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
    for (int k = 0; k < NIN; ++k) v[k] = in_range ? A.in[k][off[k]] : 0.0f;
    const float r = body.eval(v, e);
    if (in_range) A.out[ooff] = r;
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
  MagicDiv dtq, dtp;
  uint32_t lds_mask;               // bit k: input k is staged through LDS
  uint32_t lds_slot[NIN];
  uint64_t row_stride_p_index;     // elements per unit of the output's q coordinate in idx terms
};

// DIRECT: whether some operand has role 3 (below); without one, the produce loop issues no global
// load at all, so nothing in it waits on the memory counter that its stores advance.
template <class Body, bool DIRECT>
__global__ __launch_bounds__(kBlock) void ew_tile_kernel(TileArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  extern __shared__ float lds[];
  uint32_t bid = PLAST_TILE_XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
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
  const uint32_t words = body.load_words();
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
  // Operand roles, two bits each, held in one SGPR for the produce loop (re-reading them from the
  // argument block there would wait on the counter that also tracks the LDS reads):
  // 0 staged through LDS, 1 broadcast along p (one scalar per output row), 2 broadcast along q
  // (one float4 for all of the thread's rows), 3 direct (float4 along p, read per row).
  uint32_t roles = 0, slots = 0;
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    const uint32_t role = (A.lds_mask >> k & 1u) ? 0u : A.pst[k] == 0 ? 1u : A.qst[k] == 0 ? 2u : 3u;
    roles |= role << (2 * k);
    slots |= (A.lds_slot[k] & 3u) << (2 * k);
  }
  roles = __builtin_amdgcn_readfirstlane(roles);
  slots = __builtin_amdgcn_readfirstlane(slots);
  // Roles 1 and 2 are read here, before the barrier and before any store: on this architecture one
  // memory counter covers loads and stores, so a load waited for after a store also waits for it.
  const uint32_t b4 = (t & 15) * 4;
  f4 pre[NIN];
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    pre[k] = f4(0.0f);
    const uint32_t role = roles >> (2 * k) & 3u;
    const float *in = A.in[k] + base[k];
    if (role == 1u) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t a = (t >> 4) + 16 * r;
        if (q0 + a < A.eq) pre[k][r] = in[int64_t(q0 + a) * A.qst[k]];
      }
    } else if (role == 2u) {
      if (p0 + b4 < A.ep) pre[k] = load_operand<true>(in + int64_t(p0 + b4) * A.pst[k]);
    }
  }
  // consume every prefetched register on every path here, so no wait for them lands after a store
#pragma unroll
  for (int k = 0; k < NIN; ++k) asm volatile("" : "+v"(pre[k]));
  __syncthreads();
  // produce: thread t writes float4 (along p) of output rows a = t/16 + 16r, one row per body
  // evaluation (fewer live registers)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t a = (t >> 4) + 16 * r;
    f4 x[1][NIN];
    const uint64_t idx[1] = {0};  // the NEG rule never applies to a strided chain
    const bool valid[1] = {q0 + a < A.eq && p0 + b4 < A.ep};
#pragma unroll
    for (int k = 0; k < NIN; ++k) {
      const uint32_t role = roles >> (2 * k) & 3u;
      if (role == 0u) {
        const float *tile = lds + (slots >> (2 * k) & 3u) * (kTile * (kTile + kTilePad));
#pragma unroll
        for (int c = 0; c < 4; ++c) x[0][k][c] = tile[(b4 + c) * (kTile + kTilePad) + a];
      } else if (role == 1u) {
        x[0][k] = f4(pre[k][r]);
      } else if (role == 2u) {
        x[0][k] = pre[k];
      } else if (DIRECT && valid[0]) {
        x[0][k] = load_operand<true>(A.in[k] + base[k] + int64_t(q0 + a) * A.qst[k] +
                                     int64_t(p0 + b4) * A.pst[k]);
      } else {
        x[0][k] = f4(0.0f);
      }
    }
    f4 res[1];
    body.template eval_units_with<1>(words, x, idx, valid, res);
    if (valid[0])
      store_stream<PLAST_TILE_NT_STORE>(res[0], reinterpret_cast<f4 *>(A.out + base[NIN] +
                                                   int64_t(q0 + a) * A.qst[NIN] + int64_t(p0 + b4)));
  }
}

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 (a loop whose index is a constant
// expression).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr uint32_t tile_role(uint32_t roles, int k) { return (roles >> (2 * k)) & 3u; }

// Tile kernel with compile-time operand roles (two bits per operand in ROLES, same meaning as
// above) for spaces whose q and p extents are multiples of the tile (no edge guards), and for the
// role patterns launch_tile_fixed lists. Every global read of the tile is issued before the
// barrier, into registers sized for exactly the roles present, from one base address per operand
// plus a constant row step; the produce loop reads only LDS and registers, so the compiler places
// no memory-counter wait between the stores of one row and the next.
template <class Body, uint32_t ROLES>
__global__ __launch_bounds__(kBlock) void ew_tile_fixed_kernel(TileArgs<Body::NIN> A, Body body) {
  constexpr int NIN = Body::NIN;
  extern __shared__ float lds[];
  const uint32_t bid = PLAST_TILE_XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const uint32_t bq = A.dtp.div(bid);         // blockIdx = (batch * tq + tqi) * tp + tpi
  const uint32_t tpi = bid - bq * A.tp;
  const uint32_t bi = A.dtq.div(bq);
  const uint32_t tqi = bq - bi * A.tq;
  int64_t base[NIN + 1] = {};
  uint32_t rem = bi;
  for (int d = A.nbatch - 1; d >= 0; --d) {
    const uint32_t nxt = A.bdv[d].div(rem);
    const int64_t c = int64_t(rem - nxt * A.bdv[d].d);
    rem = nxt;
#pragma unroll
    for (int k = 0; k <= NIN; ++k) base[k] += c * A.bst[k][d];
  }
  const int64_t q0 = int64_t(tqi) * kTile, p0 = int64_t(tpi) * kTile;
  const int t = threadIdx.x;
  const uint32_t l4 = (t & 15) * 4, r16 = t >> 4;
  const uint32_t words = body.load_words();

  // staged (role 0): float4 along q of tile rows p0 + r16 + 16r; role 1: the scalar of each output
  // row q0 + r16 + 16r; role 2: one float4 along p; role 3: float4 along p of each output row
  f4 v[NIN][4];
  static_for<NIN>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr uint32_t role = tile_role(ROLES, k);
    const float *in = A.in[k] + base[k];
    if constexpr (role == 0) {
      const float *src = in + (q0 + l4) * A.qst[k] + (p0 + r16) * A.pst[k];
      const int64_t step = 16 * A.pst[k];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[k][r] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(src + r * step));
    } else if constexpr (role == 1) {
      const float *src = in + (q0 + r16) * A.qst[k];
      const int64_t step = 16 * A.qst[k];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[k][r] = f4(src[r * step]);
    } else if constexpr (role == 2) {
      v[k][0] = load_operand<true>(in + (p0 + l4) * A.pst[k]);
    } else {
      const float *src = in + (q0 + r16) * A.qst[k] + (p0 + l4);
      const int64_t step = 16 * A.qst[k];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[k][r] = load_operand<true>(src + r * step);
    }
  });
  // staged operands to LDS, in operand order (the host numbers their slots the same way)
  static_for<NIN>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    if constexpr (tile_role(ROLES, k) == 0) {
      int slot = 0;
      for (int j = 0; j < k; ++j) slot += tile_role(ROLES, j) == 0 ? 1 : 0;
      float *tile = lds + slot * (kTile * (kTile + kTilePad));
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) tile[(r16 + 16 * r) * (kTile + kTilePad) + l4 + c] = v[k][r][c];
    }
  });
  __syncthreads();
  float *dst = A.out + base[NIN] + (q0 + r16) * A.qst[NIN] + (p0 + l4);
  const int64_t dstep = 16 * A.qst[NIN];
  // TR output rows per body evaluation: an interpreted body pays its dispatch once per TR rows
  constexpr int TR = Body::kTileRows;
#pragma unroll
  for (int h = 0; h < 4 / TR; ++h) {
    f4 x[TR][NIN];
#pragma unroll
    for (int u = 0; u < TR; ++u) {
      const int r = h * TR + u;
      const uint32_t a = r16 + 16 * r;
      static_for<NIN>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (tile_role(ROLES, k) == 0) {
          int slot = 0;
          for (int j = 0; j < k; ++j) slot += tile_role(ROLES, j) == 0 ? 1 : 0;
          const float *tile = lds + slot * (kTile * (kTile + kTilePad));
#pragma unroll
          for (int c = 0; c < 4; ++c) x[u][k][c] = tile[(l4 + c) * (kTile + kTilePad) + a];
        } else if constexpr (tile_role(ROLES, k) == 2) {
          x[u][k] = v[k][0];
        } else {
          x[u][k] = v[k][r];
        }
      });
    }
    uint64_t idx[TR];
    bool valid[TR];
#pragma unroll
    for (int u = 0; u < TR; ++u) {
      idx[u] = 0;  // the NEG rule never applies to a strided chain
      valid[u] = true;
    }
    f4 res[TR];
    body.template eval_units_with<TR>(words, x, idx, valid, res);
#pragma unroll
    for (int u = 0; u < TR; ++u)
      store_stream<PLAST_TILE_NT_STORE>(res[u], reinterpret_cast<f4 *>(dst + (h * TR + u) * dstep));
  }
}

constexpr uint32_t tile_roles(uint32_t r0, uint32_t r1 = 0, uint32_t r2 = 0) {
  return r0 | r1 << 2 | r2 << 4;
}

// Launch the fixed-role kernel when `roles` is one of the instantiated patterns.
template <class Body>
bool launch_tile_fixed(const TileArgs<Body::NIN> &A, const Body &body, uint32_t roles,
                       unsigned blocks, size_t lds_bytes) {
  constexpr int NIN = Body::NIN;
#define PLAST_TILE_CASE(R)                                                                         \
  case R:                                                                                          \
    ew_tile_fixed_kernel<Body, R><<<blocks, kBlock, lds_bytes, stream()>>>(A, body);               \
    return true;
  if constexpr (NIN == 1) {
    switch (roles) { PLAST_TILE_CASE(tile_roles(0)) default: return false; }
  } else if constexpr (NIN == 2) {
    switch (roles) {
      PLAST_TILE_CASE(tile_roles(0, 0))
      PLAST_TILE_CASE(tile_roles(0, 1))
      PLAST_TILE_CASE(tile_roles(1, 0))
      PLAST_TILE_CASE(tile_roles(0, 2))
      PLAST_TILE_CASE(tile_roles(2, 0))
      PLAST_TILE_CASE(tile_roles(0, 3))
      PLAST_TILE_CASE(tile_roles(3, 0))
    default: return false;
    }
  } else if constexpr (NIN == 3 && Body::kTileFixed3) {
    switch (roles) {
      PLAST_TILE_CASE(tile_roles(0, 1, 2))
      PLAST_TILE_CASE(tile_roles(0, 2, 1))
      PLAST_TILE_CASE(tile_roles(0, 1, 1))
      PLAST_TILE_CASE(tile_roles(0, 2, 2))
      PLAST_TILE_CASE(tile_roles(0, 3, 3))
    default: return false;
    }
  } else {
    return false;
  }
#undef PLAST_TILE_CASE
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
  if (blocks > max_blocks(kBlock)) return false;
  const size_t lds_bytes = size_t(slots) * kTile * (kTile + kTilePad) * sizeof(float);
  bool direct = false;
  uint32_t roles = 0;
  for (int k = 0; k < NIN; ++k) {
    const uint32_t role = (A.lds_mask >> k & 1u) ? 0u : A.pst[k] == 0 ? 1u : A.qst[k] == 0 ? 2u : 3u;
    direct = direct || role == 3u;
    roles |= role << (2 * k);
  }
  A.dtq = MagicDiv::make(A.tq);
  A.dtp = MagicDiv::make(A.tp);
  const bool full = A.eq % kTile == 0 && A.ep % kTile == 0;
  if (full && launch_tile_fixed(A, body, roles, unsigned(blocks), lds_bytes)) return true;
  if (direct) ew_tile_kernel<Body, true><<<unsigned(blocks), kBlock, lds_bytes, stream()>>>(A, body);
  else ew_tile_kernel<Body, false><<<unsigned(blocks), kBlock, lds_bytes, stream()>>>(A, body);
  return true;
}

// ------------------------------------------------------------------------- host dispatch

// Returns false (launching nothing) when the grid would exceed the dispatch limit.
template <class Body, bool REUSE>
bool launch_vec(const EwArgs<Body::NIN> &A, const Body &body, int in_ax) {
  using L = VecLaunch<Body, REUSE>;
  const uint64_t blocks = (A.units + uint64_t(L::block) * L::unroll - 1) / (uint64_t(L::block) * L::unroll);
  if (blocks > max_blocks(L::block)) return false;
  const unsigned grid = unsigned(blocks);
  switch (in_ax) {
  case 0: ew_vec_kernel<Body, 0, REUSE><<<grid, L::block, 0, stream()>>>(A, body); break;
  case 1: ew_vec_kernel<Body, 1, REUSE><<<grid, L::block, 0, stream()>>>(A, body); break;
  case 2: ew_vec_kernel<Body, 2, REUSE><<<grid, L::block, 0, stream()>>>(A, body); break;
  default: ew_vec_kernel<Body, -1, REUSE><<<grid, L::block, 0, stream()>>>(A, body); break;
  }
  return true;
}

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
    // a broadcast-inner operand is a scalar load; only float4-streamed operands decide the policy
    const bool done = (A.reused & ~A.bcast_inner) != 0 ? launch_vec<Body, true>(A, body, in_ax)
                                                       : launch_vec<Body, false>(A, body, in_ax);
    if (done) return true;
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
