// chain_jit.hpp — fused elementwise chains compiled into straight-line kernels at first use.
#pragma once

#include <cstdint>

#include "plast_hip.h"

namespace plast {

// Launch the compiled form of `t` over a flat space of `units` float4 units: input k is read
// unit-stride, or as one broadcast scalar when bit k of `bcast` is set; the output is unit-stride.
// Returns false, having launched nothing, when the chain compiler is switched off, the space is
// below its size threshold or beyond one launch, or the runtime compiler is unavailable; the
// caller then runs the tape interpreter, which computes the same bits.
bool chain_jit_launch(const PlastFusedTape &t, const float *const *in, uint32_t bcast, float *out,
                      uint64_t units, uint64_t simd_end);

// The compiled form over [units / inner4, inner4] float4 units (rows form): input k starts row r at
// in[k] + r * ist[k]; bit k of `scalar` makes it one value per row, bit k of `reread` marks a row
// stride of 0 (the same row re-read for every row); output rows start at out + r * ost.
bool chain_jit_rows_launch(const PlastFusedTape &t, const float *const *in, const int64_t *ist,
                           uint32_t scalar, uint32_t reread, float *out, int64_t ost,
                           uint64_t units, uint32_t inner4, uint64_t simd_end);

// Where a transposed-operand tile launch reads and writes (the interpreter's TileArgs, with the
// output's strides at index PLAST_TAPE_MAX_INPUTS and magic divisors as {mul, shift, d}).
struct ChainTileGeometry {
  const float *in[PLAST_TAPE_MAX_INPUTS];
  float *out;
  int64_t bst[PLAST_TAPE_MAX_INPUTS + 1][PLAST_MAX_NDIM];
  uint32_t bdv[PLAST_MAX_NDIM][3];
  int64_t qst[PLAST_TAPE_MAX_INPUTS + 1];
  int64_t pst[PLAST_TAPE_MAX_INPUTS + 1];
  uint32_t nbatch, tq, tp;
  uint32_t dtq[3], dtp[3];
};

// The compiled form of `t` as a transposed-operand tile kernel over whole 64x64 tiles: operand k's
// role is bits 2k..2k+1 of `roles` (0 staged through LDS, 1 broadcast along p, 2 broadcast along
// q, 3 read directly), as ew_tile_fixed_kernel takes them. Same threshold and fallback as above.
bool chain_jit_tile_launch(const PlastFusedTape &t, const ChainTileGeometry &g, uint32_t roles,
                           uint64_t elements, uint64_t simd_end, unsigned blocks, size_t lds_bytes);

}  // namespace plast
