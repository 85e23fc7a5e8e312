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

}  // namespace plast
