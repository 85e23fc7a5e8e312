// common.hpp — shared host/device machinery of the gfx950 backend: error reporting, the library
// stream, workspace, 32-bit magic-number division and host-side dimension collapsing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/plast_hip.h"

namespace plast {

constexpr int kMaxRank = PLAST_MAX_NDIM;
constexpr int kBlock = 256;  // threads per workgroup for streaming kernels (4 wave64s)

// Launch-shape knobs, measured on MI355X (overridable with -D for sweeps).
// Vectorised elementwise kernel, per kind of launch: fixed bodies whose operands all stream once
// (EW), fixed bodies with an operand re-read along a broadcast axis (EWR), fused-chain tapes (TAPE).
// BLOCK: threads per workgroup; UNROLL: float4 units per lane; XCD 1: consecutive workgroup ranges
// are mapped onto one XCD each. Measured on MI355X over 64M-element launches: streaming bodies
// 6.56 -> 7.03-7.15 TB/s with one unit per lane and the XCD mapping (256/4/0 before); the
// broadcast multiply of config 3 6.91 -> 7.02 TB/s at 512/2 (the XCD mapping costs it 10%); the
// tape interpreter is fastest at 256/2 without the mapping (one unit per lane: -10 to -15%).
#ifndef PLAST_EW_BLOCK
#define PLAST_EW_BLOCK 256
#endif
#ifndef PLAST_EW_UNROLL
#define PLAST_EW_UNROLL 1
#endif
#ifndef PLAST_EW_XCD
#define PLAST_EW_XCD 1
#endif
#ifndef PLAST_EWR_BLOCK
#define PLAST_EWR_BLOCK 512
#endif
#ifndef PLAST_EWR_UNROLL
#define PLAST_EWR_UNROLL 2
#endif
#ifndef PLAST_EWR_XCD
#define PLAST_EWR_XCD 0
#endif
// Tape launches streaming every operand once: workgroup size. Measured in one process on config 2's
// chain (two calls): 256 lanes 6555 / 6699 GB/s, 512 6692 / 6801, 384 6650, 768 6661, 1024 6425,
// 256 with the XCD numbering 6395.
#ifndef PLAST_TAPE_BLOCK
#define PLAST_TAPE_BLOCK 512
#endif
#ifndef PLAST_TAPE_UNROLL
#define PLAST_TAPE_UNROLL 2
#endif
#ifndef PLAST_TAPE_XCD
#define PLAST_TAPE_XCD 0
#endif
// Workgroup size of a tape launch that re-reads an operand (a broadcast one) from cache. Measured
// in one process on relu(X + b) over [16384, 4096]: 256 lanes 6372 GB/s, 512 6539, 1024 6593
// (every tape instantiation stays under 128 VGPRs, no spills); config 1's call unchanged.
#ifndef PLAST_TAPE_REUSE_BLOCK
#define PLAST_TAPE_REUSE_BLOCK 1024
#endif
#ifndef PLAST_TAPE_TILE_ROWS
#define PLAST_TAPE_TILE_ROWS 2  // fused chains in the transposed-operand tile: rows per evaluation
#endif
#ifndef PLAST_ROW_UNROLL
#define PLAST_ROW_UNROLL 4   // float4 loads in flight per lane, row reductions
#endif
#ifndef PLAST_ROW_WAVES
// Row reductions: split few long rows into ordered segments up to this many waves. Measured on a
// whole-tensor sum / max of 2^28 floats (one row): 2048 segments (two workgroups per CU) 6.73 /
// 6.32 TB/s, 3072 the same, 4096 6.44-6.48 / 6.16 (a longer finalize), 8192 and up 6.05 / 5.79;
// 1536 and fewer leave CUs idle.
#define PLAST_ROW_WAVES 2048
#endif
// Rows in flight per lane, leading-axis reductions, for one-, two- and three-operand producers.
// Measured (two alternating runs): one operand with 2 rather than 4 rows, the axis-0 sum of
// [4096, 65536] 6.60-6.64 -> 6.72-6.74 TB/s, config 5's bias gradient 6.24-6.26 -> 6.41-6.42, the
// [16384, 4096] bias gradient 5.24-5.31 -> 5.61-5.64 (1 row loses 11-17% on the first two); two
// operands (the one-pass relu-gradient modulation and bias sum) 5.38-5.65 with 4 rows, 5.59-5.82
// with 2, 6.02-6.06 with 1. Three operands (the fused leaky_relu(x + bias) backward, the
// [16384, 4096] step, in one process): 2 rows 6.00-6.01 TB/s against 5.77-5.91 with 1.
#ifndef PLAST_COL_UNROLL
#define PLAST_COL_UNROLL 2
#endif
#ifndef PLAST_COL_UNROLL2
#define PLAST_COL_UNROLL2 1
#endif
#ifndef PLAST_COL_UNROLL3
#define PLAST_COL_UNROLL3 2  // three operands and more
#endif
// Stores of a storing producer in the leading-axis kernels (1: nontemporal, 0: ordinary, -1:
// nontemporal exactly when the stored buffer is also an operand, read in the same pass). Measured
// in one process on [16384, 4096]: the fused leaky_relu(x + bias) step (dx read and written)
// 5.36-5.41 -> 5.91-5.92 TB/s with nontemporal stores; the one-pass epilogue (dc only written)
// 6.25-6.28 -> 5.94 with them.
#ifndef PLAST_COL_NT_STORE
#define PLAST_COL_NT_STORE -1
#endif
// Leading-axis finalize: lanes per output when there are at least twice as many chunks (1: one
// lane, batches of 16 loads in sequence). Measured (two alternating runs): 8 lanes took config 1's
// grad_b (16 chunks) from 9.4-9.9 to 7.3-7.5 us per call and the one-pass epilogue (64 chunks)
// +3%, the [16384, 4096] bias gradient unchanged; 4 lanes lost 5% on that bias gradient. In one
// process (two calls, either order): 16 lanes took that bias gradient from 5603 / 5731 to
// 5748 / 5864 GB/s and the one-pass epilogue +0.7-1.5%; 32 lanes land between.
#ifndef PLAST_COL_FIN_Q
#define PLAST_COL_FIN_Q 16
#endif
// Small leading-axis sums (at most PLAST_COL_SMALL_MAX input elements) in one launch: workgroups
// of PLAST_COL_SMALL_S4 float4 columns (PLAST_COL_SMALL_S4_3 for three operands and more) that
// walk every row, instead of row chunks plus a finalize; PLAST_COL_SMALL3 = 0 sends three-operand
// producers to the chunked pass, whose chunks keep at least PLAST_COL_MIN_ROWS3 rows.
// PLAST_COL_SMALL_XCD numbers the column slices per XCD, so that the slices sharing a 128-byte
// line run on one XCD. Measured in one process (device time of calls replayed from a graph),
// config 1's fused step [1024, 256] (the forward, then the backward's 3-operand sum) in GB/s:
// slices of 4 float4 columns 403, of 1 float4 column 453 without and 589 with the numbering,
// against 571 for the chunked pass (16-row chunks) with its finalize launch and 475 for that pass
// with the last workgroup merging the partials itself (a device-scope fence per workgroup; it
// also cost the [16384, 4096] sums 25-40%, and was removed). Config 1's grad_b (1 operand):
// 355 -> 386 with 2 float4 columns per slice and the numbering.
#ifndef PLAST_COL_SMALL_MAX
#define PLAST_COL_SMALL_MAX (1u << 21)
#endif
#ifndef PLAST_COL_SMALL_S4
#define PLAST_COL_SMALL_S4 2
#endif
#ifndef PLAST_COL_SMALL_S4_3
#define PLAST_COL_SMALL_S4_3 1
#endif
// rows each lane loads per batch in the small leading-axis sum (three operands and more: config 1's
// fused backward step 10.6 -> 10.0 us on the device with 4, 10.1 with 2, against 8; one operand
// keeps 8, with 2 its grad_b launch ran 9% slower)
#ifndef PLAST_COL_SMALL_U
#define PLAST_COL_SMALL_U 8
#endif
#ifndef PLAST_COL_SMALL_U3
#define PLAST_COL_SMALL_U3 4
#endif
#ifndef PLAST_COL_SMALL3
#define PLAST_COL_SMALL3 1
#endif
#ifndef PLAST_COL_MIN_ROWS3
#define PLAST_COL_MIN_ROWS3 64
#endif
#ifndef PLAST_COL_SMALL_XCD
#define PLAST_COL_SMALL_XCD 1
#endif
// Workgroups a leading-axis reduction is chunked up to (512, 2048 and 4096 measured slower on every
// leading-axis workload of the bench). A row stream for whole contiguous rows
// of 2048-16384 columns (one 1024-lane workgroup per CU walking every G-th row, its column sums
// in registers, then a finalize over the per-workgroup partials) was measured against this in one
// process and removed: the [16384, 4096] bias gradient 5.40 against 5.62 TB/s, the one-pass
// modulation + bias gradient 5.57 against 6.18.
#ifndef PLAST_COL_BLOCKS
#define PLAST_COL_BLOCKS 1024
#endif
// Store policy per kernel family (1: nontemporal, 0: ordinary stores).
#ifndef PLAST_EW_NT_STORE
#define PLAST_EW_NT_STORE -1  // -1: nontemporal exactly when the launch re-reads an operand
#endif
#ifndef PLAST_TILE_XCD
#define PLAST_TILE_XCD 1     // transposed-operand tiles: XCD-contiguous workgroup numbering
#endif
#ifndef PLAST_TILE_NT_STORE
#define PLAST_TILE_NT_STORE 0
#endif
#ifndef PLAST_CE_NT_STORE
#define PLAST_CE_NT_STORE 1
#endif
// Persistent row kernels: workgroup numbers renumbered so that each XCD holds a contiguous range
// (1) or dispatch order (0). Measured in one process: softmax forward 5947 against 5920 GB/s, the
// one-pass step unchanged (5759 / 5760): neutral within the 1-1.3% that two copies of one build
// differ by in such a comparison.
#ifndef PLAST_ROW_XCD
#define PLAST_ROW_XCD 1
#endif
// Persistent row kernels: rows taken in pairs from a device counter (1) or the static strided
// schedule (0; the one-pass step always uses it in deterministic mode). Measured with copies of
// whole 128 KB rows by persistent 1024-lane workgroups on MI355X: 5.64-5.75 TB/s with the static
// schedule (the odd XCDs finish about 8% after the even ones), 6.35-6.43 taking rows from a
// counter, against 6.53 for the flat copy.
#ifndef PLAST_ROW_DYNAMIC
#define PLAST_ROW_DYNAMIC 1
#endif
#ifndef PLAST_CE_STEP_NT_LOAD
#define PLAST_CE_STEP_NT_LOAD 1  // the one-pass step's row loads: nontemporal (1) or ordinary (0)
#endif
#ifndef PLAST_COPY_NT_STORE
#define PLAST_COPY_NT_STORE 0
#endif
#ifndef PLAST_SGD_XCD
#define PLAST_SGD_XCD 1      // SGD launches holding one tensor entry
#endif
#ifndef PLAST_ADAM_XCD
#define PLAST_ADAM_XCD 0     // Adam/AdamW launches holding one tensor entry
#endif
#ifndef PLAST_SGD_BLOCK
#define PLAST_SGD_BLOCK 256  // optimizer workgroup sizes
#endif
#ifndef PLAST_ADAM_BLOCK
#define PLAST_ADAM_BLOCK 64
#endif
#ifndef PLAST_ADAM_NT_LOAD
#define PLAST_ADAM_NT_LOAD 1  // Adam/AdamW parameter and moment loads
#endif
#ifndef PLAST_ADAM_NT_STORE
#define PLAST_ADAM_NT_STORE 1
#endif
#ifndef PLAST_COPY_UNROLL
#define PLAST_COPY_UNROLL 1  // float4 per lane, device copy (256 MiB: 6.75 -> 7.07 TB/s with the
#endif                       // XCD numbering, against 4 per lane without)
#ifndef PLAST_COPY_XCD
#define PLAST_COPY_XCD 1
#endif
// XCD-contiguous workgroup numbering elsewhere, measured (4 alternating runs each): row and
// leading-axis reductions lose 3-12% with it (not used there); the flat cross-entropy backward
// gains 2.8% when accumulating (on); a single-tensor SGD launch gains with it, a launch over many
// tensors loses (on for one-entry launches only); Adam/AdamW with 64-lane workgroups lose 3% with
// it (off).
#ifndef PLAST_CE_BWD_XCD
#define PLAST_CE_BWD_XCD 1
#endif
#ifndef PLAST_CE_UNROLL
#define PLAST_CE_UNROLL 8     // cross-entropy forward: float4 loads in flight per lane
#endif
#ifndef PLAST_OPT_UNROLL
#define PLAST_OPT_UNROLL 1    // optimizer updates: float4 units per lane
#endif
// Softmax forward and backward variants measured at [32768, 32000] in one process (so on the same
// box and in the same process state): the persistent forward with one barrier per row (per-wave
// maxima and sums merged after it) 5.81 TB/s against 5.89 for two; the backward with the input
// gradient's loads issued with y and dy 5.64 against 5.62-5.64 without, and 5.54-5.65 at 1024
// lanes. Neither was kept.
// Softmax backward: the input gradient's read-modify-write nontemporal (1) or ordinary (0).
// Measured at [32768, 32000] in one process: 5.96 TB/s against 5.61.
#ifndef PLAST_SOFTMAX_BWD_NT
#define PLAST_SOFTMAX_BWD_NT 1
#endif
// Softmax backward, rows held in registers: lanes per row.
// Softmax backward: dx float4 units per lane loaded together with y and dy, ahead of the row's
// reduction (at least V: all of them). Measured in one process at [32768, 32000]: none 5946 GB/s,
// 4 units 5538, 8 units 5690, all 16 6099 (1024 lanes with all 8: 6103).
#ifndef PLAST_SOFTMAX_BWD_PRE
#define PLAST_SOFTMAX_BWD_PRE 32
#endif
#ifndef PLAST_SOFTMAX_BWD_BLOCK
#define PLAST_SOFTMAX_BWD_BLOCK 512
#endif
#ifndef PLAST_SOFTMAX_BLOCK
#define PLAST_SOFTMAX_BLOCK 256  // softmax rows held in registers: lanes per row
#endif
#ifndef PLAST_CE_FWD_WAVES
#define PLAST_CE_FWD_WAVES 4    // cross-entropy forward: rows (one wave each) per workgroup
#endif
#ifndef PLAST_CE_BWD_BLOCK
#define PLAST_CE_BWD_BLOCK 256  // cross-entropy backward, flat form: workgroup size
#endif
// One-pass cross-entropy step: lanes per workgroup (one row). Measured on config 5's step (two
// alternating runs): 1024 lanes x 8 float4 (119 VGPRs) 5.68-5.70 TB/s, 512 x 16 (189) 5.50. In
// one process: 1024 x 8 with two register sets 5760, 512 x 16 with two 5559, 512 x 16 with three
// (254 VGPRs, two rows in flight while one is processed) 5565, and 5623 with the XCD numbering.
#ifndef PLAST_CE_STEP_BLOCK
#define PLAST_CE_STEP_BLOCK 1024
#endif
// The cross-entropy forward op keeps one wave per row: the one-pass step's row loop without its
// gradient (persistent 1024-lane workgroups) measured 5.85 TB/s against 6.52 over [32768, 32000]
// in one process and was removed.
#ifndef PLAST_CE_STEP_WPC
#define PLAST_CE_STEP_WPC 1  // one-pass cross-entropy step: persistent workgroups per CU
#endif
#ifndef PLAST_CE_BWD_UNROLL
#define PLAST_CE_BWD_UNROLL 1  // float4 units per lane, cross-entropy backward
#endif

typedef float f4 __attribute__((ext_vector_type(4)));

// The dispatch packet's grid size is 32-bit: a launch holds fewer than 2^32 work-items per
// dimension, i.e. at most max_blocks(threads) workgroups of `threads` lanes along x.
constexpr uint64_t max_blocks(uint64_t threads) { return (uint64_t(1) << 32) / threads - 1; }

// Workgroups are dispatched round-robin over the 8 XCDs. xcd_block renumbers the first
// 8 * (grid / 8) of them (a permutation) so that XCD x owns the x-th contiguous range of workgroup
// numbers, and so of the data a streaming kernel maps onto them.
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t grid) {
  const uint32_t per = grid / 8;
  return b < per * 8 ? (b % 8) * per + b / 8 : b;
}

// Store of a streamed float4 result with a compile-time cache policy.
template <bool NT>
__device__ __forceinline__ void store_stream(f4 v, f4 *p) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// ------------------------------------------------------------------------- runtime / errors

void report_error(const char *where, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
hipStream_t stream();
// Compute units of the library's device.
int num_cus();
// Whether results must be independent of timing (the one-pass step's row order is then static).
bool deterministic();
// The device the library runs on (its stream's), fixed at initialisation.
int library_device();
// Called at the end of every entry point: checks the launch and, in synchronous mode, waits.
void finish(const char *where);
// True between plast_hip_capture_begin and plast_hip_capture_end (the stream records a graph).
bool capturing();
bool ensure_init();
// Device scratch of at least `bytes`, owned by the library and reused across calls. Slot 0 holds
// the reduction engine's partial summaries; slot 1 an op's own temporaries (tie counts, extremes);
// slot 2 the staging buffer of host transfers of strided tensors.
void *workspace(size_t bytes, int slot = 0);

#define PLAST_HIP_TRY(where, expr)                                                                 \
  do {                                                                                             \
    hipError_t _e = (expr);                                                                        \
    if (_e != hipSuccess) {                                                                        \
      ::plast::report_error(where, "%s: %s", #expr, hipGetErrorString(_e));                        \
      return;                                                                                      \
    }                                                                                              \
  } while (0)

// ------------------------------------------------------------------------- magic division

// Unsigned 32-bit division by a run-time constant d >= 1 using one mul_hi, an add and a shift:
// q = (umulhi(n, m) + n) >> s, exact for every n < 2^32 (round-up multiplier method,
// Granlund & Montgomery 1994). The 33-bit intermediate is formed in 64 bits.
struct MagicDiv {
  uint32_t mul;
  uint32_t shift;
  uint32_t d;
  static MagicDiv make(uint32_t d) {
    MagicDiv m;
    m.d = d;
    uint32_t s = 0;
    while ((uint64_t(1) << s) < d) ++s;
    m.shift = s;
    m.mul = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
    return m;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#ifdef __HIP_DEVICE_COMPILE__
    uint64_t hi = __umulhi(n, mul);
#else
    uint64_t hi = (uint64_t(n) * mul) >> 32;
#endif
    return uint32_t((hi + n) >> shift);
  }
};

// ------------------------------------------------------------------------- iteration spaces

// An iteration space over `rank` dims (outermost first) shared by up to kMaxOps operands, each with
// its own element strides (0 on broadcast axes). Built from the reference's Tensor metadata.
constexpr int kMaxOps = 6;

struct Space {
  int rank = 0;
  int nops = 0;
  uint64_t shape[kMaxRank];
  int64_t st[kMaxOps][kMaxRank];
  uint64_t numel() const {
    uint64_t n = 1;
    for (int d = 0; d < rank; ++d) n *= shape[d];
    return n;
  }
};

// Right-aligned strides of tensor `t` inside an iteration space of shape `shape[0..rank)`:
// missing leading axes and size-1 axes get stride 0 (numpy broadcasting, the rule of
// include/kernels/kernel_macros.h:156-168).
void bcast_strides(const Tensor *t, const uint64_t *shape, int rank, int64_t *out);

// Drop size-1 axes and merge neighbouring axes that are jointly contiguous for every operand.
void collapse(Space &s);

// Numpy broadcast shape of two tensors; false when incompatible (cpu_utils.c:78-100).
bool broadcast_shape(const Tensor *a, const Tensor *b, uint64_t *shape, int *rank);

uint64_t numel(const Tensor *t);
bool same_shape(const Tensor *a, const Tensor *b);
// Row-major contiguity with every stride checked (size-1 axes ignored).
bool contiguous(const Tensor *t);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline unsigned ceil_div(uint64_t a, uint64_t b) { return unsigned((a + b - 1) / b); }

// Reference AVX2 block end: contiguous loops are 8-wide SIMD below n - n%8 (kernel_macros.h:195).
inline uint64_t simd_end(uint64_t n) { return n - n % 8; }

}  // namespace plast
