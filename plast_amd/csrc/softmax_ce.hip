// softmax_ce.hip — fused softmax cross-entropy over the rows of [N, C] logits with int32 labels,
// and softmax / log-softmax over the last axis.
//
// Forward, per row (the reference chain MAX -> SUB -> EXP -> SUM -> LOG -> SUB -> MUL(onehot) ->
// SUM -> NEG of src/api/loss.c:97-169, one HBM read):
//   m = the reference's max fold from -FLT_MAX (bit-exact, NaN and signed-zero rules included)
//   s = sum_j expf(x_j - m)         (parallel sum; the reference sums serially)
//   l = logf(s)
//   t = 0 + ((x_label - m) - l), or NaN when any other term 0 * ((x_j - m) - l) is NaN
//   loss = 0 - t inside the reference's SIMD blocks of its NEG node, -t in its tail
// stats[row] = (m, l) for the backward.
// Backward: dx[row, j] (+)= dloss[row] * (exp((x - m) - l) - onehot).
// The fast paths evaluate exp with exp_le0 (about 1 ulp); the exact-refold paths use expf.
#include <atomic>
#include <cfloat>

#include "common.hpp"

// Device scratch of the allocation-free one-pass step (softmax_cross_entropy_step_noalloc_hip):
// the workgroups' column sums, kScratchFloats floats (32 MiB: 256 workgroups of rows up to 32768
// floats, the widest one-pass row of 1024-lane workgroups; wider ones, of a build with narrower
// workgroups, run on fewer workgroups). Each GPU the library runs on holds its own copy until the
// process ends. Host code never passes this name to a kernel (it
// is a host-side stand-in there): noalloc_scratch() looks the device address up once per device.
static __device__ __align__(256) float scratch[uint64_t(1) << 23];

namespace plast {
namespace {

constexpr uint64_t kScratchFloats = uint64_t(1) << 23;
static_assert(sizeof(scratch) == kScratchFloats * sizeof(float), "scratch size");

// The device address of `scratch` on the library's device, found with hipGetSymbolAddress, with
// that device current, on the first call there (null, after reporting, when the lookup fails).
float *noalloc_scratch(const char *where) {
  static std::atomic<float *> addr[64] = {};
  const int dev = library_device();
  if (dev < 0 || dev >= 64) {
    report_error(where, "device %d is out of range", dev);
    return nullptr;
  }
  float *a = addr[dev].load(std::memory_order_acquire);
  if (a) return a;
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
  void *p = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess || !p) {
    report_error(where, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    return nullptr;
  }
  a = static_cast<float *>(p);
  addr[dev].store(a, std::memory_order_release);
  return a;
}

constexpr int kCeBlock = 256;
constexpr int kCeWaves = kCeBlock / 64;

// exp(t) for the shifted logits of a softmax (t <= 0), from the hardware base-2 exponential
// (v_exp_f32, accurate to 1 ulp). t*log2(e) is carried as p + d: p = t*L rounded, d = that
// product's rounding error (one FMA) plus t times the error of L itself, so
// exp(t) = 2^p * 2^d with 2^d = 1 + d*ln2 (|d| < 2^-17 for |t| < 87). About 1 ulp from the
// correctly rounded result; 6 VALU ops where the library expf takes about 15. Below t = -87 the
// result would be subnormal (< 2^-125.5) and 0 is returned; -inf gives 0 and NaN stays NaN.
// Used only where the result feeds a sum or a gradient compared to 1e-5 relative.
__device__ __forceinline__ float exp_le0(float t) {
  constexpr float kL = 1.44269502162933349609375f;   // log2(e) rounded to fp32
  constexpr float kLlo = 1.925963033500011079e-8f;   // log2(e) - kL
  constexpr float kLn2 = 0.693147180559945309f;
  const float p = t * kL;
  const float d = __builtin_fmaf(t, kLlo, __builtin_fmaf(t, kL, -p));
  const float r = __builtin_amdgcn_exp2f(p);
  const float e = __builtin_fmaf(r, d * kLn2, r);
  return t < -87.0f ? 0.0f : e;
}

// exp_le0 without the range clamp, for finite t <= 0 only (-inf would give NaN): below t = -87 it
// returns the subnormal or zero that 2^p gives. Two instructions fewer.
__device__ __forceinline__ float exp_le0_finite(float t) {
  constexpr float kL = 1.44269502162933349609375f;
  constexpr float kLlo = 1.925963033500011079e-8f;
  constexpr float kLn2 = 0.693147180559945309f;
  const float p = t * kL;
  const float d = __builtin_fmaf(t, kLlo, __builtin_fmaf(t, kL, -p));
  const float r = __builtin_amdgcn_exp2f(p);
  return __builtin_fmaf(r, d * kLn2, r);
}

// Block-wide reductions over W waves (lds holds W + 1 floats), combined in wave order.
template <int W = kCeWaves>
__device__ __forceinline__ float block_sum(float v, float *lds) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) r += lds[w];
  return r;
}

template <int W = kCeWaves>
__device__ __forceinline__ float block_fmax(float v, float *lds) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < W; ++w) r = fmaxf(r, lds[w]);
  return r;
}

template <int W = kCeWaves>
__device__ __forceinline__ bool block_any(bool b, float *lds) {
  return block_sum<W>(b ? 1.0f : 0.0f, lds) > 0.0f;
}

// The reference's serial max fold, for rows whose fast-path extreme is ambiguous (NaN or zero).
__device__ float serial_max_fold(const float *row, uint32_t C) {
  float acc = -FLT_MAX;
  for (uint32_t j = 0; j < C; ++j) acc = acc > row[j] ? acc : row[j];
  return acc;
}

// Row max with exact reference bits: fast block fmax + NaN flag; thread 0 refolds serially when
// the fast value could differ (a NaN in the row, or a zero maximum whose sign depends on order).
template <int W = kCeWaves>
__device__ __forceinline__ float row_max_exact(float m, bool nan, const float *row, uint32_t C,
                                               float *lds) {
  m = block_fmax<W>(m, lds);
  nan = block_any<W>(nan, lds);
  if (nan || m == 0.0f) {
    __syncthreads();
    if (threadIdx.x == 0) lds[W] = serial_max_fold(row, C);
    __syncthreads();
    return lds[W];
  }
  return m > -FLT_MAX ? m : -FLT_MAX;
}

// Any row length or alignment: three passes over the row (max, exp-sum, terms).
__global__ __launch_bounds__(kCeBlock) void ce_fwd_generic_kernel(const float *__restrict__ x,
                                                                  const int32_t *__restrict__ lab,
                                                                  float *__restrict__ stats,
                                                                  float *__restrict__ loss,
                                                                  uint32_t C, uint64_t simd_end) {
  __shared__ float lds[kCeWaves + 1];
  const uint64_t row = blockIdx.x;
  const float *xr = x + row * C;
  float m = -__builtin_huge_valf();
  bool nan = false;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) {
    m = fmaxf(m, xr[j]);
    nan = nan || xr[j] != xr[j];
  }
  const float mx = row_max_exact(m, nan, xr, C, lds);
  float s = 0.0f;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) s += expf(xr[j] - mx);
  s = block_sum(s, lds);
  const float l = logf(s);
  const int32_t y = lab[row];
  bool bad = false;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) {
    const float ls = (xr[j] - mx) - l;
    if (int32_t(j) != y) bad = bad || !(fabsf(ls) <= FLT_MAX);
  }
  bad = block_any(bad, lds);
  if (threadIdx.x == 0) {
    float t;
    if (bad) t = __builtin_nanf("");
    else if (y >= 0 && uint32_t(y) < C) t = 0.0f + ((xr[y] - mx) - l);
    else t = 0.0f;
    loss[row] = row < simd_end ? 0.0f - t : -t;
    stats[2 * row] = mx;
    stats[2 * row + 1] = l;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fminf(v, __shfl_xor(v, m));
  return v;
}

constexpr int kCeUnroll = PLAST_CE_UNROLL;  // float4 loads in flight per lane

// One wave64 per row, a single read of the row. Each lane keeps an online (max, exp-sum) pair,
// rescaling its sum when its max grows; the wave merges the pairs. Rows for which the fast
// values could differ from the reference chain's bits (a non-finite logit, a zero or non-finite
// max, or a shifted-and-normalised logit that overflows to -inf) are recomputed exactly by the
// same wave from memory.
constexpr int kCeFwdWaves = PLAST_CE_FWD_WAVES;  // rows (waves) per workgroup

__global__ __launch_bounds__(64 * kCeFwdWaves) void ce_fwd_wave_kernel(const float *__restrict__ x,
                                                          const int32_t *__restrict__ lab,
                                                          float *__restrict__ stats,
                                                          float *__restrict__ loss, uint64_t N,
                                                          uint32_t C, uint64_t simd_end) {
  const int lane = threadIdx.x & 63;
  const uint64_t row = uint64_t(blockIdx.x) * kCeFwdWaves + (threadIdx.x >> 6);
  if (row >= N) return;  // whole wave
  const float *xr = x + row * C;
  const int32_t y = lab[row];
  const float ninf = -__builtin_huge_valf();
  float m = ninf, s = 0.0f, mn = __builtin_huge_valf();
  const uint32_t C4 = C / 4;
  const f4 *x4 = reinterpret_cast<const f4 *>(xr);
  for (uint32_t q0 = lane; q0 < C4; q0 += 64 * kCeUnroll) {
    f4 v[kCeUnroll];
#pragma unroll
    for (int u = 0; u < kCeUnroll; ++u) {
      const uint32_t q = q0 + uint32_t(u) * 64;
      if (q < C4) v[u] = __builtin_nontemporal_load(x4 + q);
    }
#pragma unroll
    for (int u = 0; u < kCeUnroll; ++u) {
      if (q0 + uint32_t(u) * 64 >= C4) continue;
      const float g = fmaxf(fmaxf(v[u][0], v[u][1]), fmaxf(v[u][2], v[u][3]));
      if (g > m) {
        s = m == ninf ? s * 0.0f : s * exp_le0(m - g);
        m = g;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float e = v[u][c];
        mn = fminf(mn, e);
        s += exp_le0(e - m);
      }
    }
  }
  const float M = wave_max(m);
  const float sc = m == ninf ? s * 0.0f : s * exp_le0(m - M);
  float S = wave_sum(sc);
  // a NaN logit reaches the sum (fmaxf skips NaN, exp(NaN - m) does not); an infinite one makes
  // M or the minimum below non-finite
  const bool nonfin = !(S <= FLT_MAX);
  mn = wave_min(mn);
  float mx = M;
  bool exact = false;
  if (!(fabsf(M) <= FLT_MAX) || M == 0.0f || nonfin) {
    exact = true;
  }
  float l = logf(S);
  if (!exact && C > 0) {
    // the most negative shifted-normalised logit must stay finite (else 0 * -inf = NaN)
    if (!(fabsf((mn - mx) - l) <= FLT_MAX)) exact = true;
  }
  bool bad = false;
  if (exact) {
    // the reference chain, element by element (rare rows)
    float acc = -FLT_MAX;
    if (lane == 0)
      for (uint32_t j = 0; j < C; ++j) acc = acc > xr[j] ? acc : xr[j];
    mx = __shfl(acc, 0);
    float t = 0.0f;
    for (uint32_t j = lane; j < C; j += 64) t += expf(xr[j] - mx);
    S = wave_sum(t);
    l = logf(S);
    bool b = false;
    for (uint32_t j = lane; j < C; j += 64) {
      const float ls = (xr[j] - mx) - l;
      if (int32_t(j) != y) b = b || !(fabsf(ls) <= FLT_MAX);
    }
    bad = __any(b);
  }
  if (lane == 0) {
    float t;
    if (bad) t = __builtin_nanf("");
    else if (y >= 0 && uint32_t(y) < C) t = 0.0f + ((xr[y] - mx) - l);
    else t = 0.0f;
    loss[row] = row < simd_end ? 0.0f - t : -t;
    stats[2 * row] = mx;
    stats[2 * row + 1] = l;
  }
}

// Backward, any alignment: the scalar kernel's chunk of a row is kBwdUnroll * 4 * kCeBlock
// elements.
constexpr int kBwdUnroll = PLAST_CE_BWD_UNROLL;

// Backward, float4 path over the flattened [N, C] gradient: one float4 per lane, its row found by
// magic division; the per-row constants are cached vector loads shared by the wave.
constexpr int kCeFlatBlock = PLAST_CE_BWD_BLOCK;

template <bool OVERWRITE>
__global__ __launch_bounds__(kCeFlatBlock) void ce_bwd_flat_kernel(const float *__restrict__ x,
                                                               const int32_t *__restrict__ lab,
                                                               const float *__restrict__ stats,
                                                               const float *__restrict__ dloss,
                                                               float *dx, MagicDiv dc4,
                                                               uint32_t units) {
  const uint32_t q = (PLAST_CE_BWD_XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x) * kCeFlatBlock + threadIdx.x;
  if (q >= units) return;
  const uint32_t row = dc4.div(q);
  const uint32_t j4 = q - row * dc4.d;
  const f4 xv = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(x) + q);
  f4 dv;
  if constexpr (!OVERWRITE) dv = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(dx) + q);
  const float m = stats[2 * uint64_t(row)], l = stats[2 * uint64_t(row) + 1], g = dloss[row];
  const int32_t y = lab[row];
  f4 r;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float sm = exp_le0((xv[c] - m) - l);
    const float oh = int32_t(j4 * 4 + c) == y ? 1.0f : 0.0f;
    const float gv = g * (sm - oh);
    if constexpr (OVERWRITE) r[c] = gv;
    else r[c] = dv[c] + gv;
  }
  store_stream<PLAST_CE_NT_STORE>(r, reinterpret_cast<f4 *>(dx) + q);
}

// Backward, any alignment: one element per lane per step.
template <bool OVERWRITE>
__global__ __launch_bounds__(kCeBlock) void ce_bwd_scalar_kernel(const float *__restrict__ x,
                                                                 const int32_t *__restrict__ lab,
                                                                 const float *__restrict__ stats,
                                                                 const float *__restrict__ dloss,
                                                                 float *dx, uint32_t C,
                                                                 uint32_t chunks) {
  const uint64_t row = blockIdx.x / chunks;
  const uint32_t chunk = blockIdx.x - uint32_t(row) * chunks;
  const float m = stats[2 * row], l = stats[2 * row + 1], g = dloss[row];
  const int32_t y = lab[row];
  const float *xr = x + row * C;
  float *dr = dx + row * C;
  const uint32_t j0 = chunk * (kCeBlock * kBwdUnroll * 4);
  const uint32_t j1 = j0 + kCeBlock * kBwdUnroll * 4 < C ? j0 + kCeBlock * kBwdUnroll * 4 : C;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kCeBlock) {
    const float sm = exp_le0((xr[j] - m) - l);
    const float oh = int32_t(j) == y ? 1.0f : 0.0f;
    const float gv = g * (sm - oh);
    dr[j] = OVERWRITE ? gv : dr[j] + gv;
  }
}

// ---- a whole cross-entropy training step in one pass: the forward's row statistics and loss,
// the backward's dx = dloss * (softmax - onehot), and the bias gradient sum_rows dx, reading each
// logit once and writing each gradient once. Persistent workgroups of kStepBlock lanes walk rows
// in pairs taken from a device counter (in deterministic mode, rows b, b + G, b + 2G, ...); a row
// is held in registers (V float4 per lane; lanes past the row are
// masked), and the next row's loads are issued into a second register set before the current row is
// reduced, so memory keeps streaming through the row's two block reductions. Per row, with the
// forward kernel's semantics (ce_fwd_wave_kernel): M = the block max, S = sum exp(x - M) in the
// block's fixed order, l = logf(S); rows whose fast values could differ from the reference chain's
// bits (a non-finite S or M, a zero M, an overflowing shifted-normalised logit) are recomputed
// exactly from memory. Each lane adds the dx of its columns into the workgroup's column sums in LDS
// (a slot per lane and unit; a lane only ever touches its own slots, so no synchronisation is
// needed) across the workgroup's rows; at the end the workgroup writes them to part[b][C], and
// ce_step_tail adds the G rows of part in workgroup order. No atomics: the bias gradient is fixed
// by which rows each workgroup took (the static schedule of deterministic mode fixes that too).
// Registers hold the two row sets only (the column sums there would spill at 1024 lanes per
// workgroup, whose wave count caps a lane at 128 VGPRs).
// A persistent row kernel's workgroup number b, which picks its rows and its partial-sum row:
// the dispatch index, or (PLAST_ROW_XCD) that index renumbered so that each XCD holds a
// contiguous range of b.
__device__ __forceinline__ uint32_t row_block() {
  if constexpr (PLAST_ROW_XCD) return xcd_block(blockIdx.x, gridDim.x);
  else return blockIdx.x;
}

// The rows a persistent row kernel's workgroup walks under the static schedule: r, r + S, ...
// below rend, that is rows b, b + G, ..., so the grid sweeps the tensor front to back.
__device__ __forceinline__ void row_range(uint32_t N, uint32_t G, uint32_t &r, uint32_t &S,
                                          uint32_t &rend) {
  r = row_block();
  rend = N;
  S = G;
}

// Dynamic row order for the persistent row kernels. Workgroups take pairs of rows (2P, 2P + 1) in
// increasing P from a device counter, so the rows in flight across the chip stay a compact band at
// the front of the tensor and a workgroup that runs faster (on MI355X the odd XCDs stream about 8%
// slower than the even ones under these loads) takes more rows; a static schedule of rows b, b + G,
// ... leaves the fast XCDs idle at the end and spreads the band. One counter pair per kernel
// family: [next pair, workgroups done]. The workgroup that finishes last returns both to zero for
// the next launch (every earlier ticket has returned by then), so no reset is launched and a
// captured graph replays it unchanged. Launches of one family overlapping on one device would
// share the counter: the library issues them on its one stream.
enum : int { kTicketStep = 0, kTicketSoftmax = 2 };
static __device__ unsigned int g_row_tickets[4];

// One ticket (a pair index), taken by lane 0 of wave 0; every other lane gets 0. The register is
// set to 0 before the branch and the atomic returns into it, so nothing reads the atomic's result
// where the branch rejoins: the wait for it falls where lane 0 first uses it. An increment
// (global_atomic_inc, bounded by 2^32 - 1, so it never wraps here) rather than an add: the
// compiler turns a uniform add into a wave-wide form whose result it reads, with a wait for every
// outstanding load, right after the branch.
__device__ __forceinline__ uint32_t take_ticket(int family) {
  uint32_t v = 0;
  if (threadIdx.x == 0) v = atomicInc(&g_row_tickets[family], 0xffffffffu);
  return v;
}

// The end of a workgroup's ticket walk: `last` is its final ticket (its value makes lane 0 wait
// for that atomic to return); the last workgroup out zeroes the family's counters.
__device__ __forceinline__ void tickets_done(int family, uint32_t last) {
  if (threadIdx.x != 0) return;
  asm volatile("" ::"v"(last));
  __threadfence();
  if (atomicAdd(&g_row_tickets[family + 1], 1u) == gridDim.x - 1) {
    __hip_atomic_store(&g_row_tickets[family], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&g_row_tickets[family + 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// A row unit of the persistent row kernels: nontemporal (NT) or ordinary load.
template <bool NT>
__device__ __forceinline__ f4 load_row_unit(const f4 *p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Keeps the row loads just issued where they are. Without it the compiler may move a prefetch of
// the next row down to where its values are first used (past the loop's back edge, behind the
// wait for the current row), which shortens the registers' live ranges but leaves nothing in
// flight while the current row is reduced. A compiler-only barrier: no instruction is emitted.
__device__ __forceinline__ void pin_loads() {
  asm volatile("" ::: "memory");
}

constexpr int kStepBlock = PLAST_CE_STEP_BLOCK;
// The widest row the LDS column sums allow: a float4 slot per lane and unit within 159 KiB of a
// CU's 160 (1024 lanes: 8 units, rows up to 32768 floats; 512 lanes: 16 units, 65536 floats).
constexpr int step_max_units() {
  int v = 16;
  while (v > 1 && size_t(kStepBlock) * size_t(v) * 16 > size_t(159) * 1024) v /= 2;
  return v;
}
constexpr int kStepMaxV = step_max_units();
constexpr uint64_t kStepMaxC = uint64_t(kStepBlock) * 4 * kStepMaxV;
static_assert(kScratchFloats / kStepMaxC >= 256, "the device array holds a CU-sized grid of the widest rows");

// Exact row statistics for the rare rows the fast path cannot take: the reference's serial max
// fold, then the exp-sum with expf and the "some other term is non-finite" flag of the one-hot
// product (the whole block takes this branch).
template <int W>
__device__ void ce_row_exact(const float *row, uint32_t C, int32_t y, float *lds, float &mx,
                             float &l, bool &bad) {
  constexpr int BS = W * 64;
  __syncthreads();
  if (threadIdx.x == 0) lds[W] = serial_max_fold(row, C);
  __syncthreads();
  mx = lds[W];
  float t = 0.0f;
  for (uint32_t j = threadIdx.x; j < C; j += BS) t += expf(row[j] - mx);
  l = logf(block_sum<W>(t, lds));
  bool b = false;
  for (uint32_t j = threadIdx.x; j < C; j += BS) {
    const float ls = (row[j] - mx) - l;
    if (int32_t(j) != y) b = b || !(fabsf(ls) <= FLT_MAX);
  }
  bad = block_any<W>(b, lds);
}

template <int V, bool DYN>
__global__ __launch_bounds__(kStepBlock) void ce_step_kernel(
    const float *__restrict__ x, const int32_t *__restrict__ lab, const float *__restrict__ dloss,
    float *__restrict__ stats, float *__restrict__ loss, float *__restrict__ dx,
    float *__restrict__ part, uint32_t N, uint32_t C, uint32_t simd_end) {
  constexpr int BS = kStepBlock, W = BS / 64;
  // one area per reduction of a row: a reduction's single barrier orders its writes after every
  // read of the same area in the previous row (which precede the other reduction's barrier)
  __shared__ float red1[2 * W], red2[W], ex[W + 2];
  __shared__ uint32_t tk;  // the next pair, from lane 0 of wave 0 (dynamic order)
  extern __shared__ f4 colsum[];  // BS * V float4: the workgroup's column sums, then padding
  const uint32_t C4 = C / 4, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // row indices are 32-bit (the host checks N < 2^32): a 64-bit bound compare would be made in
  // vector registers, which the loop head may find still tied to an in-flight memory operation
  const uint32_t G = gridDim.x;
  const float ninf = -__builtin_huge_valf(), pinf = __builtin_huge_valf();
#pragma unroll
  for (int u = 0; u < V; ++u) colsum[t + uint32_t(u) * BS] = f4(0.0f);

  // The lane index is made opaque in each row step, so the per-unit offsets and masks derived
  // from it are recomputed there (a few adds) instead of being hoisted out of the row loop, where
  // they would be spilled to scratch at this register budget.
  auto lane_index = [&]() {
    uint32_t i = t;
    asm volatile("" : "+v"(i));
    return i;
  };
  // Every load is issued unconditionally (a lane past the row reads the row's last float4, and the
  // prefetch past the last row re-reads that row): a load under a branch may not have been issued,
  // so the wait before the current row's first use could not count the prefetch as outstanding and
  // would wait for it too. Lanes past the row are masked where their values are used.
  // Addresses are a row base (uniform) plus a 32-bit byte offset per lane, which the loads and
  // stores take in one register (a 64-bit address per unit would take two).
  // The row's label and upstream gradient are loaded with it, a row ahead of their use (a load
  // issued when the row's processing starts would stall it for a memory round trip).
  auto load_row = [&](uint32_t r, f4 (&v)[V], int32_t &yl, float &gl) {
    const uint32_t rc = r < N ? r : N - 1;
    yl = lab[rc];
    gl = dloss[rc];
    const char *xr = reinterpret_cast<const char *>(x + uint64_t(rc) * C);
    const uint32_t ti = lane_index();
#pragma unroll
    for (int u = 0; u < V; ++u) {
      const uint32_t q = ti + uint32_t(u) * BS;
      const uint32_t off = (q < C4 ? q : C4 - 1) * 16u;
      v[u] = load_row_unit<PLAST_CE_STEP_NT_LOAD>(reinterpret_cast<const f4 *>(xr + off));
    }
    pin_loads();
  };

  // One row held in v: v is overwritten with e = exp(x - M) by the sum pass, so the gradient
  // pass is one multiply per element, dx = e * (dloss / S) (the softmax exp((x - m) - l) as
  // e / S, within 2 ulp of it), with the one-hot term applied to the label's element alone. A
  // row's VALU work is then about 14 instructions per element, under the memory time (the
  // recomputed-exponential form took 36 and was issue-bound).
  // With `next`, lane 0 of wave 0 publishes `give` (a ticket) before the row's first barrier and
  // every lane reads it into *next after it.
  auto process = [&](uint32_t r, f4 (&v)[V], const int32_t y, const float g, uint32_t give,
                     uint32_t *next) {
    // Consume every unit of the row here, on every path: a unit used only under a branch that some
    // waves skip (the row's ragged last unit) would leave its load pending past the loop's back
    // edge, and reusing its registers there would wait for every load, the prefetch included.
#pragma unroll
    for (int u = 0; u < V; ++u) asm volatile("" ::"v"(v[u][0]), "v"(v[u][1]), "v"(v[u][2]), "v"(v[u][3]));
    if (next && t == 0) tk = give;
    const uint32_t ti = lane_index();
    const uint32_t full = C4 / BS;  // units every lane holds inside the row
    // first reduction: the row's max and min (lanes past the row hold a copy of its last float4, which
    // changes neither)
    float m = ninf, mn = pinf;
#pragma unroll
    for (int u = 0; u < V; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        m = fmaxf(m, v[u][c]);
        mn = fminf(mn, v[u][c]);
      }
    m = wave_max(m);
    mn = wave_min(mn);
    if (lane == 0) {
      red1[wave] = m;
      red1[W + wave] = mn;
    }
    // the label's logit, taken by the lane that holds it before the sum pass overwrites v
    const bool live = y >= 0 && uint32_t(y) < C;
    const uint32_t yq = live ? uint32_t(y) >> 2 : 0;
    const bool owner = ti == yq % BS;
    float xy = 0.0f;
    if (owner) {
#pragma unroll
      for (int u = 0; u < V; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (uint32_t(u) == yq / BS && c == int(y & 3)) xy = v[u][c];
    }
    __syncthreads();
    if (next) *next = tk;
    float M = red1[0], MN = red1[W];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      M = fmaxf(M, red1[w]);
      MN = fminf(MN, red1[W + w]);
    }
    // second reduction: e = exp(x - M) into v, and its sum. A NaN logit reaches the sum; an infinite one,
    // or an x - M that overflows, sends the row to the exact path below, so every value used from
    // here on came from a finite argument and the unclamped exponential is exact enough.
    float sl = 0.0f;
#pragma unroll
    for (int u = 0; u < V; ++u) {
      const bool in = uint32_t(u) < full || ti + uint32_t(u) * BS < C4;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float e = exp_le0_finite(v[u][c] - M);
        v[u][c] = e;
        sl += in ? e : 0.0f;
      }
    }
    sl = wave_sum(sl);
    if (lane == 0) red2[wave] = sl;
    __syncthreads();
    float S = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) S += red2[w];
    float mx = M, l = 0.0f;
    bool exact = !(fabsf(M) <= FLT_MAX) || M == 0.0f || !(S <= FLT_MAX);
    if (!exact) {
      l = logf(S);
      // the most negative shifted-normalised logit must stay finite (else 0 * -inf = NaN)
      exact = !(fabsf((MN - mx) - l) <= FLT_MAX);
    }
    bool bad = false;
    if (exact) ce_row_exact<W>(x + uint64_t(r) * C, C, y, ex, mx, l, bad);
    // the lane holding the label's logit writes the loss and the statistics
    if (owner) {
      float tt = 0.0f;
      if (bad) tt = __builtin_nanf("");
      else if (live) tt = 0.0f + ((xy - mx) - l);
      loss[r] = r < simd_end ? 0.0f - tt : -tt;
      stats[2 * uint64_t(r)] = mx;
      stats[2 * uint64_t(r) + 1] = l;
    }
    // the gradient, written once and added into the lane's column sums
    f4 *d4 = reinterpret_cast<f4 *>(dx + uint64_t(r) * C);
    char *dr = reinterpret_cast<char *>(d4);
    if (!exact) {
      const float gs = g * (1.0f / S);
      const float inv = 1.0f / S;
      // each unit's gradient stored as soon as it is formed (the stores go out first), then the
      // column sums, whose LDS reads and writes then run back to back without a branch between
      // them (+1.4% over adding each unit before its store, in one process)
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const uint32_t q = ti + uint32_t(u) * BS;
        f4 o = v[u] * gs;
        if (owner && uint32_t(u) == yq / BS && live) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (c == int(y & 3)) o[c] = g * (v[u][c] * inv - 1.0f);
        }
        if (uint32_t(u) < full || q < C4)
          store_stream<PLAST_CE_NT_STORE>(o, reinterpret_cast<f4 *>(dr + q * 16u));
        v[u] = o;
      }
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const uint32_t q = ti + uint32_t(u) * BS;
        colsum[q] = colsum[q] + v[u];  // lanes past the row add into padding slots
      }
    } else {
      // the exact statistics: the gradient from memory, as the backward op computes it
      const f4 *x4 = reinterpret_cast<const f4 *>(x + uint64_t(r) * C);
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const uint32_t q = ti + uint32_t(u) * BS;
        if (q >= C4) continue;
        const f4 xv = x4[q];
        f4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float sm = exp_le0((xv[c] - mx) - l);
          const float oh = int32_t(q * 4 + c) == y ? 1.0f : 0.0f;
          o[c] = g * (sm - oh);
        }
        colsum[q] = colsum[q] + o;
        store_stream<PLAST_CE_NT_STORE>(o, d4 + q);
      }
    }
  };

  // Two register sets used in turn (a copy out of a set whose loads are in flight would wait for
  // them), each reloaded right after its row is processed, so one row is always in flight and the
  // youngest memory operations at the loop's back edge are loads: the loop head may reuse a
  // register a store of the previous row still reads, and that wait then leaves the prefetch alone
  // (with the stores last, it would wait for every load too). Rows go in pairs, an odd last row
  // after the loop: an exit between the pair's two rows would join the loop's back edge, and the
  // waits at the loop head would then have to assume the first set's loads were the latest issued
  // (waiting for the second set's prefetch too).
  f4 xa[V], xb[V];
  int32_t ya, yb;
  float ga, gb;
  if constexpr (DYN) {
    // pairs of rows (2P, 2P + 1) from the ticket counter; the ticket for the pair after next is
    // taken right before the first set's reload, so the wait for that reload covers it
    if (t == 0) tk = take_ticket(kTicketStep);
    __syncthreads();
    uint32_t P = tk, Pn = 0;
    uint32_t ahead = take_ticket(kTicketStep);
    load_row(2 * P, xa, ya, ga);
    load_row(2 * P + 1, xb, yb, gb);
    while (2 * P + 1 < N) {
      process(2 * P, xa, ya, ga, ahead, &Pn);
      ahead = take_ticket(kTicketStep);
      load_row(2 * Pn, xa, ya, ga);
      process(2 * P + 1, xb, yb, gb, 0, nullptr);
      load_row(2 * Pn + 1, xb, yb, gb);
      P = Pn;
    }
    if (2 * P < N) process(2 * P, xa, ya, ga, 0, nullptr);
    tickets_done(kTicketStep, ahead);
  } else {
    uint32_t r, S, rend;
    row_range(N, G, r, S, rend);
    load_row(r, xa, ya, ga);
    load_row(r + S, xb, yb, gb);
    for (; r + S < rend; r += 2 * S) {
      process(r, xa, ya, ga, 0, nullptr);
      load_row(r + 2 * S, xa, ya, ga);
      process(r + S, xb, yb, gb, 0, nullptr);
      load_row(r + 3 * S, xb, yb, gb);
    }
    if (r < rend) process(r, xa, ya, ga, 0, nullptr);
  }
  // the workgroup's column sums: partial row b of part, in dispatch order under the dynamic
  // order (the rows each workgroup took vary from run to run) and by the static schedule's
  // numbering otherwise
  f4 *p4 = reinterpret_cast<f4 *>(part + uint64_t(DYN ? blockIdx.x : row_block()) * C);
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t q = t + uint32_t(u) * BS;
    if (q < C4) p4[q] = colsum[q];
  }
}

// The step's tail, one launch after the row kernel: with `mean`, workgroup 0 writes the mean of
// the rows' losses; the next `nfin` workgroups (with `dbias`) sum the row kernel's column sums.
//
// dbias[c] = the sum over workgroups b = 0 .. G-1 of part[b][c], deterministically: a workgroup
// takes 32 columns; its lane group q (of 8) sums the q-th eighth of the b range in order (32 lanes
// read 32 adjacent columns, 128 B, per row), then lane c adds the 8 group sums in q order.
//
// The mean is the reference chain's last node: MEAN over the rows' losses (loss.c:161-163; the
// full reduction of reduce_ops.c:24-31 with POST_MEAN, acc / n). Its order is that of 1024 virtual
// lanes: virtual lane L sums rows L, L + 1024, ... in order, each virtual wave of 64 lanes combines
// its sums in a butterfly, and the 16 wave sums are added in wave order; a sum that overflowed
// (finite terms, not a NaN) is summed again serially in row order, as the reference's order
// decides it. Then divided by N (N = 0: 0 / 0, NaN, as the reference's mean of nothing). Lane p of
// the 256 holds virtual lanes p + 256k (k < 4), which fall in virtual wave p / 64 + 4k at the same
// position, so its four butterflies are those of the virtual waves; each lane keeps 32 loads in
// flight (8 rows of 1024 at a time), as many as four rounds over config 5's 32768 rows.
constexpr int kFinCols = 32, kFinGroups = kCeBlock / kFinCols;
// partial rows (column sums) and rows of 1024 losses (mean) loaded at a time; 16 or 32 and 16
// measured no faster (the launch's duration is not its loads' latency)
constexpr uint32_t kFinBatch = 8, kMeanRounds = 8;
constexpr uint32_t kMeanVirt = 1024, kMeanHold = kMeanVirt / kCeBlock;
static_assert(kMeanVirt % kCeBlock == 0, "the mean's virtual lanes split evenly over the workgroup");
__global__ __launch_bounds__(kCeBlock) void ce_step_tail(const float *__restrict__ part,
                                                         float *__restrict__ dbias, uint32_t C,
                                                         uint32_t G, const float *__restrict__ loss,
                                                         float *__restrict__ mean, uint32_t N) {
  __shared__ float sh[kFinGroups][kFinCols];
  const uint32_t t = threadIdx.x;
  if (mean && blockIdx.x == 0) {
    const uint32_t lane = t & 63, wave = t >> 6;
    float s[kMeanHold] = {};
    for (uint32_t i0 = t; i0 < N; i0 += kMeanVirt * kMeanRounds) {
      float v[kMeanRounds][kMeanHold];
#pragma unroll
      for (uint32_t m = 0; m < kMeanRounds; ++m)
#pragma unroll
        for (uint32_t k = 0; k < kMeanHold; ++k) {
          const uint32_t i = i0 + m * kMeanVirt + k * kCeBlock;
          v[m][k] = loss[i < N ? i : N - 1];
        }
#pragma unroll
      for (uint32_t m = 0; m < kMeanRounds; ++m)
#pragma unroll
        for (uint32_t k = 0; k < kMeanHold; ++k)
          if (i0 + m * kMeanVirt + k * kCeBlock < N) s[k] += v[m][k];
    }
    float *ws = &sh[0][0];  // the virtual waves' sums, in virtual wave order
#pragma unroll
    for (uint32_t k = 0; k < kMeanHold; ++k) {
      const float w = wave_sum(s[k]);
      if (lane == 0) ws[wave + k * (kCeBlock / 64)] = w;
    }
    __syncthreads();
    if (t != 0) return;
    float p = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < kMeanVirt / 64; ++w) p += ws[w];
    if (!(fabsf(p) <= FLT_MAX) && p == p) {
      p = 0.0f;
      for (uint32_t i = 0; i < N; ++i) p = p + loss[i];
    }
    mean[0] = p / float(N);
    return;
  }
  const uint32_t cl = t % kFinCols, q = t / kFinCols;
  const uint32_t c = (blockIdx.x - (mean ? 1u : 0u)) * kFinCols + cl;
  const uint32_t per = (G + kFinGroups - 1) / kFinGroups;
  const uint32_t b0 = q * per, b1 = b0 + per < G ? b0 + per : G;
  float s = 0.0f;
  if (c < C) {
    for (uint32_t b = b0; b < b1; b += kFinBatch) {
      float v[kFinBatch];
#pragma unroll
      for (uint32_t k = 0; k < kFinBatch; ++k)
        v[k] = b + k < b1 ? part[uint64_t(b + k) * C + c] : 0.0f;
#pragma unroll
      for (uint32_t k = 0; k < kFinBatch; ++k)
        if (b + k < b1) s += v[k];
    }
  }
  sh[q][cl] = s;
  __syncthreads();
  if (q != 0 || c >= C) return;
  float u = sh[0][cl];
#pragma unroll
  for (int g = 1; g < kFinGroups; ++g) u += sh[g][cl];
  dbias[c] = u;
}

// Whether ce_step_kernel<V> may be launched with its dynamic LDS (raising its limit once: beyond
// the default the kernel has to opt in).
template <int V>
bool ce_step_lds_ok() {
  static bool granted = false;
  if (granted) return true;
  const int bytes = kStepBlock * V * int(sizeof(f4));
  for (const void *k : {reinterpret_cast<const void *>(&ce_step_kernel<V, true>),
                        reinterpret_cast<const void *>(&ce_step_kernel<V, false>)})
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
      (void)hipGetLastError();  // not an error of the call: the caller takes the three passes
      return false;
    }
  granted = true;
  return true;
}

// The float4 units per lane for rows of C floats from V up (0: none of this build's kernels).
template <int V>
int ce_step_units(uint64_t C) {
  if constexpr (V > kStepMaxV) {
    return 0;
  } else {
    if (C <= uint64_t(kStepBlock) * 4 * V) return ce_step_lds_ok<V>() ? V : 0;
    return ce_step_units<V * 2>(C);
  }
}

// The one-pass step with V units per lane over `grid` workgroups, their column sums in
// part[grid][C].
template <int V>
void ce_step_launch_v(int want, unsigned grid, float *part, const float *logits,
                      const int32_t *labels, const float *dloss, float *stats, float *loss,
                      float *dlogits, uint32_t N, uint32_t C) {
  if constexpr (V <= kStepMaxV) {
    if (want != V) {
      ce_step_launch_v<V * 2>(want, grid, part, logits, labels, dloss, stats, loss, dlogits, N, C);
      return;
    }
    const size_t lds = size_t(kStepBlock) * V * sizeof(f4);
    // the dynamic row order unless results must not depend on timing (plast_hip_set_deterministic)
    if (deterministic())
      ce_step_kernel<V, false><<<grid, kStepBlock, lds, stream()>>>(
          logits, labels, dloss, stats, loss, dlogits, part, N, C, uint32_t(simd_end(N)));
    else
      ce_step_kernel<V, true><<<grid, kStepBlock, lds, stream()>>>(
          logits, labels, dloss, stats, loss, dlogits, part, N, C, uint32_t(simd_end(N)));
  }
}

// The one-pass step's arguments: -1 (after reporting) when unusable, 0 when the rows need the three
// passes, else the float4 units per lane of the register-resident row (its LDS opt-in granted).
int ce_step_form(const float *logits, const int32_t *labels, const float *dloss, const float *stats,
                 const float *loss, const float *dlogits, uint64_t N, uint64_t C,
                 const char *where) {
  if (!logits || !labels || !dloss || !stats || !loss || !dlogits) {
    report_error(where, "logits, labels, dloss, stats, loss and dlogits are required");
    return -1;
  }
  if (C == 0 || C >= (uint64_t(1) << 31)) {
    report_error(where, "rows of %llu elements are not supported", (unsigned long long)C);
    return -1;
  }
  if (N >= (uint64_t(1) << 31)) {
    report_error(where, "more than 2^31 rows are not supported (%llu)", (unsigned long long)N);
    return -1;
  }
  // the column sums live in LDS (one float4 slot per lane and unit, the row's plus padding): the
  // kernel must be allowed that much of it
  if (C % 4 == 0 && C <= kStepMaxC && aligned16(logits) && aligned16(dlogits))
    return ce_step_units<1>(C);
  return 0;
}

// The one-pass step's workgroup count, shared by the allocating and the allocation-free entry
// points so that both sum the bias gradient in the same order: one workgroup per row up to
// PLAST_CE_STEP_WPC per CU, and no more than the allocation-free step's device array holds column
// sums for (kScratchFloats / C; on MI355X, 256 CUs of rows up to 32768 floats, never binding).
uint64_t ce_step_grid(uint64_t N, uint64_t C) {
  uint64_t grid = uint64_t(num_cus()) * PLAST_CE_STEP_WPC;
  if (grid > kScratchFloats / C) grid = kScratchFloats / C;
  return N < grid ? N : grid;
}

// The one-pass step over `grid` workgroups with their column sums in part[grid][C], then the tail:
// their sum into dbias and the loss's mean, as wanted.
// The step's tail: dbias from the column sums part[G][C] when dbias is wanted, and the mean of
// loss[0 .. N) when mean_loss is; one launch, or none when neither is wanted.
void step_tail(const float *part, float *dbias, uint64_t C, unsigned G, const float *loss,
               float *mean_loss, uint64_t N) {
  const uint64_t nfin = dbias ? ceil_div(C, kFinCols) : 0;
  const uint64_t blocks = nfin + (mean_loss ? 1 : 0);
  if (blocks)
    ce_step_tail<<<unsigned(blocks), kCeBlock, 0, stream()>>>(part, dbias, uint32_t(C), G, loss,
                                                             mean_loss, uint32_t(N));
}

void ce_step_launch(int V, unsigned grid, float *part, const float *logits, const int32_t *labels,
                    const float *dloss, float *stats, float *loss, float *dlogits, float *dbias,
                    float *mean_loss, uint64_t N, uint64_t C) {
  const uint32_t c32 = uint32_t(C);
  ce_step_launch_v<1>(V, grid, part, logits, labels, dloss, stats, loss, dlogits, uint32_t(N), c32);
  step_tail(part, dbias, C, grid, loss, mean_loss, N);
}

bool check_ce(const Tensor *x, const Tensor *lab, const Tensor *st, const char *where) {
  if (x->dtype != FLOAT32 || x->ndim != 2 || !contiguous(x)) {
    report_error(where, "logits must be a contiguous fp32 [N, C] tensor");
    return false;
  }
  if (lab->dtype != INT32 || numel(lab) != x->shape[0] || !contiguous(lab)) {
    report_error(where, "labels must be a contiguous int32 tensor of N elements");
    return false;
  }
  if (st->dtype != FLOAT32 || numel(st) != 2 * x->shape[0] || !contiguous(st)) {
    report_error(where, "stats must be a contiguous fp32 tensor of 2N elements");
    return false;
  }
  if (x->shape[1] >= (uint64_t(1) << 31)) {
    report_error(where, "rows longer than 2^31 elements are not supported");
    return false;
  }
  return true;
}

// ---- softmax and log-softmax over the last axis. The reference composes them in Python
// (plast/nn/functional.py:75-97): MAX(dim, keepdim) -> SUB -> EXP -> SUM(dim, keepdim) -> DIV for
// softmax, -> LOG -> SUB for log-softmax. One workgroup per row: the reference's max (bit-exact),
// s = sum_j expf(x_j - m) in the block's fixed order (the reference sums serially), then
// y = expf(x - m) / s or (x - m) - logf(s): every other step is the reference's own operation.
template <bool LOG>
__global__ __launch_bounds__(kCeBlock) void softmax_fwd_kernel(const float *__restrict__ x,
                                                               float *__restrict__ y, uint32_t C) {
  __shared__ float lds[kCeWaves + 1];
  const uint64_t row = blockIdx.x;
  const float *xr = x + row * C;
  float *yr = y + row * C;
  float m = -__builtin_huge_valf();
  bool nan = false;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) {
    const float v = xr[j];
    m = fmaxf(m, v);
    nan = nan || v != v;
  }
  const float mx = row_max_exact(m, nan, xr, C, lds);
  float s = 0.0f;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) s += expf(xr[j] - mx);
  s = block_sum(s, lds);
  if constexpr (LOG) {
    const float l = logf(s);
    for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) yr[j] = (xr[j] - mx) - l;
  } else {
    for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) yr[j] = expf(xr[j] - mx) / s;
  }
}

constexpr int kSoftmaxBlock = PLAST_SOFTMAX_BLOCK;

// The same with the row held in registers, for rows of up to BS * 4 * V floats in whole
// float4 (C % 4 == 0, 16-byte aligned rows): one read and one write per element. Each lane keeps V
// float4 of the row; lanes past the row hold -inf, which adds exp(-inf) = 0 to no sum (they are
// masked) and never wins the max. Same operations and order as softmax_fwd_kernel's three passes
// but the exp-sum's grouping (per lane, then the block's fixed tree).
template <bool LOG, int V, int BS = kSoftmaxBlock>
__global__ __launch_bounds__(BS) void softmax_fwd_reg_kernel(const float *__restrict__ x,
                                                             float *__restrict__ y, uint32_t C) {
  constexpr int W = BS / 64;
  __shared__ float lds[W + 1];
  const uint64_t row = blockIdx.x;
  const float *xr = x + row * C;
  const uint32_t C4 = C / 4;
  const f4 *x4 = reinterpret_cast<const f4 *>(xr);
  f4 *y4 = reinterpret_cast<f4 *>(y + row * C);
  const float ninf = -__builtin_huge_valf();
  f4 v[V];
  float m = ninf;
  bool nan = false;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t q = threadIdx.x + uint32_t(u) * BS;
    v[u] = q < C4 ? __builtin_nontemporal_load(x4 + q) : f4(ninf);
  }
#pragma unroll
  for (int u = 0; u < V; ++u) {
    m = fmaxf(m, fmaxf(fmaxf(v[u][0], v[u][1]), fmaxf(v[u][2], v[u][3])));
    nan = nan || v[u][0] != v[u][0] || v[u][1] != v[u][1] || v[u][2] != v[u][2] ||
          v[u][3] != v[u][3];
  }
  const float mx = row_max_exact<W>(m, nan, xr, C, lds);
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const bool in = threadIdx.x + uint32_t(u) * BS < C4;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float t = v[u][c] - mx;
      const float e = expf(t);
      v[u][c] = LOG ? t : e;
      s += in ? e : 0.0f;
    }
  }
  s = block_sum<W>(s, lds);
  const float l = LOG ? logf(s) : 0.0f;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t q = threadIdx.x + uint32_t(u) * BS;
    if (q >= C4) continue;
    f4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = LOG ? v[u][c] - l : v[u][c] / s;
    y4[q] = r;
  }
}

// Softmax / log-softmax forward over rows of whole float4 (up to kStepBlock * 4 * V floats) by
// persistent kStepBlock-lane workgroups, one per CU, walking rows G apart with the next row's loads
// in flight while the current one is reduced: the row loop of ce_step_kernel (two register sets,
// unconditional clamped loads, every loaded value consumed on every path). Per row: the reference's
// max (row_max_exact's rules: the fast maximum unless the row holds a NaN or its maximum is zero,
// then the serial fold), then e = exp(x - max) and its sum in the block's fixed order, then
// y = e * (1 / S) or (x - max) - log S. Without a NaN every x - max is <= 0 or -inf, where exp_le0
// holds (about 1 ulp); a row with a NaN, whose fold may stop below some elements, takes expf and a
// division.
template <bool LOG, int V, bool DYN>
__global__ __launch_bounds__(kStepBlock) void softmax_fwd_step_kernel(const float *__restrict__ x,
                                                                      float *__restrict__ y,
                                                                      uint32_t N, uint32_t C) {
  constexpr int BS = kStepBlock, W = BS / 64;
  // one area per reduction of a row (see ce_step_kernel)
  __shared__ float red1[2 * W], red2[W], ex[2];
  __shared__ uint32_t tk;  // the next pair, from lane 0 of wave 0 (dynamic order)
  const uint32_t C4 = C / 4, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t G = gridDim.x;
  const float ninf = -__builtin_huge_valf();
  auto lane_index = [&]() {
    uint32_t i = t;
    asm volatile("" : "+v"(i));
    return i;
  };
  auto load_row = [&](uint32_t r, f4 (&v)[V]) {
    const char *xr = reinterpret_cast<const char *>(x + uint64_t(r < N ? r : N - 1) * C);
    const uint32_t ti = lane_index();
#pragma unroll
    for (int u = 0; u < V; ++u) {
      const uint32_t q = ti + uint32_t(u) * BS;
      const uint32_t off = (q < C4 ? q : C4 - 1) * 16u;
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(xr + off));
    }
    pin_loads();
  };
  // process(r, v, give, next): with `next`, lane 0 of wave 0 publishes `give` (a ticket) before the
  // row's first barrier and every lane reads it into *next after it
  auto process = [&](uint32_t r, f4 (&v)[V], uint32_t give, uint32_t *next) {
#pragma unroll
    for (int u = 0; u < V; ++u) asm volatile("" ::"v"(v[u][0]), "v"(v[u][1]), "v"(v[u][2]), "v"(v[u][3]));
    if (next && t == 0) tk = give;
    const uint32_t ti = lane_index();
    const uint32_t full = C4 / BS;
    // first reduction: the fast maximum and whether the row holds a NaN (lanes past the row hold a copy of
    // its last float4, which changes neither)
    float m = ninf;
    bool nan = false;
#pragma unroll
    for (int u = 0; u < V; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        m = fmaxf(m, v[u][c]);
        nan = nan || v[u][c] != v[u][c];
      }
    m = wave_max(m);
    const float nanw = wave_max(nan ? 1.0f : 0.0f);
    if (lane == 0) {
      red1[wave] = m;
      red1[W + wave] = nanw;
    }
    __syncthreads();
    if (next) *next = tk;
    float M = red1[0], anynan = red1[W];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      M = fmaxf(M, red1[w]);
      anynan = fmaxf(anynan, red1[W + w]);
    }
    const bool special = anynan != 0.0f;
    float mx;
    if (special || M == 0.0f) {
      if (t == 0) ex[0] = serial_max_fold(x + uint64_t(r) * C, C);
      __syncthreads();
      mx = ex[0];
    } else {
      mx = M > -FLT_MAX ? M : -FLT_MAX;
    }
    // second reduction: e = exp(x - mx), kept in v (log-softmax keeps x - mx), and the row's sum. A row with
    // a NaN is summed from memory with expf instead (rare; it keeps the registers of the fast
    // path free), each lane over the same elements in the same order as the fast path.
    const f4 *x4 = reinterpret_cast<const f4 *>(x + uint64_t(r) * C);
    float sl = 0.0f;
    if (!special) {
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const bool in = uint32_t(u) < full || ti + uint32_t(u) * BS < C4;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float d = v[u][c] - mx;
          const float e = exp_le0(d);
          v[u][c] = LOG ? d : e;
          sl += in ? e : 0.0f;
        }
      }
    } else {
      for (uint32_t q = ti; q < C4; q += BS) {
        const f4 xv = x4[q];
#pragma unroll
        for (int c = 0; c < 4; ++c) sl += expf(xv[c] - mx);
      }
    }
    sl = wave_sum(sl);
    if (lane == 0) red2[wave] = sl;
    __syncthreads();
    float S = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) S += red2[w];
    f4 *y4 = reinterpret_cast<f4 *>(y + uint64_t(r) * C);
    char *dr = reinterpret_cast<char *>(y4);
    const float l = LOG ? logf(S) : 0.0f;
    if (!special) {
      const float inv = 1.0f / S;
#pragma unroll
      for (int u = 0; u < V; ++u) {
        const uint32_t q = ti + uint32_t(u) * BS;
        f4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = LOG ? v[u][c] - l : v[u][c] * inv;
        if (uint32_t(u) < full || q < C4)
          store_stream<true>(o, reinterpret_cast<f4 *>(dr + q * 16u));
      }
    } else {
      for (uint32_t q = ti; q < C4; q += BS) {
        const f4 xv = x4[q];
        f4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float d = xv[c] - mx;
          o[c] = LOG ? d - l : expf(d) / S;
        }
        y4[q] = o;
      }
    }
  };
  f4 xa[V], xb[V];
  if constexpr (DYN) {
    // pairs of rows (2P, 2P + 1) from the ticket counter; the ticket for the pair after next is
    // taken right before the first set's reload, so the wait for that reload covers it
    if (t == 0) tk = take_ticket(kTicketSoftmax);
    __syncthreads();
    uint32_t P = tk, Pn = 0;
    uint32_t ahead = take_ticket(kTicketSoftmax);
    load_row(2 * P, xa);
    load_row(2 * P + 1, xb);
    while (2 * P + 1 < N) {
      process(2 * P, xa, ahead, &Pn);
      ahead = take_ticket(kTicketSoftmax);
      load_row(2 * Pn, xa);
      process(2 * P + 1, xb, 0, nullptr);
      load_row(2 * Pn + 1, xb);
      P = Pn;
    }
    if (2 * P < N) process(2 * P, xa, 0, nullptr);
    tickets_done(kTicketSoftmax, ahead);
  } else {
    uint32_t r, S, rend;
    row_range(N, G, r, S, rend);
    load_row(r, xa);
    load_row(r + S, xb);
    // rows in pairs, an odd last row after the loop (see ce_step_kernel)
    for (; r + S < rend; r += 2 * S) {
      process(r, xa, 0, nullptr);
      load_row(r + 2 * S, xa);
      process(r + S, xb, 0, nullptr);
      load_row(r + 3 * S, xb);
    }
    if (r < rend) process(r, xa, 0, nullptr);
  }
}

// Backward from the forward output y: dx += y * (dy - sum_j dy_j y_j) (softmax) or
// dx += dy - expf(y) * sum_j dy_j (log-softmax), the gradient of the reference chain (its MAX
// branch contributes zero in exact arithmetic); the row sum in the block's fixed order.
template <bool LOG>
__global__ __launch_bounds__(kCeBlock) void softmax_bwd_kernel(const float *__restrict__ y,
                                                               const float *__restrict__ dy,
                                                               float *dx, uint32_t C) {
  __shared__ float lds[kCeWaves + 1];
  const uint64_t row = blockIdx.x;
  const float *yr = y + row * C, *gr = dy + row * C;
  float *dr = dx + row * C;
  float t = 0.0f;
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) t += LOG ? gr[j] : gr[j] * yr[j];
  t = block_sum(t, lds);
  for (uint32_t j = threadIdx.x; j < C; j += kCeBlock) {
    const float g = LOG ? gr[j] - expf(yr[j]) * t : yr[j] * (gr[j] - t);
    dr[j] = dr[j] + g;
  }
}

// The backward with y and dy of a row held in registers (rows of whole float4 up to BS * 4 * V
// floats): y, dy and dx are each read once and dx written once. The sum's grouping is per lane,
// then the block's fixed tree.
template <bool LOG, int V, int BS>
__global__ __launch_bounds__(BS) void softmax_bwd_reg_kernel(const float *__restrict__ y,
                                                             const float *__restrict__ dy,
                                                             float *dx, uint32_t C) {
  constexpr int W = BS / 64;
  __shared__ float lds[W + 1];
  const uint64_t row = blockIdx.x;
  const uint32_t C4 = C / 4;
  const f4 *y4 = reinterpret_cast<const f4 *>(y + row * C);
  const f4 *g4 = reinterpret_cast<const f4 *>(dy + row * C);
  f4 *d4 = reinterpret_cast<f4 *>(dx + row * C);
  // Loads are unconditional (a lane past the row reads the row's last float4, masked where it is
  // used): the compiler waits for every outstanding load before the first use of a lane-masked
  // one.
  // the first kPre units of dx (all of them by default) are loaded with y and dy, so that their
  // latency overlaps the row's reduction
  constexpr int kPre = PLAST_SOFTMAX_BWD_PRE < V ? PLAST_SOFTMAX_BWD_PRE : V;
  f4 yv[V], gv[V], dv[kPre > 0 ? kPre : 1];
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t q = threadIdx.x + uint32_t(u) * BS;
    const uint32_t qc = q < C4 ? q : C4 - 1;
    yv[u] = __builtin_nontemporal_load(y4 + qc);
    gv[u] = __builtin_nontemporal_load(g4 + qc);
    if (u < kPre) dv[u] = PLAST_SOFTMAX_BWD_NT ? __builtin_nontemporal_load(d4 + qc) : d4[qc];
  }
  float t = 0.0f;
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const bool in = threadIdx.x + uint32_t(u) * BS < C4;
#pragma unroll
    for (int c = 0; c < 4; ++c) t += in ? (LOG ? gv[u][c] : gv[u][c] * yv[u][c]) : 0.0f;
  }
  t = block_sum<W>(t, lds);
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t q = threadIdx.x + uint32_t(u) * BS;
    if (q >= C4) continue;
    f4 d;
    if (u < kPre) d = dv[u < kPre ? u : 0];
    else d = PLAST_SOFTMAX_BWD_NT ? __builtin_nontemporal_load(d4 + q) : d4[q];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      d[c] = d[c] + (LOG ? gv[u][c] - expf(yv[u][c]) * t : yv[u][c] * (gv[u][c] - t));
    store_stream<PLAST_SOFTMAX_BWD_NT>(d, d4 + q);
  }
}

bool check_softmax(const Tensor *x, const Tensor *y, KernelParams p, const char *where) {
  if (x->dtype != FLOAT32 || x->ndim < 1 || !contiguous(x)) {
    report_error(where, "input must be a contiguous fp32 tensor");
    return false;
  }
  if (y->dtype != FLOAT32 || !contiguous(y) || y->ndim != x->ndim || numel(y) != numel(x)) {
    report_error(where, "output must be a contiguous fp32 tensor shaped like the input");
    return false;
  }
  if (p.dim != x->ndim - 1) {
    report_error(where, "only the last axis (dim %llu) is supported, got dim %llu",
                 (unsigned long long)(x->ndim - 1), (unsigned long long)p.dim);
    return false;
  }
  if (x->shape[x->ndim - 1] >= (uint64_t(1) << 31)) {
    report_error(where, "rows longer than 2^31 elements are not supported");
    return false;
  }
  return true;
}

template <bool LOG>
void softmax_forward(const Tensor **inputs, Tensor *output, KernelParams params,
                     const char *where) {
  if (!ensure_init()) return;
  const Tensor *x = inputs[0];
  if (!check_softmax(x, output, params, where)) return;
  const uint32_t C = uint32_t(x->shape[x->ndim - 1]);
  const uint64_t N = C ? numel(x) / C : 0;
  const uint64_t R = max_blocks(kCeBlock);
  // float4 units per lane for a register-resident row (0: the three-pass kernel)
  int V = 0;
  if (C % 4 == 0 && aligned16(x->data) && aligned16(output->data))
    for (int v = 1; v <= 32 && !V; v *= 2)
      if (uint64_t(C) <= uint64_t(kSoftmaxBlock) * 4 * v) V = v;
  // rows of 2048..32768 floats: the persistent form (rows at a time below 2^31)
  int SV = 0;
  if (V && C >= 2048 && N < (uint64_t(1) << 31))
    for (int v = 1; v <= 8 && !SV; v *= 2)
      if (uint64_t(C) <= uint64_t(kStepBlock) * 4 * v) SV = v;
  if (SV) {
    const unsigned G = unsigned(N < uint64_t(num_cus()) ? N : uint64_t(num_cus()));
    const float *px = static_cast<const float *>(x->data);
    float *py = static_cast<float *>(output->data);
    const uint32_t n32 = uint32_t(N);
    constexpr bool D = PLAST_ROW_DYNAMIC;
    switch (SV) {
      case 1: softmax_fwd_step_kernel<LOG, 1, D><<<G, kStepBlock, 0, stream()>>>(px, py, n32, C); break;
      case 2: softmax_fwd_step_kernel<LOG, 2, D><<<G, kStepBlock, 0, stream()>>>(px, py, n32, C); break;
      case 4: softmax_fwd_step_kernel<LOG, 4, D><<<G, kStepBlock, 0, stream()>>>(px, py, n32, C); break;
      default: softmax_fwd_step_kernel<LOG, 8, D><<<G, kStepBlock, 0, stream()>>>(px, py, n32, C); break;
    }
    finish(where);
    return;
  }
  for (uint64_t r0 = 0; r0 < N; r0 += R) {
    const unsigned n = unsigned(N - r0 < R ? N - r0 : R);
    const float *px = static_cast<const float *>(x->data) + r0 * C;
    float *py = static_cast<float *>(output->data) + r0 * C;
    switch (V) {
      case 1: softmax_fwd_reg_kernel<LOG, 1><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      case 2: softmax_fwd_reg_kernel<LOG, 2><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      case 4: softmax_fwd_reg_kernel<LOG, 4><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      case 8: softmax_fwd_reg_kernel<LOG, 8><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      case 16: softmax_fwd_reg_kernel<LOG, 16><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      case 32: softmax_fwd_reg_kernel<LOG, 32><<<n, kSoftmaxBlock, 0, stream()>>>(px, py, C); break;
      default: softmax_fwd_kernel<LOG><<<n, kCeBlock, 0, stream()>>>(px, py, C); break;
    }
  }
  finish(where);
}

template <bool LOG>
void softmax_backward(Tensor **inputs, const Tensor *output, KernelParams params,
                      const char *where) {
  if (!ensure_init()) return;
  Tensor *x = inputs[0];
  if (!x->requires_grad || !x->grad) return;
  if (!check_softmax(x, output, params, where)) return;
  if (!output->grad || !contiguous(output->grad) || !contiguous(x->grad)) {
    report_error(where, "needs the output gradient and a contiguous input gradient");
    return;
  }
  const uint32_t C = uint32_t(x->shape[x->ndim - 1]);
  const uint64_t N = C ? numel(x) / C : 0;
  const uint64_t R = max_blocks(kCeBlock);
  constexpr int BS = PLAST_SOFTMAX_BWD_BLOCK;  // y and dy in registers: 512 lanes keep V at 16
                                              // for 32768-float rows
  int V = 0;
  if (C % 4 == 0 && aligned16(output->data) && aligned16(output->grad->data) &&
      aligned16(x->grad->data))
    for (int v = 1; v <= 16 && !V && v * BS <= 8192; v *= 2)
      if (uint64_t(C) <= uint64_t(BS) * 4 * v) V = v;
  for (uint64_t r0 = 0; r0 < N; r0 += R) {
    const unsigned n = unsigned(N - r0 < R ? N - r0 : R);
    const float *py = static_cast<const float *>(output->data) + r0 * C;
    const float *pg = static_cast<const float *>(output->grad->data) + r0 * C;
    float *pd = static_cast<float *>(x->grad->data) + r0 * C;
    switch (V) {
      case 1: softmax_bwd_reg_kernel<LOG, 1, BS><<<n, BS, 0, stream()>>>(py, pg, pd, C); break;
      case 2: softmax_bwd_reg_kernel<LOG, 2, BS><<<n, BS, 0, stream()>>>(py, pg, pd, C); break;
      case 4: softmax_bwd_reg_kernel<LOG, 4, BS><<<n, BS, 0, stream()>>>(py, pg, pd, C); break;
      case 8: softmax_bwd_reg_kernel<LOG, 8, BS><<<n, BS, 0, stream()>>>(py, pg, pd, C); break;
      case 16:
        if constexpr (16 * BS <= 8192)
          softmax_bwd_reg_kernel<LOG, 16, BS><<<n, BS, 0, stream()>>>(py, pg, pd, C);
        break;
      default: softmax_bwd_kernel<LOG><<<n, kCeBlock, 0, stream()>>>(py, pg, pd, C); break;
    }
  }
  finish(where);
}

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

void softmax_cross_entropy_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  (void)params;
  const char *where = "softmax_cross_entropy_hip_forward";
  if (!ensure_init()) return;
  const Tensor *x = inputs[0], *lab = inputs[1], *st = inputs[2];
  if (!check_ce(x, lab, st, where)) return;
  const uint64_t N = x->shape[0];
  const uint32_t C = uint32_t(x->shape[1]);
  if (output->dtype != FLOAT32 || numel(output) != N || !contiguous(output)) {
    report_error(where, "output must be a contiguous fp32 tensor of N elements");
    return;
  }
  if (N == 0) return;
  // The NEG node of the reference chain runs over the [N] (or [N,1]) loss tensor.
  const uint64_t se = simd_end(N);
  const bool vec = C % 4 == 0 && aligned16(static_cast<const float *>(x->data)) && C > 0;
  // rows per launch: one workgroup per row (generic) or one wave per row (vectorised)
  const uint64_t R = max_blocks(kCeBlock);
  for (uint64_t r0 = 0; r0 < N; r0 += R) {
    const uint64_t n = N - r0 < R ? N - r0 : R;
    const float *px = static_cast<const float *>(x->data) + r0 * C;
    const int32_t *pl = static_cast<const int32_t *>(lab->data) + r0;
    float *ps = static_cast<float *>(st->data) + 2 * r0;
    float *po = static_cast<float *>(output->data) + r0;
    const uint64_t ser = se > r0 ? se - r0 : 0;  // the rule's boundary, relative to this range
    if (vec)
      ce_fwd_wave_kernel<<<unsigned(ceil_div(n, kCeFwdWaves)), 64 * kCeFwdWaves, 0, stream()>>>(
          px, pl, ps, po, n, C, ser);
    else
      ce_fwd_generic_kernel<<<unsigned(n), kCeBlock, 0, stream()>>>(px, pl, ps, po, C, ser);
  }
  finish(where);
}

// params.keepdim == 1 writes the gradient instead of accumulating it, for callers that own a
// gradient buffer with no other contribution (saves one HBM read of [N, C]).
void softmax_cross_entropy_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  const char *where = "softmax_cross_entropy_hip_backward";
  if (!ensure_init()) return;
  Tensor *x = inputs[0];
  const Tensor *lab = inputs[1], *st = inputs[2];
  if (!x->requires_grad || !x->grad) return;
  if (!check_ce(x, lab, st, where)) return;
  if (!output->grad || !contiguous(x->grad)) {
    report_error(where, "needs the loss gradient and a contiguous logits gradient");
    return;
  }
  const uint64_t N = x->shape[0];
  const uint32_t C = uint32_t(x->shape[1]);
  if (N == 0 || C == 0) return;

  const bool vec = C % 4 == 0 && aligned16(x->data) && aligned16(x->grad->data);
  // each workgroup covers kBwdUnroll float4 per lane of one row
  const uint32_t per_block = kCeBlock * kBwdUnroll * 4;
  const uint32_t chunks = ceil_div(C, per_block);
  const bool over = params.keepdim == 1;
  const uint64_t C4 = C / 4;
  // rows per launch, so that every grid below stays within the dispatch limit
  uint64_t R = max_blocks(kCeBlock) / chunks;
  if (vec && C4 && R > max_blocks(kCeBlock) * kCeBlock / C4) R = max_blocks(kCeBlock) * kCeBlock / C4;
  if (vec && C4 && R > max_blocks(kCeFlatBlock) * kCeFlatBlock / C4)
    R = max_blocks(kCeFlatBlock) * kCeFlatBlock / C4;
  if (R == 0) R = 1;
  for (uint64_t r0 = 0; r0 < N; r0 += R) {
    const uint64_t n = N - r0 < R ? N - r0 : R;
    const float *px = static_cast<const float *>(x->data) + r0 * C;
    float *pd = static_cast<float *>(x->grad->data) + r0 * C;
    const int32_t *pl = static_cast<const int32_t *>(lab->data) + r0;
    const float *ps = static_cast<const float *>(st->data) + 2 * r0;
    const float *pg = static_cast<const float *>(output->grad->data) + r0;
    const unsigned grid = unsigned(uint64_t(chunks) * n);
    const uint64_t units = n * C4;
    if (vec) {
      const MagicDiv dc4 = MagicDiv::make(uint32_t(C4));
      const unsigned g = unsigned(ceil_div(units, kCeFlatBlock));
      if (over)
        ce_bwd_flat_kernel<true><<<g, kCeFlatBlock, 0, stream()>>>(px, pl, ps, pg, pd, dc4, uint32_t(units));
      else
        ce_bwd_flat_kernel<false><<<g, kCeFlatBlock, 0, stream()>>>(px, pl, ps, pg, pd, dc4, uint32_t(units));
    } else if (over)
      ce_bwd_scalar_kernel<true><<<grid, kCeBlock, 0, stream()>>>(px, pl, ps, pg, pd, C, chunks);
    else
      ce_bwd_scalar_kernel<false><<<grid, kCeBlock, 0, stream()>>>(px, pl, ps, pg, pd, C, chunks);
  }
  finish(where);
}

void softmax_cross_entropy_step_hip(const float *logits, const int32_t *labels, const float *dloss,
                                    float *stats, float *loss, float *dlogits, float *dbias,
                                    float *mean_loss, u64 N, u64 C) {
  const char *where = "softmax_cross_entropy_step_hip";
  if (!ensure_init()) return;
  if (N == 0) {
    step_tail(nullptr, nullptr, 0, 0, loss, mean_loss, 0);
    if (mean_loss) finish(where);
    return;
  }
  const int V = ce_step_form(logits, labels, dloss, stats, loss, dlogits, N, C, where);
  if (V < 0) return;
  if (V == 0) {
    // any other row: the forward, the overwriting backward and the column sum as three passes
    Tensor tx, tl, ts, to, tg, tdx;
    memset(&tx, 0, sizeof tx);
    tx.ndim = 2;
    tx.shape[0] = N, tx.shape[1] = C, tx.strides[0] = C, tx.strides[1] = 1;
    tx.data = const_cast<float *>(logits), tx.dtype = FLOAT32, tx.device = GPU;
    tx.requires_grad = true;
    tdx = tx;
    tdx.data = dlogits, tdx.requires_grad = false;
    tx.grad = &tdx;
    tl = tx;
    tl.ndim = 1, tl.shape[0] = N, tl.strides[0] = 1, tl.data = const_cast<int32_t *>(labels);
    tl.dtype = INT32, tl.requires_grad = false, tl.grad = nullptr;
    ts = tl;
    ts.shape[0] = 2 * N, ts.data = stats, ts.dtype = FLOAT32;
    to = tl;
    to.data = loss, to.dtype = FLOAT32;
    tg = to;
    tg.data = const_cast<float *>(dloss);
    to.grad = &tg;
    const Tensor *fin[3] = {&tx, &tl, &ts};
    softmax_cross_entropy_hip_forward(fin, &to, KernelParams{0, 0, 0.0f});
    Tensor *bin[3] = {&tx, &tl, &ts};
    softmax_cross_entropy_hip_backward(bin, &to, KernelParams{0, 1, 0.0f});
    if (dbias) bias_grad_reduce_hip(dlogits, dbias, N * C, C);
    if (mean_loss) {
      step_tail(nullptr, nullptr, 0, 0, loss, mean_loss, N);
      finish(where);
    }
    return;
  }
  const uint64_t grid = ce_step_grid(N, C);
  // the workgroups' column sums (written even when no bias gradient is wanted; then unread)
  float *part = static_cast<float *>(workspace(sizeof(float) * grid * C));
  if (!part) return;
  ce_step_launch(V, unsigned(grid), part, logits, labels, dloss, stats, loss, dlogits, dbias,
                 mean_loss, N, C);
  finish(where);
}

void softmax_cross_entropy_step_noalloc_hip(const float *logits, const int32_t *labels,
                                            const float *dloss, float *stats, float *loss,
                                            float *dlogits, float *dbias, float *mean_loss, u64 N,
                                            u64 C) {
  const char *where = "softmax_cross_entropy_step_noalloc_hip";
  if (!ensure_init()) return;
  if (N == 0) {
    step_tail(nullptr, nullptr, 0, 0, loss, mean_loss, 0);
    if (mean_loss) finish(where);
    return;
  }
  const int V = ce_step_form(logits, labels, dloss, stats, loss, dlogits, N, C, where);
  if (V < 0) return;
  if (V == 0) {
    report_error(where, "rows of %llu floats are not one-pass rows (whole float4, 16-byte aligned "
                 "logits and dlogits, at most %llu floats): the three-pass form allocates",
                 (unsigned long long)C, (unsigned long long)kStepMaxC);
    return;
  }
  float *part = noalloc_scratch(where);
  if (!part) return;
  const uint64_t grid = ce_step_grid(N, C);
  ce_step_launch(V, unsigned(grid), part, logits, labels, dloss, stats, loss, dlogits, dbias,
                 mean_loss, N, C);
  finish(where);
}

void softmax_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  softmax_forward<false>(inputs, output, params, "softmax_hip_forward");
}
void softmax_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  softmax_backward<false>(inputs, output, params, "softmax_hip_backward");
}
void log_softmax_hip_forward(const Tensor **inputs, Tensor *output, KernelParams params) {
  softmax_forward<true>(inputs, output, params, "log_softmax_hip_forward");
}
void log_softmax_hip_backward(Tensor **inputs, const Tensor *output, KernelParams params) {
  softmax_backward<true>(inputs, output, params, "log_softmax_hip_backward");
}

}  // extern "C"
