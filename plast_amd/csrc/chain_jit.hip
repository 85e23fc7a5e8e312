// chain_jit.hip — fused elementwise chains compiled into straight-line kernels at first use.
//
// The tape interpreter (TapeBody) pays one instruction dispatch per tape step and per evaluation, so
// it evaluates two float4 units per lane to amortise that; the shape that streams fastest on MI355X
// is one float4 per lane with XCD-contiguous workgroups, where the dispatch would be paid per unit.
// For spaces of at least kMinUnits float4 units this file writes the tape out as HIP source — the
// interpreter's statement for each instruction, component by component, through the same ocml
// functions, compiled with the library's flags (contraction off, no packed fp32) — compiles it once
// per distinct tape and launch form with hiprtc for the device's architecture, and launches it:
//  - flat form: inputs unit-stride or broadcast scalars, one float4 per lane;
//  - rows form: rows of float4 units where an input may be re-read for every row (a bias row)
//    or be one scalar per row, one float4 per lane;
//  - tile form: the transposed-operand tile of ew_tile_fixed_kernel (64x64 tiles, operand roles
//    fixed per kernel) with the tape inlined per output row.
// Immediates are kernel arguments, so tapes that differ only in constants share a kernel. Compiled
// modules stay loaded until the process ends. Every result bit equals the interpreter's.
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "chain_jit.hpp"
#include "common.hpp"

// The kernels' parameter blocks. Each is declared once here and pasted as text into the generated
// source, so host and device agree on the layout.
#define PLAST_JIT_FLAT_ARGS                                                                        \
  struct JitArgs {                                                                                 \
    const float *in[4];                                                                            \
    float *out;                                                                                    \
    unsigned long long units;                                                                      \
    unsigned long long simd_end;                                                                   \
    float imm[16];                                                                                 \
  };
#define PLAST_JIT_TILE_ARGS                                                                        \
  struct JitTileArgs {                                                                             \
    const float *in[4];                                                                            \
    float *out;                                                                                    \
    long long bst[5][8];                                                                           \
    unsigned bdv[8][3];                                                                            \
    long long qst[5];                                                                              \
    long long pst[5];                                                                              \
    unsigned nbatch;                                                                               \
    unsigned tq;                                                                                   \
    unsigned tp;                                                                                   \
    unsigned dtq[3];                                                                               \
    unsigned dtp[3];                                                                               \
    unsigned long long simd_end;                                                                   \
    float imm[16];                                                                                 \
  };
#define PLAST_JIT_ROWS_ARGS                                                                        \
  struct JitRowsArgs {                                                                             \
    const float *in[4];                                                                            \
    float *out;                                                                                    \
    unsigned long long units;                                                                      \
    unsigned long long simd_end;                                                                   \
    float imm[16];                                                                                 \
    long long ist[4];                                                                              \
    long long ost;                                                                                 \
    unsigned dm[3];                                                                                \
  };
#define PLAST_JIT_STR2(...) #__VA_ARGS__
#define PLAST_JIT_STR(...) PLAST_JIT_STR2(__VA_ARGS__)

namespace plast {
namespace {

PLAST_JIT_FLAT_ARGS
PLAST_JIT_TILE_ARGS
PLAST_JIT_ROWS_ARGS
static_assert(PLAST_TAPE_MAX_INPUTS == 4 && PLAST_TAPE_MAX_INS == 16 && PLAST_MAX_NDIM == 8,
              "the parameter blocks above are written for these limits");

constexpr uint64_t kMinUnits = uint64_t(1) << 18;  // 2^20 elements: below that, compiling costs more
constexpr int kJitBlock = 256;                     // lanes per workgroup, every form
constexpr int kJitTile = 64, kJitTilePad = 1;      // the interpreter's tile (kTile, kTilePad)
// Rows form launch shape, measured on a [16384, 4096] bias + relu chain: two float4 units per lane
// with ordinary stores 6.48 -> 6.76 TB/s (one unit, or nontemporal stores, or XCD numbering slower).
#ifndef PLAST_JIT_ROWS_UNROLL
#define PLAST_JIT_ROWS_UNROLL 2     // rows form: float4 units per lane
#endif
#ifndef PLAST_JIT_ROWS_NT_STORE
#define PLAST_JIT_ROWS_NT_STORE 0   // rows form with a re-read input: nontemporal stores
#endif
#ifndef PLAST_JIT_ROWS_XCD
#define PLAST_JIT_ROWS_XCD 0        // rows form with a re-read input: XCD-contiguous workgroups
#endif

struct Entry {
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
  bool ok = false;
};

std::mutex g_mu;
std::unordered_map<std::string, Entry> g_cache;
int g_mode = -1;  // -1: not decided yet (PLAST_HIP_CHAIN_JIT=0 in the environment switches it off)
uint64_t g_launches = 0;
bool g_logged = false;

int mode_locked() {
  if (g_mode < 0) {
    const char *e = std::getenv("PLAST_HIP_CHAIN_JIT");
    g_mode = (e && e[0] == '0') ? 0 : 1;
  }
  return g_mode;
}

// What the generated code depends on: the form and its layout pattern, the inputs and every
// instruction but its immediate.
std::string key_of(char form, uint32_t pattern, const PlastFusedTape &t, int device) {
  std::string k;
  k.push_back(form);
  k.append(reinterpret_cast<const char *>(&pattern), sizeof pattern);
  k.push_back(char(t.num_inputs));
  k.push_back(char(device));
  for (uint32_t i = 0; i < t.num_ins; ++i) {
    k.push_back(char(t.ins[i].op));
    k.push_back(char(t.ins[i].src));
    k.push_back(char(t.ins[i].idx));
    k.push_back(char(t.ins[i].acc_rhs));
  }
  return k;
}

// The operand of instruction i, as it reads inside the per-component loop.
std::string operand(const PlastTapeIns &ins, int i) {
  if (ins.src == TAPE_SRC_INPUT) return "x" + std::to_string(ins.idx) + "[c]";
  if (ins.src == TAPE_SRC_IMM) return "A.imm[" + std::to_string(i) + "]";
  return "a";  // TAPE_SRC_ACC, and TAPE_SRC_NONE as the interpreter reads it
}

// The tape over component c of the float4 operands x0..x3, into `dst`[c]: per instruction the
// interpreter's case (TapeBody::eval_units in ew.hpp). `simd` names the NEG rule's side.
std::string tape_loop(const PlastFusedTape &t, const std::string &dst, const std::string &ind) {
  std::string s;
  s += ind + "for (int c = 0; c < 4; ++c) {\n";
  const std::string in2 = ind + "  ";
  s += in2 + "float a = x" + std::to_string(t.ins[0].idx) + "[c];\n";
  for (uint32_t i = 1; i < t.num_ins; ++i) {
    const PlastTapeIns &ins = t.ins[i];
    const std::string o = operand(ins, int(i)), I = std::to_string(i);
    switch (ins.op) {
    case TAPE_ADD: s += in2 + "a = a + " + o + ";\n"; break;
    case TAPE_MUL: s += in2 + "a = a * " + o + ";\n"; break;
    case TAPE_SUB: s += in2 + (ins.acc_rhs ? "a = " + o + " - a;\n" : "a = a - " + o + ";\n"); break;
    case TAPE_DIV: s += in2 + (ins.acc_rhs ? "a = " + o + " / a;\n" : "a = a / " + o + ";\n"); break;
    case TAPE_LEAKY_RELU: s += in2 + "a = a > 0.0f ? a : a * A.imm[" + I + "];\n"; break;
    case TAPE_EXP: s += in2 + "a = expf(a);\n"; break;
    case TAPE_LOG: s += in2 + "a = logf(a);\n"; break;
    case TAPE_NEG: s += in2 + "a = simd ? 0.0f - a : -a;\n"; break;
    case TAPE_ABS: s += in2 + "a = fabsf(a);\n"; break;
    case TAPE_SIN: s += in2 + "a = sinf(a);\n"; break;
    case TAPE_COS: s += in2 + "a = cosf(a);\n"; break;
    case TAPE_TAN: s += in2 + "a = tanf(a);\n"; break;
    default: break;  // a later TAPE_LOAD is a no-op in the interpreter too
    }
  }
  s += in2 + dst + "[c] = a;\n";
  s += ind + "}\n";
  return s;
}

const std::string kPrelude = "typedef float f4 __attribute__((ext_vector_type(4)));\n";

// XCD-contiguous numbering of the first 8 * (grid / 8) workgroups (xcd_block in common.hpp).
const std::string kXcdBlock =
    "  const unsigned per = gridDim.x / 8;\n"
    "  unsigned bid = blockIdx.x;\n"
    "  if (bid < per * 8) bid = (bid % 8) * per + bid / 8;\n";

// Flat form: bit k of bcast marks input k as one broadcast scalar.
std::string flat_source(const PlastFusedTape &t, uint32_t bcast) {
  std::string s = kPrelude + PLAST_JIT_STR(PLAST_JIT_FLAT_ARGS) + "\n";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(kJitBlock) +
       ") void plast_chain(JitArgs A) {\n";
  s += kXcdBlock;
  s += "  const unsigned long long q = (unsigned long long)bid * " + std::to_string(kJitBlock) +
       " + threadIdx.x;\n";
  s += "  if (q >= A.units) return;\n";
  s += "  const bool simd = q * 4 < A.simd_end;\n";
  s += "  (void)simd;\n";
  for (uint32_t k = 0; k < t.num_inputs; ++k) {
    const std::string K = std::to_string(k);
    if (bcast >> k & 1u)
      s += "  const f4 x" + K + " = f4(A.in[" + K + "][0]);\n";
    else
      s += "  const f4 x" + K + " = __builtin_nontemporal_load((const f4 *)A.in[" + K + "] + q);\n";
    s += "  (void)x" + K + ";\n";
  }
  s += "  f4 r;\n";
  s += tape_loop(t, "r", "  ");
  s += "  ((f4 *)A.out)[q] = r;\n";
  s += "}\n";
  return s;
}

// Rows form over [rows, inner] (inner a multiple of 4, unit-stride output rows): bits 0-3 of
// `pattern` mark inputs that are one scalar per row, bits 8-11 inputs re-read for every row (row
// stride 0); those are read with ordinary loads (the re-read hits in cache), the streamed ones
// with nontemporal loads, and a launch with a re-read input keeps dispatch order.
std::string rows_source(const PlastFusedTape &t, uint32_t pattern) {
  const uint32_t scalar = pattern & 0xfu, reread = (pattern >> 8) & 0xfu;
  constexpr int U = PLAST_JIT_ROWS_UNROLL;
  const bool nt_store = reread && PLAST_JIT_ROWS_NT_STORE;
  const bool xcd = !reread || PLAST_JIT_ROWS_XCD;
  std::string s = kPrelude + PLAST_JIT_STR(PLAST_JIT_ROWS_ARGS) + "\n";
  s += "static __device__ __forceinline__ unsigned mdiv(unsigned n, const unsigned *m) {\n"
       "  const unsigned long long hi = __umulhi(n, m[0]);\n"
       "  return (unsigned)((hi + n) >> m[1]);\n"
       "}\n";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(kJitBlock) +
       ") void plast_chain_rows(JitRowsArgs A) {\n";
  if (xcd) s += kXcdBlock;
  else s += "  const unsigned bid = blockIdx.x;\n";
  for (int u = 0; u < U; ++u) {
    const std::string q = "q" + std::to_string(u), row = "row" + std::to_string(u),
                      col = "col" + std::to_string(u);
    s += "  const unsigned " + q + " = bid * " + std::to_string(kJitBlock * U) + " + " +
         std::to_string(u * kJitBlock) + " + threadIdx.x;\n";
    s += "  const bool ok" + std::to_string(u) + " = " + q + " < A.units;\n";
    s += "  const unsigned " + row + " = mdiv(" + q + ", A.dm);\n";
    s += "  const long long " + col + " = (long long)(" + q + " - " + row + " * A.dm[2]) * 4;\n";
  }
  // every load of every unit first, then the chains, then the stores
  for (int u = 0; u < U; ++u) {
    const std::string us = std::to_string(u), row = "row" + us, col = "col" + us;
    for (uint32_t k = 0; k < t.num_inputs; ++k) {
      const std::string K = std::to_string(k), X = "x" + K + "_" + us;
      const std::string at = "A.in[" + K + "] + (long long)" + row + " * A.ist[" + K + "]";
      s += "  f4 " + X + " = f4(0.0f);\n";
      if (scalar >> k & 1u)
        s += "  if (ok" + us + ") " + X + " = f4(*(" + at + "));\n";
      else if (reread >> k & 1u)
        s += "  if (ok" + us + ") " + X + " = *(const f4 *)(" + at + " + " + col + ");\n";
      else
        s += "  if (ok" + us + ") " + X + " = __builtin_nontemporal_load((const f4 *)(" + at + " + " +
             col + "));\n";
    }
  }
  for (int u = 0; u < U; ++u) {
    const std::string us = std::to_string(u);
    s += "  if (ok" + us + ") {\n";
    s += "    const bool simd = (unsigned long long)q" + us + " * 4 < A.simd_end;\n";
    s += "    (void)simd;\n";
    for (uint32_t k = 0; k < t.num_inputs; ++k) {
      const std::string K = std::to_string(k);
      s += "    const f4 x" + K + " = x" + K + "_" + us + ";\n";
      s += "    (void)x" + K + ";\n";
    }
    s += "    f4 r;\n";
    s += tape_loop(t, "r", "    ");
    s += "    f4 *dst = (f4 *)(A.out + (long long)row" + us + " * A.ost + col" + us + ");\n";
    s += nt_store ? "    __builtin_nontemporal_store(r, dst);\n" : "    *dst = r;\n";
    s += "  }\n";
  }
  s += "}\n";
  return s;
}

// Tile form: the structure of ew_tile_fixed_kernel (ew_impl.hpp) with compile-time roles. Every
// global read of the tile is issued before the barrier; the transposed operands go through LDS.
std::string tile_source(const PlastFusedTape &t, uint32_t roles) {
  const int nin = int(t.num_inputs), OUT = PLAST_TAPE_MAX_INPUTS;
  const std::string T = std::to_string(kJitTile), TP = std::to_string(kJitTile + kJitTilePad),
                    O = std::to_string(OUT);
  auto role = [&](int k) { return (roles >> (2 * k)) & 3u; };
  auto tile_at = [&](int slot) { return std::to_string(slot * kJitTile * (kJitTile + kJitTilePad)); };
  std::string s = kPrelude + PLAST_JIT_STR(PLAST_JIT_TILE_ARGS) + "\n";
  s += "static __device__ __forceinline__ unsigned mdiv(unsigned n, const unsigned *m) {\n"
       "  const unsigned long long hi = __umulhi(n, m[0]);\n"
       "  return (unsigned)((hi + n) >> m[1]);\n"
       "}\n";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(kJitBlock) +
       ") void plast_chain_tile(JitTileArgs A) {\n";
  s += "  extern __shared__ float lds[];\n";
  s += kXcdBlock;
  s += "  const unsigned bq = mdiv(bid, A.dtp);\n"
       "  const unsigned tpi = bid - bq * A.tp;\n"
       "  const unsigned bi = mdiv(bq, A.dtq);\n"
       "  const unsigned tqi = bq - bi * A.tq;\n";
  s += "  long long base[" + std::to_string(OUT + 1) + "] = {};\n";
  s += "  unsigned rem = bi;\n";
  s += "  for (int d = (int)A.nbatch - 1; d >= 0; --d) {\n"
       "    const unsigned nxt = mdiv(rem, A.bdv[d]);\n"
       "    const long long c = (long long)(rem - nxt * A.bdv[d][2]);\n"
       "    rem = nxt;\n";
  for (int k = 0; k < nin; ++k)
    s += "    base[" + std::to_string(k) + "] += c * A.bst[" + std::to_string(k) + "][d];\n";
  s += "    base[" + O + "] += c * A.bst[" + O + "][d];\n";
  s += "  }\n";
  s += "  const long long q0 = (long long)tqi * " + T + ", p0 = (long long)tpi * " + T + ";\n";
  s += "  const int t = threadIdx.x;\n";
  s += "  const unsigned l4 = (t & 15) * 4, r16 = t >> 4;\n";
  s += "  const bool simd = 0 < A.simd_end;\n";
  s += "  (void)simd;\n";
  int slot = 0;
  std::vector<int> slot_of(nin, -1);
  for (int k = 0; k < nin; ++k) {
    const std::string K = std::to_string(k);
    const std::string in = "A.in[" + K + "] + base[" + K + "]";
    switch (role(k)) {
    case 0:  // staged: float4 along q of tile rows p0 + r16 + 16r, nontemporal
      slot_of[k] = slot++;
      s += "  f4 v" + K + "[4];\n";
      s += "  { const float *src = " + in + " + (q0 + l4) * A.qst[" + K + "] + (p0 + r16) * A.pst[" +
           K + "];\n";
      s += "    const long long step = 16 * A.pst[" + K + "];\n";
      s += "    for (int r = 0; r < 4; ++r) v" + K +
           "[r] = __builtin_nontemporal_load((const f4 *)(src + r * step)); }\n";
      break;
    case 1:  // the scalar of each output row q0 + r16 + 16r
      s += "  float v" + K + "[4];\n";
      s += "  { const float *src = " + in + " + (q0 + r16) * A.qst[" + K + "];\n";
      s += "    const long long step = 16 * A.qst[" + K + "];\n";
      s += "    for (int r = 0; r < 4; ++r) v" + K + "[r] = src[r * step]; }\n";
      break;
    case 2:  // one float4 along p
      s += "  const f4 v" + K + " = *(const f4 *)(" + in + " + (p0 + l4) * A.pst[" + K + "]);\n";
      break;
    default:  // float4 along p of each output row
      s += "  f4 v" + K + "[4];\n";
      s += "  { const float *src = " + in + " + (q0 + r16) * A.qst[" + K + "] + (p0 + l4);\n";
      s += "    const long long step = 16 * A.qst[" + K + "];\n";
      s += "    for (int r = 0; r < 4; ++r) v" + K + "[r] = *(const f4 *)(src + r * step); }\n";
      break;
    }
  }
  for (int k = 0; k < nin; ++k) {
    if (slot_of[k] < 0) continue;
    const std::string K = std::to_string(k);
    s += "  { float *tile = lds + " + tile_at(slot_of[k]) + ";\n";
    s += "    for (int r = 0; r < 4; ++r)\n";
    s += "      for (int c = 0; c < 4; ++c) tile[(r16 + 16 * r) * " + TP + " + l4 + c] = v" + K +
         "[r][c]; }\n";
  }
  s += "  __syncthreads();\n";
  s += "  float *dst = A.out + base[" + O + "] + (q0 + r16) * A.qst[" + O + "] + (p0 + l4);\n";
  s += "  const long long dstep = 16 * A.qst[" + O + "];\n";
  s += "#pragma unroll\n";
  s += "  for (int r = 0; r < 4; ++r) {\n";
  s += "    const unsigned row = r16 + 16 * r;\n";
  s += "    (void)row;\n";
  for (int k = 0; k < nin; ++k) {
    const std::string K = std::to_string(k);
    switch (role(k)) {
    case 0:
      s += "    f4 x" + K + ";\n";
      s += "    { const float *tile = lds + " + tile_at(slot_of[k]) + ";\n";
      s += "      for (int c = 0; c < 4; ++c) x" + K + "[c] = tile[(l4 + c) * " + TP + " + row]; }\n";
      break;
    case 1: s += "    const f4 x" + K + " = f4(v" + K + "[r]);\n"; break;
    case 2: s += "    const f4 x" + K + " = v" + K + ";\n"; break;
    default: s += "    const f4 x" + K + " = v" + K + "[r];\n"; break;
    }
    s += "    (void)x" + K + ";\n";
  }
  s += "    f4 res;\n";
  s += tape_loop(t, "res", "    ");
  s += "    *(f4 *)(dst + r * dstep) = res;\n";
  s += "  }\n";
  s += "}\n";
  return s;
}

void log_once(const char *what, const std::string &detail) {
  if (g_logged) return;
  g_logged = true;
  std::fprintf(stderr, "plast_hip: chain compiler unavailable (%s), fused chains run on the tape "
                       "interpreter%s%s\n", what, detail.empty() ? "" : ": ", detail.c_str());
}

bool compile(const std::string &src, const char *name, int device, Entry &e) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    log_once("hipGetDeviceProperties", "");
    return false;
  }
  std::string arch(prop.gcnArchName);
  arch = "--offload-arch=" + arch.substr(0, arch.find(':'));
  hiprtcProgram p;
  if (hiprtcCreateProgram(&p, src.c_str(), "plast_chain.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    log_once("hiprtcCreateProgram", "");
    return false;
  }
  // the library's own code-generation flags: no contraction, scalar fp32 forms
  const char *opts[] = {arch.c_str(), "-O3", "-std=c++17", "-ffp-contract=off",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult r = hiprtcCompileProgram(p, int(sizeof(opts) / sizeof(opts[0])), opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(p, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(p, &log[0]);
    log_once(hiprtcGetErrorString(r), log);
    hiprtcDestroyProgram(&p);
    return false;
  }
  size_t n = 0;
  hiprtcGetCodeSize(p, &n);
  std::vector<char> code(n);
  hiprtcGetCode(p, code.data());
  hiprtcDestroyProgram(&p);
  if (hipModuleLoadData(&e.mod, code.data()) != hipSuccess ||
      hipModuleGetFunction(&e.fn, e.mod, name) != hipSuccess) {
    (void)hipGetLastError();
    log_once("hipModuleLoadData", "");
    return false;
  }
  return true;
}

// The cached kernel for (form, pattern, tape), compiling it on first use; null when unavailable.
hipFunction_t kernel_for(char form, uint32_t pattern, const PlastFusedTape &t) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return nullptr;  // the library's device is current
  std::lock_guard<std::mutex> lock(g_mu);
  if (!mode_locked()) return nullptr;
  const std::string key = key_of(form, pattern, t, device);
  auto it = g_cache.find(key);
  if (it == g_cache.end()) {
    Entry e;
    if (form == 'F') e.ok = compile(flat_source(t, pattern), "plast_chain", device, e);
    else if (form == 'R') e.ok = compile(rows_source(t, pattern), "plast_chain_rows", device, e);
    else e.ok = compile(tile_source(t, pattern), "plast_chain_tile", device, e);
    it = g_cache.emplace(key, e).first;
  }
  return it->second.ok ? it->second.fn : nullptr;
}

bool launch(hipFunction_t fn, void *args, unsigned blocks, size_t lds_bytes) {
  void *params[] = {args};
  if (hipModuleLaunchKernel(fn, blocks, 1, 1, kJitBlock, 1, 1, unsigned(lds_bytes), stream(), params,
                            nullptr) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  ++g_launches;
  return true;
}

bool well_formed(const PlastFusedTape *t) {
  return t && t->num_ins > 0 && t->num_ins <= PLAST_TAPE_MAX_INS && t->num_inputs > 0 &&
         t->num_inputs <= PLAST_TAPE_MAX_INPUTS;
}

u64 copy_out(const std::string &src, char *buf, u64 cap) {
  if (buf && cap) {
    const size_t n = src.size() < cap - 1 ? src.size() : size_t(cap - 1);
    std::memcpy(buf, src.data(), n);
    buf[n] = '\0';
  }
  return src.size();
}

}  // namespace

bool chain_jit_launch(const PlastFusedTape &t, const float *const *in, uint32_t bcast, float *out,
                      uint64_t units, uint64_t simd_end) {
  if (units < kMinUnits) return false;
  const uint64_t blocks = (units + kJitBlock - 1) / kJitBlock;
  if (blocks > max_blocks(kJitBlock)) return false;
  const hipFunction_t fn = kernel_for('F', bcast, t);
  if (!fn) return false;
  JitArgs a = {};
  for (uint32_t k = 0; k < t.num_inputs; ++k) a.in[k] = in[k];
  a.out = out;
  a.units = units;
  a.simd_end = simd_end;
  for (uint32_t i = 0; i < t.num_ins; ++i) a.imm[i] = t.ins[i].imm;
  return launch(fn, &a, unsigned(blocks), 0);
}

bool chain_jit_rows_launch(const PlastFusedTape &t, const float *const *in, const int64_t *ist,
                           uint32_t scalar, uint32_t reread, float *out, int64_t ost,
                           uint64_t units, uint32_t inner4, uint64_t simd_end) {
  if (units < kMinUnits || units >= (uint64_t(1) << 32) || inner4 == 0) return false;
  const uint64_t per_block = uint64_t(kJitBlock) * PLAST_JIT_ROWS_UNROLL;
  const uint64_t blocks = (units + per_block - 1) / per_block;
  if (blocks > max_blocks(kJitBlock)) return false;
  const hipFunction_t fn = kernel_for('R', (scalar & 0xfu) | (reread & 0xfu) << 8, t);
  if (!fn) return false;
  JitRowsArgs a = {};
  for (uint32_t k = 0; k < t.num_inputs; ++k) {
    a.in[k] = in[k];
    a.ist[k] = ist[k];
  }
  a.out = out;
  a.ost = ost;
  a.units = units;
  a.simd_end = simd_end;
  for (uint32_t i = 0; i < t.num_ins; ++i) a.imm[i] = t.ins[i].imm;
  const MagicDiv m = MagicDiv::make(inner4);
  a.dm[0] = m.mul;
  a.dm[1] = m.shift;
  a.dm[2] = m.d;
  return launch(fn, &a, unsigned(blocks), 0);
}

bool chain_jit_tile_launch(const PlastFusedTape &t, const ChainTileGeometry &g, uint32_t roles,
                           uint64_t elements, uint64_t simd_end, unsigned blocks, size_t lds_bytes) {
  if (elements / 4 < kMinUnits) return false;
  const hipFunction_t fn = kernel_for('T', roles, t);
  if (!fn) return false;
  JitTileArgs a = {};
  for (int k = 0; k < PLAST_TAPE_MAX_INPUTS; ++k) a.in[k] = g.in[k];
  a.out = g.out;
  std::memcpy(a.bst, g.bst, sizeof a.bst);
  std::memcpy(a.bdv, g.bdv, sizeof a.bdv);
  std::memcpy(a.qst, g.qst, sizeof a.qst);
  std::memcpy(a.pst, g.pst, sizeof a.pst);
  a.nbatch = g.nbatch;
  a.tq = g.tq;
  a.tp = g.tp;
  std::memcpy(a.dtq, g.dtq, sizeof a.dtq);
  std::memcpy(a.dtp, g.dtp, sizeof a.dtp);
  a.simd_end = simd_end;
  for (uint32_t i = 0; i < t.num_ins; ++i) a.imm[i] = t.ins[i].imm;
  return launch(fn, &a, blocks, lds_bytes);
}

}  // namespace plast

using namespace plast;

extern "C" {

int plast_hip_set_chain_jit(int mode) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int prev = mode_locked();
  g_mode = mode != 0 ? 1 : 0;
  return prev;
}

u64 plast_hip_chain_jit_launches(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return g_launches;
}

u64 plast_hip_chain_jit_source(const PlastFusedTape *tape, u32 bcast, char *buf, u64 cap) {
  return well_formed(tape) ? copy_out(flat_source(*tape, bcast), buf, cap) : 0;
}

u64 plast_hip_chain_jit_rows_source(const PlastFusedTape *tape, u32 pattern, char *buf, u64 cap) {
  return well_formed(tape) ? copy_out(rows_source(*tape, pattern), buf, cap) : 0;
}

u64 plast_hip_chain_jit_tile_source(const PlastFusedTape *tape, u32 roles, char *buf, u64 cap) {
  return well_formed(tape) ? copy_out(tile_source(*tape, roles), buf, cap) : 0;
}

}  // extern "C"
