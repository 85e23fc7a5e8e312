// chain_jit.hip — fused elementwise chains compiled into straight-line kernels at first use.
//
// The tape interpreter (TapeBody) pays one instruction dispatch per tape step and per evaluation, so
// it evaluates two float4 units per lane to amortise that; the shape that streams fastest on MI355X
// is one float4 per lane with XCD-contiguous workgroups, where the dispatch would be paid per unit.
// For flat spaces of at least kMinUnits float4 units this file writes the tape out as HIP source —
// the same per-element operations in the same order, through the same ocml functions, compiled
// with contraction off — compiles it once per distinct tape with hiprtc for the device's
// architecture, and launches it with the one-unit shape. Immediates are kernel arguments, so tapes
// that differ only in constants share one kernel. Compiled modules stay loaded until the process
// ends. The fused op's semantics are unchanged: every result bit equals the interpreter's.
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

namespace plast {
namespace {

constexpr uint64_t kMinUnits = uint64_t(1) << 18;  // 2^20 elements: below that, compiling costs more
constexpr int kJitBlock = 256;

// The generated kernel's parameter block (its source declares the same struct).
struct JitArgs {
  const float *in[PLAST_TAPE_MAX_INPUTS];
  float *out;
  uint64_t units;
  uint64_t simd_end;
  float imm[PLAST_TAPE_MAX_INS];
};

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

// What the generated code depends on: inputs, broadcast pattern and every instruction but its
// immediate.
std::string key_of(const PlastFusedTape &t, uint32_t bcast, int device) {
  std::string k;
  k.push_back(char(t.num_inputs));
  k.push_back(char(bcast));
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

// Per instruction the interpreter's case (TapeBody::eval_units in ew.hpp), component by component.
std::string source_of(const PlastFusedTape &t, uint32_t bcast) {
  const std::string NI = std::to_string(PLAST_TAPE_MAX_INPUTS), NS = std::to_string(PLAST_TAPE_MAX_INS);
  std::string s;
  s += "typedef float f4 __attribute__((ext_vector_type(4)));\n";
  s += "struct JitArgs { const float *in[" + NI + "]; float *out; unsigned long long units;\n";
  s += "  unsigned long long simd_end; float imm[" + NS + "]; };\n";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(kJitBlock) +
       ") void plast_chain(JitArgs A) {\n";
  // XCD-contiguous numbering of the first 8 * (grid / 8) workgroups (xcd_block in common.hpp)
  s += "  const unsigned per = gridDim.x / 8;\n";
  s += "  unsigned b = blockIdx.x;\n";
  s += "  if (b < per * 8) b = (b % 8) * per + b / 8;\n";
  s += "  const unsigned long long q = (unsigned long long)b * " + std::to_string(kJitBlock) +
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
  s += "  for (int c = 0; c < 4; ++c) {\n";
  s += "    float a = x" + std::to_string(t.ins[0].idx) + "[c];\n";
  for (uint32_t i = 1; i < t.num_ins; ++i) {
    const PlastTapeIns &ins = t.ins[i];
    const std::string o = operand(ins, int(i)), I = std::to_string(i);
    switch (ins.op) {
    case TAPE_ADD: s += "    a = a + " + o + ";\n"; break;
    case TAPE_MUL: s += "    a = a * " + o + ";\n"; break;
    case TAPE_SUB: s += ins.acc_rhs ? "    a = " + o + " - a;\n" : "    a = a - " + o + ";\n"; break;
    case TAPE_DIV: s += ins.acc_rhs ? "    a = " + o + " / a;\n" : "    a = a / " + o + ";\n"; break;
    case TAPE_LEAKY_RELU: s += "    a = a > 0.0f ? a : a * A.imm[" + I + "];\n"; break;
    case TAPE_EXP: s += "    a = expf(a);\n"; break;
    case TAPE_LOG: s += "    a = logf(a);\n"; break;
    case TAPE_NEG: s += "    a = simd ? 0.0f - a : -a;\n"; break;
    case TAPE_ABS: s += "    a = fabsf(a);\n"; break;
    case TAPE_SIN: s += "    a = sinf(a);\n"; break;
    case TAPE_COS: s += "    a = cosf(a);\n"; break;
    case TAPE_TAN: s += "    a = tanf(a);\n"; break;
    default: break;  // a later TAPE_LOAD is a no-op in the interpreter too
    }
  }
  s += "    r[c] = a;\n";
  s += "  }\n";
  s += "  ((f4 *)A.out)[q] = r;\n";
  s += "}\n";
  return s;
}

void log_once(const char *what, const std::string &detail) {
  if (g_logged) return;
  g_logged = true;
  std::fprintf(stderr, "plast_hip: chain compiler unavailable (%s), fused chains run on the tape "
                       "interpreter%s%s\n", what, detail.empty() ? "" : ": ", detail.c_str());
}

bool compile(const std::string &src, int device, Entry &e) {
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
      hipModuleGetFunction(&e.fn, e.mod, "plast_chain") != hipSuccess) {
    (void)hipGetLastError();
    log_once("hipModuleLoadData", "");
    return false;
  }
  return true;
}

}  // namespace

bool chain_jit_launch(const PlastFusedTape &t, const float *const *in, uint32_t bcast, float *out,
                      uint64_t units, uint64_t simd_end) {
  if (units < kMinUnits) return false;
  const uint64_t blocks = (units + kJitBlock - 1) / kJitBlock;
  if (blocks > max_blocks(kJitBlock)) return false;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return false;  // the library's device is current
  hipFunction_t fn = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!mode_locked()) return false;
    const std::string key = key_of(t, bcast, device);
    auto it = g_cache.find(key);
    if (it == g_cache.end()) {
      Entry e;
      e.ok = compile(source_of(t, bcast), device, e);
      it = g_cache.emplace(key, e).first;
    }
    if (!it->second.ok) return false;
    fn = it->second.fn;
  }
  JitArgs a = {};
  for (uint32_t k = 0; k < t.num_inputs; ++k) a.in[k] = in[k];
  a.out = out;
  a.units = units;
  a.simd_end = simd_end;
  for (uint32_t i = 0; i < t.num_ins; ++i) a.imm[i] = t.ins[i].imm;
  void *params[] = {&a};
  if (hipModuleLaunchKernel(fn, unsigned(blocks), 1, 1, kJitBlock, 1, 1, 0, stream(), params,
                            nullptr) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  ++g_launches;
  return true;
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
  if (!tape || tape->num_ins == 0 || tape->num_ins > PLAST_TAPE_MAX_INS ||
      tape->num_inputs == 0 || tape->num_inputs > PLAST_TAPE_MAX_INPUTS)
    return 0;
  const std::string src = source_of(*tape, bcast);
  if (buf && cap) {
    const size_t n = src.size() < cap - 1 ? src.size() : size_t(cap - 1);
    std::memcpy(buf, src.data(), n);
    buf[n] = '\0';
  }
  return src.size();
}

}  // extern "C"
