// optim.hip — optimizer updates (SGD, Adam, AdamW) and zero_grad over lists of parameter tensors.
//
// One launch updates every tensor of a call: a table of entries (each tensor's pointers, element
// count and first workgroup) tells a workgroup, by a uniform binary search, which tensor it
// streams in float4 units (a scalar loop covers a tensor's last partial unit or an unaligned
// tensor). Up to kGroup entries travel in the kernel argument block; a call with more keeps its
// table in device memory, uploaded only when it differs from the last one (a training loop passes
// the same parameters every step). While a graph is being captured, such a call is instead split
// into launches of kGroup entries, so that no copy is recorded. Per element the update is the reference CPU
// statement in its operation order (src/optimizers/cpu/{sgd.c:16-28, adam.c:62-66,
// adamw.c:128-135}); the library is built without FMA contraction and sqrt/divide are correctly
// rounded, so every element matches the CPU update bit for bit.
#include <cmath>
#include <cstring>
#include <mutex>
#include <unordered_set>
#include <vector>

#include "common.hpp"
#include "opt_plan.hpp"

namespace plast {
namespace {

constexpr int kGroup = 64;         // tensors per launch (kernel argument block stays under 4 KiB)
constexpr int kOptUnroll = PLAST_OPT_UNROLL;  // float4 units per lane

enum class Opt { Sgd, Adam, AdamW };

// Workgroup size and XCD numbering per update, measured on MI355X over one 64M parameter with its
// buffers at several relative placements: Adam's seven streams run at 6.30-6.34 TB/s with 64-lane
// workgroups in dispatch order, against 5.6-6.1 TB/s with 256 lanes and XCD numbering (the larger
// workgroups were also the ones whose rate moved with placement); SGD keeps 256 lanes, XCD order.
template <Opt OPT>
constexpr int kOptBlock = OPT == Opt::Sgd ? PLAST_SGD_BLOCK : PLAST_ADAM_BLOCK;
template <Opt OPT>
constexpr bool kOptXcd = (OPT == Opt::Sgd ? PLAST_SGD_XCD : PLAST_ADAM_XCD) != 0;

struct OptScalars {
  float lr;        // SGD: lr; Adam/AdamW: lr_t (bias-corrected)
  float beta1, beta2, one_minus_beta1, one_minus_beta2, eps;
  float decay;     // AdamW: lr * weight_decay
};

struct OptArgs {
  float *p[kGroup];
  const float *g[kGroup];
  float *m[kGroup];
  float *v[kGroup];
  uint64_t n[kGroup];
  uint32_t first_block[kGroup + 1];  // workgroups [first_block[i], first_block[i+1]) update tensor i
  uint32_t vec_mask;                 // bit i: tensor i's pointers are 16-byte aligned
  int count;
  OptScalars s;
};

template <Opt OPT>
__device__ __forceinline__ void update(const OptScalars &A, float &p, float g, float &m, float &v) {
  if constexpr (OPT == Opt::Sgd) {
    p = p - A.lr * g;  // sgd.c:25
  } else {
    if constexpr (OPT == Opt::AdamW) p = p - A.decay * p;             // adamw.c:130
    m = A.beta1 * m + A.one_minus_beta1 * g;                          // adam.c:63
    v = A.beta2 * v + A.one_minus_beta2 * g * g;                      // adam.c:64
    p = p - A.lr * m / (sqrtf(v) + A.eps);                            // adam.c:65
  }
}

// Cache policy for parameters and moments, measured on MI355X: Adam/AdamW (four streams read,
// three written) run fastest with nontemporal loads and stores (64M parameters: 5.6 -> 5.85
// TB/s), SGD (two read, one written) with ordinary ones (7.2 vs 6.6 TB/s).
template <Opt OPT>
constexpr bool kOptNtLoad = OPT != Opt::Sgd && PLAST_ADAM_NT_LOAD != 0;
template <Opt OPT>
constexpr bool kOptNtStore = OPT != Opt::Sgd && PLAST_ADAM_NT_STORE != 0;

template <bool NT>
__device__ __forceinline__ f4 ld(const float *p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
  else return *reinterpret_cast<const f4 *>(p);
}

// The float4 units of one entry that workgroup `wb` (its number within the entry) updates.
template <Opt OPT>
__device__ __forceinline__ void update_entry(const OptScalars &S, float *P, const float *G, float *M,
                                             float *V, uint64_t n, bool vec, uint32_t wb) {
  constexpr bool kMoments = OPT != Opt::Sgd;
  constexpr int kBs = kOptBlock<OPT>;
  const uint64_t unit0 = uint64_t(wb) * (kBs * kOptUnroll) + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kOptUnroll; ++u) {
    const uint64_t e = (unit0 + uint64_t(u) * kBs) * 4;
    if (e >= n) continue;
    if (e + 4 <= n && vec) {
      f4 p = ld<kOptNtLoad<OPT>>(P + e);
      const f4 g = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(G + e));
      f4 m = f4(0.0f), v = f4(0.0f);
      if constexpr (kMoments) {
        m = ld<kOptNtLoad<OPT>>(M + e);
        v = ld<kOptNtLoad<OPT>>(V + e);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float pc = p[c], mc = m[c], vc = v[c];
        update<OPT>(S, pc, g[c], mc, vc);
        p[c] = pc;
        m[c] = mc;
        v[c] = vc;
      }
      store_stream<kOptNtStore<OPT>>(p, reinterpret_cast<f4 *>(P + e));
      if constexpr (kMoments) {
        store_stream<kOptNtStore<OPT>>(m, reinterpret_cast<f4 *>(M + e));
        store_stream<kOptNtStore<OPT>>(v, reinterpret_cast<f4 *>(V + e));
      }
    } else {
      const uint64_t end = e + 4 < n ? e + 4 : n;
      for (uint64_t j = e; j < end; ++j) {
        float p = P[j], m = 0.0f, v = 0.0f;
        if constexpr (kMoments) {
          m = M[j];
          v = V[j];
        }
        update<OPT>(S, p, G[j], m, v);
        P[j] = p;
        if constexpr (kMoments) {
          M[j] = m;
          V[j] = v;
        }
      }
    }
  }
}

// Entries in the kernel argument block. XCD: XCD-contiguous workgroup numbering (used for
// launches holding one tensor entry).
template <Opt OPT, bool XCD>
__global__ __launch_bounds__(kOptBlock<OPT>) void opt_kernel(OptArgs A) {
  constexpr bool kMoments = OPT != Opt::Sgd;
  const uint32_t b = XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  // the last entry whose first workgroup is at or before b (uniform binary search)
  int i = 0, hi = A.count - 1;
  while (i < hi) {
    const int mid = (i + hi + 1) >> 1;
    if (A.first_block[mid] <= b) i = mid;
    else hi = mid - 1;
  }
  update_entry<OPT>(A.s, A.p[i], A.g[i], kMoments ? A.m[i] : nullptr, kMoments ? A.v[i] : nullptr,
                    A.n[i], (A.vec_mask >> i & 1u) != 0, b - A.first_block[i]);
}

// Entries in device memory (a call with more than kGroup of them).
template <Opt OPT>
__global__ __launch_bounds__(kOptBlock<OPT>) void opt_table_kernel(OptScalars S,
                                                                   const OptEntry *__restrict__ T,
                                                                   int count) {
  constexpr bool kMoments = OPT != Opt::Sgd;
  const uint32_t b = blockIdx.x;
  int i = 0, hi = count - 1;
  while (i < hi) {
    const int mid = (i + hi + 1) >> 1;
    if (T[mid].first_block <= b) i = mid;
    else hi = mid - 1;
  }
  const OptEntry &E = T[i];
  update_entry<OPT>(S, E.p, E.g, kMoments ? E.m : nullptr, kMoments ? E.v : nullptr, E.n,
                    E.vec != 0, b - E.first_block);
}

bool f32_param(const Tensor *t) { return t && t->grad && t->dtype == FLOAT32 && t->grad->data && t->data; }

// The device copy of the last table of more than kGroup entries (see OptTableCache).
std::mutex g_table_mu;
OptTableCache g_table;

// The table in device memory, uploaded if it differs from the last one. The upload waits for the
// library stream (earlier launches may still read the old table, and the host vector must outlive
// the copy); it happens only when the parameter list changes.
const OptEntry *device_table(const std::vector<OptEntry> &e, const char *where) {
  return g_table.get(
      e,
      [&]() {
        if (hipStreamSynchronize(stream()) == hipSuccess) return true;
        report_error(where, "waiting for the library stream failed");
        return false;
      },
      [&](size_t n) -> OptEntry * {
        OptEntry *p = nullptr;
        if (hipMalloc(&p, n * sizeof(OptEntry)) == hipSuccess) return p;
        report_error(where, "allocation of the tensor table (%zu entries) failed", n);
        return nullptr;
      },
      [](OptEntry *p) { (void)hipFree(p); },
      [&](OptEntry *dst, const std::vector<OptEntry> &src) {
        if (hipMemcpyAsync(dst, src.data(), src.size() * sizeof(OptEntry),
                           hipMemcpyHostToDevice, stream()) == hipSuccess &&
            hipStreamSynchronize(stream()) == hipSuccess)
          return true;
        report_error(where, "upload of the tensor table failed");
        return false;
      });
}

// Launch OPT over parameters[0..count); m/v may be null for SGD. Every tensor's entries are
// collected first: up to kGroup of them run from the kernel argument block, more from a device
// table in one launch (or, during a graph capture, in launches of kGroup).
template <Opt OPT>
void launch_updates(OptArgs base, Tensor **params, Tensor **m, Tensor **v, int count,
                    const char *where) {
  constexpr int kBs = kOptBlock<OPT>;
  const uint64_t per_block = uint64_t(kBs) * kOptUnroll * 4;
  // a tensor longer than one launch's grid allows is updated as several entries
  const uint64_t max_piece = max_blocks(kBs) / 2 * per_block;
  std::vector<OptEntry> entries;
  for (int k = 0; k < count; ++k) {
    Tensor *t = params[k];
    if (!t || !t->grad) continue;  // the reference skips these (sgd.c:20-22, adam.c:53-55)
    if (!f32_param(t)) {
      report_error(where, "parameter %d is not a float32 tensor with a gradient buffer", k);
      continue;
    }
    float *P = static_cast<float *>(t->data);
    const float *G = static_cast<const float *>(t->grad->data);
    float *M = m ? static_cast<float *>(m[k]->data) : nullptr;
    float *V = v ? static_cast<float *>(v[k]->data) : nullptr;
    bool aligned = aligned16(P) && aligned16(G);
    if (m) aligned = aligned && aligned16(M) && aligned16(V);
    add_tensor(entries, P, G, M, V, numel(t), aligned, per_block, max_piece);
  }
  if (entries.empty()) return;

  // one launch from a device table: every workgroup number fits one grid
  const uint64_t total = total_blocks(entries);
  if (entries.size() > size_t(kGroup) && !capturing() && total <= max_blocks(kBs)) {
    std::vector<OptEntry> table = entries;
    number_entries(table);
    std::lock_guard<std::mutex> lk(g_table_mu);
    const OptEntry *T = device_table(table, where);
    if (!T) return;
    opt_table_kernel<OPT><<<unsigned(total), kBs, 0, stream()>>>(base.s, T, int(table.size()));
    return;
  }

  // launches of up to kGroup entries from the kernel argument block
  for (const OptLaunch &g : group_entries(entries, size_t(kGroup), max_blocks(kBs))) {
    OptArgs A = base;
    A.count = int(g.count);
    A.vec_mask = 0;
    uint32_t blocks = 0;
    for (size_t j = 0; j < g.count; ++j) {
      const OptEntry &e = entries[g.first + j];
      A.p[j] = e.p;
      A.g[j] = e.g;
      A.m[j] = e.m;
      A.v[j] = e.v;
      A.n[j] = e.n;
      A.first_block[j] = blocks;
      if (e.vec) A.vec_mask |= 1u << j;
      blocks += e.first_block;
    }
    A.first_block[g.count] = blocks;
    if (kOptXcd<OPT> && g.count == 1) opt_kernel<OPT, true><<<blocks, kBs, 0, stream()>>>(A);
    else opt_kernel<OPT, false><<<blocks, kBs, 0, stream()>>>(A);
  }
}

// Moment arrays this library allocated (freed by the release calls).
std::mutex g_own_mu;
std::unordered_set<Tensor **> g_owned;

// Zero-filled device tensors shaped like each parameter (the reference allocates them with
// init(..., zeros) on the first step: adam.c:29-46).
bool alloc_moments(Tensor **params, int count, Tensor ***m_out, Tensor ***v_out, const char *where) {
  Tensor **m = static_cast<Tensor **>(calloc(size_t(count), sizeof(Tensor *)));
  Tensor **v = static_cast<Tensor **>(calloc(size_t(count), sizeof(Tensor *)));
  if (!m || !v) {
    free(m);
    free(v);
    report_error(where, "host allocation of the moment arrays failed");
    return false;
  }
  for (int k = 0; k < count; ++k) {
    const Tensor *p = params[k];
    if (!p) continue;
    for (Tensor **arr : {m, v}) {
      Tensor *t = static_cast<Tensor *>(calloc(1, sizeof(Tensor)));
      const uint64_t n = numel(p);
      void *data = nullptr;
      if (!t || (n && hipMalloc(&data, n * sizeof(float)) != hipSuccess)) {
        free(t);
        report_error(where, "allocation of a moment tensor (%llu floats) failed",
                     (unsigned long long)n);
        continue;
      }
      t->data = data;
      t->ndim = p->ndim;
      uint64_t s = 1;
      for (uint64_t d = p->ndim; d-- > 0;) {
        t->shape[d] = p->shape[d];
        t->strides[d] = s;
        s *= p->shape[d];
      }
      t->dtype = FLOAT32;
      t->device = GPU;
      if (n) zeros_hip(t, n);  // a fill kernel (no memset node if a caller captures this)
      arr[k] = t;
    }
  }
  *m_out = m;
  *v_out = v;
  std::lock_guard<std::mutex> lk(g_own_mu);
  g_owned.insert(m);
  g_owned.insert(v);
  return true;
}

void release_moments(Tensor ***m, Tensor ***v, int count) {
  std::lock_guard<std::mutex> lk(g_own_mu);
  for (Tensor ***arr : {m, v}) {
    if (!*arr || !g_owned.count(*arr)) continue;
    for (int k = 0; k < count; ++k) {
      Tensor *t = (*arr)[k];
      if (!t) continue;
      if (t->data) (void)hipFree(t->data);
      free(t);
    }
    g_owned.erase(*arr);
    free(*arr);
    *arr = nullptr;
  }
}

// The reference's bias-corrected step, evaluated as its C source does: lr (float) times a double
// sqrt of a float, divided by a float, rounded once to float (adam.c:48-49).
float bias_corrected_lr(float lr, float beta1, float beta2, int t) {
  const double num = double(lr) * ::sqrt(double(1.0f - ::powf(beta2, float(t))));
  const double den = double(1.0f - ::powf(beta1, float(t)));
  return float(num / den);
}

template <class OptT, Opt OPT>
void adam_like_step(OptT *o, Tensor **params, int count, const char *where) {
  if (!o) {
    report_error(where, "optimizer is NULL");
    return;
  }
  if (!ensure_init()) return;
  o->t++;
  if (count <= 0 || !params) return;
  if (!o->m) {
    if (!alloc_moments(params, count, &o->m, &o->v, where)) return;
  }
  for (int k = 0; k < count; ++k) {
    if (!params[k] || !params[k]->grad) continue;
    if (!o->m[k] || !o->v[k] || numel(o->m[k]) != numel(params[k]) ||
        numel(o->v[k]) != numel(params[k])) {
      report_error(where, "moment tensors of parameter %d are missing or mis-sized", k);
      return;
    }
  }
  OptArgs A;
  memset(&A, 0, sizeof A);
  A.s.lr = bias_corrected_lr(o->lr, o->beta1, o->beta2, o->t);
  A.s.beta1 = o->beta1;
  A.s.beta2 = o->beta2;
  A.s.one_minus_beta1 = 1.0f - o->beta1;
  A.s.one_minus_beta2 = 1.0f - o->beta2;
  A.s.eps = o->epsilon;
  if constexpr (OPT == Opt::AdamW) A.s.decay = o->lr * o->weight_decay;
  launch_updates<OPT>(A, params, o->m, o->v, count, where);
  finish(where);
}

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

void sgd_step_hip(SGD *optimizer, Tensor **parameters, int num_parameters) {
  const char *where = "sgd_step_hip";
  if (!optimizer) {
    report_error(where, "SGD is NULL");
    return;
  }
  if (!ensure_init() || num_parameters <= 0 || !parameters) return;
  OptArgs A;
  memset(&A, 0, sizeof A);
  A.s.lr = optimizer->lr;
  launch_updates<Opt::Sgd>(A, parameters, nullptr, nullptr, num_parameters, where);
  finish(where);
}

void adam_step_hip(Adam *optimizer, Tensor **parameters, int num_parameters) {
  adam_like_step<Adam, Opt::Adam>(optimizer, parameters, num_parameters, "adam_step_hip");
}

void adamw_step_hip(AdamW *optimizer, Tensor **parameters, int num_parameters) {
  adam_like_step<AdamW, Opt::AdamW>(optimizer, parameters, num_parameters, "adamw_step_hip");
}

void zero_grad_hip(Tensor *t) {
  if (!t || !t->grad) return;
  if (!ensure_init()) return;
  zeros_hip(t->grad, numel(t->grad));
}

void plast_hip_adam_release(Adam *optimizer, int num_parameters) {
  if (optimizer) release_moments(&optimizer->m, &optimizer->v, num_parameters);
}

void plast_hip_adamw_release(AdamW *optimizer, int num_parameters) {
  if (optimizer) release_moments(&optimizer->m, &optimizer->v, num_parameters);
}

}  // extern "C"
