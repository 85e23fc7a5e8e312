// pack.hip — strided <-> contiguous copies: the tensor pack used before handing a view to code
// that reads flat buffers (cuda_tensor_pack_init / cuda_tensor_pack_release,
// src/kernels/cuda/cuda_pack.cu:28-96), and host transfers of strided tensors (the bindings'
// numpy() / copy_from_numpy, src/python/bindings.cpp:81-151).
//
// The copy is the elementwise engine with an identity body: host-side dimension collapsing, float4
// streaming where the view is contiguous along its innermost axis, the LDS-tiled transpose for a
// view whose unit-stride axis is not the innermost (a permuted tensor), SGPR-resident strides
// otherwise. Elements are moved as 4-byte words, so float and int32 copy bit for bit; an 8-byte
// element (int64) is two words, i.e. one more axis of extent 2 and stride 1.
#include <mutex>
#include <vector>

#include "ew_impl.hpp"

namespace plast {
namespace {

// Pack buffers are pooled: hipMalloc/hipFree of a large buffer costs far more than the gather, and
// callers pack the same shapes over and over (every matmul call packs its strided operands).
// Released buffers wait here; a request takes the smallest one that fits within 2x. The pool
// keeps at most kPoolBytes; work that reads a pack must be ordered before its release (it is when
// it runs on the library stream, where the next pack into a reused buffer also runs).
constexpr uint64_t kPoolBytes = uint64_t(8) << 30;
struct PoolBuf {
  void *ptr;
  uint64_t bytes;
};
std::mutex g_pool_mu;
std::vector<PoolBuf> g_pool;

void *pool_take(uint64_t bytes) {
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    int best = -1;
    for (int i = 0; i < int(g_pool.size()); ++i)
      if (g_pool[i].bytes >= bytes && g_pool[i].bytes <= 2 * bytes &&
          (best < 0 || g_pool[i].bytes < g_pool[best].bytes))
        best = i;
    if (best >= 0) {
      void *p = g_pool[best].ptr;
      g_pool.erase(g_pool.begin() + best);
      return p;
    }
  }
  void *p = nullptr;
  return hipMalloc(&p, bytes) == hipSuccess ? p : nullptr;
}

uint64_t alloc_size(void *p) {
  size_t bytes = 0;
  void *base = nullptr;
  return hipMemGetAddressRange(&base, &bytes, p) == hipSuccess ? uint64_t(bytes) : 0;
}

void pool_give(void *p) {
  std::vector<void *> drop;
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool.push_back(PoolBuf{p, alloc_size(p)});
    uint64_t total = 0;
    for (const PoolBuf &b : g_pool) total += b.bytes;
    while (total > kPoolBytes && !g_pool.empty()) {  // drop the oldest
      total -= g_pool.front().bytes;
      drop.push_back(g_pool.front().ptr);
      g_pool.erase(g_pool.begin());
    }
  }
  if (!drop.empty()) {
    (void)hipStreamSynchronize(stream());
    for (void *q : drop) (void)hipFree(q);
  }
}

struct CopyBody : ScalarBody<CopyBody> {
  static constexpr int NIN = 1;
  __device__ __forceinline__ float eval(const float *v, uint64_t) const { return v[0]; }
};

uint64_t elem_words(DTYPE d) { return d == INT64 ? 2 : 1; }

// Space over tensor t viewed as 4-byte words: operand `strided` follows t's strides, the other
// operand is the contiguous image. False when t has more axes than a space can hold.
bool word_space(const Tensor *t, Space &s, int strided) {
  const uint64_t w = elem_words(t->dtype);
  const int rank = int(t->ndim) + (w > 1 ? 1 : 0);
  if (rank > kMaxRank) return false;
  s.rank = rank;
  s.nops = 2;
  int64_t contig = 1;
  if (w > 1) {
    s.shape[rank - 1] = w;
    s.st[0][rank - 1] = s.st[1][rank - 1] = 1;
    contig = int64_t(w);
  }
  for (int d = int(t->ndim) - 1; d >= 0; --d) {
    s.shape[d] = t->shape[d];
    const int64_t own = t->shape[d] == 1 ? 0 : int64_t(t->strides[d]) * int64_t(w);
    s.st[strided][d] = own;
    s.st[1 - strided][d] = t->shape[d] == 1 ? 0 : contig;
    contig *= int64_t(t->shape[d]);
  }
  return true;
}

// Strided tensor t -> contiguous buffer dst (numel(t) elements).
bool pack_into(const Tensor *t, void *dst, const char *where) {
  Space s;
  if (!word_space(t, s, 0)) {
    report_error(where, "rank %llu is too large", (unsigned long long)t->ndim);
    return false;
  }
  const void *ins[1] = {t->data};
  return launch_elementwise(CopyBody{}, ins, dst, s, where);
}

// Contiguous buffer src -> strided tensor t. Every element of t must have its own address.
bool unpack_from(const void *src, Tensor *t, const char *where) {
  for (uint64_t d = 0; d < t->ndim; ++d)
    if (t->shape[d] > 1 && t->strides[d] == 0) {
      report_error(where, "destination has a broadcast (stride 0) axis %llu",
                   (unsigned long long)d);
      return false;
    }
  Space s;
  if (!word_space(t, s, 1)) {
    report_error(where, "rank %llu is too large", (unsigned long long)t->ndim);
    return false;
  }
  const void *ins[1] = {src};
  return launch_elementwise(CopyBody{}, ins, t->data, s, where);
}

uint64_t tensor_bytes(const Tensor *t) { return numel(t) * 4 * elem_words(t->dtype); }

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

void hip_tensor_pack_init(HipTensorPack *p, const Tensor *t) {
  const char *where = "hip_tensor_pack_init";
  p->data = nullptr;
  p->_d_buf = nullptr;
  if (!t || !ensure_init()) return;
  if (contiguous(t)) {
    p->data = t->data;
    return;
  }
  const uint64_t bytes = tensor_bytes(t);
  if (bytes == 0) return;
  p->_d_buf = pool_take(bytes);
  if (!p->_d_buf) {
    report_error(where, "device allocation of %llu bytes failed", (unsigned long long)bytes);
    return;
  }
  if (!pack_into(t, p->_d_buf, where)) {
    pool_give(p->_d_buf);
    p->_d_buf = nullptr;
    return;
  }
  p->data = p->_d_buf;
  finish(where);
}

void hip_tensor_pack_release(HipTensorPack *p) {
  if (!p) return;
  if (p->_d_buf) pool_give(p->_d_buf);
  p->_d_buf = nullptr;
  p->data = nullptr;
}

void plast_hip_pack_trim(void) {
  std::vector<PoolBuf> drop;
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    drop.swap(g_pool);
  }
  if (drop.empty() || !ensure_init()) return;
  (void)hipStreamSynchronize(stream());
  for (const PoolBuf &b : drop) (void)hipFree(b.ptr);
}

void *plast_hip_host_alloc(u64 bytes) {
  if (!ensure_init()) return nullptr;
  void *p = nullptr;
  if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
    report_error("plast_hip_host_alloc", "hipHostMalloc(%llu) failed", (unsigned long long)bytes);
    return nullptr;
  }
  return p;
}

void plast_hip_host_free(void *p) {
  if (p) (void)hipHostFree(p);
}

int plast_hip_tensor_to_host(const Tensor *t, void *dst) {
  const char *where = "plast_hip_tensor_to_host";
  if (!t || !dst || !ensure_init()) return -1;
  const int errors_before = plast_hip_error_count();
  const uint64_t bytes = tensor_bytes(t);
  if (bytes == 0) return 0;
  const void *src = t->data;
  if (!contiguous(t)) {
    void *stage = workspace(bytes, 2);
    if (!stage || !pack_into(t, stage, where)) return -1;
    src = stage;
  }
  if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream()) != hipSuccess ||
      hipStreamSynchronize(stream()) != hipSuccess) {
    report_error(where, "device-to-host copy of %llu bytes failed", (unsigned long long)bytes);
    return -1;
  }
  return plast_hip_error_count() != errors_before ? -1 : 0;
}

int plast_hip_tensor_from_host(Tensor *t, const void *src) {
  const char *where = "plast_hip_tensor_from_host";
  if (!t || !src || !ensure_init()) return -1;
  const int errors_before = plast_hip_error_count();
  const uint64_t bytes = tensor_bytes(t);
  if (bytes == 0) return 0;
  const bool direct = contiguous(t);
  void *dst = direct ? t->data : workspace(bytes, 2);
  if (!dst) return -1;
  if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()) != hipSuccess) {
    report_error(where, "host-to-device copy of %llu bytes failed", (unsigned long long)bytes);
    return -1;
  }
  if (!direct && !unpack_from(dst, t, where)) return -1;
  // the caller may release its host buffer on return
  if (hipStreamSynchronize(stream()) != hipSuccess) {
    report_error(where, "synchronize failed");
    return -1;
  }
  return plast_hip_error_count() != errors_before ? -1 : 0;
}

}  // extern "C"
