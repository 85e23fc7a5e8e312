// runtime.hip — library state (device, stream, errors, workspace), the arena / fill hooks of the
// reference's L0/L1 layer, timing marks, deterministic input generation and the copy ceiling.
#include <cstdarg>
#include <cstdlib>
#include <vector>

#include "common.hpp"
#include "ws_ledger.hpp"

namespace plast {

namespace {
int g_device = 0;
bool g_inited = false;
bool g_sync = true;
bool g_capturing = false;  // the library stream is recording a graph
bool g_deterministic = false;  // results must not depend on timing (plast_hip_set_deterministic)
hipStream_t g_stream = nullptr;
int g_err_count = 0;
char g_err_msg[512] = "";
constexpr int kSlots = 3;
WorkspaceLedger<kSlots> g_ws;  // workspace slots, and the graphs captured over them
std::vector<void *> g_deferred_frees;  // arena_free_hip calls made while capturing
hipEvent_t g_t0 = nullptr, g_t1 = nullptr;
int g_cus = 256;  // compute units of the device (MI355X: 256), read at init
}  // namespace

void report_error(const char *where, const char *fmt, ...) {
  char body[400];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(body, sizeof body, fmt, ap);
  va_end(ap);
  snprintf(g_err_msg, sizeof g_err_msg, "plast_hip %s: %s", where, body);
  ++g_err_count;
  fprintf(stderr, "%s\n", g_err_msg);
}

bool ensure_init() {
  if (g_inited) return true;
  hipError_t e = hipSetDevice(g_device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&g_t0);
  if (e == hipSuccess) e = hipEventCreate(&g_t1);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, g_device);
  if (e != hipSuccess) {
    report_error("init", "device %d: %s", g_device, hipGetErrorString(e));
    return false;
  }
  g_inited = true;
  return true;
}

hipStream_t stream() {
  ensure_init();
  return g_stream;
}

int num_cus() { return g_cus > 0 ? g_cus : 1; }
bool capturing() { return g_capturing; }
bool deterministic() { return g_deterministic; }

int library_device() { return g_device; }

void finish(const char *where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    report_error(where, "kernel launch: %s", hipGetErrorString(e));
    return;
  }
  if (g_sync && !g_capturing) {
    e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) report_error(where, "synchronize: %s", hipGetErrorString(e));
  }
}

// Frees an outgrown workspace buffer once the work queued on the library stream (which may still
// read it) has finished.
static void release_workspace(void *p) {
  (void)hipStreamSynchronize(g_stream);
  (void)hipFree(p);
}

// Hands the buffers arena_free_hip was given during a capture to the ledger once the capture has
// ended: retired while a graph is alive (the capture's own graph may have been recorded using
// them, and its replays keep those addresses), freed at once otherwise.
static void release_deferred_frees() {
  for (void *p : g_deferred_frees) g_ws.free_after_capture(p, release_workspace);
  g_deferred_frees.clear();
}

void *workspace(size_t bytes, int slot) {
  if (slot < 0 || slot >= kSlots) return nullptr;
  if (bytes <= g_ws.bytes(slot)) return g_ws.buffer(slot);
  if (g_capturing) {
    report_error("workspace", "%zu bytes needed while capturing a graph: run the work once before "
                 "capturing it", bytes);
    return nullptr;
  }
  const size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
  return g_ws.grow(
      slot, bytes, want,
      [](size_t n) -> void * {
        void *p = nullptr;
        const hipError_t e = hipMalloc(&p, n);
        if (e != hipSuccess) {
          report_error("workspace", "hipMalloc(%zu): %s", n, hipGetErrorString(e));
          return nullptr;
        }
        return p;
      },
      release_workspace);
}

// ------------------------------------------------------------------------- metadata helpers

uint64_t numel(const Tensor *t) {
  uint64_t n = 1;
  for (uint64_t d = 0; d < t->ndim; ++d) n *= t->shape[d];
  return n;
}

bool same_shape(const Tensor *a, const Tensor *b) {
  if (a->ndim != b->ndim) return false;
  for (uint64_t d = 0; d < a->ndim; ++d)
    if (a->shape[d] != b->shape[d]) return false;
  return true;
}

bool contiguous(const Tensor *t) {
  uint64_t want = 1;
  for (uint64_t d = t->ndim; d-- > 0;) {
    if (t->shape[d] != 1 && t->strides[d] != want) return false;
    want *= t->shape[d];
  }
  return true;
}

void bcast_strides(const Tensor *t, const uint64_t *shape, int rank, int64_t *out) {
  int lead = rank - int(t->ndim);
  for (int d = 0; d < rank; ++d) {
    int s = d - lead;
    if (s < 0 || t->shape[s] == 1 || shape[d] == 1)
      out[d] = 0;
    else
      out[d] = int64_t(t->strides[s]);
  }
}

bool broadcast_shape(const Tensor *a, const Tensor *b, uint64_t *shape, int *rank) {
  int r = int(a->ndim > b->ndim ? a->ndim : b->ndim);
  for (int i = 0; i < r; ++i) {
    uint64_t x = i < int(a->ndim) ? a->shape[a->ndim - 1 - i] : 1;
    uint64_t y = i < int(b->ndim) ? b->shape[b->ndim - 1 - i] : 1;
    if (x != y && x != 1 && y != 1) return false;
    shape[r - 1 - i] = x > y ? x : y;
  }
  *rank = r;
  return true;
}

void collapse(Space &s) {
  // 1) drop size-1 axes (their strides never matter)
  int r = 0;
  for (int d = 0; d < s.rank; ++d) {
    if (s.shape[d] == 1) continue;
    s.shape[r] = s.shape[d];
    for (int k = 0; k < s.nops; ++k) s.st[k][r] = s.st[k][d];
    ++r;
  }
  s.rank = r;
  if (r == 0) {
    // a single element: keep one axis of extent 1 so kernels have something to iterate
    s.rank = 1;
    s.shape[0] = 1;
    for (int k = 0; k < s.nops; ++k) s.st[k][0] = 0;
    return;
  }
  // 2) merge axis d into axis d-1 when, for every operand, stepping d-1 equals shape[d] steps of d
  int w = 0;
  for (int d = 1; d < s.rank; ++d) {
    bool ok = true;
    for (int k = 0; k < s.nops && ok; ++k)
      ok = s.st[k][w] == s.st[k][d] * int64_t(s.shape[d]);
    if (ok) {
      s.shape[w] *= s.shape[d];
      for (int k = 0; k < s.nops; ++k) s.st[k][w] = s.st[k][d];
    } else {
      ++w;
      s.shape[w] = s.shape[d];
      for (int k = 0; k < s.nops; ++k) s.st[k][w] = s.st[k][d];
    }
  }
  s.rank = w + 1;
}

// ------------------------------------------------------------------------- kernels

namespace {

// Word-pattern fill, one uint4 per lane over [0, n4) plus the n % 4 tail words; workgroups are
// numbered XCD-contiguously (measured: a 1 GiB fill 5.85 -> 6.9 TB/s against a grid-stride loop).
__global__ __launch_bounds__(kBlock) void fill_u32_kernel(uint32_t *p, uint64_t n, uint32_t v) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const uint64_t n4 = n / 4;
  const uint64_t i = uint64_t(xcd_block(blockIdx.x, gridDim.x)) * kBlock + threadIdx.x;
  if (i < n4) reinterpret_cast<u4 *>(p)[i] = u4(v);
  if (i < n - n4 * 4) p[n4 * 4 + i] = v;
}

__global__ __launch_bounds__(kBlock) void fill_bytes_kernel(unsigned char *p, uint64_t n,
                                                            unsigned char v) {
  uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) p[i] = v;
}

void fill_u32(void *p, uint64_t n, uint32_t v, const char *where) {
  if (n == 0) return;
  if (!aligned16(p)) {
    // unaligned start: byte path is only correct for byte-uniform patterns
    report_error(where, "fill target %p is not 16-byte aligned", p);
    return;
  }
  // launches of at most max_blocks workgroups, each starting on a whole uint4
  const uint64_t max_words = max_blocks(kBlock) * kBlock * 4;
  for (uint64_t off = 0; off < n; off += max_words) {
    const uint64_t len = n - off < max_words ? n - off : max_words;
    const uint64_t blocks = (len / 4 + kBlock - 1) / kBlock;
    fill_u32_kernel<<<unsigned(blocks ? blocks : 1), kBlock, 0, stream()>>>(
        static_cast<uint32_t *>(p) + off, len, v);
  }
}

// splitmix64 finaliser: a bijective 64-bit mix, so (seed, i) -> hash is a counter-based generator.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hash_at(uint64_t seed, uint64_t i) {
  return mix64(seed * 0x9e3779b97f4a7c15ull + mix64(i + 0x632be59bd9b4e019ull));
}
// 24 random bits -> [0, 1) exactly representable
__device__ __forceinline__ float unit_float(uint64_t h) { return float(h >> 40) * 0x1p-24f; }

__global__ __launch_bounds__(kBlock) void uniform_kernel(float *p, uint64_t n, uint64_t seed,
                                                         float lo, float span) {
  uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    p[i] = lo + span * unit_float(hash_at(seed, i));
}

__global__ __launch_bounds__(kBlock) void normal_kernel(float *p, uint64_t n, uint64_t seed,
                                                        float mean, float sd) {
  uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    uint64_t h = hash_at(seed, i);
    float u1 = (float(h >> 40) + 1.0f) * 0x1p-24f;  // (0, 1]
    float u2 = float((h >> 16) & 0xffffffu) * 0x1p-24f;
    float r = sqrtf(-2.0f * logf(u1));
    p[i] = mean + sd * r * cospif(2.0f * u2);
  }
}

__global__ __launch_bounds__(kBlock) void randint_kernel(int32_t *p, uint64_t n, uint64_t seed,
                                                         int32_t lo, uint64_t span) {
  uint64_t stride = uint64_t(gridDim.x) * kBlock;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    p[i] = lo + int32_t(hash_at(seed, i) % span);
}

unsigned gen_blocks(uint64_t n) {
  uint64_t b = (n + kBlock - 1) / kBlock;
  if (b > 32768) b = 32768;
  return unsigned(b ? b : 1);
}

// Streaming copy: kCopyUnroll float4 per lane, whole tile per workgroup, nontemporal loads (the
// data is touched once), tail handled by a scalar guard.
constexpr int kCopyUnroll = PLAST_COPY_UNROLL;
__global__ __launch_bounds__(kBlock) void copy_kernel(f4 *__restrict__ dst,
                                                      const f4 *__restrict__ src, uint64_t n4) {
  const uint32_t b = PLAST_COPY_XCD ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  uint64_t base = uint64_t(b) * (kBlock * kCopyUnroll) + threadIdx.x;
  f4 v[kCopyUnroll];
#pragma unroll
  for (int k = 0; k < kCopyUnroll; ++k) {
    uint64_t i = base + uint64_t(k) * kBlock;
    if (i < n4) v[k] = __builtin_nontemporal_load(src + i);
  }
#pragma unroll
  for (int k = 0; k < kCopyUnroll; ++k) {
    uint64_t i = base + uint64_t(k) * kBlock;
    if (i < n4) store_stream<PLAST_COPY_NT_STORE>(v[k], dst + i);
  }
}

__global__ void copy_tail_kernel(float *dst, const float *src, uint64_t from, uint64_t n) {
  uint64_t i = from + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

}  // namespace
}  // namespace plast

using namespace plast;

extern "C" {

int plast_hip_init(int device) {
  if (g_inited && device != g_device) {
    report_error("plast_hip_init", "already initialised on device %d", g_device);
    return -1;
  }
  g_device = device;
  return ensure_init() ? 0 : -1;
}

void plast_hip_set_sync(int sync) { g_sync = sync != 0; }
void plast_hip_set_deterministic(int on) { g_deterministic = on != 0; }
int plast_hip_deterministic(void) { return g_deterministic ? 1 : 0; }

int plast_hip_capture_begin(void) {
  if (!ensure_init()) return -1;
  if (g_capturing) {
    report_error("plast_hip_capture_begin", "a capture is already open");
    return -1;
  }
  const hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    report_error("plast_hip_capture_begin", "%s", hipGetErrorString(e));
    return -1;
  }
  g_capturing = true;
  return 0;
}

void *plast_hip_capture_end(void) {
  if (!ensure_init()) return nullptr;
  if (!g_capturing) {
    report_error("plast_hip_capture_end", "no capture is open");
    return nullptr;
  }
  g_capturing = false;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &graph);
  if (e != hipSuccess || !graph) {
    release_deferred_frees();
    report_error("plast_hip_capture_end", "%s", hipGetErrorString(e));
    return nullptr;
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) {
    release_deferred_frees();
    report_error("plast_hip_capture_end", "instantiate: %s", hipGetErrorString(e));
    return nullptr;
  }
  g_ws.graph_created(exec);
  // buffers freed during the capture live as long as the graphs (this one included)
  release_deferred_frees();
  return exec;
}

int plast_hip_graph_launch(void *graph) {
  if (!ensure_init() || !graph) return -1;
  if (g_capturing) {
    report_error("plast_hip_graph_launch", "cannot launch a graph while capturing");
    return -1;
  }
  const int before = g_err_count;
  const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph), g_stream);
  if (e != hipSuccess) {
    report_error("plast_hip_graph_launch", "%s", hipGetErrorString(e));
    return -1;
  }
  finish("plast_hip_graph_launch");
  return g_err_count == before ? 0 : -1;
}

void plast_hip_graph_destroy(void *graph) {
  if (!graph) return;
  // a replay may still be running on the library stream
  if (g_inited) (void)hipStreamSynchronize(g_stream);
  (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
  // the last graph gone: free the workspace buffers that were outgrown while graphs held them
  g_ws.graph_destroyed(graph, release_workspace);
}

int plast_hip_workspace_reserve(int slot, uint64_t bytes) {
  if (!ensure_init()) return -1;
  if (slot < 0 || slot >= kSlots) {
    report_error("plast_hip_workspace_reserve", "slot %d is not one of 0..%d", slot, kSlots - 1);
    return -1;
  }
  return bytes == 0 || workspace(size_t(bytes), slot) ? 0 : -1;
}

uint64_t plast_hip_workspace_bytes(int slot) {
  return slot >= 0 && slot < kSlots ? uint64_t(g_ws.bytes(slot)) : 0;
}

int plast_hip_graphs_alive(void) { return int(g_ws.live_graphs()); }

int plast_hip_workspace_retired(void) { return int(g_ws.retired()); }

int plast_hip_synchronize(void) {
  if (!ensure_init()) return -1;
  hipError_t e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) {
    report_error("plast_hip_synchronize", "%s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}

void *plast_hip_stream(void) { return stream(); }
int plast_hip_error_count(void) { return g_err_count; }
const char *plast_hip_last_error(void) { return g_err_msg; }
void plast_hip_clear_error(void) {
  g_err_count = 0;
  g_err_msg[0] = 0;
}

int plast_hip_timer_begin(void) {
  if (!ensure_init()) return -1;
  return hipEventRecord(g_t0, g_stream) == hipSuccess ? 0 : -1;
}

float plast_hip_timer_end(void) {
  if (!ensure_init()) return -1.0f;
  if (hipEventRecord(g_t1, g_stream) != hipSuccess) return -1.0f;
  if (hipEventSynchronize(g_t1) != hipSuccess) return -1.0f;
  float ms = -1.0f;
  if (hipEventElapsedTime(&ms, g_t0, g_t1) != hipSuccess) return -1.0f;
  return ms;
}

// ---- arena hooks (include/core/arena_cuda.h:9-14)

void *arena_alloc_hip(u64 size) {
  if (!ensure_init()) exit(EXIT_FAILURE);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, size ? size : 1);
  if (e != hipSuccess) {
    report_error("arena_alloc_hip", "hipMalloc(%llu): %s", (unsigned long long)size,
                 hipGetErrorString(e));
    exit(EXIT_FAILURE);
  }
  return p;
}

void arena_free_hip(void *ptr) {
  if (!ptr || !ensure_init()) return;
  if (g_capturing) {
    // neither a wait nor hipFree may happen while the stream records (either would invalidate
    // the capture), and the captured kernels may use the buffer: it is freed with the last graph
    g_deferred_frees.push_back(ptr);
    return;
  }
  PLAST_HIP_TRY("arena_free_hip", hipStreamSynchronize(g_stream));
  PLAST_HIP_TRY("arena_free_hip", hipFree(ptr));
}

// A fill kernel rather than hipMemsetAsync, so a captured graph holds no memset node.
void arena_memset_hip(void *ptr, int value, u64 size) {
  if (!ensure_init() || size == 0) return;
  const unsigned char b = static_cast<unsigned char>(value);
  if (aligned16(ptr) && size % 4 == 0)
    fill_u32(ptr, size / 4, 0x01010101u * b, "arena_memset_hip");
  else
    fill_bytes_kernel<<<gen_blocks(size), kBlock, 0, stream()>>>(static_cast<unsigned char *>(ptr),
                                                                 size, b);
  finish("arena_memset_hip");
}

static void copy_async(void *dest, const void *src, u64 size, hipMemcpyKind kind,
                       const char *where) {
  if (!ensure_init() || size == 0) return;
  PLAST_HIP_TRY(where, hipMemcpyAsync(dest, src, size, kind, g_stream));
  // host buffers may be released by the caller right after return: always wait for H2D/D2H
  if (kind != hipMemcpyDeviceToDevice) {
    PLAST_HIP_TRY(where, hipStreamSynchronize(g_stream));
    return;
  }
  finish(where);
}

void arena_memcpy_h2d_hip(void *dest, const void *src, u64 size) {
  copy_async(dest, src, size, hipMemcpyHostToDevice, "arena_memcpy_h2d_hip");
}
void arena_memcpy_d2h_hip(void *dest, const void *src, u64 size) {
  copy_async(dest, src, size, hipMemcpyDeviceToHost, "arena_memcpy_d2h_hip");
}
void arena_memcpy_d2d_hip(void *dest, const void *src, u64 size) {
  copy_async(dest, src, size, hipMemcpyDeviceToDevice, "arena_memcpy_d2d_hip");
}

// ---- fill hooks (include/kernels/cuda/cuda_tensor_init.h:9-11)

static uint64_t dtype_bytes(DTYPE d) { return d == INT64 ? 8 : 4; }

void zeros_hip(Tensor *t, u64 num_elements) {
  if (!t || !ensure_init()) return;
  uint64_t bytes = num_elements * dtype_bytes(t->dtype);
  if (aligned16(t->data) && bytes % 4 == 0)
    fill_u32(t->data, bytes / 4, 0u, "zeros_hip");
  else
    fill_bytes_kernel<<<gen_blocks(bytes), kBlock, 0, stream()>>>(
        static_cast<unsigned char *>(t->data), bytes, 0);
  finish("zeros_hip");
}

static void ones_into(void *data, DTYPE dt, u64 n, const char *where) {
  if (dt == FLOAT32) {
    fill_u32(data, n, 0x3f800000u, where);
  } else if (dt == INT32) {
    fill_u32(data, n, 1u, where);
  } else {
    report_error(where, "unsupported dtype %d", int(dt));
    return;
  }
  finish(where);
}

void ones_hip(Tensor *t, u64 num_elements) {
  if (!t || !ensure_init()) return;
  ones_into(t->data, t->dtype, num_elements, "ones_hip");
}

void set_ones_grad_hip(Tensor *t) {
  if (!t || !t->grad || !ensure_init()) return;
  ones_into(t->grad->data, t->dtype, numel(t), "set_ones_grad_hip");
}

// ---- input generation and copy ceiling

void plast_hip_fill_uniform(float *dst, u64 n, u64 seed, float lo, float hi) {
  if (!ensure_init() || n == 0) return;
  uniform_kernel<<<gen_blocks(n), kBlock, 0, stream()>>>(dst, n, seed, lo, hi - lo);
  finish("plast_hip_fill_uniform");
}

void plast_hip_fill_normal(float *dst, u64 n, u64 seed, float mean, float std) {
  if (!ensure_init() || n == 0) return;
  normal_kernel<<<gen_blocks(n), kBlock, 0, stream()>>>(dst, n, seed, mean, std);
  finish("plast_hip_fill_normal");
}

void plast_hip_fill_randint(i32 *dst, u64 n, u64 seed, i32 lo, i32 hi) {
  if (!ensure_init() || n == 0) return;
  if (hi <= lo) {
    report_error("plast_hip_fill_randint", "empty range [%d, %d)", lo, hi);
    return;
  }
  randint_kernel<<<gen_blocks(n), kBlock, 0, stream()>>>(dst, n, seed, lo, uint64_t(hi - lo));
  finish("plast_hip_fill_randint");
}

void plast_hip_copy(float *dst, const float *src, u64 n) {
  if (!ensure_init() || n == 0) return;
  if (!aligned16(dst) || !aligned16(src)) {
    report_error("plast_hip_copy", "pointers must be 16-byte aligned");
    return;
  }
  const uint64_t n4 = n / 4;
  const uint64_t max_units = max_blocks(kBlock) * (kBlock * kCopyUnroll);
  for (uint64_t off = 0; off < n4; off += max_units) {
    const uint64_t len = n4 - off < max_units ? n4 - off : max_units;
    copy_kernel<<<ceil_div(len, kBlock * kCopyUnroll), kBlock, 0, stream()>>>(
        reinterpret_cast<f4 *>(dst) + off, reinterpret_cast<const f4 *>(src) + off, len);
  }
  if (n % 4) copy_tail_kernel<<<1, 4, 0, stream()>>>(dst, src, n4 * 4, n);
  finish("plast_hip_copy");
}

}  // extern "C"
