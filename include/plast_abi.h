/*
 * plast_abi.h — the data structures that cross plast's op-dispatch boundary.
 *
 * Every struct here is byte-for-byte layout compatible with the reference library's own
 * definition, so a `Tensor *` built by the reference (Python bindings, C model API, scheduler)
 * can be handed straight to this library's HIP entry points, and vice versa:
 *
 *   Tensor        include/core/tensor.h:20-30
 *   KernelParams  include/core/definitions.h:19-23
 *   Arena / ArenaBlock / DEVICE   include/core/arena.h:16-28
 *   Op, ForwardKernel, BackwardKernel, OP_TYPE   include/core/op.h:5-44
 *   Node          include/core/node.h:5-14
 *   DAG           include/core/graph.h:7-13
 *   SGD / Adam / AdamW   include/optimizers/{sgd.h:5-7, adam.h:5-15, adamw.h:5-16}
 *
 * tests/test_abi.py compiles a translation unit that includes both this header and the reference
 * headers and static_asserts equal sizeof/offsetof for every field.
 *
 * Extensions (appended after the reference's last enumerator so every existing numeric value is
 * unchanged): DTYPE gains INT64 (argmax indices); OP_TYPE gains ARGMAX, FUSED_ELEMENTWISE,
 * SOFTMAX_CROSS_ENTROPY, SOFTMAX and LOG_SOFTMAX.
 */
#ifndef PLAST_ABI_H
#define PLAST_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t i32;
typedef int64_t i64;
typedef uint8_t u8;
typedef uint32_t u32;
typedef uint64_t u64;

/* Maximum tensor rank (include/core/definitions.h:17). */
#define PLAST_MAX_NDIM 8
/* `KernelParams.dim` value that selects a reduction over every element (reduce_ops.c:69). */
#define PLAST_DIM_ALL (PLAST_MAX_NDIM + 1)

typedef enum DTYPE { INT32 = 0, FLOAT32 = 1, INT64 = 2 } DTYPE;

/* Device tag. The reference's second value is spelled CUDA; here it is simply "the GPU". */
typedef enum DEVICE { CPU = 0, GPU = 1 } DEVICE;

typedef struct ArenaBlock {
  struct ArenaBlock *prev;
  u64 capacity;
  u64 offset;
  void *buffer;
} ArenaBlock;

typedef struct Arena {
  ArenaBlock *current;
  DEVICE device;
} Arena;

/* Shape and strides are in elements, row-major. Metadata always lives in host memory; `data`
 * (and `grad->data`) is device memory when device == GPU. */
typedef struct Tensor {
  struct Tensor *grad;
  struct Node *creator;
  void *data;
  u64 shape[PLAST_MAX_NDIM];
  u64 strides[PLAST_MAX_NDIM];
  u64 ndim;
  DTYPE dtype;
  DEVICE device;
  bool requires_grad;
} Tensor;

/* dim: reduction/transposition axis (PLAST_DIM_ALL = every element); keepdim: 0/1 (second
 * transpose axis for TRANSPOSE); fval: leaky-relu slope. FUSED_ELEMENTWISE carries a
 * `const PlastFusedTape *` in `dim`, the same way the reference's CONV2D node carries an Arena
 * pointer there (src/python/bindings.cpp:183-185). */
typedef struct KernelParams {
  u64 dim;
  u64 keepdim;
  float fval;
} KernelParams;

typedef void (*ForwardKernel)(const Tensor **inputs, Tensor *output, KernelParams params);
typedef void (*BackwardKernel)(Tensor **inputs, const Tensor *output, KernelParams params);

typedef enum OP_TYPE {
  ADD,
  SUB,
  MUL,
  DIV,
  MATMUL,
  LEAKY_RELU,
  LOG,
  EXP,
  ABS,
  NEG,
  SIN,
  COS,
  TAN,
  VIEW,
  TRANSPOSE,
  UNSQUEEZE,
  SQUEEZE,
  EXPAND,
  FLATTEN,
  BROADCAST,
  MEAN,
  MIN,
  MAX,
  SUM,
  CONV2D,
  MATMUL_RELU,
  MATMUL_BIAS_RELU,
  CONV_RELU,
  /* extensions */
  ARGMAX,
  FUSED_ELEMENTWISE,
  SOFTMAX_CROSS_ENTROPY,
  SOFTMAX,
  LOG_SOFTMAX,
  PLAST_NUM_OP_TYPES
} OP_TYPE;

/* Slot names keep the reference's field order; the second and fourth slots are the GPU slots. */
typedef struct Op {
  ForwardKernel cpu_forward;
  ForwardKernel gpu_forward;
  BackwardKernel cpu_backward;
  BackwardKernel gpu_backward;
} Op;

typedef struct Node {
  Tensor **inputs;
  Tensor *output;
  Op op;
  OP_TYPE op_type;
  int num_inputs;
  bool visited;
  bool on_stack;
  KernelParams params;
} Node;

typedef struct DAG {
  Node **nodes;
  u32 count;
  u32 capacity;
  bool changed;
  Arena *arena;
} DAG;

/* Optimizer state, layout-identical to include/optimizers/sgd.h:5-7, adam.h:5-15 and
 * adamw.h:5-16. `m` and `v` are the per-parameter moment tensors, allocated on the first step. */
typedef struct SGD {
  float lr;
} SGD;

typedef struct Adam {
  float lr;
  float beta1;
  float beta2;
  float epsilon;
  int t;
  Tensor **m;
  Tensor **v;
  Arena *data_arena;
  Arena *optimizer_arena;
} Adam;

typedef struct AdamW {
  float lr;
  float beta1;
  float beta2;
  float epsilon;
  float weight_decay;
  int t;
  Tensor **m;
  Tensor **v;
  Arena *data_arena;
  Arena *optimizer_arena;
} AdamW;

#ifdef __cplusplus
}
#endif

#endif /* PLAST_ABI_H */
