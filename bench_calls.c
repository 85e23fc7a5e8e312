/* Host timing loop for bench.py: makes C-ABI entry-point calls back to back from C, the way the
 * reference's executor calls its op slots (src/core/node.c:22-32 from src/core/graph.c:57-65), so
 * that a per-call figure carries no Python cost. The entry points come in as function pointers:
 * this file links nothing but libc and runs no GPU code of its own. Built by
 * plast_amd/build.py:build_bench_helper into bench_calls.so. */
#define _POSIX_C_SOURCE 199309L
#include <time.h>

#include "plast_abi.h"

typedef struct BenchCall {
  ForwardKernel fn;
  const Tensor **inputs;
  Tensor *output;
  KernelParams params;
} BenchCall;

/* Makes `rounds` rounds of the calls calls[0..ncalls), then calls sync() (the library's
 * plast_hip_synchronize, so queued GPU work is drained). Returns the wall-clock microseconds of the
 * whole loop, sync included, or -1 if sync() fails or errors() (plast_hip_error_count) is non-zero
 * afterwards. The caller drains the stream before the call. */
double bench_call_loop(const BenchCall *calls, int ncalls, int rounds, int (*sync)(void),
                       int (*errors)(void)) {
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int r = 0; r < rounds; ++r)
    for (int i = 0; i < ncalls; ++i) calls[i].fn(calls[i].inputs, calls[i].output, calls[i].params);
  const int rc = sync();
  clock_gettime(CLOCK_MONOTONIC, &t1);
  if (rc != 0 || errors() != 0) return -1.0;
  return (double)(t1.tv_sec - t0.tv_sec) * 1e6 + (double)(t1.tv_nsec - t0.tv_nsec) / 1e3;
}
