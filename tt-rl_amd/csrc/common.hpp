// Shared declarations for the libttrl_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ttrl_hip.h"

namespace ttrl {

// Sets the thread-local message returned by ttrl_last_error() and returns code.
int set_error(int code, const char* fmt, ...);
int hip_error(hipError_t e, const char* what);
hipStream_t stream_of(ttrl_ctx* ctx);
// Device words zeroed when the context opens, for kernels whose last
// workgroup finishes a reduction: kSyncCounters counters (each kernel that
// uses one leaves it at zero), then float partials (kSyncPartials).
constexpr int kSyncCounters = 64, kSyncPartials = 2 * 1024;
constexpr int kSyncDqnHead = 0;  // counter of ttrl_dqn_head
constexpr int kSyncDqnTail = 1;  // counter of ttrl_dqn_tail
unsigned* ctx_sync_words(ttrl_ctx* ctx);
// Partial sums of deferred Adam steps: kAdamSlots slots of kAdamSlotFloats,
// each kept from its step to its finish (ttrl_adam_finish_slots).
constexpr int kAdamSlots = 8, kAdamSlotFloats = 1024;
float* ctx_adam_partials(ttrl_ctx* ctx);
// Converts a pending launch error into a status code.
int check_launch(const char* name);

inline unsigned ceil_div(long a, long b) { return unsigned((a + b - 1) / b); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Deterministic (fixed-order) reduction of one float per thread over a
// block of NT threads.  Wavefronts of 64 fold with DPP-free shuffles, then
// wave partials are summed in wave order through LDS.  Every thread gets the
// total.
template <int NT>
__device__ inline float block_sum(float v, float* scratch /* >= NT/64 floats */) {
  static_assert(NT % 64 == 0, "block must be whole wavefronts");
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

}  // namespace ttrl

#define TTRL_REQUIRE(cond, ...)                                      \
  do {                                                               \
    if (!(cond)) return ::ttrl::set_error(TTRL_EINVAL, __VA_ARGS__); \
  } while (0)
