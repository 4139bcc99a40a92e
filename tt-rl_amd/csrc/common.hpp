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
// Gradient banks: split-K partials of weight gradients whose sum an
// optimizer step forms later (ttrl_conv2d_backward_deferred); a bank's
// contents live until the next deferred launch that names it.
constexpr int kGradBanks = 4;
constexpr long kGradBankFloats = 1L << 20;
float* ctx_grad_bank(ttrl_ctx* ctx, int bank);
// Converts a pending launch error into a status code.
int check_launch(const char* name);

inline unsigned ceil_div(long a, long b) { return unsigned((a + b - 1) / b); }

// Division by a runtime-constant positive divisor d with a multiply-high:
// q = (umulhi(n, m) + n) >> s, m = floor(2^32 (2^s - d) / d) + 1, s = ceil(log2 d)
// (exact for 0 <= n < 2^31).
struct FDiv {
  uint32_t m = 0, s = 0;
  int d = 1;
  __host__ void set(int divisor) {
    d = divisor;
    s = 0;
    while ((1u << s) < uint32_t(divisor)) ++s;
    const uint64_t two32 = uint64_t(1) << 32;
    m = uint32_t((two32 * ((uint64_t(1) << s) - uint64_t(divisor))) / uint64_t(divisor) + 1);
  }
  __device__ __forceinline__ int div(int n) const {
    const uint32_t hi = __umulhi(uint32_t(n), m);
    return int((uint64_t(hi) + uint32_t(n)) >> s);
  }
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Touches every 64-byte line of the first BYTES bytes of the kernel's
// argument segment with independent scalar loads and waits for them once,
// so the argument reads that follow hit the scalar cache instead of taking
// one memory round trip per line, one after another.
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  typedef __attribute__((address_space(4))) const uint32_t kword;
  kword* ka = (kword*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t t = 0;
#pragma unroll
  for (int o = 0; o < BYTES / 4; o += 16) t ^= ka[o];
  asm volatile("" ::"s"(t));
}

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
