// Rollout-side device work of the PPO update, so the rollout stays resident
// in HBM and every minibatch step of an update replays one captured graph.
//
// gather    dst_s[i] = src_s[idx[c * stride + i]] for every source s (frames,
//           actions, old log-probs, advantages, returns, old values): the
//           minibatch assembly of RolloutBuffer.minibatches
//           (ttrl/buffers/rollout.py:239-282) by index from the resident
//           flattened rollout, the index table holding every epoch's
//           shuffled minibatches; c is a device step counter.
// step end  ring[c][:] = metrics, then c += 1: the per-minibatch metric
//           read of ttrl/algos/ppo/learn.py:94-112 kept on the device and
//           read once per update.
#include "common.hpp"

#include <algorithm>
#include <cstdint>

namespace ttrl {
namespace {

constexpr int kGatherMaxSrc = 8;
constexpr int kGatherThreads = 256;

struct GatherSrc {
  const unsigned char* src;
  unsigned char* dst;
  long row_bytes;
};

struct GatherArgs {
  GatherSrc s[kGatherMaxSrc];
  int n;             // rows gathered per step
  long rows;         // rows of every source
  const int* idx;    // index table
  long idx_len;      // entries in the table
  const int* counter;  // step counter (null: slot 0)
  int stride;        // table entries per step
};

// blockIdx.y picks the source; x-blocks stride over that source's rows in
// 16-byte units when its rows allow, else 4-byte units.
__global__ __launch_bounds__(kGatherThreads) void k_gather_rows(GatherArgs a) {
  const GatherSrc s = a.s[blockIdx.y];
  const long base = a.counter ? long(*a.counter) * a.stride : 0;
  const bool vec = (s.row_bytes & 15) == 0;
  const unsigned units = unsigned(vec ? s.row_bytes >> 4 : s.row_bytes >> 2);
  const unsigned total = unsigned(a.n) * units;  // < 2^31, checked on the host
  for (unsigned u = blockIdx.x * kGatherThreads + threadIdx.x; u < total; u += gridDim.x * kGatherThreads) {
    const unsigned i = u / units, k = u - i * units;
    const long slot = base + i;
    if (slot < 0 || slot >= a.idx_len) continue;
    const long r = a.idx[slot];
    if (r < 0 || r >= a.rows) continue;
    if (vec) {
      const uint4* src = reinterpret_cast<const uint4*>(s.src + r * s.row_bytes);
      uint4* dst = reinterpret_cast<uint4*>(s.dst + long(i) * s.row_bytes);
      dst[k] = src[k];
    } else {
      const unsigned* src = reinterpret_cast<const unsigned*>(s.src + r * s.row_bytes);
      unsigned* dst = reinterpret_cast<unsigned*>(s.dst + long(i) * s.row_bytes);
      dst[k] = src[k];
    }
  }
}

__global__ __launch_bounds__(64) void k_step_end(int* counter, const float* __restrict__ src, int n,
                                                 float* __restrict__ ring, int slots) {
  const int c = *counter;
  if (c >= 0 && c < slots)
    for (int i = threadIdx.x; i < n; i += 64) ring[long(c) * n + i] = src[i];
  __syncthreads();
  if (threadIdx.x == 0) *counter = c + 1;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_gather_rows(ttrl_ctx* ctx, int n, int nsrc, const void* const* src, void* const* dst, const long* row_bytes,
                     long rows, const int* idx, long idx_len, const int* counter, int stride) {
  TTRL_REQUIRE(ctx && src && dst && row_bytes && idx, "ttrl_gather_rows: null argument");
  TTRL_REQUIRE(nsrc >= 1 && nsrc <= kGatherMaxSrc, "ttrl_gather_rows: 1..%d sources, got %d", kGatherMaxSrc, nsrc);
  TTRL_REQUIRE(n >= 0 && rows >= 0 && idx_len >= 0 && stride >= 0, "ttrl_gather_rows: negative extent");
  if (n == 0) return TTRL_OK;
  GatherArgs a{};
  long most = 0;
  for (int s = 0; s < nsrc; ++s) {
    TTRL_REQUIRE(src[s] && dst[s], "ttrl_gather_rows: null pointer in source %d", s);
    TTRL_REQUIRE(row_bytes[s] > 0 && row_bytes[s] % 4 == 0, "ttrl_gather_rows: source %d rows of %ld bytes (need a "
                 "positive multiple of 4)", s, row_bytes[s]);
    const bool vec = row_bytes[s] % 16 == 0;
    if (vec)
      TTRL_REQUIRE((reinterpret_cast<uintptr_t>(src[s]) | reinterpret_cast<uintptr_t>(dst[s])) % 16 == 0,
                   "ttrl_gather_rows: source %d is not 16-byte aligned", s);
    else
      TTRL_REQUIRE((reinterpret_cast<uintptr_t>(src[s]) | reinterpret_cast<uintptr_t>(dst[s])) % 4 == 0,
                   "ttrl_gather_rows: source %d is not 4-byte aligned", s);
    a.s[s] = GatherSrc{static_cast<const unsigned char*>(src[s]), static_cast<unsigned char*>(dst[s]), row_bytes[s]};
    most = std::max(most, long(n) * (vec ? row_bytes[s] / 16 : row_bytes[s] / 4));
  }
  TTRL_REQUIRE(most < (1L << 31), "ttrl_gather_rows: %ld units in one source exceed 2^31", most);
  a.n = n;
  a.rows = rows;
  a.idx = idx;
  a.idx_len = idx_len;
  a.counter = counter;
  a.stride = stride;
  const long blocks = std::min<long>(4096, (most + kGatherThreads - 1) / kGatherThreads);
  hipLaunchKernelGGL(k_gather_rows, dim3(unsigned(blocks), unsigned(nsrc)), dim3(kGatherThreads), 0, stream_of(ctx),
                     a);
  return check_launch("ttrl_gather_rows");
}

int ttrl_step_end(ttrl_ctx* ctx, int* counter, const float* metrics, int n, float* ring, int slots) {
  TTRL_REQUIRE(ctx && counter, "ttrl_step_end: null argument");
  TTRL_REQUIRE(n >= 0 && slots >= 0 && (n == 0 || (metrics && ring)), "ttrl_step_end: bad metric ring");
  hipLaunchKernelGGL(k_step_end, dim3(1), dim3(64), 0, stream_of(ctx), counter, metrics, n, ring, slots);
  return check_launch("ttrl_step_end");
}

}  // extern "C"
