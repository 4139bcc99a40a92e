// Optimizer-side kernels over flat parameter arenas: the fused Adam step
// with a device-resident update counter and the sum of squared gradients,
// a standalone sum of squares, the Polyak blend and a fill kernel.
//
// Reference semantics:
//   Adam (S = m/(1-b1), V = v/(1-b2) storage, fused scalars)
//                          ttrl/engine/optim/adam.py:93-134, ttrl/engine/optim/scalars.py:13-27
//   grad_sq_device         ttrl/algos/grads.py:46-60
//   Polyak blend           ttrl/algos/sac/targets.py:45-52
//
// The Adam scalars depend on the update count t.  The count lives on the
// device, so one captured graph replays correctly for every t: the update
// kernel reads t_old and uses t = t_old + 1, and the finishing kernel (one
// block, after every update block has run) stores t and the reduced
// sum of squares.  All reductions are fixed-order.
#include "common.hpp"

#include <cmath>
#include <cstdint>
#include <mutex>

namespace ttrl {

constexpr int kOptThreads = 256;
constexpr int kOptMaxBlocks = 1024;

float* ctx_workspace(ttrl_ctx* ctx, long* floats);

// Block `blk` of `nblk` of one Adam update: its grid-stride share of the
// range and its partial sum of g^2 into partials[blk].  The same code serves
// a single-range launch and a range of a multi-range launch, so both give
// the same bits.
__device__ __forceinline__ void adam_block(float* __restrict__ p, const float* __restrict__ g,
                                           float* __restrict__ S, float* __restrict__ V, long n,
                                           const int* __restrict__ step, float lr, float b1, float b2, float eps,
                                           float wd, float* __restrict__ partials, int blk, int nblk) {
  __shared__ float sc[2];
  __shared__ float red[kOptThreads / 64];
  if (threadIdx.x == 0) {
    const int t = *step + 1;
    const double bc1 = 1.0 - pow(double(b1), double(t));
    const double bc2 = 1.0 - pow(double(b2), double(t));
    const double c = sqrt((1.0 - double(b2)) / bc2);
    sc[0] = float(double(lr) * (1.0 - double(b1)) / bc1 / c);
    sc[1] = float(double(eps) / c);
  }
  __syncthreads();
  const float alpha_t = sc[0], eps_t = sc[1];
  float gsq = 0.f;
  const long n4 = n / 4;
  const long stride = long(nblk) * kOptThreads;
  for (long i = blk * long(kOptThreads) + threadIdx.x; i < n4; i += stride) {
    f32x4 pv = reinterpret_cast<f32x4*>(p)[i];
    const f32x4 gv = reinterpret_cast<const f32x4*>(g)[i];
    f32x4 sv = reinterpret_cast<f32x4*>(S)[i];
    f32x4 vv = reinterpret_cast<f32x4*>(V)[i];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float graw = gv[q];
      gsq += graw * graw;
      const float gg = wd != 0.f ? graw + wd * pv[q] : graw;
      vv[q] = gg * gg + b2 * vv[q];
      sv[q] = gg + b1 * sv[q];
      const float upd = (sv[q] / (sqrtf(vv[q]) + eps_t)) * alpha_t;
      pv[q] = pv[q] - upd;
    }
    reinterpret_cast<f32x4*>(p)[i] = pv;
    reinterpret_cast<f32x4*>(S)[i] = sv;
    reinterpret_cast<f32x4*>(V)[i] = vv;
  }
  // Tail (n % 4) handled by block 0.
  if (blk == 0) {
    for (long i = n4 * 4 + threadIdx.x; i < n; i += kOptThreads) {
      const float graw = g[i];
      gsq += graw * graw;
      const float gg = wd != 0.f ? graw + wd * p[i] : graw;
      V[i] = gg * gg + b2 * V[i];
      S[i] = gg + b1 * S[i];
      p[i] = p[i] - (S[i] / (sqrtf(V[i]) + eps_t)) * alpha_t;
    }
  }
  const float tot = block_sum<kOptThreads>(gsq, red);
  if (threadIdx.x == 0) partials[blk] = tot;
}

__global__ __launch_bounds__(kOptThreads) void k_adam(float* __restrict__ p, const float* __restrict__ g,
                                                      float* __restrict__ S, float* __restrict__ V, long n,
                                                      const int* __restrict__ step, float lr, float b1, float b2,
                                                      float eps, float wd, float* __restrict__ partials) {
  adam_block(p, g, S, V, n, step, lr, b1, b2, eps, wd, partials, int(blockIdx.x), int(gridDim.x));
}

// Up to kMultiRanges deferred Adam ranges and a Polyak blend in one launch:
// blocks [r.block0, r.block0 + r.blocks) run range r (r.blocks = the grid a
// single-range launch of it uses), the rest the blend.
constexpr int kMultiRanges = 4;
struct AdamRange {
  float* p;
  const float* g;
  float* S;
  float* V;
  long n;
  const int* step;
  float lr, b1, b2, eps, wd;
  float* partials;
  int block0, blocks;
};
struct AdamMulti {
  AdamRange r[kMultiRanges];
  int nr;
  float* pd;
  const float* ps;
  long pn;
  float keep, tau;
  int pblock0, pblocks;
};
__global__ __launch_bounds__(kOptThreads) void k_adam_multi(AdamMulti a) {
  const int b = int(blockIdx.x);
#pragma unroll
  for (int i = 0; i < kMultiRanges; ++i) {
    if (i >= a.nr) break;
    const AdamRange& r = a.r[i];
    if (b >= r.block0 && b < r.block0 + r.blocks) {
      adam_block(r.p, r.g, r.S, r.V, r.n, r.step, r.lr, r.b1, r.b2, r.eps, r.wd, r.partials, b - r.block0,
                 r.blocks);
      return;
    }
  }
  const long stride = long(a.pblocks) * kOptThreads;
  for (long i = (b - a.pblock0) * long(kOptThreads) + threadIdx.x; i < a.pn; i += stride)
    a.pd[i] = a.pd[i] * a.keep + a.ps[i] * a.tau;
}

// The finishes of up to kAdamSlots deferred steps, one block each: the
// partials of slot f.slot[b] summed as k_finish sums them.
struct FinishSlots {
  const float* parts[kAdamSlots];
  int count[kAdamSlots];
  int* step[kAdamSlots];
  float* out[kAdamSlots];
  int accumulate[kAdamSlots];
};
__global__ __launch_bounds__(kOptThreads) void k_finish_slots(FinishSlots f) {
  __shared__ float red[kOptThreads / 64];
  const int b = int(blockIdx.x);
  float s = 0.f;
  for (int i = threadIdx.x; i < f.count[b]; i += kOptThreads) s += f.parts[b][i];
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) {
    if (f.out[b]) *f.out[b] = f.accumulate[b] ? *f.out[b] + tot : tot;
    *f.step[b] = *f.step[b] + 1;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_finish(const float* __restrict__ partials, int nparts,
                                                        int* __restrict__ step, float* __restrict__ out,
                                                        int accumulate) {
  __shared__ float red[kOptThreads / 64];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kOptThreads) s += partials[i];
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) {
    if (out) *out = accumulate ? *out + tot : tot;
    if (step) *step = *step + 1;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_sumsq(const float* __restrict__ x, long n,
                                                       float* __restrict__ partials) {
  __shared__ float red[kOptThreads / 64];
  float s = 0.f;
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    s += v * v;
  }
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kOptThreads) void k_polyak(float* __restrict__ dst, const float* __restrict__ src,
                                                        long n, float keep, float tau) {
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) {
    dst[i] = dst[i] * keep + src[i] * tau;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_fill(float* __restrict__ p, long n, float v) {
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void k_fill_i32(int* __restrict__ p, long n, int v) {
  for (long i = blockIdx.x * long(blockDim.x) + threadIdx.x; i < n; i += long(gridDim.x) * blockDim.x) p[i] = v;
}

inline unsigned grid_for(long n, long per_thread = 1) {
  long b = (n / per_thread + kOptThreads - 1) / kOptThreads;
  if (b < 1) b = 1;
  if (b > kOptMaxBlocks) b = kOptMaxBlocks;
  return unsigned(b);
}

// Scratch of the allocation-free Adam step: one partial sum of squared
// gradients per workgroup of k_adam.  A launch uses at most kOptMaxBlocks
// workgroups, so this bounds nothing about n.  Each GPU holds its own copy;
// host code reaches it only through the address hipGetSymbolAddress gives
// for the current device (static_scratch_for), never through the name.
constexpr int kStaticScratchFloats = kOptMaxBlocks;
__device__ __align__(256) float scratch[kStaticScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, resolved once per
// device (with that device current) and kept.
int static_scratch_for(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice (ttrl_adam_step_static)");
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(TTRL_EINVAL, "ttrl_adam_step_static: device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_error(e, "hipGetSymbolAddress (ttrl_adam_step_static scratch)");
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return TTRL_OK;
}

int check_adam_args(const float* p, const float* g, const float* m_s, const float* v_s, long n, const int* step,
                    float lr, float beta1, float beta2, float eps, float weight_decay, const char* name) {
  TTRL_REQUIRE(p && g && m_s && v_s && step, "%s: null argument", name);
  TTRL_REQUIRE(n > 0, "%s: empty parameter range", name);
  TTRL_REQUIRE(lr > 0.f && eps > 0.f && beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f &&
                   weight_decay >= 0.f,
               "%s: bad hyper-parameters", name);
  TTRL_REQUIRE(((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                 reinterpret_cast<uintptr_t>(m_s) | reinterpret_cast<uintptr_t>(v_s)) & 15) == 0,
               "%s: buffers must be 16-byte aligned", name);
  return TTRL_OK;
}

}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_adam_step(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n, int* step, float lr,
                   float beta1, float beta2, float eps, float weight_decay, float* grad_sq, int accumulate_grad_sq) {
  TTRL_REQUIRE(ctx, "ttrl_adam_step: null ctx");
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step");
  if (rc) return rc;
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const unsigned blocks = grid_for(n, 4);
  TTRL_REQUIRE(wsf >= long(blocks), "ttrl_adam_step: workspace too small");
  hipStream_t st = stream_of(ctx);
  hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(kOptThreads), 0, st, p, g, m_s, v_s, n, step, lr, beta1, beta2,
                     eps, weight_decay, ws);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), step, grad_sq,
                     accumulate_grad_sq);
  return check_launch("ttrl_adam_step");
}

int ttrl_adam_step_static(void* stream, float* p, const float* g, float* m_s, float* v_s, long n, int* step,
                          float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                          int accumulate_grad_sq) {
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step_static");
  if (rc) return rc;
  const unsigned blocks = grid_for(n, 4);
  TTRL_REQUIRE(blocks <= unsigned(kStaticScratchFloats),
               "ttrl_adam_step_static: %u workgroups exceed the %d partial sums of the static scratch", blocks,
               kStaticScratchFloats);
  float* partials = nullptr;
  rc = static_scratch_for(&partials);
  if (rc) return rc;
  // Every workgroup writes its own partial before k_finish reads them, so
  // nothing in the scratch needs clearing between calls.
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(kOptThreads), 0, st, p, g, m_s, v_s, n, step, lr, beta1, beta2,
                     eps, weight_decay, partials);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, partials, int(blocks), step, grad_sq,
                     accumulate_grad_sq);
  return check_launch("ttrl_adam_step_static");
}

int ttrl_adam_step_deferred(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n,
                            const int* step, float lr, float beta1, float beta2, float eps, float weight_decay,
                            int slot) {
  TTRL_REQUIRE(ctx, "ttrl_adam_step_deferred: null ctx");
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step_deferred");
  if (rc) return rc;
  TTRL_REQUIRE(slot >= 0 && slot < kAdamSlots, "ttrl_adam_step_deferred: slot %d outside [0, %d)", slot,
               kAdamSlots);
  static_assert(kAdamSlotFloats >= kOptMaxBlocks, "a slot holds one launch's partials");
  hipLaunchKernelGGL(k_adam, dim3(grid_for(n, 4)), dim3(kOptThreads), 0, stream_of(ctx), p, g, m_s, v_s, n, step,
                     lr, beta1, beta2, eps, weight_decay, ctx_adam_partials(ctx) + long(slot) * kAdamSlotFloats);
  return check_launch("ttrl_adam_step_deferred");
}

int ttrl_adam_multi(ttrl_ctx* ctx, int nranges, const ttrl_adam_range* ranges, float* polyak_dst,
                    const float* polyak_src, long polyak_n, float tau) {
  TTRL_REQUIRE(ctx, "ttrl_adam_multi: null ctx");
  TTRL_REQUIRE(nranges >= 0 && nranges <= kMultiRanges && (nranges == 0 || ranges),
               "ttrl_adam_multi: %d ranges outside [0, %d]", nranges, kMultiRanges);
  TTRL_REQUIRE(polyak_n >= 0 && (polyak_n == 0 || (polyak_dst && polyak_src)),
               "ttrl_adam_multi: null Polyak buffer");
  TTRL_REQUIRE(tau >= 0.f && tau <= 1.f, "ttrl_adam_multi: tau must be in [0, 1]");
  AdamMulti a{};
  a.nr = nranges;
  int blocks = 0;
  bool slot_used[kAdamSlots] = {};
  for (int i = 0; i < nranges; ++i) {
    const ttrl_adam_range& r = ranges[i];
    int rc = check_adam_args(r.p, r.g, r.m_s, r.v_s, r.n, r.step, r.lr, r.beta1, r.beta2, r.eps, r.weight_decay,
                             "ttrl_adam_multi");
    if (rc) return rc;
    TTRL_REQUIRE(r.slot >= 0 && r.slot < kAdamSlots && !slot_used[r.slot],
                 "ttrl_adam_multi: range %d: slot %d outside [0, %d) or taken twice", i, r.slot, kAdamSlots);
    slot_used[r.slot] = true;
    const int nb = int(grid_for(r.n, 4));
    a.r[i] = AdamRange{r.p, r.g, r.m_s, r.v_s, r.n, r.step, r.lr, r.beta1, r.beta2, r.eps, r.weight_decay,
                       ctx_adam_partials(ctx) + long(r.slot) * kAdamSlotFloats, blocks, nb};
    blocks += nb;
  }
  a.pd = polyak_dst;
  a.ps = polyak_src;
  a.pn = polyak_n;
  a.keep = 1.f - tau;
  a.tau = tau;
  a.pblock0 = blocks;
  a.pblocks = polyak_n > 0 ? int(grid_for(polyak_n)) : 0;
  blocks += a.pblocks;
  if (blocks == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_adam_multi, dim3(unsigned(blocks)), dim3(kOptThreads), 0, stream_of(ctx), a);
  return check_launch("ttrl_adam_multi");
}

int ttrl_adam_finish_slots(ttrl_ctx* ctx, int n, const ttrl_adam_finish* f) {
  TTRL_REQUIRE(ctx && (n == 0 || f), "ttrl_adam_finish_slots: null argument");
  TTRL_REQUIRE(n >= 0 && n <= kAdamSlots, "ttrl_adam_finish_slots: %d finishes outside [0, %d]", n, kAdamSlots);
  if (n == 0) return TTRL_OK;
  FinishSlots fs{};
  for (int i = 0; i < n; ++i) {
    TTRL_REQUIRE(f[i].slot >= 0 && f[i].slot < kAdamSlots, "ttrl_adam_finish_slots: slot %d outside [0, %d)",
                 f[i].slot, kAdamSlots);
    TTRL_REQUIRE(f[i].n > 0 && f[i].step, "ttrl_adam_finish_slots: finish %d: empty range or null step", i);
    fs.parts[i] = ctx_adam_partials(ctx) + long(f[i].slot) * kAdamSlotFloats;
    fs.count[i] = int(grid_for(f[i].n, 4));
    fs.step[i] = f[i].step;
    fs.out[i] = f[i].grad_sq;
    fs.accumulate[i] = f[i].accumulate;
  }
  hipLaunchKernelGGL(k_finish_slots, dim3(unsigned(n)), dim3(kOptThreads), 0, stream_of(ctx), fs);
  return check_launch("ttrl_adam_finish_slots");
}

int ttrl_sum_squares(ttrl_ctx* ctx, const float* x, long n, float* out, int accumulate) {
  TTRL_REQUIRE(ctx && x && out, "ttrl_sum_squares: null argument");
  TTRL_REQUIRE(n >= 0, "ttrl_sum_squares: negative length");
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const unsigned blocks = grid_for(n > 0 ? n : 1, 4);
  hipStream_t st = stream_of(ctx);
  hipLaunchKernelGGL(k_sumsq, dim3(blocks), dim3(kOptThreads), 0, st, x, n, ws);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), (int*)nullptr, out,
                     accumulate);
  return check_launch("ttrl_sum_squares");
}

int ttrl_polyak(ttrl_ctx* ctx, float* dst, const float* src, long n, float tau) {
  TTRL_REQUIRE(ctx && dst && src, "ttrl_polyak: null argument");
  TTRL_REQUIRE(tau >= 0.f && tau <= 1.f, "ttrl_polyak: tau must be in [0, 1]");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_polyak, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, src, n, 1.f - tau,
                     tau);
  return check_launch("ttrl_polyak");
}

int ttrl_fill_f32(ttrl_ctx* ctx, float* dst, float value, long n) {
  TTRL_REQUIRE(ctx && (dst || n == 0), "ttrl_fill_f32: null argument");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_fill, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, n, value);
  return check_launch("ttrl_fill_f32");
}

int ttrl_fill_i32(ttrl_ctx* ctx, int* dst, int value, long n) {
  TTRL_REQUIRE(ctx && (dst || n == 0), "ttrl_fill_i32: null argument");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, n, value);
  return check_launch("ttrl_fill_i32");
}

}  // extern "C"
