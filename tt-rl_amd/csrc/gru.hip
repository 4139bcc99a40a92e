// GRU cell arithmetic of one timestep of an unrolled GRU, forward and
// backward, fused per element (ttrl/engine/recurrent.py:39-168, PyTorch's
// gate order and placement of the reset gate):
//
//   r = sigmoid(gi_r + gh_r)   z = sigmoid(gi_z + gh_z)
//   n = tanh(gi_n + r * gh_n)  h' = (1 - z) * n + z * h
//
// gi = x W_ih + b_ih and gh = h W_hh + b_hh are [B][3H] rows produced by the
// GEMMs around these kernels (all timesteps' gi by one GEMM before the
// unroll).  The state entering step t is hin_t = h_{t-1} * (1 - done_t)
// (apply_done_mask, ttrl/engine/ops/functional.py:40-46); the forward kernel
// of step t writes h_t and hin_{t+1}.  The backward recomputes r, z, n from
// gi, gh and hin (the same expressions, so the same values) and writes the
// gate gradients d gi, d gh for the batched weight-gradient GEMMs and the
// direct part z * dh of d hin_t, to which a GEMM adds d gh W_hh^T.
#include "common.hpp"

#include <cmath>

namespace ttrl {
namespace {

constexpr int kGruThreads = 256;

__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

__device__ __forceinline__ float keep_f(const float* done, int b) { return done ? 1.f - done[b] : 1.f; }

__global__ __launch_bounds__(kGruThreads) void k_gru_mask(int B, int H, const float* __restrict__ h,
                                                          const float* __restrict__ done, float* __restrict__ out) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H);
    out[i] = h[i] * keep_f(done, b);
  }
}

__global__ __launch_bounds__(kGruThreads) void k_gru_step(int B, int H, const float* __restrict__ gi,
                                                          const float* __restrict__ gh,
                                                          const float* __restrict__ hin, float* __restrict__ hout,
                                                          const float* __restrict__ done_next,
                                                          float* __restrict__ hin_next) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H), j = int(i - long(b) * H);
    const float* gib = gi + long(b) * 3 * H;
    const float* ghb = gh + long(b) * 3 * H;
    const float r = sigmoid_f(gib[j] + ghb[j]);
    const float z = sigmoid_f(gib[H + j] + ghb[H + j]);
    const float c = tanhf(gib[2 * H + j] + r * ghb[2 * H + j]);
    const float h = hin[i];
    const float out = (1.f - z) * c + z * h;
    hout[i] = out;
    if (hin_next) hin_next[i] = out * keep_f(done_next, b);
  }
}

// dh_t = dout_t + (1 - done_{t+1}) * dhin_{t+1} (dout, dhin_next nullable).
__global__ __launch_bounds__(kGruThreads) void k_gru_step_bwd(int B, int H, const float* __restrict__ gi,
                                                              const float* __restrict__ gh,
                                                              const float* __restrict__ hin,
                                                              const float* __restrict__ dout,
                                                              const float* __restrict__ dhin_next,
                                                              const float* __restrict__ done_next,
                                                              float* __restrict__ dgi, float* __restrict__ dgh,
                                                              float* __restrict__ dhin) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H), j = int(i - long(b) * H);
    const float* gib = gi + long(b) * 3 * H;
    const float* ghb = gh + long(b) * 3 * H;
    const float r = sigmoid_f(gib[j] + ghb[j]);
    const float z = sigmoid_f(gib[H + j] + ghb[H + j]);
    const float hn = ghb[2 * H + j];
    const float c = tanhf(gib[2 * H + j] + r * hn);
    const float h = hin[i];
    float dh = dout ? dout[i] : 0.f;
    if (dhin_next) dh += keep_f(done_next, b) * dhin_next[i];
    const float dc = dh * (1.f - z);
    const float dz = dh * (h - c);
    const float dcp = dc * (1.f - c * c);
    const float dr = dcp * hn;
    const float drp = dr * (r * (1.f - r));
    const float dzp = dz * (z * (1.f - z));
    float* dgib = dgi + long(b) * 3 * H;
    float* dghb = dgh + long(b) * 3 * H;
    dgib[j] = drp;
    dgib[H + j] = dzp;
    dgib[2 * H + j] = dcp;
    dghb[j] = drp;
    dghb[H + j] = dzp;
    dghb[2 * H + j] = dcp * r;
    dhin[i] = dh * z;
  }
}

unsigned grid_for(long n) {
  long g = (n + kGruThreads - 1) / kGruThreads;
  return unsigned(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_gru_mask(ttrl_ctx* ctx, int B, int H, const float* h, const float* done, float* out) {
  TTRL_REQUIRE(ctx && h && out, "ttrl_gru_mask: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_mask: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_mask, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, h, done,
                     out);
  return check_launch("ttrl_gru_mask");
}

int ttrl_gru_step(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin, float* hout,
                  const float* done_next, float* hin_next) {
  TTRL_REQUIRE(ctx && gi && gh && hin && hout, "ttrl_gru_step: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_step: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_step, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, gi, gh, hin,
                     hout, done_next, hin_next);
  return check_launch("ttrl_gru_step");
}

int ttrl_gru_step_backward(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin,
                           const float* dout, const float* dhin_next, const float* done_next, float* dgi, float* dgh,
                           float* dhin) {
  TTRL_REQUIRE(ctx && gi && gh && hin && dgi && dgh && dhin, "ttrl_gru_step_backward: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_step_backward: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_step_bwd, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, gi, gh,
                     hin, dout, dhin_next, done_next, dgi, dgh, dhin);
  return check_launch("ttrl_gru_step_backward");
}

}  // extern "C"
