// Acting-step kernels: the last linear layer of an acting network fused with
// the per-lane decision the agent takes from it, so one acting step ends in
// one launch and a few bytes per lane go back to the host.
//
//   greedy    q = h W + b, action = first index of the row maximum
//             (ttrl/algos/dqn/agent.py:97-119 with
//             ttrl/engine/ops/reduce.py:82-99's tie rule)
//   squashed  [mean | clamp(log_std)] = h [W_mean | W_log_std] + b
//             (ttrl/nets/heads.py:65-93), then the tanh-squashed Gaussian
//             action and its log-density at host-drawn noise, or tanh(mean)
//             with logp 0 when deterministic (ttrl/algos/sac/policy.py:42-59,
//             ttrl/algos/gaussian.py:106-167); the learner's policy head
//             takes the same launch with the pre-squash u kept for its
//             backward (ttrl_sac_head_sample)
//
// One wavefront per lane row.  Lane l accumulates columns k = l, l+64, ... of
// the row's dot products with every output column; the 64 partial sums of
// each column are combined by an xor butterfly, which leaves the identical
// total in every lane, so any lane can take the decision.  The layer is tiny
// (K <= a few thousand, N <= 32): latency, not bandwidth or MFMA, bounds it.
#include "common.hpp"

#include <cmath>

namespace ttrl {
namespace {

constexpr int kActThreads = 256;  // four wavefronts, four lane rows per workgroup
constexpr int kActRows = kActThreads / 64;
constexpr int kActMaxN = 32;
constexpr int kActDepth = 4;  // columns per lane whose loads are in flight together
constexpr float kActLog2 = 0.69314718055994530942f;
constexpr float kActLog2Pi = 1.83787706640934548356f;

enum class ActMode { Greedy, Squashed };

struct ActArgs {
  int B, K, N, n1;  // N outputs per row: columns [0, n1) from W1/b1, [n1, N) from W2/b2
  const float* h;   // [B][K]
  const float* W1;  // [K][n1]
  const float* b1;  // [n1] or null
  const float* W2;  // [K][N - n1] or null when n1 == N
  const float* b2;  // [N - n1] or null
  float* q;         // greedy: [B][N] or null
  int* actions;     // greedy: [B]
  float lo, hi;     // squashed: log_std clamp
  const float* noise;  // squashed: [B][n1], unused when deterministic
  const float* centre;
  const float* half_width;
  float log_det;
  int deterministic;
  float* head;    // squashed: [B][2 n1] = [mean | clamped log_std] or null
  float* action;  // squashed: [B][n1]
  float* logp;    // squashed: [B]
  float* u;       // squashed: [B][n1] pre-squash sample, or null
};

__device__ __forceinline__ float softplus_act(float x) {
  const float r = x > 0.f ? x : 0.f;
  return r + logf(expf(-fabsf(x)) + 1.f);
}

template <ActMode MODE, int NP>
__global__ __launch_bounds__(kActThreads) void k_head_act(ActArgs a) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * kActRows + (threadIdx.x >> 6);
  if (b >= a.B) return;  // uniform per wavefront
  const int N = a.N, n1 = a.n1, n2 = a.N - a.n1;
  const float* hb = a.h + long(b) * a.K;
  float acc[NP];
#pragma unroll
  for (int n = 0; n < NP; ++n) acc[n] = 0.f;
  // The squashed sample's per-lane inputs (lane i < n1 owns action
  // dimension i, its mean and log_std biases among them), loaded ahead of
  // the dot products so their latency overlaps them.
  const int own = lane < n1 ? lane : n1 - 1;
  float noise_v = 0.f, half_v = 0.f, centre_v = 0.f, bias_mu = 0.f, bias_ls = 0.f;
  if constexpr (MODE == ActMode::Squashed) {
    if (!a.deterministic) noise_v = a.noise[long(b) * n1 + own];
    half_v = a.half_width[own];
    centre_v = a.centre[own];
    if (a.b1) bias_mu = a.b1[own];
    if (a.b2) bias_ls = a.b2[own];
  }
  // kActDepth columns per lane in flight at once: a round's loads are all
  // issued before its products, so a row pays one memory latency per
  // 64 * kActDepth columns; the columns past the last whole round follow
  // one at a time.  Each lane sums its columns in ascending k.
  int k0 = lane;
  for (; k0 + 64 * (kActDepth - 1) < a.K; k0 += 64 * kActDepth) {
    float x[kActDepth], w[kActDepth][NP];
#pragma unroll
    for (int r = 0; r < kActDepth; ++r) {
      const int k = k0 + 64 * r;
      x[r] = hb[k];
      const float* w1 = a.W1 + long(k) * n1;
      const float* w2 = a.W2 + long(k) * n2;
#pragma unroll
      for (int n = 0; n < NP; ++n) w[r][n] = n < n1 ? w1[n] : n < N ? w2[n - n1] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < kActDepth; ++r)
#pragma unroll
      for (int n = 0; n < NP; ++n)
        if (n < N) acc[n] += x[r] * w[r][n];
  }
  for (int k = k0; k < a.K; k += 64) {
    const float x = hb[k];
    const float* w1 = a.W1 + long(k) * n1;
    const float* w2 = a.W2 + long(k) * n2;
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      if (n < n1) acc[n] += x * w1[n];
      else if (n < N) acc[n] += x * w2[n - n1];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
#pragma unroll
    for (int n = 0; n < NP; ++n) acc[n] += __shfl_xor(acc[n], off);
  }
  // Every lane now holds the same sums.
  if constexpr (MODE == ActMode::Greedy) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      if (n < n1) acc[n] += a.b1 ? a.b1[n] : 0.f;
      else if (n < N) acc[n] += a.b2 ? a.b2[n - n1] : 0.f;
    }
    float mine = 0.f;
#pragma unroll
    for (int n = 0; n < NP; ++n) mine = lane == n ? acc[n] : mine;
    if (a.q && lane < N) a.q[long(b) * N + lane] = mine;
    if (lane == 0) {
      int best = 0;
      float bv = acc[0];
#pragma unroll
      for (int n = 1; n < NP; ++n)
        if (n < N && acc[n] > bv) {
          bv = acc[n];
          best = n;
        }
      a.actions[b] = best;
    }
  } else {
    // Lane i < d owns action dimension i.
    const int d = n1;
    float mu = 0.f, lsr = 0.f;
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      mu = lane == n ? acc[n] : mu;
      lsr = lane + d == n ? acc[n] : lsr;
    }
    mu += bias_mu;
    lsr += bias_ls;
    float normal = 0.f, corr = 0.f;
    if (lane < d) {
      const float ls = fminf(fmaxf(lsr, a.lo), a.hi);
      if (a.head) {
        a.head[long(b) * 2 * d + lane] = mu;
        a.head[long(b) * 2 * d + d + lane] = ls;
      }
      float t;
      if (a.deterministic) {
        t = tanhf(mu);
      } else {
        const float sigma = expf(ls);
        const float u = mu + sigma * noise_v;
        if (a.u) a.u[long(b) * d + lane] = u;
        const float z = (u - mu) / sigma;
        normal = (z * z) * -0.5f - ls;
        corr = ((kActLog2 - u) - softplus_act(u * -2.f)) * 2.f;
        t = tanhf(u);
      }
      a.action[long(b) * d + lane] = t * half_v + centre_v;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      normal += __shfl_xor(normal, off);
      corr += __shfl_xor(corr, off);
    }
    if (lane == 0)
      a.logp[b] = a.deterministic ? 0.f : ((normal - 0.5f * float(d) * kActLog2Pi) - corr) - a.log_det;
  }
}

template <ActMode MODE>
int launch_head_act(ttrl_ctx* ctx, const ActArgs& a, int width, const char* name) {
  const dim3 grid(unsigned((a.B + kActRows - 1) / kActRows));
  if (width <= 8)
    hipLaunchKernelGGL((k_head_act<MODE, 8>), grid, dim3(kActThreads), 0, stream_of(ctx), a);
  else if (width <= 16)
    hipLaunchKernelGGL((k_head_act<MODE, 16>), grid, dim3(kActThreads), 0, stream_of(ctx), a);
  else
    hipLaunchKernelGGL((k_head_act<MODE, 32>), grid, dim3(kActThreads), 0, stream_of(ctx), a);
  return check_launch(name);
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_q_act(ttrl_ctx* ctx, int B, int K, int A, const float* h, const float* W, const float* bias, float* q_out,
               int* actions) {
  TTRL_REQUIRE(ctx && h && W && actions, "ttrl_q_act: null argument");
  TTRL_REQUIRE(B >= 0 && K > 0 && A > 0, "ttrl_q_act: bad extents (B=%d, K=%d, A=%d)", B, K, A);
  TTRL_REQUIRE(A <= kActMaxN, "ttrl_q_act: at most %d actions, got %d", kActMaxN, A);
  if (B == 0) return TTRL_OK;
  ActArgs a{};
  a.B = B;
  a.K = K;
  a.N = A;
  a.n1 = A;
  a.h = h;
  a.W1 = W;
  a.b1 = bias;
  a.W2 = W;  // never read: every column comes from W1
  a.q = q_out;
  a.actions = actions;
  return launch_head_act<ActMode::Greedy>(ctx, a, A, "ttrl_q_act");
}

int ttrl_gaussian_act(ttrl_ctx* ctx, int B, int K, int d, const float* h, const float* W_mean, const float* b_mean,
                      const float* W_log_std, const float* b_log_std, float log_std_min, float log_std_max,
                      const float* noise, const float* centre, const float* half_width, float log_det,
                      int deterministic, float* head_out, float* action, float* logp) {
  TTRL_REQUIRE(ctx && h && W_mean && W_log_std && centre && half_width && action && logp,
               "ttrl_gaussian_act: null argument");
  TTRL_REQUIRE(deterministic || noise, "ttrl_gaussian_act: a stochastic step needs noise");
  TTRL_REQUIRE(B >= 0 && K > 0 && d > 0, "ttrl_gaussian_act: bad extents (B=%d, K=%d, d=%d)", B, K, d);
  TTRL_REQUIRE(2 * d <= kActMaxN, "ttrl_gaussian_act: at most %d action dimensions, got %d", kActMaxN / 2, d);
  TTRL_REQUIRE(log_std_min < log_std_max, "ttrl_gaussian_act: log_std_min must be < log_std_max");
  if (B == 0) return TTRL_OK;
  ActArgs a{};
  a.B = B;
  a.K = K;
  a.N = 2 * d;
  a.n1 = d;
  a.h = h;
  a.W1 = W_mean;
  a.b1 = b_mean;
  a.W2 = W_log_std;
  a.b2 = b_log_std;
  a.lo = log_std_min;
  a.hi = log_std_max;
  a.noise = noise;
  a.centre = centre;
  a.half_width = half_width;
  a.log_det = log_det;
  a.deterministic = deterministic ? 1 : 0;
  a.head = head_out;
  a.action = action;
  a.logp = logp;
  return launch_head_act<ActMode::Squashed>(ctx, a, 2 * d, "ttrl_gaussian_act");
}

int ttrl_sac_head_sample(ttrl_ctx* ctx, const ttrl_sac_head_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_sac_head_sample: null argument");
  TTRL_REQUIRE(d->x && d->W1 && d->W2 && d->noise && d->centre && d->half_width && d->head && d->action &&
                   d->logp && d->u,
               "ttrl_sac_head_sample: null buffer");
  TTRL_REQUIRE(d->rows >= 0 && d->K > 0 && d->d > 0, "ttrl_sac_head_sample: bad extents (rows=%d, K=%d, d=%d)",
               d->rows, d->K, d->d);
  TTRL_REQUIRE(2 * d->d <= kActMaxN, "ttrl_sac_head_sample: at most %d action dimensions, got %d", kActMaxN / 2,
               d->d);
  TTRL_REQUIRE(d->lo < d->hi, "ttrl_sac_head_sample: log_std_min must be < log_std_max");
  if (d->rows == 0) return TTRL_OK;
  ActArgs a{};
  a.B = d->rows;
  a.K = d->K;
  a.N = 2 * d->d;
  a.n1 = d->d;
  a.h = d->x;
  a.W1 = d->W1;
  a.b1 = d->b1;
  a.W2 = d->W2;
  a.b2 = d->b2;
  a.lo = d->lo;
  a.hi = d->hi;
  a.noise = d->noise;
  a.centre = d->centre;
  a.half_width = d->half_width;
  a.log_det = d->log_det;
  a.head = d->head;
  a.action = d->action;
  a.logp = d->logp;
  a.u = d->u;
  return launch_head_act<ActMode::Squashed>(ctx, a, 2 * d->d, "ttrl_sac_head_sample");
}

}  // extern "C"
