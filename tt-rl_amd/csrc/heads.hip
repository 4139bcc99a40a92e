// Fused loss heads.  Each is one workgroup over the batch: the per-sample
// arithmetic of the reference's composed ops, the batch means as fixed-order
// block reductions, and the gradient of the loss with respect to the network
// outputs written in the same pass, so the backward needs no extra launch.
//
// DQN head (ttrl/algos/dqn/losses.py:77-140): Q(s,a) by one-hot gather
// (ttrl/engine/ops/functional.py:126-132), double-DQN argmax with the first
// index winning ties (ttrl/engine/ops/reduce.py:82-99), n-step target
// r + discounts*(1-done)*Q'(s', a*) (ttrl/engine/ops/functional.py:40-46),
// Huber through the clipped-quadratic identity (functional.py:56-69),
// importance weights, mean; dL/dQ = onehot * w/B * clip(e, -delta, delta).
//
// SAC heads (ttrl/algos/sac/losses.py:25-94, ttrl/algos/sac/policy.py:30-40,
// ttrl/algos/gaussian.py:55-117): reparameterised tanh-squashed Gaussian
// sample and log-density in its stable forms, its backward, the twin-critic
// soft target and loss, and the actor and temperature losses.
#include "common.hpp"

#include <cmath>

namespace ttrl {

constexpr int kHeadThreads = 256;
constexpr float kLog2 = 0.69314718055994530942f;
constexpr float kLog2Pi = 1.83787706640934548356f;

__device__ inline float relu_f(float x) { return x > 0.f ? x : 0.f; }

// softplus(x) = relu(x) + log(1 + exp(-|x|))  (ttrl/algos/gaussian.py:55-62)
__device__ inline float softplus_f(float x) { return relu_f(x) + logf(expf(-fabsf(x)) + 1.f); }

// min(a, b) through the relu identity a - relu(a - b) (ttrl/engine/ops/select.py:39-47):
// the gradient goes to b iff a > b.
__device__ inline float min_relu(float a, float b) { return a - relu_f(a - b); }

__global__ __launch_bounds__(kHeadThreads) void k_dqn_loss(
    int B, int A, const float* __restrict__ q, const float* __restrict__ qsel, const float* __restrict__ qval,
    const float* __restrict__ onehot, const float* __restrict__ rewards, const float* __restrict__ dones,
    const float* __restrict__ discounts, const float* __restrict__ weights, float delta, float* __restrict__ loss,
    float* __restrict__ mean_q, float* __restrict__ td_abs, float* __restrict__ dq, float* __restrict__ next_act,
    float* __restrict__ td_target) {
  __shared__ float red[kHeadThreads / 64];
  const float invB = 1.f / float(B);
  float sum_h = 0.f, sum_p = 0.f;
  for (int b = threadIdx.x; b < B; b += kHeadThreads) {
    const float* qb = q + long(b) * A;
    const float* ob = onehot + long(b) * A;
    float pred = 0.f;
    for (int a = 0; a < A; ++a) pred += qb[a] * ob[a];
    const float* sb = qsel + long(b) * A;
    int best = 0;
    float bv = sb[0];
    for (int a = 1; a < A; ++a)
      if (sb[a] > bv) {
        bv = sb[a];
        best = a;
      }
    const float nv = qval[long(b) * A + best];
    const float y = rewards[b] + (nv * (1.f - dones[b])) * discounts[b];
    const float e = pred - y;
    const float ae = fabsf(e);
    const float quad = ae - relu_f(ae - delta);
    const float lin = ae - quad;
    const float h = (quad * quad) * 0.5f + lin * delta;
    const float w = weights ? weights[b] : 1.f;
    sum_h += weights ? h * w : h;
    sum_p += pred;
    if (td_abs) td_abs[b] = ae;
    if (next_act) next_act[b] = float(best);
    if (td_target) td_target[b] = y;
    const float clip = fminf(fmaxf(e, -delta), delta);
    const float gscale = (weights ? w * invB : invB) * clip;
    for (int a = 0; a < A; ++a) dq[long(b) * A + a] = ob[a] * gscale;
  }
  const float th = block_sum<kHeadThreads>(sum_h, red);
  const float tp = block_sum<kHeadThreads>(sum_p, red);
  if (threadIdx.x == 0) {
    *loss = th * invB;
    if (mean_q) *mean_q = tp * invB;
  }
}

// head = [mean | log_std] per row (log_std already clamped).
__global__ __launch_bounds__(kHeadThreads) void k_sac_sample(int B, int d, const float* __restrict__ head,
                                                             const float* __restrict__ noise,
                                                             const float* __restrict__ centre,
                                                             const float* __restrict__ half_width, float log_det,
                                                             float* __restrict__ action, float* __restrict__ logp,
                                                             float* __restrict__ u_out) {
  for (int b = blockIdx.x * kHeadThreads + threadIdx.x; b < B; b += gridDim.x * kHeadThreads) {
    const float* hb = head + long(b) * 2 * d;
    float normal = 0.f, corr = 0.f;
    for (int i = 0; i < d; ++i) {
      const float mu = hb[i], ls = hb[d + i];
      const float sigma = expf(ls);
      const float u = mu + sigma * noise[long(b) * d + i];
      const float z = (u - mu) / sigma;
      normal += (z * z) * -0.5f - ls;
      corr += ((kLog2 - u) - softplus_f(u * -2.f)) * 2.f;
      const float t = tanhf(u);
      action[long(b) * d + i] = t * half_width[i] + centre[i];
      if (u_out) u_out[long(b) * d + i] = u;
    }
    normal -= 0.5f * float(d) * kLog2Pi;
    logp[b] = (normal - corr) - log_det;
  }
}

// Backward of k_sac_sample to the head's [mean | log_std] outputs.
// g_action0 (+ g_action1): dL/d action; g_logp: dL/d logp per row.
__global__ __launch_bounds__(kHeadThreads) void k_sac_sample_bwd(
    int B, int d, const float* __restrict__ head, const float* __restrict__ noise, const float* __restrict__ u_in,
    const float* __restrict__ half_width, const float* __restrict__ g_action0, const float* __restrict__ g_action1,
    const float* __restrict__ g_logp, float lo, float hi, float* __restrict__ d_head, float beta) {
  for (int b = blockIdx.x * kHeadThreads + threadIdx.x; b < B; b += gridDim.x * kHeadThreads) {
    const float* hb = head + long(b) * 2 * d;
    const float glp = g_logp ? g_logp[b] : 0.f;
    for (int i = 0; i < d; ++i) {
      const float mu = hb[i], ls = hb[d + i];
      const float sigma = expf(ls);
      const float eps = noise[long(b) * d + i];
      const float u = u_in[long(b) * d + i];
      const float z = (u - mu) / sigma;
      const float t = tanhf(u);
      float ga = 0.f;
      if (g_action0) ga += g_action0[long(b) * d + i];
      if (g_action1) ga += g_action1[long(b) * d + i];
      // d logp / d u (explicit): -z/sigma from the Gaussian, +2 tanh(u) from
      // the squash correction; d logp / d mean (explicit) = z/sigma;
      // d logp / d log_std (explicit) = z^2 - 1.
      const float gu = ga * half_width[i] * (1.f - t * t) + glp * (2.f * t - z / sigma);
      const float gmu = gu + glp * (z / sigma);
      float gls = gu * (sigma * eps) + glp * (z * z - 1.f);
      gls = (ls > lo && ls < hi) ? gls : 0.f;
      float* dm = d_head + long(b) * 2 * d + i;
      float* dl = d_head + long(b) * 2 * d + d + i;
      *dm = beta != 0.f ? *dm * beta + gmu : gmu;
      *dl = beta != 0.f ? *dl * beta + gls : gls;
    }
  }
}

// Twin-critic soft target and loss.  q, qt: [2][B].
__global__ __launch_bounds__(kHeadThreads) void k_sac_critic_loss(
    int B, const float* __restrict__ q, const float* __restrict__ qt, const float* __restrict__ logp_next,
    const float* __restrict__ log_alpha, const float* __restrict__ rewards, const float* __restrict__ dones,
    const float* __restrict__ discounts, const float* __restrict__ weights, float* __restrict__ loss,
    float* __restrict__ q_target, float* __restrict__ dq, float* __restrict__ td_abs, float* __restrict__ alpha_out) {
  __shared__ float red[kHeadThreads / 64];
  const float alpha = expf(*log_alpha);
  const float invB = 1.f / float(B);
  float s1 = 0.f, s2 = 0.f;
  for (int b = threadIdx.x; b < B; b += kHeadThreads) {
    const float soft = min_relu(qt[b], qt[B + b]) - logp_next[b] * alpha;
    const float y = rewards[b] + (soft * (1.f - dones[b])) * discounts[b];
    const float e1 = q[b] - y, e2 = q[B + b] - y;
    const float w = weights ? weights[b] : 1.f;
    s1 += weights ? (e1 * e1) * w : e1 * e1;
    s2 += weights ? (e2 * e2) * w : e2 * e2;
    q_target[b] = y;
    const float gs = (weights ? w : 1.f) * (0.5f * invB) * 2.f;
    dq[b] = e1 * gs;
    dq[B + b] = e2 * gs;
    if (td_abs) td_abs[b] = (fabsf(e1) + fabsf(e2)) * 0.5f;
  }
  const float t1 = block_sum<kHeadThreads>(s1, red);
  const float t2 = block_sum<kHeadThreads>(s2, red);
  if (threadIdx.x == 0) {
    *loss = (t1 * invB + t2 * invB) * 0.5f;
    if (alpha_out) *alpha_out = alpha;
  }
}

// Actor loss mean(alpha*logp - min(q1, q2)) and the temperature loss
// -mean(log_alpha * (logp + target_entropy)), with their gradients.
__global__ __launch_bounds__(kHeadThreads) void k_sac_actor_loss(
    int B, const float* __restrict__ q, const float* __restrict__ logp, const float* __restrict__ log_alpha,
    float target_entropy, int learn_alpha, float* __restrict__ actor_loss, float* __restrict__ alpha_loss,
    float* __restrict__ dq, float* __restrict__ g_logp, float* __restrict__ d_log_alpha) {
  __shared__ float red[kHeadThreads / 64];
  const float la = *log_alpha;
  const float alpha = expf(la);
  const float invB = 1.f / float(B);
  float sa = 0.f, se = 0.f;
  for (int b = threadIdx.x; b < B; b += kHeadThreads) {
    const float q1 = q[b], q2 = q[B + b];
    const float lp = logp[b];
    sa += lp * alpha - min_relu(q1, q2);
    se += lp + target_entropy;
    const bool second = q1 - q2 > 0.f;
    dq[b] = second ? 0.f : -invB;
    dq[B + b] = second ? -invB : 0.f;
    g_logp[b] = alpha * invB;
  }
  const float ta = block_sum<kHeadThreads>(sa, red);
  const float te = block_sum<kHeadThreads>(se, red);
  if (threadIdx.x == 0) {
    *actor_loss = ta * invB;
    if (learn_alpha) {
      if (alpha_loss) *alpha_loss = (la * (te * invB)) * -1.f;
      if (d_log_alpha) *d_log_alpha = (te * invB) * -1.f;
    }
  }
}

inline unsigned rows_grid(int B) {
  unsigned g = unsigned((B + kHeadThreads - 1) / kHeadThreads);
  return g ? g : 1;
}

}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_dqn_loss(ttrl_ctx* ctx, int B, int A, const float* q, const float* q_next_select,
                  const float* q_next_value, const float* actions_onehot, const float* rewards, const float* dones,
                  const float* discounts, const float* is_weights, float delta, float* loss, float* mean_q,
                  float* td_abs, float* dq, float* next_actions, float* td_target) {
  TTRL_REQUIRE(ctx && q && q_next_select && q_next_value && actions_onehot && rewards && dones && discounts &&
                   loss && dq,
               "ttrl_dqn_loss: null argument");
  TTRL_REQUIRE(B > 0 && A > 0, "ttrl_dqn_loss: empty batch or action set");
  TTRL_REQUIRE(delta > 0.f, "ttrl_dqn_loss: huber delta must be > 0");
  hipLaunchKernelGGL(k_dqn_loss, dim3(1), dim3(kHeadThreads), 0, stream_of(ctx), B, A, q, q_next_select,
                     q_next_value, actions_onehot, rewards, dones, discounts, is_weights, delta, loss, mean_q, td_abs,
                     dq, next_actions, td_target);
  return check_launch("ttrl_dqn_loss");
}

int ttrl_sac_sample(ttrl_ctx* ctx, int B, int d, const float* head, const float* noise, const float* centre,
                    const float* half_width, float log_det, float* action, float* logp, float* u_out) {
  TTRL_REQUIRE(ctx && head && noise && centre && half_width && action && logp, "ttrl_sac_sample: null argument");
  TTRL_REQUIRE(B > 0 && d > 0, "ttrl_sac_sample: empty batch");
  hipLaunchKernelGGL(k_sac_sample, dim3(rows_grid(B)), dim3(kHeadThreads), 0, stream_of(ctx), B, d, head, noise,
                     centre, half_width, log_det, action, logp, u_out);
  return check_launch("ttrl_sac_sample");
}

int ttrl_sac_sample_backward(ttrl_ctx* ctx, int B, int d, const float* head, const float* noise, const float* u,
                             const float* half_width, const float* g_action0, const float* g_action1,
                             const float* g_logp, float log_std_min, float log_std_max, float* d_head, float beta) {
  TTRL_REQUIRE(ctx && head && noise && u && half_width && d_head, "ttrl_sac_sample_backward: null argument");
  TTRL_REQUIRE(B > 0 && d > 0, "ttrl_sac_sample_backward: empty batch");
  hipLaunchKernelGGL(k_sac_sample_bwd, dim3(rows_grid(B)), dim3(kHeadThreads), 0, stream_of(ctx), B, d, head,
                     noise, u, half_width, g_action0, g_action1, g_logp, log_std_min, log_std_max, d_head, beta);
  return check_launch("ttrl_sac_sample_backward");
}

int ttrl_sac_critic_loss(ttrl_ctx* ctx, int B, const float* q, const float* q_next_target, const float* logp_next,
                         const float* log_alpha, const float* rewards, const float* dones, const float* discounts,
                         const float* is_weights, float* loss, float* q_target, float* dq, float* td_abs,
                         float* alpha_out) {
  TTRL_REQUIRE(ctx && q && q_next_target && logp_next && log_alpha && rewards && dones && discounts && loss &&
                   q_target && dq,
               "ttrl_sac_critic_loss: null argument");
  TTRL_REQUIRE(B > 0, "ttrl_sac_critic_loss: empty batch");
  hipLaunchKernelGGL(k_sac_critic_loss, dim3(1), dim3(kHeadThreads), 0, stream_of(ctx), B, q, q_next_target,
                     logp_next, log_alpha, rewards, dones, discounts, is_weights, loss, q_target, dq, td_abs,
                     alpha_out);
  return check_launch("ttrl_sac_critic_loss");
}

int ttrl_sac_actor_loss(ttrl_ctx* ctx, int B, const float* q, const float* logp, const float* log_alpha,
                        float target_entropy, int learn_alpha, float* actor_loss, float* alpha_loss, float* dq,
                        float* g_logp, float* d_log_alpha) {
  TTRL_REQUIRE(ctx && q && logp && log_alpha && actor_loss && dq && g_logp, "ttrl_sac_actor_loss: null argument");
  TTRL_REQUIRE(B > 0, "ttrl_sac_actor_loss: empty batch");
  hipLaunchKernelGGL(k_sac_actor_loss, dim3(1), dim3(kHeadThreads), 0, stream_of(ctx), B, q, logp, log_alpha,
                     target_entropy, learn_alpha, actor_loss, alpha_loss, dq, g_logp, d_log_alpha);
  return check_launch("ttrl_sac_actor_loss");
}

}  // extern "C"
