// PPO's per-rollout and per-minibatch elementwise work: the GAE reverse
// scan, advantage normalisation, the clipped-ratio objective with its
// log-softmax / entropy terms and their gradients, and a device-side global
// gradient-norm clip.
//
// Reference semantics:
//   GAE recursion, padding cut         ttrl/buffers/rollout.py:195-226
//   advantage normalisation            ttrl/buffers/rollout.py:269-270
//   clipped surrogate, value clip,
//   entropy bonus, masked mean         ttrl/algos/ppo/loss.py:27-83
//   log-prob and entropy of the head   ttrl/algos/ppo/policy.py:64-76,
//                                      ttrl/engine/ops/functional.py:160-178
//   minimum / maximum / clamp gates    ttrl/engine/ops/select.py:39-63
//   clip_grad_norm                     ttrl/algos/grads.py:13-43
#include "common.hpp"

#include <algorithm>
#include <cmath>

namespace ttrl {
namespace {

constexpr int kGaeLanes = 64;   // lanes (envs) per workgroup: one wavefront scans
constexpr int kGaeChunk = 64;   // time steps staged in LDS per pass
constexpr int kRedThreads = 1024;

// Deterministic block sum: a fixed tree over the block's threads.
template <int NT, class T>
__device__ inline T tree_sum(T v, T* sh) {
  const int t = threadIdx.x;
  sh[t] = v;
  __syncthreads();
#pragma unroll
  for (int s = NT / 2; s > 0; s >>= 1) {
    if (t < s) sh[t] += sh[t + s];
    __syncthreads();
  }
  const T r = sh[0];
  __syncthreads();
  return r;
}

// One thread per env lane walks t = T-1 .. 0; the block first stages a
// chunk of time steps of its 64 lanes in LDS with coalesced loads.  Every
// product is rounded as the reference's float32 numpy recursion rounds it
// (no contraction into fused multiply-adds).
__global__ __launch_bounds__(256) void k_gae(int T, int N, const float* __restrict__ rewards,
                                             const float* __restrict__ values, const float* __restrict__ dones,
                                             const float* __restrict__ valid, const float* __restrict__ last_values,
                                             float gamma, float gl, float* __restrict__ adv, float* __restrict__ ret) {
#pragma clang fp contract(off)
  // Rewards are overwritten in place by the advantages once read.
  __shared__ float r_s[kGaeChunk][kGaeLanes], v_s[kGaeChunk][kGaeLanes], d_s[kGaeChunk][kGaeLanes],
      m_s[kGaeChunk][kGaeLanes];
  const int n0 = blockIdx.x * kGaeLanes;
  const int lane = threadIdx.x;  // scanning thread when < kGaeLanes
  const int n = n0 + lane;
  float last_gae = 0.f;
  float next_v = (lane < kGaeLanes && n < N) ? last_values[n] : 0.f;
  for (int t1 = T; t1 > 0; t1 -= kGaeChunk) {
    const int t0 = t1 - kGaeChunk > 0 ? t1 - kGaeChunk : 0;
    const int rows = t1 - t0;
    __syncthreads();
    for (int i = threadIdx.x; i < rows * kGaeLanes; i += blockDim.x) {
      const int tt = i / kGaeLanes, c = i - tt * kGaeLanes;
      const bool in = n0 + c < N;
      const long idx = long(t0 + tt) * N + n0 + c;
      r_s[tt][c] = in ? rewards[idx] : 0.f;
      v_s[tt][c] = in ? values[idx] : 0.f;
      d_s[tt][c] = in ? dones[idx] : 0.f;
      m_s[tt][c] = (in && valid) ? valid[idx] : 1.f;
    }
    __syncthreads();
    if (lane < kGaeLanes) {
      for (int tt = rows - 1; tt >= 0; --tt) {
        const float not_done = 1.f - d_s[tt][lane];
        const float gv = gamma * next_v;
        const float delta = (r_s[tt][lane] + gv * not_done) - v_s[tt][lane];
        last_gae = delta + (gl * not_done) * last_gae;
        last_gae = last_gae * m_s[tt][lane];
        r_s[tt][lane] = last_gae;
        next_v = v_s[tt][lane];
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < rows * kGaeLanes; i += blockDim.x) {
      const int tt = i / kGaeLanes, c = i - tt * kGaeLanes;
      if (n0 + c >= N) continue;
      const long idx = long(t0 + tt) * N + n0 + c;
      adv[idx] = r_s[tt][c];
      ret[idx] = r_s[tt][c] + v_s[tt][c];
    }
  }
}

// (a - mean) / (std + eps) over the entries with valid > 0 (population
// std); entries with valid == 0 are written as 0.  One workgroup, two passes.
__global__ __launch_bounds__(kRedThreads) void k_adv_normalize(const float* __restrict__ a,
                                                               const float* __restrict__ valid, long n, float eps,
                                                               float* __restrict__ out, float* __restrict__ stats) {
  __shared__ double sh[kRedThreads];
  double s = 0.0, c = 0.0;
  for (long i = threadIdx.x; i < n; i += kRedThreads) {
    const bool v = !valid || valid[i] > 0.f;
    s += v ? double(a[i]) : 0.0;
    c += v ? 1.0 : 0.0;
  }
  const double sum = tree_sum<kRedThreads>(s, sh);
  const double cnt = tree_sum<kRedThreads>(c, sh);
  const double mean = cnt > 0.0 ? sum / cnt : 0.0;
  double q = 0.0;
  for (long i = threadIdx.x; i < n; i += kRedThreads) {
    const bool v = !valid || valid[i] > 0.f;
    const double d = double(a[i]) - mean;
    q += v ? d * d : 0.0;
  }
  const double var = cnt > 0.0 ? tree_sum<kRedThreads>(q, sh) / cnt : 0.0;
  const float meanf = float(mean), stdf = float(std::sqrt(var));
  const float denom = stdf + eps;
  for (long i = threadIdx.x; i < n; i += kRedThreads) {
    const bool v = !valid || valid[i] > 0.f;
    out[i] = v ? (a[i] - meanf) / denom : 0.f;
  }
  if (threadIdx.x == 0 && stats) {
    stats[0] = meanf;
    stats[1] = stdf;
  }
}

struct PpoCfg {
  int B, A;
  float clip, vclip, vcoef, ecoef;
  int ldz;   // row stride of logits / dlogits
  int ldv;   // element stride of values / dvalues
  int kl;    // also write out[4] = approx_kl = mean(expm1(r) - r), r = new_logp - old_logp
};

// The PPO objective for one minibatch in one workgroup: per row the
// log-softmax of the policy logits, the action's log-prob, the entropy, the
// clipped surrogate and the clipped value error; masked means over the
// rows; and the gradient of the total loss with respect to the logits and
// the value head.  Tie and bound gradients follow the relu identities of the
// reference: minimum(a, b) = a - relu(a - b) routes a tie to a, maximum(a,
// b) = a + relu(b - a) routes a tie to a, clamp has zero gradient at its
// bounds.
__global__ __launch_bounds__(kRedThreads) void k_ppo_loss(
    PpoCfg cfg, const float* __restrict__ logits, const int* __restrict__ actions, const float* __restrict__ old_logp,
    const float* __restrict__ adv, const float* __restrict__ returns, const float* __restrict__ old_value,
    const float* __restrict__ value, const float* __restrict__ valid, float* __restrict__ out,
    float* __restrict__ new_logp, float* __restrict__ dlogits, float* __restrict__ dvalue) {
  __shared__ float sh[kRedThreads];
  const int B = cfg.B, A = cfg.A;
  float wsum = 0.f;
  for (int i = threadIdx.x; i < B; i += kRedThreads) wsum += valid ? valid[i] : 1.f;
  const float total = tree_sum<kRedThreads>(wsum, sh);  // sum_all(valid)
  const float inv = 1.f / total;

  float s_pol = 0.f, s_val = 0.f, s_ent = 0.f, s_kl = 0.f;
  for (int i = threadIdx.x; i < B; i += kRedThreads) {
    const float* z = logits + long(i) * cfg.ldz;
    const float w = valid ? valid[i] : 1.f;
    if (!(w > 0.f)) {
      // An excluded slot (autoreset padding of a recurrent minibatch): no
      // loss term and no gradient; its old log-prob counts as 0 in the
      // approximate KL, as the reference zeroes the field before the
      // forward (ttrl/algos/ppo/recurrent.py:214-224).
      float mx = z[0];
      for (int j = 1; j < A; ++j) mx = fmaxf(mx, z[j]);
      float se = 0.f;
      for (int j = 0; j < A; ++j) se += expf(z[j] - mx);
      const int a = actions[i];
      const float lp = (a >= 0 && a < A) ? (z[a] - mx) - logf(se) : 0.f;
      new_logp[i] = lp;
      s_kl += expm1f(lp) - lp;
      float* dz0 = dlogits + long(i) * cfg.ldz;
      for (int j = 0; j < A; ++j) dz0[j] = 0.f;
      dvalue[long(i) * cfg.ldv] = 0.f;
      continue;
    }
    float mx = z[0];
    for (int j = 1; j < A; ++j) mx = fmaxf(mx, z[j]);
    float se = 0.f;
    for (int j = 0; j < A; ++j) se += expf(z[j] - mx);
    const float lse = logf(se);
    // An action outside [0, A) matches no one-hot lane, as in the reference's
    // one_hot_gather: its log-prob is 0 and carries no gradient.
    const int a = actions[i];
    const bool act_in = a >= 0 && a < A;
    const float lp = act_in ? (z[a] - mx) - lse : 0.f;
    float H = 0.f;
    for (int j = 0; j < A; ++j) {
      const float l = (z[j] - mx) - lse;
      H -= expf(l) * l;
    }
    new_logp[i] = lp;

    // clipped surrogate
    const float lr = lp - old_logp[i];
    s_kl += expm1f(lr) - lr;  // Schulman's k3 estimator (ttrl/algos/ppo/learn.py:101-104)
    const float r = expf(lr);
    const float lo = 1.f - cfg.clip, hi = 1.f + cfg.clip;
    const float rc = fminf(fmaxf(r, lo), hi);
    const float Ad = adv[i];
    const float u = r * Ad, c = rc * Ad;
    const float surr = u - fmaxf(u - c, 0.f);
    const bool take_u = !(u - c > 0.f);
    const float dclamp = (r > lo && r < hi) ? 1.f : 0.f;
    const float dsurr_dr = take_u ? Ad : dclamp * Ad;

    // clipped value error
    const float v = value[long(i) * cfg.ldv], ov = old_value[i], R = returns[i];
    const float dv = v - ov;
    const float dvc = fminf(fmaxf(dv, -cfg.vclip), cfg.vclip);
    const float eu = v - R, ec = (ov + dvc) - R;
    const float qu = eu * eu, qc = ec * ec;
    const bool take_c = qc - qu > 0.f;
    const float vmax = take_c ? qc : qu;
    const float dvclamp = (dv > -cfg.vclip && dv < cfg.vclip) ? 1.f : 0.f;
    const float dq_dv = take_c ? 2.f * ec * dvclamp : 2.f * eu;

    s_pol += surr * w;
    s_val += vmax * w;
    s_ent += H * w;

    // d loss / d logits: -(w/total) dsurr/dr * r * (onehot - p) + ecoef (w/total) p (logp + H)
    const float gp = act_in ? -w * inv * dsurr_dr * r : 0.f;
    const float ge = cfg.ecoef * w * inv;
    float* dz = dlogits + long(i) * cfg.ldz;
    for (int j = 0; j < A; ++j) {
      const float l = (z[j] - mx) - lse;
      const float p = expf(l);
      dz[j] = gp * ((j == a ? 1.f : 0.f) - p) + ge * p * (l + H);
    }
    dvalue[long(i) * cfg.ldv] = cfg.vcoef * 0.5f * w * inv * dq_dv;
  }
  const float pol = -tree_sum<kRedThreads>(s_pol, sh) * inv;
  const float val = 0.5f * tree_sum<kRedThreads>(s_val, sh) * inv;
  const float ent = tree_sum<kRedThreads>(s_ent, sh) * inv;
  const float kl = cfg.kl ? tree_sum<kRedThreads>(s_kl, sh) / float(B) : 0.f;
  if (threadIdx.x == 0) {
    out[0] = (pol + val * cfg.vcoef) + ent * -cfg.ecoef;
    out[1] = pol;
    out[2] = val;
    out[3] = ent;
    if (cfg.kl) out[4] = kl;
  }
}

constexpr int kRedWaves = kRedThreads / 64;

// Deterministic sums of NV values over the block: each wavefront folds its
// lanes with xor shuffles and keeps lane 0's result, then the wavefront
// partials are added in wavefront order.  Every thread gets the totals.
template <int NV>
__device__ inline void block_sums(float (&v)[NV], float* sh /* NV * kRedWaves */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_xor(v[k], off, 64);
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < NV; ++k) sh[k * kRedWaves + wave] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float t = sh[k * kRedWaves];
#pragma unroll
    for (int w = 1; w < kRedWaves; ++w) t += sh[k * kRedWaves + w];
    v[k] = t;
  }
  __syncthreads();
}

// One row's operands, the logits in registers (A <= AM).
template <int AM>
struct PpoRowIn {
  float z[AM];
  int a;
  float w, olp, adv, v, ov, R;
};

template <int AM>
__device__ __forceinline__ void ppo_row_load(const PpoCfg& cfg, const float* logits, const int* actions,
                                             const float* old_logp, const float* adv, const float* returns,
                                             const float* old_value, const float* value, const float* valid, int i,
                                             PpoRowIn<AM>& r) {
  const float* z = logits + long(i) * cfg.ldz;
#pragma unroll
  for (int j = 0; j < AM; ++j) r.z[j] = z[min(j, cfg.A - 1)];  // every load unconditional
  r.a = actions[i];
  const float wv = *(valid ? valid + i : old_logp + i);
  r.w = valid ? wv : 1.f;
  r.olp = old_logp[i];
  r.adv = adv[i];
  r.v = value[long(i) * cfg.ldv];
  r.ov = old_value[i];
  r.R = returns[i];
}

// The row's terms and gradients: the expressions of k_ppo_loss, in its order.
template <int AM>
__device__ __forceinline__ void ppo_row(const PpoCfg& cfg, const PpoRowIn<AM>& r, float inv, int i,
                                        float* new_logp, float* dlogits, float* dvalue, float (&acc)[4]) {
  const int A = cfg.A, a = r.a;
  float mx = r.z[0];
#pragma unroll
  for (int j = 1; j < AM; ++j)
    if (j < A) mx = fmaxf(mx, r.z[j]);
  float se = 0.f;
#pragma unroll
  for (int j = 0; j < AM; ++j)
    if (j < A) se += expf(r.z[j] - mx);
  const bool act_in = a >= 0 && a < A;
  float za = 0.f;  // z[a], selected without indexing the registers at run time
#pragma unroll
  for (int j = 0; j < AM; ++j)
    if (j == a) za = r.z[j];
  float* dz = dlogits + long(i) * cfg.ldz;
  if (!(r.w > 0.f)) {
    // an excluded slot: no loss term and no gradient (see k_ppo_loss)
    const float lp = act_in ? (za - mx) - logf(se) : 0.f;
    new_logp[i] = lp;
    acc[3] += expm1f(lp) - lp;
#pragma unroll
    for (int j = 0; j < AM; ++j)
      if (j < A) dz[j] = 0.f;
    dvalue[long(i) * cfg.ldv] = 0.f;
    return;
  }
  const float lse = logf(se);
  const float lp = act_in ? (za - mx) - lse : 0.f;
  float H = 0.f;
#pragma unroll
  for (int j = 0; j < AM; ++j) {
    if (j < A) {
      const float l = (r.z[j] - mx) - lse;
      H -= expf(l) * l;
    }
  }
  new_logp[i] = lp;
  const float lr = lp - r.olp;
  acc[3] += expm1f(lr) - lr;
  const float ratio = expf(lr);
  const float lo = 1.f - cfg.clip, hi = 1.f + cfg.clip;
  const float rc = fminf(fmaxf(ratio, lo), hi);
  const float Ad = r.adv;
  const float u = ratio * Ad, c = rc * Ad;
  const float surr = u - fmaxf(u - c, 0.f);
  const bool take_u = !(u - c > 0.f);
  const float dclamp = (ratio > lo && ratio < hi) ? 1.f : 0.f;
  const float dsurr_dr = take_u ? Ad : dclamp * Ad;
  const float dv = r.v - r.ov;
  const float dvc = fminf(fmaxf(dv, -cfg.vclip), cfg.vclip);
  const float eu = r.v - r.R, ec = (r.ov + dvc) - r.R;
  const float qu = eu * eu, qc = ec * ec;
  const bool take_c = qc - qu > 0.f;
  const float vmax = take_c ? qc : qu;
  const float dvclamp = (dv > -cfg.vclip && dv < cfg.vclip) ? 1.f : 0.f;
  const float dq_dv = take_c ? 2.f * ec * dvclamp : 2.f * eu;
  const float w = r.w;
  acc[0] += surr * w;
  acc[1] += vmax * w;
  acc[2] += H * w;
  const float gp = act_in ? -w * inv * dsurr_dr * ratio : 0.f;
  const float ge = cfg.ecoef * w * inv;
#pragma unroll
  for (int j = 0; j < AM; ++j) {
    if (j < A) {
      const float l = (r.z[j] - mx) - lse;
      const float p = expf(l);
      dz[j] = gp * ((j == a ? 1.f : 0.f) - p) + ge * p * (l + H);
    }
  }
  dvalue[long(i) * cfg.ldv] = cfg.vcoef * 0.5f * w * inv * dq_dv;
}

// k_ppo_loss with its latency cut for A <= AM: a thread's first row is
// loaded before anything waits, the sums are two shuffle-and-LDS reductions
// (the valid count, then the four loss sums together) instead of five
// barrier trees.  Same per-row expressions; the block sums add in another
// (fixed) order.
template <int AM>
__global__ __launch_bounds__(kRedThreads) void k_ppo_loss_rows(
    PpoCfg cfg, const float* __restrict__ logits, const int* __restrict__ actions, const float* __restrict__ old_logp,
    const float* __restrict__ adv, const float* __restrict__ returns, const float* __restrict__ old_value,
    const float* __restrict__ value, const float* __restrict__ valid, float* __restrict__ out,
    float* __restrict__ new_logp, float* __restrict__ dlogits, float* __restrict__ dvalue) {
  __shared__ float sh[4 * kRedWaves];
  const int B = cfg.B, tid = threadIdx.x;
  PpoRowIn<AM> r0;
  ppo_row_load<AM>(cfg, logits, actions, old_logp, adv, returns, old_value, value, valid, min(tid, B - 1), r0);
  float wsum[1] = {tid < B ? r0.w : 0.f};
  for (int i = tid + kRedThreads; i < B; i += kRedThreads) wsum[0] += valid ? valid[i] : 1.f;
  block_sums<1>(wsum, sh);  // sum_all(valid)
  const float inv = 1.f / wsum[0];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // surrogate, value error, entropy, approximate KL
  if (tid < B) ppo_row<AM>(cfg, r0, inv, tid, new_logp, dlogits, dvalue, acc);
  for (int i = tid + kRedThreads; i < B; i += kRedThreads) {
    PpoRowIn<AM> r;
    ppo_row_load<AM>(cfg, logits, actions, old_logp, adv, returns, old_value, value, valid, i, r);
    ppo_row<AM>(cfg, r, inv, i, new_logp, dlogits, dvalue, acc);
  }
  block_sums<4>(acc, sh);
  if (tid == 0) {
    const float pol = -acc[0] * inv;
    const float val = 0.5f * acc[1] * inv;
    const float ent = acc[2] * inv;
    out[0] = (pol + val * cfg.vcoef) + ent * -cfg.ecoef;
    out[1] = pol;
    out[2] = val;
    out[3] = ent;
    if (cfg.kl) out[4] = acc[3] / float(B);
  }
}

// The objective's launch: the register-row kernel for up to 32 actions.
void launch_ppo_loss(hipStream_t st, const PpoCfg& cfg, const float* logits, const int* actions,
                     const float* old_logp, const float* adv, const float* returns, const float* old_value,
                     const float* value, const float* valid, float* out, float* new_logp, float* dlogits,
                     float* dvalue) {
  const dim3 g(1), b(kRedThreads);
  if (cfg.A <= 8)
    hipLaunchKernelGGL(k_ppo_loss_rows<8>, g, b, 0, st, cfg, logits, actions, old_logp, adv, returns, old_value,
                       value, valid, out, new_logp, dlogits, dvalue);
  else if (cfg.A <= 18)
    hipLaunchKernelGGL(k_ppo_loss_rows<18>, g, b, 0, st, cfg, logits, actions, old_logp, adv, returns, old_value,
                       value, valid, out, new_logp, dlogits, dvalue);
  else if (cfg.A <= 32)
    hipLaunchKernelGGL(k_ppo_loss_rows<32>, g, b, 0, st, cfg, logits, actions, old_logp, adv, returns, old_value,
                       value, valid, out, new_logp, dlogits, dvalue);
  else
    hipLaunchKernelGGL(k_ppo_loss, g, b, 0, st, cfg, logits, actions, old_logp, adv, returns, old_value, value,
                       valid, out, new_logp, dlogits, dvalue);
}

// g *= max_norm / (norm + 1e-6) when norm = sqrt(*sq) exceeds max_norm; the
// norm before clipping is left in *norm_out.
__global__ __launch_bounds__(256) void k_clip_scale(float* __restrict__ g, long n, const float* __restrict__ sq,
                                                    float max_norm, float* __restrict__ norm_out) {
  const double total = std::sqrt(double(*sq));
  if (blockIdx.x == 0 && threadIdx.x == 0 && norm_out) *norm_out = float(total);
  if (!(total > double(max_norm))) return;
  const float scale = float(double(max_norm) / (total + 1e-6));
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += long(gridDim.x) * 256) g[i] *= scale;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_gae(ttrl_ctx* ctx, int T, int N, const float* rewards, const float* values, const float* dones,
             const float* valid, const float* last_values, double gamma, double lam, float* advantages,
             float* returns) {
  TTRL_REQUIRE(ctx && rewards && values && dones && last_values && advantages && returns, "ttrl_gae: null argument");
  TTRL_REQUIRE(T > 0 && N > 0, "ttrl_gae: T and N must be positive (got %d, %d)", T, N);
  const unsigned blocks = unsigned((N + kGaeLanes - 1) / kGaeLanes);
  // The reference multiplies float32 arrays by Python floats: gamma is rounded
  // to float32 on its own, gamma*lam is formed in double and then rounded.
  hipLaunchKernelGGL(k_gae, dim3(blocks), dim3(256), 0, stream_of(ctx), T, N, rewards, values, dones, valid,
                     last_values, float(gamma), float(gamma * lam), advantages, returns);
  return check_launch("ttrl_gae");
}

int ttrl_normalize_advantages(ttrl_ctx* ctx, const float* adv, const float* valid, long n, float eps, float* out,
                              float* stats) {
  TTRL_REQUIRE(ctx && adv && out, "ttrl_normalize_advantages: null argument");
  TTRL_REQUIRE(n > 0, "ttrl_normalize_advantages: empty input");
  hipLaunchKernelGGL(k_adv_normalize, dim3(1), dim3(kRedThreads), 0, stream_of(ctx), adv, valid, n, eps, out, stats);
  return check_launch("ttrl_normalize_advantages");
}

int ttrl_ppo_loss(ttrl_ctx* ctx, int B, int A, const float* logits, const int* actions, const float* old_logp,
                  const float* advantages, const float* returns, const float* old_values, const float* values,
                  const float* valid, float clip_eps, float value_clip_eps, float value_coef, float entropy_coef,
                  float* out4, float* new_logp, float* dlogits, float* dvalues) {
  TTRL_REQUIRE(ctx && logits && actions && old_logp && advantages && returns && old_values && values && out4 &&
                   new_logp && dlogits && dvalues,
               "ttrl_ppo_loss: null argument");
  TTRL_REQUIRE(B > 0 && A > 0, "ttrl_ppo_loss: B and A must be positive (got %d, %d)", B, A);
  TTRL_REQUIRE(clip_eps > 0.f && value_clip_eps > 0.f, "ttrl_ppo_loss: clip ranges must be positive");
  PpoCfg cfg{B, A, clip_eps, value_clip_eps, value_coef, entropy_coef, A, 1, 0};
  launch_ppo_loss(stream_of(ctx), cfg, logits, actions, old_logp, advantages, returns, old_values, values, valid, out4,
                  new_logp, dlogits, dvalues);
  return check_launch("ttrl_ppo_loss");
}

int ttrl_ppo_loss_packed(ttrl_ctx* ctx, int B, int A, const float* head, const int* actions, const float* old_logp,
                         const float* advantages, const float* returns, const float* old_values, const float* valid,
                         float clip_eps, float value_clip_eps, float value_coef, float entropy_coef, float* out5,
                         float* new_logp, float* dhead) {
  TTRL_REQUIRE(ctx && head && actions && old_logp && advantages && returns && old_values && out5 && new_logp &&
                   dhead,
               "ttrl_ppo_loss_packed: null argument");
  TTRL_REQUIRE(B > 0 && A > 0, "ttrl_ppo_loss_packed: B and A must be positive (got %d, %d)", B, A);
  TTRL_REQUIRE(clip_eps > 0.f && value_clip_eps > 0.f, "ttrl_ppo_loss_packed: clip ranges must be positive");
  PpoCfg cfg{B, A, clip_eps, value_clip_eps, value_coef, entropy_coef, A + 1, A + 1, 1};
  launch_ppo_loss(stream_of(ctx), cfg, head, actions, old_logp, advantages, returns, old_values, head + A, valid, out5,
                  new_logp, dhead, dhead + A);
  return check_launch("ttrl_ppo_loss_packed");
}

int ttrl_clip_grad_norm(ttrl_ctx* ctx, float* g, long n, float max_norm, float* sq_scratch, float* norm_out) {
  TTRL_REQUIRE(ctx && g && sq_scratch, "ttrl_clip_grad_norm: null argument");
  TTRL_REQUIRE(max_norm > 0.f, "ttrl_clip_grad_norm: max_norm must be > 0, got %g", double(max_norm));
  int rc = ttrl_sum_squares(ctx, g, n, sq_scratch, 0);
  if (rc) return rc;
  const unsigned blocks = unsigned(std::min<long>(2048, (n + 255) / 256 > 0 ? (n + 255) / 256 : 1));
  hipLaunchKernelGGL(k_clip_scale, dim3(blocks), dim3(256), 0, stream_of(ctx), g, n, sq_scratch, max_norm, norm_out);
  return check_launch("ttrl_clip_grad_norm");
}

}  // extern "C"
