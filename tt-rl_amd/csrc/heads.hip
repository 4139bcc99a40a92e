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
#include "dqn_row.hpp"

#include <cmath>

namespace ttrl {

constexpr int kHeadThreads = 256;
constexpr float kLog2 = 0.69314718055994530942f;
constexpr float kLog2Pi = 1.83787706640934548356f;

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
    const long o = long(b) * A;
    const DqnRow r = dqn_row(b, A, q + o, qsel + o, qval + o, onehot + o, rewards, dones, discounts, weights, delta,
                             invB, td_abs, next_act, td_target, dq + o);
    sum_h += r.h;
    sum_p += r.pred;
  }
  const float th = block_sum<kHeadThreads>(sum_h, red);
  const float tp = block_sum<kHeadThreads>(sum_p, red);
  if (threadIdx.x == 0) {
    *loss = th * invB;
    if (mean_q) *mean_q = tp * invB;
  }
}

// The Q head's last linear layer for the online(s), online(s') and
// target(s') features (groups 0, 1, 2; two groups for vanilla DQN, where the
// target both selects and values), then the DQN head above, in one launch.
// Workgroup j owns samples [j*RB, (j+1)*RB) of every group (RB <= 64): per
// group, W is staged in LDS as [K][AP] rows padded with zeros to AP (8, 16
// or 32) actions, so a lane's k-slice reads whole 16-byte chunks with no
// per-action branch.  The wavefronts are split evenly over the groups; a
// wavefront owns every WPG-th sample row of its group and takes RU rows at
// a time (RU * AP = 32 sums) with all their loads in flight together, its
// lanes split the K-sum, and a reduce-scatter over the lanes finishes the
// 32 sums in 32 exchanges.  Each sample's target, Huber term
// and dL/dQ need only its own row; the batch means are a butterfly over
// wavefront 0, which holds the workgroup's samples.  A batch of at most 64
// is one workgroup and writes the means directly; a larger batch sums the
// per-workgroup partials, in workgroup order, in the workgroup that
// finishes last (a device-scope counter, reset by that workgroup for the
// next launch).
// Range-checked loads: an offset past `bytes` reads zero.  The base and
// size are wave-uniform; readfirstlane keeps the resource in scalar
// registers (one in vector registers would loop over the lanes per load).
__device__ inline __amdgpu_buffer_rsrc_t head_res(const float* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<float*>((uint64_t(hi) << 32) | lo), static_cast<short>(0),
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)), 0x00020000);
}
__device__ inline float head_ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// One level of a reduce-scatter over the lanes: lanes l and l ^ O swap
// halves of their first 2 HALF sums, each keeping the upper half if l & O,
// and add.  Compile-time offsets keep every index static.
template <int O, int HALF>
__device__ __forceinline__ void scatter_level(float* acc, int lane) {
  const bool up = (lane & O) != 0;
#pragma unroll
  for (int t = 0; t < HALF; ++t) {
    const float keep = up ? acc[t + HALF] : acc[t];
    const float send = up ? acc[t] : acc[t + HALF];
    acc[t] = keep + __shfl_xor(send, O, 64);
  }
}

constexpr int kDqnHeadThreads = 1024;
constexpr int kDqnHeadMaxA = 32;
constexpr int kDqnHeadRows = 64;         // samples per workgroup (wavefront 0 finishes them)
constexpr int kDqnHeadLds = 128 * 1024;  // dynamic LDS (gfx950: 160 KiB per workgroup)
constexpr int kDqnHeadMaxBlocks = 1024;
struct DqnHeadGroups {
  const float* h[3];
  const float* W[3];
  const float* b[3];
  float* q[3];
};
template <int AP>
__global__ __launch_bounds__(kDqnHeadThreads) void k_dqn_head(
    int B, int K, int A, int G, int RB, DqnHeadGroups p, const float* __restrict__ onehot,
    const float* __restrict__ rewards, const float* __restrict__ dones, const float* __restrict__ discounts,
    const float* __restrict__ weights, float delta, float* __restrict__ loss, float* __restrict__ mean_q,
    float* __restrict__ td_abs, float* __restrict__ dq, float* __restrict__ next_act, float* __restrict__ td_target,
    unsigned* __restrict__ counter, float* __restrict__ partials) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* Ws = lds;                     // [G][K][AP]
  float* qs = lds + long(G) * K * AP;  // [G][RB][A]
  constexpr int KU = 8;                                      // k-loads per lane and row in flight together
  constexpr int RU = AP <= 8 ? 4 : (AP <= 16 ? 2 : 1);     // rows in flight together (RU * AP accumulators)
  // The wavefront index and everything derived from it are scalar: a
  // per-lane index would fetch p.h[g] with a vector load whose wait also
  // waits for every row load issued before it.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b0 = blockIdx.x * RB;
  const int nrows = min(RB, B - b0);
  // Wavefront (g, j) owns rows j, j + WPG, j + 2 WPG, ... of group g.
  const int WPG = (kDqnHeadThreads / 64) / G;
  const int g = wave / WPG, j = wave - g * WPG;
  const int my_rows = g < G && j < nrows ? (nrows - j + WPG - 1) / WPG : 0;
  const float* hg = g == 0 ? p.h[0] : (g == 1 ? p.h[1] : p.h[2]);  // read only for g < G
  const float* bg = g == 0 ? p.b[0] : (g == 1 ? p.b[1] : p.b[2]);
  float* qg = g == 0 ? p.q[0] : (g == 1 ? p.q[1] : p.q[2]);
  auto row_res = [&](int r) {  // the r-th row of this wavefront; none past my_rows
    const bool ok = r < my_rows;
    return head_res(ok ? hg + long(b0 + j + r * WPG) * K : p.h[0], ok ? uint32_t(K) * 4u : 0u);
  };
  // The first rows' first K-slice is in flight while the workgroup stages W.
  float hv[RU][KU];
#pragma unroll
  for (int u = 0; u < RU; ++u)
#pragma unroll
    for (int uu = 0; uu < KU; ++uu) hv[u][uu] = head_ld(row_res(u), uint32_t(uu * 64 + lane) * 4u);  // zero past K
  // The batch inputs of the samples this workgroup finishes, also early.
  const int mine = b0 + int(threadIdx.x);
  const bool fin = int(threadIdx.x) < nrows;
  const float r_in = fin ? rewards[mine] : 0.f, d_in = fin ? dones[mine] : 0.f;
  const float disc_in = fin ? discounts[mine] : 0.f, w_in = (fin && weights) ? weights[mine] : 1.f;
  // Every group's W at once, staged in chunks of kDqnHeadThreads * SU
  // words per group with all groups' loads in flight before any store.
  constexpr int SU = 4;
  const int per_group = K * AP;
  for (int t0 = 0; t0 < per_group; t0 += kDqnHeadThreads * SU) {
    float v[3][SU];
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      const __amdgpu_buffer_rsrc_t rw = head_res(p.W[gg < G ? gg : 0], gg < G ? uint32_t(K) * uint32_t(A) * 4u : 0u);
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int t = t0 + u * kDqnHeadThreads + threadIdx.x;
        const int k = t / AP, a = t - k * AP;
        v[gg][u] = head_ld(rw, (a < A && t < per_group) ? (uint32_t(k) * uint32_t(A) + uint32_t(a)) * 4u : 0x40000000u);
      }
    }
#pragma unroll
    for (int gg = 0; gg < 3; ++gg) {
      if (gg >= G) break;
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int t = t0 + u * kDqnHeadThreads + threadIdx.x;
        if (t < per_group) Ws[gg * per_group + t] = v[gg][u];
      }
    }
  }
  __syncthreads();
  const float* Wg = Ws + long(g < G ? g : 0) * K * AP;
  static_assert(RU * AP == 32, "the lane reduction scatters 32 sums over 32 lanes");
  // After the lane reduction lane l (and l + 32) holds sum number
  // bitrev5(l & 31): each level's upper partner keeps the upper half.
  const int vi = ((lane & 1) << 4) | ((lane & 2) << 2) | (lane & 4) | ((lane & 8) >> 2) | ((lane & 16) >> 4);
  const int vu = vi / AP, va = vi - vu * AP;
  for (int r0 = 0; r0 < my_rows; r0 += RU) {  // wave-uniform
    float acc[RU * AP];  // [row][action]
#pragma unroll
    for (int t = 0; t < RU * AP; ++t) acc[t] = 0.f;
    for (int k0 = 0; k0 < K; k0 += 64 * KU) {
      if (r0 > 0 || k0 > 0) {
#pragma unroll
        for (int u = 0; u < RU; ++u)
#pragma unroll
          for (int uu = 0; uu < KU; ++uu) hv[u][uu] = head_ld(row_res(r0 + u), uint32_t(k0 + uu * 64 + lane) * 4u);
      }
#pragma unroll
      for (int uu = 0; uu < KU; ++uu) {
        const int k = min(k0 + uu * 64 + lane, K - 1);  // a real row of Ws; hv is zero past K
        const float4* wr = reinterpret_cast<const float4*>(Wg + k * AP);
#pragma unroll
        for (int c = 0; c < AP / 4; ++c) {
          const float4 w4 = wr[c];
#pragma unroll
          for (int u = 0; u < RU; ++u) {
            float* au = acc + u * AP + 4 * c;
            au[0] = fmaf(hv[u][uu], w4.x, au[0]);
            au[1] = fmaf(hv[u][uu], w4.y, au[1]);
            au[2] = fmaf(hv[u][uu], w4.z, au[2]);
            au[3] = fmaf(hv[u][uu], w4.w, au[3]);
          }
        }
      }
    }
    // Reduce-scatter over the lanes: at offset o a lane keeps half of the
    // sums it holds (the upper half if lane & o) and adds its partner's
    // copy of that half, so five levels exchange 16 + 8 + 4 + 2 + 1 values
    // and leave each lane one sum over its half-wave; the last exchange adds
    // the other half-wave.
    scatter_level<1, 16>(acc, lane);
    scatter_level<2, 8>(acc, lane);
    scatter_level<4, 4>(acc, lane);
    scatter_level<8, 2>(acc, lane);
    scatter_level<16, 1>(acc, lane);
    float v = acc[0] + __shfl_xor(acc[0], 32, 64);
    if (lane < 32 && va < A && r0 + vu < my_rows) {
      const int i = j + (r0 + vu) * WPG;
      if (bg) v += bg[va];
      qs[(g * RB + i) * A + va] = v;
      qg[long(b0 + i) * A + va] = v;
    }
  }
  __syncthreads();
  const float invB = 1.f / float(B);
  float sum_h = 0.f, sum_p = 0.f;
  if (fin) {
    const int i = threadIdx.x, b = mine;
    const long o = long(b) * A;
    const DqnRow r = dqn_row_v(b, A, qs + i * A, qs + (RB + i) * A, qs + ((G - 1) * RB + i) * A, onehot + o, r_in,
                               d_in, disc_in, w_in, weights != nullptr, delta, invB, td_abs, next_act, td_target,
                               dq + o);
    sum_h = r.h;
    sum_p = r.pred;
  }
  if (wave != 0) return;  // the workgroup's samples are all in wavefront 0 (nrows <= 64)
  float th = sum_h, tp = sum_p;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    th += __shfl_xor(th, off, 64);
    tp += __shfl_xor(tp, off, 64);
  }
  if (gridDim.x == 1) {
    if (threadIdx.x == 0) {
      *loss = th * invB;
      if (mean_q) *mean_q = tp * invB;
    }
    return;
  }
  if (threadIdx.x == 0) {
    partials[2 * blockIdx.x] = th;
    partials[2 * blockIdx.x + 1] = tp;
    __threadfence();  // the partials are visible device-wide before the count
    if (atomicAdd(counter, 1u) == gridDim.x - 1) {
      __threadfence();
      float sh = 0.f, sp = 0.f;
      for (unsigned jj = 0; jj < gridDim.x; ++jj) {  // workgroup order: the same sum on every run
        sh += __hip_atomic_load(&partials[2 * jj], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sp += __hip_atomic_load(&partials[2 * jj + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *loss = sh * invB;
      if (mean_q) *mean_q = sp * invB;
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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

int ttrl_dqn_head(ttrl_ctx* ctx, int B, int K, int A, int groups, const float* const* h, const float* const* W,
                  const float* const* bias, float* const* q_out, const float* actions_onehot, const float* rewards,
                  const float* dones, const float* discounts, const float* is_weights, float delta, float* loss,
                  float* mean_q, float* td_abs, float* dq, float* next_actions, float* td_target) {
  TTRL_REQUIRE(ctx && h && W && q_out && actions_onehot && rewards && dones && discounts && loss && dq,
               "ttrl_dqn_head: null argument");
  TTRL_REQUIRE(groups == 2 || groups == 3, "ttrl_dqn_head: 2 (vanilla) or 3 (double) groups, got %d", groups);
  TTRL_REQUIRE(B > 0 && K > 0 && A > 0, "ttrl_dqn_head: empty extents");
  TTRL_REQUIRE(A <= kDqnHeadMaxA, "ttrl_dqn_head: at most %d actions", kDqnHeadMaxA);
  TTRL_REQUIRE(delta > 0.f, "ttrl_dqn_head: huber delta must be > 0");
  const int ap = A <= 8 ? 8 : (A <= 16 ? 16 : 32);
  const int rb = B < kDqnHeadRows ? B : kDqnHeadRows;  // sample rows per workgroup
  const int blocks = (B + rb - 1) / rb;
  const size_t lds = (size_t(groups) * K * ap + size_t(groups) * rb * A) * sizeof(float);
  TTRL_REQUIRE(lds <= size_t(kDqnHeadLds), "ttrl_dqn_head: %d groups of K=%d x %d actions exceed the %d-byte LDS",
               groups, K, A, kDqnHeadLds);
  TTRL_REQUIRE(blocks <= kDqnHeadMaxBlocks, "ttrl_dqn_head: batch %d needs more than %d workgroups", B,
               kDqnHeadMaxBlocks);
  DqnHeadGroups p{};
  for (int g = 0; g < groups; ++g) {
    TTRL_REQUIRE(h[g] && W[g] && q_out[g], "ttrl_dqn_head: null pointer in group %d", g);
    p.h[g] = h[g];
    p.W[g] = W[g];
    p.b[g] = bias ? bias[g] : nullptr;
    p.q[g] = q_out[g];
  }
  unsigned* counter = ctx_sync_words(ctx);
  float* partials = reinterpret_cast<float*>(counter + kSyncCounters);
  auto launch = [&](auto kernel) -> int {
    // Above 64 KiB of LDS a kernel needs the larger limit set once.
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kDqnHeadLds);
    if (attr != hipSuccess && lds > size_t(64 * 1024)) return hip_error(attr, "ttrl_dqn_head: LDS limit");
    hipLaunchKernelGGL(kernel, dim3(unsigned(blocks)), dim3(kDqnHeadThreads), lds, stream_of(ctx), B, K, A, groups,
                       rb, p, actions_onehot, rewards, dones, discounts, is_weights, delta, loss, mean_q, td_abs, dq,
                       next_actions, td_target, counter + kSyncDqnHead, partials);
    return check_launch("ttrl_dqn_head");
  };
  if (ap == 8) return launch(k_dqn_head<8>);
  if (ap == 16) return launch(k_dqn_head<16>);
  return launch(k_dqn_head<32>);
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
