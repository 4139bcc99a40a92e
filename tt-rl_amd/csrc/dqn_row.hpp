// One sample of the DQN update head, shared by the loss kernels.
//
// Q(s,a) by one-hot gather (ttrl/engine/ops/functional.py:126-132),
// double-DQN argmax with the first index winning ties
// (ttrl/engine/ops/reduce.py:82-99), n-step target r + discounts*(1-done)*
// Q'(s', a*) (ttrl/engine/ops/functional.py:40-46), Huber through the
// clipped-quadratic identity (functional.py:56-69), importance weight;
// dL/dQ = onehot * w/B * clip(e, -delta, delta).
#pragma once

#include "common.hpp"

namespace ttrl {

__device__ inline float relu_f(float x) { return x > 0.f ? x : 0.f; }

// One sample of the DQN head: Q(s, a) of the taken action, the double-DQN
// target from the selection row `sb` and the valuation row `vb`, Huber,
// the per-sample outputs and dL/dQ for row b.  Returns (w * huber, pred).
struct DqnRow {
  float h, pred;
};
__device__ inline DqnRow dqn_row_v(int b, int A, const float* qb, const float* sb, const float* vb, const float* ob,
                                   float reward, float done, float discount, float w, bool has_w, float delta,
                                   float invB, float* td_abs, float* next_act, float* td_target, float* dqb) {
  float pred = 0.f;
  for (int a = 0; a < A; ++a) pred += qb[a] * ob[a];
  int best = 0;
  float bv = sb[0];
  for (int a = 1; a < A; ++a)
    if (sb[a] > bv) {
      bv = sb[a];
      best = a;
    }
  const float nv = vb[best];
  const float y = reward + (nv * (1.f - done)) * discount;
  const float e = pred - y;
  const float ae = fabsf(e);
  const float quad = ae - relu_f(ae - delta);
  const float lin = ae - quad;
  const float h = (quad * quad) * 0.5f + lin * delta;
  if (td_abs) td_abs[b] = ae;
  if (next_act) next_act[b] = float(best);
  if (td_target) td_target[b] = y;
  const float clip = fminf(fmaxf(e, -delta), delta);
  const float gscale = (has_w ? w * invB : invB) * clip;
  for (int a = 0; a < A; ++a) dqb[a] = ob[a] * gscale;
  return DqnRow{has_w ? h * w : h, pred};
}
// dqn_row_v over rows held in registers, AP entries of which the first A
// are actions: the same operations in the same order (padding entries are
// skipped by selects, so no per-action branch or memory access).  dqb
// receives dL/dQ, zero past A.
template <int AP>
__device__ inline DqnRow dqn_row_r(int b, int A, const float (&qb)[AP], const float (&sb)[AP], const float (&vb)[AP],
                                   const float (&ob)[AP], float reward, float done, float discount, float w,
                                   bool has_w, float delta, float invB, float* td_abs, float* next_act,
                                   float* td_target, float (&dqb)[AP]) {
  float pred = 0.f;
#pragma unroll
  for (int a = 0; a < AP; ++a) pred = a < A ? pred + qb[a] * ob[a] : pred;
  // the valuation row's entry rides along with the running argmax (a
  // select by the final index would become an indexed scratch access)
  int best = 0;
  float bv = sb[0], nv = vb[0];
#pragma unroll
  for (int a = 1; a < AP; ++a) {
    const bool take = a < A && sb[a] > bv;
    bv = take ? sb[a] : bv;
    nv = take ? vb[a] : nv;
    best = take ? a : best;
  }
  const float y = reward + (nv * (1.f - done)) * discount;
  const float e = pred - y;
  const float ae = fabsf(e);
  const float quad = ae - relu_f(ae - delta);
  const float lin = ae - quad;
  const float h = (quad * quad) * 0.5f + lin * delta;
  if (td_abs) td_abs[b] = ae;
  if (next_act) next_act[b] = float(best);
  if (td_target) td_target[b] = y;
  const float clip = fminf(fmaxf(e, -delta), delta);
  const float gscale = (has_w ? w * invB : invB) * clip;
#pragma unroll
  for (int a = 0; a < AP; ++a) dqb[a] = a < A ? ob[a] * gscale : 0.f;
  return DqnRow{has_w ? h * w : h, pred};
}

__device__ inline DqnRow dqn_row(int b, int A, const float* qb, const float* sb, const float* vb, const float* ob,
                                 const float* rewards, const float* dones, const float* discounts,
                                 const float* weights, float delta, float invB, float* td_abs, float* next_act,
                                 float* td_target, float* dqb) {
  return dqn_row_v(b, A, qb, sb, vb, ob, rewards[b], dones[b], discounts[b], weights ? weights[b] : 1.f,
                   weights != nullptr, delta, invB, td_abs, next_act, td_target, dqb);
}

}  // namespace ttrl
