// The Adam step's device arithmetic, shared by the optimizer kernels and the
// fused update stages that step parameters as they form their gradients
// (ttrl/engine/optim/adam.py:93-134, ttrl/engine/optim/scalars.py:13-27):
// S = m / (1 - b1) and V = v / (1 - b2) are stored, and one pair of fused
// scalars per step folds the bias corrections into the step size and eps.
#pragma once

#include "common.hpp"

#include <cmath>

namespace ttrl {

// The step's fused scalars (alpha_t, eps_t) at update count t.
// adam_scalars forms them from the count *step + 1 once per workgroup, by
// thread 0; every thread of the workgroup calls it (a barrier).  A wave's
// loads complete in the order they were issued, so thread 0's wait for the
// count also waits for every load issued before it.
__device__ __forceinline__ void adam_scalars_at(int t, float lr, float b1, float b2, float eps, float& alpha_t,
                                                float& eps_t) {
  const double bc1 = 1.0 - pow(double(b1), double(t));
  const double bc2 = 1.0 - pow(double(b2), double(t));
  const double c = sqrt((1.0 - double(b2)) / bc2);
  alpha_t = float(double(lr) * (1.0 - double(b1)) / bc1 / c);
  eps_t = float(double(eps) / c);
}
// adam_scalars_of takes the count the caller read (the same in every
// thread); a caller that reads it before its other loads waits for no
// later load when thread 0 uses it.
__device__ __forceinline__ void adam_scalars_of(int step, float lr, float b1, float b2, float eps, float* alpha_t,
                                                float* eps_t) {
  __shared__ float sc[2];
  if (threadIdx.x == 0) adam_scalars_at(step + 1, lr, b1, b2, eps, sc[0], sc[1]);
  __syncthreads();
  *alpha_t = sc[0];
  *eps_t = sc[1];
}
__device__ __forceinline__ void adam_scalars(const int* __restrict__ step, float lr, float b1, float b2, float eps,
                                             float* alpha_t, float* eps_t) {
  adam_scalars_of(*step, lr, b1, b2, eps, alpha_t, eps_t);
}

// The update of one parameter p with gradient graw; graw^2 is added to gsq.
// Every product and sum is rounded on its own (no contraction into FMAs), so
// every kernel that steps a parameter gives the same bits however the
// compiler schedules it.
__device__ __forceinline__ void adam1(float& p, float graw, float& s, float& v, float b1, float b2, float wd,
                                      float eps_t, float alpha_t, float& gsq) {
#pragma clang fp contract(off)
  gsq += graw * graw;
  const float gg = wd != 0.f ? graw + wd * p : graw;
  v = gg * gg + b2 * v;
  s = gg + b1 * s;
  const float upd = (s / (sqrtf(v) + eps_t)) * alpha_t;
  p = p - upd;
}

}  // namespace ttrl
