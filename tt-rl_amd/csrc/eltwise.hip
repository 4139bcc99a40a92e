// Generic elementwise, broadcast, reduction and strided-copy kernels behind
// the primitive op surface of the engine (ttrl/engine/ops/__init__.py:32-44):
// add/sub/mul/div with tensor, broadcast or scalar operands
// (ttrl/engine/ops/elementwise.py:15-148), the unary ops and their backward
// factors (ttrl/engine/ops/unary.py:21-150), sum/max/argmax along one axis
// (ttrl/engine/ops/reduce.py:12-99), the broadcast-gradient reduction
// (ttrl/engine/ops/broadcast.py:11-54), concat/split/slice copies
// (ttrl/engine/ops/shape.py:10-151) and the device one-hot
// (ttrl/engine/ops/functional.py:112-123).
//
// These serve composed, eager or test-time use of single ops; the hot update
// paths run the fused layer and loss kernels instead.
#include "common.hpp"

#include <cmath>

namespace ttrl {

constexpr int kEwThreads = 256;
constexpr int kMaxDims = 6;

struct Dims {
  int nd;
  long shape[kMaxDims];
  long sa[kMaxDims];
  long sb[kMaxDims];
  long sy[kMaxDims];
};

__device__ inline float unary_op(int op, float x, float s) {
  switch (op) {
    case TTRL_U_RELU: return x > 0.f ? x : 0.f;
    case TTRL_U_ABS: return fabsf(x);
    case TTRL_U_SIGN: return x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f);
    case TTRL_U_SQUARE: return x * x;
    case TTRL_U_EXP: return expf(x);
    case TTRL_U_LOG: return logf(x);
    case TTRL_U_TANH: return tanhf(x);
    case TTRL_U_SIGMOID: return 1.f / (1.f + expf(-x));
    case TTRL_U_SQRT: return sqrtf(x);
    case TTRL_U_NEG: return -x;
    case TTRL_U_ADD_S: return x + s;
    case TTRL_U_MUL_S: return x * s;
    case TTRL_U_RSUB_S: return s - x;
    case TTRL_U_DIV_S: return x / s;
    case TTRL_U_EQZ: return x == 0.f ? 1.f : 0.f;
    case TTRL_U_GTZ: return x > 0.f ? 1.f : 0.f;
    case TTRL_U_ISFINITE: return isfinite(x) ? 1.f : 0.f;
    default: return x;
  }
}

__device__ inline float binary_op(int op, float a, float b) {
  switch (op) {
    case TTRL_B_ADD: return a + b;
    case TTRL_B_SUB: return a - b;
    case TTRL_B_MUL: return a * b;
    case TTRL_B_DIV: return a / b;
    case TTRL_B_RELU_BW: return b > 0.f ? a : 0.f;
    case TTRL_B_MAX: return fmaxf(a, b);
    case TTRL_B_MIN: return fminf(a, b);
    case TTRL_B_EQ: return a == b ? 1.f : 0.f;
    default: return a;
  }
}

__global__ __launch_bounds__(kEwThreads) void k_unary(int op, const float* __restrict__ a, float* __restrict__ y,
                                                      long n, float s) {
  for (long i = blockIdx.x * long(kEwThreads) + threadIdx.x; i < n; i += long(gridDim.x) * kEwThreads)
    y[i] = unary_op(op, a[i], s);
}

__global__ __launch_bounds__(kEwThreads) void k_binary(int op, const float* __restrict__ a,
                                                       const float* __restrict__ b, float* __restrict__ y, long n,
                                                       Dims d) {
  for (long i = blockIdx.x * long(kEwThreads) + threadIdx.x; i < n; i += long(gridDim.x) * kEwThreads) {
    long rem = i, ia = 0, ib = 0;
    for (int k = d.nd - 1; k >= 0; --k) {
      const long c = rem % d.shape[k];
      rem /= d.shape[k];
      ia += c * d.sa[k];
      ib += c * d.sb[k];
    }
    y[i] = binary_op(op, a[ia], b[ib]);
  }
}

__global__ __launch_bounds__(kEwThreads) void k_copy_strided(const float* __restrict__ a, float* __restrict__ y,
                                                             long n, Dims d) {
  for (long i = blockIdx.x * long(kEwThreads) + threadIdx.x; i < n; i += long(gridDim.x) * kEwThreads) {
    long rem = i, ia = 0, iy = 0;
    for (int k = d.nd - 1; k >= 0; --k) {
      const long c = rem % d.shape[k];
      rem /= d.shape[k];
      ia += c * d.sa[k];
      iy += c * d.sy[k];
    }
    y[iy] = a[ia];
  }
}

// Reduce the middle axis of a [outer][dim][inner] view, one thread per
// output, in index order (deterministic).
__global__ __launch_bounds__(kEwThreads) void k_reduce(int op, const float* __restrict__ a, float* __restrict__ y,
                                                       long outer, long dim, long inner) {
  const long n = outer * inner;
  for (long i = blockIdx.x * long(kEwThreads) + threadIdx.x; i < n; i += long(gridDim.x) * kEwThreads) {
    const long o = i / inner, in = i - o * inner;
    const float* p = a + o * dim * inner + in;
    if (op == TTRL_R_SUM) {
      float s = 0.f;
      for (long k = 0; k < dim; ++k) s += p[k * inner];
      y[i] = s;
    } else if (op == TTRL_R_MAX) {
      float m = p[0];
      for (long k = 1; k < dim; ++k) m = fmaxf(m, p[k * inner]);
      y[i] = m;
    } else {  // argmax, first index of the maximum
      float m = p[0];
      long best = 0;
      for (long k = 1; k < dim; ++k)
        if (p[k * inner] > m) {
          m = p[k * inner];
          best = k;
        }
      y[i] = float(best);
    }
  }
}

// Full sum of a long vector: one block, fixed order (strided partial sums
// per thread, then a block reduction).
__global__ __launch_bounds__(kEwThreads) void k_sum_all(const float* __restrict__ a, long n, float* __restrict__ y) {
  __shared__ float red[kEwThreads / 64];
  float s = 0.f;
  for (long i = threadIdx.x; i < n; i += kEwThreads) s += a[i];
  const float t = block_sum<kEwThreads>(s, red);
  if (threadIdx.x == 0) *y = t;
}

__global__ __launch_bounds__(kEwThreads) void k_onehot(const float* __restrict__ idx, float* __restrict__ y, long B,
                                                       int A) {
  const long n = B * A;
  for (long i = blockIdx.x * long(kEwThreads) + threadIdx.x; i < n; i += long(gridDim.x) * kEwThreads) {
    const long b = i / A;
    const int a = int(i - b * A);
    y[i] = (float(a) - idx[b]) == 0.f ? 1.f : 0.f;
  }
}

inline unsigned ew_grid(long n) {
  long b = (n + kEwThreads - 1) / kEwThreads;
  if (b < 1) b = 1;
  if (b > 4096) b = 4096;
  return unsigned(b);
}

int make_dims(int nd, const long* shape, const long* sa, const long* sb, const long* sy, Dims& d, long& n) {
  TTRL_REQUIRE(nd >= 1 && nd <= kMaxDims, "elementwise: rank %d outside [1, %d]", nd, kMaxDims);
  d.nd = nd;
  n = 1;
  for (int k = 0; k < nd; ++k) {
    TTRL_REQUIRE(shape[k] >= 0, "elementwise: negative extent");
    d.shape[k] = shape[k];
    d.sa[k] = sa ? sa[k] : 0;
    d.sb[k] = sb ? sb[k] : 0;
    d.sy[k] = sy ? sy[k] : 0;
    n *= shape[k];
  }
  return TTRL_OK;
}

}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_unary(ttrl_ctx* ctx, int op, const float* a, float* y, long n, float scalar) {
  TTRL_REQUIRE(ctx && ((a && y) || n == 0), "ttrl_unary: null argument");
  TTRL_REQUIRE(op >= 0 && op < TTRL_U_COUNT, "ttrl_unary: unknown op %d", op);
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_unary, dim3(ew_grid(n)), dim3(kEwThreads), 0, stream_of(ctx), op, a, y, n, scalar);
  return check_launch("ttrl_unary");
}

int ttrl_binary(ttrl_ctx* ctx, int op, const float* a, const float* b, float* y, int ndim, const long* shape,
                const long* stride_a, const long* stride_b) {
  TTRL_REQUIRE(ctx && a && b && y && shape && stride_a && stride_b, "ttrl_binary: null argument");
  TTRL_REQUIRE(op >= 0 && op < TTRL_B_COUNT, "ttrl_binary: unknown op %d", op);
  Dims d;
  long n = 0;
  int rc = make_dims(ndim, shape, stride_a, stride_b, nullptr, d, n);
  if (rc) return rc;
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_binary, dim3(ew_grid(n)), dim3(kEwThreads), 0, stream_of(ctx), op, a, b, y, n, d);
  return check_launch("ttrl_binary");
}

int ttrl_copy_strided(ttrl_ctx* ctx, const float* a, float* y, int ndim, const long* shape, const long* stride_a,
                      const long* stride_y) {
  TTRL_REQUIRE(ctx && a && y && shape && stride_a && stride_y, "ttrl_copy_strided: null argument");
  Dims d;
  long n = 0;
  int rc = make_dims(ndim, shape, stride_a, nullptr, stride_y, d, n);
  if (rc) return rc;
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_copy_strided, dim3(ew_grid(n)), dim3(kEwThreads), 0, stream_of(ctx), a, y, n, d);
  return check_launch("ttrl_copy_strided");
}

int ttrl_reduce(ttrl_ctx* ctx, int op, const float* a, float* y, long outer, long dim, long inner) {
  TTRL_REQUIRE(ctx && a && y, "ttrl_reduce: null argument");
  TTRL_REQUIRE(op >= 0 && op < TTRL_R_COUNT, "ttrl_reduce: unknown op %d", op);
  TTRL_REQUIRE(outer >= 1 && dim >= 1 && inner >= 1, "ttrl_reduce: empty extent");
  if (op == TTRL_R_SUM && outer == 1 && inner == 1) {
    hipLaunchKernelGGL(k_sum_all, dim3(1), dim3(kEwThreads), 0, stream_of(ctx), a, dim, y);
  } else {
    hipLaunchKernelGGL(k_reduce, dim3(ew_grid(outer * inner)), dim3(kEwThreads), 0, stream_of(ctx), op, a, y, outer,
                       dim, inner);
  }
  return check_launch("ttrl_reduce");
}

int ttrl_one_hot(ttrl_ctx* ctx, const float* indices, float* y, long batch, int num_classes) {
  TTRL_REQUIRE(ctx && indices && y, "ttrl_one_hot: null argument");
  TTRL_REQUIRE(batch >= 0 && num_classes > 0, "ttrl_one_hot: bad extents");
  if (batch == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_onehot, dim3(ew_grid(batch * num_classes)), dim3(kEwThreads), 0, stream_of(ctx), indices, y,
                     batch, num_classes);
  return check_launch("ttrl_one_hot");
}

}  // extern "C"
