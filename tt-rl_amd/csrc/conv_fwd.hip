// Convolution forward (implicit GEMM, bias / ReLU epilogue): the layer's
// patch layout picks one of three loader instantiations.
//   conv fwd + bias, input-scale fold   ttrl/engine/conv/forward.py:160-205
//   output size (H + 2p - k)/s + 1      ttrl/engine/conv/geometry.py:94-119
#include "conv.hpp"

namespace ttrl {
namespace {

template <int MODE, unsigned CFGS>
int conv_forward_mode(ttrl_ctx* ctx, const ConvGeo& g, int groups, const void* const* x, const float* const* wt,
                      const float* const* bias, float* const* y, float x_scale, int relu, const char* name) {
  const int K = g.C * g.KH * g.KW;
  LdConvFwd<MODE> la{g, {}, input_bytes(g)};
  LdColK lb;  // B(k, n=o) = Wt[k][o]
  EpStore ep;
  for (int i = 0; i < groups; ++i) {
    la.x[i] = x[i];
    lb.p[i] = wt[i];
    ep.C[i] = y[i];
    ep.bias[i] = bias ? bias[i] : nullptr;
  }
  lb.ld = g.O;
  lb.rows = g.O;
  lb.K = K;
  bool al = true;
  for (int i = 0; i < groups; ++i) al = al && (reinterpret_cast<uintptr_t>(wt[i]) & 15) == 0;
  lb.vec_ok(al);
  ep.M = g.M;
  ep.N = g.O;
  ep.ldc = g.O;
  ep.alpha = x_scale;
  ep.relu = relu;
  return run_gemm<CFGS>(ctx, la, lb, ep, g.M, g.O, K, groups, name);
}

int conv_forward(ttrl_ctx* ctx, const ConvGeo& g, int groups, const void* const* x, const float* const* wt,
                 const float* const* bias, float* const* y, float x_scale, int relu, const char* name) {
  bool xal = true;
  for (int i = 0; i < groups; ++i) {
    TTRL_REQUIRE(x[i] && wt[i] && y[i], "%s: null pointer in group %d", name, i);
    xal = xal && input_aligned(g, x[i]);
  }
  switch (patch_mode(g, xal)) {
    case kPatchNhwcVec:
      return conv_forward_mode<kPatchNhwcVec, kConvFwdCfgs>(ctx, g, groups, x, wt, bias, y, x_scale, relu, name);
    case kPatchU8Word:
      return conv_forward_mode<kPatchU8Word, kConvFwdCfgs>(ctx, g, groups, x, wt, bias, y, x_scale, relu, name);
    default:
      return conv_forward_mode<kPatchGeneral, kConvGeneralCfgs>(ctx, g, groups, x, wt, bias, y, x_scale, relu, name);
  }
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_conv_out_size(int size, int kernel, int stride, int padding, int* out) {
  TTRL_REQUIRE(out, "ttrl_conv_out_size: null out");
  TTRL_REQUIRE(kernel > 0 && stride > 0 && padding >= 0 && size > 0, "ttrl_conv_out_size: bad arguments");
  const int span = size + 2 * padding - kernel;
  TTRL_REQUIRE(span >= 0, "ttrl_conv_out_size: kernel %d larger than padded size %d", kernel, size + 2 * padding);
  TTRL_REQUIRE(span % stride == 0, "ttrl_conv_out_size: ragged geometry (size %d, kernel %d, stride %d, padding %d)",
               size, kernel, stride, padding);
  *out = span / stride + 1;
  return TTRL_OK;
}

int ttrl_conv2d_forward(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, const float* wt,
                        const float* bias, float* y, float x_scale, int relu) {
  TTRL_REQUIRE(ctx && x && wt && y, "ttrl_conv2d_forward: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  const void* xs[1] = {x};
  const float* ws[1] = {wt};
  const float* bs[1] = {bias};
  float* ys[1] = {y};
  return conv_forward(ctx, g, 1, xs, ws, bs, ys, x_scale, relu, "ttrl_conv2d_forward");
}

int ttrl_conv2d_forward_multi(ttrl_ctx* ctx, const ttrl_conv_geom* geom, int groups, const void* const* x,
                              const float* const* wt, const float* const* bias, float* const* y, float x_scale,
                              int relu) {
  TTRL_REQUIRE(ctx && x && wt && y, "ttrl_conv2d_forward_multi: null argument");
  TTRL_REQUIRE(groups >= 1 && groups <= kMaxGroups, "ttrl_conv2d_forward_multi: 1..%d groups", kMaxGroups);
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  return conv_forward(ctx, g, groups, x, wt, bias, y, x_scale, relu, "ttrl_conv2d_forward_multi");
}

}  // extern "C"
