// Convolution weight gradient: dW = sum over pixels of patch^T dZ, the bias
// gradient folded in as an implicit ones row of the patch matrix.
//   dW = sum over taps of X-slice^T dY  ttrl/engine/conv/backward.py:45-78
#include "conv.hpp"

namespace ttrl {
namespace {

template <int MODE, unsigned CFGS>
int conv_backward_weight_mode(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy,
                              float* dwt, float* db, float beta, long reserved) {
  const int Kp = g.C * g.KH * g.KW;
  LdConvPatchT<MODE> la{g, {x}, input_bytes(g), db ? 1 : 0};
  LdColK lb;  // B(r=o, k=m) = dZ[m][o]
  lb.p[0] = dy;
  lb.ld = g.O;
  lb.rows = g.O;
  lb.K = g.M;
  lb.vec_ok((reinterpret_cast<uintptr_t>(dy) & 15) == 0);
  EpStore ep;
  ep.M = db ? Kp + 1 : Kp;
  ep.N = g.O;
  ep.C[0] = dwt;
  ep.ldc = g.O;
  ep.rsplit = Kp;
  ep.Cr[0] = db;
  ep.alpha = x_scale;  // d/dW of conv(s*x, W) = s * dW(x, dY); the bias row is unscaled
  ep.alpha_r = 1.f;
  ep.beta = beta;
  return run_gemm<CFGS>(ctx, la, lb, ep, ep.M, g.O, g.M, 1, "ttrl_conv2d_backward_weight", reserved);
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_conv2d_backward_weight(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                const float* dy, const float* ymask, float* dwt, float* db, float beta) {
  TTRL_REQUIRE(ctx && x && dy && dwt, "ttrl_conv2d_backward_weight: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  long reserved = 0;
  if (ymask) {
    dy = relu_mask_into_workspace(ctx, dy, ymask, long(g.M) * g.O, 0, 1, &reserved, &rc);
    if (rc) return rc;
  }
  switch (patch_mode(g, input_aligned(g, x))) {
    case kPatchNhwcVec:
      return conv_backward_weight_mode<kPatchNhwcVec, kConvDwCfgs>(ctx, g, x, x_scale, dy, dwt, db, beta, reserved);
    case kPatchU8Word:
      return conv_backward_weight_mode<kPatchU8Word, kConvDwCfgs>(ctx, g, x, x_scale, dy, dwt, db, beta, reserved);
    default:
      return conv_backward_weight_mode<kPatchGeneral, kConvGeneralCfgs>(ctx, g, x, x_scale, dy, dwt, db, beta,
                                                                         reserved);
  }
}

}  // extern "C"
