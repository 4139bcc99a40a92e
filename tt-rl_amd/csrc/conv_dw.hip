// Convolution weight gradient: dW = sum over pixels of patch^T dZ, the bias
// gradient folded in as an implicit ones row of the patch matrix.
//   dW = sum over taps of X-slice^T dY  ttrl/engine/conv/backward.py:45-78
#include "conv.hpp"

namespace ttrl {
namespace {

// bank not null: the split-K partials stay there and *out describes them.
template <int MODE, unsigned CFGS>
int conv_backward_weight_mode(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy,
                              float* dwt, float* db, float beta, long reserved, float* bank = nullptr,
                              ttrl_grad_source* out = nullptr) {
  const ConvDwProblem<MODE> p = conv_dw_problem<MODE>(g, x, x_scale, dy, dwt, db, beta);
  if (!bank)
    return run_gemm<CFGS>(ctx, p.la, p.lb, p.ep, p.q.M, p.q.N, p.q.K, 1, "ttrl_conv2d_backward_weight", reserved);
  GemmPlan plan{};
  const int rc = run_gemm_deferred<CFGS>(ctx, p.la, p.lb, p.ep, p.q.M, p.q.N, p.q.K, 1,
                                         "ttrl_conv2d_backward_weight_deferred", &plan, bank, kGradBankFloats);
  if (rc == TTRL_OK) *out = conv_dw_source(g, x_scale, dwt, db, bank, plan);
  return rc;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_conv2d_backward_weight_deferred(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                         const float* dy, const float* ymask, float* dwt, float* db, int bank,
                                         ttrl_grad_source* out) {
  TTRL_REQUIRE(ctx && x && dy && dwt && out, "ttrl_conv2d_backward_weight_deferred: null argument");
  TTRL_REQUIRE(bank >= 0 && bank < kGradBanks, "ttrl_conv2d_backward_weight_deferred: bank %d outside [0, %d)", bank,
               kGradBanks);
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  long reserved = 0;
  if (ymask) {
    dy = relu_mask_into_workspace(ctx, dy, ymask, long(g.M) * g.O, 0, 1, &reserved, &rc);
    if (rc) return rc;
  }
  float* b = ctx_grad_bank(ctx, bank);
  switch (patch_mode(g, input_aligned(g, x))) {
    case kPatchNhwcVec:
      return conv_backward_weight_mode<kPatchNhwcVec, kConvDwCfgs>(ctx, g, x, x_scale, dy, dwt, db, 0.f, reserved, b,
                                                                   out);
    case kPatchU8Word:
      return conv_backward_weight_mode<kPatchU8Word, kConvDwCfgs>(ctx, g, x, x_scale, dy, dwt, db, 0.f, reserved, b,
                                                                  out);
    default:
      return conv_backward_weight_mode<kPatchGeneral, kConvGeneralCfgs>(ctx, g, x, x_scale, dy, dwt, db, 0.f,
                                                                         reserved, b, out);
  }
}

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
