// A convolution layer's whole backward: weight (+ bias) gradient and input
// gradient in one call.  The two GEMMs are independent given dZ, so the
// weight gradient and the first launch of the input gradient (its first
// four residue classes) run as one paired launch.
//   dW = sum over taps of X-slice^T dY  ttrl/engine/conv/backward.py:45-78
//   dX = conv_transpose2d(dY, W)        ttrl/engine/conv/backward.py:33-42
#include "conv.hpp"

namespace ttrl {
namespace {

// One tile shape for both GEMMs of a pair.
constexpr unsigned kConvPairCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x32K2) | cfg_bit(T64x32K2);

// bank not null: the weight gradient's split-K partials stay there (room
// for kGradBankFloats) and *out describes them.
template <int MODE>
int conv_backward_pair(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy, const float* wt,
                       float* dwt, float* db, float beta_w, float* dx, const float* xmask, float beta_x,
                       long reserved, float* bank = nullptr, ttrl_grad_source* out = nullptr) {
  const ConvDwProblem<MODE> w = conv_dw_problem<MODE>(g, x, x_scale, dy, dwt, db, beta_w);
  int rc = TTRL_OK;
  for (int c0 = 0; c0 < g.S * g.S && rc == TTRL_OK; c0 += kMaxGroups) {
    const ConvDxProblem d = conv_dx_problem(g, c0, dy, wt, dx, xmask, x_scale, beta_x);
    if (c0 == 0) {
      GemmPlan p1{};
      rc = run_gemm_pair<kConvPairCfgs>(ctx, w.la, w.lb, w.ep, w.q, d.la, d.lb, d.ep, d.q, "ttrl_conv2d_backward",
                                        reserved, bank, bank ? kGradBankFloats : 0, &p1);
      if (rc == TTRL_OK && bank) *out = conv_dw_source(g, x_scale, dwt, db, bank, p1);
    } else
      rc = run_gemm<kConvDxCfgs>(ctx, d.la, d.lb, d.ep, d.q.M, d.q.N, d.q.K, d.q.groups, "ttrl_conv2d_backward",
                                 reserved);
  }
  return rc;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_conv2d_backward_deferred(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                  const float* dy, const float* ymask, const float* wt, float* dwt, float* db,
                                  float* dx, const float* xmask, float beta_x, int bank, ttrl_grad_source* out) {
  TTRL_REQUIRE(ctx && x && dy && wt && dwt && dx && out, "ttrl_conv2d_backward_deferred: null argument");
  TTRL_REQUIRE(bank >= 0 && bank < kGradBanks, "ttrl_conv2d_backward_deferred: bank %d outside [0, %d)", bank,
               kGradBanks);
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  TTRL_REQUIRE(!g.u8, "ttrl_conv2d_backward_deferred: a uint8 frame input has no gradient");
  long reserved = 0;
  if (ymask) {
    dy = relu_mask_into_workspace(ctx, dy, ymask, long(g.M) * g.O, 0, 1, &reserved, &rc);
    if (rc) return rc;
  }
  float* b = ctx_grad_bank(ctx, bank);
  if (patch_mode(g, input_aligned(g, x)) == kPatchNhwcVec)
    return conv_backward_pair<kPatchNhwcVec>(ctx, g, x, x_scale, dy, wt, dwt, db, 0.f, dx, xmask, beta_x, reserved, b,
                                             out);
  return conv_backward_pair<kPatchGeneral>(ctx, g, x, x_scale, dy, wt, dwt, db, 0.f, dx, xmask, beta_x, reserved, b,
                                           out);
}

int ttrl_conv2d_backward(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale, const float* dy,
                         const float* ymask, const float* wt, float* dwt, float* db, float beta_w, float* dx,
                         const float* xmask, float beta_x) {
  TTRL_REQUIRE(ctx && x && dy && wt && dwt && dx, "ttrl_conv2d_backward: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  TTRL_REQUIRE(!g.u8, "ttrl_conv2d_backward: a uint8 frame input has no gradient");
  long reserved = 0;
  if (ymask) {
    dy = relu_mask_into_workspace(ctx, dy, ymask, long(g.M) * g.O, 0, 1, &reserved, &rc);
    if (rc) return rc;
  }
  if (patch_mode(g, input_aligned(g, x)) == kPatchNhwcVec)
    return conv_backward_pair<kPatchNhwcVec>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x,
                                             reserved);
  return conv_backward_pair<kPatchGeneral>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x, reserved);
}

}  // extern "C"
