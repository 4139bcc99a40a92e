// Convolution input gradient, per residue class (ih + p) mod s,
// (iw + p) mod s: inside one class every input pixel is reached by the same
// kernel taps, so each class is a plain GEMM and every dX element is
// written exactly once (no atomics).
//   dX = conv_transpose2d(dY, W)        ttrl/engine/conv/backward.py:33-42
#include "conv.hpp"

using namespace ttrl;

extern "C" {

int ttrl_conv2d_backward_input(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const float* dy, const float* ymask,
                               const float* wt, float* dx, const float* xmask, float x_scale, float beta) {
  TTRL_REQUIRE(ctx && dy && wt && dx, "ttrl_conv2d_backward_input: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  TTRL_REQUIRE(!g.u8, "ttrl_conv2d_backward_input: a uint8 frame input has no gradient");
  long reserved = 0;
  if (ymask) {
    dy = relu_mask_into_workspace(ctx, dy, ymask, long(g.M) * g.O, 0, 1, &reserved, &rc);
    if (rc) return rc;
  }
  for (int c0 = 0; c0 < g.S * g.S; c0 += kMaxGroups) {
    const ConvDxProblem p = conv_dx_problem(g, c0, dy, wt, dx, xmask, x_scale, beta);
    rc = run_gemm<kConvDxCfgs>(ctx, p.la, p.lb, p.ep, p.q.M, p.q.N, p.q.K, p.q.groups, "ttrl_conv2d_backward_input",
                               reserved);
    if (rc) return rc;
  }
  return TTRL_OK;
}

}  // extern "C"
