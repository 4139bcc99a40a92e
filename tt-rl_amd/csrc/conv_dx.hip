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
  const int Kd = g.TH * g.TW * g.O;
  const int classes = g.S * g.S;
  // One launch covers up to kMaxGroups residue classes; the largest class
  // (ih0 = iw0 = 0) has ceil(H/S) * ceil(W/S) pixels per image.
  const int Mmax = g.B * ((g.H + g.S - 1) / g.S) * ((g.W + g.S - 1) / g.S);
  for (int c0 = 0; c0 < classes; c0 += kMaxGroups) {
    const int n = std::min(kMaxGroups, classes - c0);
    set_classes(g, c0);
    LdConvDxA la{g, dy, uint32_t(long(g.M) * g.O * 4)};
    LdConvDxB lb{g, wt, uint32_t(long(g.C) * g.KH * g.KW * g.O * 4)};
    EpConvDx ep{g, dx, xmask, x_scale, beta};
    rc = run_gemm<kConvDxCfgs>(ctx, la, lb, ep, Mmax, g.C, Kd, n, "ttrl_conv2d_backward_input", reserved);
    if (rc) return rc;
  }
  return TTRL_OK;
}

}  // extern "C"
