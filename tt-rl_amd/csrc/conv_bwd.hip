// A convolution layer's whole backward: weight (+ bias) gradient and input
// gradient in one call.  The two GEMMs are independent given dZ, so the
// weight gradient and the first launch of the input gradient (its first
// four residue classes) can run as one paired launch, which saves a launch
// but makes both problems take one tile shape; at large batches the two as
// separate launches, each with its own tile shape, are faster.  Both calls
// (the plain one and the one that leaves the weight gradient's split-K
// partials to the optimizer step) time the two ways once per geometry
// (outside capture, on scratch outputs) and keep the faster for the context.
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

// The two gradients as separate launches, each GEMM with its own plan; bank
// as for conv_backward_pair.
template <int MODE>
int conv_backward_split(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy,
                        const float* wt, float* dwt, float* db, float beta_w, float* dx, const float* xmask,
                        float beta_x, long reserved, float* bank = nullptr, ttrl_grad_source* out = nullptr) {
  constexpr unsigned kDw = MODE == kPatchGeneral ? kConvGeneralCfgs : kConvDwCfgs;
  const ConvDwProblem<MODE> w = conv_dw_problem<MODE>(g, x, x_scale, dy, dwt, db, beta_w);
  int rc = TTRL_OK;
  if (bank) {
    GemmPlan plan{};
    rc = run_gemm_deferred<kDw>(ctx, w.la, w.lb, w.ep, w.q.M, w.q.N, w.q.K, 1, "ttrl_conv2d_backward_deferred",
                                &plan, bank, kGradBankFloats);
    if (rc == TTRL_OK) *out = conv_dw_source(g, x_scale, dwt, db, bank, plan);
  } else {
    rc = run_gemm<kDw>(ctx, w.la, w.lb, w.ep, w.q.M, w.q.N, w.q.K, 1, "ttrl_conv2d_backward", reserved);
  }
  for (int c0 = 0; c0 < g.S * g.S && rc == TTRL_OK; c0 += kMaxGroups) {
    const ConvDxProblem d = conv_dx_problem(g, c0, dy, wt, dx, xmask, x_scale, beta_x);
    rc = run_gemm<kConvDxCfgs>(ctx, d.la, d.lb, d.ep, d.q.M, d.q.N, d.q.K, d.q.groups, "ttrl_conv2d_backward",
                               reserved);
  }
  return rc;
}

// Whether the paired launch is the faster way for this geometry.  Kept in
// the context's plan table as {cfg 1: pair, 0: separate; 0, 0, 0, 1, 0}, so
// it is exported and imported with the GEMM plans and every later call,
// eager or captured, takes the same path; an entry of any other form (an
// imported table's) is decided again and replaced.  Without timing (under
// capture, or tuning off) a pair is taken for at most 4096 output pixels,
// where the saved launch matters most.
inline GemmPlan pair_choice(bool pair) { return GemmPlan{pair ? 1 : 0, 0, 0, 0, 1, 0}; }
inline bool is_pair_choice(const GemmPlan& p) {
  return (p.cfg == 0 || p.cfg == 1) && p.bm == 0 && p.bn == 0 && p.tbk == 0 && p.splits == 1 && p.kchunk == 0;
}
template <int MODE>
bool pair_is_faster(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy,
                    const float* wt, const float* xmask, long reserved, float* bank) {
  char keybuf[192];
  snprintf(keybuf, sizeof(keybuf), "ttrl_conv2d_backward:pair|%d|%d|%d|%d|%d|%d|%d|%d|%d|%d|%ld|%d|%d", MODE, g.B,
           g.C, g.H, g.W, g.O, g.KH, g.KW, g.S, g.P, reserved, xmask ? 1 : 0, bank ? 1 : 0);
  const std::string key(keybuf);
  if (const GemmPlan* hit = ctx_plan_find(ctx, key))
    if (is_pair_choice(*hit)) return hit->cfg == 1;
  bool pair = long(g.M) <= 4096;
  hipEvent_t e0, e1;
  if (!ctx_capturing(ctx) && gemm_tuning_enabled() && ctx_tune_events(ctx, &e0, &e1)) {
    const size_t nw = size_t(g.KH) * g.KW * g.C * g.O, nx = size_t(g.B) * g.H * g.W * g.C;
    float* out = nullptr;
    if (hipMalloc(&out, (nw + size_t(g.O) + nx) * sizeof(float)) == hipSuccess) {
      float *sw = out, *sb = out + nw, *sx = out + nw + g.O;
      hipStream_t st = stream_of(ctx);
      int rc = TTRL_OK;
      ttrl_grad_source src{};  // the deferred form's partials go to the bank the real call then overwrites
      auto paired = [&] {
        if (rc == TTRL_OK) rc = conv_backward_pair<MODE>(ctx, g, x, x_scale, dy, wt, sw, sb, 0.f, sx, xmask, 0.f,
                                                         reserved, bank, &src);
      };
      auto split = [&] {
        if (rc == TTRL_OK) rc = conv_backward_split<MODE>(ctx, g, x, x_scale, dy, wt, sw, sb, 0.f, sx, xmask, 0.f,
                                                          reserved, bank, &src);
      };
      paired();  // first runs: each GEMM's own plan is tuned here
      split();
      const float tp = rc == TTRL_OK ? time_best_of(e0, e1, st, paired) : -1.f;
      const float ts = rc == TTRL_OK ? time_best_of(e0, e1, st, split) : -1.f;
      if (tp > 0.f && ts > 0.f) pair = tp <= ts;
      if (gemm_tuning_log())
        fprintf(stderr, "[ttrl gemm tune] conv2d backward B=%d C=%d %dx%d O=%d k=%d s=%d: pair %.2f us, "
                "separate %.2f us\n", g.B, g.C, g.H, g.W, g.O, g.KH, g.S, tp * 1e3f / 3.f, ts * 1e3f / 3.f);
      (void)hipStreamSynchronize(st);
      (void)hipFree(out);
      (void)hipGetLastError();
    }
  }
  ctx_plan_store(ctx, key, pair_choice(pair));
  return pair;
}

template <int MODE>
int conv_backward_chosen(ttrl_ctx* ctx, const ConvGeo& g, const void* x, float x_scale, const float* dy,
                         const float* wt, float* dwt, float* db, float beta_w, float* dx, const float* xmask,
                         float beta_x, long reserved, float* bank = nullptr, ttrl_grad_source* out = nullptr) {
  if (pair_is_faster<MODE>(ctx, g, x, x_scale, dy, wt, xmask, reserved, bank))
    return conv_backward_pair<MODE>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x, reserved, bank,
                                    out);
  return conv_backward_split<MODE>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x, reserved, bank,
                                   out);
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
    return conv_backward_chosen<kPatchNhwcVec>(ctx, g, x, x_scale, dy, wt, dwt, db, 0.f, dx, xmask, beta_x, reserved,
                                               b, out);
  return conv_backward_chosen<kPatchGeneral>(ctx, g, x, x_scale, dy, wt, dwt, db, 0.f, dx, xmask, beta_x, reserved,
                                             b, out);
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
    return conv_backward_chosen<kPatchNhwcVec>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x,
                                               reserved);
  return conv_backward_chosen<kPatchGeneral>(ctx, g, x, x_scale, dy, wt, dwt, db, beta_w, dx, xmask, beta_x,
                                             reserved);
}

}  // extern "C"
