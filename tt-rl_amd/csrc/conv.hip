// Convolution as implicit GEMM on the FP32 MFMA core, for the Nature-CNN
// tower: forward with bias/ReLU epilogue (uint8 NCHW frames or fp32 NHWC
// activations), weight gradient with the bias gradient folded in as an
// implicit ones row, and an atomic-free input gradient.
//
// Layouts owned here (the reference's prepared layout is ttnn's business and
// is not reproduced; its logical weight is OIHW, ttrl/engine/conv/module.py:28-105):
//   fp32 activations   NHWC, [B][H][W][C]  (flattened-NHWC, ttrl/engine/conv/__init__.py:10-13)
//   uint8 frames       NCHW, [B][C][H][W]  (env frames, ttrl/spaces/obs.py:245-248)
//   weight master      Wt[k][O], k = (kh, kw, c) for NHWC inputs and
//                      k = (c, kh, kw) for NCHW uint8 inputs
//
// Reference semantics:
//   conv fwd + bias, input-scale fold   ttrl/engine/conv/forward.py:160-205
//   dW = sum over taps of X-slice^T dY  ttrl/engine/conv/backward.py:45-78
//   dX = conv_transpose2d(dY, W)        ttrl/engine/conv/backward.py:33-42
//   output size (H + 2p - k)/s + 1      ttrl/engine/conv/geometry.py:94-119
//
// The input gradient is computed per residue class (ih + p) mod s,
// (iw + p) mod s: inside one class every input pixel is reached by the same
// kernel taps (kh = ch + s*jh, kw = cw + s*jw), so each class is a plain GEMM
// over (jh, jw, o) and every dX element is written exactly once.
//
// Index arithmetic uses multiply-high division by the layer's constant
// extents (FDiv), precomputed on the host.
#include "tile_gemm.hpp"

#include <algorithm>

namespace ttrl {


struct ConvGeo {
  int B, C, H, W, O, KH, KW, S, P, OH, OW, u8;
  int M;                           // B * OH * OW
  FDiv d_ohow, d_ow, d_c, d_kw, d_khkw, d_o, d_tw;
  int TH, TW;                      // taps per class along h and w: ceil(K / S)
  // The input gradient's residue classes cls0 .. cls0+3 (one launch), by group.
  int cls0;
  int ih0[kMaxGroups], iw0[kMaxGroups], nh[kMaxGroups], nw[kMaxGroups];
  FDiv d_nhnw[kMaxGroups], d_nw[kMaxGroups];

  __device__ inline int kp() const { return C * KH * KW; }
  // (c, kh, kw) of patch index k, in this layer's k order.
  __device__ inline void split_k(int k, int& c, int& kh, int& kw) const {
    if (u8) {
      c = d_khkw.div(k);
      const int t = k - c * KH * KW;
      kh = d_kw.div(t);
      kw = t - kh * KW;
    } else {
      const int tap = d_c.div(k);
      c = k - tap * C;
      kh = d_kw.div(tap);
      kw = tap - kh * KW;
    }
  }
  __device__ inline void split_m(int m, int& b, int& oh, int& ow) const {
    b = d_ohow.div(m);
    const int rem = m - b * OH * OW;
    oh = d_ow.div(rem);
    ow = rem - oh * OW;
  }
};

// Patch elements of output pixel m at patch index k (zero outside the image).
struct ConvPatch {
  ConvGeo g;
  const void* x[kMaxGroups];

  // Element index of (m, k) in the input, or -1 outside the image.
  __device__ inline long index(int m, int k) const {
    if (m >= g.M || k >= g.kp()) return -1;
    int b, oh, ow, c, kh, kw;
    g.split_m(m, b, oh, ow);
    g.split_k(k, c, kh, kw);
    const int ih = oh * g.S + kh - g.P, iw = ow * g.S + kw - g.P;
    if (ih < 0 || ih >= g.H || iw < 0 || iw >= g.W) return -1;
    if (g.u8) return ((long(b) * g.C + c) * g.H + ih) * g.W + iw;
    return ((long(b) * g.H + ih) * g.W + iw) * g.C + c;
  }
  // Issue the loads of patch indices k..k+3 (k % 4 == 0) of pixel m.
  __device__ inline void issue4(int m, int k, int grp, Fetch4& f) const {
    f.m = f32x4{1.f, 1.f, 1.f, 1.f};
    if (m < g.M && k < g.kp()) {
      int b, oh, ow, c, kh, kw;
      g.split_m(m, b, oh, ow);
      g.split_k(k, c, kh, kw);
      const int ih = oh * g.S + kh - g.P, iw = ow * g.S + kw - g.P;
      if (g.u8) {
        // k..k+3 are kw..kw+3 of one kernel row when KW % 4 == 0.
        if ((g.KW & 3) == 0 && ((g.W & 3) == 0) && ((iw & 3) == 0) && k + 3 < g.kp()) {
          const bool in = ih >= 0 && ih < g.H && iw >= 0 && iw + 3 < g.W;
          const long i = in ? ((long(b) * g.C + c) * g.H + ih) * g.W + iw : 0;
          f.v.x = __uint_as_float(*reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(x[grp]) + i));
          f.ok = in ? (0xFu | kU8Word) : 0u;
          return;
        }
      } else if ((g.C & 3) == 0 && k + 3 < g.kp()) {
        // k..k+3 are channels c..c+3 of one tap.
        const bool in = ih >= 0 && ih < g.H && iw >= 0 && iw < g.W;
        const long i = in ? ((long(b) * g.H + ih) * g.W + iw) * g.C + c : 0;
        f.v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x[grp]) + i);
        f.ok = in ? 0xFu : 0u;
        return;
      }
    }
    f.ok = g.u8 ? kU8Each : 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long idx = index(m, k + j);
      const long i = idx < 0 ? 0 : idx;
      if (g.u8) f.v[j] = __uint_as_float(uint32_t(static_cast<const uint8_t*>(x[grp])[i]));
      else f.v[j] = static_cast<const float*>(x[grp])[i];
      f.ok |= uint32_t(idx >= 0) << j;
    }
  }
};

// Forward A operand: A(m, k) = patch(m, k).
struct LdConvFwd {
  static constexpr bool KCONTIG = true;
  ConvPatch p;
  __device__ inline bool masked(int) const { return false; }
  __device__ inline void issue(int r, int k, int grp, Fetch4& f) const { p.issue4(r, k, grp, f); }
};

// Weight-gradient A operand: A(r = k, k = m) = patch(m, r), with the ones row
// at r == kp when the bias gradient is wanted.
struct LdConvPatchT {
  static constexpr bool KCONTIG = false;
  ConvPatch p;
  int ones;
  __device__ inline bool masked(int) const { return false; }
  __device__ inline void issue(int r, int m, int grp, Fetch4& f) const {
    const int kp = p.g.kp();
    if (r + 3 < kp) {
      p.issue4(m, r, grp, f);
      return;
    }
    // The tail chunk: patch rows, then the ones row, then nothing.
    f.m = f32x4{1.f, 1.f, 1.f, 1.f};
    f.ok = 0;
    const bool mv = m < p.g.M;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = r + j;
      if (rr < kp) {
        const long idx = mv ? p.index(m, rr) : -1;
        const long i = idx < 0 ? 0 : idx;
        f.v[j] = p.g.u8 ? float(static_cast<const uint8_t*>(p.x[grp])[i]) : static_cast<const float*>(p.x[grp])[i];
        f.ok |= uint32_t(idx >= 0) << j;
      } else {
        f.v[j] = (ones && rr == kp) ? 1.f : 0.f;
        f.ok |= uint32_t(mv) << j;
      }
    }
  }
};

// Input-gradient A operand of class `cls`: A(r, k = (jh, jw, o)) = dZ at the
// output pixel that tap (kh, kw) = (ch + s*jh, cw + s*jw) connects to input
// pixel r; dZ = dY * [Y > 0] when a mask is given.
struct LdConvDxA {
  static constexpr bool KCONTIG = true;
  ConvGeo g;
  const float* dy;
  const float* ymask;
  // dZ element index, or -1 when the tap or the output pixel falls outside.
  __device__ inline long index(int r, int k, int grp) const {
    const int cls = g.cls0 + grp;
    const int rows = g.B * g.nh[grp] * g.nw[grp];
    if (r >= rows || k >= g.TH * g.TW * g.O) return -1;
    const int b = g.d_nhnw[grp].div(r);
    const int rem = r - b * g.nh[grp] * g.nw[grp];
    const int i = g.d_nw[grp].div(rem), j = rem - i * g.nw[grp];
    const int ch = cls / g.S, cw = cls - ch * g.S;
    const int ih = g.ih0[grp] + g.S * i, iw = g.iw0[grp] + g.S * j;
    const int jt = g.d_o.div(k), o = k - jt * g.O;
    const int jh = g.d_tw.div(jt), jw = jt - jh * g.TW;
    const int kh = ch + g.S * jh, kw = cw + g.S * jw;
    if (kh >= g.KH || kw >= g.KW) return -1;
    const int th = ih + g.P - kh, tw = iw + g.P - kw;
    if (th < 0 || tw < 0) return -1;
    const int oh = th / g.S, ow = tw / g.S;
    if (oh >= g.OH || ow >= g.OW) return -1;
    return ((long(b) * g.OH + oh) * g.OW + ow) * g.O + o;
  }
  __device__ inline bool masked(int) const { return ymask != nullptr; }
  __device__ inline void issue(int r, int k, int grp, Fetch4& f) const {
    if ((g.O & 3) == 0) {
      // k % 4 == 0 and O % 4 == 0: the four k share one tap and output pixel.
      const long idx = index(r, k, grp);
      const long i = idx < 0 ? 0 : idx;
      f.v = *reinterpret_cast<const f32x4*>(dy + i);
      if (ymask) f.m = *reinterpret_cast<const f32x4*>(ymask + i);
      f.ok = idx >= 0 ? 0xFu : 0u;
      return;
    }
    f.ok = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long idx = index(r, k + j, grp);
      const long i = idx < 0 ? 0 : idx;
      f.v[j] = dy[i];
      f.m[j] = ymask ? ymask[i] : 1.f;
      f.ok |= uint32_t(idx >= 0) << j;
    }
  }
};

// Input-gradient B operand of class `cls`: B(k = (jh, jw, o), n = c) =
// Wt[(kh, kw, c)][o]; stored here as rows n, k contiguous.
struct LdConvDxB {
  static constexpr bool KCONTIG = true;
  ConvGeo g;
  const float* wt;
  __device__ inline long index(int c, int k, int grp) const {
    const int cls = g.cls0 + grp;
    if (c >= g.C || k >= g.TH * g.TW * g.O) return -1;
    const int ch = cls / g.S, cw = cls - ch * g.S;
    const int jt = g.d_o.div(k), o = k - jt * g.O;
    const int jh = g.d_tw.div(jt), jw = jt - jh * g.TW;
    const int kh = ch + g.S * jh, kw = cw + g.S * jw;
    if (kh >= g.KH || kw >= g.KW) return -1;
    return ((long(kh) * g.KW + kw) * g.C + c) * g.O + o;
  }
  __device__ inline bool masked(int) const { return false; }
  __device__ inline void issue(int c, int k, int grp, Fetch4& f) const {
    if ((g.O & 3) == 0) {
      const long idx = index(c, k, grp);
      f.v = *reinterpret_cast<const f32x4*>(wt + (idx < 0 ? 0 : idx));
      f.ok = idx >= 0 ? 0xFu : 0u;
      return;
    }
    f.ok = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long idx = index(c, k + j, grp);
      f.v[j] = wt[idx < 0 ? 0 : idx];
      f.ok |= uint32_t(idx >= 0) << j;
    }
  }
};

// Input-gradient epilogue: class row r -> NHWC input pixel.
struct EpConvDx {
  ConvGeo g;
  float* dx;
  float alpha, beta;
  __device__ inline int rows(int grp) const { return g.B * g.nh[grp] * g.nw[grp]; }
  __device__ inline void store(int r, int c, float acc, int grp) const {
    if (r >= rows(grp) || c >= g.C) return;
    const int b = g.d_nhnw[grp].div(r);
    const int rem = r - b * g.nh[grp] * g.nw[grp];
    const int i = g.d_nw[grp].div(rem), j = rem - i * g.nw[grp];
    const int ih = g.ih0[grp] + g.S * i, iw = g.iw0[grp] + g.S * j;
    float* dst = dx + ((long(b) * g.H + ih) * g.W + iw) * g.C + c;
    float v = alpha * acc;
    if (beta != 0.f) v += beta * *dst;
    *dst = v;
  }
};

namespace {

// Residue-class tables of classes cls0 .. cls0+kMaxGroups-1 (empty past S*S).
void set_classes(ConvGeo& g, int cls0) {
  g.cls0 = cls0;
  for (int grp = 0; grp < kMaxGroups; ++grp) {
    const int cls = cls0 + grp;
    g.ih0[grp] = g.iw0[grp] = g.nh[grp] = g.nw[grp] = 0;
    g.d_nhnw[grp].set(1);
    g.d_nw[grp].set(1);
    if (cls >= g.S * g.S) continue;
    const int ch = cls / g.S, cw = cls % g.S;
    g.ih0[grp] = ((ch - g.P) % g.S + g.S) % g.S;
    g.iw0[grp] = ((cw - g.P) % g.S + g.S) % g.S;
    g.nh[grp] = g.ih0[grp] < g.H ? (g.H - g.ih0[grp] + g.S - 1) / g.S : 0;
    g.nw[grp] = g.iw0[grp] < g.W ? (g.W - g.iw0[grp] + g.S - 1) / g.S : 0;
    g.d_nhnw[grp].set(g.nh[grp] * g.nw[grp] > 0 ? g.nh[grp] * g.nw[grp] : 1);
    g.d_nw[grp].set(g.nw[grp] > 0 ? g.nw[grp] : 1);
  }
}

int make_geo(const ttrl_conv_geom* s, ConvGeo& g) {
  TTRL_REQUIRE(s, "conv: null geometry");
  TTRL_REQUIRE(s->batch > 0 && s->in_c > 0 && s->in_h > 0 && s->in_w > 0 && s->out_c > 0 && s->kernel > 0 &&
                   s->stride > 0 && s->padding >= 0,
               "conv: non-positive geometry field");
  const int span_h = s->in_h + 2 * s->padding - s->kernel;
  const int span_w = s->in_w + 2 * s->padding - s->kernel;
  TTRL_REQUIRE(span_h >= 0 && span_w >= 0, "conv: kernel %d larger than the padded input", s->kernel);
  TTRL_REQUIRE(span_h % s->stride == 0 && span_w % s->stride == 0,
               "conv: ragged geometry (in %dx%d, k %d, s %d, p %d) leaves input rows that feed no output",
               s->in_h, s->in_w, s->kernel, s->stride, s->padding);
  TTRL_REQUIRE(s->in_layout == TTRL_LAYOUT_NHWC_F32 || s->in_layout == TTRL_LAYOUT_NCHW_U8,
               "conv: unknown input layout %d", s->in_layout);
  g.B = s->batch;
  g.C = s->in_c;
  g.H = s->in_h;
  g.W = s->in_w;
  g.O = s->out_c;
  g.KH = g.KW = s->kernel;
  g.S = s->stride;
  g.P = s->padding;
  g.OH = span_h / s->stride + 1;
  g.OW = span_w / s->stride + 1;
  g.u8 = s->in_layout == TTRL_LAYOUT_NCHW_U8 ? 1 : 0;
  g.M = g.B * g.OH * g.OW;
  const long bigs[] = {long(g.B) * g.OH * g.OW, long(g.B) * g.H * g.W * g.C, long(g.C) * g.KH * g.KW * g.O};
  for (long v : bigs) TTRL_REQUIRE(v < (1L << 31), "conv: extent %ld exceeds 2^31", v);
  g.d_ohow.set(g.OH * g.OW);
  g.d_ow.set(g.OW);
  g.d_c.set(g.C);
  g.d_kw.set(g.KW);
  g.d_khkw.set(g.KH * g.KW);
  g.d_o.set(g.O);
  g.TH = (g.KH + g.S - 1) / g.S;
  g.TW = (g.KW + g.S - 1) / g.S;
  g.d_tw.set(g.TW);
  set_classes(g, 0);
  return TTRL_OK;
}

int conv_forward(ttrl_ctx* ctx, const ConvGeo& g, int groups, const void* const* x, const float* const* wt,
                 const float* const* bias, float* const* y, float x_scale, int relu, const char* name) {
  const int K = g.C * g.KH * g.KW;
  LdConvFwd la{ConvPatch{g, {}}};
  LdColK lb;  // B(k, n=o) = Wt[k][o]
  EpStore ep;
  for (int i = 0; i < groups; ++i) {
    TTRL_REQUIRE(x[i] && wt[i] && y[i], "%s: null pointer in group %d", name, i);
    la.p.x[i] = x[i];
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
  return run_gemm(ctx, la, lb, ep, g.M, g.O, K, groups, name);
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

int ttrl_conv2d_backward_weight(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                const float* dy, const float* ymask, float* dwt, float* db, float beta) {
  TTRL_REQUIRE(ctx && x && dy && dwt, "ttrl_conv2d_backward_weight: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  const int Kp = g.C * g.KH * g.KW;
  LdConvPatchT la{ConvPatch{g, {x}}, db ? 1 : 0};
  LdColK lb;  // B(r=o, k=m) = dZ[m][o]
  lb.p[0] = dy;
  lb.mask[0] = ymask;
  lb.ld = g.O;
  lb.rows = g.O;
  lb.K = g.M;
  lb.vec_ok(((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(ymask)) & 15) == 0);
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
  return run_gemm(ctx, la, lb, ep, ep.M, g.O, g.M, 1, "ttrl_conv2d_backward_weight");
}

int ttrl_conv2d_backward_input(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const float* dy, const float* ymask,
                               const float* wt, float* dx, float x_scale, float beta) {
  TTRL_REQUIRE(ctx && dy && wt && dx, "ttrl_conv2d_backward_input: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  TTRL_REQUIRE(!g.u8, "ttrl_conv2d_backward_input: a uint8 frame input has no gradient");
  const int Kd = g.TH * g.TW * g.O;
  const int classes = g.S * g.S;
  // One launch covers up to kMaxGroups residue classes; the largest class
  // (ih0 = iw0 = 0) has ceil(H/S) * ceil(W/S) pixels per image.
  const int Mmax = g.B * ((g.H + g.S - 1) / g.S) * ((g.W + g.S - 1) / g.S);
  for (int c0 = 0; c0 < classes; c0 += kMaxGroups) {
    const int n = std::min(kMaxGroups, classes - c0);
    set_classes(g, c0);
    LdConvDxA la{g, dy, ymask};
    LdConvDxB lb{g, wt};
    EpConvDx ep{g, dx, x_scale, beta};
    rc = run_gemm(ctx, la, lb, ep, Mmax, g.C, Kd, n, "ttrl_conv2d_backward_input");
    if (rc) return rc;
  }
  return TTRL_OK;
}

}  // extern "C"
