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
#include "tile_gemm.hpp"

namespace ttrl {

struct ConvGeo {
  int B, C, H, W, O, KH, KW, S, P, OH, OW, u8;
  __device__ inline int kp() const { return C * KH * KW; }
  // (c, kh, kw) of patch index k, in this layer's k order.
  __device__ inline void split_k(int k, int& c, int& kh, int& kw) const {
    if (u8) {
      c = k / (KH * KW);
      const int t = k - c * KH * KW;
      kh = t / KW;
      kw = t - kh * KW;
    } else {
      const int tap = k / C;
      c = k - tap * C;
      kh = tap / KW;
      kw = tap - kh * KW;
    }
  }
};

// Patch value of output pixel m at patch index k (zero outside the image).
struct ConvPatch {
  ConvGeo g;
  const float* xf;
  const uint8_t* xu;

  __device__ inline float at(int m, int k) const {
    const int M = g.B * g.OH * g.OW;
    if (m >= M || k >= g.kp()) return 0.f;
    const int b = m / (g.OH * g.OW);
    const int rem = m - b * g.OH * g.OW;
    const int oh = rem / g.OW, ow = rem - oh * g.OW;
    int c, kh, kw;
    g.split_k(k, c, kh, kw);
    const int ih = oh * g.S + kh - g.P, iw = ow * g.S + kw - g.P;
    if (ih < 0 || ih >= g.H || iw < 0 || iw >= g.W) return 0.f;
    if (g.u8) return float(xu[((long(b) * g.C + c) * g.H + ih) * g.W + iw]);
    return xf[((long(b) * g.H + ih) * g.W + iw) * g.C + c];
  }
  // Four consecutive patch indices k..k+3 (k % 4 == 0) of pixel m.
  __device__ inline f32x4 at4(int m, int k) const {
    const int M = g.B * g.OH * g.OW;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (m >= M || k >= g.kp()) return v;
    const int b = m / (g.OH * g.OW);
    const int rem = m - b * g.OH * g.OW;
    const int oh = rem / g.OW, ow = rem - oh * g.OW;
    int c, kh, kw;
    g.split_k(k, c, kh, kw);
    const int ih = oh * g.S + kh - g.P, iw = ow * g.S + kw - g.P;
    if (g.u8) {
      // k..k+3 are kw..kw+3 of one kernel row when KW % 4 == 0.
      if ((g.KW & 3) == 0 && ih >= 0 && ih < g.H && iw >= 0 && iw + 3 < g.W && ((iw & 3) == 0) &&
          ((g.W & 3) == 0)) {
        const uint32_t w4 =
            *reinterpret_cast<const uint32_t*>(xu + ((long(b) * g.C + c) * g.H + ih) * g.W + iw);
        v.x = float(w4 & 0xff);
        v.y = float((w4 >> 8) & 0xff);
        v.z = float((w4 >> 16) & 0xff);
        v.w = float(w4 >> 24);
        return v;
      }
    } else if ((g.C & 3) == 0) {
      // k..k+3 are channels c..c+3 of one tap.
      if (ih < 0 || ih >= g.H || iw < 0 || iw >= g.W) return v;
      return *reinterpret_cast<const f32x4*>(xf + ((long(b) * g.H + ih) * g.W + iw) * g.C + c);
    }
    v.x = at(m, k);
    v.y = at(m, k + 1);
    v.z = at(m, k + 2);
    v.w = at(m, k + 3);
    return v;
  }
};

// Forward A operand: A(m, k) = patch(m, k).
struct LdConvFwd {
  static constexpr bool KCONTIG = true;
  ConvPatch p;
  __device__ inline f32x4 load4(int r, int k, int) const { return p.at4(r, k); }
};

// Weight-gradient A operand: A(r = k, k = m) = patch(m, r), with the ones row
// at r == kp when the bias gradient is wanted.
struct LdConvPatchT {
  static constexpr bool KCONTIG = false;
  ConvPatch p;
  int ones;
  __device__ inline f32x4 load4(int r, int m, int) const {
    const int kp = p.g.kp();
    const int M = p.g.B * p.g.OH * p.g.OW;
    if (m >= M) return f32x4{0.f, 0.f, 0.f, 0.f};
    if (r + 3 < kp) return p.at4(m, r);
    f32x4 v;
    v.x = r < kp ? p.at(m, r) : (ones && r == kp ? 1.f : 0.f);
    v.y = r + 1 < kp ? p.at(m, r + 1) : (ones && r + 1 == kp ? 1.f : 0.f);
    v.z = r + 2 < kp ? p.at(m, r + 2) : (ones && r + 2 == kp ? 1.f : 0.f);
    v.w = r + 3 < kp ? p.at(m, r + 3) : (ones && r + 3 == kp ? 1.f : 0.f);
    return v;
  }
};

// Residue-class bookkeeping of the input gradient.
struct DxClass {
  int ch, cw, ih0, iw0, nh, nw, rows;
};

__device__ inline DxClass dx_class(const ConvGeo& g, int cls) {
  DxClass d;
  d.ch = cls / g.S;
  d.cw = cls - d.ch * g.S;
  d.ih0 = ((d.ch - g.P) % g.S + g.S) % g.S;
  d.iw0 = ((d.cw - g.P) % g.S + g.S) % g.S;
  d.nh = d.ih0 < g.H ? (g.H - d.ih0 + g.S - 1) / g.S : 0;
  d.nw = d.iw0 < g.W ? (g.W - d.iw0 + g.S - 1) / g.S : 0;
  d.rows = g.B * d.nh * d.nw;
  return d;
}

// Input-gradient A operand of class `cls`: A(r, k = (jh, jw, o)) = dZ at the
// output pixel that tap (kh, kw) = (ch + s*jh, cw + s*jw) connects to input
// pixel r; dZ = dY * [Y > 0] when a mask is given.
struct LdConvDxA {
  static constexpr bool KCONTIG = true;
  ConvGeo g;
  const float* dy;
  const float* ymask;
  int TW;
  // dZ element (input pixel r of class cls, k = (jh, jw, o)); index < 0 when
  // the tap or the output pixel falls outside the layer.
  __device__ inline long index(const DxClass& d, int r, int k) const {
    const int Kd = ((g.KH + g.S - 1) / g.S) * TW * g.O;
    if (r >= d.rows || k >= Kd) return -1;
    const int b = r / (d.nh * d.nw);
    const int rem = r - b * d.nh * d.nw;
    const int i = rem / d.nw, j = rem - i * d.nw;
    const int ih = d.ih0 + g.S * i, iw = d.iw0 + g.S * j;
    const int jt = k / g.O, o = k - jt * g.O;
    const int jh = jt / TW, jw = jt - jh * TW;
    const int kh = d.ch + g.S * jh, kw = d.cw + g.S * jw;
    if (kh >= g.KH || kw >= g.KW) return -1;
    const int th = ih + g.P - kh, tw = iw + g.P - kw;
    if (th < 0 || tw < 0) return -1;
    const int oh = th / g.S, ow = tw / g.S;
    if (oh >= g.OH || ow >= g.OW) return -1;
    return ((long(b) * g.OH + oh) * g.OW + ow) * g.O + o;
  }
  __device__ inline float at(const DxClass& d, int r, int k) const {
    const long i = index(d, r, k);
    if (i < 0) return 0.f;
    return (!ymask || ymask[i] > 0.f) ? dy[i] : 0.f;
  }
  __device__ inline f32x4 load4(int r, int k, int cls) const {
    const DxClass d = dx_class(g, cls);
    if ((g.O & 3) == 0) {
      // k % 4 == 0 and O % 4 == 0: the four k share one tap and output pixel.
      const long i = index(d, r, k);
      if (i < 0) return f32x4{0.f, 0.f, 0.f, 0.f};
      f32x4 v = *reinterpret_cast<const f32x4*>(dy + i);
      if (ymask) {
        const f32x4 mk = *reinterpret_cast<const f32x4*>(ymask + i);
        v.x = mk.x > 0.f ? v.x : 0.f;
        v.y = mk.y > 0.f ? v.y : 0.f;
        v.z = mk.z > 0.f ? v.z : 0.f;
        v.w = mk.w > 0.f ? v.w : 0.f;
      }
      return v;
    }
    return f32x4{at(d, r, k), at(d, r, k + 1), at(d, r, k + 2), at(d, r, k + 3)};
  }
};

// Input-gradient B operand of class `cls`: B(k = (jh, jw, o), n = c) =
// Wt[(kh, kw, c)][o]; stored here as rows n, k contiguous.
struct LdConvDxB {
  static constexpr bool KCONTIG = true;
  ConvGeo g;
  const float* wt;
  int TW;
  __device__ inline long index(int c, int k, int cls) const {
    const int Kd = ((g.KH + g.S - 1) / g.S) * TW * g.O;
    if (c >= g.C || k >= Kd) return -1;
    const int ch = cls / g.S, cw = cls - ch * g.S;
    const int jt = k / g.O, o = k - jt * g.O;
    const int jh = jt / TW, jw = jt - jh * TW;
    const int kh = ch + g.S * jh, kw = cw + g.S * jw;
    if (kh >= g.KH || kw >= g.KW) return -1;
    return ((long(kh) * g.KW + kw) * g.C + c) * g.O + o;
  }
  __device__ inline float at(int c, int k, int cls) const {
    const long i = index(c, k, cls);
    return i < 0 ? 0.f : wt[i];
  }
  __device__ inline f32x4 load4(int c, int k, int cls) const {
    if ((g.O & 3) == 0) {
      const long i = index(c, k, cls);
      if (i < 0) return f32x4{0.f, 0.f, 0.f, 0.f};
      return *reinterpret_cast<const f32x4*>(wt + i);
    }
    return f32x4{at(c, k, cls), at(c, k + 1, cls), at(c, k + 2, cls), at(c, k + 3, cls)};
  }
};

// Input-gradient epilogue: class row r -> NHWC input pixel.
struct EpConvDx {
  ConvGeo g;
  float* dx;
  float alpha, beta;
  __device__ inline int rows(int cls) const { return dx_class(g, cls).rows; }
  __device__ inline void store(int r, int c, float acc, int cls) const {
    const DxClass d = dx_class(g, cls);
    if (r >= d.rows || c >= g.C) return;
    const int b = r / (d.nh * d.nw);
    const int rem = r - b * d.nh * d.nw;
    const int i = rem / d.nw, j = rem - i * d.nw;
    const int ih = d.ih0 + g.S * i, iw = d.iw0 + g.S * j;
    float* dst = dx + ((long(b) * g.H + ih) * g.W + iw) * g.C + c;
    float v = alpha * acc;
    if (beta != 0.f) v += beta * *dst;
    *dst = v;
  }
};

namespace {

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
  TTRL_REQUIRE(s->in_layout == TTRL_LAYOUT_NHWC_F32 || s->in_layout == TTRL_LAYOUT_NCHW_U8,
               "conv: unknown input layout %d", s->in_layout);
  return TTRL_OK;
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
  const int M = g.B * g.OH * g.OW, K = g.C * g.KH * g.KW;
  LdConvFwd la{ConvPatch{g, static_cast<const float*>(x), static_cast<const uint8_t*>(x)}};
  LdColK lb;  // B(k, n=o) = Wt[k][o]
  lb.p = wt;
  lb.ld = g.O;
  lb.rows = g.O;
  lb.K = K;
  lb.vec = (g.O % 4) == 0;
  EpStore ep;
  ep.M = M;
  ep.N = g.O;
  ep.C = y;
  ep.ldc = g.O;
  ep.alpha = x_scale;
  ep.bias = bias;
  ep.relu = relu;
  return run_gemm(ctx, la, lb, ep, M, g.O, K, 1, "ttrl_conv2d_forward");
}

int ttrl_conv2d_backward_weight(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                const float* dy, const float* ymask, float* dwt, float* db, float beta) {
  TTRL_REQUIRE(ctx && x && dy && dwt, "ttrl_conv2d_backward_weight: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  const int M = g.B * g.OH * g.OW, Kp = g.C * g.KH * g.KW;
  LdConvPatchT la{ConvPatch{g, static_cast<const float*>(x), static_cast<const uint8_t*>(x)}, db ? 1 : 0};
  LdColK lb;  // B(r=o, k=m) = dZ[m][o]
  lb.p = dy;
  lb.ld = g.O;
  lb.rows = g.O;
  lb.K = M;
  lb.mask = ymask;
  lb.vec = (g.O % 4) == 0;
  EpStore ep;
  ep.M = db ? Kp + 1 : Kp;
  ep.N = g.O;
  ep.C = dwt;
  ep.ldc = g.O;
  ep.rsplit = Kp;
  ep.Cr = db;
  ep.alpha = x_scale;  // d/dW of conv(s*x, W) = s * dW(x, dY); the bias row is unscaled
  ep.alpha_r = 1.f;
  ep.beta = beta;
  return run_gemm(ctx, la, lb, ep, ep.M, g.O, M, 1, "ttrl_conv2d_backward_weight");
}

int ttrl_conv2d_backward_input(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const float* dy, const float* ymask,
                               const float* wt, float* dx, float x_scale, float beta) {
  TTRL_REQUIRE(ctx && dy && wt && dx, "ttrl_conv2d_backward_input: null argument");
  ConvGeo g;
  int rc = make_geo(geom, g);
  if (rc) return rc;
  TTRL_REQUIRE(!g.u8, "ttrl_conv2d_backward_input: a uint8 frame input has no gradient");
  const int TH = (g.KH + g.S - 1) / g.S, TW = (g.KW + g.S - 1) / g.S;
  const int Kd = TH * TW * g.O;
  const int classes = g.S * g.S;
  // The largest class: ih0 = 0 gives ceil(H/S) rows per dimension.
  const int Mmax = g.B * ((g.H + g.S - 1) / g.S) * ((g.W + g.S - 1) / g.S);
  LdConvDxA la{g, dy, ymask, TW};
  LdConvDxB lb{g, wt, TW};
  EpConvDx ep{g, dx, x_scale, beta};
  return run_gemm(ctx, la, lb, ep, Mmax, g.C, Kd, classes, "ttrl_conv2d_backward_input");
}

}  // extern "C"
