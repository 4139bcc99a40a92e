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
#pragma once

#include "tile_gemm.hpp"

#include <algorithm>

namespace ttrl {

// Tile shapes each convolution GEMM may use (each one is a separate kernel).
constexpr unsigned kConvFwdCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T128x32) | cfg_bit(T64x64) |
                                  cfg_bit(T32x32K2) | cfg_bit(T64x32K2) | cfg_bit(T64x64K2);
constexpr unsigned kConvDwCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T64x64) |
                                 cfg_bit(T32x32K2) | cfg_bit(T32x32K4) | cfg_bit(T32x64K2);
constexpr unsigned kConvDxCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T128x32) | cfg_bit(T32x32K2) |
                                 cfg_bit(T64x32K2);
// The element-by-element patch path (padding, odd channel counts) only.
constexpr unsigned kConvGeneralCfgs = cfg_bit(T32x32) | cfg_bit(T64x32);

struct ConvGeo {
  int B, C, H, W, O, KH, KW, S, P, OH, OW, u8;
  int M;                           // B * OH * OW
  FDiv d_ohow, d_ow, d_c, d_kw, d_khkw, d_o, d_tw, d_s;
  int TH, TW;                      // taps per class along h and w: ceil(K / S)
  // The input gradient's residue classes cls0 .. cls0+3 (one launch), by group.
  int cls0;
  int ih0[kMaxGroups], iw0[kMaxGroups], nh[kMaxGroups], nw[kMaxGroups];
  FDiv d_nhnw[kMaxGroups], d_nw[kMaxGroups];
};

// The forward / weight-gradient view of a layer on the device: extents and
// the divisions that split a pixel index m into (b, oh, ow) and a patch
// index k into (c, kh, kw), 23 words pinned in scalar registers.
struct ConvCore {
  int M, S, P, H, W, C, u8, kp, KW, ohow, OW;
  FDiv dm1, dm2;  // m / (OH*OW), then / OW
  FDiv dk1, dk2;  // k / (KH*KW) (uint8 NCHW: c first) or k / C (NHWC: tap first), then / KW

  __device__ __forceinline__ void split_m(int m, int& b, int& oh, int& ow) const {
    b = dm1.div(m);
    const int rem = m - b * ohow;
    oh = dm2.div(rem);
    ow = rem - oh * OW;
  }
  __device__ __forceinline__ void split_k(int k, int& c, int& kh, int& kw) const {
    const int first = dk1.div(k);
    const int rest = k - first * dk1.d;
    const int tap = u8 ? rest : first;
    c = u8 ? first : rest;
    kh = dk2.div(tap);
    kw = tap - kh * KW;
  }
};

__device__ __forceinline__ ConvCore conv_core(const ConvGeo& g) {
  return ConvCore{g.M, g.S, g.P, g.H, g.W, g.C, g.u8, g.C * g.KH * g.KW, g.KW, g.OH * g.OW, g.OW,
                  g.d_ohow, g.d_ow, g.u8 ? g.d_khkw : g.d_c, g.d_kw};
}

// Patch element (m, k) of the input: element offset, or -1 outside the image.
__device__ __forceinline__ long patch_index(const ConvCore& g, int m, int k) {
  if (m >= g.M || k >= g.kp) return -1;
  int b, oh, ow, c, kh, kw;
  g.split_m(m, b, oh, ow);
  g.split_k(k, c, kh, kw);
  const int ih = oh * g.S + kh - g.P, iw = ow * g.S + kw - g.P;
  if (ih < 0 || ih >= g.H || iw < 0 || iw >= g.W) return -1;
  if (g.u8) return ((long(b) * g.C + c) * g.H + ih) * g.W + iw;
  return ((long(b) * g.H + ih) * g.W + iw) * g.C + c;
}

// One patch element, any layout (the general path).
__device__ __forceinline__ float patch_elem(__amdgpu_buffer_rsrc_t rs, const ConvCore& g, int m, int k) {
  const long idx = patch_index(g, m, k);
  if (g.u8) return __uint_as_float(ld_u8(rs, idx < 0 ? kBad : uint32_t(idx)));
  return ld_f1(rs, idx < 0 ? kBad : uint32_t(idx) * 4u);
}

// How four consecutive patch indices k..k+3 (k % 4 == 0) lie in memory.
enum PatchMode {
  kPatchNhwcVec = 0,  // fp32 NHWC, C % 4 == 0, no padding: four channels of one tap, one 16-byte load
  kPatchU8Word = 1,   // uint8 NCHW, KW, W, S multiples of 4, no padding: four kw of one row, one aligned word
  kPatchGeneral = 2,  // element by element, any geometry
};

__host__ inline int patch_mode(const ConvGeo& g, bool aligned) {
  if (g.P == 0 && !g.u8 && g.C % 4 == 0 && aligned) return kPatchNhwcVec;
  if (g.P == 0 && g.u8 && g.KW % 4 == 0 && g.W % 4 == 0 && g.S % 4 == 0 && aligned) return kPatchU8Word;
  return kPatchGeneral;
}

// Vector modes (no padding).  pixel_base: byte offset of output pixel m's
// first tap, (b, oh*S, ow*S); kBad past the last pixel.  tap_off: byte
// offset of patch chunk k..k+3 relative to it; kBad past the patch.  Their
// sum is in range exactly when both are valid.
__device__ __forceinline__ uint32_t pixel_base(const ConvCore& g, int m) {
  if (m >= g.M) return kBad;
  int b, oh, ow;
  g.split_m(m, b, oh, ow);
  const int ih0 = oh * g.S, iw0 = ow * g.S;
  const int e = g.u8 ? (b * g.C * g.H + ih0) * g.W + iw0 : ((b * g.H + ih0) * g.W + iw0) * g.C;
  return uint32_t(e) * (g.u8 ? 1u : 4u);
}
__device__ __forceinline__ uint32_t tap_off(const ConvCore& g, int k) {
  if (k >= g.kp) return kBad;
  int c, kh, kw;
  g.split_k(k, c, kh, kw);
  const int e = g.u8 ? (c * g.H + kh) * g.W + kw : (kh * g.W + kw) * g.C + c;
  return uint32_t(e) * (g.u8 ? 1u : 4u);
}

// Forward A operand: A(m, k) = patch(m, k).  MODE is how four consecutive
// patch indices lie in memory (PatchMode); the vector modes assume no
// padding, so a real pixel's taps are all inside the image and the byte
// offset alone carries validity.
template <int MODE>
struct LdConvFwd {
  ConvGeo g;
  const void* x[kMaxGroups];
  uint32_t xbytes;

  struct Params {
    ConvCore g;
    const void* x;
    uint32_t xbytes;
  };
  struct Live {
    static constexpr bool KCONTIG = true;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    struct Row { uint32_t base; };  // vector modes: byte offset of the pixel's first tap; general: m
    struct Kp { uint32_t off; int k; };
    __device__ __forceinline__ int fmt() const {
      if constexpr (MODE == kPatchU8Word) return kU8Word;
      else if constexpr (MODE == kPatchNhwcVec) return kF32;
      else return q.g.u8 ? kU8Each : kF32;
    }
    __device__ __forceinline__ Row row(int m) const {
      if constexpr (MODE == kPatchGeneral) return Row{uint32_t(m)};
      else return Row{pixel_base(q.g, m)};
    }
    __device__ __forceinline__ Kp kpos(int k) const {
      if constexpr (MODE == kPatchGeneral) return Kp{0u, k};
      else return Kp{tap_off(q.g, k), k};
    }
    __device__ __forceinline__ void issue(const Row& r, const Kp& kp, Fetch4& f) const {
      if constexpr (MODE == kPatchNhwcVec) {
        f.v = ld_f4(rs, r.base + kp.off);
      } else if constexpr (MODE == kPatchU8Word) {
        f.v.x = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, r.base + kp.off, 0, 0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) f.v[j] = patch_elem(rs, q.g, int(r.base), kp.k + j);
      }
    }
  };
  __device__ __forceinline__ Live live(int grp) const {
    const Params q = pin_pod(Params{conv_core(g), x[grp], xbytes});
    return Live{q, make_res(q.x, q.xbytes)};
  }
};

// Weight-gradient A operand: A(r = k, k = m) = patch(m, r), with the ones row
// at r == kp when the bias gradient is wanted.  MODE as for LdConvFwd; the
// chunk that holds the ones row goes element by element in every mode.
template <int MODE>
struct LdConvPatchT {
  ConvGeo g;
  const void* x[kMaxGroups];
  uint32_t xbytes;
  int ones;

  struct Params {
    ConvCore g;
    const void* x;
    uint32_t xbytes;
    int ones;
  };
  struct Live {
    static constexpr bool KCONTIG = false;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    struct Row { uint32_t tap; int r; bool whole; };
    struct Ks { int m; };
    __device__ __forceinline__ int fmt() const {
      if constexpr (MODE == kPatchU8Word) return kU8Word;
      else return q.g.u8 ? kU8Each : kF32;
    }
    __device__ __forceinline__ Row row(int r) const {
      const bool whole = MODE != kPatchGeneral && r + 3 < q.g.kp;
      return Row{whole ? tap_off(q.g, r) : 0u, r, whole};
    }
    __device__ __forceinline__ Ks kstage(const Row&, int m) const { return Ks{m}; }
    __device__ __forceinline__ void issue(const Row& r, const Ks& ks, int dm, Fetch4& f) const {
      const int m = ks.m + dm;
      if constexpr (MODE != kPatchGeneral) {
        if (r.whole) {
          const uint32_t off = pixel_base(q.g, m) + r.tap;
          if constexpr (MODE == kPatchNhwcVec) f.v = ld_f4(rs, off);
          else f.v.x = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
          return;
        }
      }
      // The general path and the tail chunk: patch rows, then the ones row.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rr = r.r + j;
        if (rr < q.g.kp) {
          f.v[j] = patch_elem(rs, q.g, m, rr);
        } else {
          const float one = (q.ones && rr == q.g.kp && m < q.g.M) ? 1.f : 0.f;
          f.v[j] = q.g.u8 ? __uint_as_float(uint32_t(one)) : one;
        }
      }
    }
  };
  __device__ __forceinline__ Live live(int grp) const {
    const Params q = pin_pod(Params{conv_core(g), x[grp], xbytes, ones});
    return Live{q, make_res(q.x, q.xbytes)};
  }
};

// Input-gradient A operand of class `cls`: A(r, k = (jh, jw, o)) = dZ at the
// output pixel that tap (kh, kw) = (ch + s*jh, cw + s*jw) connects to input
// pixel r: oh = ohc(r) - jh, ow = owc(r) - jw with ohc = (ih + p - ch) / s.
struct LdConvDxA {
  ConvGeo g;
  const float* dy;
  uint32_t dybytes;

  struct Params {
    const float* dy;
    uint32_t bytes;
    int rows, nw;
    FDiv d_nhnw, d_nw;
    int ch, cw, ihp, iwp, S;  // ihp = ih0 + P - ch: ohc = (ihp + S*i) / S
    FDiv d_s;
    int OH, OW, O, kmax;  // kmax = TH*TW*O
    FDiv d_o, d_tw;
    int TW, KH, KW;
  };
  struct Live {
    static constexpr bool KCONTIG = true;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    struct Row { int base, ohc, owc; };  // base = element offset of dZ(b, ohc, owc, 0)
    struct Kp { int off, jh, jw; bool v; int k; };
    __device__ __forceinline__ int fmt() const { return kF32; }
    __device__ __forceinline__ Row row(int r) const {
      if (r >= q.rows) return Row{0, -(1 << 28), 0};
      const int b = q.d_nhnw.div(r);
      const int rem = r - b * q.d_nhnw.d;
      const int i = q.d_nw.div(rem), j = rem - i * q.nw;
      const int ohc = q.d_s.div(q.ihp + q.S * i);
      const int owc = q.d_s.div(q.iwp + q.S * j);
      return Row{((b * q.OH + ohc) * q.OW + owc) * q.O, ohc, owc};
    }
    __device__ __forceinline__ Kp kpos(int k) const {
      if (k >= q.kmax) return Kp{0, 0, 0, false, k};
      const int jt = q.d_o.div(k), o = k - jt * q.O;
      const int jh = q.d_tw.div(jt), jw = jt - jh * q.TW;
      const bool v = q.ch + q.S * jh < q.KH && q.cw + q.S * jw < q.KW;
      return Kp{o - (jh * q.OW + jw) * q.O, jh, jw, v, k};
    }
    __device__ __forceinline__ void issue(const Row& r, const Kp& kp, Fetch4& f) const {
      if ((q.O & 3) == 0) {  // the four k share one tap and output pixel
        const int oh = r.ohc - kp.jh, ow = r.owc - kp.jw;
        const bool in = kp.v && oh >= 0 && oh < q.OH && ow >= 0 && ow < q.OW;
        f.v = ld_f4(rs, in ? uint32_t(r.base + kp.off) * 4u : kBad);
        return;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = kp.k + j;
        bool in = k < q.kmax;
        int off = 0;
        if (in) {
          const int jt = q.d_o.div(k), o = k - jt * q.O;
          const int jh = q.d_tw.div(jt), jw = jt - jh * q.TW;
          const int oh = r.ohc - jh, ow = r.owc - jw;
          in = q.ch + q.S * jh < q.KH && q.cw + q.S * jw < q.KW && oh >= 0 && oh < q.OH && ow >= 0 && ow < q.OW;
          off = r.base - (jh * q.OW + jw) * q.O + o;
        }
        f.v[j] = ld_f1(rs, in ? uint32_t(off) * 4u : kBad);
      }
    }
  };
  __device__ __forceinline__ Live live(int grp) const {
    const int c = g.cls0 + grp, ch = c / g.S, cw = c - ch * g.S;
    const Params q = pin_pod(Params{dy, dybytes, g.B * g.nh[grp] * g.nw[grp], g.nw[grp], g.d_nhnw[grp], g.d_nw[grp],
                                    ch, cw, g.ih0[grp] + g.P - ch, g.iw0[grp] + g.P - cw, g.S, g.d_s, g.OH, g.OW,
                                    g.O, g.TH * g.TW * g.O, g.d_o, g.d_tw, g.TW, g.KH, g.KW});
    return Live{q, make_res(q.dy, q.bytes)};
  }
};

// Input-gradient B operand of class `cls`: B(k = (jh, jw, o), n = c) =
// Wt[(kh, kw, c)][o]; stored here as rows n, k contiguous.
struct LdConvDxB {
  ConvGeo g;
  const float* wt;
  uint32_t wbytes;

  struct Params {
    const float* wt;
    uint32_t bytes;
    int C, O, ch, cw, S, KH, KW, kmax, TW;
    FDiv d_o, d_tw;
  };
  struct Live {
    static constexpr bool KCONTIG = true;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    struct Row { uint32_t off; int c; };  // byte offset of Wt[(0,0,c)][0], kBad past C
    struct Kp { uint32_t off; int k; };
    __device__ __forceinline__ int fmt() const { return kF32; }
    __device__ __forceinline__ Row row(int c) const { return Row{c < q.C ? uint32_t(c * q.O) * 4u : kBad, c}; }
    __device__ __forceinline__ Kp kpos(int k) const {
      if (k >= q.kmax) return Kp{kBad, k};
      const int jt = q.d_o.div(k), o = k - jt * q.O;
      const int jh = q.d_tw.div(jt), jw = jt - jh * q.TW;
      const int kh = q.ch + q.S * jh, kw = q.cw + q.S * jw;
      const bool v = kh < q.KH && kw < q.KW;
      return Kp{v ? uint32_t((kh * q.KW + kw) * q.C * q.O + o) * 4u : kBad, k};
    }
    __device__ __forceinline__ void issue(const Row& r, const Kp& kp, Fetch4& f) const {
      if ((q.O & 3) == 0) {
        f.v = ld_f4(rs, r.off + kp.off);
        return;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = kp.k + j;
        bool in = r.c < q.C && k < q.kmax;
        int off = 0;
        if (in) {
          const int jt = q.d_o.div(k), o = k - jt * q.O;
          const int jh = q.d_tw.div(jt), jw = jt - jh * q.TW;
          const int kh = q.ch + q.S * jh, kw = q.cw + q.S * jw;
          in = kh < q.KH && kw < q.KW;
          off = (r.c + (kh * q.KW + kw) * q.C) * q.O + o;
        }
        f.v[j] = ld_f1(rs, in ? uint32_t(off) * 4u : kBad);
      }
    }
  };
  __device__ __forceinline__ Live live(int grp) const {
    const int c = g.cls0 + grp, ch = c / g.S, cw = c - ch * g.S;
    const Params q = pin_pod(Params{wt, wbytes, g.C, g.O, ch, cw, g.S, g.KH, g.KW, g.TH * g.TW * g.O, g.TW, g.d_o,
                                    g.d_tw});
    return Live{q, make_res(q.wt, q.bytes)};
  }
};

// Input-gradient epilogue: class row r -> NHWC input pixel, times
// [xmask > 0] when the input was a ReLU output.
struct EpConvDx {
  ConvGeo g;
  float* dx;
  const float* xmask;
  float alpha, beta;
  __device__ __forceinline__ int rows(int grp) const { return g.B * g.nh[grp] * g.nw[grp]; }
  __host__ long tune_span() const { return long(g.B) * g.H * g.W * g.C + 64; }
  __host__ EpConvDx tune_copy(float* sink) const {
    EpConvDx e = *this;
    e.dx = sink;
    e.beta = 0.f;
    return e;
  }
  // One residue class's epilogue with its tables bound: buffer loads and
  // stores, an element outside the class reading zero and storing nothing.
  struct Bound {
    int rows, C, H, W, S, nw, ih0, iw0;
    FDiv d_nhnw, d_nw;
    __amdgpu_buffer_rsrc_t rdx, rxm, rold;  // rxm, rold empty when absent (read zero)
    bool has_xm;
    float alpha, beta;
    __device__ __forceinline__ EpAux aux(int r, int c) const {
      EpAux x{nullptr, 0.f, 1.f, 0.f, kBad};
      const int b = d_nhnw.div(r);
      const int rem = r - b * d_nhnw.d;
      const int i = d_nw.div(rem), j = rem - i * nw;
      const int ih = ih0 + S * i, iw = iw0 + S * j;
      x.off = (r < rows && c < C) ? uint32_t(((b * H + ih) * W + iw) * C + c) * 4u : kBad;
      x.keep = ld_f1(rxm, x.off);
      x.old = ld_f1(rold, x.off);
      return x;
    }
    __device__ __forceinline__ void store(int, int, float acc, const EpAux& x) const {
      float v = alpha * acc;
      if (has_xm && !(x.keep > 0.f)) v = 0.f;
      v += beta * x.old;
      st_f1(rdx, x.off, v);
    }
  };
  struct Params {
    float* dx;
    const float* xm;
    uint32_t bytes;
    int rows, C, H, W, S, nw, ih0, iw0;
    FDiv d_nhnw, d_nw;
    float alpha, beta;
  };
  template <class F>
  __device__ __forceinline__ void with_bound(int grp, F&& f) const {
    const Params q = pin_pod(Params{dx, xmask, uint32_t(long(g.B) * g.H * g.W * g.C * 4), rows(grp), g.C, g.H, g.W,
                                    g.S, g.nw[grp], g.ih0[grp], g.iw0[grp], g.d_nhnw[grp], g.d_nw[grp], alpha, beta});
    f(Bound{q.rows, q.C, q.H, q.W, q.S, q.nw, q.ih0, q.iw0, q.d_nhnw, q.d_nw, make_res(q.dx, q.bytes),
            make_res(q.xm, q.xm ? q.bytes : 0u), make_res(q.dx, q.beta != 0.f ? q.bytes : 0u), q.xm != nullptr,
            q.alpha, q.beta});
  }
};


// Residue-class tables of classes cls0 .. cls0+kMaxGroups-1 (empty past S*S).
inline void set_classes(ConvGeo& g, int cls0) {
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

inline int make_geo(const ttrl_conv_geom* s, ConvGeo& g) {
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
  // Buffer loads address operands with 32-bit byte offsets below 2^30.
  const long bigs[] = {long(g.B) * g.OH * g.OW * g.O * 4, long(g.B) * g.H * g.W * g.C * (g.u8 ? 1 : 4),
                       long(g.C) * g.KH * g.KW * g.O * 4};
  for (long v : bigs) TTRL_REQUIRE(v < kMaxOperandBytes, "conv: an operand of %ld bytes exceeds 2^30", v);
  g.d_ohow.set(g.OH * g.OW);
  g.d_ow.set(g.OW);
  g.d_c.set(g.C);
  g.d_kw.set(g.KW);
  g.d_khkw.set(g.KH * g.KW);
  g.d_o.set(g.O);
  g.TH = (g.KH + g.S - 1) / g.S;
  g.TW = (g.KW + g.S - 1) / g.S;
  g.d_tw.set(g.TW);
  g.d_s.set(g.S);
  set_classes(g, 0);
  return TTRL_OK;
}

inline uint32_t input_bytes(const ConvGeo& g) { return uint32_t(long(g.B) * g.H * g.W * g.C * (g.u8 ? 1 : 4)); }

inline bool input_aligned(const ConvGeo& g, const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & (g.u8 ? 3 : 15)) == 0;
}

// The weight-gradient GEMM of a layer: dWt_aug[r][o] = x_scale * sum_m
// patch(m, r) dZ[m][o], row kp (when db is wanted) the bias gradient.
template <int MODE>
struct ConvDwProblem {
  LdConvPatchT<MODE> la;
  LdColK lb;
  EpStore ep;
  GemmDims q;
};
template <int MODE>
inline ConvDwProblem<MODE> conv_dw_problem(const ConvGeo& g, const void* x, float x_scale, const float* dy, float* dwt,
                                           float* db, float beta) {
  const int Kp = g.C * g.KH * g.KW;
  ConvDwProblem<MODE> p{LdConvPatchT<MODE>{g, {x}, input_bytes(g), db ? 1 : 0}, LdColK{}, EpStore{}, GemmDims{}};
  p.lb.p[0] = dy;  // B(r=o, k=m) = dZ[m][o]
  p.lb.ld = g.O;
  p.lb.rows = g.O;
  p.lb.K = g.M;
  p.lb.vec_ok((reinterpret_cast<uintptr_t>(dy) & 15) == 0);
  p.ep.M = db ? Kp + 1 : Kp;
  p.ep.N = g.O;
  p.ep.C[0] = dwt;
  p.ep.ldc = g.O;
  p.ep.rsplit = Kp;
  p.ep.Cr[0] = db;
  p.ep.alpha = x_scale;  // d/dW of conv(s*x, W) = s * dW(x, dY); the bias row is unscaled
  p.ep.alpha_r = 1.f;
  p.ep.beta = beta;
  p.q = GemmDims{p.ep.M, g.O, g.M, 1};
  return p;
}

// The gradient source of a weight-gradient launch that ran `plan` with its
// partials in `part`: split partials when the plan split K (the epilogue's
// alpha = x_scale for the weight rows, 1 for the bias row), nothing pending
// otherwise.
inline ttrl_grad_source conv_dw_source(const ConvGeo& g, float x_scale, float* dwt, float* db, const float* part,
                                       const GemmPlan& plan) {
  ttrl_grad_source s{};
  s.rows = g.C * g.KH * g.KW;
  s.cols = g.O;
  s.dw = dwt;
  s.db = db;
  if (plan.splits > 1) {
    s.kind = TTRL_GRAD_SPLITS;
    s.part = part;
    s.splits = plan.splits;
    s.scale = x_scale;
    s.bias_scale = 1.f;
  }
  return s;
}

// The input-gradient GEMM of residue classes c0 .. c0+n-1 (n <= kMaxGroups).
struct ConvDxProblem {
  LdConvDxA la;
  LdConvDxB lb;
  EpConvDx ep;
  GemmDims q;
};
inline ConvDxProblem conv_dx_problem(ConvGeo g, int c0, const float* dy, const float* wt, float* dx,
                                     const float* xmask, float x_scale, float beta) {
  const int n = std::min(kMaxGroups, g.S * g.S - c0);
  set_classes(g, c0);
  // The largest class (ih0 = iw0 = 0) has ceil(H/S) * ceil(W/S) pixels per image.
  const int Mmax = g.B * ((g.H + g.S - 1) / g.S) * ((g.W + g.S - 1) / g.S);
  return ConvDxProblem{LdConvDxA{g, dy, uint32_t(long(g.M) * g.O * 4)},
                       LdConvDxB{g, wt, uint32_t(long(g.C) * g.KH * g.KW * g.O * 4)},
                       EpConvDx{g, dx, xmask, x_scale, beta}, GemmDims{Mmax, g.C, g.TH * g.TW * g.O, n}};
}

}  // namespace ttrl
