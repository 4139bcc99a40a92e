// Dense layers on the FP32 MFMA core: the generic `matmul` op and the fused
// linear layer (bias, ReLU, clamp epilogues; masked-ReLU backward; bias
// gradient folded into the weight-gradient GEMM as an implicit ones row).
//
// Reference semantics:
//   matmul fwd/bwd        ttrl/engine/ops/matmul.py:55-86
//   Linear y = x@W + b    ttrl/engine/layers.py:22-61 (W stored (in, out))
//   relu / relu_bw        ttrl/engine/ops/unary.py:25-37
//   bias-gradient sum     ttrl/engine/ops/broadcast.py:11-30
//   log_std clamp         ttrl/nets/heads.py:65-93, ttrl/engine/ops/select.py:52-63
#include "tile_gemm.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace ttrl {

namespace {

struct Costed {
  double t;
  GemmPlan p;
};

// Every (tile, split) the cost model admits, with its estimate in cycles:
//   rounds * (latency + stages_per_block * blocks_per_cu * max(mfma, fetch))
//   + a reduction pass when K is split,
// with mfma = 32 cycles per 16x16x4 MFMA of one wavefront (the FP32 MFMA
// issue interval), fetch = stage bytes at 64 B/cycle per CU, and the
// workgroups a CU holds limited by LDS (160 KiB) and registers (two).
std::vector<Costed> costed_plans(int M, int N, int K, int groups, long ws_floats, unsigned allowed) {
  constexpr double kLatency = 2500.0, kReduceFixed = 4000.0, kCus = 256.0;
  std::vector<Costed> out;
  for (int c = 0; c < kNumCfg; ++c) {
    if (!(allowed & (1u << c))) continue;
    const TileDims t = tile_dims(c);
    const long tiles = long(ceil_div(M, t.bm)) * ceil_div(N, t.bn) * groups;
    const int stages = std::max(1, (K + t.tbk - 1) / t.tbk);
    const double lds = 4.0 * (t.bm + t.bn) * (t.tbk + 4);
    const double bpc = std::max(1.0, std::min(2.0, std::floor(160.0 * 1024.0 / lds)));
    const double mfma = double(t.bm / t.wgm / 16) * (t.bn / t.wgn / 16) * (t.tbk / 4 / t.wgk) * 32.0;
    const double fetch = 4.0 * (t.bm + t.bn) * t.tbk / 64.0;
    for (int sp = 1; sp <= stages; ++sp) {
      const int spb = (stages + sp - 1) / sp;
      const int real = (stages + spb - 1) / spb;  // splits that own a stage
      if (real != sp) continue;
      if (sp > 1 && long(sp) * groups * M * N > ws_floats) break;
      const double blocks = double(tiles) * sp;
      const double per_cu = std::min(bpc, std::ceil(blocks / kCus));
      const double rounds = std::ceil(blocks / (kCus * bpc));
      double tt = rounds * (kLatency + spb * per_cu * std::max(mfma, fetch));
      if (sp > 1) tt += kReduceFixed + double(groups) * M * N * sp * 4.0 / (kCus * 32.0);
      out.push_back(Costed{tt, GemmPlan{c, t.bm, t.bn, t.tbk, sp, spb * t.tbk}});
    }
  }
  std::stable_sort(out.begin(), out.end(), [](const Costed& a, const Costed& b) { return a.t < b.t; });
  return out;
}

}  // namespace

GemmPlan plan_gemm(int M, int N, int K, int groups, long ws_floats, unsigned allowed) {
  const std::vector<Costed> all = costed_plans(M, N, K, groups, ws_floats, allowed);
  return all.empty() ? GemmPlan{T32x32, 32, 32, 256, 1, 256} : all.front().p;
}

std::vector<GemmPlan> plan_candidates(int M, int N, int K, int groups, long ws_floats, unsigned allowed,
                                      int max_n) {
  const std::vector<Costed> all = costed_plans(M, N, K, groups, ws_floats, allowed);
  std::vector<GemmPlan> out;
  // the model's best split of every tile shape, then the next best overall
  for (int c = 0; c < kNumCfg; ++c)
    for (const Costed& x : all)
      if (x.p.cfg == c) {
        out.push_back(x.p);
        break;
      }
  for (const Costed& x : all) {
    if (int(out.size()) >= max_n) break;
    bool seen = false;
    for (const GemmPlan& q : out) seen = seen || (q.cfg == x.p.cfg && q.splits == x.p.splits);
    if (!seen) out.push_back(x.p);
  }
  return out;
}

bool plan_with_splits(int cfg, int M, int N, int K, int groups, long ws_floats, int splits, GemmPlan* out) {
  const TileDims t = tile_dims(cfg);
  const int stages = std::max(1, (K + t.tbk - 1) / t.tbk);
  const int sp = std::max(1, std::min(splits, stages));
  const int spb = (stages + sp - 1) / sp;
  const GemmPlan p{cfg, t.bm, t.bn, t.tbk, (stages + spb - 1) / spb, spb * t.tbk};
  if (p.splits > 1 && long(p.splits) * groups * M * N > ws_floats) return false;
  *out = p;
  return true;
}

bool plan_valid(const GemmPlan& p, int M, int N, int K, int groups, long ws_floats, unsigned allowed) {
  if (p.cfg < 0 || p.cfg >= kNumCfg || !(allowed & (1u << p.cfg))) return false;
  const TileDims t = tile_dims(p.cfg);
  if (p.bm != t.bm || p.bn != t.bn || p.tbk != t.tbk) return false;
  if (p.splits < 1 || p.kchunk < t.tbk || p.kchunk % t.tbk) return false;
  const int stages = std::max(1, (K + t.tbk - 1) / t.tbk);
  const int spb = p.kchunk / t.tbk;
  if (p.splits != (stages + spb - 1) / spb) return false;  // the splits exactly cover K
  return p.splits == 1 || long(p.splits) * groups * M * N <= ws_floats;
}

bool gemm_forced(unsigned allowed, int M, int N, int K, int groups, long ws_floats, GemmPlan* out) {
  const char* v = std::getenv("TTRL_GEMM_FORCE");
  if (!v || !*v) return false;
  int cfg = -1, splits = 0;
  if (std::sscanf(v, "%d:%d", &cfg, &splits) < 1 || cfg < 0 || cfg >= kNumCfg || !(allowed & (1u << cfg)))
    return false;
  GemmPlan p = plan_gemm(M, N, K, groups, ws_floats, 1u << cfg);
  if (splits > 0) {
    GemmPlan q;
    if (plan_with_splits(cfg, M, N, K, groups, ws_floats, splits, &q)) p = q;
  }
  *out = p;
  return true;
}

bool gemm_tuning_log() {
  static const bool on = [] {
    const char* v = std::getenv("TTRL_GEMM_TUNE_LOG");
    return v && v[0] == '1';
  }();
  return on;
}

bool gemm_tuning_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("TTRL_GEMM_TUNE");
    return !(v && v[0] == '0');
  }();
  return on;
}

const float* relu_mask_into_workspace(ttrl_ctx* ctx, const float* src, const float* mask, long n, long gs,
                                      int groups, long* reserved, int* rc);

namespace {

constexpr unsigned kMatmulCfgs = cfg_bit(T32x32) | cfg_bit(T64x64) | cfg_bit(T128x64) | cfg_bit(T32x32K4);
constexpr unsigned kSmallK = cfg_bit(T32x32K2) | cfg_bit(T32x32K4) | cfg_bit(T64x32K2) | cfg_bit(T32x64K2);
constexpr unsigned kLinFwdCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T64x64) | kSmallK;
constexpr unsigned kShallow = cfg_bit(T32x32S) | cfg_bit(T64x64S) | cfg_bit(T128x64S);
constexpr unsigned kLinDwCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T64x64) |
                                cfg_bit(T128x64) | kSmallK | cfg_bit(T64x64K2) | kShallow;
constexpr unsigned kLinDxCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T64x64) | kSmallK |
                                cfg_bit(T32x32S);
// A layer's dW and dx in one launch (k_gemm_pair): one tile shape for both.
constexpr unsigned kLinPairCfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T32x32K2) |
                                  cfg_bit(T64x32K2) | cfg_bit(T32x32S) | cfg_bit(T64x64S);

__global__ __launch_bounds__(256) void k_relu_mask(float* dst, const float* src, const float* mask, long n, long gs,
                                                   int groups) {
  const long total = n * groups;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += long(gridDim.x) * 256) {
    const long g = i / n, j = i - g * n;
    const long s = g * gs + j;
    dst[i] = mask[s] > 0.f ? src[s] : 0.f;
  }
}

// Buffer loads address an operand with 32-bit byte offsets.
inline bool fits(const LdRowK& l) { return l.bytes() < kMaxOperandBytes; }
inline bool fits(const LdColK& l) { return l.bytes() < kMaxOperandBytes && l.bytes2() < kMaxOperandBytes; }
inline bool fits(const LdRowKCat& l) { return l.bytes1() < kMaxOperandBytes && l.bytes2() < kMaxOperandBytes; }
#define TTRL_FITS(la, lb, name) \
  TTRL_REQUIRE(fits(la) && fits(lb), "%s: an operand of 2^30 bytes or more is not supported", name)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <class T>
inline void groups_of(T* (&dst)[kMaxGroups], T* base, long stride, int groups) {
  fill_groups(dst, base, stride, groups);
}

inline bool all_aligned(const float* const (&p)[kMaxGroups], int groups) {
  for (int g = 0; g < groups; ++g)
    if (p[g] && !aligned16(p[g])) return false;
  return true;
}

}  // namespace

const float* relu_mask_into_workspace(ttrl_ctx* ctx, const float* src, const float* mask, long n, long gs,
                                      int groups, long* reserved, int* rc) {
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const long need = (n * groups + 63) / 64 * 64;
  if (need + *reserved > wsf / 2) {
    *rc = set_error(TTRL_ENOMEM, "relu mask: %ld floats exceed half of the %ld-float workspace", need, wsf);
    return nullptr;
  }
  float* dst = ws + wsf - *reserved - need;
  *reserved += need;
  const long total = n * groups;
  unsigned blocks = unsigned(std::min<long>(4096, (total + 255) / 256));
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(k_relu_mask, dim3(blocks), dim3(256), 0, stream_of(ctx), dst, src, mask, n, gs, groups);
  *rc = check_launch("relu mask");
  return dst;
}

// Back-to-back v_mfma_f32_16x16x4f32 on eight independent accumulators per
// wavefront (no memory traffic inside the loop), for the achievable FP32
// matrix rate; each lane's sum is stored so the work is kept.
constexpr int kRateChains = 8;
__global__ __launch_bounds__(256) void k_mfma_rate(int iters, float* __restrict__ out) {
  f32x4 acc[kRateChains];
#pragma unroll
  for (int j = 0; j < kRateChains; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float a = float(threadIdx.x & 63) * (1.f / 64.f), b = 1.f / 1024.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < kRateChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kRateChains; ++j) s += (acc[j][0] + acc[j][1]) + (acc[j][2] + acc[j][3]);
  out[long(blockIdx.x) * blockDim.x + threadIdx.x] = s;
}

}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_mfma_rate(ttrl_ctx* ctx, int workgroups, int iters, float* out, double* flops) {
  TTRL_REQUIRE(ctx && out && flops, "ttrl_mfma_rate: null argument");
  TTRL_REQUIRE(workgroups > 0 && workgroups <= 65536 && iters > 0 && iters <= (1 << 24),
               "ttrl_mfma_rate: %d workgroups of %d iterations outside [1, 65536] x [1, 2^24]", workgroups, iters);
  hipLaunchKernelGGL(k_mfma_rate, dim3(unsigned(workgroups)), dim3(256), 0, stream_of(ctx), iters, out);
  *flops = double(workgroups) * 4.0 * double(iters) * kRateChains * 2.0 * 16 * 16 * 4;
  return check_launch("ttrl_mfma_rate");
}

int ttrl_matmul(ttrl_ctx* ctx, int M, int N, int K, const float* A, long lda, int ta, const float* B, long ldb,
                int tb, float* C, long ldc, float alpha, float beta) {
  TTRL_REQUIRE(ctx && A && B && C, "ttrl_matmul: null argument");
  TTRL_REQUIRE(M >= 0 && N >= 0 && K >= 0, "ttrl_matmul: negative extent");
  EpStore ep;
  ep.M = M;
  ep.N = N;
  ep.C[0] = C;
  ep.ldc = ldc;
  ep.alpha = K == 0 ? 0.f : alpha;  // an empty reduction still defines C = beta*C
  ep.beta = beta;
  const int Kr = K > 0 ? K : 1;
  if (!ta && !tb) {
    LdRowK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdColK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    TTRL_FITS(la, lb, "ttrl_matmul");
    return run_gemm<kMatmulCfgs>(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (!ta && tb) {
    LdRowK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdRowK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    TTRL_FITS(la, lb, "ttrl_matmul");
    return run_gemm<kMatmulCfgs>(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (ta && !tb) {
    LdColK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdColK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    TTRL_FITS(la, lb, "ttrl_matmul");
    return run_gemm<kMatmulCfgs>(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else {
    LdColK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdRowK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    TTRL_FITS(la, lb, "ttrl_matmul");
    return run_gemm<kMatmulCfgs>(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  }
}

// Forward of `groups` linear layers given per-group pointer tables.
static int linear_forward_tables(ttrl_ctx* ctx, int M, int K, int N, int groups, const float* const (&x)[kMaxGroups],
                                 long ldx, const float* const (&x2)[kMaxGroups], long ldx2, int k1,
                                 const float* const (&W)[kMaxGroups], const float* const (&b)[kMaxGroups],
                                 const float* const (&W2)[kMaxGroups], const float* const (&b2)[kMaxGroups], int n1,
                                 float* const (&y)[kMaxGroups], int relu, int clamp_col, float lo, float hi,
                                 const char* name) {
  const bool split_w = W2[0] != nullptr;
  EpStore ep;
  ep.M = M;
  ep.N = N;
  ep.ldc = N;
  for (int g = 0; g < kMaxGroups; ++g) {
    ep.C[g] = y[g];
    ep.bias[g] = b[g];
    if (split_w) {
      ep.Cc[g] = y[g] ? y[g] + n1 : nullptr;  // same row-major [M][N] output, rebased column
      ep.bias2[g] = b2[g];
    }
  }
  if (split_w) {
    ep.csplit = n1;
    ep.ldcc = N;
  }
  ep.relu = relu;
  ep.clamp_col = clamp_col > 0 ? clamp_col : (1 << 30);
  ep.lo = lo;
  ep.hi = hi;

  LdColK lb;  // B(k, n) = W[k][n]
  lb.ld = split_w ? n1 : N;
  lb.rows = N;
  lb.K = K;
  for (int g = 0; g < kMaxGroups; ++g) {
    lb.p[g] = W[g];
    lb.p2[g] = W2[g];
  }
  if (split_w) {
    lb.ld2 = N - n1;
    lb.split = n1;
  }
  lb.vec_ok(all_aligned(W, groups));
  if (x2[0]) {
    LdRowKCat la;
    for (int g = 0; g < kMaxGroups; ++g) {
      la.p1[g] = x[g];
      la.p2[g] = x2[g];
    }
    la.ld1 = ldx;
    la.ld2 = ldx2;
    la.rows = M;
    la.k1 = k1;
    la.K = K;
    TTRL_FITS(la, lb, name);
    return run_gemm<kLinFwdCfgs>(ctx, la, lb, ep, M, N, K, groups, name);
  }
  LdRowK la;
  for (int g = 0; g < kMaxGroups; ++g) la.p[g] = x[g];
  la.ld = ldx;
  la.rows = M;
  la.K = K;
  la.vec_ok(all_aligned(x, groups));
  TTRL_FITS(la, lb, name);
    return run_gemm<kLinFwdCfgs>(ctx, la, lb, ep, M, N, K, groups, name);
}

int ttrl_linear_forward(ttrl_ctx* ctx, const ttrl_linear_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_linear_forward: null argument");
  TTRL_REQUIRE(d->x && d->W && d->y, "ttrl_linear_forward: x, W and y are required");
  TTRL_REQUIRE(d->M >= 0 && d->K > 0 && d->N > 0 && d->groups >= 1 && d->groups <= kMaxGroups,
               "ttrl_linear_forward: bad extents");
  const int n1 = d->W2 ? d->n1 : d->N;
  TTRL_REQUIRE(n1 > 0 && n1 <= d->N, "ttrl_linear_forward: n1 out of range");
  const int k1 = d->x2 ? d->k1 : d->K;
  TTRL_REQUIRE(k1 > 0 && k1 <= d->K, "ttrl_linear_forward: k1 out of range");
  const float* x[kMaxGroups];
  const float* x2[kMaxGroups];
  const float* W[kMaxGroups];
  const float* b[kMaxGroups];
  const float* W2[kMaxGroups];
  const float* b2[kMaxGroups];
  float* y[kMaxGroups];
  groups_of(x, d->x, d->gx, d->groups);
  groups_of(x2, d->x2, d->gx2, d->groups);
  groups_of(W, d->W, d->gW, d->groups);
  groups_of(b, d->b, d->gb, d->groups);
  groups_of(W2, d->W2, d->gW, d->groups);
  groups_of(b2, d->b2, d->gb, d->groups);
  groups_of(y, d->y, d->gy, d->groups);
  for (int g = 0; g < d->groups; ++g) {
    if (d->xg[g]) x[g] = d->xg[g];
    if (d->x2g[g]) x2[g] = d->x2g[g];
    if (d->Wg[g]) W[g] = d->Wg[g];
    if (d->bg[g]) b[g] = d->bg[g];
  }
  return linear_forward_tables(ctx, d->M, d->K, d->N, d->groups, x, d->ldx, x2, d->ldx2, k1, W, b, W2, b2, n1, y,
                               d->relu, d->clamp_col, d->lo, d->hi, "ttrl_linear_forward");
}

int ttrl_linear_forward_multi(ttrl_ctx* ctx, int M, int K, int N, int groups, const float* const* x,
                              const float* const* W, const float* const* b, float* const* y, int relu) {
  TTRL_REQUIRE(ctx && x && W && y, "ttrl_linear_forward_multi: null argument");
  TTRL_REQUIRE(M >= 0 && K > 0 && N > 0 && groups >= 1 && groups <= kMaxGroups,
               "ttrl_linear_forward_multi: bad extents (at most %d groups)", kMaxGroups);
  const float* xt[kMaxGroups] = {};
  const float* none[kMaxGroups] = {};
  const float* Wt[kMaxGroups] = {};
  const float* bt[kMaxGroups] = {};
  float* yt[kMaxGroups] = {};
  for (int g = 0; g < groups; ++g) {
    TTRL_REQUIRE(x[g] && W[g] && y[g], "ttrl_linear_forward_multi: null pointer in group %d", g);
    xt[g] = x[g];
    Wt[g] = W[g];
    bt[g] = b ? b[g] : nullptr;
    yt[g] = y[g];
  }
  return linear_forward_tables(ctx, M, K, N, groups, xt, K, none, 0, K, Wt, bt, none, none, N, yt, relu, 0, 0.f,
                               0.f, "ttrl_linear_forward_multi");
}

int ttrl_linear_backward(ttrl_ctx* ctx, const ttrl_linear_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_linear_backward: null argument");
  TTRL_REQUIRE(d->dy && d->W, "ttrl_linear_backward: dy and W are required");
  TTRL_REQUIRE(d->M >= 0 && d->K > 0 && d->N > 0 && d->groups >= 1 && d->groups <= kMaxGroups,
               "ttrl_linear_backward: bad extents");
  const int G = d->groups;
  const int n1 = d->W2 ? d->n1 : d->N;
  TTRL_REQUIRE(n1 > 0 && n1 <= d->N, "ttrl_linear_backward: n1 out of range");
  const float* dy[kMaxGroups];
  groups_of(dy, d->dy, d->gy, G);
  long reserved = 0;
  if (d->ymask) {
    // dZ = dy * [ymask > 0] once, densely, for both products below.
    int rc = TTRL_OK;
    const long n = long(d->M) * d->N;
    const float* dz = relu_mask_into_workspace(ctx, d->dy, d->ymask, n, d->gy, G, &reserved, &rc);
    if (rc) return rc;
    groups_of(dy, dz, n, G);
  }
  const bool dyal = all_aligned(dy, G);

  // dW_aug[k][n] = sum_m xaug[m][k] dZ[m][n], xaug = [x | 1]; row K is db.
  LdColK wa;  // A(r=k_in, k=m) = x[m][k_in]
  LdColK wb;  // B(r=n, k=m) = dZ[m][n]
  EpStore wep;
  GemmDims wq{0, 0, 0, G};
  if (d->dW) {
    TTRL_REQUIRE(d->x && !d->x2, "ttrl_linear_backward: dW needs a single dense input x");
    TTRL_REQUIRE(!d->W2 || d->dW2, "ttrl_linear_backward: a split weight needs dW2");
    const bool with_b = d->db != nullptr;
    TTRL_REQUIRE(!with_b || !d->W2 || d->db2, "ttrl_linear_backward: a split bias needs db2");
    groups_of(wa.p, d->x, d->gx, G);
    wa.ld = d->ldx;
    wa.rows = with_b ? d->K + 1 : d->K;
    wa.K = d->M;
    wa.real_rows = d->K;
    wa.ones = with_b;
    wa.vec_ok(all_aligned(wa.p, G));
    for (int g = 0; g < kMaxGroups; ++g) wb.p[g] = dy[g];
    wb.ld = d->N;
    wb.rows = d->N;
    wb.K = d->M;
    wb.vec_ok(dyal);
    wep.M = wa.rows;
    wep.N = d->N;
    groups_of(wep.C, d->dW, d->gW, G);
    wep.ldc = n1;
    wep.rsplit = d->K;
    groups_of(wep.Cr, d->db, d->gb, G);
    wep.beta = d->beta_w;
    if (d->W2) {
      wep.csplit = n1;
      groups_of(wep.Cc, d->dW2, d->gW, G);
      wep.ldcc = d->N - n1;
      groups_of(wep.Crc, d->db2, d->gb, G);
    }
    TTRL_FITS(wa, wb, "ttrl_linear_backward");
    wq = GemmDims{wa.rows, d->N, d->M > 0 ? d->M : 1, G};
  }
  if (!d->dx)
    return d->dW ? run_gemm<kLinDwCfgs>(ctx, wa, wb, wep, wq.M, wq.N, wq.K, G, "ttrl_linear_backward dW", reserved)
                 : TTRL_OK;

  const int c0 = d->dx_cols > 0 ? d->dx_col0 : 0;
  const int nc = d->dx_cols > 0 ? d->dx_cols : d->K;
  TTRL_REQUIRE(c0 >= 0 && c0 + nc <= d->K, "ttrl_linear_backward: dx column range out of bounds");
  LdRowK xa;  // A(m, k=n) = dZ[m][n]
  for (int g = 0; g < kMaxGroups; ++g) xa.p[g] = dy[g];
  xa.ld = d->N;
  xa.rows = d->M;
  xa.K = d->N;
  xa.vec_ok(dyal);
  EpStore xep;
  xep.M = d->M;
  xep.N = nc;
  groups_of(xep.C, d->dx, d->gdx, G);
  groups_of(xep.mask, d->dxmask, d->gdx, G);
  xep.ldc = d->lddx > 0 ? d->lddx : nc;
  xep.beta = d->beta_x;
  const GemmDims xq{d->M, nc, d->N, G};
  // dW and dx are independent given dZ: one paired launch when both are wanted.
  auto finish = [&](const auto& xb) -> int {
    TTRL_FITS(xa, xb, "ttrl_linear_backward");
    if (d->dW && d->M > 0)
      return run_gemm_pair<kLinPairCfgs>(ctx, wa, wb, wep, wq, xa, xb, xep, xq, "ttrl_linear_backward", reserved);
    if (d->dW) {
      const int rc = run_gemm<kLinDwCfgs>(ctx, wa, wb, wep, wq.M, wq.N, wq.K, G, "ttrl_linear_backward dW", reserved);
      if (rc) return rc;
    }
    return run_gemm<kLinDxCfgs>(ctx, xa, xb, xep, d->M, nc, d->N, G, "ttrl_linear_backward dx", reserved);
  };
  if (d->W2) {
    LdRowKCat xb;  // B(r=k_in, k=n): n < n1 from W[k_in][n], else W2[k_in][n-n1]
    groups_of(xb.p1, d->W ? d->W + long(c0) * n1 : nullptr, d->gW, G);
    groups_of(xb.p2, d->W2 + long(c0) * (d->N - n1), d->gW, G);
    xb.ld1 = n1;
    xb.ld2 = d->N - n1;
    xb.rows = nc;
    xb.k1 = n1;
    xb.K = d->N;
    return finish(xb);
  }
  LdRowK xb;  // B(r=k_in, k=n) = W[k_in][n]
  groups_of(xb.p, d->W + long(c0) * d->N, d->gW, G);
  xb.ld = d->N;
  xb.rows = nc;
  xb.K = d->N;
  xb.vec_ok(all_aligned(xb.p, G));
  return finish(xb);
}

}  // extern "C"
