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

namespace ttrl {

GemmPlan plan_gemm(int M, int N, int K, int groups, long ws_floats, int force_cfg, int force_splits) {
  static const int order[] = {T128x64, T64x128, T64x64, T128x32, T64x32, T32x64, T32x32};
  const int mfit = ((M + 31) / 32) * 32, nfit = ((N + 31) / 32) * 32;
  int cfg = -1;
  if (force_cfg >= 0 && force_cfg < kNumCfg) {
    cfg = force_cfg;
  } else {
    for (int c : order) {
      const TileDims t = tile_dims(c);
      if (t.bm > mfit || t.bn > nfit) continue;
      const long tiles = long(ceil_div(M, t.bm)) * ceil_div(N, t.bn) * groups;
      if (tiles >= 240) {
        cfg = c;
        break;
      }
    }
    if (cfg < 0) cfg = (nfit >= 64 && mfit <= 32) ? T32x64 : T32x32;
  }
  const TileDims t = tile_dims(cfg);
  GemmPlan p{cfg, t.bm, t.bn, t.tbk, 1, t.tbk};
  const long tiles = long(ceil_div(M, t.bm)) * ceil_div(N, t.bn) * groups;
  const int stages = (K + t.tbk - 1) / t.tbk;  // LDS stages of the whole reduction
  int splits = 1;
  if (force_splits > 0) {
    splits = force_splits;
  } else if (stages > 1 && tiles < 160) {
    // Too few workgroups to cover the chip: split K until ~480 are in flight.
    const long want = (480 + tiles - 1) / tiles;
    splits = int(want < stages ? want : stages);
  } else if (stages > 4) {
    // Enough workgroups, but long serial reductions: cap them at 4 stages.
    splits = (stages + 3) / 4;
  }
  while (splits > 1 && long(splits) * groups * M * N > ws_floats) --splits;
  if (splits < 1) splits = 1;
  const int stages_per = (stages + splits - 1) / splits;
  p.kchunk = stages_per * t.tbk;
  p.splits = (K + p.kchunk - 1) / p.kchunk;
  if (p.splits < 1) p.splits = 1;
  return p;
}

namespace {

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
}  // namespace ttrl

using namespace ttrl;

extern "C" {

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
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (!ta && tb) {
    LdRowK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdRowK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (ta && !tb) {
    LdColK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdColK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else {
    LdColK la; la.p[0] = A; la.ld = lda; la.rows = M; la.K = K; la.vec_ok(aligned16(A));
    LdRowK lb; lb.p[0] = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec_ok(aligned16(B));
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
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
  lb.vec_ok(all_aligned(W, groups));
  if (split_w) {
    lb.ld2 = N - n1;
    lb.split = n1;
  }
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
    return run_gemm(ctx, la, lb, ep, M, N, K, groups, name);
  }
  LdRowK la;
  for (int g = 0; g < kMaxGroups; ++g) la.p[g] = x[g];
  la.ld = ldx;
  la.rows = M;
  la.K = K;
  la.vec_ok(all_aligned(x, groups));
  return run_gemm(ctx, la, lb, ep, M, N, K, groups, name);
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
  const float* ym[kMaxGroups];
  groups_of(dy, d->dy, d->gy, G);
  groups_of(ym, d->ymask, d->gy, G);
  const bool dyal = all_aligned(dy, G) && all_aligned(ym, G);

  if (d->dW) {
    TTRL_REQUIRE(d->x && !d->x2, "ttrl_linear_backward: dW needs a single dense input x");
    TTRL_REQUIRE(!d->W2 || d->dW2, "ttrl_linear_backward: a split weight needs dW2");
    // dW_aug[k][n] = sum_m xaug[m][k] dZ[m][n], xaug = [x | 1]; row K is db.
    const bool with_b = d->db != nullptr;
    TTRL_REQUIRE(!with_b || !d->W2 || d->db2, "ttrl_linear_backward: a split bias needs db2");
    LdColK la;  // A(r=k_in, k=m) = x[m][k_in]
    groups_of(la.p, d->x, d->gx, G);
    la.ld = d->ldx;
    la.rows = with_b ? d->K + 1 : d->K;
    la.K = d->M;
    la.real_rows = d->K;
    la.ones = with_b;
    la.vec_ok(all_aligned(la.p, G));
    LdColK lb;  // B(r=n, k=m) = dZ[m][n]
    for (int g = 0; g < kMaxGroups; ++g) {
      lb.p[g] = dy[g];
      lb.mask[g] = ym[g];
    }
    lb.ld = d->N;
    lb.rows = d->N;
    lb.K = d->M;
    lb.vec_ok(dyal);
    EpStore ep;
    ep.M = la.rows;
    ep.N = d->N;
    groups_of(ep.C, d->dW, d->gW, G);
    ep.ldc = n1;
    ep.rsplit = d->K;
    groups_of(ep.Cr, d->db, d->gb, G);
    ep.beta = d->beta_w;
    if (d->W2) {
      ep.csplit = n1;
      groups_of(ep.Cc, d->dW2, d->gW, G);
      ep.ldcc = d->N - n1;
      groups_of(ep.Crc, d->db2, d->gb, G);
    }
    int rc = run_gemm(ctx, la, lb, ep, la.rows, d->N, d->M > 0 ? d->M : 1, G, "ttrl_linear_backward dW");
    if (rc) return rc;
  }
  if (d->dx) {
    const int c0 = d->dx_cols > 0 ? d->dx_col0 : 0;
    const int nc = d->dx_cols > 0 ? d->dx_cols : d->K;
    TTRL_REQUIRE(c0 >= 0 && c0 + nc <= d->K, "ttrl_linear_backward: dx column range out of bounds");
    LdRowK la;  // A(m, k=n) = dZ[m][n]
    for (int g = 0; g < kMaxGroups; ++g) {
      la.p[g] = dy[g];
      la.mask[g] = ym[g];
    }
    la.ld = d->N;
    la.rows = d->M;
    la.K = d->N;
    la.vec_ok(dyal);
    EpStore ep;
    ep.M = d->M;
    ep.N = nc;
    groups_of(ep.C, d->dx, d->gdx, G);
    ep.ldc = d->lddx > 0 ? d->lddx : nc;
    ep.beta = d->beta_x;
    if (d->W2) {
      LdRowK2 lb;  // B(r=k_in, k=n): n < n1 from W[k_in][n], else W2[k_in][n-n1]
      groups_of(lb.p1, d->W ? d->W + long(c0) * n1 : nullptr, d->gW, G);
      groups_of(lb.p2, d->W2 + long(c0) * (d->N - n1), d->gW, G);
      lb.ld1 = n1;
      lb.ld2 = d->N - n1;
      lb.rows = nc;
      lb.k1 = n1;
      lb.K = d->N;
      return run_gemm(ctx, la, lb, ep, d->M, nc, d->N, G, "ttrl_linear_backward dx");
    }
    LdRowK lb;  // B(r=k_in, k=n) = W[k_in][n]
    groups_of(lb.p, d->W + long(c0) * d->N, d->gW, G);
    lb.ld = d->N;
    lb.rows = nc;
    lb.K = d->N;
    lb.vec_ok(all_aligned(lb.p, G));
    return run_gemm(ctx, la, lb, ep, d->M, nc, d->N, G, "ttrl_linear_backward dx");
  }
  return TTRL_OK;
}

}  // extern "C"
