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
  GemmPlan p{T32x32, 32, 32, 1, 0};
  const int mfit = ((M + 31) / 32) * 32, nfit = ((N + 31) / 32) * 32;
  bool chosen = false;
  if (force_cfg >= 0) {
    p.cfg = force_cfg;
    chosen = true;
  } else {
    for (int cfg : order) {
      int bm, bn;
      tile_dims(cfg, bm, bn);
      if (bm > mfit || bn > nfit) continue;
      const long tiles = long(ceil_div(M, bm)) * ceil_div(N, bn) * groups;
      if (tiles >= 192) {
        p.cfg = cfg;
        chosen = true;
        break;
      }
    }
    if (!chosen) p.cfg = (nfit >= 64 && mfit <= 32) ? T32x64 : T32x32;
  }
  tile_dims(p.cfg, p.bm, p.bn);
  const long tiles = long(ceil_div(M, p.bm)) * ceil_div(N, p.bn) * groups;
  int splits = 1;
  if (force_splits > 0) {
    splits = force_splits;
  } else if (tiles < 128 && K >= 8 * TBK) {
    splits = int((256 + tiles - 1) / tiles);
    const int max_by_k = K / (4 * TBK);
    if (splits > max_by_k) splits = max_by_k;
    if (splits < 1) splits = 1;
  }
  while (splits > 1 && long(splits) * groups * M * N > ws_floats) --splits;
  int chunk = (K + splits - 1) / splits;
  chunk = ((chunk + TBK - 1) / TBK) * TBK;
  if (chunk <= 0) chunk = TBK;
  p.splits = (K + chunk - 1) / chunk;
  if (p.splits < 1) p.splits = 1;
  p.kchunk = chunk;
  return p;
}

namespace {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

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
  ep.C = C;
  ep.ldc = ldc;
  ep.alpha = alpha;
  ep.beta = beta;
  if (K == 0) {
    // An empty reduction still defines C = beta*C.
    ep.alpha = 0.f;
  }
  const bool va = aligned16(A) && lda % 4 == 0, vb = aligned16(B) && ldb % 4 == 0;
  const int Kr = K > 0 ? K : 1;
  if (!ta && !tb) {
    LdRowK la; la.p = A; la.ld = lda; la.rows = M; la.K = K; la.vec = va;
    LdColK lb; lb.p = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec = vb;
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (!ta && tb) {
    LdRowK la; la.p = A; la.ld = lda; la.rows = M; la.K = K; la.vec = va;
    LdRowK lb; lb.p = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec = vb;
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else if (ta && !tb) {
    LdColK la; la.p = A; la.ld = lda; la.rows = M; la.K = K; la.vec = va;
    LdColK lb; lb.p = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec = vb;
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  } else {
    LdColK la; la.p = A; la.ld = lda; la.rows = M; la.K = K; la.vec = va;
    LdRowK lb; lb.p = B; lb.ld = ldb; lb.rows = N; lb.K = K; lb.vec = vb;
    return run_gemm(ctx, la, lb, ep, M, N, Kr, 1, "ttrl_matmul");
  }
}

int ttrl_linear_forward(ttrl_ctx* ctx, const ttrl_linear_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_linear_forward: null argument");
  TTRL_REQUIRE(d->x && d->W && d->y, "ttrl_linear_forward: x, W and y are required");
  TTRL_REQUIRE(d->M >= 0 && d->K > 0 && d->N > 0 && d->groups >= 1, "ttrl_linear_forward: bad extents");
  const int n1 = d->W2 ? d->n1 : d->N;
  TTRL_REQUIRE(n1 > 0 && n1 <= d->N, "ttrl_linear_forward: n1 out of range");
  const int k1 = d->x2 ? d->k1 : d->K;
  TTRL_REQUIRE(k1 > 0 && k1 <= d->K, "ttrl_linear_forward: k1 out of range");

  EpStore ep;
  ep.M = d->M;
  ep.N = d->N;
  ep.C = d->y;
  ep.ldc = d->N;
  ep.gC = d->gy;
  ep.bias = d->b;
  ep.gb = d->gb;
  if (d->W2) {
    ep.csplit = n1;
    ep.Cc = d->y + n1;  // same row-major [M][N] output, rebased column
    ep.ldcc = d->N;
    ep.gCc = d->gy;
    ep.bias2 = d->b2;
    ep.gb2 = d->gb;
  }
  ep.relu = d->relu;
  ep.clamp_col = d->clamp_col > 0 ? d->clamp_col : (1 << 30);
  ep.lo = d->lo;
  ep.hi = d->hi;

  LdColK lb;  // B(k, n) = W[k][n]
  lb.p = d->W;
  lb.ld = n1;
  lb.gs = d->gW;
  lb.rows = d->N;
  lb.K = d->K;
  lb.vec = aligned16(d->W) && n1 % 4 == 0 && d->gW % 4 == 0;
  if (d->W2) {
    lb.p2 = d->W2;
    lb.ld2 = d->N - n1;
    lb.split = n1;
  }
  if (d->x2) {
    LdRowKCat la;
    la.p1 = d->x;
    la.ld1 = d->ldx;
    la.gs1 = d->gx;
    la.p2 = d->x2;
    la.ld2 = d->ldx2;
    la.gs2 = d->gx2;
    la.rows = d->M;
    la.k1 = k1;
    la.K = d->K;
    return run_gemm(ctx, la, lb, ep, d->M, d->N, d->K, d->groups, "ttrl_linear_forward");
  }
  LdRowK la;
  la.p = d->x;
  la.ld = d->ldx;
  la.gs = d->gx;
  la.rows = d->M;
  la.K = d->K;
  la.vec = aligned16(d->x) && d->ldx % 4 == 0 && d->gx % 4 == 0;
  return run_gemm(ctx, la, lb, ep, d->M, d->N, d->K, d->groups, "ttrl_linear_forward");
}

int ttrl_linear_backward(ttrl_ctx* ctx, const ttrl_linear_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_linear_backward: null argument");
  TTRL_REQUIRE(d->dy && d->W, "ttrl_linear_backward: dy and W are required");
  TTRL_REQUIRE(d->M >= 0 && d->K > 0 && d->N > 0 && d->groups >= 1, "ttrl_linear_backward: bad extents");
  const int n1 = d->W2 ? d->n1 : d->N;
  TTRL_REQUIRE(n1 > 0 && n1 <= d->N, "ttrl_linear_backward: n1 out of range");
  const bool dyvec = aligned16(d->dy) && d->N % 4 == 0 && d->gy % 4 == 0 &&
                     (!d->ymask || aligned16(d->ymask));

  if (d->dW) {
    TTRL_REQUIRE(d->x && !d->x2, "ttrl_linear_backward: dW needs a single dense input x");
    TTRL_REQUIRE(!d->W2 || d->dW2, "ttrl_linear_backward: a split weight needs dW2");
    // dW_aug[k][n] = sum_m xaug[m][k] dZ[m][n], xaug = [x | 1]; row K is db.
    const bool with_b = d->db != nullptr;
    LdColK la;  // A(r=k_in, k=m) = x[m][k_in]
    la.p = d->x;
    la.ld = d->ldx;
    la.gs = d->gx;
    la.rows = with_b ? d->K + 1 : d->K;
    la.K = d->M;
    la.real_rows = d->K;
    la.ones = with_b;
    la.vec = aligned16(d->x) && d->ldx % 4 == 0 && d->gx % 4 == 0;
    LdColK lb;  // B(r=n, k=m) = dZ[m][n]
    lb.p = d->dy;
    lb.ld = d->N;
    lb.gs = d->gy;
    lb.rows = d->N;
    lb.K = d->M;
    lb.mask = d->ymask;
    lb.vec = dyvec;
    EpStore ep;
    ep.M = la.rows;
    ep.N = d->N;
    ep.C = d->dW;
    ep.ldc = n1;
    ep.gC = d->gW;
    ep.rsplit = d->K;
    ep.Cr = d->db;
    ep.gCr = d->gb;
    ep.beta = d->beta_w;
    if (d->W2) {
      ep.csplit = n1;
      ep.Cc = d->dW2;
      ep.ldcc = d->N - n1;
      ep.gCc = d->gW;
      ep.Crc = d->db2;
      ep.gCrc = d->gb;
      TTRL_REQUIRE(!with_b || d->db2, "ttrl_linear_backward: a split bias needs db2");
    }
    int rc = run_gemm(ctx, la, lb, ep, la.rows, d->N, d->M > 0 ? d->M : 1, d->groups, "ttrl_linear_backward dW");
    if (rc) return rc;
  }
  if (d->dx) {
    const int c0 = d->dx_cols > 0 ? d->dx_col0 : 0;
    const int nc = d->dx_cols > 0 ? d->dx_cols : d->K;
    TTRL_REQUIRE(c0 >= 0 && c0 + nc <= d->K, "ttrl_linear_backward: dx column range out of bounds");
    LdRowK la;  // A(m, k=n) = dZ[m][n]
    la.p = d->dy;
    la.ld = d->N;
    la.gs = d->gy;
    la.rows = d->M;
    la.K = d->N;
    la.mask = d->ymask;
    la.vec = dyvec;
    EpStore ep;
    ep.M = d->M;
    ep.N = nc;
    ep.C = d->dx;
    ep.ldc = d->lddx > 0 ? d->lddx : nc;
    ep.gC = d->gdx;
    ep.beta = d->beta_x;
    if (d->W2) {
      // B(r=k_in, k=n): n < n1 from W[k_in][n], else W2[k_in][n-n1].
      LdRowK2 lb{d->W + long(c0) * n1, d->W2 + long(c0) * (d->N - n1), n1, d->N - n1, d->gW, nc, n1, d->N};
      return run_gemm(ctx, la, lb, ep, d->M, nc, d->N, d->groups, "ttrl_linear_backward dx");
    }
    LdRowK lb;  // B(r=k_in, k=n) = W[k_in][n]
    lb.p = d->W + long(c0) * d->N;
    lb.ld = d->N;
    lb.gs = d->gW;
    lb.rows = nc;
    lb.K = d->N;
    lb.vec = aligned16(lb.p) && d->N % 4 == 0 && d->gW % 4 == 0;
    return run_gemm(ctx, la, lb, ep, d->M, nc, d->N, d->groups, "ttrl_linear_backward dx");
  }
  return TTRL_OK;
}

}  // extern "C"
