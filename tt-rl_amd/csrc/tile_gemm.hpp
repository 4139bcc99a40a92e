// FP32 MFMA tile GEMM core for gfx950: C[g](m, n) = sum_k A[g](m, k) * B[g](k, n).
//
// Work decomposition.  A workgroup of WGM x WGN wavefronts (64 lanes each)
// owns a BM x BN output tile; each wavefront owns a (BM/WGM) x (BN/WGN)
// sub-tile built from 16x16 v_mfma_f32_16x16x4f32 fragments.  The reduction
// runs in TBK-wide slices staged through LDS with k contiguous per row, so
// every lane feeds four consecutive MFMAs from one 128-bit LDS read:
// lane l of step s supplies A(row l%16, k = 4*(l/16)+s) and
// B(k = 4*(l/16)+s, col l%16), a fixed permutation of k shared by both
// operands, so the 16-wide slice is summed exactly once.
//
// Operands are produced by loader objects, so one core serves dense matrices
// (either storage order), implicit-GEMM convolution patches, masked ReLU
// gradients and the implicit ones row that folds a bias gradient into a
// weight-gradient GEMM.  A loader with KCONTIG returns four consecutive k of
// one row; otherwise four consecutive rows at one k.  Loaders bounds-check
// and return zeros outside the operand, so ragged M, N and K need no padding.
//
// blockIdx.z = group * splits + split: groups are independent problems
// (batched weights, convolution residue classes), splits partition K.  A
// split-K launch writes partial tiles to a workspace that a second kernel
// sums in split order, so results never depend on scheduling.
#pragma once

#include "common.hpp"

namespace ttrl {

constexpr int TBK = 32;         // reduction slice staged per LDS round
constexpr int TLDK = TBK + 4;   // padded LDS row, in floats

// ------------------------------------------------------------- loaders ---

// v(r, k) = p[g*gs + r*ld + k] * [mask(r, k) > 0]; k contiguous.
struct LdRowK {
  static constexpr bool KCONTIG = true;
  const float* p = nullptr;
  long ld = 0, gs = 0;
  int rows = 0, K = 0;
  const float* mask = nullptr;  // same indexing as p (ld, gs)
  bool vec = false;             // p, ld and gs allow aligned float4 loads

  __device__ inline float at(int r, int k, int g) const {
    const long i = g * gs + long(r) * ld + k;
    float v = p[i];
    if (mask) v = mask[i] > 0.f ? v : 0.f;
    return v;
  }
  __device__ inline f32x4 load4(int r, int k, int g) const {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (r >= rows || k >= K) return v;
    if (vec && k + 3 < K) {
      const long i = g * gs + long(r) * ld + k;
      v = *reinterpret_cast<const f32x4*>(p + i);
      if (mask) {
        const f32x4 mk = *reinterpret_cast<const f32x4*>(mask + i);
        v.x = mk.x > 0.f ? v.x : 0.f;
        v.y = mk.y > 0.f ? v.y : 0.f;
        v.z = mk.z > 0.f ? v.z : 0.f;
        v.w = mk.w > 0.f ? v.w : 0.f;
      }
      return v;
    }
    v.x = at(r, k, g);
    if (k + 1 < K) v.y = at(r, k + 1, g);
    if (k + 2 < K) v.z = at(r, k + 2, g);
    if (k + 3 < K) v.w = at(r, k + 3, g);
    return v;
  }
};

// v(r, k) = p[g*gs + k*ld + r] * [mask > 0]; r contiguous.  Rows at or past
// `real_rows` read 1.0 when `ones` is set and r == real_rows (the implicit
// ones row of a bias gradient), else 0.  Rows >= `split` read from p2 at
// column r - split with leading dimension ld2 (a second weight matrix that
// sits beside the first along the output axis).
struct LdColK {
  static constexpr bool KCONTIG = false;
  const float* p = nullptr;
  long ld = 0, gs = 0;
  int rows = 0, K = 0;
  const float* mask = nullptr;
  bool vec = false;
  int real_rows = 1 << 30;
  bool ones = false;
  const float* p2 = nullptr;
  long ld2 = 0;
  int split = 1 << 30;

  __device__ inline float at(int r, int k, int g) const {
    if (r >= rows || k >= K) return 0.f;
    if (r >= real_rows) return (ones && r == real_rows) ? 1.f : 0.f;
    if (r >= split) return p2[g * gs + long(k) * ld2 + (r - split)];
    const long i = g * gs + long(k) * ld + r;
    float v = p[i];
    if (mask) v = mask[i] > 0.f ? v : 0.f;
    return v;
  }
  __device__ inline f32x4 load4(int r, int k, int g) const {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (k >= K || r >= rows) return v;
    if (vec && r + 3 < real_rows && r + 3 < split && r + 3 < rows) {
      const long i = g * gs + long(k) * ld + r;
      v = *reinterpret_cast<const f32x4*>(p + i);
      if (mask) {
        const f32x4 mk = *reinterpret_cast<const f32x4*>(mask + i);
        v.x = mk.x > 0.f ? v.x : 0.f;
        v.y = mk.y > 0.f ? v.y : 0.f;
        v.z = mk.z > 0.f ? v.z : 0.f;
        v.w = mk.w > 0.f ? v.w : 0.f;
      }
      return v;
    }
    v.x = at(r, k, g);
    v.y = at(r + 1, k, g);
    v.z = at(r + 2, k, g);
    v.w = at(r + 3, k, g);
    return v;
  }
};

// Concatenation along k of two row-major operands: k < k1 reads p1[r*ld1+k],
// k >= k1 reads p2[r*ld2 + k-k1].  The SAC critic's concat(s, a) input.
struct LdRowKCat {
  static constexpr bool KCONTIG = true;
  const float* p1 = nullptr;
  const float* p2 = nullptr;
  long ld1 = 0, ld2 = 0, gs1 = 0, gs2 = 0;
  int rows = 0, k1 = 0, K = 0;

  __device__ inline float at(int r, int k, int g) const {
    if (r >= rows || k >= K) return 0.f;
    if (k < k1) return p1[g * gs1 + long(r) * ld1 + k];
    return p2[g * gs2 + long(r) * ld2 + (k - k1)];
  }
  __device__ inline f32x4 load4(int r, int k, int g) const {
    f32x4 v;
    v.x = at(r, k, g);
    v.y = at(r, k + 1, g);
    v.z = at(r, k + 2, g);
    v.w = at(r, k + 3, g);
    return v;
  }
};

// Concatenation along k of two row-major matrices of `rows` rows: k < k1
// reads p1[r*ld1 + k], k >= k1 reads p2[r*ld2 + k-k1] (the transposed view
// of two weight matrices that sit side by side along the output axis).
struct LdRowK2 {
  static constexpr bool KCONTIG = true;
  const float* p1;
  const float* p2;
  long ld1, ld2, gs;
  int rows, k1, K;
  __device__ inline float at(int r, int k, int g) const {
    if (r >= rows || k >= K) return 0.f;
    return k < k1 ? p1[g * gs + long(r) * ld1 + k] : p2[g * gs + long(r) * ld2 + (k - k1)];
  }
  __device__ inline f32x4 load4(int r, int k, int g) const {
    return f32x4{at(r, k, g), at(r, k + 1, g), at(r, k + 2, g), at(r, k + 3, g)};
  }
};

// ----------------------------------------------------------- epilogues ---

// Element (m, n) of group g goes to one of four row-major blocks: rows
// >= rsplit and columns >= csplit address the tail blocks with their index
// rebased to 0.  v = alpha*acc (+ bias) (relu | clamp) (+ beta*old).
struct EpStore {
  int M = 0, N = 0;
  float* C = nullptr;   long ldc = 0, gC = 0;
  float* Cr = nullptr;  long gCr = 0;                 // rows >= rsplit, ld = ldc
  float* Cc = nullptr;  long ldcc = 0, gCc = 0;       // cols >= csplit
  float* Crc = nullptr; long gCrc = 0;                // both tails, ld = ldcc
  int rsplit = 1 << 30, csplit = 1 << 30;
  float alpha = 1.f, beta = 0.f;
  float alpha_r = 1.f;                                // scale of rows >= rsplit
  const float* bias = nullptr;  long gb = 0;          // cols < csplit
  const float* bias2 = nullptr; long gb2 = 0;         // cols >= csplit
  int relu = 0;
  int clamp_col = 1 << 30;                            // cols >= clamp_col clamp to [lo, hi]
  float lo = 0.f, hi = 0.f;

  __device__ inline int rows(int) const { return M; }
  __device__ inline void store(int m, int n, float acc, int g) const {
    if (m >= M || n >= N) return;
    const bool rt = m >= rsplit, ct = n >= csplit;
    const int mm = rt ? m - rsplit : m;
    const int nn = ct ? n - csplit : n;
    float v = (rt ? alpha_r : alpha) * acc;
    if (!ct && bias) v += bias[g * gb + nn];
    if (ct && bias2) v += bias2[g * gb2 + nn];
    if (relu) v = v > 0.f ? v : 0.f;
    if (n >= clamp_col) v = fminf(fmaxf(v, lo), hi);
    float* dst;
    if (!rt && !ct) dst = C + g * gC + long(mm) * ldc + nn;
    else if (rt && !ct) dst = Cr + g * gCr + long(mm) * ldc + nn;
    else if (!rt && ct) dst = Cc + g * gCc + long(mm) * ldcc + nn;
    else dst = Crc + g * gCrc + long(mm) * ldcc + nn;
    if (beta != 0.f) v += beta * *dst;
    *dst = v;
  }
};

// ----------------------------------------------------------- the core ----

template <int ROWS, int NT, class L>
__device__ inline void stage_tile(float* T, const L& ld, int r0, int k0, int g, int tid) {
  if constexpr (L::KCONTIG) {
    constexpr int CH = TBK / 4;
#pragma unroll 2
    for (int i = tid; i < ROWS * CH; i += NT) {
      const int r = i / CH, c = (i - r * CH) * 4;
      *reinterpret_cast<f32x4*>(T + r * TLDK + c) = ld.load4(r0 + r, k0 + c, g);
    }
  } else {
    constexpr int CH = ROWS / 4;
#pragma unroll 2
    for (int i = tid; i < TBK * CH; i += NT) {
      const int k = i / CH, r = (i - k * CH) * 4;
      const f32x4 v = ld.load4(r0 + r, k0 + k, g);
      T[(r + 0) * TLDK + k] = v.x;
      T[(r + 1) * TLDK + k] = v.y;
      T[(r + 2) * TLDK + k] = v.z;
      T[(r + 3) * TLDK + k] = v.w;
    }
  }
}

template <int BM, int BN, int WGM, int WGN, bool PARTIAL, class LA, class LB, class EP>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm(LA la, LB lb, EP ep, float* ws, int M, int N,
                                                         int K, int kchunk, int splits) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "bad tile");
  __shared__ __attribute__((aligned(16))) float As[BM * TLDK];
  __shared__ __attribute__((aligned(16))) float Bs[BN * TLDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int g = blockIdx.z / splits, split = blockIdx.z - g * splits;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  if (m0 >= ep.rows(g)) return;  // uniform per block: ragged residue classes
  const int kbeg = split * kchunk;
  const int kend = min(K, kbeg + kchunk);

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lk = (lane >> 4) * 4;
  for (int k0 = kbeg; k0 < kend; k0 += TBK) {
    stage_tile<BM, NT>(As, la, m0, k0, g, tid);
    stage_tile<BN, NT>(Bs, lb, n0, k0, g, tid);
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < TBK; kb += 16) {
      f32x4 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = *reinterpret_cast<const f32x4*>(As + (wm * WTM + i * 16 + lr) * TLDK + kb + lk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const f32x4*>(Bs + (wn * WTN + j * 16 + lr) * TLDK + kb + lk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();
  }

  // Fragment (i, j) register r holds C(row 4*(lane/16) + r, col lane%16).
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
        const int n = n0 + wn * WTN + j * 16 + lr;
        if constexpr (PARTIAL) {
          if (m < M && n < N) ws[((long(g) * splits + split) * M + m) * N + n] = acc[i][j][r];
        } else {
          ep.store(m, n, acc[i][j][r], g);
        }
      }
}

// Sums split-K partials in split order and applies the epilogue.
template <class EP>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* ws, EP ep, int M, int N, int splits,
                                                       int groups) {
  const long total = long(groups) * M * N;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += long(gridDim.x) * 256) {
    const int g = int(i / (long(M) * N));
    const long mn = i - long(g) * M * N;
    const int m = int(mn / N), n = int(mn - long(m) * N);
    if (m >= ep.rows(g)) continue;
    float s = 0.f;
    const float* p = ws + (long(g) * splits) * M * N + mn;
    for (int sp = 0; sp < splits; ++sp) s += p[long(sp) * M * N];
    ep.store(m, n, s, g);
  }
}

// Tile shapes.  The host picks one per problem from the output extent.
enum TileCfg { T32x32 = 0, T64x32 = 1, T32x64 = 2, T64x64 = 3, T128x32 = 4, T128x64 = 5, T64x128 = 6 };

struct GemmPlan {
  int cfg, bm, bn, splits, kchunk;
};

inline void tile_dims(int cfg, int& bm, int& bn) {
  switch (cfg) {
    case T32x32: bm = 32; bn = 32; break;
    case T64x32: bm = 64; bn = 32; break;
    case T32x64: bm = 32; bn = 64; break;
    case T64x64: bm = 64; bn = 64; break;
    case T128x32: bm = 128; bn = 32; break;
    case T128x64: bm = 128; bn = 64; break;
    default: bm = 64; bn = 128; break;
  }
}

// Chooses a tile and a split-K factor: enough workgroups to cover the 256
// CUs, each split at least `min_k` deep, within `ws_floats` of workspace.
GemmPlan plan_gemm(int M, int N, int K, int groups, long ws_floats, int force_cfg = -1, int force_splits = 0);

// Workspace owned by the context (stream-ordered scratch for split-K).
float* ctx_workspace(ttrl_ctx* ctx, long* floats);

template <int BM, int BN, int WGM, int WGN, class LA, class LB, class EP>
inline void launch_cfg(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K, int groups,
                       const GemmPlan& p, hipStream_t st) {
  dim3 grid(ceil_div(M, BM), ceil_div(N, BN), unsigned(groups * p.splits));
  if (p.splits == 1) {
    hipLaunchKernelGGL((k_gemm<BM, BN, WGM, WGN, false, LA, LB, EP>), grid, dim3(64 * WGM * WGN), 0, st, la,
                       lb, ep, ws, M, N, K, p.kchunk, 1);
  } else {
    hipLaunchKernelGGL((k_gemm<BM, BN, WGM, WGN, true, LA, LB, EP>), grid, dim3(64 * WGM * WGN), 0, st, la,
                       lb, ep, ws, M, N, K, p.kchunk, p.splits);
    const long total = long(groups) * M * N;
    unsigned blocks = unsigned(total / 256 + 1);
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL((k_splitk_reduce<EP>), dim3(blocks), dim3(256), 0, st, ws, ep, M, N, p.splits, groups);
  }
}

template <class LA, class LB, class EP>
inline int run_gemm(ttrl_ctx* ctx, const LA& la, const LB& lb, const EP& ep, int M, int N, int K, int groups,
                    const char* name, int force_cfg = -1, int force_splits = 0) {
  if (M <= 0 || N <= 0 || groups <= 0) return TTRL_OK;
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  GemmPlan p = plan_gemm(M, N, K, groups, wsf, force_cfg, force_splits);
  hipStream_t st = stream_of(ctx);
  switch (p.cfg) {
    case T32x32: launch_cfg<32, 32, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T64x32: launch_cfg<64, 32, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T32x64: launch_cfg<32, 64, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T64x64: launch_cfg<64, 64, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T128x32: launch_cfg<128, 32, 4, 1>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T128x64: launch_cfg<128, 64, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    default: launch_cfg<64, 128, 2, 2>(la, lb, ep, ws, M, N, K, groups, p, st); break;
  }
  return check_launch(name);
}

}  // namespace ttrl
