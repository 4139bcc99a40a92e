// FP32 MFMA tile GEMM core for gfx950: C[g](m, n) = sum_k A[g](m, k) * B[g](k, n).
//
// Work decomposition.  A workgroup of WGM x WGN wavefronts (64 lanes each)
// owns a BM x BN output tile; each wavefront owns a (BM/WGM) x (BN/WGN)
// sub-tile built from 16x16 v_mfma_f32_16x16x4f32 fragments.  The reduction
// is staged through LDS in slices of TBK (up to 256): at the batch sizes of
// a learner update most workgroups own a single slice, so every global load
// of the workgroup is in flight at once and the load latency is paid once.
//
// MFMA operand order.  Lane l of step s supplies A(row l%16, k = 4*(l/16)+s)
// and B(k = 4*(l/16)+s, col l%16): a fixed permutation of each 16-wide
// k-block shared by both operands, so the block is summed exactly once.
//
// Operands come from loader objects, so one core serves dense matrices in
// either storage order, implicit-GEMM convolution patches, masked ReLU
// gradients and the implicit ones row that folds a bias gradient into a
// weight-gradient GEMM.  A KCONTIG loader returns four consecutive k of one
// row and is staged row-major ([rows][TBK+4], one 128-bit LDS read feeds four
// MFMAs); any other loader returns four consecutive rows at one k and is
// staged k-major ([TBK][rows+4], 128-bit LDS stores, 32-bit reads), so
// neither layout takes bank conflicts on its stores.  Loaders bounds-check
// and return zeros outside the operand, so ragged M, N and K need no padding.
//
// blockIdx.z = group * splits + split: groups are independent problems
// (per-group pointer tables: twin critics, online/target networks,
// convolution residue classes), splits partition K.  A split-K launch writes
// partial tiles to a workspace that a second kernel sums in split order, so
// results never depend on scheduling.
#pragma once

#include "common.hpp"

namespace ttrl {

constexpr int kMaxGroups = 4;

// Division by a runtime-constant positive divisor d with a multiply-high:
// q = (umulhi(n, m) + n) >> s, m = floor(2^32 (2^s - d) / d) + 1, s = ceil(log2 d)
// (exact for 0 <= n < 2^31).
struct FDiv {
  uint32_t m = 0, s = 0;
  int d = 1;
  __host__ void set(int divisor) {
    d = divisor;
    s = 0;
    while ((1u << s) < uint32_t(divisor)) ++s;
    const uint64_t two32 = uint64_t(1) << 32;
    m = uint32_t((two32 * ((uint64_t(1) << s) - uint64_t(divisor))) / uint64_t(divisor) + 1);
  }
  __device__ inline int div(int n) const {
    const uint32_t hi = __umulhi(uint32_t(n), m);
    return int((uint64_t(hi) + uint32_t(n)) >> s);
  }
};

// ------------------------------------------------------------- loaders ---
//
// Loaders work in two phases so that a workgroup's loads are all in flight
// before any of them is waited on: issue() computes the addresses (clamped
// into the operand, so every load is legal) and starts the loads into a
// Fetch4, recording which of the four elements are real; resolve() runs
// after every issue() of the stage and applies those predicates and the
// ReLU mask.  Issue paths never read a loaded value.

struct Fetch4 {
  f32x4 v;
  f32x4 m;      // mask values (1.0 where an element is not masked)
  uint32_t ok;  // bit j: element j lies inside the operand; kU8Word, kU8Each: v holds bytes
};

constexpr uint32_t kU8Word = 0x10u;  // v.x carries four uint8 values packed in one word
constexpr uint32_t kU8Each = 0x20u;  // each element carries one uint8 value as integer bits

__device__ inline f32x4 resolve4(const Fetch4& f, bool masked) {
  f32x4 v = f.v;
  if (f.ok & kU8Word) {
    const uint32_t w = __float_as_uint(f.v.x);
    v = f32x4{float(w & 0xffu), float((w >> 8) & 0xffu), float((w >> 16) & 0xffu), float(w >> 24)};
  } else if (f.ok & kU8Each) {
    v = f32x4{float(__float_as_uint(f.v.x)), float(__float_as_uint(f.v.y)), float(__float_as_uint(f.v.z)),
              float(__float_as_uint(f.v.w))};
  }
  v.x = ((f.ok & 1u) && (!masked || f.m.x > 0.f)) ? v.x : 0.f;
  v.y = ((f.ok & 2u) && (!masked || f.m.y > 0.f)) ? v.y : 0.f;
  v.z = ((f.ok & 4u) && (!masked || f.m.z > 0.f)) ? v.z : 0.f;
  v.w = ((f.ok & 8u) && (!masked || f.m.w > 0.f)) ? v.w : 0.f;
  return v;
}

// v(r, k) = p[g][r*ld + k] * [mask[g](r, k) > 0]; k contiguous.
struct LdRowK {
  static constexpr bool KCONTIG = true;
  const float* p[kMaxGroups] = {};
  const float* mask[kMaxGroups] = {};  // same indexing as p
  long ld = 0;
  int rows = 0, K = 0;
  bool vec = false;  // p[g], mask[g] 16-byte aligned and ld, K multiples of 4 (set by vec_ok)

  __host__ void vec_ok(bool aligned) { vec = aligned && ld % 4 == 0 && K % 4 == 0; }
  __device__ inline bool masked(int g) const { return mask[g] != nullptr; }
  __device__ inline void issue(int r, int k, int g, Fetch4& f) const {
    const bool rv = r < rows;
    const float* base = p[g];
    const float* mb = mask[g];
    if (vec) {  // uniform: K % 4 == 0, so k < K covers all four
      const bool in = rv && k < K;
      const long i = in ? long(r) * ld + k : 0;
      f.v = *reinterpret_cast<const f32x4*>(base + i);
      if (mb) f.m = *reinterpret_cast<const f32x4*>(mb + i);
      f.ok = in ? 0xFu : 0u;
      return;
    }
    f.ok = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool vj = rv && k + j < K;
      const long i = vj ? long(r) * ld + k + j : 0;
      f.v[j] = base[i];
      if (mb) f.m[j] = mb[i];
      f.ok |= uint32_t(vj) << j;
    }
  }
};

// v(r, k) = p[g][k*ld + r] * [mask > 0]; r contiguous.  Row `real_rows` reads
// 1.0 when `ones` is set (the implicit ones row of a bias gradient); rows >=
// `split` read p2[g][k*ld2 + r - split] (a second weight matrix beside the
// first along the output axis).
struct LdColK {
  static constexpr bool KCONTIG = false;
  const float* p[kMaxGroups] = {};
  const float* mask[kMaxGroups] = {};
  const float* p2[kMaxGroups] = {};
  long ld = 0, ld2 = 0;
  int rows = 0, K = 0;
  bool vec = false;
  int real_rows = 1 << 30;
  bool ones = false;
  int split = 1 << 30;

  // Vector loads need aligned bases and ld % 4 == 0; a 4-row chunk that
  // straddles `rows`, `real_rows` or `split` takes the element path.
  __host__ void vec_ok(bool aligned) { vec = aligned && ld % 4 == 0; }
  __device__ inline bool masked(int g) const { return mask[g] != nullptr; }
  __device__ inline void issue(int r, int k, int g, Fetch4& f) const {
    const bool kv = k < K;
    const float* base = p[g];
    const float* mb = mask[g];
    if (vec && r + 3 < real_rows && r + 3 < split && r + 3 < rows) {
      const long i = kv ? long(k) * ld + r : 0;
      f.v = *reinterpret_cast<const f32x4*>(base + i);
      if (mb) f.m = *reinterpret_cast<const f32x4*>(mb + i);
      f.ok = kv ? 0xFu : 0u;
      return;
    }
    f.ok = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = r + j;
      const bool in = kv && rr < rows;
      f.m[j] = 1.f;
      if (in && rr >= real_rows) {
        f.v[j] = (ones && rr == real_rows) ? 1.f : 0.f;
      } else if (in && rr >= split) {
        f.v[j] = p2[g][long(k) * ld2 + (rr - split)];
      } else {
        const long i = in ? long(k) * ld + rr : 0;
        f.v[j] = base[i];
        if (mb) f.m[j] = mb[i];
      }
      f.ok |= uint32_t(in) << j;
    }
  }
};

// Concatenation along k of two row-major operands: k < k1 reads p1[g][r*ld1+k],
// k >= k1 reads p2[g][r*ld2 + k-k1] (the SAC critic's concat(s, a) input).
struct LdRowKCat {
  static constexpr bool KCONTIG = true;
  const float* p1[kMaxGroups] = {};
  const float* p2[kMaxGroups] = {};
  long ld1 = 0, ld2 = 0;
  int rows = 0, k1 = 0, K = 0;

  __device__ inline bool masked(int) const { return false; }
  __device__ inline void issue(int r, int k, int g, Fetch4& f) const {
    f.ok = 0;
    const bool rv = r < rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = k + j;
      const bool vj = rv && kk < K;
      const bool first = kk < k1;
      const float* base = first ? p1[g] : p2[g];
      const long i = !vj ? 0 : (first ? long(r) * ld1 + kk : long(r) * ld2 + (kk - k1));
      f.v[j] = base[i];
      f.ok |= uint32_t(vj) << j;
    }
  }
};

// Concatenation along k of two row-major matrices: k < k1 reads p1[g][r*ld1 + k],
// k >= k1 reads p2[g][r*ld2 + k-k1] (the transposed view of two weight
// matrices side by side along the output axis).
struct LdRowK2 {
  static constexpr bool KCONTIG = true;
  const float* p1[kMaxGroups] = {};
  const float* p2[kMaxGroups] = {};
  long ld1 = 0, ld2 = 0;
  int rows = 0, k1 = 0, K = 0;

  __device__ inline bool masked(int) const { return false; }
  __device__ inline void issue(int r, int k, int g, Fetch4& f) const {
    f.ok = 0;
    const bool rv = r < rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = k + j;
      const bool vj = rv && kk < K;
      const bool first = kk < k1;
      const float* base = first ? p1[g] : p2[g];
      const long i = !vj ? 0 : (first ? long(r) * ld1 + kk : long(r) * ld2 + (kk - k1));
      f.v[j] = base[i];
      f.ok |= uint32_t(vj) << j;
    }
  }
};

// ----------------------------------------------------------- epilogues ---

// Element (m, n) of group g goes to one of four row-major blocks: rows
// >= rsplit and columns >= csplit address the tail blocks with their index
// rebased to 0.  v = alpha*acc (+ bias) (relu | clamp) (+ beta*old).
struct EpStore {
  int M = 0, N = 0;
  float* C[kMaxGroups] = {};    long ldc = 0;
  float* Cr[kMaxGroups] = {};                     // rows >= rsplit, ld = ldc
  float* Cc[kMaxGroups] = {};   long ldcc = 0;    // cols >= csplit
  float* Crc[kMaxGroups] = {};                    // both tails, ld = ldcc
  int rsplit = 1 << 30, csplit = 1 << 30;
  float alpha = 1.f, beta = 0.f;
  float alpha_r = 1.f;                            // scale of rows >= rsplit
  const float* bias[kMaxGroups] = {};             // cols < csplit
  const float* bias2[kMaxGroups] = {};            // cols >= csplit
  int relu = 0;
  int clamp_col = 1 << 30;                        // cols >= clamp_col clamp to [lo, hi]
  float lo = 0.f, hi = 0.f;

  __device__ inline int rows(int) const { return M; }
  __device__ inline void store(int m, int n, float acc, int g) const {
    if (m >= M || n >= N) return;
    const bool rt = m >= rsplit, ct = n >= csplit;
    const int mm = rt ? m - rsplit : m;
    const int nn = ct ? n - csplit : n;
    float v = (rt ? alpha_r : alpha) * acc;
    if (!ct && bias[g]) v += bias[g][nn];
    if (ct && bias2[g]) v += bias2[g][nn];
    if (relu) v = v > 0.f ? v : 0.f;
    if (n >= clamp_col) v = fminf(fmaxf(v, lo), hi);
    float* dst;
    if (!rt && !ct) dst = C[g] + long(mm) * ldc + nn;
    else if (rt && !ct) dst = Cr[g] + long(mm) * ldc + nn;
    else if (!rt && ct) dst = Cc[g] + long(mm) * ldcc + nn;
    else dst = Crc[g] + long(mm) * ldcc + nn;
    if (beta != 0.f) v += beta * *dst;
    *dst = v;
  }
};

// ----------------------------------------------------------- the core ----

// LDS footprint of one staged operand, in floats.
template <int ROWS, int TBK, bool KCONTIG>
struct TileLds {
  static constexpr int LD = KCONTIG ? TBK + 4 : ROWS + 4;  // padded leading dimension
  static constexpr int SIZE = KCONTIG ? ROWS * LD : TBK * LD;
};

template <int ROWS, int TBK, int NT, class L>
__device__ inline void stage_tile(float* T, const L& ld, int r0, int k0, int g, int tid) {
  using Lds = TileLds<ROWS, TBK, L::KCONTIG>;
  constexpr int CH = L::KCONTIG ? TBK / 4 : ROWS / 4;  // float4 chunks per LDS row
  constexpr int TOTAL = (L::KCONTIG ? ROWS : TBK) * CH;
  constexpr int PER = (TOTAL + NT - 1) / NT;
  constexpr int BATCH = PER < 8 ? PER : 8;  // fetches in flight per thread
  const bool masked = ld.masked(g);
#pragma unroll
  for (int j0 = 0; j0 < PER; j0 += BATCH) {
    Fetch4 f[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int i = tid + (j0 + j) * NT;
      if (j0 + j < PER && i < TOTAL) {
        const int a = i / CH, b = (i - a * CH) * 4;
        if constexpr (L::KCONTIG) ld.issue(r0 + a, k0 + b, g, f[j]);
        else ld.issue(r0 + b, k0 + a, g, f[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int i = tid + (j0 + j) * NT;
      if (j0 + j < PER && i < TOTAL) {
        const int a = i / CH, b = (i - a * CH) * 4;
        *reinterpret_cast<f32x4*>(T + a * Lds::LD + b) = resolve4(f[j], masked);
      }
    }
  }
}

// Four consecutive-k operand values of tile row `row` at k-offset kk.
template <int ROWS, int TBK, bool KCONTIG>
__device__ inline f32x4 lds_frag(const float* T, int row, int kk) {
  using Lds = TileLds<ROWS, TBK, KCONTIG>;
  if constexpr (KCONTIG) {
    return *reinterpret_cast<const f32x4*>(T + row * Lds::LD + kk);
  } else {
    return f32x4{T[(kk + 0) * Lds::LD + row], T[(kk + 1) * Lds::LD + row], T[(kk + 2) * Lds::LD + row],
                 T[(kk + 3) * Lds::LD + row]};
  }
}

template <int BM, int BN, int WGM, int WGN, int TBK, bool PARTIAL, class LA, class LB, class EP>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm(LA la, LB lb, EP ep, float* ws, int M, int N, int K,
                                                         int kchunk, int splits) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "bad tile");
  static_assert(TBK % 16 == 0, "TBK must be a multiple of 16");
  using LdsA = TileLds<BM, TBK, LA::KCONTIG>;
  using LdsB = TileLds<BN, TBK, LB::KCONTIG>;
  __shared__ __attribute__((aligned(16))) float As[LdsA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[LdsB::SIZE];

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
    if (k0 != kbeg) __syncthreads();
    stage_tile<BM, TBK, NT>(As, la, m0, k0, g, tid);
    stage_tile<BN, TBK, NT>(Bs, lb, n0, k0, g, tid);
    __syncthreads();
    const int kspan = min(TBK, kend - k0);  // multiple of 4 is not required: zero padded
#pragma unroll 2
    for (int kb = 0; kb < kspan; kb += 16) {
      f32x4 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = lds_frag<BM, TBK, LA::KCONTIG>(As, wm * WTM + i * 16 + lr, kb + lk);
#pragma unroll
      for (int j = 0; j < FN; ++j) b[j] = lds_frag<BN, TBK, LB::KCONTIG>(Bs, wn * WTN + j * 16 + lr, kb + lk);
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
                                                       int groups, FDiv dmn, FDiv dn) {
  const int MN = M * N;
  const int total = groups * MN;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
    const int g = dmn.div(i);
    const int mn = i - g * MN;
    const int m = dn.div(mn), n = mn - m * N;
    if (m >= ep.rows(g)) continue;
    float s = 0.f;
    const float* p = ws + long(g) * splits * MN + mn;
    for (int sp = 0; sp < splits; ++sp) s += p[long(sp) * MN];
    ep.store(m, n, s, g);
  }
}

// Tile shapes: BM x BN output tile, TBK reduction slice per LDS stage.
enum TileCfg { T32x32 = 0, T64x32 = 1, T32x64 = 2, T64x64 = 3, T128x32 = 4, T128x64 = 5, T64x128 = 6, kNumCfg = 7 };

struct TileDims {
  int bm, bn, tbk;
};

inline TileDims tile_dims(int cfg) {
  switch (cfg) {
    case T32x32: return {32, 32, 256};
    case T64x32: return {64, 32, 128};
    case T32x64: return {32, 64, 128};
    case T64x64: return {64, 64, 128};
    case T128x32: return {128, 32, 128};
    case T128x64: return {128, 64, 64};
    default: return {64, 128, 64};
  }
}

struct GemmPlan {
  int cfg, bm, bn, tbk, splits, kchunk;
};

// Chooses a tile and a split-K factor: enough workgroups to cover the 256
// CUs, each split a whole number of LDS stages, within `ws_floats` of
// workspace.
GemmPlan plan_gemm(int M, int N, int K, int groups, long ws_floats, int force_cfg = -1, int force_splits = 0);

// Workspace owned by the context (stream-ordered scratch for split-K).
float* ctx_workspace(ttrl_ctx* ctx, long* floats);

template <int BM, int BN, int WGM, int WGN, int TBK, class LA, class LB, class EP>
inline void launch_cfg(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K, int groups,
                       const GemmPlan& p, hipStream_t st) {
  dim3 grid(ceil_div(M, BM), ceil_div(N, BN), unsigned(groups * p.splits));
  if (p.splits == 1) {
    hipLaunchKernelGGL((k_gemm<BM, BN, WGM, WGN, TBK, false, LA, LB, EP>), grid, dim3(64 * WGM * WGN), 0, st, la,
                       lb, ep, ws, M, N, K, p.kchunk, 1);
  } else {
    hipLaunchKernelGGL((k_gemm<BM, BN, WGM, WGN, TBK, true, LA, LB, EP>), grid, dim3(64 * WGM * WGN), 0, st, la,
                       lb, ep, ws, M, N, K, p.kchunk, p.splits);
    const long total = long(groups) * M * N;
    unsigned blocks = unsigned(total / 256 + 1);
    if (blocks > 4096) blocks = 4096;
    FDiv dmn, dn;
    dmn.set(M * N);
    dn.set(N);
    hipLaunchKernelGGL((k_splitk_reduce<EP>), dim3(blocks), dim3(256), 0, st, ws, ep, M, N, p.splits, groups, dmn,
                       dn);
  }
}

template <class LA, class LB, class EP>
inline int run_gemm(ttrl_ctx* ctx, const LA& la, const LB& lb, const EP& ep, int M, int N, int K, int groups,
                    const char* name, int force_cfg = -1, int force_splits = 0) {
  if (M <= 0 || N <= 0 || groups <= 0) return TTRL_OK;
  if (groups > kMaxGroups) return set_error(TTRL_EINVAL, "%s: at most %d groups", name, kMaxGroups);
  if (long(groups) * M * N >= (1L << 31)) return set_error(TTRL_EINVAL, "%s: output too large", name);
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  GemmPlan p = plan_gemm(M, N, K, groups, wsf, force_cfg, force_splits);
  hipStream_t st = stream_of(ctx);
  switch (p.cfg) {
    case T32x32: launch_cfg<32, 32, 2, 2, 256>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T64x32: launch_cfg<64, 32, 2, 2, 128>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T32x64: launch_cfg<32, 64, 2, 2, 128>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T64x64: launch_cfg<64, 64, 2, 2, 128>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T128x32: launch_cfg<128, 32, 4, 1, 128>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    case T128x64: launch_cfg<128, 64, 2, 2, 64>(la, lb, ep, ws, M, N, K, groups, p, st); break;
    default: launch_cfg<64, 128, 2, 2, 64>(la, lb, ep, ws, M, N, K, groups, p, st); break;
  }
  return check_launch(name);
}

// Per-group pointer table from a base pointer and an element stride.
template <class T>
inline void fill_groups(T* (&dst)[kMaxGroups], T* base, long stride, int groups) {
  for (int g = 0; g < kMaxGroups; ++g) dst[g] = (base && g < groups) ? base + g * stride : nullptr;
}

}  // namespace ttrl
